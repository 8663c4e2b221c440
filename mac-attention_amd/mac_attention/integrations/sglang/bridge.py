"""Loader and Python binding for the gfx950 MAC kernels.

Replaces attention/src/mac_attention/integrations/sglang/bridge.py of the
reference: same loader names, same call signatures, same errors
(``RuntimeError`` for every failed check), but instead of JIT-compiling CUDA
with ``torch.utils.cpp_extension`` it binds the prebuilt C-ABI library
``libmac_hip.so`` (declared in ``include/mac_attention_amd.h``) with ctypes.

PyTorch is used only to read tensor metadata (pointer, dtype, shape) and the
current HIP stream; every kernel runs from the library.  If the library is
missing the loaders raise -- there is no fallback implementation.
"""

from __future__ import annotations

import ctypes
import os
from functools import lru_cache
from typing import Any

import torch  # loads the HIP runtime the library must share

_PKG_ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__)))))
LIB_PATH = os.environ.get("MAC_HIP_LIBRARY", os.path.join(_PKG_ROOT, "libmac_hip.so"))

ABI_VERSION = 2
_MAX_GROUP = 8
_HEAD_DIM = 128

_p = ctypes.c_void_p
_i32 = ctypes.c_int32
_i64 = ctypes.c_int64
_u32 = ctypes.c_uint32
_f64 = ctypes.c_double


class MacDecodeArgs(ctypes.Structure):
    """ctypes mirror of ``MacDecodeArgs`` in include/mac_attention_amd.h."""

    _fields_ = [
        ("struct_size", _u32), ("abi_version", _u32),
        ("q_post", _p), ("q_pre", _p), ("k_buffer", _p), ("v_buffer", _p),
        ("req_to_token", _p), ("req_ids", _p), ("past_lens", _p), ("out_cache_loc", _p),
        ("query_cache", _p), ("attn_cache", _p), ("lse_cache", _p), ("out", _p), ("out_lse", _p),
        ("match_dist", _p), ("match_pos", _p), ("match_slot", _p),
        ("head_hit", _p), ("head_match_slot", _p), ("head_match_pos", _p),
        ("head_prefix_end", _p), ("head_rect_start", _p), ("head_new_end", _p),
        ("group_rect_begin", _p), ("group_rect_end", _p), ("group_rect_tiles", _p),
        ("group_tail_begin", _p), ("group_tail_end", _p), ("group_tail_tiles", _p),
        ("group_mode", _p), ("complete_task_go", _p), ("complete_task_tile", _p),
        ("task_counts", _p), ("partial_o", _p), ("partial_lse", _p),
        ("cache_ready", _p), ("cache_epoch", _p), ("request_epoch", _p),
        ("N", _i32), ("Hq", _i32), ("Hkv", _i32), ("D", _i32), ("M", _i32), ("R", _i32),
        ("pool_tokens", _i64),
        ("req_to_token_rows", _i32), ("req_to_token_stride", _i32),
        ("out_cache_loc_is_i64", _i32), ("max_match_tiles", _i32), ("max_tiles_context", _i32),
        ("partial_o_is_bf16", _i32),
        ("complete_task_len", _i64),
        ("workspace_rows", _i32),
        ("max_context", _i32), ("tile_tokens", _i32), ("match_tile_slots", _i32),
        ("semantic_pos_ahead", _i32), ("front_sink_tokens", _i32), ("gen_min_limit", _i32),
        ("lookback_right", _i32), ("candidate_mode", _i32),
        ("threshold", _f64), ("sm_scale", _f64),
        ("debug_enabled", _i32), ("bench_mode", _i32),
        ("bench_hit_rate", _f64), ("bench_hit_rate_std", _f64), ("bench_skip_ratio", _f64),
        ("bench_skip_ratio_std", _f64), ("bench_match_lag_mean", _f64),
        ("bench_match_lag_std", _f64),
        ("bench_seed", _i32), ("bench_miss_mask", _i32), ("bench_layer_id", _i32),
        ("mixed_group_fallback", _i32), ("bench_exact_quota", _i32),
        ("phase_cycles", _p), ("phase_cycles_len", _i32),
    ]


EXPORTED_SYMBOLS = (
    "mac_persistent_decode_bf16",
    "mac_prefill_update_cache",
    "mac_mark_persistent_ready",
    "mac_invalidate_persistent_ready",
    "mac_update_request_state",
    "mac_update_then_downdate_bf16_inplace",
    "mac_prefill_window_attention_bf16",
    "mac_prefill_rectify_update_cache_bf16",
    "mac_decode_rope_preserve_q_bf16",
    "mac_last_error",
    "mac_abi_version",
)


class MacWindowAttentionArgs(ctypes.Structure):
    """ctypes mirror of ``MacWindowAttentionArgs``."""

    _fields_ = [
        ("struct_size", _u32), ("abi_version", _u32),
        ("q", _p), ("k_buffer", _p), ("v_buffer", _p), ("qo_indptr", _p), ("kv_indptr", _p),
        ("kv_indices", _p), ("out", _p), ("out_lse", _p),
        ("total_q", _i64), ("pool_tokens", _i64), ("kv_indices_len", _i64),
        ("B", _i32), ("Hq", _i32), ("Hkv", _i32), ("D", _i32), ("window_left", _i32),
        ("sm_scale", _f64),
    ]


class MacRectifyArgs(ctypes.Structure):
    """ctypes mirror of ``MacRectifyArgs``."""

    _fields_ = [
        ("struct_size", _u32), ("abi_version", _u32),
        ("q_post", _p), ("src_q", _p), ("o_full", _p), ("lse_full", _p), ("k_buffer", _p),
        ("v_buffer", _p), ("qo_indptr", _p), ("kv_indptr", _p), ("kv_indices", _p),
        ("q_cache", _p), ("attn_cache", _p), ("lse_cache", _p), ("q_post_cache", _p),
        ("request_length", _p), ("req_ids", _p),
        ("total_q", _i64), ("pool_tokens", _i64), ("kv_indices_len", _i64),
        ("request_length_len", _i32), ("B", _i32), ("R", _i32), ("M", _i32), ("Hq", _i32),
        ("Hkv", _i32), ("D", _i32), ("semantic_pos_ahead", _i32), ("front_sink_tokens", _i32),
        ("sink_mode", _i32), ("sm_scale", _f64),
    ]


@lru_cache(maxsize=1)
def load_library(path: str | None = None) -> ctypes.CDLL:
    """Open libmac_hip.so and declare its C signatures (no GPU work)."""
    path = path or LIB_PATH
    if not os.path.exists(path):
        raise RuntimeError(
            f"MAC HIP library not found at {path}; build it with `python -c "
            f"'import __graft_entry__ as g; g.build()'` from the repository root"
        )
    lib = ctypes.CDLL(path)
    lib.mac_last_error.restype = ctypes.c_char_p
    lib.mac_abi_version.restype = ctypes.c_int
    lib.mac_persistent_decode_bf16.argtypes = [ctypes.POINTER(MacDecodeArgs), _p]
    lib.mac_persistent_decode_bf16.restype = ctypes.c_int
    lib.mac_prefill_update_cache.argtypes = [
        _p, _p, _p, _p, _i32, _p, _i32, _p, _p, _p, _i32, _p, _p, _i32, _i32, _i32, _i32, _p, _p,
    ]
    lib.mac_prefill_update_cache.restype = ctypes.c_int
    for name in ("mac_mark_persistent_ready", "mac_invalidate_persistent_ready"):
        fn = getattr(lib, name)
        fn.argtypes = [_p, _p, _p, _p, _i32, _i32, _p]
        fn.restype = ctypes.c_int
    lib.mac_update_request_state.argtypes = [_p, _p, _p, _p, _p, _p, _i32, _i32, _p]
    lib.mac_update_request_state.restype = ctypes.c_int
    lib.mac_update_then_downdate_bf16_inplace.argtypes = [_p, _p, _i32, _p, _p, _i32, _i64, _i32, _p]
    lib.mac_update_then_downdate_bf16_inplace.restype = ctypes.c_int
    lib.mac_prefill_window_attention_bf16.argtypes = [ctypes.POINTER(MacWindowAttentionArgs), _p]
    lib.mac_prefill_window_attention_bf16.restype = ctypes.c_int
    lib.mac_prefill_rectify_update_cache_bf16.argtypes = [ctypes.POINTER(MacRectifyArgs), _p]
    lib.mac_prefill_rectify_update_cache_bf16.restype = ctypes.c_int
    lib.mac_decode_rope_preserve_q_bf16.argtypes = [
        _p, _i64, _p, _i64, _p, _i64, _p, _i64, _p, _p, _i64, _p, _i64, _i64, _i32, _p, _i32, _p, _i32,
        _i64, _i32, _i32, _i32, _i32, _p]
    lib.mac_decode_rope_preserve_q_bf16.restype = ctypes.c_int
    if lib.mac_abi_version() != ABI_VERSION:
        raise RuntimeError(
            f"{path} has ABI version {lib.mac_abi_version()}, binding expects {ABI_VERSION}"
        )
    return lib


BENCH_LIB_PATH = os.environ.get("MAC_BENCH_LIBRARY", os.path.join(_PKG_ROOT, "libmac_bench.so"))
BENCH_EXPORTED_SYMBOLS = ("mac_bench_stream_read", "mac_bench_decode_timed", "mac_bench_last_error")
NOALLOC_LIB_PATH = os.environ.get("MAC_NOALLOC_LIBRARY", os.path.join(_PKG_ROOT, "libmac_noalloc.so"))
NOALLOC_EXPORTED_SYMBOLS = ("mac_persistent_decode_bf16_noalloc", "mac_noalloc_last_error")


@lru_cache(maxsize=1)
def load_bench_library(path: str | None = None) -> ctypes.CDLL:
    """Open libmac_bench.so, the measurement helpers (not part of the decode
    library): the streaming read and the decode step timed per kernel."""
    path = path or BENCH_LIB_PATH
    if not os.path.exists(path):
        raise RuntimeError(f"measurement helper not found at {path}; build with __graft_entry__.build()")
    lib = ctypes.CDLL(path)
    lib.mac_bench_stream_read.argtypes = [_p, _i64, _p, _i32, _p]
    lib.mac_bench_stream_read.restype = ctypes.c_int
    lib.mac_bench_decode_timed.argtypes = [ctypes.POINTER(MacDecodeArgs), _p, ctypes.POINTER(ctypes.c_float)]
    lib.mac_bench_decode_timed.restype = ctypes.c_int
    lib.mac_bench_last_error.restype = ctypes.c_char_p
    return lib


@lru_cache(maxsize=1)
def load_noalloc_library(path: str | None = None) -> ctypes.CDLL:
    """Open libmac_noalloc.so (the decode step with its workspaces in a static
    device array; no reference counterpart).  It links against libmac_hip.so
    in the same directory."""
    path = path or NOALLOC_LIB_PATH
    if not os.path.exists(path):
        raise RuntimeError(f"no-allocation library not found at {path}; build with __graft_entry__.build()")
    load_library()  # the decode library it links against, with its ABI version checked
    lib = ctypes.CDLL(path)
    lib.mac_persistent_decode_bf16_noalloc.argtypes = [ctypes.POINTER(MacDecodeArgs), _p]
    lib.mac_persistent_decode_bf16_noalloc.restype = ctypes.c_int
    lib.mac_noalloc_last_error.restype = ctypes.c_char_p
    return lib


def _raise_on(lib: ctypes.CDLL, rc: int) -> None:
    if rc != 0:
        msg = lib.mac_last_error().decode(errors="replace")
        raise RuntimeError(msg or f"MAC HIP call failed with code {rc}")


# ------------------------------------------------------------- checks ----
# Messages follow the reference's TORCH_CHECKs (mac_decode_persistent.cu:4932-4945).


def _check(cond: bool, msg: str) -> None:
    if not cond:
        raise RuntimeError(msg)


def _check_tensor(t: torch.Tensor, name: str, dtype: torch.dtype, dim: int) -> None:
    _check(t.is_cuda, f"{name} must be CUDA")
    _check(t.is_contiguous(), f"{name} must be contiguous")
    _check(t.dtype == dtype, f"{name} has wrong dtype")
    _check(t.dim() == dim, f"{name} has wrong rank")


def _check_partial_o(t: torch.Tensor, name: str) -> None:
    _check(t.is_cuda, f"{name} must be CUDA")
    _check(t.is_contiguous(), f"{name} must be contiguous")
    _check(t.dtype in (torch.float32, torch.bfloat16), f"{name} must be float32 or bfloat16")
    _check(t.dim() == 5, f"{name} has wrong rank")


def _env_flag(name: str, default: int) -> int:
    raw = os.environ.get(name)
    if raw is None:
        return default
    try:
        return 1 if int(raw) != 0 else 0
    except ValueError:
        return 0


# MacDecodeArgs fields of the 30 workspace tensors (prefixes)
_WORKSPACE_FIELDS = ("match_", "head_", "group_", "complete_task_", "task_counts", "partial_")


def _ptr(t: torch.Tensor | None) -> int | None:
    if t is None or t.numel() == 0:
        return None
    return t.data_ptr()


def _stream(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


class PersistentDecodeExtension:
    """Object returned by :func:`load_mac_persistent_decode_extension`."""

    def __init__(self, lib: ctypes.CDLL):
        self._lib = lib

    def mac_persistent_decode_bf16(self, *args) -> None:
        """One fused MAC decode step (reference: mac_decode_persistent.cu:4962-5524).

        Same 68 positional arguments, same in-place outputs, returns None.
        ``query_post_cache`` is accepted and ignored, as in the reference
        (:5045-5049).  ``MAC_PERSISTENT_MIXED_GROUP_FALLBACK`` and
        ``MAC_BENCH_EXACT_QUOTA`` are read from the environment on every call.
        """
        a, device = self._marshal(*args)
        with torch.cuda.device(device):
            rc = self._lib.mac_persistent_decode_bf16(ctypes.byref(a), _stream(device))
        _raise_on(self._lib, rc)

    def mac_persistent_decode_bf16_noalloc(self, *args) -> None:
        """The same step through libmac_noalloc.so's entry point (no reference
        counterpart): the same 68 positional arguments, but the 30 workspace
        tensors and phase_cycles may be None -- they are neither checked nor
        used (the library's static device array holds the workspaces), and
        the decisions are not returned.  At most 4096 query heads per step
        and 2048 ring slots."""
        a, device = self._marshal(*args, use_workspaces=False)
        lib = load_noalloc_library()
        with torch.cuda.device(device):
            rc = lib.mac_persistent_decode_bf16_noalloc(ctypes.byref(a), _stream(device))
        if rc != 0:
            msg = lib.mac_noalloc_last_error().decode(errors="replace")
            raise RuntimeError(msg or f"MAC HIP call failed with code {rc}")

    def phase_times_ms(self, *args) -> tuple[float, float, float]:
        """Runs the same step eagerly through libmac_bench.so's timed copy of
        the decode step (HIP events around each kernel) and returns
        (decision kernel, span_attention, merge_write) milliseconds.
        Synchronises; profiling only (no reference counterpart)."""
        a, device = self._marshal(*args)
        lib = load_bench_library()
        ms = (ctypes.c_float * 3)()
        with torch.cuda.device(device):
            rc = lib.mac_bench_decode_timed(ctypes.byref(a), _stream(device), ms)
        if rc != 0:
            raise RuntimeError(lib.mac_bench_last_error().decode(errors="replace") or f"code {rc}")
        return float(ms[0]), float(ms[1]), float(ms[2])

    def _marshal(
        self,
        q_post, q_pre, k_buffer, v_buffer, req_to_token, req_ids, past_lens, out_cache_loc,
        query_cache, attn_cache, lse_cache, out, optional_lse,
        match_dist, match_pos, match_slot,
        head_hit, head_match_slot, head_match_pos, head_prefix_end, head_rect_start, head_new_end,
        group_rect_begin, group_rect_end, group_rect_tiles, group_tail_begin, group_tail_end,
        group_tail_tiles, group_mode,
        complete_task_go, complete_task_tile, tail_task_go, tail_task_tile, hit_tail_task_ho,
        hit_tail_task_tile, task_counts,
        partial_rect_o, partial_rect_lse, partial_rect_reduced_o, partial_rect_reduced_lse,
        partial_tail_o, partial_tail_lse, phase_cycles,
        max_context, tile_tokens, match_tile_slots, semantic_pos_ahead, front_sink_tokens,
        gen_min_limit, lookback_right, candidate_mode,
        threshold, sm_scale, debug_enabled, bench_mode,
        bench_hit_rate, bench_hit_rate_std, bench_skip_ratio, bench_skip_ratio_std,
        bench_match_lag_mean, bench_match_lag_std, bench_seed, bench_miss_mask, bench_layer_id,
        query_post_cache, mac_cache_ready, mac_cache_epoch, mac_request_epoch,
        use_workspaces: bool = True,
    ) -> tuple[MacDecodeArgs, torch.device]:
        """Checks the 68 arguments like the reference launcher
        (mac_decode_persistent.cu:5031-5175) and fills the C argument block.
        With use_workspaces False (the no-allocation entry point) the
        workspace tensors and phase_cycles are neither checked nor passed."""
        bf16, f32, i32, i64 = torch.bfloat16, torch.float32, torch.int32, torch.int64
        _check_tensor(q_post, "q_post", bf16, 3)
        _check_tensor(q_pre, "q_pre", bf16, 3)
        _check_tensor(k_buffer, "k_buffer", bf16, 3)
        _check_tensor(v_buffer, "v_buffer", bf16, 3)
        _check_tensor(req_to_token, "req_to_token", i32, 2)
        _check_tensor(req_ids, "req_ids", i32, 1)
        _check_tensor(past_lens, "past_lens", i32, 1)
        _check(out_cache_loc.is_cuda, "out_cache_loc must be CUDA")
        _check(out_cache_loc.is_contiguous(), "out_cache_loc must be contiguous")
        _check(out_cache_loc.dim() == 1, "out_cache_loc has wrong rank")
        _check(out_cache_loc.dtype in (i32, i64), "out_cache_loc must be int32 or int64")
        _check_tensor(query_cache, "query_cache", bf16, 4)
        if query_post_cache is not None and query_post_cache.numel() > 0:
            _check_tensor(query_post_cache, "query_post_cache", bf16, 4)
        _check_tensor(attn_cache, "attn_cache", bf16, 4)
        _check_tensor(lse_cache, "lse_cache", f32, 3)
        _check_tensor(out, "out", bf16, 3)
        _check(optional_lse.is_cuda, "optional_lse must be CUDA")
        _check(optional_lse.is_contiguous(), "optional_lse must be contiguous")
        _check(optional_lse.numel() == 0 or optional_lse.dtype == f32,
               "optional_lse must be empty or float32")
        if use_workspaces or phase_cycles is not None:
            _check(phase_cycles.is_cuda, "phase_cycles must be CUDA")
            _check(phase_cycles.dtype == i64, "phase_cycles must be int64")
            _check(phase_cycles.numel() >= 6, "phase_cycles must have at least 6 elements")
        _check_tensor(q_post, "q_post", bf16, 3)  # (the shape checks below read it)
        N, Hq, D = (int(x) for x in q_post.shape)
        Hkv = int(k_buffer.shape[1])
        if use_workspaces:
            self._check_workspaces(
                N, Hq, Hkv, query_cache, max_context, tile_tokens, match_tile_slots, semantic_pos_ahead,
                bench_mode, match_dist, match_pos, match_slot, head_hit, head_match_slot,
                head_match_pos, head_prefix_end, head_rect_start, head_new_end, group_rect_begin,
                group_rect_end, group_rect_tiles, group_tail_begin, group_tail_end, group_tail_tiles,
                group_mode, complete_task_go, complete_task_tile, tail_task_go, tail_task_tile,
                hit_tail_task_ho, hit_tail_task_tile, task_counts, partial_rect_o, partial_rect_lse,
                partial_rect_reduced_o, partial_rect_reduced_lse, partial_tail_o, partial_tail_lse)
        else:
            _check(int(bench_mode) in (0, 1, 2), "unsupported synthetic MAC bench mode")
        _check(D == _HEAD_DIM, "persistent decode v1 supports D=128 only")
        _check(tuple(q_pre.shape) == tuple(q_post.shape), "q_pre/q_post shape mismatch")
        _check(tuple(v_buffer.shape) == tuple(k_buffer.shape), "k/v shape mismatch")
        _check(int(k_buffer.shape[2]) == D, "k/v head_dim mismatch")
        _check(Hkv > 0 and Hq % Hkv == 0, "Hq must be divisible by Hkv")
        G = Hq // Hkv
        _check(0 < G <= _MAX_GROUP, "unsupported GQA group size")
        _check(req_ids.shape[0] >= N and past_lens.shape[0] >= N and out_cache_loc.shape[0] >= N,
               "batch metadata too small")
        _check(tuple(out.shape) == tuple(q_post.shape), "out shape mismatch")
        _check(optional_lse.numel() == 0 or optional_lse.numel() >= N * Hq,
               "optional_lse too small")
        R, M = int(query_cache.shape[0]), int(query_cache.shape[1])
        _check(query_cache.shape[2] == Hq and query_cache.shape[3] == D,
               "query_cache shape mismatch")
        _check(tuple(attn_cache.shape) == tuple(query_cache.shape), "attn_cache shape mismatch")
        _check(tuple(lse_cache.shape) == (R, M, Hq), "lse_cache shape mismatch")
        return self._fill(
            N, Hq, Hkv, D, M, R, q_post, q_pre, k_buffer, v_buffer, req_to_token, req_ids, past_lens,
            out_cache_loc, query_cache, attn_cache, lse_cache, out, optional_lse,
            match_dist, match_pos, match_slot,
            head_hit, head_match_slot, head_match_pos, head_prefix_end, head_rect_start, head_new_end,
            group_rect_begin, group_rect_end, group_rect_tiles, group_tail_begin, group_tail_end,
            group_tail_tiles, group_mode, complete_task_go, complete_task_tile, task_counts,
            partial_rect_o, partial_rect_lse, phase_cycles,
            max_context, tile_tokens, match_tile_slots, semantic_pos_ahead, front_sink_tokens,
            gen_min_limit, lookback_right, candidate_mode, threshold, sm_scale, debug_enabled, bench_mode,
            bench_hit_rate, bench_hit_rate_std, bench_skip_ratio, bench_skip_ratio_std,
            bench_match_lag_mean, bench_match_lag_std, bench_seed, bench_miss_mask, bench_layer_id,
            mac_cache_ready, mac_cache_epoch, mac_request_epoch, use_workspaces)

    @staticmethod
    def _check_workspaces(
        N, Hq, Hkv, query_cache, max_context, tile_tokens, match_tile_slots, semantic_pos_ahead,
        bench_mode, match_dist, match_pos, match_slot, head_hit, head_match_slot, head_match_pos,
        head_prefix_end, head_rect_start, head_new_end, group_rect_begin, group_rect_end,
        group_rect_tiles, group_tail_begin, group_tail_end, group_tail_tiles, group_mode,
        complete_task_go, complete_task_tile, tail_task_go, tail_task_tile, hit_tail_task_ho,
        hit_tail_task_tile, task_counts, partial_rect_o, partial_rect_lse, partial_rect_reduced_o,
        partial_rect_reduced_lse, partial_tail_o, partial_tail_lse,
    ) -> None:
        """The reference launcher's workspace checks (mac_decode_persistent.cu:5090-5153),
        plus the complete-task minimum this build's kernels need."""
        f32, i32 = torch.float32, torch.int32
        D = _HEAD_DIM
        G = Hq // Hkv if Hkv > 0 and Hq % Hkv == 0 else 1
        M = int(query_cache.shape[1])
        _check_tensor(match_dist, "match_dist", f32, 3)
        _check_tensor(match_pos, "match_pos", i32, 3)
        _check_tensor(match_slot, "match_slot", i32, 3)
        for name, t in (("head_hit", head_hit), ("head_match_slot", head_match_slot),
                        ("head_match_pos", head_match_pos), ("head_prefix_end", head_prefix_end),
                        ("head_rect_start", head_rect_start), ("head_new_end", head_new_end),
                        ("group_rect_begin", group_rect_begin), ("group_rect_end", group_rect_end),
                        ("group_rect_tiles", group_rect_tiles),
                        ("group_tail_begin", group_tail_begin), ("group_tail_end", group_tail_end),
                        ("group_tail_tiles", group_tail_tiles), ("group_mode", group_mode)):
            _check_tensor(t, name, i32, 2)
        for name, t in (("complete_task_go", complete_task_go),
                        ("complete_task_tile", complete_task_tile),
                        ("tail_task_go", tail_task_go), ("tail_task_tile", tail_task_tile),
                        ("hit_tail_task_ho", hit_tail_task_ho),
                        ("hit_tail_task_tile", hit_tail_task_tile), ("task_counts", task_counts)):
            _check_tensor(t, name, i32, 1)
        _check_partial_o(partial_rect_o, "partial_rect_o")
        _check_tensor(partial_rect_lse, "partial_rect_lse", f32, 4)
        _check_partial_o(partial_rect_reduced_o, "partial_rect_reduced_o")
        _check_tensor(partial_rect_reduced_lse, "partial_rect_reduced_lse", f32, 4)
        _check_partial_o(partial_tail_o, "partial_tail_o")
        _check_tensor(partial_tail_lse, "partial_tail_lse", f32, 4)
        _check(partial_rect_reduced_o.dtype == partial_rect_o.dtype
               and partial_tail_o.dtype == partial_rect_o.dtype,
               "all partial output workspaces must use the same dtype")

        max_match_tiles = int(match_dist.shape[2])
        mtc = int(partial_rect_lse.shape[2])
        mtr = int(partial_rect_reduced_lse.shape[2])
        mtt = int(partial_tail_lse.shape[2])
        tile_tokens = int(tile_tokens)
        match_tile_slots = int(match_tile_slots)
        _check(tile_tokens > 0 and match_tile_slots > 0, "tile sizes must be positive")
        _check(max_match_tiles >= (M + match_tile_slots - 1) // match_tile_slots,
               "match workspace too small")
        _check(mtc >= (int(max_context) + tile_tokens - 1) // tile_tokens,
               "rect workspace too small")
        _check(mtr >= (int(max_context) + tile_tokens * 32 - 1) // (tile_tokens * 32),
               "reduced rect workspace too small")
        _check(mtt >= (int(semantic_pos_ahead) + tile_tokens - 1) // tile_tokens,
               "tail workspace too small")
        for name, t, tiles in (("rect output", partial_rect_o, mtc),
                               ("reduced rect output", partial_rect_reduced_o, mtr),
                               ("tail output", partial_tail_o, mtt)):
            _check(t.shape[0] >= N and t.shape[1] == Hkv and t.shape[2] == tiles
                   and t.shape[3] == G and t.shape[4] == D, f"{name} workspace has wrong shape")
        for name, t, tiles in (("rect lse", partial_rect_lse, mtc),
                               ("reduced rect lse", partial_rect_reduced_lse, mtr),
                               ("tail lse", partial_tail_lse, mtt)):
            _check(t.shape[0] >= N and t.shape[1] == Hkv and t.shape[2] == tiles
                   and t.shape[3] == G, f"{name} workspace has wrong shape")
        _check(group_mode.shape[0] >= N and group_mode.shape[1] >= Hkv,
               "group_mode workspace too small")
        _check(complete_task_tile.numel() == complete_task_go.numel(),
               "complete task shape mismatch")
        _check(tail_task_tile.numel() == tail_task_go.numel(), "tail task shape mismatch")
        _check(hit_tail_task_tile.numel() == hit_tail_task_ho.numel(),
               "hit tail task shape mismatch")
        _check(task_counts.numel() >= 9, "task_counts must have at least nine elements")
        _check(int(bench_mode) in (0, 1, 2), "unsupported synthetic MAC bench mode")
        _check(complete_task_go.numel() >= N * Hq * mtc, "complete task workspace too small")
        _check(tail_task_go.numel() >= N * Hkv * mtt, "tail task workspace too small")
        _check(hit_tail_task_ho.numel() >= N * Hq * mtt, "hit tail task workspace too small")
        ws_rows = min(int(t.shape[0]) for t in (
            head_hit, head_match_slot, head_match_pos, head_prefix_end, head_rect_start,
            head_new_end, group_rect_begin, group_rect_end, group_rect_tiles, group_tail_begin,
            group_tail_end, group_tail_tiles, group_mode, match_dist, match_pos, match_slot))
        for t in (head_hit, head_match_slot, head_match_pos, head_prefix_end, head_rect_start,
                  head_new_end, match_dist, match_pos, match_slot):
            _check(t.shape[1] == Hq, "head workspace must have Hq columns")
        for t in (group_rect_begin, group_rect_end, group_rect_tiles, group_tail_begin,
                  group_tail_end, group_tail_tiles, group_mode):
            _check(t.shape[1] == Hkv, "group workspace must have Hkv columns")
        _check(ws_rows >= N, "head/group workspace has fewer rows than the batch")
        # this build's kernels keep per-group flags and the task counter there
        _check(complete_task_go.numel() >= 2 * N * Hkv + 6,
               "complete task workspace too small: needs at least 2 * N * Hkv + 6 entries")

    @staticmethod
    def _fill(
        N, Hq, Hkv, D, M, R, q_post, q_pre, k_buffer, v_buffer, req_to_token, req_ids, past_lens,
        out_cache_loc, query_cache, attn_cache, lse_cache, out, optional_lse,
        match_dist, match_pos, match_slot,
        head_hit, head_match_slot, head_match_pos, head_prefix_end, head_rect_start, head_new_end,
        group_rect_begin, group_rect_end, group_rect_tiles, group_tail_begin, group_tail_end,
        group_tail_tiles, group_mode, complete_task_go, complete_task_tile, task_counts,
        partial_rect_o, partial_rect_lse, phase_cycles,
        max_context, tile_tokens, match_tile_slots, semantic_pos_ahead, front_sink_tokens,
        gen_min_limit, lookback_right, candidate_mode, threshold, sm_scale, debug_enabled, bench_mode,
        bench_hit_rate, bench_hit_rate_std, bench_skip_ratio, bench_skip_ratio_std,
        bench_match_lag_mean, bench_match_lag_std, bench_seed, bench_miss_mask, bench_layer_id,
        mac_cache_ready, mac_cache_epoch, mac_request_epoch, use_workspaces,
    ) -> tuple[MacDecodeArgs, torch.device]:
        """The readiness-gate checks and the C argument block."""
        bf16, i64 = torch.bfloat16, torch.int64
        ready = epoch = req_epoch = None
        if mac_cache_ready is not None and mac_cache_ready.numel() > 0:
            _check(mac_cache_ready.is_cuda, "mac_cache_ready must be CUDA")
            _check(mac_cache_ready.is_contiguous(), "mac_cache_ready must be contiguous")
            _check(mac_cache_ready.dtype in (torch.bool, torch.uint8),
                   "mac_cache_ready must be bool or uint8")
            _check(mac_cache_ready.numel() >= R, "mac_cache_ready must cover every request slot")
            ready = mac_cache_ready
            if (mac_cache_epoch is not None and mac_cache_epoch.numel() > 0
                    and mac_request_epoch is not None and mac_request_epoch.numel() > 0):
                _check_tensor(mac_cache_epoch, "mac_cache_epoch", i64, 1)
                _check_tensor(mac_request_epoch, "mac_request_epoch", i64, 1)
                _check(mac_cache_epoch.numel() >= R and mac_request_epoch.numel() >= R,
                       "epoch tensors must cover every request slot")
                epoch, req_epoch = mac_cache_epoch, mac_request_epoch

        a = MacDecodeArgs()
        a.struct_size = ctypes.sizeof(MacDecodeArgs)
        a.abi_version = ABI_VERSION
        for name, t in (("q_post", q_post), ("q_pre", q_pre), ("k_buffer", k_buffer),
                        ("v_buffer", v_buffer), ("req_to_token", req_to_token),
                        ("req_ids", req_ids), ("past_lens", past_lens),
                        ("out_cache_loc", out_cache_loc), ("query_cache", query_cache),
                        ("attn_cache", attn_cache), ("lse_cache", lse_cache), ("out", out),
                        ("out_lse", optional_lse), ("match_dist", match_dist),
                        ("match_pos", match_pos), ("match_slot", match_slot),
                        ("head_hit", head_hit), ("head_match_slot", head_match_slot),
                        ("head_match_pos", head_match_pos), ("head_prefix_end", head_prefix_end),
                        ("head_rect_start", head_rect_start), ("head_new_end", head_new_end),
                        ("group_rect_begin", group_rect_begin), ("group_rect_end", group_rect_end),
                        ("group_rect_tiles", group_rect_tiles),
                        ("group_tail_begin", group_tail_begin), ("group_tail_end", group_tail_end),
                        ("group_tail_tiles", group_tail_tiles), ("group_mode", group_mode),
                        ("complete_task_go", complete_task_go),
                        ("complete_task_tile", complete_task_tile), ("task_counts", task_counts),
                        ("partial_o", partial_rect_o), ("partial_lse", partial_rect_lse),
                        ("cache_ready", ready), ("cache_epoch", epoch),
                        ("request_epoch", req_epoch)):
            if use_workspaces or not name.startswith(_WORKSPACE_FIELDS):
                setattr(a, name, _ptr(t))
        a.N, a.Hq, a.Hkv, a.D, a.M, a.R = N, Hq, Hkv, D, M, R
        a.pool_tokens = int(k_buffer.shape[0])
        a.req_to_token_rows = int(req_to_token.shape[0])
        a.req_to_token_stride = int(req_to_token.shape[1])
        a.out_cache_loc_is_i64 = 1 if out_cache_loc.dtype == i64 else 0
        if use_workspaces:
            a.max_match_tiles = int(match_dist.shape[2])
            a.max_tiles_context = int(partial_rect_lse.shape[2])
            a.partial_o_is_bf16 = 1 if partial_rect_o.dtype == bf16 else 0
            a.complete_task_len = int(complete_task_go.numel())
            a.workspace_rows = min(int(t.shape[0]) for t in (
                head_hit, head_match_slot, head_match_pos, head_prefix_end, head_rect_start,
                head_new_end, group_rect_begin, group_rect_end, group_rect_tiles, group_tail_begin,
                group_tail_end, group_tail_tiles, group_mode, match_dist, match_pos, match_slot))
        a.max_context = int(max_context)
        a.tile_tokens = int(tile_tokens)
        a.match_tile_slots = int(match_tile_slots)
        a.semantic_pos_ahead = int(semantic_pos_ahead)
        a.front_sink_tokens = int(front_sink_tokens)
        a.gen_min_limit = int(gen_min_limit)
        a.lookback_right = int(lookback_right)
        a.candidate_mode = int(candidate_mode)
        a.threshold = float(threshold)
        a.sm_scale = float(sm_scale)
        a.debug_enabled = int(debug_enabled)
        a.bench_mode = int(bench_mode)
        a.bench_hit_rate = float(bench_hit_rate)
        a.bench_hit_rate_std = float(bench_hit_rate_std)
        a.bench_skip_ratio = float(bench_skip_ratio)
        a.bench_skip_ratio_std = float(bench_skip_ratio_std)
        a.bench_match_lag_mean = float(bench_match_lag_mean)
        a.bench_match_lag_std = float(bench_match_lag_std)
        a.bench_seed = int(bench_seed)
        a.bench_miss_mask = int(bench_miss_mask)
        a.bench_layer_id = int(bench_layer_id)
        a.mixed_group_fallback = _env_flag("MAC_PERSISTENT_MIXED_GROUP_FALLBACK", 1)
        a.bench_exact_quota = _env_flag("MAC_BENCH_EXACT_QUOTA", 1)
        if phase_cycles is not None:
            a.phase_cycles = _ptr(phase_cycles)
            a.phase_cycles_len = int(phase_cycles.numel())
        return a, q_post.device


class PrefillUpdateCacheExtension:
    """Object returned by :func:`load_mac_prefill_update_cache_extension`
    (reference: mac_prefill_update_cache.cu:324-512)."""

    def __init__(self, lib: ctypes.CDLL):
        self._lib = lib

    def mac_prefill_update_cache(self, q_cache, attn_cache, lse_cache, request_length, req_ids,
                                 src_q, src_attn, src_lse, offsets, lens, capacity, num_heads,
                                 head_dim, q_post_cache) -> None:
        capacity, num_heads, head_dim = int(capacity), int(num_heads), int(head_dim)
        if capacity <= 0 or req_ids.shape[0] == 0:
            return
        for name, t, dt in (("q_cache", q_cache, torch.bfloat16),
                            ("attn_cache", attn_cache, torch.bfloat16),
                            ("lse_cache", lse_cache, torch.float32),
                            ("request_length", request_length, torch.int32),
                            ("req_ids", req_ids, torch.int32), ("lens", lens, torch.int32),
                            ("offsets", offsets, torch.int32), ("src_q", src_q, torch.bfloat16),
                            ("src_attn", src_attn, torch.bfloat16),
                            ("src_lse", src_lse, torch.float32)):
            _check(t.is_cuda, f"{name} must be a CUDA tensor")
            _check(t.is_contiguous(), f"{name} must be contiguous")
            _check(t.dtype == dt, f"{name} has wrong dtype")
        R = int(q_cache.shape[0])
        _check(R > 0, "R must be > 0")
        _check(q_cache.dim() == 4, "q_cache must be [R,M,H,D]")
        _check(q_cache.shape[1] == capacity, "capacity (M) mismatch")
        _check(q_cache.shape[2] == num_heads, "num_heads (H) mismatch")
        _check(q_cache.shape[3] == head_dim, "head_dim (D) mismatch")
        _check(tuple(attn_cache.shape) == tuple(q_cache.shape), "attn_cache must match q_cache")
        _check(lse_cache.dim() == 3 and lse_cache.shape[0] == R and lse_cache.shape[1] == capacity
               and lse_cache.shape[2] == num_heads, "lse_cache shape mismatch")
        _check(src_q.dim() == 3 and src_q.shape[1] == num_heads and src_q.shape[2] == head_dim,
               "src_q must be [sumN,H,D]")
        _check(tuple(src_attn.shape) == tuple(src_q.shape), "src_attn must match src_q")
        _check(src_lse.dim() == 2 and src_lse.shape[1] == num_heads, "src_lse must be [sumN,H]")
        _check(src_lse.shape[0] == src_q.shape[0], "src_lse row count must match src_q")
        B = int(req_ids.shape[0])
        _check(offsets.shape[0] == B + 1, "offsets must be [B+1]")
        _check(lens.shape[0] == B, "lens must be [B]")
        _check(request_length.shape[0] in (R, B), "request_length must be [R] or [B]")
        qpc = None
        if q_post_cache is not None and q_post_cache.numel() > 0:
            _check(q_post_cache.is_cuda, "q_post_cache must be a CUDA tensor")
            _check(q_post_cache.is_contiguous(), "q_post_cache must be contiguous")
            _check(q_post_cache.dtype == torch.bfloat16, "q_post_cache has wrong dtype")
            _check(tuple(q_post_cache.shape) == tuple(q_cache.shape),
                   "q_post_cache must match q_cache")
            qpc = q_post_cache
        with torch.cuda.device(q_cache.device):
            rc = self._lib.mac_prefill_update_cache(
                _ptr(q_cache), _ptr(attn_cache), _ptr(lse_cache), _ptr(request_length),
                int(request_length.shape[0]), _ptr(req_ids), B, _ptr(src_q), _ptr(src_attn),
                _ptr(src_lse), int(src_q.shape[0]), _ptr(offsets), _ptr(lens), R, capacity,
                num_heads, head_dim, _ptr(qpc), _stream(q_cache.device))
        _raise_on(self._lib, rc)

    def _ready_common(self, ready, cache_epoch, request_epoch, req_ids):
        _check(ready.is_cuda, "ready must be a CUDA tensor")
        _check(ready.is_contiguous(), "ready must be contiguous")
        _check(ready.dtype == torch.bool, "ready has wrong dtype")
        for name, t, dt in (("cache_epoch", cache_epoch, torch.int64),
                            ("request_epoch", request_epoch, torch.int64),
                            ("req_ids", req_ids, torch.int32)):
            _check(t.is_cuda, f"{name} must be a CUDA tensor")
            _check(t.is_contiguous(), f"{name} must be contiguous")
            _check(t.dtype == dt, f"{name} has wrong dtype")
        _check(cache_epoch.shape[0] == ready.shape[0], "cache_epoch must match ready")
        _check(request_epoch.shape[0] == ready.shape[0], "request_epoch must match ready")

    def mac_mark_persistent_ready(self, ready, cache_epoch, request_epoch, req_ids) -> None:
        if req_ids.shape[0] == 0:
            return
        self._ready_common(ready, cache_epoch, request_epoch, req_ids)
        with torch.cuda.device(ready.device):
            rc = self._lib.mac_mark_persistent_ready(
                _ptr(ready), _ptr(cache_epoch), _ptr(request_epoch), _ptr(req_ids),
                int(req_ids.shape[0]), int(ready.shape[0]), _stream(ready.device))
        _raise_on(self._lib, rc)

    def mac_invalidate_persistent_ready(self, ready, cache_epoch, request_epoch, req_ids) -> None:
        if req_ids.shape[0] == 0:
            return
        self._ready_common(ready, cache_epoch, request_epoch, req_ids)
        with torch.cuda.device(ready.device):
            rc = self._lib.mac_invalidate_persistent_ready(
                _ptr(ready), _ptr(cache_epoch), _ptr(request_epoch), _ptr(req_ids),
                int(req_ids.shape[0]), int(ready.shape[0]), _stream(ready.device))
        _raise_on(self._lib, rc)

    def mac_update_request_state(self, req_len, match_req_len, cache_lens, req_ids, seq_lens,
                                 cur_lens) -> None:
        if req_ids.shape[0] == 0:
            return
        for name, t in (("req_len", req_len), ("match_req_len", match_req_len),
                        ("cache_lens", cache_lens), ("req_ids", req_ids), ("seq_lens", seq_lens),
                        ("cur_lens", cur_lens)):
            _check(t.is_cuda, f"{name} must be a CUDA tensor")
            _check(t.is_contiguous(), f"{name} must be contiguous")
            _check(t.dtype == torch.int32, f"{name} has wrong dtype")
        B = int(req_ids.shape[0])
        _check(match_req_len.shape[0] == req_len.shape[0], "match_req_len must match req_len")
        _check(seq_lens.shape[0] >= B, "seq_lens is shorter than req_ids")
        _check(cur_lens.shape[0] >= B, "cur_lens is shorter than req_ids")
        _check(cache_lens.shape[0] >= B, "cache_lens is shorter than req_ids")
        with torch.cuda.device(req_len.device):
            rc = self._lib.mac_update_request_state(
                _ptr(req_len), _ptr(match_req_len), _ptr(cache_lens), _ptr(req_ids),
                _ptr(seq_lens), _ptr(cur_lens), B, int(req_len.shape[0]), _stream(req_len.device))
        _raise_on(self._lib, rc)


@lru_cache(maxsize=4)
def load_mac_persistent_decode_extension(verbose: bool = False, fast_math: bool | None = None) -> Any:
    """Reference bridge.py:211-269.  The kernels are prebuilt for gfx950, so
    ``verbose`` and ``fast_math`` have nothing to select; they are accepted for
    call compatibility."""
    return PersistentDecodeExtension(load_library())


@lru_cache(maxsize=1)
def load_mac_prefill_update_cache_extension(verbose: bool = False) -> Any:
    """Reference bridge.py:172-187."""
    return PrefillUpdateCacheExtension(load_library())


# ------------------------------------------------- prefill rectification ---

_LSE_DTYPES = {torch.float32: 0, torch.bfloat16: 1, torch.float16: 2}


class MergeDowndateExtension:
    """Replaces the module built from mac_merge_downdate_cache.cu
    (reference bridge.py:191-209, binding mac_merge_downdate_cache.cu:320-407)."""

    def __init__(self, lib: ctypes.CDLL):
        self._lib = lib

    def mac_update_then_downdate_bf16_inplace(self, out1_bf16, lse1_any, out2_bf16, lse2_any) -> None:
        """(out2, lse2) <- (out1, lse1) minus (out2, lse2), in place.  Checks
        and messages of mac_merge_downdate_cache.cu:324-347."""
        _check(out1_bf16.is_cuda and out2_bf16.is_cuda, "out tensors must be CUDA")
        _check(lse1_any.is_cuda and lse2_any.is_cuda, "lse tensors must be CUDA")
        _check(out1_bf16.dtype == torch.bfloat16 and out2_bf16.dtype == torch.bfloat16,
               "out tensors must be bfloat16")
        _check(out1_bf16.dim() == 3, "out1 must be [N,H,D]")
        _check(out2_bf16.shape == out1_bf16.shape, "out shapes must match [N,H,D]")
        _check(lse1_any.dim() == 2, "lse1 must be [N,H]")
        _check(lse2_any.shape == lse1_any.shape, "lse shapes must match [N,H]")
        _check(out1_bf16.is_contiguous() and out2_bf16.is_contiguous(), "out tensors must be contiguous")
        _check(lse1_any.is_contiguous() and lse2_any.is_contiguous(), "lse tensors must be contiguous")
        _check(out1_bf16.device == out2_bf16.device, "out1/out2: tensors must be on the same device")
        _check(out1_bf16.device == lse1_any.device, "out1/lse1: tensors must be on the same device")
        _check(lse1_any.device == lse2_any.device, "lse1/lse2: tensors must be on the same device")
        for name, t in (("lse1", lse1_any), ("lse2", lse2_any)):
            _check(t.dtype in _LSE_DTYPES,
                   f"{name} must be float32, bfloat16, or float16; got {t.dtype}")
        n, h, d = (int(x) for x in out1_bf16.shape)
        _check(tuple(lse1_any.shape) == (n, h), "lse1 must be [N,H]")
        with torch.cuda.device(out1_bf16.device):
            rc = self._lib.mac_update_then_downdate_bf16_inplace(
                _ptr(out1_bf16), _ptr(lse1_any), _LSE_DTYPES[lse1_any.dtype], _ptr(out2_bf16),
                _ptr(lse2_any), _LSE_DTYPES[lse2_any.dtype], n * h, d, _stream(out1_bf16.device))
        _raise_on(self._lib, rc)


def _check_ragged(q, k_buffer, v_buffer, qo_indptr, kv_indptr, kv_indices):
    for name, t, dt in (("q", q, torch.bfloat16), ("k_buffer", k_buffer, torch.bfloat16),
                        ("v_buffer", v_buffer, torch.bfloat16), ("qo_indptr", qo_indptr, torch.int32),
                        ("kv_indptr", kv_indptr, torch.int32), ("kv_indices", kv_indices, torch.int32)):
        _check(t.is_cuda, f"{name} must be CUDA")
        _check(t.is_contiguous(), f"{name} must be contiguous")
        _check(t.dtype == dt, f"{name} has wrong dtype")
    _check(q.dim() == 3 and int(q.shape[2]) == _HEAD_DIM, "q must be [total_q,Hq,128]")
    _check(k_buffer.dim() == 3 and k_buffer.shape == v_buffer.shape, "k/v buffers must be [pool,Hkv,128]")
    _check(int(k_buffer.shape[2]) == _HEAD_DIM, "k/v head_dim mismatch")
    _check(int(q.shape[1]) % int(k_buffer.shape[1]) == 0, "Hq must be a multiple of Hkv")
    _check(qo_indptr.dim() == 1 and kv_indptr.shape == qo_indptr.shape, "indptr must be [B+1]")


class PrefillRectifyExtension:
    """Prefill rectification on gfx950.  ``window_attention_return_lse`` stands
    in for the windowed FlashInfer pass of flashinfer_hooks.py:2436-2466
    (returning natural-log lse, i.e. the value after the reference's ln 2
    scaling at :2467); ``mac_prefill_rectify_update_cache`` fuses that pass,
    the downdate (:2468-2472) and the ring write of _offload_fast_cache
    (:2482) for the rows the ring keeps."""

    def __init__(self, lib: ctypes.CDLL):
        self._lib = lib

    def window_attention_return_lse(self, q, k_buffer, v_buffer, qo_indptr, kv_indptr, kv_indices,
                                    window_left: int, sm_scale: float, out=None, out_lse=None):
        _check_ragged(q, k_buffer, v_buffer, qo_indptr, kv_indptr, kv_indices)
        total_q, hq, _ = (int(x) for x in q.shape)
        if out is None:
            out = torch.empty_like(q)
        if out_lse is None:
            out_lse = torch.empty(total_q, hq, device=q.device, dtype=torch.float32)
        _check(out.shape == q.shape and out.dtype == torch.bfloat16 and out.is_contiguous(),
               "out must be a contiguous bf16 tensor shaped like q")
        _check(tuple(out_lse.shape) == (total_q, hq) and out_lse.dtype == torch.float32
               and out_lse.is_contiguous(), "out_lse must be contiguous f32 [total_q,Hq]")
        a = MacWindowAttentionArgs()
        a.struct_size = ctypes.sizeof(MacWindowAttentionArgs)
        a.abi_version = ABI_VERSION
        a.q, a.k_buffer, a.v_buffer = _ptr(q), _ptr(k_buffer), _ptr(v_buffer)
        a.qo_indptr, a.kv_indptr, a.kv_indices = _ptr(qo_indptr), _ptr(kv_indptr), _ptr(kv_indices)
        a.out, a.out_lse = _ptr(out), _ptr(out_lse)
        a.total_q, a.pool_tokens = total_q, int(k_buffer.shape[0])
        a.kv_indices_len = int(kv_indices.shape[0])
        a.B, a.Hq, a.Hkv, a.D = int(qo_indptr.shape[0]) - 1, hq, int(k_buffer.shape[1]), _HEAD_DIM
        a.window_left, a.sm_scale = int(window_left), float(sm_scale)
        with torch.cuda.device(q.device):
            rc = self._lib.mac_prefill_window_attention_bf16(ctypes.byref(a), _stream(q.device))
        _raise_on(self._lib, rc)
        return out, out_lse

    def mac_prefill_rectify_update_cache(self, q_post, src_q, o_full, lse_full, k_buffer, v_buffer,
                                         qo_indptr, kv_indptr, kv_indices, q_cache, attn_cache,
                                         lse_cache, request_length, req_ids, semantic_pos_ahead: int,
                                         front_sink_tokens: int, sm_scale: float, q_post_cache=None,
                                         sink_mode: int = 0) -> None:
        _check_ragged(q_post, k_buffer, v_buffer, qo_indptr, kv_indptr, kv_indices)
        for name, t, dt in (("src_q", src_q, torch.bfloat16), ("o_full", o_full, torch.bfloat16),
                            ("lse_full", lse_full, torch.float32), ("q_cache", q_cache, torch.bfloat16),
                            ("attn_cache", attn_cache, torch.bfloat16),
                            ("lse_cache", lse_cache, torch.float32),
                            ("request_length", request_length, torch.int32),
                            ("req_ids", req_ids, torch.int32)):
            _check(t.is_cuda, f"{name} must be a CUDA tensor")
            _check(t.is_contiguous(), f"{name} must be contiguous")
            _check(t.dtype == dt, f"{name} has wrong dtype")
        _check(src_q.shape == q_post.shape and o_full.shape == q_post.shape,
               "src_q / o_full must match q_post [total_q,Hq,128]")
        total_q, hq, _ = (int(x) for x in q_post.shape)
        _check(tuple(lse_full.shape) == (total_q, hq), "lse_full must be [total_q,Hq]")
        _check(q_cache.dim() == 4 and int(q_cache.shape[2]) == hq and int(q_cache.shape[3]) == _HEAD_DIM,
               "q_cache must be [R,M,Hq,128]")
        _check(attn_cache.shape == q_cache.shape, "attn_cache must match q_cache")
        R, M = int(q_cache.shape[0]), int(q_cache.shape[1])
        _check(tuple(lse_cache.shape) == (R, M, hq), "lse_cache shape mismatch")
        B = int(qo_indptr.shape[0]) - 1
        _check(int(req_ids.shape[0]) == B, "req_ids must be [B]")
        _check(int(request_length.shape[0]) in (R, B), "request_length must be [R] or [B]")
        qpc = None
        if q_post_cache is not None and q_post_cache.numel() > 0:
            _check(q_post_cache.is_cuda and q_post_cache.is_contiguous()
                   and q_post_cache.dtype == torch.bfloat16 and q_post_cache.shape == q_cache.shape,
                   "q_post_cache must be a contiguous bf16 CUDA tensor matching q_cache")
            qpc = q_post_cache
        a = MacRectifyArgs()
        a.struct_size = ctypes.sizeof(MacRectifyArgs)
        a.abi_version = ABI_VERSION
        a.q_post, a.src_q, a.o_full, a.lse_full = _ptr(q_post), _ptr(src_q), _ptr(o_full), _ptr(lse_full)
        a.k_buffer, a.v_buffer = _ptr(k_buffer), _ptr(v_buffer)
        a.qo_indptr, a.kv_indptr, a.kv_indices = _ptr(qo_indptr), _ptr(kv_indptr), _ptr(kv_indices)
        a.q_cache, a.attn_cache, a.lse_cache = _ptr(q_cache), _ptr(attn_cache), _ptr(lse_cache)
        a.q_post_cache = _ptr(qpc)
        a.request_length, a.req_ids = _ptr(request_length), _ptr(req_ids)
        a.total_q, a.pool_tokens = total_q, int(k_buffer.shape[0])
        a.kv_indices_len = int(kv_indices.shape[0])
        a.request_length_len = int(request_length.shape[0])
        a.B, a.R, a.M, a.Hq, a.Hkv, a.D = B, R, M, hq, int(k_buffer.shape[1]), _HEAD_DIM
        a.semantic_pos_ahead, a.front_sink_tokens = int(semantic_pos_ahead), int(front_sink_tokens)
        a.sink_mode, a.sm_scale = int(sink_mode), float(sm_scale)
        with torch.cuda.device(q_post.device):
            rc = self._lib.mac_prefill_rectify_update_cache_bf16(ctypes.byref(a), _stream(q_post.device))
        _raise_on(self._lib, rc)


@lru_cache(maxsize=1)
def load_mac_merge_downdate_cache_extension(verbose: bool = False) -> Any:
    """Reference bridge.py:191-209."""
    return MergeDowndateExtension(load_library())


@lru_cache(maxsize=1)
def load_mac_prefill_rectify_extension(verbose: bool = False) -> Any:
    """No reference counterpart (the reference uses FlashInfer's prefill
    wrapper for the windowed pass)."""
    return PrefillRectifyExtension(load_library())


# ---------------------------------------------------- decode RoPE + scatter ---


class DecodeRopePreserveExtension:
    """Replaces the module built from mac_decode_rope_preserve.cu (reference
    bridge.py:273-290, binding mac_decode_rope_preserve.cu:174-276)."""

    def __init__(self, lib: ctypes.CDLL):
        self._lib = lib

    def mac_decode_rope_preserve_q_bf16(self, q, k, v, q_pre, k_buffer, v_buffer, cos_sin_cache,
                                        positions, cache_locs, head_dim: int, is_neox: bool) -> None:
        """Checks and messages of mac_decode_rope_preserve.cu:158-221."""
        for name, t in (("q", q), ("k", k), ("v", v)):
            _check(t.is_cuda, f"{name} must be CUDA")
            _check(t.dtype == torch.bfloat16, f"{name} has wrong dtype")
            _check(t.dim() == 2, f"{name} must have rank 2")
            _check(t.stride(1) == 1, f"{name} must have contiguous last dimension")
        for name, t in (("q_pre", q_pre), ("k_buffer", k_buffer), ("v_buffer", v_buffer)):
            _check(t.is_cuda, f"{name} must be CUDA")
            _check(t.dtype == torch.bfloat16, f"{name} has wrong dtype")
            _check(t.dim() == 3, f"{name} must have rank 3")
            _check(t.is_contiguous(), f"{name} must be contiguous")
        _check(cos_sin_cache.is_cuda, "cos_sin_cache must be CUDA")
        _check(cos_sin_cache.dtype == torch.float32, "cos_sin_cache has wrong dtype")
        _check(cos_sin_cache.dim() == 2, "cos_sin_cache must have rank 2")
        _check(cos_sin_cache.stride(1) == 1, "cos_sin_cache must have contiguous last dimension")
        _check(positions.is_cuda, "positions must be CUDA")
        _check(cache_locs.is_cuda, "cache_locs must be CUDA")
        _check(positions.dim() == 1, "positions must have rank 1")
        _check(cache_locs.dim() == 1, "cache_locs must have rank 1")
        _check(positions.dtype in (torch.int32, torch.int64), "positions must be int32 or int64")
        _check(cache_locs.dtype in (torch.int32, torch.int64), "cache_locs must be int32 or int64")
        _check(positions.is_contiguous() and cache_locs.is_contiguous(),
               "positions / cache_locs must be contiguous")
        n = int(q.shape[0])
        _check(int(k.shape[0]) == n and int(v.shape[0]) == n, "q/k/v batch mismatch")
        _check(int(positions.shape[0]) >= n and int(cache_locs.shape[0]) >= n, "metadata batch too small")
        head_dim = int(head_dim)
        _check(head_dim > 0 and int(q.shape[1]) % head_dim == 0 and int(k.shape[1]) % head_dim == 0,
               "invalid head_dim")
        hq, hkv = int(q.shape[1]) // head_dim, int(k.shape[1]) // head_dim
        _check(int(v.shape[1]) == hkv * head_dim, "v shape mismatch")
        _check(int(q_pre.shape[0]) >= n and int(q_pre.shape[1]) == hq and int(q_pre.shape[2]) == head_dim,
               "q_pre shape mismatch")
        _check(int(k_buffer.shape[1]) == hkv and int(k_buffer.shape[2]) == head_dim,
               "k_buffer shape mismatch")
        _check(v_buffer.shape == k_buffer.shape, "v_buffer shape mismatch")
        rot = int(cos_sin_cache.shape[1])
        _check(0 < rot <= head_dim and rot % 2 == 0, "invalid rotary_dim")
        if n == 0:
            return
        with torch.cuda.device(q.device):
            rc = self._lib.mac_decode_rope_preserve_q_bf16(
                _ptr(q), int(q.stride(0)), _ptr(k), int(k.stride(0)), _ptr(v), int(v.stride(0)),
                _ptr(q_pre), int(q_pre.shape[0]), _ptr(k_buffer), _ptr(v_buffer), int(k_buffer.shape[0]),
                _ptr(cos_sin_cache), int(cos_sin_cache.shape[0]), int(cos_sin_cache.stride(0)), rot,
                _ptr(positions), int(positions.dtype == torch.int64), _ptr(cache_locs),
                int(cache_locs.dtype == torch.int64), n, hq, hkv, head_dim, int(bool(is_neox)),
                _stream(q.device))
        _raise_on(self._lib, rc)


@lru_cache(maxsize=1)
def load_mac_decode_rope_preserve_extension(verbose: bool = False) -> Any:
    """Reference bridge.py:273-290."""
    return DecodeRopePreserveExtension(load_library())
