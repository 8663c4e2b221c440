"""Serving-side glue around the gfx950 MAC kernels: per-layer ring state,
readiness bookkeeping, workspace sizing and the decode/prefill entry points
that SGLang's attention backend calls.

Behaviour follows attention/src/mac_attention/integrations/sglang/ of the
reference:
  * ``MacMetadata``                 llama_hooks.py:620-889 (MACMetadata)
  * ``preserve_q_before_rope``      llama_hooks.py:510-608
  * ``try_decode_rope_preserve``    llama_hooks.py:115-175
  * ``ensure_persistent_workspace`` flashinfer_hooks.py:1546-1652
  * ready / invalidate / gate       flashinfer_hooks.py:1654-1803
  * ``try_persistent_decode``       flashinfer_hooks.py:1806-2022
  * ``offload_prefill_cache``       flashinfer_hooks.py:2300-2490 (rectification
    + _offload_fast_cache), here one fused kernel call
  * ``flashinfer_forward_decode_around`` flashinfer_hooks.py:2614-2735
Every kernel call goes to libmac_hip.so through ``bridge``; when a gate
fails the functions return ``None`` / ``False`` and the caller keeps SGLang's
own attention, exactly as in the reference.
"""

from __future__ import annotations

import os
import sys
from typing import Any, Optional

import torch

from . import bridge
from .prefill_suffix import build_prefill_suffix_plan, compact_by_segments

_EMPTY = None  # lazily created empty CPU tensor (disables optional kernel inputs)


def _empty() -> torch.Tensor:
    global _EMPTY
    if _EMPTY is None:
        _EMPTY = torch.empty(0)
    return _EMPTY


def _ceil_div(a: int, b: int) -> int:
    return (a + b - 1) // b


def candidate_mode_id(mode: str) -> int:
    """flashinfer_hooks.py:979-980"""
    return 1 if str(mode).strip().lower() == "exclude_recent_right" else 0


def bench_mode_id(mode: str) -> int:
    """flashinfer_hooks.py:1048-1054"""
    text = str(mode).strip().lower().replace("-", "_")
    return {"synthetic_head": 1, "synthetic_group": 2}.get(text, 0)


def is_graph_capturing() -> bool:
    if not torch.cuda.is_available():
        return False
    try:
        return bool(torch.cuda.is_current_stream_capturing())
    except Exception:
        return False


# ------------------------------------------------------------ metadata ----


class MacMetadata:
    """Per-layer MAC state of one attention layer: the request-indexed ring
    caches, readiness/epoch vectors and their host mirror, and the query rows
    preserved before RoPE."""

    def __init__(self, num_heads: int, num_kv_heads: int, head_dim: int):
        self.num_heads = int(num_heads)
        self.num_kv_heads = int(num_kv_heads)
        self.head_dim = int(head_dim)
        self.device: Optional[torch.device] = None
        self.dtype = torch.bfloat16
        self.unified_query_cache: Optional[torch.Tensor] = None
        self.unified_attn_cache: Optional[torch.Tensor] = None
        self.unified_lse_cache: Optional[torch.Tensor] = None
        self.unified_query_post_cache: Optional[torch.Tensor] = None
        self.mac_cache_ready: Optional[torch.Tensor] = None
        self.mac_cache_epoch: Optional[torch.Tensor] = None
        self.request_epoch: Optional[torch.Tensor] = None
        self.mac_cache_ready_host: Optional[list[bool]] = None
        self.mac_low_hit_ejected_host: Optional[list[bool]] = None
        self.req_len: Optional[torch.Tensor] = None
        self.cache_lens: Optional[torch.Tensor] = None
        self.req_ids: Optional[torch.Tensor] = None
        self.req_ids_host: Optional[list[int]] = None
        self.cur_kv_len = 0
        self.cur_q_before_rope: Optional[torch.Tensor] = None
        self.cur_q_before_rope_local_start = 0
        self.cur_q_before_rope_local_len = 0
        self.cur_q_before_rope_compacted = False
        self.decode_q_before_rope_buf: Optional[torch.Tensor] = None
        self.prefill_q_before_rope_buf: Optional[torch.Tensor] = None
        self.prefill_preserve_tail_tokens = 1
        self.cache_ext = None
        self.persistent_decode_ext = None
        self.rect_ext = None
        self.rope_ext = None

    def allocate(self, *, max_running: int, capacity: int, device, dtype=torch.bfloat16,
                 prefill_capacity: int = 1) -> None:
        """Ring caches [max_running, capacity, Hq, D] and the per-request
        vectors (llama_hooks.py:760-870); loads the kernel library."""
        dev = torch.device(device)
        hq, d = self.num_heads, self.head_dim
        self.device, self.dtype = dev, dtype
        self.unified_query_cache = torch.empty((max_running, capacity, hq, d), dtype=dtype, device=dev)
        self.unified_attn_cache = torch.empty_like(self.unified_query_cache)
        self.unified_lse_cache = torch.full((max_running, capacity, hq), float("-inf"), device=dev)
        self.unified_query_post_cache = None
        self.decode_q_before_rope_buf = torch.empty((max_running, hq, d), dtype=dtype, device=dev)
        self.prefill_q_before_rope_buf = torch.empty((max(prefill_capacity, 1), hq, d), dtype=dtype, device=dev)
        self.prefill_preserve_tail_tokens = max(1, capacity)
        i32 = torch.int32
        self.req_len = torch.zeros((max_running,), dtype=i32, device=dev)
        self.cache_lens = torch.zeros((max_running,), dtype=i32, device=dev)
        self.req_ids = torch.zeros((max_running,), dtype=i32, device=dev)
        self.request_epoch = torch.zeros((max_running,), dtype=torch.int64, device=dev)
        self.mac_cache_ready = torch.zeros((max_running,), dtype=torch.bool, device=dev)
        self.mac_cache_epoch = torch.full((max_running,), -1, dtype=torch.int64, device=dev)
        self.mac_cache_ready_host = [False] * max_running
        if dev.type == "cuda":
            self.cache_ext = bridge.load_mac_prefill_update_cache_extension()
            self.persistent_decode_ext = bridge.load_mac_persistent_decode_extension()
            self.rect_ext = bridge.load_mac_prefill_rectify_extension()
            self.rope_ext = bridge.load_mac_decode_rope_preserve_extension()


# ------------------------------------------------------ q preservation ----


def preserve_q_before_rope(metadata: MacMetadata, q: torch.Tensor, current_is_decode: bool,
                           forward_batch: Any = None, graph_safe: bool = False) -> None:
    """Keep the pre-RoPE query rows the ring will store (llama_hooks.py:510-608).

    Decode: all rows, into the persistent decode buffer when it fits.
    Prefill: the rows the scheduler marked for the ring (suffix plan),
    compacted in plan order; without marks, every row; ``graph_safe`` keeps
    only the last ``prefill_preserve_tail_tokens`` rows in the stable prefill
    buffer (the reference's compiled/piecewise-graph branch)."""
    view = q.reshape(q.shape[0], metadata.num_heads, metadata.head_dim)
    rows = int(view.shape[0])
    metadata.cur_q_before_rope_local_start = 0
    metadata.cur_q_before_rope_local_len = rows
    metadata.cur_q_before_rope_compacted = False
    buf = metadata.decode_q_before_rope_buf
    if current_is_decode and buf is not None and buf.device == q.device and buf.dtype == q.dtype \
            and buf.shape[0] >= rows:
        metadata.cur_q_before_rope = buf[:rows]
        metadata.cur_q_before_rope.copy_(view)
        return
    if current_is_decode or forward_batch is None:
        metadata.cur_q_before_rope = view.contiguous().clone()
        return
    pbuf = metadata.prefill_q_before_rope_buf
    usable = pbuf is not None and pbuf.device == q.device and pbuf.dtype == q.dtype
    if graph_safe:
        tail = min(max(1, int(metadata.prefill_preserve_tail_tokens)), rows)
        if usable and pbuf.shape[0] >= tail:
            pbuf[:tail].copy_(view[rows - tail:])
            metadata.cur_q_before_rope = pbuf[:tail]
            metadata.cur_q_before_rope_local_start = rows - tail
            metadata.cur_q_before_rope_local_len = tail
            metadata.cur_q_before_rope_compacted = True
            return
    plan = build_prefill_suffix_plan(forward_batch, int(getattr(forward_batch, "batch_size", 0)), rows,
                                     allow_backend_fallback=False)
    if plan is None:
        start, length, keep = 0, rows, True
    elif plan.total_len <= 0:
        start, length, keep = 0, 0, False
    elif len(plan.segments) == 1 and plan.segments[0].batch_index == 0:
        seg = plan.segments[0]
        try:
            start = max(0, seg.update_start - int(forward_batch.extend_prefix_lens_cpu[0]))
        except Exception:
            start = 0
        length, keep = seg.length, True
    else:
        start, length, keep = -1, int(plan.total_len), True  # several segments: no single range
    metadata.cur_q_before_rope_compacted = plan is not None
    metadata.cur_q_before_rope_local_start = int(start)
    metadata.cur_q_before_rope_local_len = int(length)
    if not keep:
        metadata.cur_q_before_rope = None
        return
    if usable and pbuf.shape[0] >= rows:
        pbuf[:rows].copy_(view)
        metadata.cur_q_before_rope = pbuf
        metadata.cur_q_before_rope_compacted = False
        return
    if plan is not None:
        metadata.cur_q_before_rope = compact_by_segments(view, plan.segments, clone=True)
    elif start == 0 and length == rows:
        metadata.cur_q_before_rope = view.contiguous().clone()
    else:
        metadata.cur_q_before_rope = view[start:start + length].contiguous().clone()


def try_decode_rope_preserve(metadata: MacMetadata, positions: torch.Tensor, q: torch.Tensor,
                             k: torch.Tensor, v: torch.Tensor, k_buffer: torch.Tensor,
                             v_buffer: torch.Tensor, cos_sin_cache: torch.Tensor, cache_loc: torch.Tensor,
                             is_neox: bool) -> bool:
    """Fused decode RoPE + q preserve + KV write (llama_hooks.py:115-175);
    False when a gate fails (the caller then runs its own RoPE and KV write)."""
    if os.environ.get("MAC_USE_FUSED_Q_PRESERVE_ROPE", "1").strip().lower() not in {"1", "true", "yes", "on"}:
        return False
    if any(t.dtype != torch.bfloat16 for t in (q, k, v, k_buffer, v_buffer)):
        return False
    if q.dim() != 2 or k.dim() != 2 or v.dim() != 2:
        return False
    if not torch.is_tensor(cos_sin_cache) or cos_sin_cache.dtype != torch.float32:
        return False
    buf = metadata.decode_q_before_rope_buf
    if buf is None or buf.device != q.device or buf.dtype != q.dtype or buf.shape[0] < q.shape[0]:
        return False
    if metadata.rope_ext is None:
        return False
    q_pre = buf[: q.shape[0]]
    metadata.cur_q_before_rope = q_pre
    metadata.cur_q_before_rope_local_start = 0
    metadata.cur_q_before_rope_local_len = int(q.shape[0])
    metadata.cur_q_before_rope_compacted = False
    metadata.rope_ext.mac_decode_rope_preserve_q_bf16(q, k, v, q_pre, k_buffer, v_buffer, cos_sin_cache,
                                                      positions, cache_loc, metadata.head_dim, bool(is_neox))
    return True


# ------------------------------------------------------------ readiness ----


def _require_kernels(metadata: MacMetadata) -> None:
    if metadata.cache_ext is None:
        raise RuntimeError("MAC ring state lives on a GPU: MacMetadata.allocate() with a CUDA device "
                           "loads the kernel library first")


def _host_req_ids(metadata: MacMetadata, req_ids: torch.Tensor) -> list[int]:
    """Request ids as host ints without a device sync while capturing."""
    if is_graph_capturing() or req_ids.device.type != "cpu":
        host = metadata.req_ids_host
        if host is not None:
            return [int(x) for x in host[: int(req_ids.numel())]]
        if is_graph_capturing():
            return []
    return [int(x) for x in req_ids.detach().cpu().tolist()]


def _low_hit_ejected(metadata: MacMetadata, reqs: list[int]) -> bool:
    ejected = metadata.mac_low_hit_ejected_host
    if ejected is None or is_graph_capturing():
        return False
    return any(r < 0 or r >= len(ejected) or ejected[r] for r in reqs)


def _env_number(name: str, default: float) -> float:
    raw = os.environ.get(name)
    if raw is None or not raw.strip():
        return default
    try:
        return float(raw)
    except ValueError:
        return default


def eject_low_hit_requests(metadata: MacMetadata, workspace: dict, batch_size: int, req_ids: torch.Tensor,
                           past_lens: torch.Tensor) -> bool:
    """The low-hit ejection policy of flashinfer_hooks.py:1500-1543, run after
    a decode step outside graph capture.  With
    ``MAC_ADAPTIVE_LOW_HIT_EJECT_THRESHOLD`` = t in [0, 1] (unset or negative:
    off), a step in which at least the fraction t of the (request, KV head)
    groups did not hit -- and, with ``MAC_ADAPTIVE_LOW_HIT_EJECT_MIN_KV`` = k
    > 0, whose requests all hold at least k cached tokens -- takes its
    requests off the MAC path: their readiness is invalidated and they are
    flagged so that no ring update marks them ready again until their next
    prefill (clear_low_hit_ejection).  ``MAC_ADAPTIVE_LOW_HIT_EJECT_LOG=1``
    prints each ejection.  Reads the step's group modes (one host sync).
    Returns whether the batch was ejected."""
    if is_graph_capturing():
        return False
    threshold = _env_number("MAC_ADAPTIVE_LOW_HIT_EJECT_THRESHOLD", -1.0)
    if threshold < 0.0 or batch_size <= 0:
        return False
    threshold = min(threshold, 1.0)
    min_kv = max(0, int(_env_number("MAC_ADAPTIVE_LOW_HIT_EJECT_MIN_KV", 0)))
    if min_kv > 0 and int(past_lens[:batch_size].min().item()) < min_kv:
        return False
    modes = workspace["group_mode"][:batch_size]
    groups = int(modes.numel())
    if groups == 0:
        return False
    missed = int((modes != 0).sum().item())
    if missed < threshold * groups:
        return False
    if os.environ.get("MAC_ADAPTIVE_LOW_HIT_EJECT_LOG", "0").strip() == "1":
        print(f"[mac_attention] low-hit ejection: {missed}/{groups} groups without a hit "
              f"(threshold {threshold:.3f})", flush=True)
    reqs = _host_req_ids(metadata, req_ids[:batch_size])
    ejected = metadata.mac_low_hit_ejected_host
    rows = len(metadata.mac_cache_ready_host) if metadata.mac_cache_ready_host is not None else 0
    if ejected is None:
        ejected = metadata.mac_low_hit_ejected_host = [False] * rows
    elif len(ejected) < rows:
        ejected.extend([False] * (rows - len(ejected)))
    for r in reqs:
        if 0 <= r < len(ejected):
            ejected[r] = True
    invalidate_persistent_ready(metadata, req_ids[:batch_size])
    return True


def clear_low_hit_ejection(metadata: MacMetadata, reqs: list[int]) -> None:
    """A new prefill of these requests rebuilds their rings: they may use the
    MAC path again (llama_hooks.py:905-918)."""
    ejected = metadata.mac_low_hit_ejected_host
    if ejected is None:
        return
    for r in reqs:
        if 0 <= r < len(ejected):
            ejected[r] = False


def mark_persistent_ready(metadata: MacMetadata, req_ids: torch.Tensor) -> None:
    """flashinfer_hooks.py:1704-1738: the rings of ``req_ids`` now hold
    current rows (cache_epoch <- request_epoch, ready <- 1)."""
    reqs = _host_req_ids(metadata, req_ids)
    if _low_hit_ejected(metadata, reqs):
        return
    if metadata.mac_cache_ready_host is not None:
        for r in reqs:
            if 0 <= r < len(metadata.mac_cache_ready_host):
                metadata.mac_cache_ready_host[r] = True
    if metadata.mac_cache_ready is None or metadata.mac_cache_epoch is None or metadata.request_epoch is None:
        return
    _require_kernels(metadata)
    metadata.cache_ext.mac_mark_persistent_ready(metadata.mac_cache_ready, metadata.mac_cache_epoch,
                                                 metadata.request_epoch, req_ids)


def invalidate_persistent_ready(metadata: MacMetadata, req_ids: torch.Tensor) -> None:
    """flashinfer_hooks.py:1741-1777: ready <- 0, cache_epoch <- -1,
    request_epoch += 1 for ``req_ids`` (a graph replay then demotes them)."""
    if metadata.mac_cache_ready_host is not None:
        for r in _host_req_ids(metadata, req_ids):
            if 0 <= r < len(metadata.mac_cache_ready_host):
                metadata.mac_cache_ready_host[r] = False
    if metadata.mac_cache_ready is None or metadata.mac_cache_epoch is None or metadata.request_epoch is None:
        return
    _require_kernels(metadata)
    metadata.cache_ext.mac_invalidate_persistent_ready(metadata.mac_cache_ready, metadata.mac_cache_epoch,
                                                       metadata.request_epoch, req_ids)


def persistent_ready(metadata: MacMetadata, req_ids: torch.Tensor) -> bool:
    """flashinfer_hooks.py:1780-1803: True when every request's ring is
    current.  While capturing a graph the in-kernel gate decides instead."""
    if is_graph_capturing():
        return True
    n = int(req_ids.numel())
    host_ids = metadata.req_ids_host
    if _low_hit_ejected(metadata, [int(x) for x in host_ids[:n]] if host_ids is not None else []):
        return False
    ready_host = metadata.mac_cache_ready_host
    if ready_host is not None and host_ids is not None:
        return all(0 <= int(r) < len(ready_host) and ready_host[int(r)] for r in host_ids[:n])
    if metadata.mac_cache_ready is None or metadata.mac_cache_epoch is None or metadata.request_epoch is None:
        return False
    idx = req_ids.long()
    ok = metadata.mac_cache_ready[idx] & (metadata.mac_cache_epoch[idx] == metadata.request_epoch[idx])
    return bool(torch.all(ok).item())


# ------------------------------------------------------------ workspace ----


def ensure_persistent_workspace(backend: Any, metadata: MacMetadata, config: Any,
                                batch_size: int) -> dict[str, torch.Tensor]:
    """The 30 workspace tensors of mac_persistent_decode_bf16, sized as
    flashinfer_hooks.py:1546-1652 sizes them and cached on ``backend`` until
    a size input changes."""
    max_running = int(max(batch_size, getattr(config, "max_running_requests", 0) or 0,
                          metadata.unified_query_cache.shape[0]))
    hq, hkv, d = metadata.num_heads, metadata.num_kv_heads, metadata.head_dim
    group = hq // hkv
    m = int(config.mac_lookback_tokens_left)
    tile = int(config.mac_persistent_tile_tokens)
    match_tile = int(config.mac_persistent_match_tile_slots)
    max_context = int(config.mac_persistent_max_context)
    sink = max(int(getattr(config, "mac_front_sink_tokens", 0)), 0)
    match_tiles = _ceil_div(m, match_tile)
    tiles_ctx = _ceil_div(max_context, tile) + _ceil_div(sink, tile)
    tiles_red = _ceil_div(tiles_ctx, 32)
    tiles_tail = max(1, _ceil_div(max(int(config.mac_semantic_pos_ahead), 1), tile))
    pdt = torch.float32 if bool(config.mac_persistent_partial_fp32) else torch.bfloat16
    dev = metadata.device
    key = (dev, max_running, hq, hkv, d, m, max_context, tile, match_tile, sink, pdt)
    ws = getattr(backend, "mac_persistent_workspace", None)
    if ws is not None and getattr(backend, "mac_persistent_workspace_key", None) == key:
        return ws
    i32, f32 = torch.int32, torch.float32

    def e(*shape, dtype=i32):
        return torch.empty(shape, device=dev, dtype=dtype)

    ws = {"match_dist": e(max_running, hq, match_tiles, dtype=f32),
          "match_pos": e(max_running, hq, match_tiles), "match_slot": e(max_running, hq, match_tiles)}
    for name in ("hit", "match_slot", "match_pos", "prefix_end", "rect_start", "new_end"):
        ws["head_" + name] = e(max_running, hq)
    for name in ("rect_begin", "rect_end", "rect_tiles", "tail_begin", "tail_end", "tail_tiles", "mode"):
        ws["group_" + name] = e(max_running, hkv)
    ws.update({
        # the reference's size, at least the 2 N Hkv + 6 entries this build's kernels use
        "complete_task_go": e(max(max_running * hq * tiles_ctx, 2 * max_running * hkv + 6)),
        "complete_task_tile": e(max(max_running * hq * tiles_ctx, 2 * max_running * hkv + 6)),
        "tail_task_go": e(max_running * hkv * tiles_tail), "tail_task_tile": e(max_running * hkv * tiles_tail),
        "hit_tail_task_ho": e(max_running * hq * tiles_tail), "hit_tail_task_tile": e(max_running * hq * tiles_tail),
        "task_counts": e(9),
        "partial_rect_o": e(max_running, hkv, tiles_ctx, group, d, dtype=pdt),
        "partial_rect_lse": e(max_running, hkv, tiles_ctx, group, dtype=f32),
        "partial_rect_reduced_o": e(max_running, hkv, tiles_red, group, d, dtype=pdt),
        "partial_rect_reduced_lse": e(max_running, hkv, tiles_red, group, dtype=f32),
        "partial_tail_o": e(max_running, hkv, tiles_tail, group, d, dtype=pdt),
        "partial_tail_lse": e(max_running, hkv, tiles_tail, group, dtype=f32),
        "phase_cycles": e(14, dtype=torch.int64),
    })
    backend.mac_persistent_workspace_key = key
    backend.mac_persistent_workspace = ws
    return ws


WORKSPACE_ORDER = (
    "match_dist", "match_pos", "match_slot", "head_hit", "head_match_slot", "head_match_pos",
    "head_prefix_end", "head_rect_start", "head_new_end", "group_rect_begin", "group_rect_end",
    "group_rect_tiles", "group_tail_begin", "group_tail_end", "group_tail_tiles", "group_mode",
    "complete_task_go", "complete_task_tile", "tail_task_go", "tail_task_tile", "hit_tail_task_ho",
    "hit_tail_task_tile", "task_counts", "partial_rect_o", "partial_rect_lse", "partial_rect_reduced_o",
    "partial_rect_reduced_lse", "partial_tail_o", "partial_tail_lse", "phase_cycles",
)


# --------------------------------------------------------------- decode ----


def _model_context_len(backend: Any) -> int:
    try:
        return int(getattr(getattr(getattr(backend, "model_runner", None), "model_config", None),
                           "context_len", 0) or 0)
    except Exception:
        return 0


def try_persistent_decode(backend: Any, forward_batch: Any, config: Any, metadata: MacMetadata,
                          q_input: torch.Tensor, k_buffer: torch.Tensor, v_buffer: torch.Tensor,
                          cache_loc: torch.Tensor, layer: Any) -> Optional[torch.Tensor]:
    """One fused MAC decode step for the batch, or ``None`` when a gate of
    flashinfer_hooks.py:1806-1907 fails (the caller then runs its own decode
    attention).  q_input [B, Hq, 128] bf16 post-RoPE; the pre-RoPE rows come
    from ``metadata.cur_q_before_rope``."""
    if not config.mac_persistent_coop or metadata.persistent_decode_ext is None:
        return None
    if str(config.mac_persistent_cache_layout).strip().lower() != "slot_major":
        return None
    if str(config.mac_persistent_candidate_mode).strip().lower() not in {"last_m", "exclude_recent_right"}:
        return None
    if q_input.dtype is not torch.bfloat16 or k_buffer.dtype is not torch.bfloat16:
        return None
    if q_input.dim() != 3 or k_buffer.dim() != 3 or v_buffer.dim() != 3:
        return None
    batch = int(forward_batch.batch_size)
    if batch <= 0 or q_input.shape[0] != batch or int(q_input.shape[2]) != 128:
        return None
    if is_graph_capturing():
        # a captured step replays for every later batch of this size: only
        # capture when the model's whole context fits the workspace
        ctx = _model_context_len(backend)
        if ctx <= 0 or ctx > int(config.mac_persistent_max_context):
            print(f"[mac_attention] persistent decode NOT captured into the graph: model context_len={ctx} "
                  f"exceeds mac_persistent_max_context={int(config.mac_persistent_max_context)} (or is "
                  "unknown); raise MAC_PERSISTENT_MAX_CONTEXT to enable.", file=sys.stderr, flush=True)
            return None
    if int(getattr(metadata, "cur_kv_len", 0) or 0) > int(config.mac_persistent_max_context):
        return None
    hq, hkv = int(q_input.shape[1]), int(k_buffer.shape[1])
    if hkv <= 0 or hq % hkv != 0 or hq // hkv > 8:
        return None
    if int(getattr(layer, "logit_cap", 0) or 0) != 0:
        return None
    if getattr(layer, "k_scale_float", None) is not None or getattr(layer, "v_scale_float", None) is not None:
        return None
    req_to_token = None  # FlashInfer: on its decode index updater; Triton / aiter: on the backend
    for owner in (getattr(backend, "indices_updater_decode", None), backend,
                  getattr(forward_batch, "req_to_token_pool", None)):
        req_to_token = getattr(owner, "req_to_token", None) if owner is not None else None
        if torch.is_tensor(req_to_token):
            break
    if not torch.is_tensor(req_to_token) or req_to_token.dtype != torch.int32 or not req_to_token.is_contiguous():
        return None
    req_ids = metadata.req_ids[:batch]
    past_lens = metadata.cache_lens[:batch]
    if req_ids.dtype != torch.int32 or not req_ids.is_contiguous():
        return None
    if past_lens.dtype != torch.int32 or not past_lens.is_contiguous():
        return None
    if not torch.is_tensor(cache_loc) or cache_loc.dtype not in (torch.int32, torch.int64) \
            or not cache_loc.is_contiguous():
        return None
    if not persistent_ready(metadata, req_ids):
        return None
    q_input = q_input.contiguous()
    if metadata.cur_q_before_rope is None:
        return None
    q_pre = metadata.cur_q_before_rope[:batch].contiguous()
    ws = ensure_persistent_workspace(backend, metadata, config, batch)
    out = torch.empty_like(q_input)
    optional_lse = torch.empty((0,), device=q_input.device, dtype=torch.float32)
    qpc = metadata.unified_query_post_cache
    if qpc is None:
        qpc = metadata.unified_query_cache.new_empty((0,))
    metadata.persistent_decode_ext.mac_persistent_decode_bf16(
        q_input, q_pre, k_buffer, v_buffer, req_to_token, req_ids, past_lens, cache_loc,
        metadata.unified_query_cache, metadata.unified_attn_cache, metadata.unified_lse_cache, out, optional_lse,
        *[ws[name] for name in WORKSPACE_ORDER],
        int(config.mac_persistent_max_context), int(config.mac_persistent_tile_tokens),
        int(config.mac_persistent_match_tile_slots), int(config.mac_semantic_pos_ahead),
        int(getattr(config, "mac_front_sink_tokens", 0)), int(config.mac_gen_min_limit),
        int(config.mac_lookback_tokens_right), candidate_mode_id(config.mac_persistent_candidate_mode),
        float(config.mac_threshold), float(layer.scaling), int(config.mac_persistent_debug),
        bench_mode_id(getattr(config, "mac_bench_mode", "off")), float(getattr(config, "mac_bench_hit_rate", 1.0)),
        float(getattr(config, "mac_bench_hit_rate_std", 0.0)), float(getattr(config, "mac_bench_skip_ratio", -1.0)),
        float(getattr(config, "mac_bench_skip_ratio_std", 0.0)),
        float(getattr(config, "mac_bench_match_lag_mean", 64.0)),
        float(getattr(config, "mac_bench_match_lag_std", 0.0)), int(getattr(config, "mac_bench_seed", 1)), -1,
        int(getattr(layer, "layer_id", 0)), qpc,
        # the in-kernel gate demotes requests whose ring is not current, also
        # on graph replays where the Python gate above does not run
        metadata.mac_cache_ready if metadata.mac_cache_ready is not None else _empty(),
        metadata.mac_cache_epoch if metadata.mac_cache_epoch is not None else _empty(),
        metadata.request_epoch if metadata.request_epoch is not None else _empty())
    eject_low_hit_requests(metadata, ws, batch, req_ids, past_lens)
    backend.mac_last_persistent_workspace = ws
    return out


def supports_mac_backend(backend: Any, layer: Any, forward_batch: Any, config: Any) -> bool:
    """flashinfer_hooks.py:916-936"""
    if not config.enable_mac:
        return False
    if getattr(backend, "num_wrappers", 1) != 1:
        return False
    if getattr(layer, "is_cross_attention", False):
        return False
    if getattr(layer, "sliding_window_size", -1) not in (-1, None):
        return False
    if getattr(getattr(layer, "attn_type", None), "value", "decoder") != "decoder":
        return False
    if getattr(forward_batch, "spec_info", None) is not None:
        return False
    metadata = getattr(layer, "mac_metadata", None)
    return metadata is not None and metadata.unified_query_cache is not None


def flashinfer_forward_decode_around(original_fn: Any, self: Any, q: torch.Tensor, k: torch.Tensor,
                                     v: torch.Tensor, layer: Any, forward_batch: Any,
                                     save_kv_cache: bool = True, **kwargs: Any) -> Any:
    """Around-hook of FlashInferAttnBackend.forward_decode
    (flashinfer_hooks.py:2614-2735), and of the ROCm backends'
    (AiterAttnBackend, TritonAttnBackend): write K/V, try the fused MAC step,
    else invalidate the batch's rings and run the backend's own decode."""
    from .config import get_mac_config

    config = getattr(layer, "mac_config", None) or getattr(self, "mac_config", None) or get_mac_config()
    if not supports_mac_backend(self, layer, forward_batch, config):
        record_decode_graph_capture(self, forward_batch, persistent=False)
        return original_fn(self, q, k, v, layer, forward_batch, save_kv_cache=save_kv_cache, **kwargs)
    metadata: MacMetadata = layer.mac_metadata
    cache_loc = forward_batch.out_cache_loc
    if k is not None and save_kv_cache:
        forward_batch.token_to_kv_pool.set_kv_buffer(layer, cache_loc, k, v, layer.k_scale, layer.v_scale)
    q_input = q.view(-1, layer.tp_q_head_num, layer.head_dim)
    k_buffer, v_buffer = forward_batch.token_to_kv_pool.get_kv_buffer(layer.layer_id)
    out = try_persistent_decode(self, forward_batch, config, metadata, q_input, k_buffer, v_buffer, cache_loc,
                                layer)
    record_decode_graph_capture(self, forward_batch, persistent=out is not None)
    if out is not None:
        return out.view(-1, layer.tp_q_head_num * layer.head_dim)
    invalidate_persistent_ready(metadata, metadata.req_ids[: int(forward_batch.batch_size)])
    return original_fn(self, q, k, v, layer, forward_batch, save_kv_cache=False, **kwargs)


# ----------------------------------------------------- decode graphs ----
#
# flashinfer_hooks.py:660-700, :835-899.  While SGLang captures a decode
# graph for a batch size, every layer's decode hook records whether it
# captured the MAC step or the backend's own decode.  When every layer of
# that graph is the MAC step, a replay needs none of the backend's decode
# metadata (the MAC kernels read the request tables and lengths themselves,
# and demote requests whose ring is not current inside the graph), so the
# backend's per-replay metadata update is skipped
# (MAC_CUDAGRAPH_SKIP_FLASHINFER_REPLAY_METADATA, default on, the
# reference's switch).  The reference's other replay duty -- waiting for
# prefill ring updates on a side stream -- has nothing to wait for here: the
# ring update runs on the compute stream, in order with the replay.


def skip_replay_metadata_enabled() -> bool:
    raw = os.environ.get("MAC_CUDAGRAPH_SKIP_FLASHINFER_REPLAY_METADATA", "1")
    return raw.strip().lower() in {"1", "true", "yes", "on"}


def decode_graph_states(backend: Any) -> dict:
    states = getattr(backend, "mac_cudagraph_decode_states", None)
    if not isinstance(states, dict):
        states = {}
        backend.mac_cudagraph_decode_states = states
    return states


def record_decode_graph_capture(backend: Any, forward_batch: Any, *, persistent: bool) -> None:
    """During a graph capture: which decode path this layer captured."""
    if not is_graph_capturing():
        return
    try:
        bs = int(getattr(forward_batch, "batch_size", 0))
    except Exception:
        return
    if bs <= 0:
        return
    state = decode_graph_states(backend).setdefault(bs, {"persistent_seen": False, "fallback_seen": False})
    state["persistent_seen" if persistent else "fallback_seen"] = True


def _graph_args(args: tuple, kwargs: dict) -> tuple:
    """(bs, forward_mode) of init_forward_metadata_capture/replay_cuda_graph:
    SGLang passes bs first and forward_mode sixth."""
    bs = args[0] if len(args) > 0 else kwargs.get("bs")
    mode = args[5] if len(args) > 5 else kwargs.get("forward_mode")
    try:
        decode = bool(mode.is_decode_or_idle())
    except Exception:
        decode = False
    return bs, decode


def init_forward_metadata_capture_cuda_graph_around(original_fn: Any, self: Any, *args: Any, **kwargs: Any) -> Any:
    """A decode graph is about to be captured for batch size bs: forget what
    an earlier capture of that size recorded."""
    from .config import get_mac_config

    bs, decode = _graph_args(args, kwargs)
    config = getattr(self, "mac_config", None) or get_mac_config()
    if skip_replay_metadata_enabled() and config.enable_mac and decode and bs is not None:
        decode_graph_states(self)[int(bs)] = {"persistent_seen": False, "fallback_seen": False}
    return original_fn(self, *args, **kwargs)


def init_forward_metadata_replay_cuda_graph_around(original_fn: Any, self: Any, *args: Any, **kwargs: Any) -> Any:
    """Skip the backend's replay metadata for decode graphs whose every layer
    captured the MAC step."""
    from .config import get_mac_config

    bs, decode = _graph_args(args, kwargs)
    if skip_replay_metadata_enabled() and bs is not None and decode:
        config = getattr(self, "mac_config", None) or get_mac_config()
        state = getattr(self, "mac_cudagraph_decode_states", {}).get(int(bs), {})
        if config.enable_mac and state.get("persistent_seen", False) and not state.get("fallback_seen", False):
            return None
    return original_fn(self, *args, **kwargs)


# -------------------------------------------------------------- prefill ----


def offload_prefill_cache(metadata: MacMetadata, config: Any, *, q_post: torch.Tensor, o_full: torch.Tensor,
                          lse_full: torch.Tensor, k_buffer: torch.Tensor, v_buffer: torch.Tensor,
                          qo_indptr: torch.Tensor, kv_indptr: torch.Tensor, kv_indices: torch.Tensor,
                          req_ids: torch.Tensor, prefix_lens: torch.Tensor, sm_scale: float,
                          sink_mode: int = 0) -> None:
    """Ring update after a prefill chunk (flashinfer_hooks.py:2300-2490):
    rectify the kept rows (full state minus the last S keys), store them with
    the preserved pre-RoPE queries, then mark the requests ready.  One fused
    kernel call replaces the reference's windowed FlashInfer pass, downdate
    and _offload_fast_cache.  ``prefix_lens`` [B] are the tokens each request
    had before the chunk (the ring's row index base); ``lse_full`` is the
    full-attention lse in natural log."""
    src_q = metadata.cur_q_before_rope
    if src_q is None or src_q.shape[0] != q_post.shape[0]:
        invalidate_persistent_ready(metadata, req_ids)
        return
    if int(config.mac_semantic_pos_ahead) <= 0:
        invalidate_persistent_ready(metadata, req_ids)
        return
    request_length = metadata.req_len.clone()
    request_length[req_ids.long()] = prefix_lens.to(torch.int32)
    metadata.rect_ext.mac_prefill_rectify_update_cache(
        q_post.contiguous(), src_q.contiguous(), o_full.contiguous(), lse_full.contiguous(), k_buffer, v_buffer,
        qo_indptr, kv_indptr, kv_indices, metadata.unified_query_cache, metadata.unified_attn_cache,
        metadata.unified_lse_cache, request_length, req_ids, int(config.mac_semantic_pos_ahead),
        int(getattr(config, "mac_front_sink_tokens", 0)), float(sm_scale),
        q_post_cache=metadata.unified_query_post_cache, sink_mode=sink_mode)
    metadata.req_len.copy_(request_length)
    mark_persistent_ready(metadata, req_ids)
