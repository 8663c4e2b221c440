"""ctypes wrapper around the CPU oracle ``libmac_oracle.so``.

TEST INFRASTRUCTURE ONLY: imported by tests/, ``__graft_entry__.smoke()`` and
the ``cpu_baseline`` leg of ``bench.py``.  The product path never imports it.

All arrays are numpy; bf16 tensors travel as ``uint16`` bit patterns.  The
helpers ``bf16_bits``/``bits_to_float`` convert between float32 and bf16 bits
with round-to-nearest-even.  The restated algorithm and its reference
citations live in ``mac_oracle.c``.
"""

from __future__ import annotations

import ctypes
import os
import subprocess
from dataclasses import dataclass, field

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "libmac_oracle.so")
_lib = None


def build() -> str:
    """Compile the oracle with gcc (make)."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH) or os.path.getmtime(_LIB_PATH) < os.path.getmtime(
            os.path.join(_HERE, "mac_oracle.c")
        ):
            build()
        _lib = ctypes.CDLL(_LIB_PATH)
        _lib.mac_oracle_decode.restype = ctypes.c_int
        _lib.mac_oracle_ring_slot_to_pos.restype = ctypes.c_int
        _lib.mac_oracle_pos_to_ring_slot.restype = ctypes.c_int
        _lib.mac_oracle_span_attention.restype = ctypes.c_double
        _lib.mac_oracle_prefill_update_cache.restype = ctypes.c_int
    return _lib


# ----------------------------------------------------------------- bf16 ----


def bf16_bits(x: np.ndarray) -> np.ndarray:
    """float32 -> bf16 bit patterns (uint16), round to nearest even."""
    f = np.ascontiguousarray(x, dtype=np.float32)
    u = f.view(np.uint32).astype(np.uint64)
    nan = (u & 0x7F800000) == 0x7F800000
    nan &= (u & 0x007FFFFF) != 0
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    r = np.where(nan, ((u >> 16) | 0x40).astype(np.uint16), r)
    return r.astype(np.uint16)


def bits_to_float(b: np.ndarray) -> np.ndarray:
    """bf16 bit patterns -> float32."""
    return (np.ascontiguousarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


# ------------------------------------------------------------ structures ---

_i32p = ctypes.POINTER(ctypes.c_int32)
_i64p = ctypes.POINTER(ctypes.c_int64)
_u16p = ctypes.POINTER(ctypes.c_uint16)
_u8p = ctypes.POINTER(ctypes.c_uint8)
_f32p = ctypes.POINTER(ctypes.c_float)
_f64p = ctypes.POINTER(ctypes.c_double)


class _DecodeArgs(ctypes.Structure):
    _fields_ = [
        ("N", ctypes.c_int), ("Hq", ctypes.c_int), ("Hkv", ctypes.c_int), ("D", ctypes.c_int),
        ("M", ctypes.c_int), ("R", ctypes.c_int), ("req_to_token_stride", ctypes.c_int),
        ("q_post", _u16p), ("q_pre", _u16p), ("k_buffer", _u16p), ("v_buffer", _u16p),
        ("req_to_token", _i32p), ("req_ids", _i32p), ("past_lens", _i32p),
        ("out_cache_loc", _i64p),
        ("query_cache", _u16p), ("attn_cache", _u16p), ("lse_cache", _f32p),
        ("cache_ready", _u8p), ("cache_epoch", _i64p), ("request_epoch", _i64p),
        ("out", _u16p), ("out_lse", _f32p),
        ("head_hit", _i32p), ("head_match_slot", _i32p), ("head_match_pos", _i32p),
        ("head_prefix_end", _i32p), ("head_rect_start", _i32p), ("head_new_end", _i32p),
        ("head_best_dist", _f64p),
        ("group_mode", _i32p), ("group_rect_begin", _i32p), ("group_rect_end", _i32p),
        ("group_tail_begin", _i32p), ("group_tail_end", _i32p),
        ("semantic_pos_ahead", ctypes.c_int), ("front_sink_tokens", ctypes.c_int),
        ("gen_min_limit", ctypes.c_int), ("lookback_right", ctypes.c_int),
        ("candidate_mode", ctypes.c_int),
        ("threshold", ctypes.c_float), ("sm_scale", ctypes.c_float),
        ("mixed_group_fallback", ctypes.c_int),
        ("bench_mode", ctypes.c_int), ("bench_exact_quota", ctypes.c_int),
        ("bench_seed", ctypes.c_int), ("bench_miss_mask", ctypes.c_int),
        ("bench_layer_id", ctypes.c_int),
        ("bench_hit_rate", ctypes.c_float), ("bench_hit_rate_std", ctypes.c_float),
        ("bench_skip_ratio", ctypes.c_float), ("bench_skip_ratio_std", ctypes.c_float),
        ("bench_match_lag_mean", ctypes.c_float), ("bench_match_lag_std", ctypes.c_float),
    ]


def _ptr(a, t):
    if a is None:
        return ctypes.cast(None, t)
    assert a.flags["C_CONTIGUOUS"], "oracle arrays must be contiguous"
    return a.ctypes.data_as(t)


@dataclass
class DecodeParams:
    semantic_pos_ahead: int
    front_sink_tokens: int = 0
    gen_min_limit: int = 0
    lookback_right: int = 0
    candidate_mode: int = 0
    threshold: float = 0.45
    sm_scale: float = 1.0 / np.sqrt(128.0)
    mixed_group_fallback: int = 1
    bench_mode: int = 0
    bench_exact_quota: int = 1
    bench_seed: int = 1
    bench_miss_mask: int = -1
    bench_layer_id: int = 0
    bench_hit_rate: float = 1.0
    bench_hit_rate_std: float = 0.0
    bench_skip_ratio: float = -1.0
    bench_skip_ratio_std: float = 0.0
    bench_match_lag_mean: float = 64.0
    bench_match_lag_std: float = 0.0


@dataclass
class DecodeResult:
    out: np.ndarray  # uint16 [N,Hq,D]
    out_lse: np.ndarray  # f32 [N,Hq]
    query_cache: np.ndarray
    attn_cache: np.ndarray
    lse_cache: np.ndarray
    head: dict = field(default_factory=dict)
    group: dict = field(default_factory=dict)


def decode(
    *,
    q_post, q_pre, k_buffer, v_buffer, req_to_token, req_ids, past_lens, out_cache_loc,
    query_cache, attn_cache, lse_cache, params: DecodeParams,
    cache_ready=None, cache_epoch=None, request_epoch=None,
) -> DecodeResult:
    """Run one MAC decode step on the CPU.  Ring caches are copied, not mutated."""
    L = lib()
    c = np.ascontiguousarray
    q_post = c(q_post, dtype=np.uint16)
    q_pre = c(q_pre, dtype=np.uint16)
    k_buffer = c(k_buffer, dtype=np.uint16)
    v_buffer = c(v_buffer, dtype=np.uint16)
    req_to_token = c(req_to_token, dtype=np.int32)
    req_ids = c(req_ids, dtype=np.int32)
    past_lens = c(past_lens, dtype=np.int32)
    out_cache_loc = c(out_cache_loc, dtype=np.int64)
    qc = np.array(query_cache, dtype=np.uint16, copy=True, order="C")
    ac = np.array(attn_cache, dtype=np.uint16, copy=True, order="C")
    lc = np.array(lse_cache, dtype=np.float32, copy=True, order="C")
    N, Hq, D = q_post.shape
    Hkv = k_buffer.shape[1]
    R, M = qc.shape[0], qc.shape[1]
    out = np.zeros((N, Hq, D), np.uint16)
    out_lse = np.zeros((N, Hq), np.float32)
    head = {k: np.zeros((N, Hq), np.int32) for k in
            ("hit", "match_slot", "match_pos", "prefix_end", "rect_start", "new_end")}
    head["best_dist"] = np.zeros((N, Hq), np.float64)
    group = {k: np.zeros((N, Hkv), np.int32) for k in
             ("mode", "rect_begin", "rect_end", "tail_begin", "tail_end")}
    if cache_ready is not None:
        cache_ready = c(cache_ready, dtype=np.uint8)
    if cache_epoch is not None:
        cache_epoch = c(cache_epoch, dtype=np.int64)
    if request_epoch is not None:
        request_epoch = c(request_epoch, dtype=np.int64)
    p = params
    a = _DecodeArgs(
        N, Hq, Hkv, D, M, R, req_to_token.shape[1],
        _ptr(q_post, _u16p), _ptr(q_pre, _u16p), _ptr(k_buffer, _u16p), _ptr(v_buffer, _u16p),
        _ptr(req_to_token, _i32p), _ptr(req_ids, _i32p), _ptr(past_lens, _i32p),
        _ptr(out_cache_loc, _i64p),
        _ptr(qc, _u16p), _ptr(ac, _u16p), _ptr(lc, _f32p),
        _ptr(cache_ready, _u8p), _ptr(cache_epoch, _i64p), _ptr(request_epoch, _i64p),
        _ptr(out, _u16p), _ptr(out_lse, _f32p),
        _ptr(head["hit"], _i32p), _ptr(head["match_slot"], _i32p), _ptr(head["match_pos"], _i32p),
        _ptr(head["prefix_end"], _i32p), _ptr(head["rect_start"], _i32p),
        _ptr(head["new_end"], _i32p), _ptr(head["best_dist"], _f64p),
        _ptr(group["mode"], _i32p), _ptr(group["rect_begin"], _i32p),
        _ptr(group["rect_end"], _i32p), _ptr(group["tail_begin"], _i32p),
        _ptr(group["tail_end"], _i32p),
        p.semantic_pos_ahead, p.front_sink_tokens, p.gen_min_limit, p.lookback_right,
        p.candidate_mode, p.threshold, p.sm_scale, p.mixed_group_fallback,
        p.bench_mode, p.bench_exact_quota, p.bench_seed, p.bench_miss_mask, p.bench_layer_id,
        p.bench_hit_rate, p.bench_hit_rate_std, p.bench_skip_ratio, p.bench_skip_ratio_std,
        p.bench_match_lag_mean, p.bench_match_lag_std,
    )
    # keep the arrays alive for the duration of the call
    a._keep = (q_post, q_pre, k_buffer, v_buffer, req_to_token, req_ids, past_lens,
               out_cache_loc, cache_ready, cache_epoch, request_epoch)
    rc = L.mac_oracle_decode(ctypes.byref(a))
    if rc != 0:
        raise ValueError(f"mac_oracle_decode failed with code {rc}")
    return DecodeResult(out, out_lse, qc, ac, lc, head, group)


def ring_slot_to_pos(past_len: int, M: int, slot: int) -> int:
    return lib().mac_oracle_ring_slot_to_pos(past_len, M, slot)


def pos_to_ring_slot(past_len: int, M: int, pos: int) -> int:
    return lib().mac_oracle_pos_to_ring_slot(past_len, M, pos)


def prefill_update_cache(q_cache, attn_cache, lse_cache, request_length, req_ids, src_q,
                         src_attn, src_lse, offsets, lens, capacity, num_heads, head_dim,
                         q_post_cache=None):
    """In-place restatement of ``mac_prefill_update_cache`` on numpy arrays."""
    for arr, dt in ((q_cache, np.uint16), (attn_cache, np.uint16), (lse_cache, np.float32),
                    (request_length, np.int32)):
        assert arr.dtype == dt and arr.flags["C_CONTIGUOUS"]
    if q_post_cache is not None:
        assert q_post_cache.dtype == np.uint16 and q_post_cache.flags["C_CONTIGUOUS"]
    c = np.ascontiguousarray
    req_ids = c(req_ids, dtype=np.int32)
    src_q = c(src_q, dtype=np.uint16)
    src_attn = c(src_attn, dtype=np.uint16)
    src_lse = c(src_lse, dtype=np.float32)
    offsets = c(offsets, dtype=np.int32)
    lens = c(lens, dtype=np.int32)
    rc = lib().mac_oracle_prefill_update_cache(
        _ptr(q_cache, _u16p), _ptr(attn_cache, _u16p), _ptr(lse_cache, _f32p),
        _ptr(request_length, _i32p), int(request_length.shape[0]), _ptr(req_ids, _i32p),
        int(req_ids.shape[0]), _ptr(src_q, _u16p), _ptr(src_attn, _u16p), _ptr(src_lse, _f32p),
        int(src_q.shape[0]), _ptr(offsets, _i32p), _ptr(lens, _i32p), int(q_cache.shape[0]),
        int(capacity), int(num_heads), int(head_dim), _ptr(q_post_cache, _u16p))
    if rc != 0:
        raise ValueError(f"mac_oracle_prefill_update_cache failed with code {rc}")


def mark_ready(ready, cache_epoch, request_epoch, req_ids):
    req_ids = np.ascontiguousarray(req_ids, dtype=np.int32)
    lib().mac_oracle_mark_ready(_ptr(ready, _u8p), _ptr(cache_epoch, _i64p),
                                _ptr(request_epoch, _i64p), _ptr(req_ids, _i32p),
                                int(req_ids.shape[0]), int(ready.shape[0]))


def invalidate_ready(ready, cache_epoch, request_epoch, req_ids):
    req_ids = np.ascontiguousarray(req_ids, dtype=np.int32)
    lib().mac_oracle_invalidate_ready(_ptr(ready, _u8p), _ptr(cache_epoch, _i64p),
                                      _ptr(request_epoch, _i64p), _ptr(req_ids, _i32p),
                                      int(req_ids.shape[0]), int(ready.shape[0]))


def update_request_state(req_len, match_req_len, cache_lens, req_ids, seq_lens, cur_lens):
    c = np.ascontiguousarray
    req_ids = c(req_ids, dtype=np.int32)
    seq_lens = c(seq_lens, dtype=np.int32)
    cur_lens = c(cur_lens, dtype=np.int32)
    lib().mac_oracle_update_request_state(
        _ptr(req_len, _i32p), _ptr(match_req_len, _i32p), _ptr(cache_lens, _i32p),
        _ptr(req_ids, _i32p), _ptr(seq_lens, _i32p), _ptr(cur_lens, _i32p),
        int(req_ids.shape[0]), int(req_len.shape[0]))


# ------------------------------------------------- prefill rectification ---

_LSE_CODES = {np.dtype(np.float32): 0, "bf16": 1, np.dtype(np.float16): 2}


def update_then_downdate(out1, lse1, out2, lse2, *, lse1_bf16=False, lse2_bf16=False):
    """In-place restatement of ``mac_update_then_downdate_bf16_inplace`` on
    numpy arrays: out1/out2 uint16 bf16 bits [..., D]; lse arrays float32,
    float16, or uint16 bf16 bits (flagged by ``lse*_bf16``).  Writes out2/lse2."""
    assert out1.dtype == np.uint16 and out2.dtype == np.uint16 and out2.flags["C_CONTIGUOUS"]
    assert lse2.flags["C_CONTIGUOUS"]
    out1 = np.ascontiguousarray(out1)
    lse1 = np.ascontiguousarray(lse1)
    c1 = 1 if lse1_bf16 else _LSE_CODES[lse1.dtype]
    c2 = 1 if lse2_bf16 else _LSE_CODES[lse2.dtype]
    D = int(out1.shape[-1])
    rows = int(out1.size // D)
    assert out2.size == out1.size and lse1.size == rows and lse2.size == rows
    lib().mac_oracle_update_then_downdate(
        _ptr(out1, _u16p), lse1.ctypes.data_as(ctypes.c_void_p), c1, _ptr(out2, _u16p),
        lse2.ctypes.data_as(ctypes.c_void_p), c2, ctypes.c_int64(rows), D)


def window_attention(q, k_buffer, v_buffer, qo_indptr, kv_indptr, kv_indices, *, window_left,
                     sm_scale):
    """Causal sliding-window attention over a ragged batch (bf16 bits in,
    bf16 bits out, natural-log lse)."""
    c = np.ascontiguousarray
    q = c(q, dtype=np.uint16)
    k_buffer = c(k_buffer, dtype=np.uint16)
    v_buffer = c(v_buffer, dtype=np.uint16)
    qo_indptr = c(qo_indptr, dtype=np.int32)
    kv_indptr = c(kv_indptr, dtype=np.int32)
    kv_indices = c(kv_indices, dtype=np.int32)
    total_q, hq, d = q.shape
    hkv = k_buffer.shape[1]
    out = np.zeros_like(q)
    lse = np.zeros((total_q, hq), np.float32)
    lib().mac_oracle_window_attention(
        _ptr(q, _u16p), _ptr(k_buffer, _u16p), _ptr(v_buffer, _u16p), _ptr(qo_indptr, _i32p),
        _ptr(kv_indptr, _i32p), _ptr(kv_indices, _i32p), int(qo_indptr.shape[0] - 1), hq, hkv, d,
        int(window_left), ctypes.c_double(sm_scale), _ptr(out, _u16p), _ptr(lse, _f32p))
    return out, lse


def rectify_update_cache(q_post, src_q, o_full, lse_full, k_buffer, v_buffer, qo_indptr,
                         kv_indptr, kv_indices, q_cache, attn_cache, lse_cache, request_length,
                         req_ids, *, semantic_pos_ahead, front_sink_tokens=0, sink_mode=0,
                         sm_scale, q_post_cache=None):
    """In-place restatement of ``mac_prefill_rectify_update_cache_bf16``
    (ring arrays and request_length are updated)."""
    c = np.ascontiguousarray
    for arr, dt in ((q_cache, np.uint16), (attn_cache, np.uint16), (lse_cache, np.float32),
                    (request_length, np.int32)):
        assert arr.dtype == dt and arr.flags["C_CONTIGUOUS"]
    q_post, src_q, o_full = (c(x, dtype=np.uint16) for x in (q_post, src_q, o_full))
    lse_full = c(lse_full, dtype=np.float32)
    k_buffer = c(k_buffer, dtype=np.uint16)
    v_buffer = c(v_buffer, dtype=np.uint16)
    qo_indptr, kv_indptr, kv_indices, req_ids = (
        c(x, dtype=np.int32) for x in (qo_indptr, kv_indptr, kv_indices, req_ids))
    r, m, hq, d = q_cache.shape
    lib().mac_oracle_rectify_update_cache(
        _ptr(q_post, _u16p), _ptr(src_q, _u16p), _ptr(o_full, _u16p), _ptr(lse_full, _f32p),
        _ptr(k_buffer, _u16p), _ptr(v_buffer, _u16p), _ptr(qo_indptr, _i32p),
        _ptr(kv_indptr, _i32p), _ptr(kv_indices, _i32p), _ptr(q_cache, _u16p),
        _ptr(attn_cache, _u16p), _ptr(lse_cache, _f32p), _ptr(q_post_cache, _u16p),
        _ptr(request_length, _i32p), int(request_length.shape[0]), _ptr(req_ids, _i32p),
        int(req_ids.shape[0]), r, m, hq, int(k_buffer.shape[1]), d, int(semantic_pos_ahead),
        int(front_sink_tokens), int(sink_mode), ctypes.c_double(sm_scale),
        ctypes.c_int64(q_post.shape[0]), ctypes.c_int64(kv_indices.shape[0]))


# ---------------------------------------------------- decode RoPE + scatter ---


def rope_preserve(q, k, v, q_pre, k_buffer, v_buffer, cos_sin_cache, positions, cache_locs, *,
                  head_dim, is_neox):
    """In-place restatement of ``mac_decode_rope_preserve_q_bf16``: q/k/v are
    uint16 bf16-bit arrays [N, H*head_dim] (row views allowed: the row stride
    is taken from the array), q_pre/k_buffer/v_buffer uint16 arrays."""
    for a in (q, k, q_pre, k_buffer, v_buffer):
        assert a.dtype == np.uint16
    for a in (q, k, v):
        assert a.strides[1] == 2
    for a in (q_pre, k_buffer, v_buffer):
        assert a.flags["C_CONTIGUOUS"]
    cs = np.ascontiguousarray(cos_sin_cache, dtype=np.float32)
    positions = np.ascontiguousarray(positions, dtype=np.int64)
    cache_locs = np.ascontiguousarray(cache_locs, dtype=np.int64)
    n = q.shape[0]
    lib().mac_oracle_rope_preserve(
        q.ctypes.data_as(_u16p), ctypes.c_int64(q.strides[0] // 2), k.ctypes.data_as(_u16p),
        ctypes.c_int64(k.strides[0] // 2), v.ctypes.data_as(_u16p), ctypes.c_int64(v.strides[0] // 2),
        _ptr(q_pre, _u16p), _ptr(k_buffer, _u16p), _ptr(v_buffer, _u16p),
        ctypes.c_int64(k_buffer.shape[0]), _ptr(cs, _f32p), ctypes.c_int64(cs.shape[0]),
        ctypes.c_int64(cs.shape[1]), int(cs.shape[1]), _ptr(positions, _i64p),
        _ptr(cache_locs, _i64p), ctypes.c_int64(n), int(q.shape[1] // head_dim),
        int(k.shape[1] // head_dim), int(head_dim), int(bool(is_neox)))
