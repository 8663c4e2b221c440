"""Synthetic decode inputs with the reference's conventions.

Restates the input builders of the reference's benchmark and tools:
  * ``_make_case`` (attention/tools/bench_mac_persistent_decode.py:61-113):
    K/V/q ~ N(0,1) bf16, ``req_to_token[n, :P] = n*kv_len + arange(P)``, the
    current token at ``n*kv_len + P``, ``req_ids = arange(B)``, unused ring
    slots ``randn + 10`` (far from any query);
  * ``_synthetic_hit_and_slot`` (benchmark/bench_mac_vs_flashinfer_direct.py:134-211):
    exact-quota rotated hit decisions per query head (``synthetic_head``) or per
    KV group (``synthetic_group``) and a match lag clamped to the ring;
  * ring entries of a hit are planted by copying the query into the matched
    slot (``apply_synthetic_cache_pattern``, :214-277).

``plant_hits`` returns the planted (n, hq) -> slot map so callers can build
exact ring entries.  Everything is numpy (CPU); ``to_device`` mirrors a case to
torch tensors on a GPU.  Large cases for benchmarking are generated directly
on the GPU by ``device_case``.
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field

import numpy as np


def _u32(x: int) -> int:
    return x & 0xFFFFFFFF


def mix_u32(x: int) -> int:
    x = _u32(x)
    x ^= x >> 16
    x = _u32(x * 0x7FEB352D)
    x ^= x >> 15
    x = _u32(x * 0x846CA68B)
    x ^= x >> 16
    return _u32(x)


def uniform01_u32(x: int) -> float:
    return float(mix_u32(x) & 0x00FFFFFF) * (1.0 / 16777216.0)


def pseudo_normal_u32(x: int) -> float:
    s = (uniform01_u32(x) + uniform01_u32(_u32(x ^ 0x9E3779B9))
         + uniform01_u32(_u32(x ^ 0x85EBCA6B)) + uniform01_u32(_u32(x ^ 0xC2B2AE35)))
    return (s - 2.0) * 1.7320508075688772


def target_miss_units(hit_rate: float, unit_total: int) -> int:
    if unit_total <= 0:
        return 0
    miss_rate = min(max(1.0 - hit_rate, 0.0), 1.0)
    return min(max(int(math.floor(miss_rate * float(unit_total) + 0.5)), 0), unit_total)


def cache_end_for_pos(pos: int, s: int) -> int:
    return max(pos + 1 - s, 0)


def ring_slot_to_pos(past_len: int, m: int, slot: int) -> int:
    if past_len < m:
        return slot
    order = slot - past_len % m
    if order < 0:
        order += m
    return past_len - m + order


def pos_to_ring_slot(past_len: int, m: int, pos: int) -> int:
    if past_len < m:
        return pos
    slot = pos - (past_len - m) + past_len % m
    if slot >= m:
        slot -= m
    if slot < 0:
        slot += m
    return slot


def synthetic_hit_and_slot(*, bench_mode: int, batch: int, hq: int, hkv: int, past_len: int,
                           n: int, hq_i: int, hkv_i: int, hit_rate: float, capacity: int,
                           semantic_pos_ahead: int, bench_seed: int = 1,
                           match_lag_mean: float = 64.0,
                           key_past_len: int | None = None) -> tuple[bool, int]:
    """Exact-quota rotated hit decision and matched ring slot of one query head
    (benchmark/bench_mac_vs_flashinfer_direct.py:134-211 with std 0 and no
    skip ratio).  ``key_past_len`` overrides the past length that seeds the
    rotation, so that ragged batches keep the exact quota."""
    kp = past_len if key_past_len is None else key_past_len
    base_key = _u32(int(bench_seed) ^ _u32(kp * 0x85EBCA6B))
    unit_total = batch * (hkv if bench_mode == 2 else hq)
    unit = n * (hkv if bench_mode == 2 else hq) + (hkv_i if bench_mode == 2 else hq_i)
    miss_units = target_miss_units(hit_rate, unit_total)
    offset = int(base_key % unit_total) if unit_total > 0 else 0
    rotated = unit + offset
    if rotated >= unit_total:
        rotated -= unit_total
    hit = past_len > 0 and capacity > 0 and not (rotated < miss_units)
    if not hit:
        return False, -1
    max_lag = min(capacity, past_len)
    new_end = cache_end_for_pos(past_len, semantic_pos_ahead)
    lag = min(max(int(round(match_lag_mean)), 1), max_lag)
    if max_lag <= 0 or new_end <= 0:
        return False, -1
    match_pos = max(past_len - lag, 0)
    return True, pos_to_ring_slot(past_len, capacity, match_pos)


def bf16_round(x: np.ndarray) -> np.ndarray:
    """Round float values to the nearest bf16 (returned as float32)."""
    f = np.ascontiguousarray(x, dtype=np.float32)
    u = f.view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint32) << 16
    return r.astype(np.uint32).view(np.float32)


def to_bits(x: np.ndarray) -> np.ndarray:
    """float -> bf16 bits (uint16)."""
    return (bf16_round(x).view(np.uint32) >> 16).astype(np.uint16)


def from_bits(b: np.ndarray) -> np.ndarray:
    return (np.ascontiguousarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


@dataclass
class Case:
    """One decode step's inputs; bf16 arrays hold float32 values already
    rounded to bf16."""

    q_post: np.ndarray
    q_pre: np.ndarray
    k: np.ndarray
    v: np.ndarray
    req_to_token: np.ndarray
    req_ids: np.ndarray
    past_lens: np.ndarray
    out_cache_loc: np.ndarray
    query_cache: np.ndarray
    attn_cache: np.ndarray
    lse_cache: np.ndarray
    semantic_pos_ahead: int
    front_sink_tokens: int = 0
    threshold: float = 0.45
    sm_scale: float = 1.0 / math.sqrt(128.0)
    cache_ready: np.ndarray | None = None
    cache_epoch: np.ndarray | None = None
    request_epoch: np.ndarray | None = None
    gen_min_limit: int = 0
    lookback_right: int = 0
    candidate_mode: int = 0
    planted: dict = field(default_factory=dict)

    @property
    def shape(self):
        n, hq, d = self.q_post.shape
        return n, hq, self.k.shape[1], d, self.query_cache.shape[1]


def paged_layout(kv_lens, r2t_cols=None):
    """req_to_token/out_cache_loc for requests stored back to back
    (tools/bench_mac_persistent_decode.py:77-85)."""
    kv_lens = [int(x) for x in kv_lens]
    b = len(kv_lens)
    cols = r2t_cols or max(kv_lens)
    r2t = np.zeros((b, cols), np.int32)
    ocl = np.zeros(b, np.int64)
    base = 0
    for n, kv in enumerate(kv_lens):
        p = kv - 1
        r2t[n, :p] = np.arange(base, base + p, dtype=np.int32)
        r2t[n, p:kv] = base + p
        ocl[n] = base + p
        base += kv
    return r2t, ocl, base


def exact_entry(q_post_head: np.ndarray, k_rows: np.ndarray, v_rows: np.ndarray, sm_scale: float):
    """Exact attention of one head over explicit K/V rows (float64)."""
    if k_rows.shape[0] == 0:
        return np.zeros(q_post_head.shape[-1]), -np.inf
    logits = (k_rows.astype(np.float64) @ q_post_head.astype(np.float64)) * sm_scale
    m = logits.max()
    w = np.exp(logits - m)
    den = w.sum()
    return (w[:, None] * v_rows.astype(np.float64)).sum(0) / den, m + np.log(den)


def random_case(*, batch: int, hq: int, hkv: int, kv_lens, capacity: int, semantic_pos_ahead: int,
                front_sink_tokens: int = 0, hit_rate: float = 0.5, bench_mode: int = 1,
                match_lag: float = 64.0, noise: float = 0.0, seed: int = 0, dim: int = 128,
                separate_pre_post: bool = True, entry_builder: str = "exact",
                threshold: float = 0.45, bench_seed: int = 1) -> Case:
    """A small decode case with planted ring matches, all on the CPU.

    Matches follow ``synthetic_hit_and_slot``; the matched slot holds
    ``sqrt(1-noise^2)*q_pre + noise*N(0,1)`` and its entry is exact attention
    of q_post over [min(F,E), E) with E = pos+1-S (``entry_builder="exact"``),
    so a hit's output equals exact full attention up to bf16 rounding.
    """
    rng = np.random.default_rng(seed)
    kv_lens = [int(x) for x in kv_lens]
    assert len(kv_lens) == batch
    r2t, ocl, pool = paged_layout(kv_lens)
    k = bf16_round(rng.standard_normal((pool, hkv, dim), dtype=np.float32))
    v = bf16_round(rng.standard_normal((pool, hkv, dim), dtype=np.float32))
    q_pre = bf16_round(rng.standard_normal((batch, hq, dim), dtype=np.float32))
    q_post = (bf16_round(rng.standard_normal((batch, hq, dim), dtype=np.float32))
              if separate_pre_post else q_pre.copy())
    qc = bf16_round(rng.standard_normal((batch, capacity, hq, dim), dtype=np.float32) + 10.0)
    ac = np.zeros((batch, capacity, hq, dim), np.float32)
    lc = np.full((batch, capacity, hq), -np.inf, np.float32)
    group = hq // hkv
    F = max(front_sink_tokens, 0)
    sm = 1.0 / math.sqrt(dim)
    planted = {}
    for n in range(batch):
        p = kv_lens[n] - 1
        for hq_i in range(hq):
            hit, slot = synthetic_hit_and_slot(
                bench_mode=bench_mode, batch=batch, hq=hq, hkv=hkv, past_len=p, n=n, hq_i=hq_i,
                hkv_i=hq_i // group, hit_rate=hit_rate, capacity=capacity,
                semantic_pos_ahead=semantic_pos_ahead, bench_seed=bench_seed,
                match_lag_mean=match_lag, key_past_len=kv_lens[0] - 1)
            if not hit:
                continue
            pos = ring_slot_to_pos(p, capacity, slot)
            src = q_pre[n, hq_i]
            if noise > 0:
                src = math.sqrt(1 - noise * noise) * src + noise * rng.standard_normal(dim)
            qc[n, slot, hq_i] = bf16_round(src)
            e = cache_end_for_pos(pos, semantic_pos_ahead)
            b0 = min(F, e)
            rows = r2t[n, b0:e]
            hkv_i = hq_i // group
            if entry_builder == "exact":
                o, lse = exact_entry(q_post[n, hq_i], k[rows, hkv_i], v[rows, hkv_i], sm)
            else:
                o, lse = rng.standard_normal(dim), float(rng.standard_normal())
            ac[n, slot, hq_i] = bf16_round(o)
            lc[n, slot, hq_i] = lse
            planted[(n, hq_i)] = (slot, pos)
    return Case(q_post=q_post, q_pre=q_pre, k=k, v=v, req_to_token=r2t,
                req_ids=np.arange(batch, dtype=np.int32),
                past_lens=np.array([x - 1 for x in kv_lens], np.int32), out_cache_loc=ocl,
                query_cache=qc, attn_cache=ac, lse_cache=lc,
                semantic_pos_ahead=semantic_pos_ahead, front_sink_tokens=front_sink_tokens,
                threshold=threshold, sm_scale=sm, planted=planted)


# ------------------------------------------------------- workspace ----


def ceil_div(a: int, b: int) -> int:
    return (a + b - 1) // b


def workspace(torch, *, batch, hq, hkv, capacity, max_context, tile_tokens, match_tile_slots,
              semantic_pos_ahead, front_sink_tokens=0, partial_dtype=None, device="cuda",
              dim=128):
    """The 30 workspace tensors in the reference's order
    (attention/tests/test_mac_persistent_decode.py:54-97)."""
    group = hq // hkv
    partial_dtype = partial_dtype or torch.float32
    mmt = ceil_div(capacity, match_tile_slots)
    mtc = ceil_div(max_context, tile_tokens) + ceil_div(max(front_sink_tokens, 0), tile_tokens)
    mtr = ceil_div(mtc, 32)
    mtt = max(1, ceil_div(max(semantic_pos_ahead, 1), tile_tokens))
    i32 = torch.int32
    e = lambda *s, dt=torch.float32: torch.empty(*s, device=device, dtype=dt)  # noqa: E731
    return [
        e(batch, hq, mmt), e(batch, hq, mmt, dt=i32), e(batch, hq, mmt, dt=i32),
        *[e(batch, hq, dt=i32) for _ in range(6)],
        *[e(batch, hkv, dt=i32) for _ in range(6)],
        e(batch, hkv, dt=i32),
        e(max(batch * hq * mtc, 2 * batch * hkv + 6), dt=i32),
        e(max(batch * hq * mtc, 2 * batch * hkv + 6), dt=i32),
        e(batch * hkv * mtt, dt=i32), e(batch * hkv * mtt, dt=i32),
        e(batch * hq * mtt, dt=i32), e(batch * hq * mtt, dt=i32),
        e(9, dt=i32),
        e(batch, hkv, mtc, group, dim, dt=partial_dtype), e(batch, hkv, mtc, group),
        e(batch, hkv, mtr, group, dim, dt=partial_dtype), e(batch, hkv, mtr, group),
        e(batch, hkv, mtt, group, dim, dt=partial_dtype), e(batch, hkv, mtt, group),
        e(14, dt=torch.int64),
    ]


def to_device(torch, case: Case, device="cuda", out_cache_loc_dtype=None):
    """Mirror a Case to torch tensors (bf16 where the reference uses bf16)."""
    bf = torch.bfloat16
    t = lambda a, dt: torch.from_numpy(np.ascontiguousarray(a)).to(device=device, dtype=dt)  # noqa: E731
    d = dict(
        q_post=t(case.q_post, bf), q_pre=t(case.q_pre, bf), k=t(case.k, bf), v=t(case.v, bf),
        req_to_token=t(case.req_to_token, torch.int32), req_ids=t(case.req_ids, torch.int32),
        past_lens=t(case.past_lens, torch.int32),
        out_cache_loc=t(case.out_cache_loc, out_cache_loc_dtype or torch.int64),
        query_cache=t(case.query_cache, bf), attn_cache=t(case.attn_cache, bf),
        lse_cache=t(case.lse_cache, torch.float32),
    )
    for name in ("cache_ready", "cache_epoch", "request_epoch"):
        a = getattr(case, name)
        if a is None:
            d[name] = torch.empty(0, device=device)
        else:
            d[name] = t(a, torch.bool if name == "cache_ready" else torch.int64)
    return d


def run_decode(torch, ext, dev: dict, case: Case, *, max_context, tile_tokens=4, match_tile_slots=4,
               partial_dtype=None, bench=None, ws=None, debug_enabled=0):
    """Call the 68-argument binding on device tensors ``dev`` (from
    ``to_device``); returns (out, out_lse, workspace)."""
    n, hq, hkv, dim, m = case.shape
    q = dev["q_post"]
    out = torch.empty_like(q)
    out_lse = torch.empty(n, hq, device=q.device)
    if ws is None:
        ws = workspace(torch, batch=n, hq=hq, hkv=hkv, capacity=m, max_context=max_context,
                       tile_tokens=tile_tokens, match_tile_slots=match_tile_slots,
                       semantic_pos_ahead=case.semantic_pos_ahead,
                       front_sink_tokens=case.front_sink_tokens, partial_dtype=partial_dtype,
                       device=q.device)
    b = dict(bench_mode=0, bench_hit_rate=1.0, bench_hit_rate_std=0.0, bench_skip_ratio=-1.0,
             bench_skip_ratio_std=0.0, bench_match_lag_mean=64.0, bench_match_lag_std=0.0,
             bench_seed=1, bench_miss_mask=-1, bench_layer_id=0)
    b.update(bench or {})
    ext.mac_persistent_decode_bf16(
        q, dev["q_pre"], dev["k"], dev["v"], dev["req_to_token"], dev["req_ids"],
        dev["past_lens"], dev["out_cache_loc"], dev["query_cache"], dev["attn_cache"],
        dev["lse_cache"], out, out_lse, *ws,
        max_context, tile_tokens, match_tile_slots, case.semantic_pos_ahead,
        case.front_sink_tokens, case.gen_min_limit, case.lookback_right, case.candidate_mode,
        case.threshold, case.sm_scale, debug_enabled, b["bench_mode"],
        b["bench_hit_rate"], b["bench_hit_rate_std"], b["bench_skip_ratio"],
        b["bench_skip_ratio_std"], b["bench_match_lag_mean"], b["bench_match_lag_std"],
        b["bench_seed"], b["bench_miss_mask"], b["bench_layer_id"],
        dev["query_cache"], dev["cache_ready"], dev["cache_epoch"], dev["request_epoch"],
    )
    return out, out_lse, ws


# ------------------------------------------------------ device cases ----


def device_case(torch, *, batch: int, hq: int, hkv: int, ctx: int, capacity: int, seed: int = 0,
                device="cuda", kv=None, chunk_rows: int = 1 << 20):
    """Benchmark-scale inputs generated on the GPU with the conventions of
    ``_make_case`` (tools/bench_mac_persistent_decode.py:61-113): every request
    has past_len = ctx and kv_len = ctx + 1, K/V/q ~ N(0,1) bf16, the ring
    holds randn + 10 rows with finite lse 0 (hit decisions then come from the
    synthetic override or from planted copies).  ``kv`` reuses a (k, v) pair
    of at least batch * (ctx + 1) rows."""
    kv_len = ctx + 1
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    bf = torch.bfloat16
    rows = batch * kv_len
    if kv is None:
        k = torch.empty(rows, hkv, 128, device=device, dtype=bf)
        v = torch.empty(rows, hkv, 128, device=device, dtype=bf)
        for t in (k, v):
            for i in range(0, rows, chunk_rows):
                t[i:i + chunk_rows].normal_(generator=g)
    else:
        k, v = kv
        assert k.shape[0] >= rows and k.shape[1] == hkv
    base = torch.arange(batch, device=device, dtype=torch.int64)[:, None] * kv_len
    r2t = (base + torch.arange(kv_len, device=device, dtype=torch.int64)[None, :]).to(torch.int32)
    r2t[:, ctx] = (base[:, 0] + ctx).to(torch.int32)
    q = torch.randn(batch, hq, 128, device=device, dtype=bf, generator=g)
    qc = torch.randn(batch, capacity, hq, 128, device=device, dtype=bf, generator=g) + 10
    return dict(
        q_post=q, q_pre=q, k=k, v=v, req_to_token=r2t.contiguous(),
        req_ids=torch.arange(batch, device=device, dtype=torch.int32),
        past_lens=torch.full((batch,), ctx, device=device, dtype=torch.int32),
        out_cache_loc=(base[:, 0] + ctx).to(torch.int32),
        query_cache=qc.contiguous(), attn_cache=torch.zeros_like(qc),
        lse_cache=torch.zeros(batch, capacity, hq, device=device, dtype=torch.float32),
        cache_ready=torch.empty(0, device=device), cache_epoch=torch.empty(0, device=device),
        request_epoch=torch.empty(0, device=device),
    )


def plant_synthetic_hits(torch, dev: dict, *, hit_rate: float, bench_mode: int, semantic_pos_ahead: int,
                         bench_seed: int = 1, match_lag_mean: float = 64.0):
    """``apply_synthetic_cache_pattern`` (benchmark/bench_mac_vs_flashinfer_direct.py:214-277):
    copy each hit head's query into its matched slot.  Returns the number of
    planted heads."""
    batch, hq, _ = dev["q_pre"].shape
    hkv = dev["k"].shape[1]
    group = hq // hkv
    cap = dev["query_cache"].shape[1]
    past = [int(x) for x in dev["past_lens"].cpu().tolist()]
    ns, hs, ss = [], [], []
    for n in range(batch):
        for hq_i in range(hq):
            hit, slot = synthetic_hit_and_slot(
                bench_mode=bench_mode, batch=batch, hq=hq, hkv=hkv, past_len=past[n], n=n,
                hq_i=hq_i, hkv_i=hq_i // group, hit_rate=hit_rate, capacity=cap,
                semantic_pos_ahead=semantic_pos_ahead, bench_seed=bench_seed,
                match_lag_mean=match_lag_mean)
            if hit and slot >= 0:
                ns.append(n)
                hs.append(hq_i)
                ss.append(slot)
    if ns:
        ni = torch.tensor(ns, device=dev["q_pre"].device)
        hi = torch.tensor(hs, device=dev["q_pre"].device)
        si = torch.tensor(ss, device=dev["q_pre"].device)
        dev["query_cache"][ni, si, hi] = dev["q_pre"][ni, hi]
    return len(ns)


def device_ragged_case(torch, *, kv_lens, hq: int, hkv: int, capacity: int, seed: int = 0,
                       device="cuda", q_post_separate: bool = True, chunk_rows: int = 1 << 20):
    """Like ``device_case`` but with one context length per request (requests
    stored back to back in the pool) and random finite ring entries
    (o ~ N(0,1), lse ~ N(0,1)) so that reuse merges are non-trivial.  Ring
    queries are randn + 10 (never matched unless planted)."""
    kv_lens = [int(x) for x in kv_lens]
    batch = len(kv_lens)
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    bf = torch.bfloat16
    rows = sum(kv_lens)
    k = torch.empty(rows, hkv, 128, device=device, dtype=bf)
    v = torch.empty(rows, hkv, 128, device=device, dtype=bf)
    for t in (k, v):
        for i in range(0, rows, chunk_rows):
            t[i:i + chunk_rows].normal_(generator=g)
    cols = max(kv_lens)
    r2t = torch.zeros(batch, cols, device=device, dtype=torch.int32)
    ocl = torch.zeros(batch, device=device, dtype=torch.int64)
    base = 0
    for n, kv in enumerate(kv_lens):
        r2t[n, :kv] = torch.arange(base, base + kv, device=device, dtype=torch.int32)
        ocl[n] = base + kv - 1
        base += kv
    q_pre = torch.randn(batch, hq, 128, device=device, dtype=bf, generator=g)
    q_post = (torch.randn(batch, hq, 128, device=device, dtype=bf, generator=g)
              if q_post_separate else q_pre)
    qc = torch.randn(batch, capacity, hq, 128, device=device, dtype=bf, generator=g) + 10
    ac = torch.randn(batch, capacity, hq, 128, device=device, dtype=bf, generator=g)
    lc = torch.randn(batch, capacity, hq, device=device, dtype=torch.float32, generator=g)
    return dict(
        q_post=q_post, q_pre=q_pre, k=k, v=v, req_to_token=r2t,
        req_ids=torch.arange(batch, device=device, dtype=torch.int32),
        past_lens=torch.tensor([x - 1 for x in kv_lens], device=device, dtype=torch.int32),
        out_cache_loc=ocl, query_cache=qc.contiguous(), attn_cache=ac.contiguous(),
        lse_cache=lc.contiguous(),
        cache_ready=torch.empty(0, device=device), cache_epoch=torch.empty(0, device=device),
        request_epoch=torch.empty(0, device=device),
    )


def plant_noisy_matches(torch, dev: dict, *, entries: dict, seed: int = 0):
    """Plant ring rows that a head matches with similarity noise:
    ``entries[(n, hq)] = (pos, eps)`` stores sqrt(1-eps^2) * q_pre + eps * N(0,1)
    at the slot of logical position ``pos`` (BASELINE configs 0-2 hit
    structure).  Small eps (<= 0.5) is a hit at threshold 0.45, eps >= 0.9 a
    miss."""
    if not entries:
        return
    g = torch.Generator(device=dev["q_pre"].device)
    g.manual_seed(seed)
    cap = dev["query_cache"].shape[1]
    past = [int(x) for x in dev["past_lens"].cpu().tolist()]
    for (n, h), (pos, eps) in sorted(entries.items()):
        slot = pos_to_ring_slot(past[n], cap, pos)
        q = dev["q_pre"][n, h].float()
        z = torch.randn(q.shape, device=q.device, generator=g)
        dev["query_cache"][n, slot, h] = (math.sqrt(1.0 - eps * eps) * q + eps * z).to(torch.bfloat16)


# ------------------------------------------------ prefill rectification ----


@dataclass
class PrefillCase:
    """A ragged prefill chunk over a page-size-1 pool.  Request b has kv_lens[b]
    keys (its prefix plus the chunk) and qo_lens[b] query rows, the last
    qo_lens[b] positions.  Values are float32 holding bf16-exact numbers."""

    q: np.ndarray            # [total_q, Hq, D]
    k: np.ndarray            # [pool, Hkv, D]
    v: np.ndarray            # [pool, Hkv, D]
    qo_indptr: np.ndarray    # [B+1] int32
    kv_indptr: np.ndarray    # [B+1] int32
    kv_indices: np.ndarray   # [kv_indptr[B]] int32, a random permutation of pool rows
    sm_scale: float = 1.0 / math.sqrt(128.0)

    def positions(self, b: int) -> np.ndarray:
        qlen = int(self.qo_indptr[b + 1] - self.qo_indptr[b])
        kvlen = int(self.kv_indptr[b + 1] - self.kv_indptr[b])
        return np.arange(kvlen - qlen, kvlen)


def prefill_case(*, qo_lens, kv_lens, hq: int, hkv: int, seed: int = 0, spare_rows: int = 7,
                 dim: int = 128, scale: float = 1.0) -> PrefillCase:
    rng = np.random.default_rng(seed)
    qo_lens = [int(x) for x in qo_lens]
    kv_lens = [int(x) for x in kv_lens]
    assert all(q <= k for q, k in zip(qo_lens, kv_lens))
    total_kv = sum(kv_lens)
    pool = total_kv + spare_rows
    perm = rng.permutation(pool)[:total_kv].astype(np.int32)
    return PrefillCase(
        q=bf16_round(rng.standard_normal((sum(qo_lens), hq, dim)) * scale),
        k=bf16_round(rng.standard_normal((pool, hkv, dim))),
        v=bf16_round(rng.standard_normal((pool, hkv, dim))),
        qo_indptr=np.concatenate([[0], np.cumsum(qo_lens)]).astype(np.int32),
        kv_indptr=np.concatenate([[0], np.cumsum(kv_lens)]).astype(np.int32),
        kv_indices=perm,
    )
