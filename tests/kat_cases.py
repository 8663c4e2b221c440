"""Known-answer cases of the reference, restated with numpy-seeded inputs.

Each function rebuilds one case of
  attention/tests/test_mac_persistent_decode.py (4 KATs, :100-466) and
  attention/tools/check_mac_persistent_decode.py (12 checks, :209-921)
with the same shapes, planted matches, ring contents and expected-value
recipe (exact attention per span + LSE merges, :9-51).  The reference draws
its tensors from torch's CUDA RNG; these cases draw them from numpy, so the
values differ but every structural property the reference asserts (hit
pattern, match position, group mode, ring-row contents, output) is the same.

A case carries its expectations: per-request expected outputs and ring rows
(float64) with the reference's tolerances, and integer workspace values.
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field

import numpy as np

from helpers import merge, ref_attention, syn

SM = 1.0 / math.sqrt(128.0)
D = 128


@dataclass
class Kat:
    name: str
    case: syn.Case
    max_context: int
    tile_tokens: int
    match_tile_slots: int
    o_tol: float
    lse_tol: float
    exp_out: dict  # n -> (o [Hq,D], lse [Hq])
    exp_ring: dict  # n -> (o [Hq,D], lse [Hq])
    head_hit: np.ndarray | None = None  # [N,Hq]
    head_match_pos: np.ndarray | None = None
    group_mode: np.ndarray | None = None
    env: dict = field(default_factory=dict)
    ring_exact_empty: bool = False  # short context: q copied bit-exactly, o = 0, lse = -inf
    min_reduce_groups: int = 0  # task_counts[3] must exceed this - 1
    tol_per_head: dict = field(default_factory=dict)  # h -> (o_tol, lse_tol)


def _bf(rng, *shape, add=0.0):
    return syn.bf16_round(rng.standard_normal(shape, dtype=np.float32) + add)


def _single_request_layout(kv_len, cols):
    p = kv_len - 1
    r2t = np.zeros((1, cols), np.int32)
    r2t[0, :p] = np.arange(p, dtype=np.int32)
    return r2t, np.array([p], np.int64)


def _case(q_post, q_pre, k, v, r2t, ocl, past_lens, qc, ac, lc, s, f=0, req_ids=None):
    b = q_post.shape[0]
    return syn.Case(
        q_post=q_post, q_pre=q_pre, k=k, v=v, req_to_token=r2t,
        req_ids=np.arange(b, dtype=np.int32) if req_ids is None else req_ids,
        past_lens=np.asarray(past_lens, np.int32), out_cache_loc=np.asarray(ocl, np.int64),
        query_cache=qc, attn_cache=ac, lse_cache=lc, semantic_pos_ahead=s, front_sink_tokens=f,
        sm_scale=SM)


def hit_clean_half_open_cache_row() -> Kat:
    """tests/test_mac_persistent_decode.py:100-191."""
    rng = np.random.default_rng(1)
    hkv, g = 2, 4
    hq = hkv * g
    m, kv_len, s = 8, 10, 3
    p = kv_len - 1
    k, v = _bf(rng, kv_len, hkv, D), _bf(rng, kv_len, hkv, D)
    q = _bf(rng, 1, hq, D)
    r2t, ocl = _single_request_layout(kv_len, 64)
    qc = _bf(rng, 1, m, hq, D)
    ac = np.zeros_like(qc)
    lc = np.full((1, m, hq), -np.inf, np.float32)
    match_pos = 5
    slot = match_pos % m
    qc[0, slot] = q[0]
    pe = max(match_pos + 1 - s, 0)
    po, pl = ref_attention(q[0], k, v, 0, pe, SM)
    po = syn.bf16_round(po)
    ac[0, slot], lc[0, slot] = po, pl
    ne = max(p + 1 - s, 0)
    ro, rl = ref_attention(q[0], k, v, pe, ne, SM)
    to, tl = ref_attention(q[0], k, v, ne, kv_len, SM)
    co, cl = merge(po, pl, ro, rl)
    oo, ol = merge(co, cl, to, tl)
    return Kat("hit_clean_half_open_cache_row", _case(q, q, k, v, r2t, ocl, [p], qc, ac, lc, s),
               16, 4, 4, 3e-2, 3e-2, {0: (oo, ol)}, {0: (co, cl)},
               head_hit=np.ones((1, hq), np.int32),
               head_match_pos=np.full((1, hq), match_pos, np.int32))


def miss_multi_request() -> Kat:
    """tests/test_mac_persistent_decode.py:194-278."""
    rng = np.random.default_rng(2)
    b, hkv, g = 2, 2, 4
    hq = hkv * g
    m, kv_len, s = 8, 12, 4
    p = kv_len - 1
    k, v = _bf(rng, b * kv_len, hkv, D), _bf(rng, b * kv_len, hkv, D)
    q = _bf(rng, b, hq, D)
    r2t = np.zeros((b, 64), np.int32)
    for n in range(b):
        r2t[n, :p] = np.arange(n * kv_len, n * kv_len + p)
    ocl = np.array([p, kv_len + p], np.int64)
    qc = _bf(rng, b, m, hq, D, add=10.0)
    ac = np.zeros_like(qc)
    lc = np.full((b, m, hq), -np.inf, np.float32)
    exp_out, exp_ring = {}, {}
    for n in range(b):
        kk, vv = k[n * kv_len:(n + 1) * kv_len], v[n * kv_len:(n + 1) * kv_len]
        exp_out[n] = ref_attention(q[n], kk, vv, 0, kv_len, SM)
        exp_ring[n] = ref_attention(q[n], kk, vv, 0, kv_len - s, SM)
    kat = Kat("miss_multi_request", _case(q, q, k, v, r2t, ocl, [p, p], qc, ac, lc, s),
              16, 4, 4, 3e-2, 3e-2, exp_out, exp_ring, head_hit=np.zeros((b, hq), np.int32),
              group_mode=np.ones((b, hkv), np.int32))
    return kat


def short_context_writes_empty_cache_row() -> Kat:
    """tests/test_mac_persistent_decode.py:281-360."""
    rng = np.random.default_rng(3)
    hkv, g = 2, 4
    hq = hkv * g
    m, kv_len, s = 8, 3, 4
    p = kv_len - 1
    k, v = _bf(rng, kv_len, hkv, D), _bf(rng, kv_len, hkv, D)
    q = _bf(rng, 1, hq, D)
    r2t, ocl = _single_request_layout(kv_len, 32)
    qc = _bf(rng, 1, m, hq, D, add=10.0)
    ac = np.ones_like(qc)
    lc = np.zeros((1, m, hq), np.float32)
    out = ref_attention(q[0], k, v, 0, kv_len, SM)
    return Kat("short_context_writes_empty_cache_row",
               _case(q, q, k, v, r2t, ocl, [p], qc, ac, lc, s), 16, 4, 4, 3e-2, 3e-2,
               {0: out}, {}, ring_exact_empty=True)


def tie_breaks_by_logical_position_after_wraparound() -> Kat:
    """tests/test_mac_persistent_decode.py:363-466: positions 6 and 7 hold the
    same query; the smaller logical position (6) must win."""
    rng = np.random.default_rng(4)
    hkv, g = 2, 4
    hq = hkv * g
    m, kv_len, s = 4, 10, 2
    p = kv_len - 1
    k, v = _bf(rng, kv_len, hkv, D), _bf(rng, kv_len, hkv, D)
    q = _bf(rng, 1, hq, D)
    r2t, ocl = _single_request_layout(kv_len, 32)
    qc = _bf(rng, 1, m, hq, D, add=10.0)
    ac = np.zeros_like(qc)
    lc = np.full((1, m, hq), -np.inf, np.float32)
    first, later = 6, 7
    fs, ls = first % m, later % m
    qc[0, fs] = q[0]
    qc[0, ls] = q[0]
    fpe = max(first + 1 - s, 0)
    fo, fl = ref_attention(q[0], k, v, 0, fpe, SM)
    fo = syn.bf16_round(fo)
    ac[0, fs], lc[0, fs] = fo, fl
    ac[0, ls] = _bf(rng, hq, D)
    lc[0, ls] = rng.standard_normal(hq).astype(np.float32)
    ne = max(p + 1 - s, 0)
    ro, rl = ref_attention(q[0], k, v, fpe, ne, SM)
    to, tl = ref_attention(q[0], k, v, ne, kv_len, SM)
    co, cl = merge(fo, fl, ro, rl)
    oo, ol = merge(co, cl, to, tl)
    return Kat("tie_breaks_by_logical_position_after_wraparound",
               _case(q, q, k, v, r2t, ocl, [p], qc, ac, lc, s), 16, 4, 2, 3e-2, 3e-2,
               {0: (oo, ol)}, {0: (co, cl)}, head_match_pos=np.full((1, hq), first, np.int32))


def front_sink_rectification() -> Kat:
    """tools/check_mac_persistent_decode.py:264-337: hit with F=3; the entry
    covers [F, prefix_end) and was built by an unrelated query."""
    rng = np.random.default_rng(5)
    hkv, g = 2, 4
    hq = hkv * g
    m, kv_len, s = 16, 20, 4
    f = 3
    p = kv_len - 1
    k, v = _bf(rng, kv_len, hkv, D), _bf(rng, kv_len, hkv, D)
    q_pre, q_post = _bf(rng, 1, hq, D), _bf(rng, 1, hq, D)
    q_match = syn.bf16_round(q_pre[0] + 0.03 * rng.standard_normal((hq, D)))
    q_build = _bf(rng, hq, D)
    r2t, ocl = _single_request_layout(kv_len, 64)
    qc = _bf(rng, 1, m, hq, D, add=10.0)
    ac = np.zeros_like(qc)
    lc = np.full((1, m, hq), -np.inf, np.float32)
    mp = 10
    slot = mp % m
    pe = max(mp + 1 - s, 0)
    ne = max(p + 1 - s, 0)
    qc[0, slot] = q_match
    eo, el = ref_attention(q_build, k, v, f, pe, SM)
    eo = syn.bf16_round(eo)
    ac[0, slot], lc[0, slot] = eo, el
    so, sl = ref_attention(q_post[0], k, v, 0, f, SM)
    ro, rl = ref_attention(q_post[0], k, v, pe, ne, SM)
    to, tl = ref_attention(q_post[0], k, v, ne, kv_len, SM)
    co, cl = merge(eo, el, ro, rl)
    oo, ol = merge(*merge(co, cl, so, sl), to, tl)
    return Kat("front_sink_rectification",
               _case(q_post, q_pre, k, v, r2t, ocl, [p], qc, ac, lc, s, f), 32, 4, 4, 7e-2, 4e-2,
               {0: (oo, ol)}, {0: (co, cl)}, head_hit=np.ones((1, hq), np.int32))


def _mixed_front_sink(name, seed, hkv, g, hit_heads, m, kv_len, s, f, mp, cols, max_context,
                      o_tol=8e-2, lse_tol=4e-2) -> Kat:
    """Shared body of check_mac_persistent_decode.py:340-446 and :460-570."""
    rng = np.random.default_rng(seed)
    hq = hkv * g
    p = kv_len - 1
    k, v = _bf(rng, kv_len, hkv, D), _bf(rng, kv_len, hkv, D)
    q_pre, q_post = _bf(rng, 1, hq, D), _bf(rng, 1, hq, D)
    q_build = _bf(rng, hq, D)
    r2t, ocl = _single_request_layout(kv_len, cols)
    qc = _bf(rng, 1, m, hq, D, add=10.0)
    ac = np.zeros_like(qc)
    lc = np.full((1, m, hq), -np.inf, np.float32)
    slot = syn.pos_to_ring_slot(p, m, mp)
    pe = max(mp + 1 - s, 0)
    ne = max(p + 1 - s, 0)
    eo, el = ref_attention(q_build, k, v, f, pe, SM)
    eo = syn.bf16_round(eo)
    for h in hit_heads:
        qc[0, slot, h] = syn.bf16_round(q_pre[0, h] + 0.03 * rng.standard_normal(D))
        ac[0, slot, h], lc[0, slot, h] = eo[h], el[h]
    so, sl = ref_attention(q_post[0], k, v, 0, f, SM)
    ro, rl = ref_attention(q_post[0], k, v, pe, ne, SM)
    to, tl = ref_attention(q_post[0], k, v, ne, kv_len, SM)
    hco, hcl = merge(eo, el, ro, rl)
    hoo, hol = merge(*merge(hco, hcl, so, sl), to, tl)
    fo, fl = ref_attention(q_post[0], k, v, 0, kv_len, SM)
    mco, mcl = ref_attention(q_post[0], k, v, f, ne, SM)
    hit = np.array([h in hit_heads for h in range(hq)])
    out_o = np.where(hit[:, None], hoo, fo)
    out_l = np.where(hit, hol, fl)
    ring_o = np.where(hit[:, None], hco, mco)
    ring_l = np.where(hit, hcl, mcl)
    return Kat(name, _case(q_post, q_pre, k, v, r2t, ocl, [p], qc, ac, lc, s, f), max_context, 4, 4,
               o_tol, lse_tol, {0: (out_o, out_l)}, {0: (ring_o, ring_l)},
               head_hit=hit.astype(np.int32)[None], env={"MAC_PERSISTENT_MIXED_GROUP_FALLBACK": "1"})


def front_sink_mixed_group_exclusion() -> Kat:
    """tools/check_mac_persistent_decode.py:340-446 (GQA-8, 6 hit / 2 miss)."""
    return _mixed_front_sink("front_sink_mixed_group_exclusion", 11, 1, 8, list(range(6)), 16, 20,
                             4, 3, 10, 64, 32)


def front_sink_group4_mixed_fastpath() -> Kat:
    """tools/check_mac_persistent_decode.py:460-462, :473-570."""
    return _mixed_front_sink("front_sink_group4_mixed_fastpath", 13, 2, 4, [0, 1, 4, 5, 6, 7], 16,
                             200, 4, 6, 190, 256, 256)


def front_sink_group8_mixed_fastpath() -> Kat:
    """tools/check_mac_persistent_decode.py:465-470, :473-570."""
    return _mixed_front_sink("front_sink_group8_mixed_fastpath", 13, 2, 8,
                             [0, 1, 2, 3] + list(range(8, 16)), 16, 200, 4, 6, 190, 256, 256)


def _full_fallback_reduce(name, g, hkv=2) -> Kat:
    """tools/check_mac_persistent_decode.py:573-636."""
    rng = np.random.default_rng(17)
    hq = hkv * g
    m, kv_len, s, f = 16, 300, 4, 6
    p = kv_len - 1
    k, v = _bf(rng, kv_len, hkv, D), _bf(rng, kv_len, hkv, D)
    q = _bf(rng, 1, hq, D)
    r2t, ocl = _single_request_layout(kv_len, 512)
    qc = _bf(rng, 1, m, hq, D, add=10.0)
    ac = np.zeros_like(qc)
    lc = np.full((1, m, hq), -np.inf, np.float32)
    ne = max(p + 1 - s, 0)
    return Kat(name, _case(q, q, k, v, r2t, ocl, [p], qc, ac, lc, s, f), 512, 4, 4, 8e-2, 4e-2,
               {0: ref_attention(q[0], k, v, 0, kv_len, SM)},
               {0: ref_attention(q[0], k, v, f, ne, SM)},
               head_hit=np.zeros((1, hq), np.int32), group_mode=np.ones((1, hkv), np.int32))


def front_sink_group4_full_fallback_reduce() -> Kat:
    return _full_fallback_reduce("front_sink_group4_full_fallback_reduce", 4)


def front_sink_group8_full_fallback_reduce() -> Kat:
    return _full_fallback_reduce("front_sink_group8_full_fallback_reduce", 8)


def large_miss_reduced_rect() -> Kat:
    """tools/check_mac_persistent_decode.py:690-734: the band spans several
    tasks, so the reduction counter task_counts[3] is positive."""
    rng = np.random.default_rng(22)
    hkv, g = 2, 4
    hq = hkv * g
    m, kv_len, s, maxc = 8, 192, 4, 256
    p = kv_len - 1
    k, v = _bf(rng, kv_len, hkv, D), _bf(rng, kv_len, hkv, D)
    q = _bf(rng, 1, hq, D)
    r2t, ocl = _single_request_layout(kv_len, maxc)
    qc = _bf(rng, 1, m, hq, D, add=10.0)
    ac = np.zeros_like(qc)
    lc = np.full((1, m, hq), -np.inf, np.float32)
    return Kat("large_miss_reduced_rect", _case(q, q, k, v, r2t, ocl, [p], qc, ac, lc, s), maxc, 4,
               4, 3e-2, 3e-2, {0: ref_attention(q[0], k, v, 0, kv_len, SM)},
               {0: ref_attention(q[0], k, v, 0, kv_len - s, SM)}, min_reduce_groups=1)


def mixed_group_reduced_rect() -> Kat:
    """tools/check_mac_persistent_decode.py:737-816: heads 0,1,3 hit, head 2
    misses; group mode 2 (mixed)."""
    rng = np.random.default_rng(23)
    hkv, g = 1, 4
    hq = hkv * g
    m, kv_len, s, maxc = 8, 192, 4, 256
    p = kv_len - 1
    k, v = _bf(rng, kv_len, hkv, D), _bf(rng, kv_len, hkv, D)
    q = _bf(rng, 1, hq, D)
    r2t, ocl = _single_request_layout(kv_len, maxc)
    qc = _bf(rng, 1, m, hq, D, add=10.0)
    ac = np.zeros_like(qc)
    lc = np.full((1, m, hq), -np.inf, np.float32)
    hit_idx = [0, 1, 3]
    mp = 186
    slot = mp % m
    pe = max(mp + 1 - s, 0)
    po, pl = ref_attention(q[0], k, v, 0, pe, SM)
    po = syn.bf16_round(po)
    for h in hit_idx:
        qc[0, slot, h] = q[0, h]
        ac[0, slot, h], lc[0, slot, h] = po[h], pl[h]
    ne = max(p + 1 - s, 0)
    ro, rl = ref_attention(q[0], k, v, pe, ne, SM)
    to, tl = ref_attention(q[0], k, v, ne, kv_len, SM)
    hco, hcl = merge(po, pl, ro, rl)
    hoo, hol = merge(hco, hcl, to, tl)
    fo, fl = ref_attention(q[0], k, v, 0, kv_len, SM)
    fco, fcl = ref_attention(q[0], k, v, 0, ne, SM)
    hit = np.array([h in hit_idx for h in range(hq)])
    return Kat("mixed_group_reduced_rect", _case(q, q, k, v, r2t, ocl, [p], qc, ac, lc, s), maxc,
               4, 4, 8e-2, 3e-2,
               {0: (np.where(hit[:, None], hoo, fo), np.where(hit, hol, fl))},
               {0: (np.where(hit[:, None], hco, fco), np.where(hit, hcl, fcl))},
               head_hit=hit.astype(np.int32)[None], group_mode=np.full((1, hkv), 2, np.int32),
               env={"MAC_PERSISTENT_MIXED_GROUP_FALLBACK": "1"})


ALL = [
    hit_clean_half_open_cache_row,
    miss_multi_request,
    short_context_writes_empty_cache_row,
    tie_breaks_by_logical_position_after_wraparound,
    front_sink_rectification,
    front_sink_mixed_group_exclusion,
    front_sink_group4_mixed_fastpath,
    front_sink_group8_mixed_fastpath,
    front_sink_group4_full_fallback_reduce,
    front_sink_group8_full_fallback_reduce,
    large_miss_reduced_rect,
    mixed_group_reduced_rect,
]


# ------------------------------------------------------- recurrence ----


def recurrence_inputs():
    """tools/check_front_sink_recurrence.py:53-128: two chained steps on a
    GQA-8 group, step 1 mixed (6 hit / 2 miss), step 2 all heads matching the
    row step 1 wrote.  Returns (step1 Case, step-2 builder, expectations)."""
    rng = np.random.default_rng(11)
    hkv, g = 1, 8
    hq = hkv * g
    cap, s, f = 16, 4, 3
    kv_len1, kv_len2 = 20, 21
    p1, p2 = kv_len1 - 1, kv_len1
    k, v = _bf(rng, kv_len2, hkv, D), _bf(rng, kv_len2, hkv, D)
    r2t = np.zeros((1, 64), np.int32)
    r2t[0, :p2] = np.arange(p2, dtype=np.int32)
    q_pre1, q_post1 = _bf(rng, 1, hq, D), _bf(rng, 1, hq, D)
    q_build = _bf(rng, hq, D)
    hit_heads = list(range(6))
    qc = _bf(rng, 1, cap, hq, D, add=10.0)
    ac = np.zeros_like(qc)
    lc = np.full((1, cap, hq), -np.inf, np.float32)
    mp1 = 10
    ms1 = mp1 % cap
    pe1 = mp1 + 1 - s
    ne1 = p1 + 1 - s
    eo, el = ref_attention(q_build, k, v, f, pe1, SM)
    eo = syn.bf16_round(eo)
    for h in hit_heads:
        qc[0, ms1, h] = syn.bf16_round(q_pre1[0, h] + 0.03 * rng.standard_normal(D))
        ac[0, ms1, h], lc[0, ms1, h] = eo[h], el[h]
    step1 = _case(q_post1, q_pre1, k, v, r2t, [p1], [p1], qc, ac, lc, s, f)
    b1o, b1l = ref_attention(q_post1[0], k, v, pe1, ne1, SM)
    e_hit = merge(eo, el, b1o, b1l)
    e_miss = ref_attention(q_post1[0], k, v, f, ne1, SM)
    q_post2 = _bf(rng, 1, hq, D)
    ne2 = p2 + 1 - s
    s2 = ref_attention(q_post2[0], k, v, 0, f, SM)
    r2 = ref_attention(q_post2[0], k, v, ne1, ne2, SM)
    t2 = ref_attention(q_post2[0], k, v, ne2, kv_len2, SM)

    def step2(qc_after, ac_after, lc_after):
        return _case(q_post2, q_pre1.copy(), k, v, r2t, [p2], [p2], qc_after, ac_after, lc_after,
                     s, f)

    def expected_step2(entry_o, entry_l):
        """Exact recurrence reference from the step-1 entries actually written."""
        o, l_ = merge(entry_o, entry_l, *r2)
        o, l_ = merge(o, l_, *s2)
        return merge(o, l_, *t2)

    return dict(step1=step1, step2=step2, hit_heads=hit_heads, e_hit=e_hit, e_miss=e_miss,
                dest1=p1 % cap, p1=p1, expected_step2=expected_step2, hq=hq)
