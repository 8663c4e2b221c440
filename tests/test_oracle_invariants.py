"""Pins the CPU oracle with properties the mathematics fixes (CPU only).

Each check uses a computation independent of the oracle's own code path:
brute-force ring addressing, numpy distances, exact softmax attention over a
single range (closed form of the span/merge composition), and the benchmark's
Python restatement of the synthetic hit hash.
"""

import math

import numpy as np
import pytest

from helpers import bits, oracle_run, orc, ref_attention, rel_l2, syn


# ------------------------------------------------------------ ring ----


@pytest.mark.parametrize("m", [1, 2, 3, 4, 7, 8, 32])
def test_ring_addressing_brute_force(m):
    """slot -> logical position is the unique pos = slot (mod M) in [P-M, P)
    once the ring is full, and the identity before (mac_decode_persistent.cu:798-848)."""
    for past in range(0, 3 * m + 5):
        for slot in range(m):
            pos = orc.ring_slot_to_pos(past, m, slot)
            if past < m:
                assert pos == slot
            else:
                cands = [x for x in range(past - m, past) if x % m == slot % m]
                assert cands == [pos]
            assert orc.pos_to_ring_slot(past, m, pos) == slot
            assert syn.ring_slot_to_pos(past, m, slot) == pos


# ------------------------------------------------------- decisions ----


def _case_with_ring(seed, hq=8, hkv=2, m=8, kv=40, s=4, f=0):
    rng = np.random.default_rng(seed)
    c = syn.random_case(batch=1, hq=hq, hkv=hkv, kv_lens=[kv], capacity=m, semantic_pos_ahead=s,
                        front_sink_tokens=f, hit_rate=0.0, seed=seed)
    return c, rng


def test_match_scan_matches_numpy_distances():
    """Best slot = numpy argmin of squared L2 over the candidate window,
    ties to the smaller logical position; hit iff d < 2D(1-thr)^2 (float32)."""
    for seed in range(6):
        c, rng = _case_with_ring(seed, m=8, kv=40)
        p = int(c.past_lens[0])
        # scatter slots at controlled distances around the threshold distance
        thr_d = np.float32(2.0) * np.float32(128) * np.float32(1 - 0.45) ** 2
        for slot in range(8):
            for h in range(8):
                scale = rng.uniform(0.2, 1.6)
                noise = rng.standard_normal(128)
                noise *= math.sqrt(float(thr_d) * scale) / np.linalg.norm(noise)
                c.query_cache[0, slot, h] = syn.bf16_round(c.q_pre[0, h] + noise)
        c.lse_cache[:] = 0.0
        res = oracle_run(c)
        for h in range(8):
            best, best_pos, best_slot = np.inf, None, None
            for slot in range(8):
                pos = syn.ring_slot_to_pos(p, 8, slot)
                if not (max(0, p - 8) <= pos < p):
                    continue
                d = float(((c.q_pre[0, h].astype(np.float64)
                            - c.query_cache[0, slot, h].astype(np.float64)) ** 2).sum())
                if d < best or (d == best and pos < best_pos):
                    best, best_pos, best_slot = d, pos, slot
            assert res.head["best_dist"][0, h] == pytest.approx(best, rel=1e-12)
            exp_hit = best < float(thr_d)
            assert bool(res.head["hit"][0, h]) == exp_hit
            if exp_hit:
                assert res.head["match_pos"][0, h] == best_pos
                assert res.head["match_slot"][0, h] == best_slot


def test_candidate_mode_and_gen_min_limit():
    c, _ = _case_with_ring(11, m=8, kv=40)
    p = int(c.past_lens[0])
    # plant an exact copy at the most recent position p-1
    slot = syn.pos_to_ring_slot(p, 8, p - 1)
    c.query_cache[0, slot] = c.q_pre[0]
    c.lse_cache[:] = 0.0
    assert oracle_run(c).head["match_pos"][0].tolist() == [p - 1] * 8
    # exclude_recent_right: candidates end at p - lookback_right
    c.candidate_mode, c.lookback_right = 1, 2
    assert oracle_run(c).head["hit"][0].sum() == 0
    c.candidate_mode, c.lookback_right = 0, 0
    # gen_min_limit above past_len makes the request ineligible
    c.gen_min_limit = p + 1
    assert oracle_run(c).head["hit"][0].sum() == 0


def test_front_sink_demotion():
    """A match whose prefix_end < F is demoted to a miss (mac_decode_persistent.cu:1285-1291)."""
    c, _ = _case_with_ring(12, m=16, kv=12, s=4, f=8)
    p = int(c.past_lens[0])
    for pos, expect_hit in ((p - 1, True), (p - 6, False)):
        cc = syn.Case(**{k: (v.copy() if isinstance(v, np.ndarray) else v)
                         for k, v in c.__dict__.items()})
        slot = syn.pos_to_ring_slot(p, 16, pos)
        cc.query_cache[0, slot] = cc.q_pre[0]
        cc.lse_cache[:] = 0.0
        pe = max(pos + 1 - 4, 0)
        res = oracle_run(cc)
        assert bool(res.head["hit"][0].all()) == (expect_hit and pe >= 8), (pos, pe)


# --------------------------------------------------- closed forms ----


@pytest.mark.parametrize("f", [0, 5, 16])
@pytest.mark.parametrize("hit_rate", [0.0, 0.5, 1.0])
def test_exact_entries_reproduce_full_attention(f, hit_rate):
    """With ring entries that are exact attention over [min(F,E), E) under the
    current query, every head's output equals exact attention over [0, kv_len)
    and every written ring row equals exact attention over [min(F,ne), ne),
    whatever the mix of hit, mixed and miss groups."""
    c = syn.random_case(batch=2, hq=16, hkv=4, kv_lens=[300, 411], capacity=16,
                        semantic_pos_ahead=24, front_sink_tokens=f, hit_rate=hit_rate,
                        match_lag=9, seed=40 + f)
    res = oracle_run(c)
    if hit_rate == 1.0:
        assert res.head["hit"].all()
    for n in range(2):
        kv = int(c.past_lens[n]) + 1
        rows = c.req_to_token[n, :kv].copy()
        rows[kv - 1] = c.out_cache_loc[n]
        k, v = c.k[rows], c.v[rows]
        full_o, full_l = ref_attention(c.q_post[n], k, v, 0, kv, c.sm_scale)
        assert rel_l2(bits(res.out[n]), full_o) < 5e-3
        np.testing.assert_allclose(res.out_lse[n], full_l, atol=1e-4)
        ne = max(kv - c.semantic_pos_ahead, 0)
        ring_o, ring_l = ref_attention(c.q_post[n], k, v, min(f, ne), ne, c.sm_scale)
        dest = int(c.past_lens[n]) % 16
        assert rel_l2(bits(res.attn_cache[n, dest]), ring_o) < 5e-3
        np.testing.assert_allclose(res.lse_cache[n, dest], ring_l, atol=1e-4)


def test_readiness_gate_forces_exact_attention_and_skips_ring_write():
    c = syn.random_case(batch=3, hq=8, hkv=2, kv_lens=[100, 120, 140], capacity=8,
                        semantic_pos_ahead=8, hit_rate=1.0, match_lag=3, seed=50,
                        entry_builder="random")
    c.cache_ready = np.array([1, 0, 1], np.uint8)
    c.cache_epoch = np.array([0, 0, 4], np.int64)
    c.request_epoch = np.array([0, 0, 5], np.int64)
    res = oracle_run(c)
    assert res.head["hit"][0].all() and not res.head["hit"][1:].any()
    for n in (1, 2):
        np.testing.assert_array_equal(res.attn_cache[n], syn.to_bits(c.attn_cache[n]))
        np.testing.assert_array_equal(res.lse_cache[n], c.lse_cache[n])
        kv = int(c.past_lens[n]) + 1
        rows = c.req_to_token[n, :kv].copy()
        rows[kv - 1] = c.out_cache_loc[n]
        full_o, _ = ref_attention(c.q_post[n], c.k[rows], c.v[rows], 0, kv, c.sm_scale)
        assert rel_l2(bits(res.out[n]), full_o) < 5e-3


def test_mixed_group_fallback_switch(monkeypatch):
    """MAC_PERSISTENT_MIXED_GROUP_FALLBACK=0 turns partially-hit groups into
    full fallback (mac_decode_persistent.cu:1336-1340)."""
    c = syn.random_case(batch=1, hq=8, hkv=2, kv_lens=[200], capacity=16, semantic_pos_ahead=8,
                        hit_rate=1.0, bench_mode=1, match_lag=5, seed=60)
    # break the planted match of head 1 so that group 0 is partially hit
    slot, _ = c.planted[(0, 1)]
    c.query_cache[0, slot, 1] += 10.0
    monkeypatch.setenv("MAC_PERSISTENT_MIXED_GROUP_FALLBACK", "1")
    r1 = oracle_run(c)
    monkeypatch.setenv("MAC_PERSISTENT_MIXED_GROUP_FALLBACK", "0")
    r0 = oracle_run(c)
    for g in range(2):
        hits = r1.head["hit"][0, 4 * g:4 * g + 4]
        if 0 < hits.sum() < 4:
            assert r1.group["mode"][0, g] == 2 and r0.group["mode"][0, g] == 1
            assert r0.head["hit"][0, 4 * g:4 * g + 4].sum() == 0
    assert r1.group["mode"][0].tolist() == [2, 0] and r0.group["mode"][0].tolist() == [1, 0]


# -------------------------------------------- synthetic bench override ----


@pytest.mark.parametrize("bench_mode", [1, 2])
@pytest.mark.parametrize("hit_rate", [0.0, 0.3, 0.8, 0.95, 1.0])
def test_bench_override_matches_benchmark_restatement(bench_mode, hit_rate):
    """The oracle's in-kernel override (mac_decode_persistent.cu:1184-1269)
    and the benchmark script's host-side planner
    (benchmark/bench_mac_vs_flashinfer_direct.py:134-211), restated in
    mac_attention.synthetic, pick the same heads and match positions."""
    b, hq, hkv, m, s = 3, 16, 4, 32, 16
    c = syn.random_case(batch=b, hq=hq, hkv=hkv, kv_lens=[500] * b, capacity=m,
                        semantic_pos_ahead=s, hit_rate=0.0, seed=70, entry_builder="random")
    c.lse_cache[:] = 0.0
    res = oracle_run(c, bench_mode=bench_mode, bench_hit_rate=hit_rate, bench_seed=3,
                     bench_match_lag_mean=12.0)
    for n in range(b):
        for h in range(hq):
            hit, slot = syn.synthetic_hit_and_slot(
                bench_mode=bench_mode, batch=b, hq=hq, hkv=hkv, past_len=499, n=n, hq_i=h,
                hkv_i=h // (hq // hkv), hit_rate=hit_rate, capacity=m, semantic_pos_ahead=s,
                bench_seed=3, match_lag_mean=12.0)
            assert bool(res.head["hit"][n, h]) == hit, (n, h)
            if hit:
                assert res.head["match_slot"][n, h] == slot
                assert res.head["match_pos"][n, h] == 499 - 12
    misses = (res.head["hit"] == 0).sum()
    units = b * (hq if bench_mode == 1 else hkv)
    per_unit = 1 if bench_mode == 1 else hq // hkv
    assert misses == syn.target_miss_units(hit_rate, units) * per_unit
