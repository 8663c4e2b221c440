"""Pins the CPU oracle of prefill rectification (CPU only).

References: the downdate kernel mac_merge_downdate_cache.cu:116-288 (MERGE),
the windowed FlashInfer pass and the composition in flashinfer_hooks.py:
2436-2482 (HOOKS), the front-sink rule HOOKS:2205-2215.  Checks use
computations independent of the oracle's code: numpy exact attention over a
range (helpers.ref_attention) and numpy LSE merges.
"""

import numpy as np
import pytest

from helpers import bits, merge, orc, ref_attention, rel_l2, syn


def _bf(x):
    return syn.to_bits(syn.bf16_round(np.asarray(x, np.float32)))


# ------------------------------------------------------------ downdate ----


def test_downdate_inverts_merge():
    """downdate(A (+) W, W) = A for states whose lse are well separated."""
    rng = np.random.default_rng(0)
    rows, d = 64, 128
    oa, ow = rng.standard_normal((rows, d)), rng.standard_normal((rows, d))
    la = rng.uniform(-2, 4, rows)
    lw = la + rng.uniform(-3, 0.5, rows)  # window weight up to ~60% of the total
    full_o, full_l = merge(oa, la, ow, lw)
    out1 = _bf(full_o)
    lse1 = full_l.astype(np.float32)
    out2 = _bf(ow)
    lse2 = lw.astype(np.float32)
    orc.update_then_downdate(out1, lse1, out2, lse2)
    assert rel_l2(bits(out2), oa) < 2e-2
    np.testing.assert_allclose(lse2, la, atol=2e-3)


def test_downdate_branches():
    """MERGE:159-174: equal lse -> empty state; lse2 > lse1 -> no-op copy of
    state 1."""
    d = 128
    rng = np.random.default_rng(1)
    o1 = _bf(rng.standard_normal((3, d)))
    o2 = _bf(rng.standard_normal((3, d)))
    lse1 = np.array([1.5, 0.25, 3.0], np.float32)
    lse2 = np.array([1.5, 0.75, 2.0], np.float32)  # equal, larger, regular
    out2 = o2.copy()
    l2 = lse2.copy()
    orc.update_then_downdate(o1, lse1, out2, l2)
    assert l2[0] == -np.inf and not bits(out2[0]).any()
    assert l2[1] == np.float32(0.25)
    np.testing.assert_array_equal(out2[1], o1[1])
    t = np.exp(-1.0)
    r = 3.0 + np.log(1 - t + 1e-7)
    np.testing.assert_allclose(l2[2], r, rtol=1e-6)
    exp_o = (bits(o1[2]).astype(np.float64) - t * bits(o2[2])) * np.exp(3.0 - r)
    assert rel_l2(bits(out2[2]), exp_o) < 5e-3


@pytest.mark.parametrize("dt1,dt2", [("f32", "bf16"), ("f16", "f32"), ("bf16", "f16")])
def test_downdate_lse_dtypes(dt1, dt2):
    """lse1/lse2 may be f32, bf16 or f16 (MERGE:361-400): the result equals
    the f32 computation on the rounded inputs, stored in lse2's type."""
    rng = np.random.default_rng(2)
    rows, d = 16, 128
    o1 = _bf(rng.standard_normal((rows, d)))
    o2 = _bf(rng.standard_normal((rows, d)))
    l1 = rng.uniform(1, 2, rows).astype(np.float32)
    l2 = (l1 - rng.uniform(0.5, 2, rows)).astype(np.float32)

    def enc(x, dt):
        if dt == "f32":
            return x.copy(), False, x.copy()
        if dt == "f16":
            h = x.astype(np.float16)
            return h, False, h.astype(np.float32)
        b = _bf(x)
        return b, True, bits(b)

    a1, f1, v1 = enc(l1, dt1)
    a2, f2, v2 = enc(l2, dt2)
    out2 = o2.copy()
    orc.update_then_downdate(o1, a1, out2, a2, lse1_bf16=f1, lse2_bf16=f2)
    ref_o = o2.copy()
    ref_l = v2.astype(np.float32).copy()
    orc.update_then_downdate(o1, v1.astype(np.float32), ref_o, ref_l)
    np.testing.assert_array_equal(out2, ref_o)
    got = a2.astype(np.float32) if not f2 else bits(a2)
    want = ref_l.astype(np.float16).astype(np.float32) if dt2 == "f16" else (
        bits(_bf(ref_l)) if dt2 == "bf16" else ref_l)
    np.testing.assert_array_equal(got, want)


# ---------------------------------------------------- window attention ----


def _rows_ref(case, b, h, lo_fn, hi_fn):
    """numpy exact attention of every query row of request b, head h over
    [lo_fn(pos), hi_fn(pos))."""
    kb, ke = int(case.kv_indptr[b]), int(case.kv_indptr[b + 1])
    rows = case.kv_indices[kb:ke]
    k, v = case.k[rows], case.v[rows]
    out, lses = [], []
    g = case.q.shape[1] // case.k.shape[1]
    for i, pos in enumerate(case.positions(b)):
        q = case.q[int(case.qo_indptr[b]) + i]
        o, l = ref_attention(q[h:h + 1], k[:, h // g:h // g + 1], v[:, h // g:h // g + 1],
                             lo_fn(pos), hi_fn(pos), case.sm_scale)
        out.append(o[0])
        lses.append(l[0])
    return np.array(out), np.array(lses)


@pytest.mark.parametrize("window_left", [-1, 0, 5, 40, 1000])
def test_window_attention_matches_numpy(window_left):
    case = syn.prefill_case(qo_lens=[7, 33, 1], kv_lens=[20, 33, 50], hq=4, hkv=2, seed=3)
    o, lse = orc.window_attention(_bf(case.q), _bf(case.k), _bf(case.v), case.qo_indptr,
                                  case.kv_indptr, case.kv_indices, window_left=window_left,
                                  sm_scale=case.sm_scale)
    for b in range(3):
        for h in range(4):
            lo = (lambda p: 0) if window_left < 0 else (lambda p: max(p - window_left, 0))
            ro, rl = _rows_ref(case, b, h, lo, lambda p: p + 1)
            r0, r1 = int(case.qo_indptr[b]), int(case.qo_indptr[b + 1])
            assert rel_l2(bits(o[r0:r1, h]), ro) < 5e-3
            np.testing.assert_allclose(lse[r0:r1, h], rl, atol=1e-5)


# ---------------------------------------------------------- rectify ----


def _rectify(case, *, S, F, sink_mode, M, request_length, req_ids, q_post_cache=False):
    hq = case.q.shape[1]
    full_o, full_l = orc.window_attention(_bf(case.q), _bf(case.k), _bf(case.v), case.qo_indptr,
                                          case.kv_indptr, case.kv_indices, window_left=-1,
                                          sm_scale=case.sm_scale)
    R = 4
    rng = np.random.default_rng(9)
    ring = dict(q=_bf(rng.standard_normal((R, M, hq, 128))),
                a=_bf(rng.standard_normal((R, M, hq, 128))),
                l=rng.standard_normal((R, M, hq)).astype(np.float32),
                qp=np.zeros((R, M, hq, 128), np.uint16) if q_post_cache else None)
    src_q = _bf(case.q * 0.5 + 1.0)  # stands for pre-RoPE rows
    rl = np.array(request_length, np.int32)
    orc.rectify_update_cache(_bf(case.q), src_q, full_o, full_l, _bf(case.k), _bf(case.v),
                             case.qo_indptr, case.kv_indptr, case.kv_indices, ring["q"], ring["a"],
                             ring["l"], rl, np.array(req_ids, np.int32), semantic_pos_ahead=S,
                             front_sink_tokens=F, sink_mode=sink_mode, sm_scale=case.sm_scale,
                             q_post_cache=ring["qp"])
    return ring, rl, src_q, full_o, full_l


@pytest.mark.parametrize("F,sink_mode", [(0, 0), (3, 0), (3, 1), (40, 1)])
def test_rectify_rows_are_prefix_states(F, sink_mode):
    """Kept rows hold exact attention over [0, E) (sink_mode 1: [min(F,E), E)),
    E = pos + 1 - S; lse -inf when F > 0 in sink_mode 0 (HOOKS:2205-2215) or
    when nothing is left."""
    S, M = 8, 6
    case = syn.prefill_case(qo_lens=[10, 4, 30], kv_lens=[10, 24, 60], hq=4, hkv=2, seed=4)
    req_ids = [2, 0, 3]
    before = np.array([5, 100, 0, 77], np.int32)
    ring, rl, src_q, _, full_l = _rectify(case, S=S, F=F, sink_mode=sink_mode, M=M,
                                     request_length=before, req_ids=req_ids, q_post_cache=True)
    for b, req in enumerate(req_ids):
        n = int(case.qo_indptr[b + 1] - case.qo_indptr[b])
        assert rl[req] == before[req] + n
        start = max(n - M, 0)
        for i in range(start, n):
            slot = (int(before[req]) + i) % M
            pos = case.positions(b)[i]
            e = pos + 1 - S
            row = int(case.qo_indptr[b]) + i
            np.testing.assert_array_equal(ring["q"][req, slot], src_q[row])
            assert (ring["qp"][req, slot] == 0x7FC0).all()
            for h in range(4):
                lo = min(F, e) if sink_mode == 1 else 0
                if e <= (F if sink_mode == 1 else 0) or e <= 0:
                    assert ring["l"][req, slot, h] == -np.inf
                    assert not bits(ring["a"][req, slot, h]).any()
                    continue
                ro, rlse = _rows_ref(case, b, h, lambda p: lo, lambda p: p + 1 - S)
                # the downdate divides by the prefix's share of the full softmax
                # mass, amplifying the bf16 rounding of o_full by that factor
                amp = float(np.exp(full_l[row, h] - rlse[i]))
                assert rel_l2(bits(ring["a"][req, slot, h]), ro[i]) < 5e-3 * (1 + amp), (b, i, h)
                if F > 0 and sink_mode == 0:
                    assert ring["l"][req, slot, h] == -np.inf
                else:
                    np.testing.assert_allclose(ring["l"][req, slot, h], rlse[i], atol=2e-3)


def test_rectify_equals_reference_composition():
    """With F = 0 the fused op equals the reference's three calls
    (HOOKS:2436-2482): window attention (window_left = S-1), downdate of the
    full state, then mac_prefill_update_cache with offsets = qo_indptr."""
    S, M, hq = 6, 5, 4
    case = syn.prefill_case(qo_lens=[9, 12], kv_lens=[30, 12], hq=hq, hkv=1, seed=5)
    req_ids = [1, 0]
    before = np.array([3, 8], np.int32)
    ring, rl, src_q, full_o, full_l = _rectify(case, S=S, F=0, sink_mode=0, M=M,
                                               request_length=before, req_ids=req_ids)
    wo, wl = orc.window_attention(_bf(case.q), _bf(case.k), _bf(case.v), case.qo_indptr,
                                  case.kv_indptr, case.kv_indices, window_left=S - 1,
                                  sm_scale=case.sm_scale)
    orc.update_then_downdate(full_o, full_l, wo, wl)
    rng = np.random.default_rng(9)
    R = 4
    q2 = _bf(rng.standard_normal((R, M, hq, 128)))
    a2 = _bf(rng.standard_normal((R, M, hq, 128)))
    l2 = rng.standard_normal((R, M, hq)).astype(np.float32)
    rl2 = before.copy()
    lens = np.diff(case.qo_indptr).astype(np.int32)
    orc.prefill_update_cache(q2, a2, l2, rl2, np.array(req_ids, np.int32), src_q, wo, wl,
                             case.qo_indptr, lens, M, hq, 128)
    np.testing.assert_array_equal(rl, rl2)
    np.testing.assert_array_equal(ring["q"], q2)
    # rows whose prefix is empty: the composition's value depends on rounding
    # (both passes cover the same keys), the fused op writes the empty state
    ok = np.isfinite(l2) & np.isfinite(ring["l"])
    assert ok.sum() > 0.5 * ok.size
    np.testing.assert_allclose(ring["l"][ok], l2[ok], atol=2e-3)
    assert rel_l2(bits(ring["a"])[ok], bits(a2)[ok]) < 2e-2
