"""Prefill rectification on the GPU against the CPU oracle: the downdate op
(mac_merge_downdate_cache.cu:116-401), the windowed prefill attention
(flashinfer_hooks.py:2436-2467) and the fused rectify + ring update.

Tolerances: integer/byte outputs (ring queries, NaN markers, request_length,
untouched rows) bit-exact; bf16 outputs within 1e-2 relative L2, widened by
the downdate's amplification of its input rounding where it applies.
"""

import math

import numpy as np
import pytest

from helpers import bits, orc, rel_l2, syn

torch = pytest.importorskip("torch")

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def merge_ext():
    from mac_attention.integrations.sglang.bridge import load_mac_merge_downdate_cache_extension

    return load_mac_merge_downdate_cache_extension(False)


@pytest.fixture(scope="module")
def rect_ext():
    from mac_attention.integrations.sglang.bridge import load_mac_prefill_rectify_extension

    return load_mac_prefill_rectify_extension(False)


@pytest.fixture(scope="module")
def cache_ext():
    from mac_attention.integrations.sglang.bridge import load_mac_prefill_update_cache_extension

    return load_mac_prefill_update_cache_extension(False)


def _bf(x):
    return syn.to_bits(syn.bf16_round(np.asarray(x, np.float32)))


def _dev_bits(b):
    """uint16 bf16 bits -> CUDA bf16 tensor (bit-exact)."""
    t = torch.from_numpy(np.ascontiguousarray(b).view(np.int16)).cuda()
    return t.view(torch.bfloat16)


def _host_bits(t):
    return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def _i32(a):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.int32)).cuda()


# ------------------------------------------------------------ downdate ----


@pytest.mark.parametrize("d", [128, 64, 100])
@pytest.mark.parametrize("dts", [(torch.float32, torch.float32), (torch.float32, torch.bfloat16),
                                 (torch.float16, torch.float32), (torch.bfloat16, torch.float16)])
def test_downdate_matches_oracle(merge_ext, d, dts):
    rng = np.random.default_rng(d)
    n, h = 37, 8
    o1 = _bf(rng.standard_normal((n, h, d)))
    o2 = _bf(rng.standard_normal((n, h, d)))
    # multiples of 1/64 below 4 are exact in f32, bf16 and f16, so the
    # special rows below keep their relation after the dtype conversion
    l1 = (np.round(rng.uniform(0, 3, (n, h)) * 64) / 64).astype(np.float32)
    l2 = (l1 - rng.uniform(0.05, 4, (n, h))).astype(np.float32)
    l2[0, :4] = l1[0, :4]          # nothing left
    l2[1, :4] = l1[1, :4] + 0.5    # invalid -> copy of state 1
    t1, t2 = (torch.from_numpy(l1).cuda().to(dts[0]), torch.from_numpy(l2).cuda().to(dts[1]))
    # oracle on the exact values the GPU sees
    r1 = t1.float().cpu().numpy()
    r2 = t2.float().cpu().numpy().copy()
    ro = o2.copy()
    orc.update_then_downdate(o1, r1, ro, r2)
    g1, g2 = _dev_bits(o1), _dev_bits(o2)
    merge_ext.mac_update_then_downdate_bf16_inplace(g1, t1, g2, t2)
    torch.cuda.synchronize()
    got_o = bits(_host_bits(g2))
    got_l = t2.float().cpu().numpy()
    exp_l = torch.from_numpy(r2).to(dts[1]).float().numpy()
    np.testing.assert_array_equal(np.isinf(got_l), np.isinf(exp_l))
    fin = np.isfinite(exp_l)
    np.testing.assert_allclose(got_l[fin], exp_l[fin], rtol=1e-2 if dts[1] != torch.float32 else 1e-5,
                               atol=1e-5)
    assert rel_l2(got_o, bits(ro)) < 1e-2
    np.testing.assert_array_equal(_host_bits(g2)[1, :4], o1[1, :4])
    assert not got_o[0, :4].any()


def test_downdate_rejects_bad_dtype(merge_ext):
    x = torch.zeros(2, 2, 128, dtype=torch.bfloat16, device="cuda")
    with pytest.raises(RuntimeError, match="lse2 must be float32, bfloat16, or float16"):
        merge_ext.mac_update_then_downdate_bf16_inplace(
            x, torch.zeros(2, 2, device="cuda"), x.clone(), torch.zeros(2, 2, device="cuda", dtype=torch.int32))


# ---------------------------------------------------- window attention ----


def _dev_case(case):
    return dict(q=_dev_bits(_bf(case.q)), k=_dev_bits(_bf(case.k)), v=_dev_bits(_bf(case.v)),
                qo=_i32(case.qo_indptr), kv=_i32(case.kv_indptr), idx=_i32(case.kv_indices))


@pytest.mark.parametrize("window_left", [-1, 0, 5, 255, 1000])
@pytest.mark.parametrize("hq,hkv", [(8, 2), (8, 8), (16, 2), (6, 2), (32, 2), (10, 2), (14, 2)])
def test_window_attention_matches_oracle(rect_ext, window_left, hq, hkv):
    case = syn.prefill_case(qo_lens=[1, 17, 300, 0, 64], kv_lens=[1, 40, 700, 9, 64], hq=hq,
                            hkv=hkv, seed=11 + hq + hkv)
    d = _dev_case(case)
    out, lse = rect_ext.window_attention_return_lse(d["q"], d["k"], d["v"], d["qo"], d["kv"], d["idx"],
                                                    window_left, case.sm_scale)
    torch.cuda.synchronize()
    eo, el = orc.window_attention(_bf(case.q), _bf(case.k), _bf(case.v), case.qo_indptr,
                                  case.kv_indptr, case.kv_indices, window_left=window_left,
                                  sm_scale=case.sm_scale)
    got = bits(_host_bits(out))
    for r in range(got.shape[0]):
        assert rel_l2(got[r], bits(eo[r])) < 1e-2, r
    np.testing.assert_allclose(lse.cpu().numpy(), el, atol=2e-4, rtol=1e-5)


@pytest.mark.parametrize("seed", range(6))
def test_window_attention_random_shapes(rect_ext, seed):
    """Random batches against the oracle: chunk and prefix lengths (row
    blocks cut short, empty chunks), GQA shapes of both kernel instances
    with absent heads, causal and windowed."""
    rng = np.random.default_rng(300 + seed)
    B = int(rng.integers(1, 7))
    hq, hkv = [(8, 2), (12, 2), (6, 2), (32, 4), (3, 1), (16, 2)][seed % 6]
    qo = rng.integers(0, 90, B)
    kv = qo + rng.integers(0, 150, B)
    window_left = int(rng.choice([-1, 0, 7, 63, 200]))
    print(f"window random shapes: seed={seed} B={B} G={hq // hkv} window_left={window_left}", flush=True)
    case = syn.prefill_case(qo_lens=qo.tolist(), kv_lens=kv.tolist(), hq=hq, hkv=hkv, seed=400 + seed)
    d = _dev_case(case)
    out, lse = rect_ext.window_attention_return_lse(d["q"], d["k"], d["v"], d["qo"], d["kv"], d["idx"],
                                                    window_left, case.sm_scale)
    torch.cuda.synchronize()
    eo, el = orc.window_attention(_bf(case.q), _bf(case.k), _bf(case.v), case.qo_indptr,
                                  case.kv_indptr, case.kv_indices, window_left=window_left,
                                  sm_scale=case.sm_scale)
    got = bits(_host_bits(out))
    for r in range(got.shape[0]):
        assert rel_l2(got[r], bits(eo[r])) < 1e-2, r
    np.testing.assert_allclose(lse.cpu().numpy(), el, atol=2e-4, rtol=1e-5)


@pytest.mark.parametrize("hkv", [16, 8, 4])
def test_window_attention_is_deterministic(rect_ext, hkv):
    """The same inputs give the same bits on every call, for both kernel
    instances (one head per wave for G <= 4, two above).  A row maximum that
    read the score MFMA's result registers before the MFMA had written them
    made G <= 4 differ by an ulp between calls in ~2% of the rows past the
    first key block."""
    B, chunk, hq, S, D = 4, 1024, 32, 256, 128
    rows = B * chunk
    print(f"window determinism: G={hq // hkv}", flush=True)
    g = torch.Generator(device="cuda")
    g.manual_seed(5)
    k = torch.randn(rows, hkv, D, device="cuda", dtype=torch.bfloat16, generator=g)
    v = torch.randn_like(k)
    q = torch.randn(rows, hq, D, device="cuda", dtype=torch.bfloat16, generator=g)
    qo = torch.arange(0, rows + 1, chunk, device="cuda", dtype=torch.int32)
    idx = torch.randperm(rows, device="cuda", generator=g).to(torch.int32)
    runs = []
    for _ in range(3):
        out, lse = rect_ext.window_attention_return_lse(q, k, v, qo, qo, idx, S - 1, 1.0 / math.sqrt(D))
        torch.cuda.synchronize()
        runs.append((out.view(torch.int16).clone(), lse.view(torch.int32).clone()))
    for out, lse in runs[1:]:
        assert torch.equal(out, runs[0][0]) and torch.equal(lse, runs[0][1])


@pytest.mark.parametrize("window_left", [255, -1])
def test_window_attention_full_grid_rounds(rect_ext, window_left):
    """8 requests x 300 rows at GQA-8: 608 tasks, one whole round of the
    512-workgroup grid and a partial one, so the windowed pass's KV-head-major,
    XCD-contiguous mapping and the partial round's plain order both run (the
    causal pass keeps row-block order); against the oracle."""
    case = syn.prefill_case(qo_lens=[300] * 8, kv_lens=[350] * 8, hq=32, hkv=4, seed=62)
    print(f"window full grid rounds: window_left={window_left}", flush=True)
    d = _dev_case(case)
    out, lse = rect_ext.window_attention_return_lse(d["q"], d["k"], d["v"], d["qo"], d["kv"], d["idx"],
                                                    window_left, case.sm_scale)
    torch.cuda.synchronize()
    eo, el = orc.window_attention(_bf(case.q), _bf(case.k), _bf(case.v), case.qo_indptr,
                                  case.kv_indptr, case.kv_indices, window_left=window_left,
                                  sm_scale=case.sm_scale)
    got = bits(_host_bits(out))
    for r in range(got.shape[0]):
        assert rel_l2(got[r], bits(eo[r])) < 1e-2, r
    np.testing.assert_allclose(lse.cpu().numpy(), el, atol=2e-4, rtol=1e-5)


def test_window_attention_many_requests(rect_ext):
    """4096 requests (the planner's maximum; its per-request tables then take
    49 KB of LDS), most of them a few rows long, some empty, one long."""
    rng = np.random.default_rng(12)
    qo = rng.integers(0, 4, 4096)
    qo[7] = 300
    kv = qo + rng.integers(0, 6, 4096)
    case = syn.prefill_case(qo_lens=qo.tolist(), kv_lens=kv.tolist(), hq=8, hkv=2, seed=12)
    d = _dev_case(case)
    out, lse = rect_ext.window_attention_return_lse(d["q"], d["k"], d["v"], d["qo"], d["kv"], d["idx"],
                                                    40, case.sm_scale)
    torch.cuda.synchronize()
    eo, el = orc.window_attention(_bf(case.q), _bf(case.k), _bf(case.v), case.qo_indptr,
                                  case.kv_indptr, case.kv_indices, window_left=40,
                                  sm_scale=case.sm_scale)
    got = bits(_host_bits(out))
    assert rel_l2(got, bits(eo)) < 1e-2
    np.testing.assert_allclose(lse.cpu().numpy(), el, atol=2e-4, rtol=1e-5)


# ---------------------------------------------------------- rectify ----


def _ring(rng, r, m, hq):
    return (_bf(rng.standard_normal((r, m, hq, 128))), _bf(rng.standard_normal((r, m, hq, 128))),
            rng.standard_normal((r, m, hq)).astype(np.float32))


def _run_rectify(rect_ext, case, *, S, F, sink_mode, M, R, req_ids, request_length, q_post_cache,
                 full=None, seed=0):
    hq = case.q.shape[1]
    rng = np.random.default_rng(seed)
    if full is None:
        full = orc.window_attention(_bf(case.q), _bf(case.k), _bf(case.v), case.qo_indptr,
                                    case.kv_indptr, case.kv_indices, window_left=-1,
                                    sm_scale=case.sm_scale)
    full_o, full_l = full
    src_q = _bf(rng.standard_normal(case.q.shape))
    qc, ac, lc = _ring(rng, R, M, hq)
    qp = np.zeros((R, M, hq, 128), np.uint16) if q_post_cache else None
    rl = np.array(request_length, np.int32)
    # oracle
    e = dict(q=qc.copy(), a=ac.copy(), l=lc.copy(), qp=None if qp is None else qp.copy(), rl=rl.copy())
    orc.rectify_update_cache(_bf(case.q), src_q, full_o, full_l, _bf(case.k), _bf(case.v),
                             case.qo_indptr, case.kv_indptr, case.kv_indices, e["q"], e["a"], e["l"],
                             e["rl"], np.array(req_ids, np.int32), semantic_pos_ahead=S,
                             front_sink_tokens=F, sink_mode=sink_mode, sm_scale=case.sm_scale,
                             q_post_cache=e["qp"])
    # GPU
    d = _dev_case(case)
    g = dict(q=_dev_bits(qc), a=_dev_bits(ac), l=torch.from_numpy(lc).cuda(),
             qp=None if qp is None else _dev_bits(qp), rl=_i32(rl))
    rect_ext.mac_prefill_rectify_update_cache(
        d["q"], _dev_bits(src_q), _dev_bits(full_o), torch.from_numpy(full_l).cuda(), d["k"], d["v"],
        d["qo"], d["kv"], d["idx"], g["q"], g["a"], g["l"], g["rl"], _i32(req_ids), S, F,
        case.sm_scale, q_post_cache=g["qp"], sink_mode=sink_mode)
    torch.cuda.synchronize()
    # amplification exp(lse_full - lse_prefix) of each written ring row: the
    # downdate divides by the prefix's share of the softmax mass
    amp = np.ones((R, M, hq))
    by_batch = len(request_length) == len(req_ids)  # this form wins when R == B
    for b, req in enumerate(req_ids):
        n = int(case.qo_indptr[b + 1] - case.qo_indptr[b])
        if n <= 0 or not 0 <= req < R:
            continue
        before = max(int(request_length[b] if by_batch else request_length[req]), 0)
        for i in range(max(n - M, 0), n):
            slot = (before + i) % M
            row = int(case.qo_indptr[b]) + i
            for h in range(hq):
                if np.isfinite(e["l"][req, slot, h]):
                    amp[req, slot, h] = float(np.exp(full_l[row, h] - e["l"][req, slot, h]))
    e["amp"] = amp
    return e, g, full_l


def _compare_ring(e, g, what):
    np.testing.assert_array_equal(g["rl"].cpu().numpy(), e["rl"], err_msg=f"{what} request_length")
    np.testing.assert_array_equal(_host_bits(g["q"]), e["q"], err_msg=f"{what} ring q")
    if e["qp"] is not None:
        np.testing.assert_array_equal(_host_bits(g["qp"]), e["qp"], err_msg=f"{what} q_post NaN rows")
    gl = g["l"].cpu().numpy()
    np.testing.assert_array_equal(np.isinf(gl), np.isinf(e["l"]), err_msg=f"{what} lse -inf pattern")
    fin = np.isfinite(e["l"])
    # 2e-3, widened like the o rows below: an error d of the window state's
    # lse moves the downdated lse by d (amp - 1)
    tol = 2e-3 * np.maximum(1.0, 0.5 * (1.0 + e["amp"]))
    bad = np.abs(gl - e["l"]) > tol
    assert not (bad & fin).any(), \
        f"{what} ring lse: {np.argwhere(bad & fin)[:5].tolist()} off by {np.abs(gl - e['l'])[bad & fin][:5]}"
    ga, ea = bits(_host_bits(g["a"])), bits(e["a"])
    r, m, hq, _ = ea.shape
    for i in range(r):
        for s in range(m):
            for h in range(hq):
                # 1e-2 relative L2, widened by the downdate's amplification
                # (rows the call did not touch have amp 1 and match exactly)
                err = rel_l2(ga[i, s, h], ea[i, s, h])
                assert err < 1e-2 * max(1.0, 0.5 * (1.0 + e["amp"][i, s, h])), \
                    f"{what} ring o at ({i},{s},{h}): rel_l2 {err:.3e}, amp {e['amp'][i, s, h]:.2f}"


@pytest.mark.parametrize("F,sink_mode", [(0, 0), (4, 0), (4, 1), (64, 1)])
def test_rectify_matches_oracle(rect_ext, F, sink_mode):
    S, M, R = 16, 12, 6
    case = syn.prefill_case(qo_lens=[30, 5, 100, 12, 0], kv_lens=[30, 50, 180, 12, 3], hq=8, hkv=2,
                            seed=21)
    req_ids = [4, 0, 2, 5, 1]
    e, g, _ = _run_rectify(rect_ext, case, S=S, F=F, sink_mode=sink_mode, M=M, R=R, req_ids=req_ids,
                           request_length=[3, 10, 0, 7, 2, 100], q_post_cache=True, seed=F)
    _compare_ring(e, g, f"F={F} sink_mode={sink_mode}")


def test_rectify_by_batch_request_length_and_bad_request(rect_ext):
    """request_length indexed by batch row (not bumped) and a request id
    outside [0, R) (its rows are skipped), PREFILL:201-269."""
    S, M, R = 8, 16, 3
    case = syn.prefill_case(qo_lens=[40, 20, 9], kv_lens=[60, 20, 9], hq=4, hkv=4, seed=23)
    e, g, _ = _run_rectify(rect_ext, case, S=S, F=0, sink_mode=0, M=M, R=R, req_ids=[2, 7, 0],
                           request_length=[5, 6, 7], q_post_cache=False, seed=5)
    _compare_ring(e, g, "by-batch")
    np.testing.assert_array_equal(g["rl"].cpu().numpy(), [5, 6, 7])


@pytest.mark.parametrize("seed", range(6))
def test_rectify_random_shapes(rect_ext, seed):
    """Random batches against the oracle: request and prefix lengths (empty
    chunks, chunks shorter and longer than the ring, prefixes shorter and
    longer than the window), GQA shapes of both kernel instances, window,
    front sink, sink mode and ring size drawn per seed."""
    rng = np.random.default_rng(100 + seed)
    B = int(rng.integers(1, 9))
    hq, hkv = [(8, 2), (16, 2), (6, 2), (32, 4), (4, 1), (12, 4)][seed % 6]
    qo = rng.integers(0, 70, B)
    kv = qo + rng.integers(0, 120, B)
    S = int(rng.choice([8, 16, 64]))
    F = int(rng.choice([0, 4, 20]))
    sink_mode = int(rng.integers(0, 2)) if F > 0 else 0
    M = int(rng.choice([4, 12, 32]))
    R = B + 2
    print(f"rectify random shapes: seed={seed} B={B} G={hq // hkv} S={S} F={F} sink_mode={sink_mode} M={M}",
          flush=True)
    case = syn.prefill_case(qo_lens=qo.tolist(), kv_lens=kv.tolist(), hq=hq, hkv=hkv, seed=200 + seed)
    e, g, _ = _run_rectify(rect_ext, case, S=S, F=F, sink_mode=sink_mode, M=M, R=R,
                           req_ids=rng.permutation(R)[:B].tolist(),
                           request_length=rng.integers(0, 40, R).tolist(), q_post_cache=bool(seed % 2),
                           seed=seed)
    _compare_ring(e, g, f"random seed={seed}")


@pytest.mark.parametrize("hq,hkv", [(6, 2), (12, 2)])
def test_rectify_group_with_absent_heads(rect_ext, hq, hkv):
    """GQA groups of 3 and 6 heads: a task covers 4 (one head per wave) or
    8 (two) heads, so its last heads are absent -- their query and full-state
    rows are read from the group's first head and never stored -- with the
    front sink as its own key segment."""
    case = syn.prefill_case(qo_lens=[40, 7, 33], kv_lens=[70, 7, 90], hq=hq, hkv=hkv, seed=71 + hq)
    e, g, _ = _run_rectify(rect_ext, case, S=16, F=4, sink_mode=1, M=20, R=4, req_ids=[3, 0, 1],
                           request_length=[5, 0, 13, 2], q_post_cache=True, seed=hq)
    _compare_ring(e, g, f"G={hq // hkv}")


@pytest.mark.parametrize("hq", [8, 16])
def test_rectify_many_requests(rect_ext, hq):
    """4096 requests (the planner's maximum: its per-request tables take 49 KB
    of LDS beside the fused form's own tiles and full-state rows; hq 8 and 16
    over 2 KV heads run the one- and the two-head-per-wave form), most a few
    rows long, some empty, one longer than the ring, in permuted ring rows."""
    rng = np.random.default_rng(31 + hq)
    B, M = 4096, 4
    qo = rng.integers(0, 4, B)
    qo[5] = 40
    kv = qo + rng.integers(0, 20, B)
    case = syn.prefill_case(qo_lens=qo.tolist(), kv_lens=kv.tolist(), hq=hq, hkv=2, seed=31 + hq)
    e, g, _ = _run_rectify(rect_ext, case, S=8, F=0, sink_mode=0, M=M, R=B + 1,
                           req_ids=rng.permutation(B).tolist(),
                           request_length=rng.integers(0, 50, B + 1).tolist(), q_post_cache=True, seed=hq)
    _compare_ring(e, g, f"4096 requests, hq={hq}")


def test_rectify_skips_requests_outside_the_buffers(rect_ext):
    """The fused rectification skips a request with fewer keys than queries
    and one whose key range runs past kv_indices, as the window pass does:
    no ring row is written and request_length is not bumped for them (the
    oracle applies the same rule); the other requests are rectified."""
    S, M, R = 8, 16, 5  # R != B: request_length indexed by request (and bumped)
    case = syn.prefill_case(qo_lens=[30, 10, 12, 8], kv_lens=[40, 10, 20, 16], hq=4, hkv=2, seed=29)
    case.kv_indptr = case.kv_indptr.copy()
    case.kv_indptr[2] = 45                 # request 1: 5 keys for 10 queries
    case.kv_indices = case.kv_indices[:80]  # request 3: keys [70, 86) past the 80 entries
    full = orc.window_attention(_bf(case.q), _bf(case.k), _bf(case.v), case.qo_indptr, case.kv_indptr,
                                np.concatenate([case.kv_indices, np.zeros(6, np.int32)]), window_left=-1,
                                sm_scale=case.sm_scale)
    e, g, _ = _run_rectify(rect_ext, case, S=S, F=0, sink_mode=0, M=M, R=R, req_ids=[0, 1, 2, 3],
                           request_length=[100, 200, 300, 400, 500], q_post_cache=False, full=full, seed=9)
    _compare_ring(e, g, "out-of-buffer requests")
    np.testing.assert_array_equal(g["rl"].cpu().numpy(), [130, 200, 312, 400, 500])


def test_rectify_equals_gpu_composition(rect_ext, merge_ext, cache_ext):
    """The fused op equals the reference's three calls run on the GPU
    (window pass -> downdate -> mac_prefill_update_cache), rows with E > 0."""
    S, M, R, hq = 32, 24, 3, 8
    case = syn.prefill_case(qo_lens=[200, 50], kv_lens=[300, 50], hq=hq, hkv=2, seed=31)
    full = orc.window_attention(_bf(case.q), _bf(case.k), _bf(case.v), case.qo_indptr,
                                case.kv_indptr, case.kv_indices, window_left=-1, sm_scale=case.sm_scale)
    e, g, _ = _run_rectify(rect_ext, case, S=S, F=0, sink_mode=0, M=M, R=R, req_ids=[2, 0],
                           request_length=[4, 0, 9], q_post_cache=False, full=full, seed=7)
    d = _dev_case(case)
    wo, wl = rect_ext.window_attention_return_lse(d["q"], d["k"], d["v"], d["qo"], d["kv"], d["idx"],
                                                  S - 1, case.sm_scale)
    merge_ext.mac_update_then_downdate_bf16_inplace(_dev_bits(full[0]), torch.from_numpy(full[1]).cuda(),
                                                    wo, wl)
    rng = np.random.default_rng(7)
    src_q = _bf(rng.standard_normal(case.q.shape))
    qc, ac, lc = _ring(rng, R, M, hq)
    q2, a2, l2 = _dev_bits(qc), _dev_bits(ac), torch.from_numpy(lc).cuda()
    rl2 = _i32([4, 0, 9])
    lens = _i32(np.diff(case.qo_indptr))
    cache_ext.mac_prefill_update_cache(q2, a2, l2, rl2, _i32([2, 0]), _dev_bits(src_q), wo, wl, d["qo"],
                                       lens, M, hq, 128, torch.empty(0, device="cuda", dtype=torch.bfloat16))
    torch.cuda.synchronize()
    np.testing.assert_array_equal(rl2.cpu().numpy(), g["rl"].cpu().numpy())
    assert torch.equal(q2, g["q"])
    fl, cl = g["l"].cpu().numpy(), l2.cpu().numpy()
    ok = np.isfinite(fl) & np.isfinite(cl)
    assert ok.mean() > 0.5
    np.testing.assert_allclose(fl[ok], cl[ok], atol=2e-3)
    assert rel_l2(bits(_host_bits(g["a"]))[ok], bits(_host_bits(a2))[ok]) < 2e-2


def test_rectify_config4_chunk(rect_ext):
    """Config-4 scale: four requests, 8192-row prefill chunks after prefixes
    of up to 24K tokens, GQA-8, S = 256, M = 32, F = 128 (both sink modes);
    the full state of the kept rows comes from the oracle."""
    hq, hkv, S, M, F, chunk = 32, 4, 256, 32, 128, 8192
    kv_lens = [chunk, chunk + 4096, chunk + 24000, chunk + 1]
    case = syn.prefill_case(qo_lens=[chunk] * 4, kv_lens=kv_lens, hq=hq, hkv=hkv, seed=41)
    # full causal state of the kept rows only (the other rows are never read)
    kept = np.concatenate([np.arange(int(case.qo_indptr[b + 1]) - M, int(case.qo_indptr[b + 1]))
                           for b in range(4)])
    sub_qo = np.arange(0, 5 * M, M, dtype=np.int32)
    fo, fl = orc.window_attention(_bf(case.q[kept]), _bf(case.k), _bf(case.v), sub_qo,
                                  case.kv_indptr, case.kv_indices, window_left=-1,
                                  sm_scale=case.sm_scale)
    full_o = _bf(np.random.default_rng(0).standard_normal(case.q.shape))
    full_l = np.zeros(case.q.shape[:2], np.float32)
    full_o[kept], full_l[kept] = fo, fl
    for sink_mode in (0, 1):
        e, g, _ = _run_rectify(rect_ext, case, S=S, F=F, sink_mode=sink_mode, M=M, R=4,
                               req_ids=[3, 1, 0, 2], request_length=[0, 17, 4096, 31],
                               q_post_cache=True, full=(full_o, full_l), seed=sink_mode)
        _compare_ring(e, g, f"config4 sink_mode={sink_mode}")
        if sink_mode == 1:
            assert np.isfinite(g["l"].cpu().numpy()).all()


@pytest.mark.parametrize("hkv", [4, 8])
def test_rectify_full_grid_rounds(rect_ext, hkv):
    """64 requests with two kept row blocks each: 512 tasks at GQA-8 (one
    whole round of the persistent grid) and 1024 at GQA-4 (two), so every
    task runs through the XCD-contiguous task mapping; ring rows against the
    oracle."""
    hq, S, M, F, B = 32, 128, 32, 0, 64
    rng = np.random.default_rng(63 + hkv)
    kv_lens = (40 + rng.integers(0, 200, B)).tolist()
    case = syn.prefill_case(qo_lens=[40] * B, kv_lens=kv_lens, hq=hq, hkv=hkv, seed=64 + hkv)
    print(f"rectify full grid rounds: hkv={hkv}", flush=True)
    kept = np.concatenate([np.arange(int(case.qo_indptr[b + 1]) - M, int(case.qo_indptr[b + 1]))
                           for b in range(B)])
    sub_qo = np.arange(0, (B + 1) * M, M, dtype=np.int32)
    fo, fl = orc.window_attention(_bf(case.q[kept]), _bf(case.k), _bf(case.v), sub_qo,
                                  case.kv_indptr, case.kv_indices, window_left=-1,
                                  sm_scale=case.sm_scale)
    full_o = _bf(rng.standard_normal(case.q.shape))
    full_l = np.zeros(case.q.shape[:2], np.float32)
    full_o[kept], full_l[kept] = fo, fl
    e, g, _ = _run_rectify(rect_ext, case, S=S, F=F, sink_mode=0, M=M, R=B,
                           req_ids=rng.permutation(B).tolist(), request_length=rng.integers(0, 90, B).tolist(),
                           q_post_cache=True, full=(full_o, full_l), seed=hkv)
    _compare_ring(e, g, f"full grid rounds hkv={hkv}")


@pytest.mark.parametrize("hkv", [8, 4])
def test_rectify_is_deterministic(rect_ext, hkv):
    """The fused op gives the same ring rows and lengths on every call, for
    both kernel instances (G = 4 and 8), with the front sink (F = 128, sink
    mode 1) as its own key segment."""
    B, chunk, hq, S, M, F, D = 4, 2048, 32, 256, 32, 128, 128
    rows = B * chunk
    print(f"rectify determinism: G={hq // hkv}", flush=True)
    g = torch.Generator(device="cuda")
    g.manual_seed(9)
    bf = torch.bfloat16
    k = torch.randn(rows, hkv, D, device="cuda", dtype=bf, generator=g)
    v = torch.randn_like(k)
    q = torch.randn(rows, hq, D, device="cuda", dtype=bf, generator=g)
    src_q = torch.randn(rows, hq, D, device="cuda", dtype=bf, generator=g)
    o_full = torch.randn(rows, hq, D, device="cuda", dtype=bf, generator=g)
    lse_full = torch.randn(rows, hq, device="cuda", generator=g) + 8.0
    qo = torch.arange(0, rows + 1, chunk, device="cuda", dtype=torch.int32)
    idx = torch.randperm(rows, device="cuda", generator=g).to(torch.int32)
    req = torch.tensor([2, 0, 3, 1], device="cuda", dtype=torch.int32)
    runs = []
    for _ in range(3):
        qc = torch.zeros(B, M, hq, D, device="cuda", dtype=bf)
        ac = torch.zeros_like(qc)
        lc = torch.zeros(B, M, hq, device="cuda")
        rl = torch.tensor([0, 5, 31, 100], device="cuda", dtype=torch.int32)
        rect_ext.mac_prefill_rectify_update_cache(q, src_q, o_full, lse_full, k, v, qo, qo, idx, qc, ac, lc, rl,
                                                  req, S, F, 1.0 / math.sqrt(D), sink_mode=1)
        torch.cuda.synchronize()
        runs.append([qc.view(torch.int16), ac.view(torch.int16), lc.view(torch.int32), rl])
    for r in runs[1:]:
        for a, b in zip(r, runs[0]):
            assert torch.equal(a, b)


def test_window_attention_skips_requests_outside_the_buffers(rect_ext):
    """A request whose query range runs past total_q (or key range past
    kv_indices) is skipped: its rows stay untouched, the others are exact."""
    case = syn.prefill_case(qo_lens=[5, 5], kv_lens=[9, 7], hq=4, hkv=2, seed=51)
    d = _dev_case(case)
    qo_bad = case.qo_indptr.copy()
    qo_bad[2] = 5000  # request 1 claims rows far beyond the 10 query rows
    out = torch.zeros_like(d["q"])
    lse = torch.full((10, 4), 7.0, device="cuda")
    rect_ext.window_attention_return_lse(d["q"], d["k"], d["v"], _i32(qo_bad), d["kv"], d["idx"], -1,
                                         case.sm_scale, out=out, out_lse=lse)
    torch.cuda.synchronize()
    eo, el = orc.window_attention(_bf(case.q), _bf(case.k), _bf(case.v), case.qo_indptr, case.kv_indptr,
                                  case.kv_indices, window_left=-1, sm_scale=case.sm_scale)
    got = bits(_host_bits(out))
    assert rel_l2(got[:5], bits(eo[:5])) < 1e-2
    assert not got[5:].any() and (lse[5:] == 7.0).all()
    np.testing.assert_allclose(lse[:5].cpu().numpy(), el[:5], atol=2e-4)
