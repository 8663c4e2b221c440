"""The no-allocation decode entry point (mac_persistent_decode_bf16_noalloc in
libmac_noalloc.so, workspaces in that library's static device array) against
the ordinary entry point on the same inputs, through the C ABI: two calls in
a row, the second with a smaller step, each compared output for output (and
with the oracle); the workspace arguments may be None; a ring of 2048 slots
(the range-split scan) at a context near 128K (chunks enlarged to fit the
array's 32 partial slots per group); replays of a captured graph; and the
size limits are refused with a clear error."""

import numpy as np
import pytest

from helpers import bits, oracle_run, rel_l2, syn

torch = pytest.importorskip("torch")

pytestmark = pytest.mark.gpu


def _args(dev, case, ws, out, out_lse, max_context, S=None, F=None):
    S = case.semantic_pos_ahead if case is not None else S
    F = case.front_sink_tokens if case is not None else F
    gml, lb, cm = (case.gen_min_limit, case.lookback_right, case.candidate_mode) if case is not None else (0, 0, 0)
    thr = case.threshold if case is not None else 0.45
    scale = case.sm_scale if case is not None else 128 ** -0.5
    return (dev["q_post"], dev["q_pre"], dev["k"], dev["v"], dev["req_to_token"], dev["req_ids"],
            dev["past_lens"], dev["out_cache_loc"], dev["query_cache"], dev["attn_cache"], dev["lse_cache"],
            out, out_lse, *ws, max_context, 32, 32, S, F, gml, lb, cm, thr, scale, 0, 0,
            1.0, 0.0, -1.0, 0.0, 64.0, 0.0, 1, -1, 0, dev["query_cache"], dev["cache_ready"], dev["cache_epoch"],
            dev["request_epoch"])


def _np(t):
    return t.float().cpu().numpy() if t.dtype == torch.bfloat16 else t.cpu().numpy()


def _state(dev, out, out_lse):
    return dict(out=_np(out), lse=_np(out_lse), q=syn.to_bits(_np(dev["query_cache"])), a=_np(dev["attn_cache"]),
                l=_np(dev["lse_cache"]))


def _assert_same(n, w, tol):
    """tol None: bit for bit; else relative L2 / absolute tolerances."""
    np.testing.assert_array_equal(n["q"], w["q"])
    fin = np.isfinite(w["l"])
    np.testing.assert_array_equal(np.isfinite(n["l"]), fin)
    if tol is None:
        np.testing.assert_array_equal(n["out"], w["out"])
        np.testing.assert_array_equal(n["lse"], w["lse"])
        np.testing.assert_array_equal(n["a"], w["a"])
        np.testing.assert_array_equal(n["l"][fin], w["l"][fin])
        return
    assert rel_l2(n["out"], w["out"]) < tol
    np.testing.assert_allclose(n["lse"], w["lse"], atol=tol, rtol=tol)
    assert rel_l2(n["a"], w["a"]) < tol
    np.testing.assert_allclose(n["l"][fin], w["l"][fin], atol=tol, rtol=tol)


CASES = [
    # (batch, hq, hkv, kv_lens, M, S, F, hit_rate, seed): the second is smaller
    (6, 32, 8, [3000, 5000, 777, 4096, 2000, 10000], 32, 64, 16, 0.6, 71),
    (3, 32, 4, [700, 1500, 300], 16, 128, 0, 0.7, 72),
]


@pytest.fixture(scope="module")
def ext():
    from mac_attention.integrations.sglang.bridge import load_mac_persistent_decode_extension

    return load_mac_persistent_decode_extension(False)


def test_noalloc_entry_matches_the_workspace_entry(ext):
    """Two calls in a row, the second smaller: the same bits as the
    workspace entry point (the same chunks, partial dtype and kernels), and
    the parity bar against the oracle.  The no-allocation calls pass None for
    every workspace."""
    for cfg in CASES:
        b, hq, hkv, kv_lens, m, s, f, hit_rate, seed = cfg
        print(f"no-alloc case {cfg}", flush=True)
        c = syn.random_case(batch=b, hq=hq, hkv=hkv, kv_lens=kv_lens, capacity=m, semantic_pos_ahead=s,
                            front_sink_tokens=f, hit_rate=hit_rate, match_lag=m // 2, seed=seed)
        c.cache_ready = np.array([1] * (b - 1) + [0], np.uint8)  # the last request fails the gate
        res = oracle_run(c)
        max_context = max(kv_lens) + 8
        runs = {}
        for mode in ("workspace", "noalloc"):
            dev = syn.to_device(torch, c)
            out = torch.empty_like(dev["q_post"])
            out_lse = torch.empty(b, hq, device="cuda")
            if mode == "workspace":
                ws = syn.workspace(torch, batch=b, hq=hq, hkv=hkv, capacity=m, max_context=max_context,
                                   tile_tokens=32, match_tile_slots=32, semantic_pos_ahead=s, front_sink_tokens=f,
                                   device="cuda")
                ext.mac_persistent_decode_bf16(*_args(dev, c, ws, out, out_lse, max_context))
            else:
                ext.mac_persistent_decode_bf16_noalloc(*_args(dev, c, [None] * 30, out, out_lse, max_context))
            torch.cuda.synchronize()
            runs[mode] = _state(dev, out, out_lse)
        n = runs["noalloc"]
        _assert_same(n, runs["workspace"], None)
        assert rel_l2(n["out"], bits(res.out)) < 1e-2
        np.testing.assert_array_equal(n["q"], res.query_cache)
        assert rel_l2(n["a"], bits(res.attn_cache)) < 1e-2


def _big_case():
    """Two requests at past_len 126976 with a 2048-slot ring (the reference
    benchmark's ring): 80% of the heads hit a planted ring copy, so groups of
    both kinds run."""
    b, hq, hkv, ctx, m, S = 2, 32, 8, 126976, 2048, 256
    dev = syn.device_case(torch, batch=b, hq=hq, hkv=hkv, ctx=ctx, capacity=m, seed=74)
    syn.plant_synthetic_hits(torch, dev, hit_rate=0.8, bench_mode=1, semantic_pos_ahead=S)
    return dev, b, hq, hkv, m, S


def test_noalloc_entry_at_a_2048_slot_ring_and_128k_context(ext):
    """The range-split ring scan and a 127K-token context, where the array's
    32 partial slots per group make the plan enlarge the long groups' chunks
    (so the sums differ from the workspace entry's only by rounding)."""
    dev, b, hq, hkv, m, S = _big_case()
    pristine = {k: dev[k].clone() for k in ("query_cache", "attn_cache", "lse_cache")}
    max_context = 131072
    runs = {}
    for mode in ("workspace", "noalloc"):
        for k, v in pristine.items():
            dev[k].copy_(v)
        out = torch.empty_like(dev["q_post"])
        out_lse = torch.empty(b, hq, device="cuda")
        print(f"no-alloc ring 2048 ctx 126976: {mode}", flush=True)
        if mode == "workspace":
            ws = syn.workspace(torch, batch=b, hq=hq, hkv=hkv, capacity=m, max_context=max_context, tile_tokens=32,
                               match_tile_slots=32, semantic_pos_ahead=S, device="cuda")
            ext.mac_persistent_decode_bf16(*_args(dev, None, ws, out, out_lse, max_context, S=S, F=0))
            hits = int(ws[3].sum())
        else:
            ext.mac_persistent_decode_bf16_noalloc(*_args(dev, None, [None] * 30, out, out_lse, max_context, S=S, F=0))
        torch.cuda.synchronize()
        runs[mode] = _state(dev, out, out_lse)
    assert hits == round(0.8 * b * hq)
    _assert_same(runs["noalloc"], runs["workspace"], 1e-3)


def test_noalloc_entry_replays_from_a_graph(ext):
    """The no-allocation step captured in a hipGraph (the callers it is for):
    three replays, with the ring restored and eager work between them, each
    equal bit for bit to an eager call of the workspace entry point."""
    b, hq, hkv, kv_lens, m, s, f, hit_rate, seed = CASES[0]
    c = syn.random_case(batch=b, hq=hq, hkv=hkv, kv_lens=kv_lens, capacity=m, semantic_pos_ahead=s,
                        front_sink_tokens=f, hit_rate=hit_rate, match_lag=m // 2, seed=seed)
    max_context = max(kv_lens) + 8
    dev = syn.to_device(torch, c)
    pristine = {k: dev[k].clone() for k in ("query_cache", "attn_cache", "lse_cache")}
    out = torch.empty_like(dev["q_post"])
    out_lse = torch.empty(b, hq, device="cuda")
    ws = syn.workspace(torch, batch=b, hq=hq, hkv=hkv, capacity=m, max_context=max_context, tile_tokens=32,
                       match_tile_slots=32, semantic_pos_ahead=s, front_sink_tokens=f, device="cuda")
    ext.mac_persistent_decode_bf16(*_args(dev, c, ws, out, out_lse, max_context))
    torch.cuda.synchronize()
    eager = _state(dev, out, out_lse)

    def restore():
        for k, v in pristine.items():
            dev[k].copy_(v)

    restore()
    stream = torch.cuda.Stream()
    with torch.cuda.stream(stream):  # warm-up outside the capture (device look-up, module load)
        ext.mac_persistent_decode_bf16_noalloc(*_args(dev, c, [None] * 30, out, out_lse, max_context))
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=stream):
        ext.mac_persistent_decode_bf16_noalloc(*_args(dev, c, [None] * 30, out, out_lse, max_context))
    torch.cuda.synchronize()
    for i in range(3):
        restore()
        out.zero_()
        out_lse.zero_()
        torch.cuda.synchronize()
        print(f"no-alloc graph replay {i}", flush=True)
        g.replay()
        torch.cuda.synchronize()
        _assert_same(_state(dev, out, out_lse), eager, None)
        # eager work between replays
        ext.mac_persistent_decode_bf16(*_args(dev, c, ws, out, out_lse, max_context))
        torch.cuda.synchronize()


def test_noalloc_entry_refuses_steps_beyond_its_array(ext):
    b, hq, hkv = 129, 32, 8  # 4128 query heads > 4096
    c = syn.random_case(batch=b, hq=hq, hkv=hkv, kv_lens=[40] * b, capacity=8, semantic_pos_ahead=8,
                        hit_rate=0.0, seed=73)
    dev = syn.to_device(torch, c)
    out = torch.empty_like(dev["q_post"])
    with pytest.raises(RuntimeError, match="at most 4096 query heads"):
        ext.mac_persistent_decode_bf16_noalloc(*_args(dev, c, [None] * 30, out, torch.empty(b, hq, device="cuda"), 64))
