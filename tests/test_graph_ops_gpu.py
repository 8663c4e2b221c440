"""Every entry point besides the decode step (covered in test_configs_gpu.py)
captured in a hipGraph: each replay -- with the op's in-place state restored
and unrelated eager work and synchronisation between replays -- must give
the eager result bit for bit.  The library allocates nothing, synchronises
nothing and records no memsets, so capture is the caller's choice, as with
the reference's ops under SGLang's CUDA-graph runner."""

import math

import numpy as np
import pytest

from helpers import syn

torch = pytest.importorskip("torch")

pytestmark = pytest.mark.gpu


def _graph_matches_eager(run, state, replays=4):
    """run() launches the op(s) on the current stream and mutates the tensors
    of `state` (name -> tensor) in place."""
    pristine = {k: v.clone() for k, v in state.items()}
    run()
    torch.cuda.synchronize()
    eager = {k: v.clone() for k, v in state.items()}
    for k, v in state.items():
        v.copy_(pristine[k])
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        run()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        run()
    for it in range(replays):
        for k, v in state.items():
            v.copy_(pristine[k])
        _ = torch.randn(1000, device="cuda").sum()  # unrelated eager work between replays
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for k, v in state.items():
            assert torch.equal(_bits(v), _bits(eager[k])), f"replay {it}: {k} differs from eager"
    del graph


def _bits(t):
    """Bit patterns (NaN markers in the ring compare equal to themselves)."""
    view = {torch.bfloat16: torch.int16, torch.float16: torch.int16, torch.float32: torch.int32}
    return t.view(view[t.dtype]) if t.dtype in view else t


def _bf(rng, *shape):
    return torch.from_numpy(rng.standard_normal(shape).astype(np.float32)).cuda().to(torch.bfloat16)


def test_decode_rope_preserve_in_a_graph():
    from mac_attention.integrations.sglang.bridge import load_mac_decode_rope_preserve_extension

    rope = load_mac_decode_rope_preserve_extension(False)
    rng = np.random.default_rng(3)
    n, hq, hkv, d, pool = 48, 32, 8, 128, 512
    qkv = _bf(rng, n, (hq + 2 * hkv) * d)
    q, k, v = qkv[:, :hq * d], qkv[:, hq * d:(hq + hkv) * d], qkv[:, (hq + hkv) * d:]
    q_pre = torch.zeros(n, hq, d, dtype=torch.bfloat16, device="cuda")
    kb = torch.zeros(pool, hkv, d, dtype=torch.bfloat16, device="cuda")
    vb = torch.zeros_like(kb)
    inv = 1.0 / (10000.0 ** (torch.arange(0, d, 2, device="cuda", dtype=torch.float32) / d))
    ang = torch.arange(4096, device="cuda", dtype=torch.float32)[:, None] * inv[None, :]
    cs = torch.cat([ang.cos(), ang.sin()], dim=1).contiguous()
    pos = torch.from_numpy(rng.integers(0, 4096, n)).cuda()
    locs = torch.from_numpy(rng.permutation(pool)[:n].astype(np.int64)).cuda()
    _graph_matches_eager(lambda: rope.mac_decode_rope_preserve_q_bf16(q, k, v, q_pre, kb, vb, cs, pos, locs,
                                                                      d, True),
                         dict(qkv=qkv, q_pre=q_pre, kb=kb, vb=vb))


def test_prefill_ring_ops_in_a_graph():
    """mac_prefill_update_cache, then mark-ready, invalidate and
    update-request-state, captured together."""
    from mac_attention.integrations.sglang.bridge import load_mac_prefill_update_cache_extension

    cache = load_mac_prefill_update_cache_extension(False)
    rng = np.random.default_rng(4)
    R, M, H, D = 6, 16, 8, 128
    req_ids = torch.tensor([3, 0, 5, 1], dtype=torch.int32, device="cuda")
    lens = torch.tensor([5, 40, 0, 16], dtype=torch.int32, device="cuda")
    offsets = torch.tensor([0, 5, 45, 45, 61], dtype=torch.int32, device="cuda")
    src_q, src_a = _bf(rng, 61, H, D), _bf(rng, 61, H, D)
    src_l = torch.randn(61, H, device="cuda")
    qc, ac = _bf(rng, R, M, H, D), _bf(rng, R, M, H, D)
    lc = torch.randn(R, M, H, device="cuda")
    qp = _bf(rng, R, M, H, D)
    rl = torch.from_numpy(rng.integers(0, 50, R).astype(np.int32)).cuda()
    ready = torch.zeros(R, dtype=torch.bool, device="cuda")
    cache_epoch = torch.full((R,), -1, dtype=torch.int64, device="cuda")
    request_epoch = torch.arange(R, dtype=torch.int64, device="cuda")
    req_len = torch.zeros(R, dtype=torch.int32, device="cuda")
    match_len = torch.zeros(R, dtype=torch.int32, device="cuda")
    cache_lens = torch.zeros(4, dtype=torch.int32, device="cuda")
    seq = torch.tensor([9, 70, 4, 33], dtype=torch.int32, device="cuda")
    cur = torch.tensor([5, 10, 4, 40], dtype=torch.int32, device="cuda")

    def run():
        cache.mac_prefill_update_cache(qc, ac, lc, rl, req_ids, src_q, src_a, src_l, offsets, lens, M, H, D, qp)
        cache.mac_mark_persistent_ready(ready, cache_epoch, request_epoch, req_ids)
        cache.mac_invalidate_persistent_ready(ready, cache_epoch, request_epoch, req_ids[2:3])
        cache.mac_update_request_state(req_len, match_len, cache_lens, req_ids, seq, cur)

    _graph_matches_eager(run, dict(qc=qc, ac=ac, lc=lc, qp=qp, rl=rl, ready=ready, cache_epoch=cache_epoch,
                                   request_epoch=request_epoch, req_len=req_len, match_len=match_len,
                                   cache_lens=cache_lens))


def test_prefill_rectification_in_a_graph():
    """The fused rectification (window state, downdate, ring write, request
    length bump) and the reference's three calls, each captured."""
    from mac_attention.integrations.sglang import bridge

    rect = bridge.load_mac_prefill_rectify_extension()
    merge = bridge.load_mac_merge_downdate_cache_extension(False)
    cache = bridge.load_mac_prefill_update_cache_extension(False)
    rng = np.random.default_rng(5)
    case = syn.prefill_case(qo_lens=[200, 50, 90], kv_lens=[300, 50, 400], hq=8, hkv=2, seed=6)
    tb = lambda a: torch.from_numpy(np.asarray(a, np.float32)).cuda().to(torch.bfloat16)  # noqa: E731
    i32 = lambda a: torch.from_numpy(np.ascontiguousarray(a, np.int32)).cuda()  # noqa: E731
    q, k, v = tb(case.q), tb(case.k), tb(case.v)
    qo, kv, idx = i32(case.qo_indptr), i32(case.kv_indptr), i32(case.kv_indices)
    rows, hq = case.q.shape[0], case.q.shape[1]
    src_q, o_full = _bf(rng, rows, hq, 128), _bf(rng, rows, hq, 128)
    lse_full = torch.randn(rows, hq, device="cuda") + 6.0
    S, M, R = 32, 24, 4
    req = i32([2, 0, 3])
    qc, ac = _bf(rng, R, M, hq, 128), _bf(rng, R, M, hq, 128)
    lc = torch.randn(R, M, hq, device="cuda")
    rl = i32([4, 0, 9, 1])
    sm = 1.0 / math.sqrt(128)
    _graph_matches_eager(
        lambda: rect.mac_prefill_rectify_update_cache(q, src_q, o_full, lse_full, k, v, qo, kv, idx, qc, ac, lc,
                                                      rl, req, S, 8, sm, sink_mode=1),
        dict(qc=qc, ac=ac, lc=lc, rl=rl))

    wo = torch.empty_like(q)
    wl = torch.empty(rows, hq, device="cuda")
    o2, l2 = o_full.clone(), lse_full.clone()
    lens = i32(np.diff(case.qo_indptr))
    empty = torch.empty(0, device="cuda", dtype=torch.bfloat16)

    def three_calls():
        rect.window_attention_return_lse(q, k, v, qo, kv, idx, S - 1, sm, out=wo, out_lse=wl)
        merge.mac_update_then_downdate_bf16_inplace(o2, l2, wo, wl)
        cache.mac_prefill_update_cache(qc, ac, lc, rl[:3], req, src_q, wo, wl, qo, lens, M, hq, 128, empty)

    _graph_matches_eager(three_calls, dict(wo=wo, wl=wl, qc=qc, ac=ac, lc=lc, rl=rl))
