"""GPU parity of the ring-cache maintenance ops (mac_prefill_update_cache and
the ready / invalidate / request-state ops) with the CPU oracle, bit for bit."""

import numpy as np
import pytest

from helpers import orc, syn

torch = pytest.importorskip("torch")

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ext():
    from mac_attention.integrations.sglang.bridge import load_mac_prefill_update_cache_extension

    return load_mac_prefill_update_cache_extension(False)


def _bits(t):
    return t.view(torch.int16).cpu().numpy().view(np.uint16)


@pytest.mark.parametrize("by_batch", [False, True])
@pytest.mark.parametrize("with_qpost", [False, True])
def test_prefill_update_cache(ext, by_batch, with_qpost):
    rng = np.random.default_rng(5 + by_batch + 2 * with_qpost)
    R, M, H, D = 6, 16, 8, 128
    B = 4 if not by_batch else 4
    req_ids = np.array([3, 0, 5, 1], np.int32)
    lens = np.array([5, 40, 0, 16], np.int32)
    offsets = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    rows = int(offsets[-1])
    src_q = syn.to_bits(rng.standard_normal((rows, H, D)))
    src_a = syn.to_bits(rng.standard_normal((rows, H, D)))
    src_l = rng.standard_normal((rows, H)).astype(np.float32)
    qc = syn.to_bits(rng.standard_normal((R, M, H, D)))
    ac = syn.to_bits(rng.standard_normal((R, M, H, D)))
    lc = rng.standard_normal((R, M, H)).astype(np.float32)
    rl = (np.array([7, 9, 2, 30], np.int32) if by_batch
          else rng.integers(0, 50, R).astype(np.int32))
    qp = syn.to_bits(rng.standard_normal((R, M, H, D))) if with_qpost else None
    # oracle
    e_qc, e_ac, e_lc, e_rl = qc.copy(), ac.copy(), lc.copy(), rl.copy()
    e_qp = qp.copy() if qp is not None else None
    orc.prefill_update_cache(e_qc, e_ac, e_lc, e_rl, req_ids, src_q, src_a, src_l, offsets, lens,
                             M, H, D, e_qp)
    dev = "cuda"
    tb = lambda a: torch.from_numpy(a.view(np.int16)).to(dev).view(torch.bfloat16)  # noqa: E731
    t = lambda a: torch.from_numpy(a).to(dev)  # noqa: E731
    g_qc, g_ac, g_lc, g_rl = tb(qc.copy()), tb(ac.copy()), t(lc.copy()), t(rl.copy())
    g_qp = tb(qp.copy()) if qp is not None else torch.empty(0, device=dev, dtype=torch.bfloat16)
    ext.mac_prefill_update_cache(g_qc, g_ac, g_lc, g_rl, t(req_ids), tb(src_q), tb(src_a), t(src_l),
                                 t(offsets), t(lens), M, H, D, g_qp)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(_bits(g_qc), e_qc)
    np.testing.assert_array_equal(_bits(g_ac), e_ac)
    np.testing.assert_array_equal(g_lc.cpu().numpy(), e_lc)
    np.testing.assert_array_equal(g_rl.cpu().numpy(), e_rl)
    if qp is not None:
        np.testing.assert_array_equal(_bits(g_qp), e_qp)


def test_ready_ops(ext):
    R = 10
    ready = torch.zeros(R, dtype=torch.bool, device="cuda")
    ce = torch.full((R,), -1, dtype=torch.int64, device="cuda")
    re = torch.arange(R, dtype=torch.int64, device="cuda") * 3
    ids = torch.tensor([1, 4, 9, -1, 12], dtype=torch.int32, device="cuda")
    e_ready, e_ce, e_re = np.zeros(R, np.uint8), np.full(R, -1, np.int64), np.arange(R, dtype=np.int64) * 3
    ext.mac_mark_persistent_ready(ready, ce, re, ids)
    orc.mark_ready(e_ready, e_ce, e_re, ids.cpu().numpy())
    torch.cuda.synchronize()
    np.testing.assert_array_equal(ready.cpu().numpy().astype(np.uint8), e_ready)
    np.testing.assert_array_equal(ce.cpu().numpy(), e_ce)
    ids2 = torch.tensor([4, 7], dtype=torch.int32, device="cuda")
    ext.mac_invalidate_persistent_ready(ready, ce, re, ids2)
    orc.invalidate_ready(e_ready, e_ce, e_re, ids2.cpu().numpy())
    torch.cuda.synchronize()
    np.testing.assert_array_equal(ready.cpu().numpy().astype(np.uint8), e_ready)
    np.testing.assert_array_equal(ce.cpu().numpy(), e_ce)
    np.testing.assert_array_equal(re.cpu().numpy(), e_re)
    req_len = torch.zeros(R, dtype=torch.int32, device="cuda")
    mrl = torch.zeros(R, dtype=torch.int32, device="cuda")
    cl = torch.zeros(3, dtype=torch.int32, device="cuda")
    ids3 = torch.tensor([2, 5, 11], dtype=torch.int32, device="cuda")
    seq = torch.tensor([100, 7, 50], dtype=torch.int32, device="cuda")
    cur = torch.tensor([1, 9, 50], dtype=torch.int32, device="cuda")
    ext.mac_update_request_state(req_len, mrl, cl, ids3, seq, cur)
    e_rl, e_mrl, e_cl = np.zeros(R, np.int32), np.zeros(R, np.int32), np.zeros(3, np.int32)
    orc.update_request_state(e_rl, e_mrl, e_cl, ids3.cpu().numpy(), seq.cpu().numpy(),
                             cur.cpu().numpy())
    torch.cuda.synchronize()
    np.testing.assert_array_equal(req_len.cpu().numpy(), e_rl)
    np.testing.assert_array_equal(mrl.cpu().numpy(), e_mrl)
    np.testing.assert_array_equal(cl.cpu().numpy(), e_cl)


@pytest.mark.parametrize("seed", range(8))
def test_prefill_update_cache_random_shapes(ext, seed):
    """Seeded random batches: head dims whose rows are not a whole number of
    16-byte vectors, rings of 1 to 16 slots, empty chunks, a request id
    outside [0, R), both request_length forms, with and without the q_post
    ring, and (odd seeds) source rows in views one element off 16-byte
    alignment, which take the element-wise path; bit for bit."""
    rng = np.random.default_rng(700 + seed)
    R = int(rng.integers(2, 8))
    B = int(rng.integers(1, R + 1))
    M = int(rng.choice([1, 3, 16]))
    H = int(rng.choice([1, 3, 8]))
    D = int(rng.choice([128, 64, 100, 7]))
    by_batch = bool(rng.integers(0, 2)) and B != R
    with_qpost = bool(seed % 3)
    req_ids = rng.permutation(R)[:B].astype(np.int32)
    if B > 1:
        req_ids[-1] = R + 3  # outside the ring: skipped
    lens = rng.integers(0, 40, B).astype(np.int32)
    offsets = np.concatenate([[0], np.cumsum(lens)[:-1]]).astype(np.int32)
    rows = int(lens.sum())
    src_q = syn.to_bits(rng.standard_normal((rows, H, D)))
    src_a = syn.to_bits(rng.standard_normal((rows, H, D)))
    src_l = rng.standard_normal((rows, H)).astype(np.float32)
    qc = syn.to_bits(rng.standard_normal((R, M, H, D)))
    ac = syn.to_bits(rng.standard_normal((R, M, H, D)))
    lc = rng.standard_normal((R, M, H)).astype(np.float32)
    rl = rng.integers(0, 50, B if by_batch else R).astype(np.int32)
    qp = syn.to_bits(rng.standard_normal((R, M, H, D))) if with_qpost else None
    print(f"prefill update random: seed={seed} R={R} B={B} M={M} H={H} D={D} by_batch={by_batch}", flush=True)
    e_qc, e_ac, e_lc, e_rl = qc.copy(), ac.copy(), lc.copy(), rl.copy()
    e_qp = qp.copy() if qp is not None else None
    orc.prefill_update_cache(e_qc, e_ac, e_lc, e_rl, req_ids, src_q, src_a, src_l,
                             np.concatenate([offsets, [rows]]).astype(np.int32), lens, M, H, D, e_qp)
    dev = "cuda"
    tb = lambda a: torch.from_numpy(a.view(np.int16)).to(dev).view(torch.bfloat16)  # noqa: E731
    t = lambda a: torch.from_numpy(a).to(dev)  # noqa: E731

    def src(a):
        if seed % 2 == 0:
            return tb(a)
        flat = torch.empty(a.size + 1, device=dev, dtype=torch.bfloat16)  # one element off alignment
        flat[1:] = tb(a).reshape(-1)
        return flat[1:].view(a.shape)

    g_qc, g_ac, g_lc, g_rl = tb(qc.copy()), tb(ac.copy()), t(lc.copy()), t(rl.copy())
    g_qp = tb(qp.copy()) if qp is not None else torch.empty(0, device=dev, dtype=torch.bfloat16)
    ext.mac_prefill_update_cache(g_qc, g_ac, g_lc, g_rl, t(req_ids), src(src_q), src(src_a), t(src_l),
                                 t(np.concatenate([offsets, [rows]]).astype(np.int32)), t(lens), M, H, D, g_qp)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(_bits(g_qc), e_qc)
    np.testing.assert_array_equal(_bits(g_ac), e_ac)
    np.testing.assert_array_equal(g_lc.cpu().numpy(), e_lc)
    np.testing.assert_array_equal(g_rl.cpu().numpy(), e_rl)
    if qp is not None:
        np.testing.assert_array_equal(_bits(g_qp), e_qp)
