"""Pins the oracle's ring-cache maintenance ops with invariants (CPU only):
the ring after an update holds the last min(len, M) source rows at
(L_before + i) % M, one update equals the same rows appended one at a time,
the by-batch form never bumps lengths, and the ready / invalidate /
request-state ops follow PREFILL:271-320."""

import numpy as np
import pytest

from helpers import orc


def _ring(R, M, H, D, rng):
    return (rng.integers(0, 1 << 16, (R, M, H, D), dtype=np.uint16),
            rng.integers(0, 1 << 16, (R, M, H, D), dtype=np.uint16),
            rng.standard_normal((R, M, H)).astype(np.float32))


@pytest.mark.parametrize("n_rows", [0, 1, 5, 16, 37])
def test_update_keeps_last_rows_at_their_positions(n_rows):
    rng = np.random.default_rng(n_rows)
    R, M, H, D = 3, 16, 2, 8
    qc, ac, lc = _ring(R, M, H, D, rng)
    q0, a0, l0 = qc.copy(), ac.copy(), lc.copy()
    src_q = rng.integers(0, 1 << 16, (n_rows, H, D), dtype=np.uint16)
    src_a = rng.integers(0, 1 << 16, (n_rows, H, D), dtype=np.uint16)
    src_l = rng.standard_normal((n_rows, H)).astype(np.float32)
    req_len = np.array([4, 29, 0], np.int32)
    orc.prefill_update_cache(qc, ac, lc, req_len, [1], src_q, src_a, src_l, [0, n_rows],
                             [n_rows], M, H, D)
    L = 29
    written = set()
    for i in range(max(0, n_rows - M), n_rows):
        slot = (L + i) % M
        written.add(slot)
        np.testing.assert_array_equal(qc[1, slot], src_q[i])
        np.testing.assert_array_equal(ac[1, slot], src_a[i])
        np.testing.assert_array_equal(lc[1, slot], src_l[i])
    for slot in set(range(M)) - written:
        np.testing.assert_array_equal(qc[1, slot], q0[1, slot])
    for r in (0, 2):
        np.testing.assert_array_equal(qc[r], q0[r])
        np.testing.assert_array_equal(ac[r], a0[r])
        np.testing.assert_array_equal(lc[r], l0[r])
    assert req_len.tolist() == [4, 29 + n_rows, 0]


def test_one_update_equals_row_by_row_appends():
    rng = np.random.default_rng(3)
    R, M, H, D = 2, 8, 2, 8
    qc, ac, lc = _ring(R, M, H, D, rng)
    qc2, ac2, lc2 = qc.copy(), ac.copy(), lc.copy()
    n = 13
    src_q = rng.integers(0, 1 << 16, (n, H, D), dtype=np.uint16)
    src_a = rng.integers(0, 1 << 16, (n, H, D), dtype=np.uint16)
    src_l = rng.standard_normal((n, H)).astype(np.float32)
    rl1 = np.array([5, 7], np.int32)
    rl2 = rl1.copy()
    orc.prefill_update_cache(qc, ac, lc, rl1, [0], src_q, src_a, src_l, [0, n], [n], M, H, D)
    for i in range(n):
        orc.prefill_update_cache(qc2, ac2, lc2, rl2, [0], src_q[i:i + 1], src_a[i:i + 1],
                                 src_l[i:i + 1], [0, 1], [1], M, H, D)
    np.testing.assert_array_equal(qc, qc2)
    np.testing.assert_array_equal(ac, ac2)
    np.testing.assert_array_equal(lc, lc2)
    np.testing.assert_array_equal(rl1, rl2)


def test_by_batch_lengths_and_q_post_sentinel():
    rng = np.random.default_rng(4)
    R, M, H, D = 4, 8, 2, 8
    qc, ac, lc = _ring(R, M, H, D, rng)
    qp = rng.integers(0, 1 << 16, (R, M, H, D), dtype=np.uint16)
    qp0 = qp.copy()
    lens = np.array([3, 2], np.int32)
    src = rng.integers(0, 1 << 16, (5, H, D), dtype=np.uint16)
    srcl = rng.standard_normal((5, H)).astype(np.float32)
    rl = np.array([6, 1], np.int32)  # one entry per batch row: indexed by b, never bumped
    orc.prefill_update_cache(qc, ac, lc, rl, [2, 0], src, src, srcl, [0, 3, 5], lens, M, H, D, qp)
    assert rl.tolist() == [6, 1]
    np.testing.assert_array_equal(qc[2, (6 + 1) % M], src[1])
    np.testing.assert_array_equal(qc[0, 2], src[4])
    assert (qp[2, [6, 7, 0]] == 0x7FC0).all() and (qp[0, [1, 2]] == 0x7FC0).all()
    untouched = np.ones((R, M), bool)
    untouched[2, [6, 7, 0]] = False
    untouched[0, [1, 2]] = False
    np.testing.assert_array_equal(qp[untouched], qp0[untouched])


def test_invalid_rows_are_skipped():
    rng = np.random.default_rng(5)
    R, M, H, D = 2, 4, 1, 8
    qc, ac, lc = _ring(R, M, H, D, rng)
    q0 = qc.copy()
    src = rng.integers(0, 1 << 16, (4, H, D), dtype=np.uint16)
    srcl = np.zeros((4, H), np.float32)
    rl = np.zeros(R, np.int32)
    # req out of range, offset beyond the source, zero length
    orc.prefill_update_cache(qc, ac, lc, rl, [5, 0, 1], src, src, srcl, [0, 3, 9, 9],
                             [2, 2, 0], M, H, D)
    np.testing.assert_array_equal(qc, q0)
    assert rl.tolist() == [0, 0]


def test_ready_ops():
    R = 6
    ready = np.zeros(R, np.uint8)
    ce = np.full(R, -1, np.int64)
    re = np.arange(R, dtype=np.int64) + 10
    orc.mark_ready(ready, ce, re, [1, 3, 9, -2])
    assert ready.tolist() == [0, 1, 0, 1, 0, 0]
    assert ce.tolist() == [-1, 11, -1, 13, -1, -1]
    orc.invalidate_ready(ready, ce, re, [3, 4])
    assert ready.tolist() == [0, 1, 0, 0, 0, 0]
    assert ce.tolist() == [-1, 11, -1, -1, -1, -1]
    assert re.tolist() == [10, 11, 12, 14, 15, 15]
    req_len = np.zeros(R, np.int32)
    mrl = np.zeros(R, np.int32)
    cl = np.zeros(3, np.int32)
    orc.update_request_state(req_len, mrl, cl, [0, 5, 8], [10, 4, 9], [3, 7, 1])
    assert cl.tolist() == [7, 0, 8]
    assert req_len.tolist() == [10, 0, 0, 0, 0, 4]
    assert mrl.tolist() == [7, 0, 0, 0, 0, 0]
