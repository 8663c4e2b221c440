"""Pins the CPU oracle of the fused decode RoPE + q-preserve + KV scatter
(mac_decode_rope_preserve.cu:36-156, ROPE) with an independent numpy
restatement: RoPE as a complex rotation (x0 + i x1) * (cos + i sin)."""

import numpy as np
import pytest

from helpers import orc, syn


def _bf(x):
    return syn.to_bits(syn.bf16_round(np.asarray(x, np.float32)))


def make_rope_case(*, n, hq, hkv, d, rot, pool, seed, max_pos=4096, qkv_fused=True):
    """Decode inputs as SGLang hands them over: q/k/v as column slices of one
    fused qkv row buffer (so q/k/v rows have a stride larger than the row)."""
    rng = np.random.default_rng(seed)
    qkv = _bf(rng.standard_normal((n, (hq + 2 * hkv) * d)))
    if qkv_fused:
        q, k, v = qkv[:, :hq * d], qkv[:, hq * d:(hq + hkv) * d], qkv[:, (hq + hkv) * d:]
    else:
        q, k, v = (np.ascontiguousarray(x) for x in (qkv[:, :hq * d], qkv[:, hq * d:(hq + hkv) * d],
                                                    qkv[:, (hq + hkv) * d:]))
    inv = 1.0 / (10000.0 ** (np.arange(0, rot, 2) / rot))
    ang = np.arange(max_pos)[:, None] * inv[None, :]
    cs = np.concatenate([np.cos(ang), np.sin(ang)], axis=1).astype(np.float32)
    positions = rng.integers(0, max_pos, n)
    cache_locs = rng.permutation(pool)[:n]
    return qkv, q, k, v, cs, positions, cache_locs


def numpy_rope(x_bits, cs_row, rot, neox):
    x = syn.from_bits(x_bits).astype(np.float64)
    half = rot // 2
    c, s = cs_row[..., :half].astype(np.float64), cs_row[..., half:rot].astype(np.float64)
    if neox:
        z = (x[..., :half] + 1j * x[..., half:rot]) * (c + 1j * s)
        y = x.copy()
        y[..., :half], y[..., half:rot] = z.real, z.imag
    else:
        z = (x[..., 0:rot:2] + 1j * x[..., 1:rot:2]) * (c + 1j * s)
        y = x.copy()
        y[..., 0:rot:2], y[..., 1:rot:2] = z.real, z.imag
    return y


def ulp_diff(a_bits, b_bits):
    a = a_bits.astype(np.int32)
    b = b_bits.astype(np.int32)
    # bf16 bit patterns are monotone within a sign; compare as signed magnitudes
    a = np.where(a & 0x8000, -(a & 0x7FFF), a)
    b = np.where(b & 0x8000, -(b & 0x7FFF), b)
    return np.abs(a - b)


@pytest.mark.parametrize("neox", [True, False])
@pytest.mark.parametrize("rot", [128, 64, 6])
def test_rope_oracle_matches_complex_rotation(neox, rot):
    n, hq, hkv, d, pool = 5, 4, 2, 128, 50
    qkv, q, k, v, cs, pos, locs = make_rope_case(n=n, hq=hq, hkv=hkv, d=d, rot=rot, pool=pool, seed=rot)
    q0, k0, v0 = q.copy(), k.copy(), v.copy()
    q_pre = np.zeros((n, hq, d), np.uint16)
    kb = np.zeros((pool, hkv, d), np.uint16)
    vb = np.zeros((pool, hkv, d), np.uint16)
    orc.rope_preserve(q, k, v, q_pre, kb, vb, cs, pos, locs, head_dim=d, is_neox=neox)
    np.testing.assert_array_equal(q_pre, q0.reshape(n, hq, d))
    np.testing.assert_array_equal(vb[locs], v0.reshape(n, hkv, d))
    untouched = np.setdiff1d(np.arange(pool), locs)
    assert not kb[untouched].any() and not vb[untouched].any()
    for x_new, x_old, h in ((q, q0, hq), (k, k0, hkv)):
        exp = numpy_rope(x_old.reshape(n, h, d), cs[pos][:, None, :], rot, neox)
        assert ulp_diff(x_new.reshape(n, h, d), _bf(exp)).max() <= 1
        np.testing.assert_array_equal(x_new.reshape(n, h, d)[..., rot:], x_old.reshape(n, h, d)[..., rot:])
    np.testing.assert_array_equal(kb[locs], k.reshape(n, hkv, d))
