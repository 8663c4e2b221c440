"""Fused decode RoPE + pre-RoPE q preserve + KV scatter on the GPU against
the CPU oracle (mac_decode_rope_preserve.cu:36-269).  Copies (q_pre, V rows,
pass-through dims) are bit-exact; rotated values are bit-exact except at most
one bf16 ulp where fp32 (GPU) and double (oracle) land on different sides of
a rounding boundary."""

import numpy as np
import pytest

from helpers import orc
from test_oracle_rope import make_rope_case, ulp_diff

torch = pytest.importorskip("torch")

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ext():
    from mac_attention.integrations.sglang.bridge import load_mac_decode_rope_preserve_extension

    return load_mac_decode_rope_preserve_extension(False)


def _dev(b):
    return torch.from_numpy(np.ascontiguousarray(b).view(np.int16)).cuda().view(torch.bfloat16)


def _host(t):
    return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


@pytest.mark.parametrize("neox", [True, False])
@pytest.mark.parametrize("rot,fused,pad", [(128, True, 0), (64, False, 0), (6, True, 0), (128, True, 1)])
@pytest.mark.parametrize("idx_dtype", [torch.int32, torch.int64])
def test_rope_preserve_matches_oracle(ext, neox, rot, fused, pad, idx_dtype):
    n, hq, hkv, d, pool = 64, 32, 8, 128, 300
    qkv, q, k, v, cs, pos, locs = make_rope_case(n=n, hq=hq, hkv=hkv, d=d, rot=rot, pool=pool,
                                                 seed=rot + pad, qkv_fused=fused)
    locs = locs.copy()
    locs[3] = pool + 5  # outside the pool: not written
    # device tensors; pad > 0 shifts the views off 16-byte alignment (element-wise kernel)
    if fused:
        width = qkv.shape[1]
        buf = np.zeros((n, width + pad), np.uint16)
        buf[:, pad:] = qkv
        g = _dev(buf)
        gq, gk, gv = g[:, pad:pad + hq * d], g[:, pad + hq * d:pad + (hq + hkv) * d], g[:, pad + (hq + hkv) * d:]
    else:
        gq, gk, gv = _dev(q), _dev(k), _dev(v)
    q_pre = torch.zeros(n, hq, d, dtype=torch.bfloat16, device="cuda")
    kb = torch.zeros(pool, hkv, d, dtype=torch.bfloat16, device="cuda")
    vb = torch.zeros_like(kb)
    ext.mac_decode_rope_preserve_q_bf16(gq, gk, gv, q_pre, kb, vb, torch.from_numpy(cs).cuda(),
                                        torch.from_numpy(pos).cuda().to(idx_dtype),
                                        torch.from_numpy(locs).cuda().to(idx_dtype), d, neox)
    torch.cuda.synchronize()
    # oracle
    eq, ek, ev = q.copy(), k.copy(), v.copy()
    e_pre = np.zeros((n, hq, d), np.uint16)
    ekb = np.zeros((pool, hkv, d), np.uint16)
    evb = np.zeros((pool, hkv, d), np.uint16)
    orc.rope_preserve(eq, ek, ev, e_pre, ekb, evb, cs, pos, locs, head_dim=d, is_neox=neox)
    np.testing.assert_array_equal(_host(q_pre), e_pre)
    np.testing.assert_array_equal(_host(vb), evb)
    np.testing.assert_array_equal(_host(gv), v)  # v is read only
    for got, exp in ((_host(gq), eq), (_host(gk), ek), (_host(kb), ekb)):
        u = ulp_diff(got, exp)
        assert u.max() <= 1 and (u == 0).mean() > 0.99
    if fused:
        np.testing.assert_array_equal(_host(g)[:, :pad], np.zeros((n, pad), np.uint16))


@pytest.mark.parametrize("seed", range(6))
def test_rope_preserve_random_shapes(ext, seed):
    """Seeded random decode batches: token count, GQA shape, rotary dims
    (whole 16-element units and not), pair layout, fused or separate q/k/v
    and views one element off alignment."""
    rng = np.random.default_rng(800 + seed)
    n = int(rng.integers(1, 80))
    hkv = int(rng.choice([1, 2, 8]))
    hq = hkv * int(rng.choice([1, 4, 8]))
    d = 128
    rot = int(rng.choice([128, 64, 32, 16, 6]))
    neox = bool(rng.integers(0, 2))
    fused = bool(rng.integers(0, 2))
    pad = int(rng.integers(0, 2)) if fused else 0
    pool = n + int(rng.integers(0, 50))
    print(f"rope random: seed={seed} n={n} hq={hq} hkv={hkv} rot={rot} neox={neox} fused={fused} pad={pad}",
          flush=True)
    qkv, q, k, v, cs, pos, locs = make_rope_case(n=n, hq=hq, hkv=hkv, d=d, rot=rot, pool=pool,
                                                 seed=900 + seed, qkv_fused=fused)
    if fused:
        width = qkv.shape[1]
        buf = np.zeros((n, width + pad), np.uint16)
        buf[:, pad:] = qkv
        g = _dev(buf)
        gq, gk, gv = g[:, pad:pad + hq * d], g[:, pad + hq * d:pad + (hq + hkv) * d], g[:, pad + (hq + hkv) * d:]
    else:
        gq, gk, gv = _dev(q), _dev(k), _dev(v)
    q_pre = torch.zeros(n, hq, d, dtype=torch.bfloat16, device="cuda")
    kb = torch.zeros(pool, hkv, d, dtype=torch.bfloat16, device="cuda")
    vb = torch.zeros_like(kb)
    ext.mac_decode_rope_preserve_q_bf16(gq, gk, gv, q_pre, kb, vb, torch.from_numpy(cs).cuda(),
                                        torch.from_numpy(pos).cuda(), torch.from_numpy(locs).cuda(), d, neox)
    torch.cuda.synchronize()
    eq, ek, ev = q.copy(), k.copy(), v.copy()
    e_pre = np.zeros((n, hq, d), np.uint16)
    ekb = np.zeros((pool, hkv, d), np.uint16)
    evb = np.zeros((pool, hkv, d), np.uint16)
    orc.rope_preserve(eq, ek, ev, e_pre, ekb, evb, cs, pos, locs, head_dim=d, is_neox=neox)
    np.testing.assert_array_equal(_host(q_pre), e_pre)
    np.testing.assert_array_equal(_host(vb), evb)
    for got, exp in ((_host(gq), eq), (_host(gk), ek), (_host(kb), ekb)):
        u = ulp_diff(got, exp)
        assert u.max() <= 1 and (u == 0).mean() > 0.98


def test_rope_rejects_bad_rotary_dim(ext):
    x = torch.zeros(2, 256, dtype=torch.bfloat16, device="cuda")
    buf = torch.zeros(4, 2, 128, dtype=torch.bfloat16, device="cuda")
    with pytest.raises(RuntimeError, match="invalid rotary_dim"):
        ext.mac_decode_rope_preserve_q_bf16(x, x.clone(), x.clone(), buf, buf.clone(), buf.clone(),
                                            torch.zeros(8, 130, device="cuda"),
                                            torch.zeros(2, dtype=torch.int64, device="cuda"),
                                            torch.zeros(2, dtype=torch.int64, device="cuda"), 128, True)
