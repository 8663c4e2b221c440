"""The FP32 torch restatement of the decode step (oracle/torch_oracle.py,
the CPU baseline bench.py times) against the C oracle on identical inputs:
decisions exact, outputs and ring rows within bf16 rounding.  Cases cover
hits, misses, mixed groups, front sinks, short requests and the readiness
gate (the same generator the GPU parity tests use)."""

import numpy as np
import pytest
import torch

from helpers import bits, oracle_run, rel_l2, syn
from oracle import torch_oracle as tor

CASES = [
    # (batch, hq, hkv, kv_lens, M, S, F, hit_rate, seed)
    (3, 32, 8, [300, 517, 1024], 32, 64, 0, 0.5, 10),
    (2, 32, 4, [777, 2049], 16, 128, 16, 0.75, 11),
    (4, 8, 8, [65, 130, 260, 1000], 8, 16, 4, 0.5, 12),
    (2, 16, 2, [5000, 1234], 32, 256, 64, 0.9, 13),
    (3, 12, 4, [40, 41, 300], 64, 8, 0, 0.3, 14),
    (1, 32, 8, [4097], 16, 256, 0, 1.0, 16),
]


def _run_torch(c, ready=None):
    f = lambda a: torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32))  # noqa: E731
    ring_q, ring_o, ring_l = f(c.query_cache).clone(), f(c.attn_cache).clone(), f(c.lse_cache).clone()
    k, v = f(c.k), f(c.v)
    params = tor.StepParams(semantic_pos_ahead=c.semantic_pos_ahead, front_sink_tokens=c.front_sink_tokens,
                            threshold=c.threshold, sm_scale=c.sm_scale)
    res = []
    for n in range(c.q_post.shape[0]):
        req = int(c.req_ids[n])
        r = tor.decode_request(q_post=f(c.q_post[n]), q_pre=f(c.q_pre[n]), k=k, v=v,
                               r2t_row=torch.from_numpy(c.req_to_token[req].astype(np.int64)),
                               P=int(c.past_lens[n]), cur_loc=int(c.out_cache_loc[n]), ring_q=ring_q[req],
                               ring_o=ring_o[req], ring_lse=ring_l[req], params=params,
                               ready=True if ready is None else bool(ready[n]))
        res.append(r)
    return res, ring_q, ring_o, ring_l


@pytest.mark.parametrize("cfg", CASES, ids=lambda c: f"B{c[0]}_Hq{c[1]}_Hkv{c[2]}_seed{c[-1]}")
def test_torch_restatement_matches_c_oracle(cfg):
    b, hq, hkv, kv_lens, m, s, f, hit_rate, seed = cfg
    c = syn.random_case(batch=b, hq=hq, hkv=hkv, kv_lens=kv_lens, capacity=m, semantic_pos_ahead=s,
                        front_sink_tokens=f, hit_rate=hit_rate, match_lag=m // 2, seed=seed)
    exp = oracle_run(c)
    got, ring_q, ring_o, ring_l = _run_torch(c)
    for n, r in enumerate(got):
        np.testing.assert_array_equal(r["head_hit"].numpy(), exp.head["hit"][n], err_msg=f"hit n={n}")
        np.testing.assert_array_equal(r["head_match_pos"].numpy(), exp.head["match_pos"][n], err_msg=f"pos n={n}")
        np.testing.assert_array_equal(r["group_mode"].numpy(), exp.group["mode"][n], err_msg=f"mode n={n}")
        assert rel_l2(r["out"].numpy(), bits(exp.out[n])) < 2e-3
        np.testing.assert_allclose(r["out_lse"].numpy(), exp.out_lse[n], rtol=1e-4, atol=1e-4)
    np.testing.assert_array_equal(syn.to_bits(ring_q.numpy()), exp.query_cache)
    assert rel_l2(ring_o.numpy(), bits(exp.attn_cache)) < 2e-3
    fin = np.isfinite(exp.lse_cache)
    np.testing.assert_array_equal(np.isfinite(ring_l.numpy()), fin)
    np.testing.assert_allclose(ring_l.numpy()[fin], exp.lse_cache[fin], rtol=1e-4, atol=1e-4)


def test_torch_restatement_readiness_gate():
    c = syn.random_case(batch=3, hq=32, hkv=8, kv_lens=[500, 600, 700], capacity=16, semantic_pos_ahead=64,
                        front_sink_tokens=8, hit_rate=1.0, match_lag=8, seed=21)
    c.cache_ready = np.array([1, 0, 1], np.uint8)
    exp = oracle_run(c)
    got, _, ring_o, _ = _run_torch(c, ready=c.cache_ready)
    for n, r in enumerate(got):
        np.testing.assert_array_equal(r["head_hit"].numpy(), exp.head["hit"][n])
        assert rel_l2(r["out"].numpy(), bits(exp.out[n])) < 2e-3
    np.testing.assert_array_equal(ring_o[1].numpy(), bits(c.attn_cache[1]) if c.attn_cache.dtype == np.uint16
                                  else c.attn_cache[1])


def test_torch_restatement_takes_bf16_pools():
    """K/V pools passed as bf16 tensors (only the gathered rows are widened)
    give the same results as the same values passed as float32."""
    c = syn.random_case(batch=2, hq=32, hkv=8, kv_lens=[700, 1500], capacity=32, semantic_pos_ahead=64,
                        front_sink_tokens=0, hit_rate=0.5, match_lag=16, seed=17)
    f = lambda a: torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32))  # noqa: E731
    params = tor.StepParams(semantic_pos_ahead=64, threshold=c.threshold, sm_scale=c.sm_scale)
    for n in range(2):
        req = int(c.req_ids[n])
        kw = dict(q_post=f(c.q_post[n]), q_pre=f(c.q_pre[n]),
                  r2t_row=torch.from_numpy(c.req_to_token[req].astype(np.int64)), P=int(c.past_lens[n]),
                  cur_loc=int(c.out_cache_loc[n]), params=params)
        rings = [(f(c.query_cache[req]).clone(), f(c.attn_cache[req]).clone(), f(c.lse_cache[req]).clone())
                 for _ in range(2)]  # (from_numpy shares the case's arrays; the step writes its ring row)
        a = tor.decode_request(k=f(c.k), v=f(c.v), ring_q=rings[0][0], ring_o=rings[0][1], ring_lse=rings[0][2], **kw)
        b = tor.decode_request(k=f(c.k).to(torch.bfloat16), v=f(c.v).to(torch.bfloat16), ring_q=rings[1][0],
                               ring_o=rings[1][1], ring_lse=rings[1][2], **kw)
        for key in ("head_hit", "head_match_pos", "group_mode", "out", "out_lse"):
            assert torch.equal(a[key], b[key]), key
        for x, y in zip(rings[0], rings[1]):
            assert torch.equal(x, y)
