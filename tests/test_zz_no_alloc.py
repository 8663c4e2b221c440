"""The no-allocation decode entry point (mac_persistent_decode_bf16_noalloc,
workspaces in the library's static device array) against the ordinary entry
point on the same inputs, through the C ABI: two calls in a row, the second
with a smaller step, each compared output for output (and with the oracle);
and the size limits are refused with a clear error."""

import numpy as np
import pytest

from helpers import bits, oracle_run, rel_l2, syn

torch = pytest.importorskip("torch")

pytestmark = pytest.mark.gpu


def _args(dev, case, ws, out, out_lse, max_context):
    return (dev["q_post"], dev["q_pre"], dev["k"], dev["v"], dev["req_to_token"], dev["req_ids"],
            dev["past_lens"], dev["out_cache_loc"], dev["query_cache"], dev["attn_cache"], dev["lse_cache"],
            out, out_lse, *ws, max_context, 32, 32, case.semantic_pos_ahead, case.front_sink_tokens,
            case.gen_min_limit, case.lookback_right, case.candidate_mode, case.threshold, case.sm_scale, 0, 0,
            1.0, 0.0, -1.0, 0.0, 64.0, 0.0, 1, -1, 0, dev["query_cache"], dev["cache_ready"], dev["cache_epoch"],
            dev["request_epoch"])


def _np(t):
    return t.float().cpu().numpy() if t.dtype == torch.bfloat16 else t.cpu().numpy()


CASES = [
    # (batch, hq, hkv, kv_lens, M, S, F, hit_rate, seed): the second is smaller
    (6, 32, 8, [3000, 5000, 777, 4096, 2000, 10000], 32, 64, 16, 0.6, 71),
    (3, 32, 4, [700, 1500, 300], 16, 128, 0, 0.7, 72),
]


def test_noalloc_entry_matches_the_workspace_entry():
    from mac_attention.integrations.sglang.bridge import load_mac_persistent_decode_extension

    ext = load_mac_persistent_decode_extension(False)
    for cfg in CASES:  # two calls in a row, the second smaller
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
            ws = syn.workspace(torch, batch=b, hq=hq, hkv=hkv, capacity=m, max_context=max_context, tile_tokens=32,
                               match_tile_slots=32, semantic_pos_ahead=s, front_sink_tokens=f, device="cuda")
            out = torch.empty_like(dev["q_post"])
            out_lse = torch.empty(b, hq, device="cuda")
            fn = ext.mac_persistent_decode_bf16 if mode == "workspace" else ext.mac_persistent_decode_bf16_noalloc
            fn(*_args(dev, c, ws, out, out_lse, max_context))
            torch.cuda.synchronize()
            runs[mode] = dict(out=_np(out), lse=_np(out_lse), q=syn.to_bits(_np(dev["query_cache"])),
                              a=_np(dev["attn_cache"]), l=_np(dev["lse_cache"]))
        w, n = runs["workspace"], runs["noalloc"]
        assert rel_l2(n["out"], w["out"]) < 1e-3
        np.testing.assert_allclose(n["lse"], w["lse"], atol=1e-3, rtol=1e-3)
        np.testing.assert_array_equal(n["q"], w["q"])
        assert rel_l2(n["a"], w["a"]) < 1e-3
        fin = np.isfinite(w["l"])
        np.testing.assert_array_equal(np.isfinite(n["l"]), fin)
        np.testing.assert_allclose(n["l"][fin], w["l"][fin], atol=1e-3, rtol=1e-3)
        # and both against the oracle, to the parity bar
        assert rel_l2(n["out"], bits(res.out)) < 1e-2
        np.testing.assert_array_equal(n["q"], res.query_cache)
        assert rel_l2(n["a"], bits(res.attn_cache)) < 1e-2


def test_noalloc_entry_refuses_steps_beyond_its_array():
    from mac_attention.integrations.sglang.bridge import load_mac_persistent_decode_extension

    ext = load_mac_persistent_decode_extension(False)
    b, hq, hkv = 129, 32, 8  # 4128 query heads > 4096
    c = syn.random_case(batch=b, hq=hq, hkv=hkv, kv_lens=[40] * b, capacity=8, semantic_pos_ahead=8,
                        hit_rate=0.0, seed=73)
    dev = syn.to_device(torch, c)
    ws = syn.workspace(torch, batch=b, hq=hq, hkv=hkv, capacity=8, max_context=64, tile_tokens=32,
                       match_tile_slots=32, semantic_pos_ahead=8, device="cuda")
    out = torch.empty_like(dev["q_post"])
    with pytest.raises(RuntimeError, match="at most 4096 query heads"):
        ext.mac_persistent_decode_bf16_noalloc(*_args(dev, c, ws, out, torch.empty(b, hq, device="cuda"), 64))
