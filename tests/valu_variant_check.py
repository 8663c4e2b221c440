"""Runs a few decode cases through the VALU span-attention kernel
(MAC_AMD_ATTN_IMPL=valu, read once per process) and checks them against the
CPU oracle.  Started as a child process by test_valu_variant_gpu.py."""

import os
import sys

sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))

import torch  # noqa: E402

import kat_cases  # noqa: E402
from helpers import oracle_run, syn  # noqa: E402
from test_decode_gpu import RANDOM_CASES, _check_against_oracle  # noqa: E402


def main():
    assert os.environ.get("MAC_AMD_ATTN_IMPL") == "valu"
    from mac_attention.integrations.sglang.bridge import load_mac_persistent_decode_extension

    ext = load_mac_persistent_decode_extension(False)
    for builder in (kat_cases.ALL[0], kat_cases.ALL[5]):
        kat = builder()
        for k, v in kat.env.items():
            os.environ[k] = v
        c = kat.case
        res = oracle_run(c)
        dev = syn.to_device(torch, c)
        out, out_lse, ws = syn.run_decode(torch, ext, dev, c, max_context=kat.max_context,
                                          tile_tokens=kat.tile_tokens, match_tile_slots=kat.match_tile_slots)
        torch.cuda.synchronize()
        _check_against_oracle(c, dev, out, out_lse, ws, res, what=f"valu {kat.name}")
        for k in kat.env:
            os.environ.pop(k)
        print(f"ok {kat.name}", flush=True)
    for cfg in RANDOM_CASES[:4]:
        b, hq, hkv, kv_lens, m, s, f, hit_rate, seed = cfg
        c = syn.random_case(batch=b, hq=hq, hkv=hkv, kv_lens=kv_lens, capacity=m, semantic_pos_ahead=s,
                            front_sink_tokens=f, hit_rate=hit_rate, match_lag=m // 2, seed=seed)
        res = oracle_run(c)
        dev = syn.to_device(torch, c)
        out, out_lse, ws = syn.run_decode(torch, ext, dev, c, max_context=max(kv_lens) + 64, tile_tokens=16,
                                          match_tile_slots=8)
        torch.cuda.synchronize()
        _check_against_oracle(c, dev, out, out_lse, ws, res, what=f"valu random {cfg}")
        print(f"ok random seed {seed}", flush=True)
    print("VALU variant OK", flush=True)


if __name__ == "__main__":
    main()
