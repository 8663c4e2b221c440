"""Writes the known-answer fixtures under tests/golden/ (one .npz per case).

Each case is one of the reference's known-answer tests
(attention/tests/test_mac_persistent_decode.py:100-466 and
attention/tools/check_mac_persistent_decode.py:209-921), rebuilt with
numpy-seeded inputs by tests/kat_cases.py.  Its expected values come from
the reference's closed-form recipe -- exact softmax attention over each span
in float64 and LSE merges (test_mac_persistent_decode.py:9-51) -- and the
integer decisions from how each case is constructed.  Nothing here runs the
C oracle or the GPU library: the fixtures are what both are checked against.

bf16 tensors are stored as their 16-bit patterns; run from the repository
root:  python tests/golden/make_golden.py
"""

from __future__ import annotations

import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
TESTS = os.path.dirname(HERE)
REPO = os.path.dirname(TESTS)
for _p in (TESTS, os.path.join(REPO, "mac-attention_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

import kat_cases  # noqa: E402
from mac_attention import synthetic as syn  # noqa: E402

BF16_FIELDS = ("q_post", "q_pre", "k", "v", "query_cache", "attn_cache")
INT_FIELDS = ("req_to_token", "req_ids", "past_lens", "out_cache_loc")
SCALARS = ("semantic_pos_ahead", "front_sink_tokens", "threshold", "sm_scale", "gen_min_limit",
           "lookback_right", "candidate_mode")


def case_arrays(kat) -> dict:
    c = kat.case
    a = {f"in_{f}": syn.to_bits(getattr(c, f)) for f in BF16_FIELDS}
    a.update({f"in_{f}": np.asarray(getattr(c, f)) for f in INT_FIELDS})
    a["in_lse_cache"] = np.asarray(c.lse_cache, np.float32)
    for n, (o, lse) in kat.exp_out.items():
        a[f"exp_out_o_{n}"] = np.asarray(o, np.float64)
        a[f"exp_out_lse_{n}"] = np.asarray(lse, np.float64)
    for n, (o, lse) in kat.exp_ring.items():
        a[f"exp_ring_o_{n}"] = np.asarray(o, np.float64)
        a[f"exp_ring_lse_{n}"] = np.asarray(lse, np.float64)
    for f in ("head_hit", "head_match_pos", "group_mode"):
        v = getattr(kat, f)
        if v is not None:
            a[f"exp_{f}"] = np.asarray(v, np.int32)
    meta = {
        "name": kat.name,
        "scalars": {s: getattr(c, s) for s in SCALARS},
        "max_context": kat.max_context, "tile_tokens": kat.tile_tokens,
        "match_tile_slots": kat.match_tile_slots, "o_tol": kat.o_tol, "lse_tol": kat.lse_tol,
        "env": kat.env, "ring_exact_empty": kat.ring_exact_empty,
        "min_reduce_groups": kat.min_reduce_groups,
        "tol_per_head": {str(h): list(t) for h, t in kat.tol_per_head.items()},
        "out_requests": sorted(int(n) for n in kat.exp_out),
        "ring_requests": sorted(int(n) for n in kat.exp_ring),
    }
    a["meta"] = np.frombuffer(json.dumps(meta, sort_keys=True).encode(), dtype=np.uint8)
    return a


def main() -> None:
    for builder in kat_cases.ALL:
        kat = builder()
        path = os.path.join(HERE, f"kat_{builder.__name__}.npz")
        np.savez_compressed(path, **case_arrays(kat))
        print(f"{path}: {os.path.getsize(path)} bytes")


if __name__ == "__main__":
    main()
