"""Loads the committed known-answer fixtures (tests/golden/kat_*.npz, written
by tests/golden/make_golden.py) back into kat_cases.Kat objects."""

from __future__ import annotations

import glob
import json
import os

import numpy as np

import kat_cases
from helpers import syn

GOLDEN_DIR = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def fixture_paths():
    return sorted(glob.glob(os.path.join(GOLDEN_DIR, "kat_*.npz")))


def load(path: str) -> kat_cases.Kat:
    z = np.load(path, allow_pickle=False)
    meta = json.loads(bytes(z["meta"]).decode())
    sc = meta["scalars"]
    case = syn.Case(
        q_post=syn.from_bits(z["in_q_post"]), q_pre=syn.from_bits(z["in_q_pre"]),
        k=syn.from_bits(z["in_k"]), v=syn.from_bits(z["in_v"]),
        req_to_token=z["in_req_to_token"], req_ids=z["in_req_ids"], past_lens=z["in_past_lens"],
        out_cache_loc=z["in_out_cache_loc"], query_cache=syn.from_bits(z["in_query_cache"]),
        attn_cache=syn.from_bits(z["in_attn_cache"]), lse_cache=z["in_lse_cache"],
        semantic_pos_ahead=int(sc["semantic_pos_ahead"]), front_sink_tokens=int(sc["front_sink_tokens"]),
        threshold=float(sc["threshold"]), sm_scale=float(sc["sm_scale"]),
        gen_min_limit=int(sc["gen_min_limit"]), lookback_right=int(sc["lookback_right"]),
        candidate_mode=int(sc["candidate_mode"]))
    get = lambda k: z[k] if k in z.files else None  # noqa: E731
    return kat_cases.Kat(
        name=meta["name"], case=case, max_context=meta["max_context"], tile_tokens=meta["tile_tokens"],
        match_tile_slots=meta["match_tile_slots"], o_tol=meta["o_tol"], lse_tol=meta["lse_tol"],
        exp_out={n: (z[f"exp_out_o_{n}"], z[f"exp_out_lse_{n}"]) for n in meta["out_requests"]},
        exp_ring={n: (z[f"exp_ring_o_{n}"], z[f"exp_ring_lse_{n}"]) for n in meta["ring_requests"]},
        head_hit=get("exp_head_hit"), head_match_pos=get("exp_head_match_pos"),
        group_mode=get("exp_group_mode"), env=meta["env"], ring_exact_empty=meta["ring_exact_empty"],
        min_reduce_groups=meta["min_reduce_groups"],
        tol_per_head={int(h): tuple(t) for h, t in meta["tol_per_head"].items()})


class _Loader:
    """A kat builder that reads a fixture (usable wherever kat_cases builders are)."""

    def __init__(self, path: str):
        self.path = path
        self.__name__ = "golden_" + os.path.basename(path)[len("kat_"):-len(".npz")]

    def __call__(self) -> kat_cases.Kat:
        return load(self.path)


LOADERS = [_Loader(p) for p in fixture_paths()]
