"""Pins the CPU oracle against the reference's known-answer cases (CPU only)."""

import os

import numpy as np
import pytest

import golden_cases
import kat_cases
from helpers import assert_close, bits, oracle_run, rel_l2


def _apply_env(monkeypatch, env):
    for k, v in env.items():
        monkeypatch.setenv(k, v)


@pytest.mark.parametrize("builder", kat_cases.ALL + golden_cases.LOADERS, ids=lambda f: f.__name__)
def test_oracle_reproduces_reference_kat(builder, monkeypatch):
    kat = builder()
    _apply_env(monkeypatch, kat.env)
    res = oracle_run(kat.case)
    c = kat.case
    if kat.head_hit is not None:
        np.testing.assert_array_equal(res.head["hit"], kat.head_hit)
    if kat.head_match_pos is not None:
        np.testing.assert_array_equal(res.head["match_pos"], kat.head_match_pos)
    if kat.group_mode is not None:
        np.testing.assert_array_equal(res.group["mode"], kat.group_mode)
    m = c.query_cache.shape[1]
    for n, (eo, el) in kat.exp_out.items():
        got = bits(res.out[n])
        assert_close(got, eo, kat.o_tol, f"{kat.name} out[{n}]")
        assert_close(res.out_lse[n], el, kat.lse_tol, f"{kat.name} out_lse[{n}]")
        assert rel_l2(got, eo) < 1e-2
    for n, (ro, rl) in kat.exp_ring.items():
        dest = int(c.past_lens[n]) % m
        got = bits(res.attn_cache[n, dest])
        assert_close(got, ro, kat.o_tol, f"{kat.name} ring o[{n}]")
        assert_close(res.lse_cache[n, dest], rl, kat.lse_tol, f"{kat.name} ring lse[{n}]")
        assert rel_l2(got, ro) < 1e-2
        # the ring row's query is the current pre-RoPE query, bit for bit
        np.testing.assert_array_equal(bits(res.query_cache[n, dest]), c.q_pre[n])
    if kat.ring_exact_empty:
        dest = int(c.past_lens[0]) % m
        np.testing.assert_array_equal(bits(res.query_cache[0, dest]), c.q_pre[0])
        assert np.all(res.attn_cache[0, dest] == 0)
        assert np.all(np.isneginf(res.lse_cache[0, dest]))


def test_oracle_two_step_recurrence():
    """tools/check_front_sink_recurrence.py: written entries exclude the sink,
    and reusing them in the next step is exact."""
    r = kat_cases.recurrence_inputs()
    os.environ.setdefault("MAC_PERSISTENT_MIXED_GROUP_FALLBACK", "1")
    res1 = oracle_run(r["step1"])
    assert res1.head["hit"][0].tolist() == [1] * 6 + [0] * 2
    d1 = r["dest1"]
    written = bits(res1.attn_cache[0, d1])
    for h in range(r["hq"]):
        exp = r["e_hit"][0][h] if h in r["hit_heads"] else r["e_miss"][0][h]
        assert rel_l2(written[h], exp) < 0.08
    step2 = r["step2"](bits(res1.query_cache), bits(res1.attn_cache), res1.lse_cache)
    res2 = oracle_run(step2)
    assert res2.head["hit"][0].tolist() == [1] * r["hq"]
    assert res2.head["match_pos"][0].tolist() == [r["p1"]] * r["hq"]
    hit = np.array([h in r["hit_heads"] for h in range(r["hq"])])
    base_o = np.where(hit[:, None], r["e_hit"][0], r["e_miss"][0])
    base_l = np.where(hit, r["e_hit"][1], r["e_miss"][1])
    ref_o, _ = r["expected_step2"](base_o, base_l)
    assert rel_l2(bits(res2.out[0]), ref_o) < 0.08
