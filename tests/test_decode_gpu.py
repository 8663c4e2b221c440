"""GPU parity of the fused MAC decode step, through the reference's 68-argument
binding (which calls the C ABI of libmac_hip.so).

Expected values: the reference's known-answer recipe (kat_cases) and the CPU
oracle on identical inputs.  Integer decisions must match the oracle exactly;
values within the reference's tolerances and 1e-2 relative L2.
"""

import numpy as np
import pytest

import golden_cases
import kat_cases
from helpers import assert_close, bits, near_threshold_heads, oracle_run, rel_l2, syn

torch = pytest.importorskip("torch")

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ext():
    from mac_attention.integrations.sglang.bridge import load_mac_persistent_decode_extension

    return load_mac_persistent_decode_extension(False)


def _np(t):
    if t.dtype == torch.bfloat16:
        return t.float().cpu().numpy()
    return t.cpu().numpy()


def _check_against_oracle(case, dev, out, out_lse, ws, res, tol=1e-2, what=""):
    n_req = case.q_post.shape[0]
    near = near_threshold_heads(res, threshold=case.threshold, what=what)
    assert not near.any(), f"{what}: inputs put a decision within 1e-6 of the threshold (logged)"
    np.testing.assert_array_equal(_np(ws[3])[:n_req], res.head["hit"], err_msg=f"{what} head_hit")
    np.testing.assert_array_equal(_np(ws[5])[:n_req], res.head["match_pos"], err_msg=f"{what} match_pos")
    np.testing.assert_array_equal(_np(ws[4])[:n_req], res.head["match_slot"], err_msg=f"{what} match_slot")
    np.testing.assert_array_equal(_np(ws[7])[:n_req], res.head["rect_start"], err_msg=f"{what} rect_start")
    np.testing.assert_array_equal(_np(ws[15])[:n_req], res.group["mode"], err_msg=f"{what} group_mode")
    np.testing.assert_array_equal(_np(ws[9])[:n_req], res.group["rect_begin"], err_msg=f"{what} rect_begin")
    got = _np(out)
    exp = bits(res.out)
    assert rel_l2(got, exp) < tol, f"{what} out rel_l2 {rel_l2(got, exp)}"
    assert_close(got, exp, 3e-2, f"{what} out")
    assert_close(_np(out_lse), res.out_lse, 3e-2, f"{what} out_lse")
    qc, ac, lc = _np(dev["query_cache"]), _np(dev["attn_cache"]), _np(dev["lse_cache"])
    np.testing.assert_array_equal(syn.to_bits(qc), res.query_cache, err_msg=f"{what} query_cache")
    assert rel_l2(ac, bits(res.attn_cache)) < tol, f"{what} attn_cache"
    assert_close(ac, bits(res.attn_cache), 3e-2, f"{what} attn_cache")
    assert_close(lc, res.lse_cache, 3e-2, f"{what} lse_cache")


# Groups of at most MAC_AMD_FUSE_TOKENS tokens are short: one computation
# (short_group) finishes each of them, inside match_decide or as one task of
# span_attention.  "fused": match_decide finishes every short group
# (MAC_AMD_FUSE_POLICY=always); "split": no group is short, every group goes
# through span_attention's pieces and merge_write; "auto": the default
# step-wide rule places the short groups.  All must give the oracle's
# results; "fused" and "auto" give the same bits.
FUSE = {"fused": ("always", None), "split": (None, "0"), "auto": (None, None)}


def _set_fuse(monkeypatch, mode):
    policy, tokens = FUSE[mode]
    for name, value in (("MAC_AMD_FUSE_POLICY", policy), ("MAC_AMD_FUSE_TOKENS", tokens)):
        if value is None:
            monkeypatch.delenv(name, raising=False)
        else:
            monkeypatch.setenv(name, value)


@pytest.mark.parametrize("fuse", list(FUSE))
@pytest.mark.parametrize("partial", ["f32", "bf16"])
@pytest.mark.parametrize("builder", kat_cases.ALL + golden_cases.LOADERS, ids=lambda f: f.__name__)
def test_reference_kat(builder, partial, fuse, ext, monkeypatch):
    kat = builder()
    for k, v in kat.env.items():
        monkeypatch.setenv(k, v)
    _set_fuse(monkeypatch, fuse)
    print(f"case={kat.name} partial={partial} fuse={fuse}", flush=True)
    _run_kat(kat, partial, ext)


def _run_kat(kat, partial, ext):
    """One known-answer case on the GPU: the decisions it pins, its expected
    outputs and ring rows, and the oracle on every output."""
    c = kat.case
    res = oracle_run(c)
    dev = syn.to_device(torch, c)
    pdt = torch.float32 if partial == "f32" else torch.bfloat16
    out, out_lse, ws = syn.run_decode(torch, ext, dev, c, max_context=kat.max_context,
                                      tile_tokens=kat.tile_tokens,
                                      match_tile_slots=kat.match_tile_slots, partial_dtype=pdt)
    torch.cuda.synchronize()
    if kat.head_hit is not None:
        np.testing.assert_array_equal(_np(ws[3]), kat.head_hit)
    if kat.head_match_pos is not None:
        np.testing.assert_array_equal(_np(ws[5]), kat.head_match_pos)
    if kat.group_mode is not None:
        np.testing.assert_array_equal(_np(ws[15]), kat.group_mode)
    if kat.min_reduce_groups:
        assert int(_np(ws[22])[3]) >= kat.min_reduce_groups
    m = c.query_cache.shape[1]
    o = _np(out)
    for n, (eo, el) in kat.exp_out.items():
        assert_close(o[n], eo, kat.o_tol, f"{kat.name} out[{n}]")
        assert_close(_np(out_lse)[n], el, kat.lse_tol, f"{kat.name} out_lse[{n}]")
    ac, lc, qc = _np(dev["attn_cache"]), _np(dev["lse_cache"]), _np(dev["query_cache"])
    for n, (ro, rl) in kat.exp_ring.items():
        dest = int(c.past_lens[n]) % m
        assert_close(ac[n, dest], ro, kat.o_tol, f"{kat.name} ring o[{n}]")
        assert_close(lc[n, dest], rl, kat.lse_tol, f"{kat.name} ring lse[{n}]")
    if kat.ring_exact_empty:
        dest = int(c.past_lens[0]) % m
        np.testing.assert_array_equal(qc[0, dest], c.q_pre[0])
        assert np.all(ac[0, dest] == 0)
        assert np.all(np.isneginf(lc[0, dest]))
    _check_against_oracle(c, dev, out, out_lse, ws, res, tol=1e-2 if partial == "f32" else 2e-2,
                          what=kat.name)


def test_two_step_recurrence(ext, monkeypatch):
    monkeypatch.setenv("MAC_PERSISTENT_MIXED_GROUP_FALLBACK", "1")
    r = kat_cases.recurrence_inputs()
    c1 = r["step1"]
    dev = syn.to_device(torch, c1)
    syn.run_decode(torch, ext, dev, c1, max_context=32)
    torch.cuda.synchronize()
    qc, ac, lc = _np(dev["query_cache"]), _np(dev["attn_cache"]), _np(dev["lse_cache"])
    d1 = r["dest1"]
    for h in range(r["hq"]):
        exp = r["e_hit"][0][h] if h in r["hit_heads"] else r["e_miss"][0][h]
        assert rel_l2(ac[0, d1, h], exp) < 0.08
    c2 = r["step2"](qc, ac, lc)
    dev2 = syn.to_device(torch, c2)
    out2, _, ws2 = syn.run_decode(torch, ext, dev2, c2, max_context=32)
    torch.cuda.synchronize()
    assert _np(ws2[3])[0].tolist() == [1] * r["hq"]
    assert _np(ws2[5])[0].tolist() == [r["p1"]] * r["hq"]
    hit = np.array([h in r["hit_heads"] for h in range(r["hq"])])
    base_o = np.where(hit[:, None], r["e_hit"][0], r["e_miss"][0])
    base_l = np.where(hit, r["e_hit"][1], r["e_miss"][1])
    ref_o, _ = r["expected_step2"](base_o, base_l)
    assert rel_l2(_np(out2)[0], ref_o) < 0.08


RANDOM_CASES = [
    # (batch, hq, hkv, kv_lens, M, S, F, hit_rate, seed)
    (3, 32, 8, [300, 517, 1024], 32, 64, 0, 0.5, 10),
    (2, 32, 4, [777, 2049], 16, 128, 16, 0.75, 11),
    (4, 8, 8, [65, 130, 260, 1000], 8, 16, 4, 0.5, 12),
    (2, 16, 2, [5000, 1234], 32, 256, 64, 0.9, 13),
    (3, 12, 4, [40, 41, 300], 64, 8, 0, 0.3, 14),
    (2, 6, 1, [200, 300], 16, 32, 8, 0.6, 15),
    (1, 32, 8, [4097], 16, 256, 0, 1.0, 16),
    (2, 32, 8, [3000, 3001], 32, 256, 128, 0.0, 17),
    (2, 10, 2, [900, 1500], 16, 64, 8, 0.6, 19),   # G = 5
    (2, 14, 2, [700, 2100], 32, 128, 0, 0.7, 20),  # G = 7
    # rings of several scan batches per wave (the scan's loop; one group per
    # CU or fewer, so the eight-wave decision kernel)
    (2, 32, 4, [3000, 700], 256, 64, 8, 0.7, 21),   # G = 8, M = 256
    (2, 16, 4, [900, 2500], 128, 32, 0, 0.6, 22),   # G = 4, M = 128
]


@pytest.mark.parametrize("fuse", list(FUSE))
@pytest.mark.parametrize("cfg", RANDOM_CASES, ids=lambda c: f"B{c[0]}_Hq{c[1]}_Hkv{c[2]}_seed{c[-1]}")
def test_random_vs_oracle(cfg, fuse, ext, monkeypatch):
    b, hq, hkv, kv_lens, m, s, f, hit_rate, seed = cfg
    _set_fuse(monkeypatch, fuse)
    print(f"random case {cfg} fuse={fuse}", flush=True)
    c = syn.random_case(batch=b, hq=hq, hkv=hkv, kv_lens=kv_lens, capacity=m, semantic_pos_ahead=s,
                        front_sink_tokens=f, hit_rate=hit_rate, match_lag=m // 2, seed=seed)
    res = oracle_run(c)
    dev = syn.to_device(torch, c, out_cache_loc_dtype=torch.int32 if seed % 2 else torch.int64)
    out, out_lse, ws = syn.run_decode(torch, ext, dev, c, max_context=max(kv_lens) + 8,
                                      tile_tokens=16, match_tile_slots=8)
    torch.cuda.synchronize()
    _check_against_oracle(c, dev, out, out_lse, ws, res, what=str(cfg))


@pytest.mark.parametrize("seed", range(8))
def test_random_shapes_vs_oracle(seed, ext, monkeypatch):
    """Seeded random steps against the oracle: batch, GQA shape (G = 1..8),
    context lengths (short and long, odd), ring size, window S, front sink,
    hit rate and the short-group policy drawn per seed."""
    rng = np.random.default_rng(500 + seed)
    b = int(rng.integers(1, 6))
    hkv = int(rng.choice([1, 2, 4, 8]))
    g = int(rng.integers(1, 9))
    hq = hkv * g
    m = int(rng.choice([8, 16, 32, 64]))
    s = int(rng.choice([8, 32, 128, 256]))
    f = int(rng.choice([0, 0, 4, 64]))
    kv_lens = [int(x) for x in rng.integers(2, 3000, b)]
    hit_rate = float(rng.choice([0.0, 0.5, 0.8, 1.0]))
    fuse = list(FUSE)[seed % len(FUSE)]
    cfg = (b, hq, hkv, kv_lens, m, s, f, hit_rate, seed)
    _set_fuse(monkeypatch, fuse)
    print(f"random shapes {cfg} fuse={fuse}", flush=True)
    c = syn.random_case(batch=b, hq=hq, hkv=hkv, kv_lens=kv_lens, capacity=m, semantic_pos_ahead=s,
                        front_sink_tokens=f, hit_rate=hit_rate, match_lag=max(m // 2, 1), seed=600 + seed)
    res = oracle_run(c)
    dev = syn.to_device(torch, c, out_cache_loc_dtype=torch.int32 if seed % 2 else torch.int64)
    out, out_lse, ws = syn.run_decode(torch, ext, dev, c, max_context=max(kv_lens) + 8,
                                      tile_tokens=16, match_tile_slots=8)
    torch.cuda.synchronize()
    _check_against_oracle(c, dev, out, out_lse, ws, res, what=str(cfg))


def _bits(dev, out, out_lse):
    return [out.view(torch.int16).clone(), out_lse.view(torch.int32).clone(),
            dev["attn_cache"].view(torch.int16).clone(), dev["lse_cache"].view(torch.int32).clone(),
            dev["query_cache"].view(torch.int16).clone()]


@pytest.mark.parametrize("hkv", [8, 4])
def test_decode_is_deterministic(hkv, ext, monkeypatch):
    """A step's results depend on its inputs only, with the default
    short-group rule: after a fresh workspace, after a step of another shape
    on the same workspace, after steps with other hits (which move the short
    groups between match_decide and span_attention), with every short group
    pinned to match_decide, and with the four- and eight-wave decision
    kernels, the outputs and ring rows are the same bits.  Mixed hits,
    misses and long groups; 64 groups or fewer per step (the eight-wave
    match_decide) and more (four waves)."""
    _set_fuse(monkeypatch, "auto")
    batch = 8 if hkv == 8 else 80
    rng = np.random.default_rng(31)
    kv_lens = rng.integers(300, 6000, batch).tolist()
    max_context = 20008
    print(f"decode determinism: Hkv={hkv} B={batch}", flush=True)

    def case(hit, seed, lens=kv_lens):
        return syn.random_case(batch=len(lens), hq=32, hkv=hkv, kv_lens=lens, capacity=32, semantic_pos_ahead=64,
                               front_sink_tokens=8, hit_rate=hit, match_lag=16, seed=seed)

    c = case(0.7, 31)
    ws = syn.workspace(torch, batch=batch, hq=32, hkv=hkv, capacity=32, max_context=max_context, tile_tokens=64,
                       match_tile_slots=8, semantic_pos_ahead=64, front_sink_tokens=8, device="cuda")
    ng = batch * hkv

    def step(cc, ws_=ws):
        dev = syn.to_device(torch, cc)
        out, out_lse, w = syn.run_decode(torch, ext, dev, cc, max_context=max_context, tile_tokens=64,
                                         match_tile_slots=8, ws=ws_)
        torch.cuda.synchronize()
        return _bits(dev, out, out_lse), _np(w[16])[ng:2 * ng].copy()

    ws[16].zero_()  # no history
    ref, placed_first = step(c)
    runs = {"no history": ref}
    runs["repeat"], placed_repeat = step(c)
    step(case(0.7, 31, [40] * (batch // 2)))  # a smaller batch on the same workspace
    runs["after another shape"], _ = step(c)
    step(case(0.0, 32, [20000] * batch))  # all long: the next step leaves its short groups to span_attention
    runs["after long steps"], placed_after_long = step(c)
    step(case(1.0, 33))
    runs["after all-hit steps"], _ = step(c)
    _set_fuse(monkeypatch, "fused")
    runs["all in match_decide"], placed_fused = step(c)
    monkeypatch.setenv("MAC_AMD_MATCH_WAVES", "4")
    runs["four-wave decisions"], _ = step(c)
    monkeypatch.delenv("MAC_AMD_MATCH_WAVES")
    # the placements differ (so both places ran short groups) ...
    assert placed_fused.sum() > 0 and placed_after_long.sum() < placed_fused.sum(), \
        (placed_fused.sum(), placed_after_long.sum())
    # ... and the bits do not
    for name, r in runs.items():
        for i, (a, b) in enumerate(zip(r, ref)):
            assert torch.equal(a, b), f"{name}: tensor {i} differs from the first step's"
    # and they are the oracle's
    dev = syn.to_device(torch, c)
    out, out_lse, w = syn.run_decode(torch, ext, dev, c, max_context=max_context, tile_tokens=64, match_tile_slots=8)
    torch.cuda.synchronize()
    _check_against_oracle(c, dev, out, out_lse, w, oracle_run(c), what=f"determinism Hkv={hkv}")


@pytest.mark.parametrize("case", [f.__name__ for f in kat_cases.ALL + golden_cases.LOADERS]
                         + [f"random_seed{c[-1]}" for c in RANDOM_CASES])
def test_four_wave_decision_kernel(case, ext, monkeypatch):
    """Steps of at most one group per CU run the eight-wave match_decide by
    default; the four-wave form (the one larger steps run) is checked on the
    same known-answer and random cases with MAC_AMD_MATCH_WAVES=4, every
    short group finished inside it (its largest share of the work)."""
    monkeypatch.setenv("MAC_AMD_MATCH_WAVES", "4")
    _set_fuse(monkeypatch, "fused")
    print(f"four-wave decision kernel: {case}", flush=True)
    if case.startswith("random_seed"):
        cfg = next(c for c in RANDOM_CASES if f"random_seed{c[-1]}" == case)
        b, hq, hkv, kv_lens, m, s, f, hit_rate, seed = cfg
        c = syn.random_case(batch=b, hq=hq, hkv=hkv, kv_lens=kv_lens, capacity=m, semantic_pos_ahead=s,
                            front_sink_tokens=f, hit_rate=hit_rate, match_lag=m // 2, seed=seed)
        dev = syn.to_device(torch, c)
        out, out_lse, ws = syn.run_decode(torch, ext, dev, c, max_context=max(kv_lens) + 8, tile_tokens=16,
                                          match_tile_slots=8)
        torch.cuda.synchronize()
        _check_against_oracle(c, dev, out, out_lse, ws, oracle_run(c), what=case)
        return
    builder = next(f for f in kat_cases.ALL + golden_cases.LOADERS if f.__name__ == case)
    kat = builder()
    for k, v in kat.env.items():
        monkeypatch.setenv(k, v)
    _run_kat(kat, "f32", ext)


def test_readiness_gate(ext):
    """Not-ready and epoch-mismatched requests run exact attention and leave
    their ring rows untouched (DECODE:208-230, :4487-4497)."""
    c = syn.random_case(batch=4, hq=32, hkv=8, kv_lens=[500, 600, 700, 800], capacity=16,
                        semantic_pos_ahead=64, front_sink_tokens=8, hit_rate=1.0, match_lag=8,
                        seed=21)
    c.cache_ready = np.array([1, 0, 1, 1], np.uint8)
    c.cache_epoch = np.array([3, 3, 2, 5], np.int64)
    c.request_epoch = np.array([3, 3, 7, 5], np.int64)
    res = oracle_run(c)
    assert res.head["hit"][1].sum() == 0 and res.head["hit"][2].sum() == 0
    assert res.head["hit"][0].sum() == 32 and res.head["hit"][3].sum() == 32
    dev = syn.to_device(torch, c)
    before = _np(dev["attn_cache"]).copy()
    out, out_lse, ws = syn.run_decode(torch, ext, dev, c, max_context=1024, tile_tokens=32)
    torch.cuda.synchronize()
    _check_against_oracle(c, dev, out, out_lse, ws, res, what="ready gate")
    after = _np(dev["attn_cache"])
    np.testing.assert_array_equal(after[1], before[1])
    np.testing.assert_array_equal(after[2], before[2])


@pytest.mark.parametrize("bench_mode", [1, 2])
def test_bench_mode_override(bench_mode, ext):
    """Synthetic bench override (DECODE:1184-1269) gives the oracle's decisions."""
    c = syn.random_case(batch=3, hq=32, hkv=8, kv_lens=[1000, 1100, 1200], capacity=32,
                        semantic_pos_ahead=64, hit_rate=0.0, seed=31, entry_builder="random")
    c.lse_cache[:] = 0.0  # every slot holds a finite entry, as in the reference's bench case
    bench = dict(bench_mode=bench_mode, bench_hit_rate=0.7, bench_match_lag_mean=16.0, bench_seed=5)
    res = oracle_run(c, bench_mode=bench_mode, bench_hit_rate=0.7, bench_match_lag_mean=16.0,
                     bench_seed=5)
    dev = syn.to_device(torch, c)
    out, out_lse, ws = syn.run_decode(torch, ext, dev, c, max_context=1300, tile_tokens=32,
                                      bench=bench)
    torch.cuda.synchronize()
    _check_against_oracle(c, dev, out, out_lse, ws, res, what=f"bench{bench_mode}")


@pytest.mark.parametrize("fuse", list(FUSE))
@pytest.mark.parametrize("batch,hkv", [(512, 8), (1024, 8), (700, 16)])
def test_many_groups(batch, hkv, fuse, ext, monkeypatch):
    """Batches of N * Hkv = 4096, 8192 and 11200 groups: the task planner's
    LDS table holds 4096 entries, so larger batches share an entry between
    two or three consecutive groups; every request against the oracle, with
    the groups finished inside match_decide and all through span_attention."""
    _set_fuse(monkeypatch, fuse)
    hq = 4 * hkv
    rng = np.random.default_rng(61 + batch)
    kv_lens = [int(x) for x in rng.integers(20, 120, size=batch)]
    c = syn.random_case(batch=batch, hq=hq, hkv=hkv, kv_lens=kv_lens, capacity=16, semantic_pos_ahead=32,
                        front_sink_tokens=4, hit_rate=0.5, match_lag=8, seed=61 + batch)
    print(f"many groups: N={batch} Hq={hq} Hkv={hkv} fuse={fuse}", flush=True)
    res = oracle_run(c)
    dev = syn.to_device(torch, c)
    out, out_lse, ws = syn.run_decode(torch, ext, dev, c, max_context=160, tile_tokens=32)
    torch.cuda.synchronize()
    _check_against_oracle(c, dev, out, out_lse, ws, res, what=f"N={batch} Hkv={hkv}")


def test_phase_cycles_stamps(ext):
    """debug_enabled >= 2 stores six device-clock stamps in phase_cycles
    (the reference's phase_cycles, DECODE:4751-4929): non-decreasing, and the
    step's ring-row and output writes are unchanged by the stamping."""
    c = syn.random_case(batch=3, hq=32, hkv=8, kv_lens=[900, 5000, 3000], capacity=32,
                        semantic_pos_ahead=64, front_sink_tokens=8, hit_rate=0.6, match_lag=8, seed=41)
    res = oracle_run(c)
    for debug in (0, 2):
        dev = syn.to_device(torch, c)
        ws = syn.workspace(torch, batch=3, hq=32, hkv=8, capacity=32, max_context=5008, tile_tokens=16,
                           match_tile_slots=8, semantic_pos_ahead=64, front_sink_tokens=8, device="cuda")
        ws[29].fill_(-7)
        out, out_lse, ws = syn.run_decode(torch, ext, dev, c, max_context=5008, tile_tokens=16,
                                          match_tile_slots=8, ws=ws, debug_enabled=debug)
        torch.cuda.synchronize()
        _check_against_oracle(c, dev, out, out_lse, ws, res, what=f"debug {debug}")
        stamps = ws[29].cpu().tolist()
        if debug == 0:
            assert stamps == [-7] * len(stamps)
        else:
            first = stamps[:6]
            assert all(s > 0 for s in first), first
            assert all(b >= a for a, b in zip(first, first[1:])), first
            assert stamps[6:] == [-7] * (len(stamps) - 6)


def _group_tokens(c):
    """Tokens of every group (sink + band + tail) from the oracle's spans."""
    r = oracle_run(c)
    g = r.group
    sink = np.minimum(c.front_sink_tokens, g["rect_end"])
    return (sink + (g["rect_end"] - g["rect_begin"]) + (g["tail_end"] - g["rect_end"])).reshape(-1).tolist()


@pytest.mark.parametrize("case", ["all_short", "one_long"])
def test_step_fuse_rule(case, ext, monkeypatch):
    """The default rule, which reads the previous step's counts: after a step
    whose groups were all short (or with no history: zeroed counts) the short
    groups are finished inside match_decide; after a small step with a long
    group they are left to span_attention.  Results equal the oracle either
    way; the step leaves its own counts for the next one and clears the
    long-group flag."""
    _set_fuse(monkeypatch, "auto")
    if case == "all_short":
        kv_lens, hit = [900, 300, 700, 64], 0.5
    else:  # request 0: misses over 5000 tokens (long groups); the others short
        kv_lens, hit = [5000, 300, 400, 200], 0.0
    c = syn.random_case(batch=4, hq=32, hkv=8, kv_lens=kv_lens, capacity=16, semantic_pos_ahead=32,
                        front_sink_tokens=4, hit_rate=hit, match_lag=8, seed=77)
    print(f"fuse rule: {case}", flush=True)
    res = oracle_run(c)
    for rep in range(2):  # the second step starts from the first one's cleared counts
        dev = syn.to_device(torch, c)
        ws = syn.workspace(torch, batch=4, hq=32, hkv=8, capacity=16, max_context=5008, tile_tokens=32,
                           match_tile_slots=4, semantic_pos_ahead=32, front_sink_tokens=4, device="cuda")
        if rep == 0:
            ws[16].zero_()
        else:
            ws[16].copy_(prev)
        out, out_lse, ws = syn.run_decode(torch, ext, dev, c, max_context=5008, tile_tokens=32, ws=ws)
        torch.cuda.synchronize()
        _check_against_oracle(c, dev, out, out_lse, ws, res, what=f"{case} step {rep}")
        ng = 4 * 8
        go = _np(ws[16])
        fused = go[ng:2 * ng]
        long_groups = 0 if case == "all_short" else 8  # request 0's groups
        if case == "all_short" or rep == 0:
            assert fused.tolist() == [0] * long_groups + [1] * (ng - long_groups)
        else:  # after a step with a long group and far fewer than 8M tokens
            assert fused.tolist() == [0] * ng
        assert go[2 * ng] == 0  # long-group flag cleared by merge_write
        # span_attention's workgroup 0 leaves this step's counts for the next
        assert go[2 * ng + 2:2 * ng + 4].tolist() == [ng - long_groups, long_groups]
        assert go[2 * ng + 4] == sum(-(-t // 64) for t in _group_tokens(c))
        prev = ws[16].clone()
