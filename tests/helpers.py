"""Shared test helpers: numpy restatement of the reference tests' reference
math, the oracle glue, and tolerance helpers."""

from __future__ import annotations

import os
import sys

import numpy as np

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(REPO, "mac-attention_amd")
for p in (REPO, PKG):
    if p not in sys.path:
        sys.path.insert(0, p)

from mac_attention import synthetic as syn  # noqa: E402
from oracle import oracle as orc  # noqa: E402


def ref_attention(q, k, v, start, end, sm_scale):
    """Exact attention per query head over token rows [start, end) of k/v
    (attention/tests/test_mac_persistent_decode.py:9-28), float64, without the
    reference's intermediate bf16 rounding."""
    hq, dim = q.shape
    hkv = k.shape[1]
    group = hq // hkv
    outs = np.zeros((hq, dim))
    lses = np.full(hq, -np.inf)
    if end <= start:
        return outs, lses
    for h in range(hq):
        kk = k[start:end, h // group].astype(np.float64)
        vv = v[start:end, h // group].astype(np.float64)
        logits = kk @ q[h].astype(np.float64) * sm_scale
        m = logits.max()
        w = np.exp(logits - m)
        outs[h] = (w[:, None] * vv).sum(0) / w.sum()
        lses[h] = m + np.log(w.sum())
    return outs, lses


def merge(o1, l1, o2, l2):
    """LSE merge of per-head states (attention/tests/test_mac_persistent_decode.py:31-51)."""
    o = np.array(o1, dtype=np.float64, copy=True)
    lse = np.array(l1, dtype=np.float64, copy=True)
    for h in range(o.shape[0]):
        if not np.isfinite(l1[h]):
            o[h], lse[h] = o2[h], l2[h]
            continue
        if not np.isfinite(l2[h]):
            continue
        m = max(l1[h], l2[h])
        w1, w2 = np.exp(l1[h] - m), np.exp(l2[h] - m)
        o[h] = (w1 * np.asarray(o1[h], np.float64) + w2 * np.asarray(o2[h], np.float64)) / (w1 + w2)
        lse[h] = m + np.log(w1 + w2)
    return o, lse


def rel_l2(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / (np.linalg.norm(b) + 1e-12))


def assert_close(actual, expected, tol, what=""):
    a = np.asarray(actual, np.float64)
    e = np.asarray(expected, np.float64)
    both_inf = np.isinf(a) & np.isinf(e) & (np.sign(a) == np.sign(e))
    err = np.where(both_inf, 0.0, np.abs(a - e))
    bound = tol + tol * np.abs(np.where(np.isfinite(e), e, 0.0))
    bad = ~(err <= bound)
    if bad.any():
        idx = np.argwhere(bad)[0]
        raise AssertionError(
            f"{what}: {int(bad.sum())} mismatches (rtol=atol={tol}); first at {tuple(idx)}: "
            f"got {a[tuple(idx)]!r} expected {e[tuple(idx)]!r}")


def oracle_params(case: syn.Case, **kw) -> orc.DecodeParams:
    p = orc.DecodeParams(
        semantic_pos_ahead=case.semantic_pos_ahead, front_sink_tokens=case.front_sink_tokens,
        gen_min_limit=case.gen_min_limit, lookback_right=case.lookback_right,
        candidate_mode=case.candidate_mode, threshold=case.threshold, sm_scale=case.sm_scale,
        mixed_group_fallback=int(os.environ.get("MAC_PERSISTENT_MIXED_GROUP_FALLBACK", "1") != "0"),
    )
    for key, val in kw.items():
        setattr(p, key, val)
    return p


def oracle_run(case: syn.Case, **kw) -> orc.DecodeResult:
    """Run the CPU oracle on a Case (ring caches are copied)."""
    return orc.decode(
        q_post=syn.to_bits(case.q_post), q_pre=syn.to_bits(case.q_pre),
        k_buffer=syn.to_bits(case.k), v_buffer=syn.to_bits(case.v),
        req_to_token=case.req_to_token, req_ids=case.req_ids, past_lens=case.past_lens,
        out_cache_loc=case.out_cache_loc, query_cache=syn.to_bits(case.query_cache),
        attn_cache=syn.to_bits(case.attn_cache), lse_cache=case.lse_cache,
        params=oracle_params(case, **kw), cache_ready=case.cache_ready,
        cache_epoch=case.cache_epoch, request_epoch=case.request_epoch)


def bits(x):
    return syn.from_bits(x)


def host_subset(torch, dev: dict, requests, *, semantic_pos_ahead, front_sink_tokens=0,
                threshold=0.45, gen_min_limit=0) -> syn.Case:
    """Copies the rows a subset of requests reads from device tensors into a
    self-contained CPU Case (its own compact KV pool and req_to_token), for
    the oracle.  Decode steps of different requests are independent, so the
    oracle's result for the subset equals the GPU's for those requests."""
    f = lambda t: t.float().cpu().numpy()  # noqa: E731
    req_ids = dev["req_ids"].cpu().numpy()
    past = dev["past_lens"].cpu().numpy()
    ocl = dev["out_cache_loc"].cpu().numpy()
    kvs, vvs, rows_list = [], [], []
    base = 0
    r2t_rows = []
    for n in requests:
        p = int(past[n])
        rows = dev["req_to_token"][int(req_ids[n]), :p].long()
        rows = torch.cat([rows, torch.tensor([int(ocl[n])], device=rows.device)])
        kvs.append(f(dev["k"][rows]))
        vvs.append(f(dev["v"][rows]))
        r2t_rows.append(np.arange(base, base + p + 1, dtype=np.int32))
        rows_list.append(base + p)
        base += p + 1
    cols = max(len(r) for r in r2t_rows)
    r2t = np.zeros((len(requests), cols), np.int32)
    for i, r in enumerate(r2t_rows):
        r2t[i, :len(r)] = r
    rid = [int(req_ids[n]) for n in requests]
    c = syn.Case(
        q_post=f(dev["q_post"][list(requests)]), q_pre=f(dev["q_pre"][list(requests)]),
        k=np.concatenate(kvs), v=np.concatenate(vvs), req_to_token=r2t,
        req_ids=np.arange(len(requests), dtype=np.int32),
        past_lens=past[list(requests)].astype(np.int32),
        out_cache_loc=np.array(rows_list, np.int64),
        query_cache=f(dev["query_cache"][rid]), attn_cache=f(dev["attn_cache"][rid]),
        lse_cache=dev["lse_cache"][rid].cpu().numpy(), semantic_pos_ahead=semantic_pos_ahead,
        front_sink_tokens=front_sink_tokens, threshold=threshold,
        sm_scale=1.0 / np.sqrt(128.0), gen_min_limit=gen_min_limit)
    for name in ("cache_ready", "cache_epoch", "request_epoch"):
        t = dev[name]
        if t.numel() > 0:
            setattr(c, name, t[rid].cpu().numpy().astype(np.uint8 if name == "cache_ready" else np.int64))
    return c


# ------------------------------------------------- near-threshold decisions ----
# The north star allows a decision to differ from the oracle only where the
# similarity s = 1 - sqrt(d / (2 D)) of the head's best ring entry lies
# within 1e-6 of the threshold (fp32 vs double distance rounding can flip it
# there); such heads are logged here and reported at the end of the run.
NEAR_THRESHOLD_BAND = 1e-6
NEAR_THRESHOLD_LOG: list = []


def similarity(dist, head_dim=128):
    return 1.0 - np.sqrt(np.maximum(np.asarray(dist, np.float64), 0.0) / (2.0 * head_dim))


def near_threshold_heads(res, threshold=0.45, what="", requests=None):
    """Bool [N, Hq]: heads whose best distance puts their similarity within
    NEAR_THRESHOLD_BAND of the threshold.  Each one is appended to
    NEAR_THRESHOLD_LOG (what, request, head, s, oracle decision)."""
    d = res.head["best_dist"]
    s = similarity(d)
    near = np.isfinite(d) & (np.abs(s - threshold) <= NEAR_THRESHOLD_BAND)
    for n, h in zip(*np.nonzero(near)):
        req = int(requests[n]) if requests is not None else int(n)
        NEAR_THRESHOLD_LOG.append(dict(what=what, request=req, head=int(h), similarity=float(s[n, h]),
                                       threshold=threshold, oracle_hit=int(res.head["hit"][n, h])))
    return near


# Relative L2 error of every decode output a parity test compared with the
# oracle, by test label (printed at the end of the run).
PARITY_LOG: dict = {}


def log_rel_l2(what, value):
    PARITY_LOG[what] = max(PARITY_LOG.get(what, 0.0), float(value))
