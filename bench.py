#!/usr/bin/env python3
"""Benchmark of the MAC decode step on one MI355X.

Headline workload: GQA-4 (Hq=32, Hkv=8), D=128,
batch 64, past_len 130048 (kv_len 130049) per request, ring of 32 cached
queries, semantic_pos_ahead 256, front sink 0, threshold 0.45, hit decisions
from the reference's synthetic_head exact-quota override (bench_mode=1,
mac_decode_persistent.cu:1184-1269) at hit ratio 0.8.  A step is one
graph-replayed decode step of one layer (match scan, scheduling, span
attention, merge and ring write).

Prints ONE JSON line (see the repository's bench contract): value = µs per
decode step (lower is better), plus
  roofline      -- the dominant kernel (span_attention): algorithmic bytes per
                   launch / its average duration from HIP events on its stream;
  step_roofline -- all algorithmic bytes of the step / graph-replayed step time;
  cpu_baseline  -- the FP32 PyTorch restatement of the step (oracle/torch_oracle.py)
                   on all host cores, over every request of the headline step;
  sweep         -- µs/step and achieved GB/s across hit ratios for GQA-4 and
                   GQA-8, and the same kernel forced to exact attention through
                   the readiness gate (the hit-0 path);
  reference_shape -- the same step at the reference's published benchmark
                   shape (ring 2048, past_len 126976) beside its H100 times.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

REPO = os.path.dirname(os.path.abspath(__file__))
for _p in (os.path.join(REPO, "mac-attention_amd"), REPO):
    if _p not in sys.path:
        sys.path.insert(0, _p)

METRIC = "µs per decode step & HBM GB/s vs hit ratio, GQA-4/8, B=64, 127K ctx"
HBM_PEAK_GBS = 8000.0
D = 128


def parse_args():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--batch", type=int, default=64)
    ap.add_argument("--ctx", type=int, default=130048)
    ap.add_argument("--hq", type=int, default=32)
    ap.add_argument("--hkv", type=int, default=8)
    ap.add_argument("--ring", type=int, default=32)
    ap.add_argument("--semantic-pos-ahead", type=int, default=256)
    ap.add_argument("--front-sink", type=int, default=0)
    ap.add_argument("--hit", type=float, default=0.8)
    ap.add_argument("--max-context", type=int, default=131072)
    ap.add_argument("--tile-tokens", type=int, default=32)
    ap.add_argument("--sweep", choices=["none", "short", "full"], default="short")
    ap.add_argument("--sweep-replays", type=int, default=30)
    ap.add_argument("--sweep-hits", default="0,0.25,0.5,0.75,0.8,0.9,1.0")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--phase-runs", type=int, default=5)
    ap.add_argument("--json-out", default=None)
    ap.add_argument("--ref-shape-hits", default="0,0.5,0.8,0.9,1.0",
                    help="hit ratios measured at the reference's published benchmark shape "
                         "(ring 2048, past_len 126976); empty to skip")
    ap.add_argument("--aux-only", action="store_true",
                    help="run only the prefill-rectification and decode-RoPE legs (prints their JSON)")
    ap.add_argument("--no-aux", action="store_true",
                    help="skip the prefill-rectification and decode-RoPE measurements")
    return ap.parse_args()


class Step:
    """One decode-step configuration bound to device tensors."""

    def __init__(self, torch, ext, dev, *, args, hkv, ring, hit, exact, bench_mode=1):
        from mac_attention import synthetic as syn

        self.torch, self.ext, self.dev = torch, ext, dev
        self.batch, self.hq, _ = dev["q_post"].shape
        self.hkv, self.ring, self.hit, self.exact = hkv, ring, hit, exact
        self.S, self.F = args.semantic_pos_ahead, args.front_sink
        self.max_context, self.tile = args.max_context, args.tile_tokens
        self.bench_mode = bench_mode
        self.ws = syn.workspace(torch, batch=self.batch, hq=self.hq, hkv=hkv, capacity=ring,
                                max_context=args.max_context, tile_tokens=args.tile_tokens,
                                match_tile_slots=32, semantic_pos_ahead=self.S,
                                front_sink_tokens=self.F, partial_dtype=torch.float32,
                                device=dev["q_post"].device)
        self.out = torch.empty_like(dev["q_post"])
        self.out_lse = torch.empty(self.batch, self.hq, device=dev["q_post"].device)
        if exact:
            # every request fails the readiness gate -> exact attention, no ring writes
            self.ready = torch.zeros(self.batch, dtype=torch.bool, device=dev["q_post"].device)
        else:
            self.ready = torch.empty(0, device=dev["q_post"].device)

    def args(self):
        d = self.dev
        e = self.torch.empty(0, device=d["q_post"].device)
        return (
            d["q_post"], d["q_pre"], d["k"], d["v"], d["req_to_token"], d["req_ids"],
            d["past_lens"], d["out_cache_loc"], d["query_cache"], d["attn_cache"],
            d["lse_cache"], self.out, self.out_lse, *self.ws,
            self.max_context, self.tile, 32, self.S, self.F, 0, 0, 0, 0.45, 1.0 / math.sqrt(D),
            0, self.bench_mode, self.hit, 0.0, -1.0, 0.0, 64.0, 0.0, 1, -1, 0,
            d["query_cache"], self.ready, e, e,
        )

    def launch(self):
        self.ext.mac_persistent_decode_bf16(*self.args())

    def phase_ms(self, runs):
        acc = [0.0, 0.0, 0.0]
        for _ in range(runs):
            t = self.ext.phase_times_ms(*self.args())
            acc = [a + b for a, b in zip(acc, t)]
        return [a / runs for a in acc]

    def scan_bytes(self, past):
        """Ring-scan bytes.  Rings scanned by the range-split launch (3+
        ranges of 256 slots) are probed: the first 128 B of every slot in the
        candidate window, the other 128 B only where the first half's squared
        distance does not exceed the threshold (+ the kernel's slack), unless
        MAC_PERSISTENT_MATCH_EARLY_EXIT=0; smaller rings are read in full."""
        import os

        import numpy as np

        torch = self.torch
        tiles = -(-self.ring // 32)
        splits = max(1, min(tiles, -(-self.ring // 256)))
        probe = splits >= 3 and os.environ.get("MAC_PERSISTENT_MATCH_EARLY_EXIT", "1").strip() != "0"
        slots = [int(min(self.ring, int(p))) for p in past]
        if not probe:
            return int(self.hq * sum(slots)) * 2 * D
        thr = float(np.float32(2.0 * D * (1.0 - 0.45) ** 2))
        thr_prune = thr + abs(thr) * 1e-4 + 1e-4
        evaluated = 0
        q = self.dev["q_pre"][: self.batch, :, :64].float()
        req = self.dev["req_ids"][: self.batch].tolist()
        for n in range(self.batch):
            m = slots[n]
            if m == 0:
                continue
            first = int(past[n]) - m  # candidate window [P - m, P): slots (P - m .. P - 1) % M
            idx = torch.arange(first, first + m, device=q.device) % self.ring
            ring = self.dev["query_cache"][req[n], idx, :, :64].float()
            d = ((ring - q[n].unsqueeze(0)) ** 2).sum(-1)
            evaluated += int((d <= thr_prune).sum())
        return (self.hq * sum(slots) + evaluated) * D

    def bytes(self):
        """Algorithmic HBM bytes of one step from the decisions it made."""
        import numpy as np

        ws = self.ws
        mode = ws[15].cpu().numpy()[: self.batch]
        rb = ws[9].cpu().numpy()[: self.batch].astype(np.int64)
        ne = ws[10].cpu().numpy()[: self.batch].astype(np.int64)
        kvl = ws[13].cpu().numpy()[: self.batch].astype(np.int64)
        hit = ws[3].cpu().numpy()[: self.batch]
        past = self.dev["past_lens"].cpu().numpy()[: self.batch].astype(np.int64)
        ng = self.batch * self.hkv
        # groups finished inside the match kernel (short spans): their K/V
        # rows are read there, not by the span-attention kernel
        fused = ws[16].cpu().numpy()[ng:2 * ng].reshape(self.batch, self.hkv) != 0
        sink = np.minimum(self.F, ne)
        tokens = sink + (ne - rb) + (kvl - ne)  # per group
        kv = int(tokens.sum()) * 2 * 2 * D
        r2t = int(tokens.max(axis=1).sum()) * 4
        long = ~fused
        kv_long = int(tokens[long].sum()) * 2 * 2 * D
        r2t_long = int(np.where(long, tokens, 0).max(axis=1).sum()) * 4
        ready = not self.exact
        full_rows = int(self.hq * np.minimum(self.ring, past).sum()) * 2 * D if ready else 0
        scan = self.scan_bytes(past) if ready else 0
        cached = int(hit.sum()) * (2 * D + 4)
        heads = self.batch * self.hq
        small = heads * (2 * D + 2 * D + 2 * D + 4) + (heads * (2 * D + 2 * D + 2 * D + 4) if ready else 0)
        # the span-attention kernel: K/V and token indices of the long groups,
        # partial rows of their heads written
        attn = kv_long + r2t_long + int(long.sum()) * (self.hq // self.hkv) * 2 * D
        return dict(total=kv + r2t + scan + cached + small, attention_kernel=attn, kv=kv,
                    fused_groups=int(fused.sum()), fused_kv=kv - kv_long,
                    ring_scan=scan, ring_scan_full_rows=full_rows, hit_heads=int(hit.sum()), heads=heads,
                    nonhit_groups=int((mode != 0).sum()), groups=int(mode.size))


def time_graph(torch, step: Step, warmup: int, steps: int):
    """Capture one decode step into a graph, replay `warmup` untimed, then time
    exactly `steps` replays with events (and the host clock) around them."""
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        for _ in range(3):
            step.launch()
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step.launch()
    for _ in range(warmup):
        graph.replay()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    start.record()
    for _ in range(steps):
        graph.replay()
    end.record()
    torch.cuda.synchronize()
    wall = (time.perf_counter() - t0) * 1e3 / steps
    ms = start.elapsed_time(end) / steps
    del graph
    return ms, wall


def measure(torch, step: Step, warmup, steps, phase_runs):
    ms, wall = time_graph(torch, step, warmup, steps)
    phases = step.phase_ms(phase_runs)
    b = step.bytes()
    return dict(
        hit_ratio=step.hit, gqa=step.hq // step.hkv, ring=step.ring, exact=step.exact,
        us_per_step=round(ms * 1e3, 2), wall_us_per_step=round(wall * 1e3, 2),
        phase_us=[round(p * 1e3, 2) for p in phases],
        algorithmic_bytes=b["total"], attention_kernel_bytes=b["attention_kernel"],
        ring_scan_bytes=b["ring_scan"], ring_scan_full_row_bytes=b["ring_scan_full_rows"],
        achieved_gbs=round(b["total"] / (ms * 1e-3) / 1e9, 1),
        frac_of_peak=round(b["total"] / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
        attention_kernel_gbs=round(b["attention_kernel"] / (phases[1] * 1e-3) / 1e9, 1),
        head_hit_ratio=round(b["hit_heads"] / b["heads"], 4),
        group_all_hit_fraction=round(1 - b["nonhit_groups"] / b["groups"], 4),
        nonhit_groups=b["nonhit_groups"], fused_groups=b["fused_groups"],
        fused_group_kv_bytes=b["fused_kv"],
    )


def cpu_baseline(args, hit):
    """The FP32 PyTorch restatement of the decode step (oracle/torch_oracle.py,
    pinned against the C oracle in tests/test_torch_oracle.py) timed on this
    host's CPU cores, on all ``args.batch`` requests of the headline step.
    Every request reads one request's K/V rows (same req_to_token row) so host
    memory stays at one request's rows while each request does its full work;
    the hit decisions are those of the synthetic_head override at ``hit``
    (matches planted where it puts them, found by the restatement's own
    ring scan)."""
    import numpy as np
    import torch

    from mac_attention import synthetic as syn
    from oracle import torch_oracle as tor

    cores = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    torch.set_num_threads(cores)
    g = torch.Generator().manual_seed(7)
    kv_len, hq, hkv, m, S = args.ctx + 1, args.hq, args.hkv, args.ring, args.semantic_pos_ahead
    k = tor.bf16(torch.randn(kv_len, hkv, D, generator=g))
    v = tor.bf16(torch.randn(kv_len, hkv, D, generator=g))
    r2t = torch.arange(kv_len, dtype=torch.int64)
    params = tor.StepParams(semantic_pos_ahead=S, front_sink_tokens=args.front_sink, sm_scale=1.0 / math.sqrt(D))
    hits = misses = 0
    elapsed = 0.0
    for n in range(args.batch):
        q_pre = tor.bf16(torch.randn(hq, D, generator=g))
        q_post = tor.bf16(torch.randn(hq, D, generator=g))
        ring_q = tor.bf16(torch.randn(m, hq, D, generator=g) + 10.0)
        ring_o = tor.bf16(torch.randn(m, hq, D, generator=g))
        ring_l = torch.zeros(m, hq)
        for h in range(hq):
            hit_h, slot = syn.synthetic_hit_and_slot(
                bench_mode=1, batch=args.batch, hq=hq, hkv=hkv, past_len=args.ctx, n=n, hq_i=h,
                hkv_i=h // (hq // hkv), hit_rate=hit, capacity=m, semantic_pos_ahead=S, bench_seed=1,
                match_lag_mean=64.0)
            if hit_h and slot >= 0:
                ring_q[slot, h] = q_pre[h]
        t0 = time.perf_counter()
        r = tor.decode_request(q_post=q_post, q_pre=q_pre, k=k, v=v, r2t_row=r2t, P=args.ctx, cur_loc=args.ctx,
                               ring_q=ring_q, ring_o=ring_o, ring_lse=ring_l, params=params)
        elapsed += time.perf_counter() - t0
        hits += int(r["head_hit"].sum())
        misses += int(hq - r["head_hit"].sum())
    return dict(value=round(elapsed * 1e6, 1), unit="us/step", cores=cores, kind="port", precision="fp32",
                sample=(f"all {args.batch} requests of the headline step (kv_len {kv_len}, Hq {hq}, Hkv {hkv}, "
                        f"ring {m}, synthetic_head hit {hit}: {hits} hit heads, {misses} missed) through "
                        f"oracle/torch_oracle.py in float32 on {cores} host cores; every request reads one "
                        f"request's K/V rows"),
                sample_head_hits=hits)


def cpu_baseline_configs():
    """The same FP32 torch restatement on BASELINE.json configs 0-2, on this
    host's cores: config 0 (B=1, ctx 4096, GQA-4, 16 cached queries at
    positions in [1024, 4000) of a 4096-slot ring, Bernoulli(0.5) hits, F=0)
    and config 1 (B=1, ctx 32768, GQA-4, F=64, 16 cached queries at positions
    in [ctx-3000, ctx-64), hit 0.5) are timed whole; config 2 (B=16, ctx
    65536, GQA-8, F=128, positions in [0.5 ctx, ctx-512) of a 32768-slot ring,
    hit 0.5) is timed on one request and scaled by 16 (requests are
    independent).  Hits are planted as sqrt(1-eps^2) q + eps N(0,1), eps 0.3
    (hit) / 0.9 (miss), as the GPU tests of these configs do.  A batch-1 step
    is the faster of two runs (the first also warms torch up)."""
    import numpy as np
    import torch

    from oracle import torch_oracle as tor

    cores = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    torch.set_num_threads(cores)
    out = {}
    specs = [  # name, Hkv, ctx, ring, F, (pos lo, pos hi), hit rate, requests in the config
        ("config0", 8, 4096, 4096, 0, (1024, 4000), None, 1),
        ("config1", 8, 32768, 4096, 64, (32768 - 3000, 32768 - 64), 0.5, 1),
        ("config2", 4, 65536, 32768, 128, (32768, 65536 - 512), 0.5, 16),
    ]
    for name, hkv, ctx, m, f, (lo, hi), hit, batch in specs:
        rng = np.random.default_rng(0)
        g = torch.Generator().manual_seed(0)
        hq, S = 32, 256
        kv_len = ctx + 1
        k = tor.bf16(torch.randn(kv_len, hkv, D, generator=g))
        v = tor.bf16(torch.randn(kv_len, hkv, D, generator=g))
        q_pre = tor.bf16(torch.randn(hq, D, generator=g))
        q_post = tor.bf16(torch.randn(hq, D, generator=g))
        ring_q = tor.bf16(torch.randn(m, hq, D, generator=g) + 10.0)
        ring_o = tor.bf16(torch.randn(m, hq, D, generator=g))
        ring_l = torch.full((m, hq), -math.inf)
        positions = sorted(rng.choice(np.arange(lo, hi), size=16, replace=False).tolist())
        hit_mask = rng.random(hq) < 0.5 if hit is None else np.isin(np.arange(hq), rng.choice(
            hq, size=int(round(hit * hq)), replace=False))
        for p_ in positions:
            slot = p_ % m
            ring_q[slot] = tor.bf16(torch.randn(hq, D, generator=g))
            ring_l[slot] = torch.randn(hq, generator=g)
        for h in range(hq):
            eps = 0.3 if hit_mask[h] else 0.9
            slot = int(rng.choice(positions)) % m
            ring_q[slot, h] = tor.bf16(math.sqrt(1 - eps * eps) * q_pre[h] + eps * torch.randn(D, generator=g))
        params = tor.StepParams(semantic_pos_ahead=S, front_sink_tokens=f, sm_scale=1.0 / math.sqrt(D))
        one = math.inf
        for _ in range(2 if batch == 1 else 1):  # small steps: the faster of two (the first warms torch up)
            rq, ro, rl = ring_q.clone(), ring_o.clone(), ring_l.clone()
            t0 = time.perf_counter()
            r = tor.decode_request(q_post=q_post, q_pre=q_pre, k=k, v=v, r2t_row=torch.arange(kv_len), P=ctx,
                                   cur_loc=ctx, ring_q=rq, ring_o=ro, ring_lse=rl, params=params)
            one = min(one, time.perf_counter() - t0)
        out[name] = dict(value=round(one * batch * 1e6, 1), unit="us/step", cores=cores, kind="port",
                         precision="fp32", requests_timed=1, requests_in_step=batch,
                         extrapolated=batch > 1, hit_heads=int(r["head_hit"].sum()),
                         sample=(f"B={batch} Hq={hq} Hkv={hkv} ctx={ctx} ring={m} F={f}: "
                                 + ("the whole step" if batch == 1 else
                                    f"one request timed, x{batch} (requests are independent)")))
    return out


def stream_read_peak(torch):
    """The rate a plain streaming read of 8 GiB reaches on this GPU
    (mac_bench_stream_read: non-temporal 16-byte loads, eight in flight per
    lane), the best of grids of 0.75 and 1 workgroups per CU (larger grids
    measured slower), and that of a plain 2 GiB device copy (4 GiB read and
    written), as context for the kernels' fractions of the 8 TB/s
    nameplate."""
    import ctypes

    from mac_attention.integrations.sglang import bridge

    lib = bridge.load_bench_library()
    nbytes = 8 << 30
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    src = torch.empty(nbytes // 4, dtype=torch.int32, device="cuda").fill_(1)
    sink = torch.empty(cus, dtype=torch.int32, device="cuda")
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    best = None
    for grid in (cus * 3 // 4, cus):
        def run():
            rc = lib.mac_bench_stream_read(ctypes.c_void_p(src.data_ptr()), ctypes.c_int64(nbytes),
                                           ctypes.c_void_p(sink.data_ptr()), ctypes.c_int32(grid), stream)
            if rc != 0:
                raise RuntimeError(lib.mac_bench_last_error().decode())

        us = _time_us(torch, run, 10)
        if best is None or us < best[0]:
            best = (us, grid)
    # a plain device-to-device copy (torch's copy kernel), bytes read +
    # written: the level for kernels that write as much as they read
    dst = torch.empty(nbytes // 16, dtype=torch.int32, device="cuda")  # 2 GiB
    half = src[: nbytes // 16]
    copy_us = _time_us(torch, lambda: dst.copy_(half), 10)
    del src, sink, dst, half
    torch.cuda.empty_cache()
    gbs = nbytes / best[0] / 1e3
    copy_gbs = (nbytes // 2) / copy_us / 1e3
    return dict(bytes=nbytes, workgroups=best[1], us=round(best[0], 1), gbs=round(gbs, 1),
                frac_of_peak=round(gbs / HBM_PEAK_GBS, 4),
                copy=dict(bytes_read_and_written=nbytes // 2, us=round(copy_us, 1), gbs=round(copy_gbs, 1),
                          frac_of_peak=round(copy_gbs / HBM_PEAK_GBS, 4)))


def aux_cpu_baselines():
    """The CPU oracle (one thread) on the aux legs' workloads.  The fused
    rectification and the ring write only touch the last M = 32 rows of each
    chunk (and, for the rectification, the S - 1 keys before them), so a
    sample of all 64 requests with 288-row chunks does exactly the per-request
    work of the 8192-row chunks; the RoPE leg runs at full size."""
    import numpy as np

    from oracle import oracle as orc

    rng = np.random.default_rng(3)
    # random bf16 bits (the top half of random float32s: timing data only)
    bf = lambda *shape: (rng.standard_normal(shape, dtype=np.float32).view(np.uint32) >> 16).astype(np.uint16)  # noqa: E731
    B, chunk, hq, hkv, S, M = 64, 288, 32, 4, 256, 32
    rows = B * chunk
    qo = np.arange(0, rows + 1, chunk, dtype=np.int32)
    idx = rng.permutation(rows).astype(np.int32)
    q_post, src_q, o_full = bf(rows, hq, D), bf(rows, hq, D), bf(rows, hq, D)
    lse_full = rng.standard_normal((rows, hq), dtype=np.float32) + 8.0
    k, v = bf(rows, hkv, D), bf(rows, hkv, D)
    qc = np.zeros((B + 1, M, hq, D), np.uint16)
    ac, lc = np.zeros_like(qc), np.zeros((B + 1, M, hq), np.float32)
    rl = np.zeros(B + 1, np.int32)
    req = np.arange(B, dtype=np.int32)
    t0 = time.perf_counter()
    orc.rectify_update_cache(q_post, src_q, o_full, lse_full, k, v, qo, qo, idx, qc, ac, lc, rl, req,
                             semantic_pos_ahead=S, front_sink_tokens=0, sink_mode=0,
                             sm_scale=1.0 / math.sqrt(D))
    rect_s = time.perf_counter() - t0
    out = {"prefill_rectify": dict(
        value=round(rect_s * 1e6, 1), unit="us", cores=1, kind="port",
        sample=f"all {B} requests with {chunk}-row chunks (the kept {M} rows and their {S}-key windows "
               f"are the whole work of an 8192-row chunk), single-threaded C oracle")}
    rl2 = np.zeros(B, np.int32)
    src_l = rng.standard_normal((rows, hq), dtype=np.float32)
    lens = np.full(B, chunk, np.int32)
    t0 = time.perf_counter()
    orc.prefill_update_cache(qc, ac, lc, rl2, req, src_q, o_full, src_l, qo, lens, M, hq, D)
    upd_s = time.perf_counter() - t0
    out["prefill_update_cache"] = dict(
        value=round(upd_s * 1e6, 1), unit="us", cores=1, kind="port",
        sample=f"all {B} batch rows with {chunk}-row chunks (the last {M} rows are copied either way), "
               f"single-threaded C oracle")
    n, hq4, hkv4, pool = 64, 32, 8, 1 << 16
    qkv = bf(n, (hq4 + 2 * hkv4) * D)
    q4, k4, v4 = qkv[:, :hq4 * D], qkv[:, hq4 * D:(hq4 + hkv4) * D], qkv[:, (hq4 + hkv4) * D:]
    q_pre = np.zeros((n, hq4, D), np.uint16)
    kb, vb = np.zeros((pool, hkv4, D), np.uint16), np.zeros((pool, hkv4, D), np.uint16)
    inv = 1.0 / (10000.0 ** (np.arange(0, D, 2, dtype=np.float64) / D))
    ang = np.arange(131072, dtype=np.float64)[:, None] * inv[None, :]
    cs = np.concatenate([np.cos(ang), np.sin(ang)], axis=1).astype(np.float32)
    pos = rng.integers(0, 131072, n).astype(np.int64)
    locs = rng.permutation(pool)[:n].astype(np.int64)
    t0 = time.perf_counter()
    orc.rope_preserve(q4, k4, v4, q_pre, kb, vb, cs, pos, locs, head_dim=D, is_neox=True)
    rope_s = time.perf_counter() - t0
    out["decode_rope"] = dict(value=round(rope_s * 1e6, 1), unit="us", cores=1, kind="port",
                              sample=f"full size ({n} tokens), single-threaded C oracle")
    return out


# The reference's published MAC decode-step times on H100 80GB (CUDA-graph
# replay, B=64, past_len 126976, ring 2048, S=256, F=0, synthetic_head):
# results/cuda_graph_hit_curves/gqa4.csv:156-169 and gqa8.csv:156-169.
REF_H100_MS = {
    4: {0.0: 19.107, 0.5: 13.806, 0.8: 6.261, 0.9: 3.556, 1.0: 0.969},
    8: {0.0: 13.228, 0.5: 8.557, 0.8: 3.694, 0.9: 2.374, 1.0: 0.708},
}
REF_SHAPE_CTX, REF_SHAPE_RING = 126976, 2048


PMC_SUMMARY = os.path.join(REPO, "profiles", "span_attention_config3_gqa4_hit0.8_pmc.txt")


def _time_us(torch, fn, reps):
    """Average µs of fn() over reps launches, HIP events on the current stream."""
    for _ in range(3):
        fn()
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for _ in range(reps):
        fn()
    b.record()
    torch.cuda.synchronize()
    return a.elapsed_time(b) * 1e3 / reps


def _time_graph_us(torch, fn, per_graph=20, replays=5):
    """GPU µs per fn() call: per_graph calls captured in one graph, replayed
    `replays` times between HIP events (how serving runs these ops, under
    graph capture; an eager Python call of a few-µs kernel measures the host's
    call overhead instead)."""
    for _ in range(3):
        fn()
    torch.cuda.synchronize()
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        for _ in range(per_graph):
            fn()
    graph.replay()
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for _ in range(replays):
        graph.replay()
    b.record()
    torch.cuda.synchronize()
    del graph
    return a.elapsed_time(b) * 1e3 / (replays * per_graph)


def measure_aux(torch):
    """The rows beside the decode step, at BASELINE config 4's prefill shape:
    64 requests, one 8192-token chunk each, GQA-8, S = 256, ring 32.
      prefill_rectify -- the fused op (kept rows only) against the reference's
                         three calls on the GPU (window attention of every row,
                         downdate of every row, mac_prefill_update_cache);
      prefill_update_cache -- the ring write of the last M rows of every chunk;
      decode_rope     -- fused RoPE + q preserve + KV write for a 64-token decode
                         batch (GQA-4, rotary_dim 128, NeoX)."""
    from mac_attention.integrations.sglang import bridge

    rect = bridge.load_mac_prefill_rectify_extension()
    merge = bridge.load_mac_merge_downdate_cache_extension()
    cache = bridge.load_mac_prefill_update_cache_extension()
    rope = bridge.load_mac_decode_rope_preserve_extension()
    B, chunk, hq, hkv, S, M = 64, 8192, 32, 4, 256, 32
    rows = B * chunk
    bf = torch.bfloat16
    dev = "cuda"
    g = torch.Generator(device=dev)
    g.manual_seed(0)
    k = torch.randn(rows, hkv, D, device=dev, dtype=bf, generator=g)
    v = torch.randn(rows, hkv, D, device=dev, dtype=bf, generator=g)
    q = torch.randn(rows, hq, D, device=dev, dtype=bf, generator=g)
    src_q = torch.randn(rows, hq, D, device=dev, dtype=bf, generator=g)
    o_full = torch.randn(rows, hq, D, device=dev, dtype=bf, generator=g)
    lse_full = torch.randn(rows, hq, device=dev, generator=g) + 8.0
    qo = torch.arange(0, rows + 1, chunk, device=dev, dtype=torch.int32)
    idx = torch.randperm(rows, device=dev, generator=g).to(torch.int32)
    qc = torch.zeros(B, M, hq, D, device=dev, dtype=bf)
    ac = torch.zeros_like(qc)
    lc = torch.zeros(B, M, hq, device=dev)
    req = torch.arange(B, device=dev, dtype=torch.int32)
    rl = torch.zeros(B + 1, device=dev, dtype=torch.int32)  # indexed by request (R = B + 1 rows)
    qc2, ac2, lc2 = (torch.zeros(B + 1, M, hq, D, device=dev, dtype=bf), torch.zeros(B + 1, M, hq, D, device=dev, dtype=bf),
                     torch.zeros(B + 1, M, hq, device=dev))
    scale = 1.0 / math.sqrt(D)

    def fused():
        rect.mac_prefill_rectify_update_cache(q, src_q, o_full, lse_full, k, v, qo, qo, idx, qc2, ac2, lc2,
                                              rl, req, S, 0, scale)

    wo = torch.empty_like(q)
    wl = torch.empty(rows, hq, device=dev)
    lens = torch.full((B,), chunk, device=dev, dtype=torch.int32)
    empty = torch.empty(0, device=dev, dtype=bf)

    def composed():
        rect.window_attention_return_lse(q, k, v, qo, qo, idx, S - 1, scale, out=wo, out_lse=wl)
        merge.mac_update_then_downdate_bf16_inplace(o_full, lse_full, wo, wl)
        cache.mac_prefill_update_cache(qc, ac, lc, rl[:B], req, src_q, wo, wl, qo, lens, M, hq, D, empty)

    fused_us = _time_graph_us(torch, fused)
    fused_eager_us = _time_us(torch, fused, 20)
    comp_us = _time_us(torch, composed, 5)
    # the window attention of every row on its own (the dominant call of the
    # three): row i of a chunk attends keys max(0, i - S + 1) .. i.  Per launch
    # it reads q (bf16) and every K/V row once and writes out (bf16) and lse
    # (f32): 9.7 GB here against 2.2 TFLOP, so HBM, not MFMA, bounds it
    # (4 D flop per (row, head, key) over 2 B per element is below the
    # ridge of 2.5 PFLOP/s / 8 TB/s).
    win_us = _time_us(torch, lambda: rect.window_attention_return_lse(q, k, v, qo, qo, idx, S - 1, scale, out=wo,
                                                                      out_lse=wl), 5)
    keys_per_chunk = sum(min(i + 1, S) for i in range(chunk))
    win_flop = 4 * D * hq * B * keys_per_chunk
    win_bytes = rows * hq * (2 * D * 2 + 4) + rows * hkv * 2 * D * 2 + rows * 4
    hbm_s, mfma_s = win_bytes / 8e12, win_flop / 2.5e15
    # mac_prefill_update_cache alone (the last M rows of every chunk into the
    # ring): q and attention rows (2 * Hq * D bf16) + lse read and written per row
    upd_us = _time_graph_us(torch, lambda: cache.mac_prefill_update_cache(qc, ac, lc, rl[:B], req, src_q, wo, wl, qo, lens,
                                                                    M, hq, D, empty))
    upd_bytes = 2 * B * M * hq * (2 * 2 * D + 4)
    # algorithmic bytes of the fused op: per (request, kv head) the K/V rows
    # of the window of the kept rows (M + S - 1 tokens), per kept row and
    # head q_post, src_q, o_full (256 B each) + lse_full read, ring q and o
    # (256 B each) + lse written
    kept = B * M
    fused_bytes = B * hkv * (M + S - 1) * 2 * D * 2 + kept * hq * (5 * 2 * D + 8)
    out = {"prefill_rectify": {
        "workload": f"B={B} requests x {chunk}-token chunk, GQA-8 (Hq={hq}, Hkv={hkv}), S={S}, ring={M}",
        "fused_us": round(fused_us, 2), "reference_three_calls_us": round(comp_us, 2),
        "speedup": round(comp_us / fused_us, 1), "fused_algorithmic_bytes": fused_bytes,
        "fused_gbs": round(fused_bytes / fused_us / 1e3, 1),
        "fused_eager_call_us": round(fused_eager_us, 2),
        "timing": "fused_us: graph-replayed calls (as under serving's graph capture); fused_eager_call_us: "
                  "back-to-back eager calls from Python"},
        "prefill_update_cache": {
            "workload": f"B={B} batch rows x {chunk} source rows, ring={M}, Hq={hq}",
            "us": round(upd_us, 2), "algorithmic_bytes": upd_bytes,
            "gbs": round(upd_bytes / upd_us / 1e3, 1)},
        "window_attention": {
            "workload": f"every row of B={B} x {chunk}-token chunks, GQA-8 (Hq={hq}, Hkv={hkv}), window {S}",
            "us": round(win_us, 1), "flop": win_flop, "algorithmic_bytes": win_bytes,
            "bound": "hbm" if hbm_s >= mfma_s else "mfma",
            "tflops": round(win_flop / win_us / 1e6, 1), "frac_bf16_peak": round(win_flop / win_us / 2.5e9, 4),
            "gbs": round(win_bytes / win_us / 1e3, 1), "frac_hbm_peak": round(win_bytes / win_us / 8e6, 4),
            "frac_roofline": round(max(hbm_s, mfma_s) / (win_us * 1e-6), 4)}}
    del k, v, q, src_q, o_full, wo
    torch.cuda.empty_cache()

    n, hq4, hkv4, pool = 64, 32, 8, 1 << 16
    qkv = torch.randn(n, (hq4 + 2 * hkv4) * D, device=dev, dtype=bf, generator=g)
    qv, kv_, vv = qkv[:, :hq4 * D], qkv[:, hq4 * D:(hq4 + hkv4) * D], qkv[:, (hq4 + hkv4) * D:]
    q_pre = torch.empty(n, hq4, D, device=dev, dtype=bf)
    kb = torch.empty(pool, hkv4, D, device=dev, dtype=bf)
    vb = torch.empty_like(kb)
    inv = 1.0 / (10000.0 ** (torch.arange(0, D, 2, device=dev, dtype=torch.float32) / D))
    ang = torch.arange(131072, device=dev, dtype=torch.float32)[:, None] * inv[None, :]
    cs = torch.cat([ang.cos(), ang.sin()], dim=1).contiguous()
    pos = torch.randint(0, 131072, (n,), device=dev, generator=g)
    loc = torch.randperm(pool, device=dev, generator=g)[:n].contiguous()
    rope_call = lambda: rope.mac_decode_rope_preserve_q_bf16(qv, kv_, vv, q_pre, kb, vb, cs, pos, loc, D, True)
    rope_us = _time_graph_us(torch, rope_call)
    rope_eager_us = _time_us(torch, rope_call, 50)
    rope_bytes = n * ((hq4 + 2 * hkv4) * D * 2 + (2 * hq4 + 3 * hkv4) * D * 2)
    out["decode_rope"] = {"workload": f"{n} decode tokens, Hq={hq4}, Hkv={hkv4}, rotary_dim {D}, NeoX",
                          "us": round(rope_us, 2), "algorithmic_bytes": rope_bytes,
                          "eager_call_us": round(rope_eager_us, 2),
                          "timing": "us: graph-replayed calls; eager_call_us: back-to-back eager calls from "
                                    "Python (host-bound for this few-µs kernel)"}
    return out


def pmc_traffic(args):
    """HBM bytes per span_attention launch from the committed rocprofv3
    FETCH_SIZE/WRITE_SIZE summary (scaled by the copy-kernel calibration it
    records).  Only valid for the workload that summary profiled."""
    default = (args.hkv == 8 and args.batch == 64 and args.ctx == 130048 and args.ring == 32
               and abs(args.hit - 0.8) < 1e-9 and args.front_sink == 0)
    if not default or not os.path.exists(PMC_SUMMARY):
        return None, None
    with open(PMC_SUMMARY) as f:
        for line in f:
            if line.startswith("traffic_bytes_per_launch="):
                return int(line.split("=", 1)[1]), os.path.relpath(PMC_SUMMARY, REPO)
    return None, None


def main():
    args = parse_args()
    if args.gpus != 1:
        print(json.dumps({"error": "this build measures one GPU; every GPU box here has one, "
                                   "so --gpus must be 1 (multi-GPU sharding is design-only)"}))
        sys.exit(2)
    import torch

    if args.aux_only:
        assert torch.cuda.is_available(), "bench.py needs a HIP device"
        print(json.dumps({"aux": measure_aux(torch)}), flush=True)
        return

    from mac_attention import synthetic as syn
    from mac_attention.integrations.sglang.bridge import load_mac_persistent_decode_extension

    assert torch.cuda.is_available(), "bench.py needs a HIP device"
    ext = load_mac_persistent_decode_extension(False)
    log = lambda *a: print(*a, file=sys.stderr, flush=True)  # noqa: E731

    sweep = []
    headline = None
    gqa_list = [args.hkv] if args.sweep == "none" else [args.hkv, args.hq // 8]
    hits = [float(x) for x in args.sweep_hits.split(",") if x.strip()]
    for hkv in gqa_list:
        t0 = time.perf_counter()
        dev = syn.device_case(torch, batch=args.batch, hq=args.hq, hkv=hkv, ctx=args.ctx,
                              capacity=args.ring, seed=0)
        torch.cuda.synchronize()
        log(f"[bench] GQA-{args.hq // hkv}: inputs ready in {time.perf_counter() - t0:.1f}s")
        syn.plant_synthetic_hits(torch, dev, hit_rate=args.hit, bench_mode=1,
                                 semantic_pos_ahead=args.semantic_pos_ahead)
        if hkv == args.hkv:
            step = Step(torch, ext, dev, args=args, hkv=hkv, ring=args.ring, hit=args.hit,
                        exact=False)
            headline = measure(torch, step, args.warmup, args.steps, args.phase_runs)
            log(f"[bench] headline {headline}")
            del step
        if args.sweep != "none":
            for exact in (True, False):
                for h in ([0.0] if exact else hits):
                    step = Step(torch, ext, dev, args=args, hkv=hkv, ring=args.ring, hit=h,
                                exact=exact)
                    r = measure(torch, step, 15, args.sweep_replays, 3)
                    sweep.append(r)
                    log(f"[bench] sweep {r}")
                    del step
        del dev
        torch.cuda.empty_cache()

    # the reference's own benchmark shape, next to its published H100 times
    ref_shape = []
    ref_hits = [float(x) for x in args.ref_shape_hits.split(",") if x.strip()]
    if ref_hits:
        rargs = argparse.Namespace(**vars(args))
        rargs.ctx, rargs.ring = REF_SHAPE_CTX, REF_SHAPE_RING
        for hkv in (args.hkv, args.hq // 8):
            gqa = args.hq // hkv
            # hit decisions come from the synthetic_head override, so one input
            # set serves every hit ratio (planted copies are cosmetic there)
            dev = syn.device_case(torch, batch=args.batch, hq=args.hq, hkv=hkv, ctx=REF_SHAPE_CTX,
                                  capacity=REF_SHAPE_RING, seed=0)
            syn.plant_synthetic_hits(torch, dev, hit_rate=args.hit, bench_mode=1,
                                     semantic_pos_ahead=args.semantic_pos_ahead)
            for h in ref_hits:
                step = Step(torch, ext, dev, args=rargs, hkv=hkv, ring=REF_SHAPE_RING, hit=h, exact=False)
                r = measure(torch, step, 15, args.sweep_replays, 3)
                ref_ms = REF_H100_MS.get(gqa, {}).get(h)
                r["ctx"] = REF_SHAPE_CTX
                r["reference_h100_us"] = None if ref_ms is None else round(ref_ms * 1e3, 1)
                r["speedup_vs_reference_h100"] = (None if ref_ms is None
                                                  else round(ref_ms * 1e3 / r["us_per_step"], 2))
                ref_shape.append(r)
                log(f"[bench] reference shape {r}")
                del step
            del dev
            torch.cuda.empty_cache()

    stream_peak = stream_read_peak(torch)
    log(f"[bench] streaming read {stream_peak}")

    aux = None
    if not args.no_aux:
        aux = measure_aux(torch)
        log(f"[bench] aux {aux}")
        torch.cuda.empty_cache()

    cpu = None
    if not args.no_cpu_baseline:
        log("[bench] timing the CPU oracle sample")
        cpu = cpu_baseline(args, args.hit)
        cpu["per_config"] = cpu_baseline_configs()
        cpu["per_config"]["config3"] = {k: cpu[k] for k in ("value", "unit", "cores", "kind", "sample")}
        log(f"[bench] cpu {cpu}")
        if aux is not None:
            for name, base in aux_cpu_baselines().items():
                aux[name]["cpu_baseline"] = base
            log(f"[bench] aux with CPU baselines {aux}")

    ms = headline["us_per_step"] / 1e3
    attn_us = headline["phase_us"][1]
    traffic, traffic_src = pmc_traffic(args)
    roof = dict(bound="hbm", achieved=headline["attention_kernel_gbs"], peak=HBM_PEAK_GBS,
                unit="GB/s", frac=round(headline["attention_kernel_gbs"] / HBM_PEAK_GBS, 4),
                traffic=traffic, traffic_source=traffic_src,
                traffic_note=("HBM bytes per launch from a separate rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE run "
                              "of this workload (the committed summary named in traffic_source), not this run"
                              if traffic is not None else None),
                kernel="span_attention", kernel_us=attn_us,
                bytes_per_launch=headline["attention_kernel_bytes"])
    line = {
        "metric": METRIC,
        "value": headline["us_per_step"],
        "unit": "us/step",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (N(0,1) bf16 K/V/q, randn+10 ring, synthetic_head hit override)",
        "config": {
            "workload": (f"MAC decode step, GQA-{args.hq // args.hkv}, B={args.batch}, "
                         f"ctx={args.ctx}, ring={args.ring}, hit={args.hit}"),
            "batch": args.batch, "ctx": args.ctx, "hq": args.hq, "hkv": args.hkv, "head_dim": D,
            "ring": args.ring, "semantic_pos_ahead": args.semantic_pos_ahead,
            "front_sink": args.front_sink, "hit_ratio": args.hit, "bench_mode": "synthetic_head",
            "graph": "hipGraph replay",
        },
        "step_roofline": dict(achieved=headline["achieved_gbs"], peak=HBM_PEAK_GBS, unit="GB/s",
                              frac=headline["frac_of_peak"],
                              bytes_per_step=headline["algorithmic_bytes"]),
        "roofline": roof,
        "cpu_baseline": cpu,
        "headline": headline,
        "sweep": sweep,
        "reference_shape": ref_shape,
        "aux": aux,
        "stream_read": stream_peak,
    }
    text = json.dumps(line)
    if args.json_out:
        with open(args.json_out, "w") as f:
            f.write(text + "\n")
    print(text, flush=True)


if __name__ == "__main__":
    main()
