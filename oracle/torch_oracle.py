"""FP32 PyTorch restatement of one MAC decode step, on the host CPU.

TEST INFRASTRUCTURE ONLY: used by tests/ (pinned against the C oracle,
``mac_oracle.c``) and by the ``cpu_baseline`` leg of ``bench.py``, which
times it on the GPU box's host cores.  The product path never imports it.

The algorithm is the reference's decode step restated with torch tensor
operations in float32, one request at a time (every request's step is
independent):
  * ring scan: squared L2 distance of each head's pre-RoPE query to every
    ring slot whose logical position is a candidate, best = smallest, ties
    to the smaller position (mac_decode_persistent.cu:942-1099, :809-811);
  * decisions: threshold distance 2 D (1 - thr)^2, front-sink demotion,
    reuse validity, group mode and spans (:1147-1402, :5342);
  * attention over the group's sink, band and tail tokens in fp32 with
    per-head band starts, LSE merges with the cached entry, the ring row at
    past_len % M (ready requests) and the output (:4280-4685, :866-890);
  * the readiness gate (:221-230).
Inputs are float32 tensors holding bf16 values; outputs written to bf16
places (ring o, out) are rounded to bf16 like the reference stores them.
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import torch


@dataclass
class StepParams:
    semantic_pos_ahead: int = 256
    front_sink_tokens: int = 0
    threshold: float = 0.45
    sm_scale: float = 1.0 / math.sqrt(128.0)
    gen_min_limit: int = 0
    candidate_mode: int = 0
    lookback_right: int = 0
    mixed_group_fallback: int = 1


def _ring_positions(P: int, M: int) -> torch.Tensor:
    """Logical position of every ring slot (mac_decode_persistent.cu:798-807)."""
    slots = torch.arange(M)
    if P < M:
        return slots
    return P - M + torch.remainder(slots - P % M, M)


def _lse_state(scores: torch.Tensor, v: torch.Tensor):
    """(o, lse) of softmax attention over the unmasked scores (masked = -inf);
    an empty row gives (0, -inf).  scores [H, T], v [T, D]."""
    m = scores.max(dim=1, keepdim=True).values
    finite = torch.isfinite(m)
    w = torch.exp(scores - torch.where(finite, m, torch.zeros_like(m)))
    w = torch.where(torch.isfinite(scores), w, torch.zeros_like(w))
    s = w.sum(dim=1, keepdim=True)
    o = (w @ v) / torch.where(s > 0, s, torch.ones_like(s))
    lse = torch.where(s[:, 0] > 0, m[:, 0] + torch.log(torch.where(s[:, 0] > 0, s[:, 0], torch.ones_like(s[:, 0]))),
                      torch.full_like(s[:, 0], -math.inf))
    return o, lse


def _merge(o1, l1, o2, l2):
    """LSE merge of per-head states (mac_decode_persistent.cu:866-890): an
    operand with non-finite lse is empty."""
    f1, f2 = torch.isfinite(l1), torch.isfinite(l2)
    m = torch.where(f1 & f2, torch.maximum(l1, l2), torch.where(f1, l1, l2))
    m0 = torch.where(torch.isfinite(m), m, torch.zeros_like(m))
    w1 = torch.where(f1, torch.exp(l1 - m0), torch.zeros_like(l1))
    w2 = torch.where(f2, torch.exp(l2 - m0), torch.zeros_like(l2))
    tot = w1 + w2
    o = (w1[:, None] * o1 + w2[:, None] * o2) / torch.where(tot > 0, tot, torch.ones_like(tot))[:, None]
    lse = torch.where(tot > 0, m0 + torch.log(torch.where(tot > 0, tot, torch.ones_like(tot))),
                      torch.full_like(tot, -math.inf))
    return o, lse


def bf16(x: torch.Tensor) -> torch.Tensor:
    return x.to(torch.bfloat16).to(torch.float32)


def decode_request(*, q_post: torch.Tensor, q_pre: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                   r2t_row: torch.Tensor, P: int, cur_loc: int, ring_q: torch.Tensor, ring_o: torch.Tensor,
                   ring_lse: torch.Tensor, params: StepParams, ready: bool = True) -> dict:
    """One request's decode step.  q_post/q_pre [Hq, D]; k/v [pool, Hkv, D]
    (float32, or bf16, whose gathered rows are widened to float32);
    r2t_row [>= P] pool rows; ring_q/ring_o [M, Hq, D], ring_lse [M, Hq] (the
    request's ring, updated in place at slot P % M when ready).  Returns the
    head decisions, group modes and the output (o [Hq, D], lse [Hq])."""
    Hq, D = q_pre.shape
    Hkv = k.shape[1]
    G = Hq // Hkv
    M = ring_q.shape[0]
    S, F = params.semantic_pos_ahead, max(params.front_sink_tokens, 0)
    thr_dist = float(torch.tensor(2.0 * D * (1.0 - params.threshold) ** 2, dtype=torch.float32))
    cand_begin = max(0, P - M)
    cand_end = P if params.candidate_mode == 0 else max(cand_begin, P - params.lookback_right)
    eligible = ready and P >= params.gen_min_limit and cand_end > cand_begin

    # ---- ring scan (fp32 squared distance) ----
    pos = _ring_positions(P, M)
    d = ((q_pre[None] - ring_q) ** 2).sum(dim=-1)  # [M, Hq]
    in_win = (pos >= cand_begin) & (pos < cand_end)
    d = torch.where(in_win[:, None], d, torch.full_like(d, math.inf))
    order = torch.argsort(pos)  # ties go to the smaller logical position
    best_i = torch.argmin(d[order], dim=0)
    best_slot = order[best_i]
    best_d = d[best_slot, torch.arange(Hq)]
    hit = (best_d < thr_dist) & torch.isfinite(best_d) & eligible

    # ---- per-head spans and group modes ----
    new_end = max(P + 1 - S, 0)
    fs_begin = min(F, new_end)
    mpos = pos[best_slot]
    prefix_end = torch.clamp(mpos + 1 - S, min=0)
    hit = hit & ~((F > 0) & (prefix_end < F))  # front-sink demotion
    entry_lse = ring_lse[best_slot, torch.arange(Hq)]
    clen = new_end - prefix_end
    valid = hit & torch.isfinite(entry_lse) & (clen >= 0) & (clen <= M)
    vg = valid.view(Hkv, G)
    n_valid = vg.sum(dim=1)
    mode = torch.where(n_valid == G, 0, torch.where((n_valid > 0) & (params.mixed_group_fallback != 0), 2, 1))
    keep = (mode[:, None] == 0) | ((mode[:, None] == 2) & vg)
    keep = keep.view(Hq)
    rect_start = torch.where(keep, prefix_end, torch.full_like(prefix_end, fs_begin))
    head_hit = keep & hit
    band_begin = torch.where(mode == 0, rect_start.view(Hkv, G).min(dim=1).values, torch.full_like(mode, fs_begin))
    band_begin = torch.clamp(band_begin, 0, new_end)

    # ---- attention per group: ring state (band) and rest (sink + tail) ----
    out = torch.zeros(Hq, D)
    out_lse = torch.full((Hq,), -math.inf)
    ring_state_o = torch.zeros(Hq, D)
    ring_state_l = torch.full((Hq,), -math.inf)
    sink_end = fs_begin
    for g in range(Hkv):
        rb = int(band_begin[g])
        toks = torch.cat([torch.arange(0, sink_end), torch.arange(rb, new_end), torch.arange(new_end, P + 1)])
        is_band = (toks >= rb) & (toks < new_end)
        phys = torch.where(toks == P, torch.tensor(cur_loc), r2t_row[torch.clamp(toks, max=max(P - 1, 0))].long())
        kg, vg_ = k[phys, g].float(), v[phys, g].float()  # [T, D] (bf16 pools: only the rows used are widened)
        heads = slice(g * G, (g + 1) * G)
        sc = (q_post[heads] @ kg.T) * params.sm_scale  # [G, T]
        band_ok = is_band[None, :] & (toks[None, :] >= rect_start[heads, None])
        neg = torch.full_like(sc, -math.inf)
        o_r, l_r = _lse_state(torch.where(band_ok, sc, neg), vg_)
        o_s, l_s = _lse_state(torch.where(~is_band[None, :], sc, neg), vg_)
        # cached entry of kept hit heads (mac_decode_persistent.cu:4343-4358)
        ent = head_hit[heads]
        e_o = ring_o[best_slot[heads], torch.arange(g * G, (g + 1) * G)]
        e_l = torch.where(ent, entry_lse[heads], torch.full_like(entry_lse[heads], -math.inf))
        o_r, l_r = _merge(o_r, l_r, e_o, e_l)
        ring_state_o[heads], ring_state_l[heads] = o_r, l_r
        o, l = _merge(o_r, l_r, o_s, l_s)
        out[heads], out_lse[heads] = o, l

    if ready and P >= 0:  # ring row at past_len % M
        dest = P % M
        ring_q[dest] = q_pre
        fin = torch.isfinite(ring_state_l)
        ring_o[dest] = torch.where(fin[:, None], bf16(ring_state_o), torch.zeros_like(ring_state_o))
        ring_lse[dest] = torch.where(fin, ring_state_l, torch.full_like(ring_state_l, -math.inf))
    out = torch.where(torch.isfinite(out_lse)[:, None], bf16(out), torch.zeros_like(out))
    return dict(out=out, out_lse=out_lse, head_hit=head_hit.to(torch.int32),
                head_match_pos=torch.where(head_hit, mpos, torch.full_like(mpos, -1)).to(torch.int32),
                group_mode=mode.to(torch.int32), best_dist=best_d)
