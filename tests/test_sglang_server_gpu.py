"""A served model's MAC path end to end through the installed hooks only.

Stand-in SGLang modules (tests/sglang_standin.py) get the real hook set
(``hook_installer.install_hooks``); a LlamaAttention layer then runs a
prefill chunk and a decode step exactly as SGLang would call it.  Nothing
calls the MAC functions directly: the scheduler hook marks the ring rows, the
attention hook keeps the pre-RoPE queries and hands the layer state to the
backend, the forward_extend hook rectifies the marked rows into the rings and
marks the requests ready, and on decode the attention hook's fused RoPE and
the forward_decode hook's MAC step produce the output.  Request 0's heads
0-3 repeat a query of their prompt, so the decode step must hit; decisions,
output and the written ring rows are checked against the CPU oracle run on
the ring state the prefill left.  Three attention backends: FlashInfer,
whose paged prefill attention with its lse comes from this build's
window-attention kernel with no window; and the backends SGLang runs on ROCm
(TritonAttnBackend, AiterAttnBackend), whose own prefill attention returns no
lse (here a float32 torch attention), so the extend hook computes the kept
rows' full prefill state itself.
"""

import math
import types

import numpy as np
import pytest

import sglang_standin
from helpers import bits, host_subset, oracle_run, rel_l2

torch = pytest.importorskip("torch")

pytestmark = pytest.mark.gpu

HQ, HKV, D, M, S = 8, 2, 128, 16, 32


def _rope_neox(positions, x, heads, cos_sin):
    """NeoX rotary embedding on [N, heads * D] rows (float32 math, bf16 out)."""
    v = x.view(-1, heads, D).float()
    c = cos_sin[positions.long(), : D // 2].unsqueeze(1)
    s = cos_sin[positions.long(), D // 2:].unsqueeze(1)
    x0, x1 = v[..., : D // 2], v[..., D // 2:]
    return torch.cat([x0 * c - x1 * s, x1 * c + x0 * s], dim=-1).to(x.dtype).view(x.shape[0], heads * D)


def _torch_prefill(q, fb, req_to_token, k_buf, v_buf, sm_scale):
    """Causal prefill attention of a chunk in float32 (the ROCm backends'
    own extend attention in the stand-in): rows of request i at positions
    prefix_i + j attend the pool rows of positions [0, prefix_i + j]."""
    qv = q.view(-1, HQ, D).float()
    outs, off = [], 0
    for i, r in enumerate(fb.req_pool_indices.tolist()):
        ext, pre = int(fb.extend_seq_lens_cpu[i]), int(fb.extend_prefix_lens_cpu[i])
        rows = req_to_token[r, : pre + ext].long()
        kx = k_buf[rows].float().repeat_interleave(HQ // HKV, dim=1)
        vx = v_buf[rows].float().repeat_interleave(HQ // HKV, dim=1)
        sc = torch.einsum("thd,shd->hts", qv[off: off + ext], kx) * sm_scale
        pos = pre + torch.arange(ext, device=q.device)
        sc = sc.masked_fill(torch.arange(pre + ext, device=q.device)[None, :] > pos[:, None], float("-inf"))
        outs.append(torch.einsum("hts,shd->thd", torch.softmax(sc, dim=-1), vx))
        off += ext
    return torch.cat(outs).to(torch.bfloat16).reshape(-1, HQ * D)


@pytest.mark.parametrize("backend_name", ["FlashInferAttnBackend", "TritonAttnBackend", "AiterAttnBackend"])
def test_prefill_populates_rings_and_decode_hits_through_installed_hooks(monkeypatch, backend_name):
    from mac_attention.integrations.sglang import bridge, hook_installer

    for key, val in (("MAC_ATTENTION_ENABLE", "1"), ("MAC_LOOKBACK_TOKENS_LEFT", str(M)),
                     ("MAC_SEMANTIC_POS_AHEAD", str(S)), ("MAC_GEN_MIN_LIMIT", "0"),
                     ("MAC_PERSISTENT_MAX_CONTEXT", "1024")):
        monkeypatch.setenv(key, val)
    monkeypatch.setattr(hook_installer, "_INSTALLED", [])
    sg = sglang_standin.install(monkeypatch)
    installed = set(hook_installer.install_hooks(strict=True))
    assert "sglang.srt.models.llama:LlamaAttention.forward" in installed

    dev = "cuda"
    g = torch.Generator(device=dev)
    g.manual_seed(11)
    prompts = [300, 517, 64]
    b = len(prompts)
    pool_rows, r2t_cols = 4096, 1024
    k_buf = torch.zeros(pool_rows, HKV, D, dtype=torch.bfloat16, device=dev)
    v_buf = torch.zeros_like(k_buf)
    perm = torch.randperm(pool_rows, generator=g, device=dev).to(torch.int32)
    req_pool = torch.tensor([2, 0, 3], dtype=torch.int32, device=dev)  # request slots in the pool
    req_to_token = torch.zeros(4, r2t_cols, dtype=torch.int32, device=dev)
    for i, r in enumerate(req_pool.tolist()):
        req_to_token[r, : prompts[i] + 1] = perm[i * r2t_cols: i * r2t_cols + prompts[i] + 1]
    inv = 1.0 / (10000.0 ** (torch.arange(0, D, 2, device=dev, dtype=torch.float32) / D))
    ang = torch.arange(2048, device=dev, dtype=torch.float32)[:, None] * inv[None, :]
    cos_sin = torch.cat([ang.cos(), ang.sin()], dim=1).contiguous()
    rect = bridge.load_mac_prefill_rectify_extension()
    sm_scale = 1.0 / math.sqrt(D)

    class KVPool:
        def set_kv_buffer(self, layer, loc, k, v, k_scale, v_scale):
            k_buf[loc.long()] = k.view(-1, HKV, D)
            v_buf[loc.long()] = v.view(-1, HKV, D)

        def get_kv_buffer(self, layer_id):
            return k_buf, v_buf

    class PrefillWrapper:
        """FlashInfer's paged prefill: full causal attention, lse in log2."""

        def __init__(self):
            self.qo = self.kv_indptr = self.kv_indices = None

        def forward_return_lse(self, q, kv, causal=True, sm_scale=None, **kw):
            o, lse = rect.window_attention_return_lse(q, kv[0], kv[1], self.qo, self.kv_indptr, self.kv_indices,
                                                      -1, sm_scale)
            return o, lse / math.log(2.0)

    wrapper = PrefillWrapper()
    if backend_name == "FlashInferAttnBackend":
        backend = sg.FlashInferAttnBackend(
            forward_metadata=types.SimpleNamespace(use_ragged=False, prefill_wrappers=[wrapper]),
            indices_updater_decode=types.SimpleNamespace(req_to_token=req_to_token),
            indices_updater_prefill=types.SimpleNamespace(req_to_token=req_to_token))
    else:
        backend = getattr(sg, backend_name)(
            req_to_token=req_to_token,
            prefill_attention=lambda q, layer, fb: _torch_prefill(q, fb, req_to_token, k_buf, v_buf, sm_scale))
    assert backend.mac_config.enable_mac  # the __init__ hook ran
    print(f"served through {backend_name}", flush=True)

    class RadixAttention:
        layer_id, tp_q_head_num, head_dim, scaling, logit_cap = 0, HQ, D, sm_scale, 0
        is_cross_attention, k_scale, v_scale, sliding_window_size = False, None, None, -1

        def __call__(self, q, k, v, fb, save_kv_cache=True):
            fn = backend.forward_decode if fb.forward_mode.is_decode_or_idle() else backend.forward_extend
            return fn(q, k, v, self, fb, save_kv_cache=save_kv_cache)

    rope_calls = []

    class Rope:
        cos_sin_cache, is_neox_style, rotary_dim = cos_sin, True, D

        def __call__(self, positions, q, k):
            rope_calls.append(int(q.shape[0]))
            return _rope_neox(positions, q, HQ, cos_sin), _rope_neox(positions, k, HKV, cos_sin)

    ident = lambda x: (x, None)  # noqa: E731
    layer = sg.LlamaAttention(HQ, HKV, D, ident, Rope(), RadixAttention(), ident)
    assert layer.mac_metadata is None  # set by the __init__ hook
    width = (HQ + 2 * HKV) * D

    # ---------------- prefill: every prompt in one chunk ----------------
    reqs = [types.SimpleNamespace(origin_input_ids=[0] * p) for p in prompts]
    sched = sg.ScheduleBatch(reqs, prefix_lens=[0] * b, seq_lens=torch.tensor(prompts))
    sched.prepare_for_extend()
    fb = sg.ForwardBatch.init_new(sched.get_model_worker_batch(), model_runner=None)
    assert fb.mac_prefill_cache_update_starts == [p - M for p in prompts]
    total = sum(prompts)
    positions = torch.cat([torch.arange(p, device=dev) for p in prompts])
    locs = torch.cat([req_to_token[r, :p] for r, p in zip(req_pool.tolist(), prompts)]).long()
    fb.__dict__.update(
        forward_mode=sglang_standin.ForwardMode(False), batch_size=b, req_pool_indices=req_pool,
        seq_lens=torch.tensor(prompts, device=dev), seq_lens_cpu=torch.tensor(prompts),
        extend_seq_lens=torch.tensor(prompts, device=dev), extend_seq_lens_cpu=list(prompts),
        extend_prefix_lens_cpu=[0] * b, out_cache_loc=locs, token_to_kv_pool=KVPool(), attn_backend=backend,
        spec_info=None, req_to_token_pool=types.SimpleNamespace(size=4))
    wrapper.qo = torch.tensor(np.concatenate([[0], np.cumsum(prompts)]), dtype=torch.int32, device=dev)
    wrapper.kv_indptr = wrapper.qo
    wrapper.kv_indices = locs.to(torch.int32)
    hidden = torch.randn(total, width, device=dev, generator=g).to(torch.bfloat16)
    q_pre_prefill = hidden[:, : HQ * D].clone().view(total, HQ, D)
    prefill_out = layer.forward(positions, hidden, fb)
    torch.cuda.synchronize()
    if backend_name != "FlashInferAttnBackend":  # the backend's own prefill ran and gave the layer's output
        assert f"{backend_name}.forward_extend (SGLang's own)" in sg.calls
        q_rot = _rope_neox(positions, hidden[:, : HQ * D], HQ, cos_sin)
        torch.testing.assert_close(prefill_out, _torch_prefill(q_rot, fb, req_to_token, k_buf, v_buf, sm_scale))
    meta = layer.mac_metadata
    assert meta is not None and rope_calls == [total]
    lse = meta.unified_lse_cache.cpu().numpy()
    for i, r in enumerate(req_pool.tolist()):  # every kept row written
        assert np.isfinite(lse[r]).all(), f"request {i}: ring rows left empty"
    assert meta.mac_cache_ready[req_pool.long()].all()
    assert meta.req_len[req_pool.long()].tolist() == prompts

    # ---------------- decode: heads 0-3 of request 0 repeat position P - 3 ----------------
    rings = {k: t.clone() for k, t in (("query_cache", meta.unified_query_cache),
                                       ("attn_cache", meta.unified_attn_cache), ("lse_cache", meta.unified_lse_cache))}
    seq = [p + 1 for p in prompts]
    dloc = torch.stack([req_to_token[r, p] for r, p in zip(req_pool.tolist(), prompts)]).long()
    fb = sg.ForwardBatch(
        forward_mode=sglang_standin.ForwardMode(True), batch_size=b, req_pool_indices=req_pool,
        seq_lens=torch.tensor(seq, device=dev), seq_lens_cpu=torch.tensor(seq), extend_seq_lens=None,
        extend_seq_lens_cpu=None, out_cache_loc=dloc, token_to_kv_pool=KVPool(), attn_backend=backend,
        spec_info=None, req_to_token_pool=types.SimpleNamespace(size=4))
    hidden = torch.randn(b, width, device=dev, generator=g).to(torch.bfloat16)
    hidden[0, : 4 * D] = q_pre_prefill[prompts[0] - 3, :4].reshape(-1)
    q_pre = hidden[:, : HQ * D].clone().view(b, HQ, D)
    k_new = hidden[:, HQ * D: (HQ + HKV) * D].clone()
    out = layer.forward(torch.tensor(prompts, device=dev), hidden, fb)
    torch.cuda.synchronize()
    assert rope_calls == [total]  # decode used the fused RoPE kernel, not the module's RoPE
    ws = backend.mac_last_persistent_workspace
    q_post = hidden[:, : HQ * D].view(b, HQ, D)  # rotated in place by the fused kernel
    assert not torch.equal(q_post, q_pre)
    torch.testing.assert_close(k_buf[dloc, :, :].float(), _rope_neox(torch.tensor(prompts, device=dev), k_new,
                                                                        HKV, cos_sin).view(b, HKV, D).float(),
                               atol=0.02, rtol=0.02)

    view = dict(q_post=q_post, q_pre=q_pre, k=k_buf, v=v_buf, req_to_token=req_to_token, req_ids=req_pool,
                past_lens=torch.tensor(prompts, dtype=torch.int32, device=dev), out_cache_loc=dloc,
                cache_ready=meta.mac_cache_ready, cache_epoch=meta.mac_cache_epoch,
                request_epoch=meta.request_epoch, **rings)
    sub = host_subset(torch, view, list(range(b)), semantic_pos_ahead=S, gen_min_limit=0)
    expect = oracle_run(sub)
    hit = ws["head_hit"][:b].cpu().numpy()
    np.testing.assert_array_equal(hit, expect.head["hit"])
    assert hit[0, :4].all(), hit
    np.testing.assert_array_equal(ws["head_match_pos"][:b].cpu().numpy(), expect.head["match_pos"])
    np.testing.assert_array_equal(ws["group_mode"][:b].cpu().numpy(), expect.group["mode"])
    assert rel_l2(out.view(b, HQ, D).float().cpu().numpy(), bits(expect.out)) < 1e-2
    for i, r in enumerate(req_pool.tolist()):  # ring row written at past_len % M
        dest = prompts[i] % M
        got = meta.unified_attn_cache[r, dest].float().cpu().numpy()
        assert rel_l2(got, bits(expect.attn_cache[i, dest])) < 1e-2
        assert torch.equal(meta.unified_query_cache[r, dest], q_pre[i])
