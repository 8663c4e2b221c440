"""The serving glue end to end on the GPU: a prefill chunk populates the
rings through offload_prefill_cache (fused rectification), the requests are
marked ready, and the next decode step goes through the FlashInfer
forward_decode hook into the fused MAC step.  The decode result is checked
against the CPU oracle run on the ring state the prefill left behind.
SGLang objects are small stand-ins."""

import math
import types

import numpy as np
import pytest

from helpers import bits, host_subset, oracle_run, rel_l2, syn

torch = pytest.importorskip("torch")

pytestmark = pytest.mark.gpu


def test_prefill_then_decode_through_the_hooks():
    from mac_attention.integrations.sglang import persistent
    from mac_attention.integrations.sglang.config import MacSGLangConfig

    hq, hkv, d, m, S = 8, 2, 128, 16, 32
    kv_lens = [300, 517, 64]
    prompts = [x - 1 for x in kv_lens]
    b = len(kv_lens)
    dev = syn.device_ragged_case(torch, kv_lens=kv_lens, hq=hq, hkv=hkv, capacity=m, seed=7)
    cfg = MacSGLangConfig(enable_mac=True, mac_lookback_tokens_left=m, mac_gen_min_limit=0,
                          mac_semantic_pos_ahead=S, mac_persistent_max_context=1024)
    meta = persistent.MacMetadata(hq, hkv, d)
    meta.allocate(max_running=4, capacity=m, device="cuda", prefill_capacity=sum(prompts))
    sm_scale = 1.0 / math.sqrt(d)

    # ---- prefill: every prompt in one chunk ----
    g = torch.Generator(device="cuda")
    g.manual_seed(3)
    total = sum(prompts)
    q_post = torch.randn(total, hq, d, device="cuda", generator=g).to(torch.bfloat16)
    src_q = torch.randn(total, hq, d, device="cuda", generator=g).to(torch.bfloat16)
    qo = torch.tensor(np.concatenate([[0], np.cumsum(prompts)]), dtype=torch.int32, device="cuda")
    kv_idx = torch.cat([dev["req_to_token"][i, :p] for i, p in enumerate(prompts)]).contiguous()
    o_full, lse_full = meta.rect_ext.window_attention_return_lse(q_post, dev["k"], dev["v"], qo, qo, kv_idx,
                                                                 -1, sm_scale)
    meta.cur_q_before_rope = src_q
    req_ids = torch.arange(b, dtype=torch.int32, device="cuda")
    persistent.offload_prefill_cache(meta, cfg, q_post=q_post, o_full=o_full, lse_full=lse_full, k_buffer=dev["k"],
                                     v_buffer=dev["v"], qo_indptr=qo, kv_indptr=qo, kv_indices=kv_idx,
                                     req_ids=req_ids, prefix_lens=torch.zeros(b, dtype=torch.int32, device="cuda"),
                                     sm_scale=sm_scale)
    torch.cuda.synchronize()
    assert meta.req_len[:b].tolist() == prompts
    assert meta.mac_cache_ready[:b].all() and not meta.mac_cache_ready[b:].any()
    assert (meta.mac_cache_epoch[:b] == meta.request_epoch[:b]).all()
    assert meta.mac_cache_ready_host[:b] == [True] * b
    lse = meta.unified_lse_cache[:b].cpu().numpy()
    assert np.isfinite(lse).all()  # every ring row was written (all prompts >= M rows, E > 0)

    # ---- decode: heads 0-3 of request 0 repeat the query of position P-3 ----
    q_dec_pre = torch.randn(b, hq, d, device="cuda", generator=g).to(torch.bfloat16)
    row = int(qo[0]) + prompts[0] - 3
    q_dec_pre[0, :4] = src_q[row, :4]
    q_dec_post = torch.randn(b, hq, d, device="cuda", generator=g).to(torch.bfloat16)
    meta.req_ids[:b] = req_ids
    meta.cache_lens[:b] = torch.tensor(prompts, dtype=torch.int32, device="cuda")
    meta.req_ids_host = list(range(b))
    persistent.preserve_q_before_rope(meta, q_dec_pre.view(b, hq * d), current_is_decode=True)

    ring_view = dict(q_post=q_dec_post, q_pre=q_dec_pre, k=dev["k"], v=dev["v"], req_to_token=dev["req_to_token"],
                     req_ids=req_ids, past_lens=meta.cache_lens[:b], out_cache_loc=dev["out_cache_loc"],
                     query_cache=meta.unified_query_cache, attn_cache=meta.unified_attn_cache,
                     lse_cache=meta.unified_lse_cache, cache_ready=meta.mac_cache_ready,
                     cache_epoch=meta.mac_cache_epoch, request_epoch=meta.request_epoch)
    sub = host_subset(torch, ring_view, list(range(b)), semantic_pos_ahead=S, gen_min_limit=0)
    expect = oracle_run(sub)

    pool = types.SimpleNamespace(get_kv_buffer=lambda layer_id: (dev["k"], dev["v"]),
                                 set_kv_buffer=lambda *a: pytest.fail("decode K/V are already in the pool"))
    backend = types.SimpleNamespace(num_wrappers=1, indices_updater_decode=types.SimpleNamespace(
        req_to_token=dev["req_to_token"]))
    layer = types.SimpleNamespace(mac_metadata=meta, mac_config=cfg, tp_q_head_num=hq, head_dim=d, layer_id=0,
                                  scaling=sm_scale, logit_cap=0, is_cross_attention=False,
                                  k_scale=None, v_scale=None)
    fb = types.SimpleNamespace(batch_size=b, out_cache_loc=dev["out_cache_loc"], token_to_kv_pool=pool,
                               spec_info=None)
    out = persistent.flashinfer_forward_decode_around(
        lambda *a, **k: pytest.fail("fell back to the backend's own decode"), backend,
        q_dec_post.view(b, hq * d), None, None, layer, fb)
    torch.cuda.synchronize()
    ws = backend.mac_last_persistent_workspace
    hit = ws["head_hit"][:b].cpu().numpy()
    np.testing.assert_array_equal(hit, expect.head["hit"])
    assert hit[0, :4].all()
    np.testing.assert_array_equal(ws["head_match_pos"][:b].cpu().numpy(), expect.head["match_pos"])
    np.testing.assert_array_equal(ws["group_mode"][:b].cpu().numpy(), expect.group["mode"])
    assert rel_l2(out.view(b, hq, d).float().cpu().numpy(), bits(expect.out)) < 1e-2
