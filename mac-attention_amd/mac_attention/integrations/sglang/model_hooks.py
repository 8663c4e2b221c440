"""Model-side SGLang hooks: per-layer MAC state, pre-RoPE query
preservation inside the attention module, and the ring update after a
prefill chunk inside FlashInfer's forward_extend.

Behaviour follows the reference's llama_hooks.py (attention forward
:1341-1470, MACMetadata.prepare_forward_batch :932-1029, Qwen MoE attention
:1064-1284, model forward :1852-1876) and flashinfer_hooks.py
(init_forward_metadata :703-735, forward_extend :2847-3010, prefill ring
update :2237-2490).  The design here is this build's: one forward wrapper
serves every supported attention class (a Qwen3 attention's q/k norm is
applied when the module has one), the batch bookkeeping is one
mac_update_request_state launch, and the ring update is the fused
rectification kernel (``persistent.offload_prefill_cache``) on the rows the
scheduler marked.
"""

from __future__ import annotations

import math
from typing import Any, Optional

import torch

from . import persistent
from .config import get_mac_config
from .prefill_suffix import build_prefill_suffix_plan, compact_by_segments, compact_kv_indices_by_segments

_LN2 = math.log(2.0)


# ---------------------------------------------------------- batch state ----


def _host_ints(value: Any, n: int) -> Optional[list[int]]:
    if value is None:
        return None
    if torch.is_tensor(value):
        if value.device.type != "cpu":
            return None
        value = value[:n].tolist()
    try:
        return [int(x) for x in list(value)[:n]]
    except Exception:
        return None


def _max_running(forward_batch: Any, config: Any) -> int:
    """Ring rows to allocate: one per request slot of the pool."""
    pool = getattr(forward_batch, "req_to_token_pool", None)
    size = int(getattr(pool, "size", 0) or 0)
    return max(size, int(getattr(config, "max_running_requests", 0) or 0), int(forward_batch.batch_size), 1)


def ensure_layer_state(module: Any, forward_batch: Any, hidden_states: torch.Tensor, config: Any):
    """The module's MacMetadata, with its ring caches allocated for the pool
    (re-allocated when the pool or the capacity changes)."""
    meta = getattr(module, "mac_metadata", None)
    if meta is None:
        meta = persistent.MacMetadata(module.num_heads, module.num_kv_heads, module.head_dim)
        module.mac_metadata = meta
    capacity = int(config.mac_lookback_tokens_left)
    rows = _max_running(forward_batch, config)
    qc = meta.unified_query_cache
    if (qc is None or qc.device != hidden_states.device or qc.dtype != hidden_states.dtype
            or qc.shape[0] < rows or qc.shape[1] != capacity):
        chunk = int(getattr(config, "chunked_prefill_size", 0) or 0)
        meta.allocate(max_running=rows, capacity=capacity, device=hidden_states.device, dtype=hidden_states.dtype,
                      prefill_capacity=max(chunk, int(hidden_states.shape[0])))
        meta.match_req_len = torch.zeros_like(meta.req_len)
    return meta


_BATCH_STATE = "_mac_batch_state"


def batch_state(forward_batch: Any, device: torch.device, *, fresh: bool = False) -> dict:
    """The forward's request ids, sequence lengths and new-token counts as
    int32 device tensors (plus host copies when they are at hand).  The model
    forward hook builds it once per forward (``fresh``) and every layer
    reuses it (llama_hooks.py:1852-1876 prepares the batch once in the model
    forward); without that hook each layer builds its own and keeps none, so
    a forward batch object reused across forwards never serves stale
    lengths."""
    cached = getattr(forward_batch, _BATCH_STATE, None)
    if not fresh and cached is not None and cached["device"] == device:
        return cached
    b = int(forward_batch.batch_size)
    capturing = persistent.is_graph_capturing()
    req = forward_batch.req_pool_indices[:b].to(device=device, dtype=torch.int32)
    seq = forward_batch.seq_lens[:b].to(device=device, dtype=torch.int32)
    if forward_batch.forward_mode.is_decode_or_idle():
        cur = torch.ones_like(seq)
    elif getattr(forward_batch, "extend_seq_lens", None) is not None:
        cur = forward_batch.extend_seq_lens[:b].to(device=device, dtype=torch.int32)
    else:
        cur = torch.tensor(forward_batch.extend_seq_lens_cpu[:b], dtype=torch.int32, device=device)
    req_host = None
    if not capturing:
        req_host = _host_ints(forward_batch.req_pool_indices, b) or [int(x) for x in req.tolist()]
    seq_host = None if capturing else _host_ints(getattr(forward_batch, "seq_lens_cpu", None), b)
    state = dict(device=device, batch=b, req_ids=req, seq=seq, cur=cur, req_ids_host=req_host, seq_host=seq_host)
    if fresh:
        try:
            setattr(forward_batch, _BATCH_STATE, state)
        except AttributeError:  # a batch object that takes no new attributes: built per layer
            pass
    return state


def prepare_batch(meta: Any, forward_batch: Any) -> None:
    """Per-layer request bookkeeping (llama_hooks.py:932-1029): request ids,
    the tokens already cached before this step (``cache_lens`` = seq_len -
    new tokens, the decode step's past_len) and ``req_len`` by request, in
    one mac_update_request_state launch, from the forward's batch_state."""
    b = int(forward_batch.batch_size)
    if b <= 0 or meta.req_ids is None:
        return
    st = batch_state(forward_batch, meta.req_ids.device)
    meta.req_ids[:b].copy_(st["req_ids"])
    meta.req_ids_host = st["req_ids_host"]
    if st["req_ids_host"] and not forward_batch.forward_mode.is_decode_or_idle():
        persistent.clear_low_hit_ejection(meta, st["req_ids_host"])  # a prefill rebuilds their rings
    if st["seq_host"]:
        meta.cur_kv_len = max(st["seq_host"])
    match = getattr(meta, "match_req_len", None)
    if match is None:
        match = meta.match_req_len = torch.zeros_like(meta.req_len)
    meta.cache_ext.mac_update_request_state(meta.req_len, match, meta.cache_lens[:b], meta.req_ids[:b], st["seq"],
                                            st["cur"])


def model_forward_around(original_fn: Any, self: Any, *args: Any, **kwargs: Any) -> Any:
    """LlamaModel / Qwen MoE model forward (input_ids, positions,
    forward_batch, ...): the settings and the batch state are attached to the
    forward batch once, before any layer runs (llama_hooks.py:1852-1876)."""
    input_ids = kwargs.get("input_ids", args[0] if len(args) > 0 else None)
    positions = kwargs.get("positions", args[1] if len(args) > 1 else None)
    forward_batch = kwargs.get("forward_batch", args[2] if len(args) > 2 else None)
    config = get_mac_config()
    if config.enable_mac and forward_batch is not None and int(getattr(forward_batch, "batch_size", 0) or 0) > 0:
        ref = positions if torch.is_tensor(positions) else input_ids
        if torch.is_tensor(ref) and ref.device.type == "cuda":
            forward_batch.mac_config = config
            batch_state(forward_batch, ref.device, fresh=True)
    return original_fn(self, *args, **kwargs)


# ----------------------------------------------------- attention forward ----


def attention_init_after(result: Any, self: Any, *args: Any, **kwargs: Any) -> Any:
    """LlamaAttention / Qwen MoE attention __init__: a module gets its MAC
    state on its first forward; start without one."""
    self.mac_metadata = None
    return result


def _fused_decode_rope(module: Any, meta: Any, positions: torch.Tensor, q, k, v, forward_batch: Any) -> bool:
    """Decode: RoPE + pre-RoPE copy + K/V pool write in one kernel
    (persistent.try_decode_rope_preserve); False sends the caller through
    its own rotary embedding and K/V write."""
    rope = getattr(module, "rotary_emb", None)
    attn = getattr(module, "attn", None)
    pool = getattr(forward_batch, "token_to_kv_pool", None)
    if rope is None or attn is None or pool is None or not hasattr(rope, "cos_sin_cache"):
        return False
    if getattr(rope, "rotary_dim", meta.head_dim) != meta.head_dim:
        return False
    k_buffer, v_buffer = pool.get_kv_buffer(attn.layer_id)
    return persistent.try_decode_rope_preserve(meta, positions, q, k, v, k_buffer, v_buffer, rope.cos_sin_cache,
                                               forward_batch.out_cache_loc,
                                               bool(getattr(rope, "is_neox_style", True)))


def attention_forward_around(original_fn: Any, self: Any, *args: Any, **kwargs: Any) -> Any:
    """Attention forward of a supported model (positions, hidden_states,
    forward_batch): the same projections, RoPE and attention call as the
    model's own forward, plus the pre-RoPE query rows the ring stores and the
    layer's MAC state handed to the attention backend."""
    names = ("positions", "hidden_states", "forward_batch")
    vals = [kwargs.get(name, args[i] if len(args) > i else None) for i, name in enumerate(names)]
    positions, hidden_states, forward_batch = vals
    config = get_mac_config()
    if (positions is None or hidden_states is None or forward_batch is None or not config.enable_mac
            or hidden_states.device.type != "cuda"):
        return original_fn(self, *args, **kwargs)
    meta = ensure_layer_state(self, forward_batch, hidden_states, config)
    prepare_batch(meta, forward_batch)
    qkv, _ = self.qkv_proj(hidden_states)
    q, k, v = qkv.split([self.q_size, self.kv_size, self.kv_size], dim=-1)
    if hasattr(self, "_apply_qk_norm"):  # Qwen3: per-head RMS norm of q and k before RoPE
        q, k = self._apply_qk_norm(q, k)
    decode = bool(forward_batch.forward_mode.is_decode_or_idle())
    fused = decode and _fused_decode_rope(self, meta, positions, q, k, v, forward_batch)
    if not fused:
        persistent.preserve_q_before_rope(meta, q, decode, forward_batch, graph_safe=persistent.is_graph_capturing())
        q, k = self.rotary_emb(positions, q, k)
    self.attn.mac_metadata = meta
    self.attn.mac_config = config
    out = self.attn(q, k, v, forward_batch, save_kv_cache=not fused)
    output, _ = self.o_proj(out)
    return output


# ------------------------------------------------------ FlashInfer extend ----


def flashinfer_backend_init_after(result: Any, self: Any, *args: Any, **kwargs: Any) -> Any:
    """FlashInferAttnBackend.__init__: the settings the hooks read."""
    self.mac_config = get_mac_config()
    return result


def flashinfer_init_forward_metadata_around(original_fn: Any, self: Any, forward_batch: Any, *args: Any,
                                            **kwargs: Any) -> Any:
    """FlashInferAttnBackend.init_forward_metadata (flashinfer_hooks.py:703-735):
    SGLang's own metadata, then the scheduler's ring marks and the chunk's
    prefix / extend lengths kept on the backend as well.  A piecewise
    CUDA-graph replay runs forward_extend on a static forward batch that
    lost these plugin attributes; the suffix plan falls back to the
    backend's copies (prefill_suffix.build_prefill_suffix_plan)."""
    result = original_fn(self, forward_batch, *args, **kwargs)
    config = getattr(self, "mac_config", None) or get_mac_config()
    if config.enable_mac:
        self.mac_prefill_cache_update_starts_current = getattr(forward_batch, "mac_prefill_cache_update_starts", None)
        self.mac_extend_prefix_lens_cpu_current = getattr(forward_batch, "extend_prefix_lens_cpu", None)
        self.mac_extend_seq_lens_cpu_current = getattr(forward_batch, "extend_seq_lens_cpu", None)
    return result


def _prefill_kv_indices(backend: Any, forward_batch: Any, meta: Any, b: int) -> tuple[torch.Tensor, list[int]]:
    """Page-size-1 KV pool rows of every request of the batch, concatenated
    (request i: its positions [0, seq_len_i)), and the per-request lengths."""
    seq = _host_ints(getattr(forward_batch, "seq_lens_cpu", None), b)
    if seq is None:
        seq = [int(x) for x in forward_batch.seq_lens[:b].tolist()]
    given = getattr(backend, "mac_prefill_kv_indices", None)
    if torch.is_tensor(given) and given.numel() >= sum(seq):
        return given[: sum(seq)], seq
    r2t = backend.indices_updater_prefill.req_to_token
    reqs = meta.req_ids_host or [int(x) for x in forward_batch.req_pool_indices[:b].tolist()]
    rows = [r2t[r, :s] for r, s in zip(reqs, seq)]
    return torch.cat(rows).to(torch.int32).contiguous(), seq


def update_rings_after_prefill(backend: Any, forward_batch: Any, config: Any, meta: Any, q_input: torch.Tensor,
                               k_buffer: torch.Tensor, v_buffer: torch.Tensor, o: torch.Tensor, lse: torch.Tensor,
                               layer: Any) -> None:
    """Rings of the chunk's requests (flashinfer_hooks.py:2237-2490): the
    rows the scheduler marked (every row without marks) are rectified from
    the full prefill state (o, natural-log lse) and stored with their
    pre-RoPE queries; the requests are then marked ready."""
    b = int(forward_batch.batch_size)
    req_ids = meta.req_ids[:b]
    src_q = meta.cur_q_before_rope
    if src_q is None:
        persistent.invalidate_persistent_ready(meta, req_ids)
        return
    dev = q_input.device
    plan = build_prefill_suffix_plan(forward_batch, b, int(q_input.shape[0]))
    if plan is not None and plan.total_len <= 0:
        return  # the scheduler kept no row of this chunk
    kv_indices, seq = _prefill_kv_indices(backend, forward_batch, meta, b)
    i32 = dict(dtype=torch.int32, device=dev)
    if plan is None:  # every row of every request
        ext = _host_ints(getattr(forward_batch, "extend_seq_lens_cpu", None), b)
        qo = torch.tensor([0] + list(_cumsum(ext)), **i32)
        kv_indptr = torch.tensor([0] + list(_cumsum(seq)), **i32)
        prefix = torch.tensor([s - e for s, e in zip(seq, ext)], **i32)
        rows = (q_input, o, lse, src_q)
        ids = req_ids
    else:
        segs = plan.segments
        if meta.cur_q_before_rope_compacted:
            src = src_q[-int(plan.total_len):] if src_q.shape[0] >= plan.total_len else src_q
        else:
            src = compact_by_segments(src_q, segs)
        rows = (compact_by_segments(q_input, segs), compact_by_segments(o, segs), compact_by_segments(lse, segs), src)
        qo = torch.tensor(plan.offsets, **i32)
        kv_indptr = torch.tensor(plan.kv_offsets, **i32)
        kv_indices = compact_kv_indices_by_segments(kv_indices, segs, batch_size=b)
        ids = req_ids.index_select(0, torch.tensor(plan.req_indices, dtype=torch.long, device=dev)).contiguous()
        prefix = torch.tensor(plan.request_lengths, **i32)
    q_rows, o_rows, lse_rows, src_rows = rows
    meta.cur_q_before_rope = src_rows
    persistent.offload_prefill_cache(meta, config, q_post=q_rows, o_full=o_rows, lse_full=lse_rows,
                                     k_buffer=k_buffer, v_buffer=v_buffer, qo_indptr=qo, kv_indptr=kv_indptr,
                                     kv_indices=kv_indices, req_ids=ids, prefix_lens=prefix,
                                     sm_scale=float(layer.scaling))


def _cumsum(xs):
    total = 0
    for x in xs:
        total += int(x)
        yield total


def flashinfer_forward_extend_around(original_fn: Any, self: Any, q: torch.Tensor, k: torch.Tensor,
                                     v: torch.Tensor, layer: Any, forward_batch: Any, save_kv_cache: bool = True,
                                     **kwargs: Any) -> Any:
    """Around-hook of FlashInferAttnBackend.forward_extend
    (flashinfer_hooks.py:2847-3010): the paged prefill attention with its
    lse, then the ring update of the chunk.  Ragged prefill, unsupported
    layers and chunks the scheduler keeps no row of run SGLang's own path."""
    config = getattr(layer, "mac_config", None) or getattr(self, "mac_config", None) or get_mac_config()
    fm = getattr(self, "forward_metadata", None)
    if (not persistent.supports_mac_backend(self, layer, forward_batch, config) or fm is None
            or getattr(fm, "use_ragged", True)):
        return original_fn(self, q, k, v, layer, forward_batch, save_kv_cache=save_kv_cache, **kwargs)
    meta = layer.mac_metadata
    b = int(forward_batch.batch_size)
    q_input = q.contiguous().view(-1, layer.tp_q_head_num, layer.head_dim)
    plan = build_prefill_suffix_plan(forward_batch, b, int(q_input.shape[0]))
    if plan is not None and plan.total_len <= 0:
        return original_fn(self, q, k, v, layer, forward_batch, save_kv_cache=save_kv_cache, **kwargs)
    if k is not None and save_kv_cache:
        forward_batch.token_to_kv_pool.set_kv_buffer(layer, forward_batch.out_cache_loc, k, v, layer.k_scale,
                                                     layer.v_scale)
    k_buffer, v_buffer = forward_batch.token_to_kv_pool.get_kv_buffer(layer.layer_id)
    wrapper = fm.prefill_wrappers[self._get_wrapper_idx(layer)]
    o, lse_log2 = wrapper.forward_return_lse(q_input, (k_buffer, v_buffer), causal=True, sm_scale=layer.scaling,
                                             window_left=getattr(layer, "sliding_window_size", -1),
                                             logits_soft_cap=getattr(layer, "logit_cap", 0.0))
    lse = lse_log2 * _LN2  # FlashInfer returns log2; the ring stores natural-log lse
    update_rings_after_prefill(self, forward_batch, config, meta, q_input, k_buffer, v_buffer, o, lse, layer)
    return o.view(-1, layer.tp_q_head_num * layer.head_dim)


# ----------------------------------------------- ROCm attention backends ----
#
# SGLang on ROCm serves attention with AiterAttnBackend (when aiter is
# installed) or TritonAttnBackend, not FlashInfer.  The hooks below attach
# the same MAC path to them: construction and init_forward_metadata as for
# FlashInfer (backend_init_after, flashinfer_init_forward_metadata_around are
# backend-agnostic), the fused MAC step on decode
# (persistent.flashinfer_forward_decode_around, also backend-agnostic), and
# on extend the backend's own prefill attention followed by the ring update.
# These backends return no lse, so the full prefill state (o, lse) of the
# rows the ring keeps -- at most M per request -- comes from this build's
# window-attention kernel with no window (causal attention over [0, pos]),
# the role FlashInfer's forward_return_lse plays in flashinfer_hooks.py:2847-3010.


def _req_to_token(backend: Any, forward_batch: Any) -> Optional[torch.Tensor]:
    """The request-to-token table: FlashInfer keeps it on its index updaters,
    the Triton and aiter backends as ``req_to_token``, SGLang's forward batch
    on its ``req_to_token_pool``."""
    for owner in (getattr(backend, "indices_updater_prefill", None), getattr(backend, "indices_updater_decode", None),
                  backend, getattr(forward_batch, "req_to_token_pool", None)):
        t = getattr(owner, "req_to_token", None) if owner is not None else None
        if torch.is_tensor(t):
            return t
    return None


def _ring_rows(forward_batch: Any, b: int, total_q: int, capacity: int):
    """The chunk rows the ring keeps: the scheduler's marked suffix of each
    request (every row without marks), cut to its last ``capacity`` rows
    (mac_prefill_update_cache keeps no more, PREFILL:201-269).  Returns the
    plan (None without marks) and per kept segment (batch row, first chunk
    row, absolute position of that row, rows, request kv length), or None
    when the chunk's lengths are not on the host."""
    from .prefill_suffix import PrefillSuffixSegment

    plan = build_prefill_suffix_plan(forward_batch, b, total_q)
    if plan is not None:
        segs = list(plan.segments)
    else:
        ext = _host_ints(getattr(forward_batch, "extend_seq_lens_cpu", None), b)
        pre = _host_ints(getattr(forward_batch, "extend_prefix_lens_cpu", None), b) or [0] * b
        if ext is None or sum(ext) != total_q:
            return plan, None
        segs, q_base, kv_base = [], 0, 0
        for i in range(b):
            if ext[i] > 0:
                segs.append(PrefillSuffixSegment(i, q_base, pre[i], ext[i], kv_base, pre[i] + ext[i]))
            q_base += ext[i]
            kv_base += pre[i] + ext[i]
    kept = []
    for s in segs:
        n = min(s.length, capacity)
        skip = s.length - n
        kept.append((s.batch_index, s.source_start + skip, s.update_start + skip, n, s.kv_len))
    return plan, kept


def _src_rows(meta: Any, plan: Any, kept: list, rows: int) -> Optional[list[int]]:
    """Indices into the preserved pre-RoPE rows of the kept chunk rows, or
    None when they were not kept (persistent.preserve_q_before_rope keeps
    every row, the plan's rows compacted in plan order, or a tail)."""
    src = meta.cur_q_before_rope
    if src is None:
        return None
    idx = []
    if not meta.cur_q_before_rope_compacted:
        for _, first, _, n, _ in kept:
            idx.extend(range(first, first + n))
    elif plan is not None and int(src.shape[0]) == int(plan.total_len):
        where, off = {}, 0
        for s in plan.segments:
            where[s.batch_index] = (s.source_start, off)
            off += s.length
        for bi, first, _, n, _ in kept:
            start, o = where[bi]
            idx.extend(range(o + first - start, o + first - start + n))
    else:  # a preserved tail of the chunk
        base = int(meta.cur_q_before_rope_local_start)
        for _, first, _, n, _ in kept:
            if first < base:
                return None
            idx.extend(range(first - base, first - base + n))
    return idx if all(0 <= i < int(src.shape[0]) for i in idx) else None


def update_rings_from_own_prefill(backend: Any, forward_batch: Any, config: Any, meta: Any, q_input: torch.Tensor,
                                  k_buffer: torch.Tensor, v_buffer: torch.Tensor, layer: Any) -> None:
    """Ring update after a prefill chunk whose attention backend returned no
    lse: the kept rows' full prefill state from the window-attention kernel
    (no window), then the fused rectification (persistent.offload_prefill_cache)
    and the ready marks."""
    b = int(forward_batch.batch_size)
    dev = q_input.device
    req_ids = meta.req_ids[:b]
    capacity = int(meta.unified_query_cache.shape[1])
    plan, kept = _ring_rows(forward_batch, b, int(q_input.shape[0]), capacity)
    if plan is not None and plan.total_len <= 0:
        return  # the scheduler kept no row of this chunk
    r2t = _req_to_token(backend, forward_batch)
    src_idx = _src_rows(meta, plan, kept, int(q_input.shape[0])) if kept is not None else None
    if kept is None or not kept or r2t is None or src_idx is None:
        persistent.invalidate_persistent_ready(meta, req_ids)
        return
    reqs = meta.req_ids_host or [int(x) for x in forward_batch.req_pool_indices[:b].tolist()]
    i32 = dict(dtype=torch.int32, device=dev)
    rows = torch.tensor([r for _, first, _, n, _ in kept for r in range(first, first + n)], dtype=torch.long,
                        device=dev)
    qo = torch.tensor([0] + list(_cumsum(n for _, _, _, n, _ in kept)), **i32)
    kv_indptr = torch.tensor([0] + list(_cumsum(kv for *_, kv in kept)), **i32)
    kv_indices = torch.cat([r2t[reqs[bi], :kv] for bi, _, _, _, kv in kept]).to(torch.int32).contiguous()
    ids = req_ids.index_select(0, torch.tensor([bi for bi, *_ in kept], dtype=torch.long, device=dev)).contiguous()
    prefix = torch.tensor([pos for _, _, pos, _, _ in kept], **i32)
    q_rows = q_input.index_select(0, rows).contiguous()
    o_full, lse_full = meta.rect_ext.window_attention_return_lse(q_rows, k_buffer, v_buffer, qo, kv_indptr,
                                                                 kv_indices, -1, float(layer.scaling))
    meta.cur_q_before_rope = meta.cur_q_before_rope.index_select(
        0, torch.tensor(src_idx, dtype=torch.long, device=dev)).contiguous()
    meta.cur_q_before_rope_compacted = True
    persistent.offload_prefill_cache(meta, config, q_post=q_rows, o_full=o_full, lse_full=lse_full,
                                     k_buffer=k_buffer, v_buffer=v_buffer, qo_indptr=qo, kv_indptr=kv_indptr,
                                     kv_indices=kv_indices, req_ids=ids, prefix_lens=prefix,
                                     sm_scale=float(layer.scaling))


def rocm_forward_extend_around(original_fn: Any, self: Any, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                               layer: Any, forward_batch: Any, save_kv_cache: bool = True, **kwargs: Any) -> Any:
    """Around-hook of AiterAttnBackend / TritonAttnBackend.forward_extend: the
    backend's own prefill attention (its output is the layer's, and it writes
    the chunk's K/V), then the ring update of the rows the ring keeps."""
    config = getattr(layer, "mac_config", None) or getattr(self, "mac_config", None) or get_mac_config()
    out = original_fn(self, q, k, v, layer, forward_batch, save_kv_cache=save_kv_cache, **kwargs)
    if not persistent.supports_mac_backend(self, layer, forward_batch, config):
        return out
    meta = layer.mac_metadata
    q_input = q.contiguous().view(-1, layer.tp_q_head_num, layer.head_dim)
    k_buffer, v_buffer = forward_batch.token_to_kv_pool.get_kv_buffer(layer.layer_id)
    update_rings_from_own_prefill(self, forward_batch, config, meta, q_input, k_buffer, v_buffer, layer)
    return out
