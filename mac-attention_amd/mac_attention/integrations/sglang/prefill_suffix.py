"""Which prefill rows feed the MAC ring cache.

The scheduler marks, per request of an extend batch, the first absolute
position whose row should reach the ring (``mac_prefill_cache_update_starts``,
-1 = none).  The plan turns that into compact row segments and the
``offsets / lens / request_lengths`` vectors that mac_prefill_update_cache and
the fused rectification consume.  Same data types, fields and rules as
attention/src/mac_attention/integrations/sglang/prefill_suffix.py of the
reference (:9-30 types, :45-134 planning, :137-174 compaction).
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Any, Optional, Sequence

import torch


@dataclass(frozen=True)
class PrefillSuffixSegment:
    batch_index: int      # request within the batch
    source_start: int     # first row in the batch's concatenated extend rows
    update_start: int     # absolute position of that row (request length before it)
    length: int           # rows kept from source_start
    kv_source_start: int  # start of the request's KV indices in the batch's list
    kv_len: int           # prefix + extend length of the request


@dataclass(frozen=True)
class PrefillSuffixPlan:
    segments: tuple[PrefillSuffixSegment, ...]
    total_len: int
    req_indices: tuple[int, ...]
    request_lengths: tuple[int, ...]
    lens: tuple[int, ...]
    offsets: tuple[int, ...]
    kv_offsets: tuple[int, ...]


def _host_ints(value: Any, n: int) -> Optional[list[int]]:
    """First n entries as Python ints, or None when they are not on the host."""
    if value is None:
        return None
    if torch.is_tensor(value):
        return None if value.device.type != "cpu" else [int(x) for x in value[:n].tolist()]
    try:
        return [int(x) for x in list(value)[:n]]
    except Exception:
        return None


def build_prefill_suffix_plan(forward_batch: Any, batch_size: int, total_q_len: int, *,
                              allow_backend_fallback: bool = True) -> Optional[PrefillSuffixPlan]:
    """``None``: no scheduler marks (callers keep every row).  An empty plan:
    the scheduler skipped every request of this chunk."""
    backend = getattr(forward_batch, "attn_backend", None) if allow_backend_fallback else None

    def field(name: str, backend_name: str):
        v = getattr(forward_batch, name, None)
        if v is None and backend is not None:
            v = getattr(backend, backend_name, None)
        return _host_ints(v, batch_size)

    starts = field("mac_prefill_cache_update_starts", "mac_prefill_cache_update_starts_current")
    if starts is None:
        return None
    prefix = field("extend_prefix_lens_cpu", "mac_extend_prefix_lens_cpu_current")
    extend = field("extend_seq_lens_cpu", "mac_extend_seq_lens_cpu_current")
    if prefix is None or extend is None or min(len(starts), len(prefix), len(extend)) < batch_size:
        return None
    extend = [max(0, x) for x in extend[:batch_size]]
    if sum(extend) != int(total_q_len):
        return None

    segments = []
    q_base = kv_base = 0
    for b in range(batch_size):
        pre = max(0, prefix[b])
        kv_len = pre + extend[b]
        start = starts[b]
        if start >= 0 and extend[b] > 0:
            local = max(start - pre, 0)   # a mark inside the prefix starts at the chunk
            if local < extend[b]:
                segments.append(PrefillSuffixSegment(b, q_base + local, pre + local, extend[b] - local,
                                                     kv_base, kv_len))
        q_base += extend[b]
        kv_base += kv_len

    offsets, kv_offsets = [0], [0]
    for s in segments:
        offsets.append(offsets[-1] + s.length)
        kv_offsets.append(kv_offsets[-1] + s.kv_len)
    return PrefillSuffixPlan(
        segments=tuple(segments), total_len=offsets[-1],
        req_indices=tuple(s.batch_index for s in segments),
        request_lengths=tuple(s.update_start for s in segments),
        lens=tuple(s.length for s in segments), offsets=tuple(offsets),
        kv_offsets=tuple(kv_offsets))


def _gather(tensor: torch.Tensor, ranges: Sequence[tuple[int, int]]) -> torch.Tensor:
    if not ranges:
        return tensor[:0]
    if len(ranges) == 1:
        a, n = ranges[0]
        return tensor[a:a + n]
    return torch.cat([tensor[a:a + n] for a, n in ranges], dim=0)


def compact_by_segments(tensor: torch.Tensor, segments: Sequence[PrefillSuffixSegment], *,
                        clone: bool = False) -> torch.Tensor:
    """Rows of the segments, concatenated in plan order."""
    out = _gather(tensor, [(s.source_start, s.length) for s in segments]).contiguous()
    return out.clone() if clone else out


def compact_kv_indices_by_segments(kv_indices: torch.Tensor, segments: Sequence[PrefillSuffixSegment], *,
                                   batch_size: int) -> torch.Tensor:
    """KV index lists of the planned requests, in plan order (the whole list
    when every request is planned)."""
    if len(segments) == batch_size and all(s.batch_index == i for i, s in enumerate(segments)):
        return kv_indices.contiguous()
    return _gather(kv_indices, [(s.kv_source_start, s.kv_len) for s in segments]).contiguous()
