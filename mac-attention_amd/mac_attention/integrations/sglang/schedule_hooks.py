"""Scheduler-side marks: which prefill rows reach the MAC ring.

Reference: attention/src/mac_attention/integrations/sglang/schedule_hooks.py
(:8-24 the rule, :27-66 the four hooks).  The ring of a request holds its
last ``mac_lookback_tokens_left`` (M) positions, so of a prompt of length L
only positions ``[L - M, L)`` are ever stored; for an extend chunk covering
``[prefix_len, seq_len)`` the first row to keep is ``max(prefix_len, L - M)``,
or none (-1) when that lies past the chunk.  The marks travel
ScheduleBatch -> ModelWorkerBatch -> ForwardBatch as
``mac_prefill_cache_update_starts`` and feed ``prefill_suffix``.
"""

from __future__ import annotations

from typing import Any, Optional, Sequence

from .config import get_mac_config

MARKS_ATTR = "mac_prefill_cache_update_starts"


def ring_update_starts(prompt_lens: Sequence[int], prefix_lens: Sequence[int], seq_lens: Sequence[int],
                       capacity: int) -> list[int]:
    """First absolute position of each request's chunk that the ring keeps
    (-1: none).  ``prompt_lens`` are the full prompt lengths."""
    starts = []
    for prompt, prefix, seq in zip(prompt_lens, prefix_lens, seq_lens):
        first_kept = max(int(prefix), int(prompt) - capacity, 0)
        starts.append(first_kept if first_kept < int(seq) else -1)
    return starts


def _host_list(x: Any) -> list[int]:
    if hasattr(x, "detach"):
        x = x.detach().cpu().tolist()
    return [int(v) for v in x]


def _marks_for(batch: Any) -> Optional[list[int]]:
    config = get_mac_config()
    capacity = int(getattr(config, "mac_lookback_tokens_left", 0) or 0)
    if not config.enable_mac or capacity <= 0:
        return None
    if not (hasattr(batch, "prefix_lens") and hasattr(batch, "seq_lens") and hasattr(batch, "reqs")):
        return None
    prompts = [len(r.origin_input_ids) for r in batch.reqs]
    return ring_update_starts(prompts, _host_list(batch.prefix_lens), _host_list(batch.seq_lens), capacity)


def schedule_prepare_for_extend_after(result: Any, self: Any, *args: Any, **kwargs: Any) -> Any:
    """ScheduleBatch.prepare_for_extend: mark the new extend batch."""
    setattr(self, MARKS_ATTR, _marks_for(self))
    return result


def schedule_mix_with_running_after(result: Any, self: Any, running_batch: Any, *args: Any,
                                    **kwargs: Any) -> Any:
    """ScheduleBatch.mix_with_running: decode requests mixed into an extend
    batch write no ring rows from it."""
    marks = getattr(self, MARKS_ATTR, None)
    if marks is not None:
        marks.extend([-1] * int(running_batch.batch_size()))
    return result


def schedule_get_model_worker_batch_after(result: Any, self: Any, *args: Any, **kwargs: Any) -> Any:
    """ScheduleBatch.get_model_worker_batch: carry the marks along."""
    setattr(result, MARKS_ATTR, getattr(self, MARKS_ATTR, None))
    return result


def forward_batch_init_new_after(result: Any, cls: Any, batch: Any, model_runner: Any) -> Any:
    """ForwardBatch.init_new: carry the marks onto the forward batch."""
    setattr(result, MARKS_ATTR, getattr(batch, MARKS_ATTR, None))
    return result
