"""Installs MAC-Attention into SGLang by wrapping SGLang methods in place.

Interface of attention/src/mac_attention/integrations/sglang/hook_installer.py
of the reference (HookSpec :18-23, targets :46-243, resolution and wrapping
:246-330, scheduler-process launch sites :313-372): a hook spec names
``"module:Class.attr"``, a hook callable and its kind -- ``around`` hooks
receive the original function first, ``after`` hooks receive its result
first and may replace it.  Wrapped functions carry ``__mac_attention_hooked__``
so installing twice is a no-op.

Targets, by group:
  * server arguments: the MAC settings and flags (plugin.py);
  * scheduler: which prefill rows reach the ring (schedule_hooks.py);
  * models: the model forward prepares the batch state once; LlamaAttention
    and the Qwen2 / Qwen3 MoE attentions keep their pre-RoPE queries and
    hand the layer's MAC state to the attention backend (model_hooks.py; the
    Qwen classes are optional);
  * FlashInfer backend: settings at construction, the ring marks kept on the
    backend (init_forward_metadata), the ring update after each prefill
    chunk (forward_extend) and the fused MAC decode step (forward_decode);
  * the ROCm backends (AiterAttnBackend, TritonAttnBackend; optional): the
    same four targets, with the ring update computing the kept rows' full
    prefill state itself, since these backends return no lse.
  * decode graphs (FlashInfer and ROCm backends, optional): during capture
    each layer records which decode path it captured; a replay of a graph
    whose every layer is the MAC step skips the backend's replay metadata
    (flashinfer_hooks.py:660-700, :835-899).
Profiling-only and CUDA-graph-trace hooks of the reference are not part of
this build, nor the wait for side-stream ring updates before a graph
replay: the ring update here runs on the compute stream, in order with the
replay.
"""

from __future__ import annotations

from dataclasses import dataclass
from functools import wraps
from importlib import import_module
from typing import Any, Callable, Iterable, Iterator, Literal

HookKind = Literal["around", "after"]

_INSTALLED: list[str] = []

_ATTN_CLASSES = (
    ("sglang.srt.models.llama", "LlamaAttention", False),
    ("sglang.srt.models.qwen2_moe", "Qwen2MoeAttention", True),
    ("sglang.srt.models.qwen3_moe", "Qwen3MoeAttention", True),
)
_MODEL_CLASSES = (
    ("sglang.srt.models.llama", "LlamaModel", False),
    ("sglang.srt.models.qwen2_moe", "Qwen2MoeModel", True),
    ("sglang.srt.models.qwen3_moe", "Qwen3MoeModel", True),
)
_FLASHINFER = "sglang.srt.layers.attention.flashinfer_backend:FlashInferAttnBackend"
# the attention backends SGLang runs on ROCm (optional: an SGLang build has
# the ones its platform supports)
_ROCM_BACKENDS = (
    "sglang.srt.layers.attention.aiter_backend:AiterAttnBackend",
    "sglang.srt.layers.attention.triton_backend:TritonAttnBackend",
)


@dataclass(frozen=True)
class HookSpec:
    target: str
    hook: Callable[..., Any]
    kind: HookKind
    optional: bool = False


def iter_hook_specs() -> Iterable[HookSpec]:
    from . import model_hooks, schedule_hooks
    from .persistent import (flashinfer_forward_decode_around, init_forward_metadata_capture_cuda_graph_around,
                             init_forward_metadata_replay_cuda_graph_around)
    from .plugin import (server_args_add_cli_args_around, server_args_from_cli_args_after,
                         server_args_post_init_after)

    server = "sglang.srt.server_args:ServerArgs"
    yield HookSpec(f"{server}.add_cli_args", server_args_add_cli_args_around, "around")
    yield HookSpec(f"{server}.from_cli_args", server_args_from_cli_args_after, "after")
    yield HookSpec(f"{server}.__post_init__", server_args_post_init_after, "after")

    sched = "sglang.srt.managers.schedule_batch:ScheduleBatch"
    yield HookSpec(f"{sched}.prepare_for_extend", schedule_hooks.schedule_prepare_for_extend_after, "after")
    yield HookSpec(f"{sched}.mix_with_running", schedule_hooks.schedule_mix_with_running_after, "after")
    yield HookSpec(f"{sched}.get_model_worker_batch", schedule_hooks.schedule_get_model_worker_batch_after,
                   "after", optional=True)
    yield HookSpec("sglang.srt.model_executor.forward_batch_info:ForwardBatch.init_new",
                   schedule_hooks.forward_batch_init_new_after, "after")

    for module, cls, optional in _ATTN_CLASSES:
        yield HookSpec(f"{module}:{cls}.__init__", model_hooks.attention_init_after, "after", optional)
        yield HookSpec(f"{module}:{cls}.forward", model_hooks.attention_forward_around, "around", optional)
    for module, cls, optional in _MODEL_CLASSES:
        yield HookSpec(f"{module}:{cls}.forward", model_hooks.model_forward_around, "around", optional)

    yield HookSpec(f"{_FLASHINFER}.__init__", model_hooks.flashinfer_backend_init_after, "after")
    yield HookSpec(f"{_FLASHINFER}.init_forward_metadata", model_hooks.flashinfer_init_forward_metadata_around,
                   "around")
    yield HookSpec(f"{_FLASHINFER}.forward_extend", model_hooks.flashinfer_forward_extend_around, "around")
    yield HookSpec(f"{_FLASHINFER}.forward_decode", flashinfer_forward_decode_around, "around")

    for backend in _ROCM_BACKENDS:
        yield HookSpec(f"{backend}.__init__", model_hooks.flashinfer_backend_init_after, "after", True)
        yield HookSpec(f"{backend}.init_forward_metadata", model_hooks.flashinfer_init_forward_metadata_around,
                       "around", True)
        yield HookSpec(f"{backend}.forward_extend", model_hooks.rocm_forward_extend_around, "around", True)
        yield HookSpec(f"{backend}.forward_decode", flashinfer_forward_decode_around, "around", True)

    # decode graphs: skip the backend's replay metadata when every layer
    # captured the MAC step (optional: SGLang builds without graph support)
    for backend in (_FLASHINFER, *_ROCM_BACKENDS):
        yield HookSpec(f"{backend}.init_forward_metadata_capture_cuda_graph",
                       init_forward_metadata_capture_cuda_graph_around, "around", True)
        yield HookSpec(f"{backend}.init_forward_metadata_replay_cuda_graph",
                       init_forward_metadata_replay_cuda_graph_around, "around", True)


def _resolve_target(target: str) -> tuple[Any, str]:
    module_name, qualname = target.split(":", 1)
    obj = import_module(module_name)
    *owners, attr = qualname.split(".")
    for name in owners:
        obj = getattr(obj, name)
    return obj, attr


def resolvable_specs(specs: Iterable[HookSpec] | None = None) -> Iterator[HookSpec]:
    """The specs to register: every required one, and the optional ones whose
    target this SGLang has."""
    for spec in (iter_hook_specs() if specs is None else specs):
        if spec.optional:
            try:
                owner, attr = _resolve_target(spec.target)
            except (ImportError, AttributeError):
                continue
            if not hasattr(owner, attr):
                continue
        yield spec


def _wrap(spec: HookSpec, original: Callable[..., Any]) -> Callable[..., Any]:
    hook, around = spec.hook, spec.kind == "around"

    @wraps(original)
    def wrapped(*args: Any, **kwargs: Any) -> Any:
        if around:
            return hook(original, *args, **kwargs)
        result = original(*args, **kwargs)
        replacement = hook(result, *args, **kwargs)
        return result if replacement is None else replacement

    wrapped.__mac_attention_hooked__ = True
    wrapped.__mac_attention_hook_target__ = spec.target
    wrapped.__mac_attention_hook_kind__ = spec.kind
    wrapped.__mac_attention_original__ = original
    return wrapped


def install_hook(spec: HookSpec) -> bool:
    """Wraps one target; False when it is already wrapped or (optional
    specs) missing.  classmethod/staticmethod descriptors keep their kind."""
    owner, attr = _resolve_target(spec.target)
    raw = owner.__dict__.get(attr, None) if hasattr(owner, "__dict__") else None
    if raw is None:
        raw = getattr(owner, attr, None)
    if raw is None:
        if spec.optional:
            return False
        raise AttributeError(f"{owner!r} has no attribute {attr!r}")
    fn = raw.__func__ if isinstance(raw, (classmethod, staticmethod)) else raw
    if getattr(fn, "__mac_attention_hooked__", False):
        return False
    wrapped = _wrap(spec, fn)
    if isinstance(raw, classmethod):
        wrapped = classmethod(wrapped)
    elif isinstance(raw, staticmethod):
        wrapped = staticmethod(wrapped)
    setattr(owner, attr, wrapped)
    return True


def install_hooks(strict: bool = True, specs: Iterable[HookSpec] | None = None,
                  child_processes: bool = True) -> tuple[str, ...]:
    """Installs every spec (default: ``iter_hook_specs()``).  With
    ``strict`` a target that cannot be resolved raises; otherwise it is
    skipped.  ``child_processes``: also point SGLang's scheduler-process
    launch sites at an entry point that installs the hooks in the child
    (sites this SGLang lacks are skipped).  Returns what this call wrapped."""
    done = []
    for spec in (iter_hook_specs() if specs is None else specs):
        try:
            if install_hook(spec):
                done.append(spec.target)
        except (ImportError, AttributeError):
            if strict and not spec.optional:
                raise
    if child_processes:
        from .child_process import install_child_wrappers

        done.extend(install_child_wrappers())
    _INSTALLED.extend(done)
    return tuple(done)


def is_installed() -> bool:
    return bool(_INSTALLED)
