"""Installs MAC-Attention into SGLang by wrapping SGLang methods in place.

Interface of attention/src/mac_attention/integrations/sglang/hook_installer.py
of the reference (HookSpec :18-23, targets :46-243, resolution and wrapping
:246-330): a hook spec names ``"module:Class.attr"``, a hook callable and its
kind -- ``around`` hooks receive the original function first, ``after`` hooks
receive its result first and may replace it.  Wrapped functions carry
``__mac_attention_hooked__`` so installing twice is a no-op.

This build hooks what the gfx950 decode path needs: the server-args plumbing
(settings, validation) and FlashInferAttnBackend.forward_decode, which tries
the fused MAC step before the backend's own decode.  The model-side hooks of
the reference (RoPE preservation inside LlamaAttention, the prefill ring
update inside forward_extend, scheduler marks) call the functions of
``persistent`` the same way and are left to the serving integration.
"""

from __future__ import annotations

from dataclasses import dataclass
from functools import wraps
from importlib import import_module
from typing import Any, Callable, Iterable, Literal

HookKind = Literal["around", "after"]

_INSTALLED: list[str] = []


@dataclass(frozen=True)
class HookSpec:
    target: str
    hook: Callable[..., Any]
    kind: HookKind
    optional: bool = False


def iter_hook_specs() -> Iterable[HookSpec]:
    from .persistent import flashinfer_forward_decode_around
    from .plugin import (server_args_add_cli_args_around, server_args_from_cli_args_after,
                         server_args_post_init_after)

    yield HookSpec("sglang.srt.server_args:ServerArgs.add_cli_args", server_args_add_cli_args_around, "around")
    yield HookSpec("sglang.srt.server_args:ServerArgs.from_cli_args", server_args_from_cli_args_after, "after")
    yield HookSpec("sglang.srt.server_args:ServerArgs.__post_init__", server_args_post_init_after, "after")
    yield HookSpec("sglang.srt.layers.attention.flashinfer_backend:FlashInferAttnBackend.forward_decode",
                   flashinfer_forward_decode_around, "around")


def _resolve_target(target: str) -> tuple[Any, str]:
    module_name, qualname = target.split(":", 1)
    obj = import_module(module_name)
    *owners, attr = qualname.split(".")
    for name in owners:
        obj = getattr(obj, name)
    return obj, attr


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


def install_hooks(strict: bool = True, specs: Iterable[HookSpec] | None = None) -> tuple[str, ...]:
    """Installs every spec (default: ``iter_hook_specs()``).  With
    ``strict`` a target that cannot be resolved raises; otherwise it is
    skipped.  Returns the targets wrapped by this call."""
    done = []
    for spec in (iter_hook_specs() if specs is None else specs):
        try:
            if install_hook(spec):
                done.append(spec.target)
        except (ImportError, AttributeError):
            if strict and not spec.optional:
                raise
    _INSTALLED.extend(done)
    return tuple(done)


def is_installed() -> bool:
    return bool(_INSTALLED)
