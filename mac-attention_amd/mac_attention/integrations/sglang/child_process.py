"""Hooks in SGLang's scheduler processes.

SGLang runs the model in scheduler processes it starts itself (spawned, so
they do not inherit the parent's wrapped methods).  This module's entry
point stands in for ``run_scheduler_process``: it installs the hooks in the
child, then runs SGLang's own function.  ``install_child_wrappers`` points the
launch sites at it.  Reference: child_process.py:1-21 and
hook_installer.py:313-372 (the same launch sites).
"""

from __future__ import annotations

import inspect
import os
from importlib import import_module
from typing import Any, Callable


def run_scheduler_process_with_mac_hooks(*args: Any, **kwargs: Any) -> Any:
    """Scheduler process entry point: hooks first, then SGLang's scheduler."""
    from .hook_installer import install_hooks

    newly = install_hooks()
    if os.environ.get("MAC_ATTENTION_SGLANG_DEBUG") == "1":
        print(f"[MAC-Attention] scheduler process: {len(newly)} hook(s) installed", flush=True)
    scheduler = import_module("sglang.srt.managers.scheduler")
    return scheduler.run_scheduler_process(*args, **kwargs)


# (module, attribute) pairs that hold SGLang's scheduler entry point, and
# functions whose keyword default names it
_ENTRY_ATTRS = (
    ("sglang.srt.entrypoints.engine", "run_scheduler_process"),
    ("sglang.srt.entrypoints.http_server", "run_scheduler_process"),
    ("sglang.srt.managers.data_parallel_controller", "run_scheduler_process"),
)
_ENGINE_CLASS = ("sglang.srt.entrypoints.engine", "Engine", "run_scheduler_process_func")
_DEFAULT_ARGS = (
    ("sglang.srt.entrypoints.http_server", "launch_server", "run_scheduler_process_func"),
    ("sglang.srt.managers.data_parallel_controller", "run_data_parallel_controller_process",
     "run_scheduler_process_func"),
)


def _swap_default(fn: Callable[..., Any], name: str, value: Any) -> bool:
    """Replace the default of keyword parameter ``name`` of ``fn``."""
    try:
        params = list(inspect.signature(fn).parameters.values())
    except (TypeError, ValueError):
        return False
    defaults = list(fn.__defaults__ or ())
    positional = [p for p in params if p.kind in (p.POSITIONAL_ONLY, p.POSITIONAL_OR_KEYWORD)]
    first_default = len(positional) - len(defaults)
    for i, p in enumerate(positional):
        if p.name == name and i >= first_default:
            if defaults[i - first_default] is value:
                return False
            defaults[i - first_default] = value
            fn.__defaults__ = tuple(defaults)
            return True
    kw = dict(fn.__kwdefaults__ or {})
    if name in kw and kw[name] is not value:
        kw[name] = value
        fn.__kwdefaults__ = kw
        return True
    return False


def install_child_wrappers() -> tuple[str, ...]:
    """Point every launch site SGLang has at the hooked entry point; returns
    the sites changed.  Sites this SGLang does not have are skipped."""
    entry = run_scheduler_process_with_mac_hooks
    changed = []

    def module(name):
        try:
            return import_module(name)
        except ImportError:
            return None

    for mod_name, attr in _ENTRY_ATTRS:
        mod = module(mod_name)
        if mod is not None and hasattr(mod, attr) and getattr(mod, attr) is not entry:
            setattr(mod, attr, entry)
            changed.append(f"{mod_name}:{attr}")
    mod = module(_ENGINE_CLASS[0])
    cls = getattr(mod, _ENGINE_CLASS[1], None) if mod is not None else None
    if cls is not None and hasattr(cls, _ENGINE_CLASS[2]) and getattr(cls, _ENGINE_CLASS[2]) is not entry:
        setattr(cls, _ENGINE_CLASS[2], staticmethod(entry))
        changed.append(f"{_ENGINE_CLASS[0]}:{_ENGINE_CLASS[1]}.{_ENGINE_CLASS[2]}")
    for mod_name, fn_name, param in _DEFAULT_ARGS:
        mod = module(mod_name)
        fn = getattr(mod, fn_name, None) if mod is not None else None
        if fn is not None and _swap_default(fn, param, entry):
            changed.append(f"{mod_name}:{fn_name}.{param}")
    return tuple(changed)
