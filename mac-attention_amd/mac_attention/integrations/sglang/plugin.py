"""SGLang plugin entry point and the server-arguments hooks.

SGLang loads ``register_plugin`` through the ``sglang.srt.plugins`` entry
point group (``mac_attention = mac_attention.integrations.sglang.plugin:
register_plugin``, declared in the repository's pyproject.toml; reference
pyproject.toml:27-28 and plugin.py:1-69 for the behaviour).  An SGLang with a
hook registry gets every hook of ``hook_installer`` registered with it; an
older one gets the methods wrapped in place.  Settings come from the
environment (``config``); the ``--mac-*`` flags are added to SGLang's parser
only when MAC_ATTENTION_EXPOSE_CLI_ARGS is set.
"""

from __future__ import annotations

import os
from importlib import import_module
from typing import Any, Optional

from . import hook_installer
from .config import MacSGLangConfig, add_cli_args, get_mac_config, install_on_server_args


def _flag(name: str, default: bool) -> bool:
    """An on/off switch: unset gives ``default``; "1", "true", "yes" and "on"
    (any case) turn it on, anything else off, as the reference reads them."""
    raw = os.environ.get(name)
    return default if raw is None else raw.strip().lower() in {"1", "true", "yes", "on"}


# ------------------------------------------------------- server arguments ----


def server_args_add_cli_args_around(original_fn: Any, parser: Any) -> Any:
    """ServerArgs.add_cli_args: SGLang's flags, then the MAC flags if exposed."""
    parsed = original_fn(parser)
    if _flag("MAC_ATTENTION_EXPOSE_CLI_ARGS", False):
        add_cli_args(parser)
    return parsed


def server_args_from_cli_args_after(result: Any, cls: Any, args: Any) -> Any:
    """ServerArgs.from_cli_args: settings from the parsed flags."""
    return install_on_server_args(result, MacSGLangConfig.from_namespace(args))


def server_args_post_init_after(result: Any, self: Any) -> Any:
    """ServerArgs.__post_init__: an enabled configuration is validated and
    applied to the server arguments (backend selection, limits)."""
    config = get_mac_config(self)
    if config.enable_mac:
        install_on_server_args(self, config)
    return result


# --------------------------------------------------------------- plugin ----


def _hook_registry() -> Optional[tuple[Any, Any]]:
    """(HookRegistry, HookType) of an SGLang that has a plugin hook registry,
    else None.  Only the absence of that module means "no registry"; any
    other import failure is SGLang's and is raised."""
    try:
        module = import_module("sglang.srt.plugins.hook_registry")
    except ModuleNotFoundError as exc:
        if exc.name is not None and (exc.name == "sglang" or exc.name.startswith("sglang.srt.plugins")):
            return None
        raise
    return module.HookRegistry, module.HookType


def register_plugin() -> None:
    """Entry point SGLang calls at startup.  MAC_ATTENTION_SGLANG_STRICT
    (default on) makes a required target SGLang lacks an error."""
    strict = _flag("MAC_ATTENTION_SGLANG_STRICT", True)
    registry = _hook_registry()
    if registry is None:
        hook_installer.install_hooks(strict=strict)
        return
    if hook_installer.is_installed():
        # a launcher already wrapped the methods in place; registering the
        # same hooks would wrap them a second time
        return
    hook_registry, hook_type = registry
    for spec in hook_installer.resolvable_specs():
        hook_registry.register(spec.target, spec.hook, getattr(hook_type, spec.kind.upper()))
