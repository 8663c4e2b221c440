"""SGLang plugin entry point (``sglang.srt.plugins`` entry point
``mac_attention = mac_attention.integrations.sglang.plugin:register_plugin``)
and the server-args hooks; reference plugin.py:1-69."""

from __future__ import annotations

import os
from typing import Any

from .config import MacSGLangConfig, add_cli_args, get_mac_config, install_on_server_args


def _env_flag(name: str, default: str = "0") -> bool:
    return os.environ.get(name, default).strip().lower() in {"1", "true", "yes", "on"}


def server_args_add_cli_args_around(original_fn: Any, parser: Any) -> Any:
    """SGLang's flags, plus the ``--mac-*`` flags only when
    MAC_ATTENTION_EXPOSE_CLI_ARGS is set (settings normally come from the
    environment)."""
    result = original_fn(parser)
    if _env_flag("MAC_ATTENTION_EXPOSE_CLI_ARGS"):
        add_cli_args(parser)
    return result


def server_args_from_cli_args_after(result: Any, cls: Any, args: Any) -> Any:
    return install_on_server_args(result, MacSGLangConfig.from_namespace(args))


def server_args_post_init_after(result: Any, self: Any) -> Any:
    config = get_mac_config(self)
    if config.enable_mac:
        install_on_server_args(self, config)
    return result


def register_plugin() -> None:
    """Registers the hooks with SGLang's hook registry when it has one, else
    wraps the targets directly (MAC_ATTENTION_SGLANG_STRICT, default 1,
    makes a missing target an error)."""
    strict = _env_flag("MAC_ATTENTION_SGLANG_STRICT", "1")
    from .hook_installer import _resolve_target, install_hooks, is_installed, iter_hook_specs

    try:
        from sglang.srt.plugins.hook_registry import HookRegistry, HookType
    except ModuleNotFoundError as exc:
        if exc.name and exc.name.startswith("sglang.srt.plugins"):
            install_hooks(strict=strict)
            return
        raise
    if is_installed():  # already wrapped directly: registering again would wrap twice
        return
    kinds = {"around": HookType.AROUND, "after": HookType.AFTER}
    for spec in iter_hook_specs():
        if spec.optional:
            try:
                owner, attr = _resolve_target(spec.target)
            except Exception:
                continue
            if not hasattr(owner, attr):
                continue
        HookRegistry.register(spec.target, spec.hook, kinds[spec.kind])
