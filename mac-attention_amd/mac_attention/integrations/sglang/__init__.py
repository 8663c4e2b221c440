"""SGLang integration for MAC-Attention on MI355X.

Mirrors attention/src/mac_attention/integrations/sglang/__init__.py of the
reference: ``install_hooks`` / ``is_installed`` are imported lazily so that the
kernel bridge can be used without SGLang installed.
"""

__all__ = ["install_hooks", "is_installed"]


def __getattr__(name):
    if name in __all__:
        from . import hook_installer

        return getattr(hook_installer, name)
    raise AttributeError(name)
