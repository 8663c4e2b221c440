"""MAC-Attention settings for SGLang serving.

Same settings, defaults, environment variables, JSON transport variable and
command-line flags as attention/src/mac_attention/integrations/sglang/
config.py of the reference (fields :118-154, env aliases :14-45, flags
:204-370, validation :373-414), so a deployment configured for the reference
keeps its configuration.  Here every setting is declared once in ``_SPECS``
(type, default, env aliases, flag help) and the dataclass, the parsers and the
argparse flags are derived from that table.
"""

from __future__ import annotations

import argparse
import json
import os
from dataclasses import asdict, dataclass, field, make_dataclass
from typing import Any, Callable, Optional

MAC_CONFIG_ENV = "MAC_ATTENTION_SGLANG_CONFIG"

_TRUE = {"1", "true", "t", "yes", "y", "on"}
_FALSE = {"0", "false", "f", "no", "n", "off"}


def _to_bool(value: Any) -> bool:
    if isinstance(value, bool):
        return value
    if value is None:
        return False
    if isinstance(value, (int, float)):
        return bool(value)
    text = str(value).strip().lower()
    if text in _TRUE:
        return True
    if text in _FALSE:
        return False
    raise ValueError(f"Cannot parse boolean value: {value!r}")


_BENCH_MODES = ("off", "synthetic_head", "synthetic-head", "synthetic_group", "synthetic-group")


@dataclass(frozen=True)
class _Spec:
    name: str
    parse: Callable[[Any], Any]
    default: Any
    env: tuple[str, ...] = ()
    flag_help: Optional[str] = None       # None: no command-line flag
    choices: Optional[tuple[str, ...]] = None


def _env_name(name: str) -> tuple[str, ...]:
    return (name.upper(),)


# One row per setting (reference config.py:118-154 for names and defaults).
_SPECS: tuple[_Spec, ...] = (
    _Spec("enable_mac", _to_bool, False, ("MAC_ATTENTION_ENABLE", "MAC_ENABLE", "ENABLE_MAC"),
          "Enable MAC-Attention for supported SGLang models and backends."),
    _Spec("mac_threshold", float, 0.45, _env_name("mac_threshold"), "MAC query match threshold."),
    _Spec("mac_lookback_tokens_left", int, 512, _env_name("mac_lookback_tokens_left"),
          "Number of ring-cache rows kept per request for MAC matching."),
    _Spec("mac_lookback_tokens_right", int, 0, _env_name("mac_lookback_tokens_right"),
          "Reserved for right-side MAC matching; current SGLang hook supports 0."),
    _Spec("mac_gen_min_limit", int, 2048, _env_name("mac_gen_min_limit"),
          "Minimum cached context length before MAC decode matching is attempted."),
    _Spec("mac_semantic_pos_ahead", int, 256, _env_name("mac_semantic_pos_ahead"),
          "Rectification band size used by fused MAC decode cache writes."),
    _Spec("mac_front_sink_tokens", int, 0, _env_name("mac_front_sink_tokens"),
          "Number of front tokens additionally recomputed when MAC decode hits."),
    _Spec("mac_profile", int, 0, _env_name("mac_profile"), "Enable lightweight MAC hit/skipped-token profiling."),
    _Spec("mac_profile_path", str, "", _env_name("mac_profile_path"), "Directory for MAC profiling logs."),
    _Spec("mac_disable_cuda_graph", _to_bool, True, _env_name("mac_disable_cuda_graph"),
          "Disable SGLang CUDA graph when MAC is enabled."),
    _Spec("mac_force_paged_prefill", _to_bool, True, _env_name("mac_force_paged_prefill"),
          "Force paged prefill so MAC can cache long prompts."),
    _Spec("mac_persistent_coop", _to_bool, True, _env_name("mac_persistent_coop")),
    _Spec("mac_persistent_max_context", int, 131072, _env_name("mac_persistent_max_context"),
          "Maximum context length supported by persistent MAC decode workspace."),
    _Spec("mac_persistent_fast_window", int, 8192, _env_name("mac_persistent_fast_window")),
    _Spec("mac_persistent_tile_tokens", int, 32, _env_name("mac_persistent_tile_tokens"),
          "Logical token tile size for persistent MAC decode."),
    _Spec("mac_persistent_stage_tokens", int, 64, _env_name("mac_persistent_stage_tokens"),
          "K/V staging tile size for persistent MAC decode."),
    _Spec("mac_persistent_match_tile_slots", int, 32, _env_name("mac_persistent_match_tile_slots"),
          "Ring-cache slots scanned by each persistent MAC match CTA."),
    _Spec("mac_persistent_debug", int, 0, _env_name("mac_persistent_debug")),
    _Spec("mac_persistent_partial_fp32", _to_bool, True, _env_name("mac_persistent_partial_fp32")),
    _Spec("mac_persistent_cache_layout", str, "slot_major", _env_name("mac_persistent_cache_layout")),
    _Spec("mac_persistent_candidate_mode", str, "last_M", _env_name("mac_persistent_candidate_mode"),
          "Candidate-set mode for persistent MAC matching.", ("last_M", "exclude_recent_right")),
    _Spec("mac_persistent_fast_math", _to_bool, True, _env_name("mac_persistent_fast_math")),
    _Spec("mac_bench_mode", str, "off", _env_name("mac_bench_mode"),
          "Latency-only synthetic MAC benchmark mode. Keeps the SGLang decode workflow but "
          "overrides persistent MAC hit/match metadata in-kernel.", _BENCH_MODES),
    _Spec("mac_bench_hit_rate", float, 1.0, _env_name("mac_bench_hit_rate"),
          "Mean per-query-head hit probability used by synthetic MAC benchmark mode."),
    _Spec("mac_bench_hit_rate_std", float, 0.0, _env_name("mac_bench_hit_rate_std"),
          "Per-token/layer standard deviation applied to synthetic MAC hit probability."),
    _Spec("mac_bench_skip_ratio", float, -1.0, _env_name("mac_bench_skip_ratio"),
          "Target skipped-prefix ratio for synthetic MAC hits. Use a negative value to instead "
          "control match lag directly."),
    _Spec("mac_bench_skip_ratio_std", float, 0.0, _env_name("mac_bench_skip_ratio_std"),
          "Per-token/layer standard deviation for synthetic skipped-prefix ratio."),
    _Spec("mac_bench_match_lag_mean", float, 64.0, _env_name("mac_bench_match_lag_mean"),
          "Mean lag in tokens between current decode position and synthetic match position, "
          "used when --mac-bench-skip-ratio is negative."),
    _Spec("mac_bench_match_lag_std", float, 0.0, _env_name("mac_bench_match_lag_std"),
          "Standard deviation of synthetic match lag in tokens."),
    _Spec("mac_bench_seed", int, 1, _env_name("mac_bench_seed"),
          "Deterministic seed for synthetic MAC benchmark hit/lag generation."),
)
_BY_NAME = {s.name: s for s in _SPECS}


def _normalize(values: dict[str, Any]) -> dict[str, Any]:
    return {name: _BY_NAME[name].parse(value) for name, value in values.items()}


def _env_overrides() -> dict[str, Any]:
    """First alias present in the environment wins, per setting."""
    found = {}
    for spec in _SPECS:
        for env in spec.env:
            if env in os.environ:
                found[spec.name] = os.environ[env]
                break
    return found


def _env_state() -> tuple[tuple[str, Optional[str]], ...]:
    names = {MAC_CONFIG_ENV}
    for spec in _SPECS:
        names.update(spec.env)
    return tuple((n, os.environ.get(n)) for n in sorted(names))


class _ConfigMethods:
    @classmethod
    def defaults(cls) -> dict[str, Any]:
        return {s.name: s.default for s in _SPECS}

    @classmethod
    def from_namespace(cls, args: argparse.Namespace):
        values = {s.name: getattr(args, s.name, s.default) for s in _SPECS}
        values.update(_env_overrides())
        return cls(**_normalize(values))

    @classmethod
    def from_env(cls):
        """Settings from the JSON transport variable and the per-setting
        variables (which win); ``None`` when neither is present."""
        values = cls.defaults()
        found = False
        raw = os.environ.get(MAC_CONFIG_ENV)
        if raw:
            try:
                data = json.loads(raw)
            except json.JSONDecodeError:
                data = {}
            values.update({k: v for k, v in data.items() if k in values})
            found = True
        env = _env_overrides()
        values.update(env)
        if not (found or env):
            return None
        return cls(**_normalize(values))

    @classmethod
    def from_server_args(cls, server_args: Any):
        env_cfg = cls.from_env()
        values = asdict(env_cfg) if env_cfg is not None else cls.defaults()
        if server_args is not None:
            for name in values:
                if hasattr(server_args, name):
                    values[name] = getattr(server_args, name)
        values.update(_env_overrides())
        return cls(**_normalize(values))

    def install_env(self) -> None:
        os.environ[MAC_CONFIG_ENV] = json.dumps(asdict(self), sort_keys=True)


MacSGLangConfig = make_dataclass(
    "MacSGLangConfig",
    [(s.name, type(s.default), field(default=s.default)) for s in _SPECS],
    bases=(_ConfigMethods,),
    namespace={"__module__": __name__,
               "__doc__": "MAC-Attention serving settings (reference config.py:118-188)."},
)


def add_cli_args(parser: argparse.ArgumentParser) -> None:
    """Adds ``--mac-*`` flags (reference config.py:204-370); flags already on
    the parser are left alone."""
    existing = getattr(parser, "_option_string_actions", {})
    for spec in _SPECS:
        if spec.flag_help is None:
            continue
        flag = "--" + spec.name.replace("_", "-")
        if flag in existing:
            continue
        kwargs: dict[str, Any] = dict(default=spec.default, help=spec.flag_help)
        if spec.parse is _to_bool:
            kwargs.update(type=_to_bool, nargs="?", const=True)
        else:
            kwargs.update(type=spec.parse)
        if spec.choices:
            kwargs["choices"] = spec.choices
        parser.add_argument(flag, **kwargs)


_cache: dict[str, Any] = {"config": None, "key": None}


def install_on_server_args(server_args: Any, config) -> Any:
    """Copies the settings onto the server args, publishes them to child
    processes through the environment and validates an enabled configuration
    (reference config.py:373-414)."""
    if server_args is not None:
        for name, value in asdict(config).items():
            setattr(server_args, name, value)
    config.install_env()
    _cache["config"], _cache["key"] = config, (id(server_args), _env_state())
    if not config.enable_mac:
        return server_args
    if config.mac_lookback_tokens_left <= 0:
        raise ValueError("MAC-Attention requires MAC_LOOKBACK_TOKENS_LEFT > 0")
    if config.mac_lookback_tokens_right != 0:
        raise ValueError("The SGLang MAC plugin currently supports MAC_LOOKBACK_TOKENS_RIGHT=0")
    if str(config.mac_bench_mode).strip().lower() not in _BENCH_MODES:
        raise ValueError("MAC_BENCH_MODE must be off, synthetic_head, or synthetic_group")
    for attr, what in (("decode_attention_backend", "decode"), ("prefill_attention_backend", "prefill")):
        backend = getattr(server_args, attr, None)
        if backend not in (None, "flashinfer"):
            raise ValueError(f"MAC-Attention requires FlashInfer {what} attention")
    if server_args is not None:
        if getattr(server_args, "attention_backend", None) != "flashinfer":
            setattr(server_args, "attention_backend", "flashinfer")
        if config.mac_disable_cuda_graph:
            for attr in ("disable_cuda_graph", "disable_piecewise_cuda_graph"):
                if hasattr(server_args, attr):
                    setattr(server_args, attr, True)
    return server_args


def get_mac_config(server_args: Any = None):
    """Settings for ``server_args`` (SGLang's global server args when None),
    recomputed whenever a MAC environment variable changes."""
    if server_args is None:
        try:
            from sglang.srt.server_args import get_global_server_args

            server_args = get_global_server_args()
        except Exception:
            server_args = None
    key = (id(server_args), _env_state())
    if _cache["config"] is not None and _cache["key"] == key:
        return _cache["config"]
    config = MacSGLangConfig.from_server_args(server_args)
    _cache["config"], _cache["key"] = config, key
    return config


def install_env_config(server_args: Any = None):
    """Resolve the settings and publish them in ``MAC_ATTENTION_SGLANG_CONFIG``
    (reference config.py:449-454)."""
    config = MacSGLangConfig.from_server_args(server_args)
    install_on_server_args(server_args, config)
    return config
