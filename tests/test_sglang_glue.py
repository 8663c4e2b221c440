"""SGLang glue on the CPU: settings, plugin flags, pre-RoPE query
preservation, the prefill suffix plan, the hook installer and the gates of
the persistent decode step (no kernel call is reached here).

Scenarios follow the reference's attention/tests/test_sglang_plugin_config.py
and test_sglang_q_preserve.py; SGLang itself is not installed, so its classes
are replaced by small stand-ins.
"""

import argparse
import json
import os
import sys
import types

import pytest
import torch

from helpers import PKG  # noqa: F401  (puts the package on sys.path)
from mac_attention.integrations.sglang import hook_installer, persistent
from mac_attention.integrations.sglang.config import (MAC_CONFIG_ENV, MacSGLangConfig, get_mac_config,
                                                      install_env_config)
from mac_attention.integrations.sglang.plugin import server_args_add_cli_args_around
from mac_attention.integrations.sglang.prefill_suffix import (build_prefill_suffix_plan,
                                                              compact_kv_indices_by_segments)


@pytest.fixture(autouse=True)
def clean_env():
    """Each test starts without MAC variables; whatever a test (or the code
    under test, which publishes its JSON) sets is removed afterwards."""
    saved = {k: v for k, v in os.environ.items() if k.startswith(("MAC_", "ENABLE_MAC"))}
    for k in saved:
        del os.environ[k]
    yield
    for k in [k for k in os.environ if k.startswith(("MAC_", "ENABLE_MAC"))]:
        del os.environ[k]
    os.environ.update(saved)


# ------------------------------------------------------------- settings ----


def test_env_enable_alone_gives_defaults(monkeypatch):
    monkeypatch.setenv("MAC_ATTENTION_ENABLE", "1")
    cfg = MacSGLangConfig.from_env()
    assert cfg.enable_mac and cfg.mac_threshold == 0.45
    assert (cfg.mac_lookback_tokens_left, cfg.mac_lookback_tokens_right) == (512, 0)
    assert cfg.mac_semantic_pos_ahead == 256 and cfg.mac_persistent_tile_tokens == 32
    assert cfg.mac_persistent_partial_fp32 is True


def test_no_mac_environment_means_no_config():
    assert MacSGLangConfig.from_env() is None


def test_per_setting_variables_beat_json_transport(monkeypatch):
    monkeypatch.setenv(MAC_CONFIG_ENV, json.dumps({"enable_mac": False, "mac_threshold": 0.7,
                                                   "mac_persistent_tile_tokens": 64,
                                                   "mac_persistent_partial_fp32": False,
                                                   "unknown_key": 3}))
    monkeypatch.setenv("MAC_ENABLE", "yes")
    monkeypatch.setenv("MAC_THRESHOLD", "0.45")
    cfg = MacSGLangConfig.from_env()
    assert cfg.enable_mac and cfg.mac_threshold == 0.45
    assert cfg.mac_persistent_tile_tokens == 64 and cfg.mac_persistent_partial_fp32 is False


def test_install_env_config_publishes_json_for_children(monkeypatch):
    monkeypatch.setenv("MAC_ATTENTION_ENABLE", "1")
    monkeypatch.setenv("MAC_PERSISTENT_TILE_TOKENS", "32")
    cfg = install_env_config()
    child = json.loads(os.environ[MAC_CONFIG_ENV])
    assert cfg.enable_mac and child["enable_mac"] is True and child["mac_persistent_tile_tokens"] == 32


def test_get_mac_config_follows_environment_changes(monkeypatch):
    args = types.SimpleNamespace()
    monkeypatch.setenv("MAC_ATTENTION_ENABLE", "1")
    assert get_mac_config(args).enable_mac is True
    monkeypatch.setenv("MAC_ATTENTION_ENABLE", "0")
    assert get_mac_config(args).enable_mac is False


def test_enabled_config_validation_and_backend_selection(monkeypatch):
    monkeypatch.setenv("MAC_ATTENTION_ENABLE", "1")
    args = types.SimpleNamespace(attention_backend="triton", disable_cuda_graph=False)
    install_env_config(args)
    assert args.attention_backend == "flashinfer" and args.disable_cuda_graph is True
    monkeypatch.setenv("MAC_LOOKBACK_TOKENS_RIGHT", "4")
    with pytest.raises(ValueError, match="LOOKBACK_TOKENS_RIGHT=0"):
        install_env_config(types.SimpleNamespace())
    monkeypatch.delenv("MAC_LOOKBACK_TOKENS_RIGHT")
    monkeypatch.delenv(MAC_CONFIG_ENV)  # the failed install published right=4 for child processes
    with pytest.raises(ValueError, match="FlashInfer decode"):
        install_env_config(types.SimpleNamespace(decode_attention_backend="triton"))


def _sglang_flags(parser):
    parser.add_argument("--official-arg", default="ok")
    return parser


def test_mac_flags_hidden_by_default():
    parser = argparse.ArgumentParser()
    server_args_add_cli_args_around(_sglang_flags, parser)
    flags = set(parser._option_string_actions)
    assert "--official-arg" in flags and "--enable-mac" not in flags and "--mac-threshold" not in flags


def test_mac_flags_exposed_on_request(monkeypatch):
    monkeypatch.setenv("MAC_ATTENTION_EXPOSE_CLI_ARGS", "1")
    parser = argparse.ArgumentParser()
    server_args_add_cli_args_around(_sglang_flags, parser)
    ns = parser.parse_args(["--enable-mac", "--mac-threshold", "0.5", "--mac-bench-mode", "synthetic_group"])
    assert ns.enable_mac is True and ns.mac_threshold == 0.5 and ns.mac_bench_mode == "synthetic_group"
    cfg = MacSGLangConfig.from_namespace(ns)
    assert cfg.enable_mac and cfg.mac_threshold == 0.5


# ---------------------------------------------------- q preservation ----


def _meta(decode_buf=None):
    m = persistent.MacMetadata(num_heads=2, num_kv_heads=1, head_dim=4)
    m.decode_q_before_rope_buf = decode_buf
    return m


def _fb(starts, prefix, extend):
    return types.SimpleNamespace(mac_prefill_cache_update_starts=starts, extend_prefix_lens_cpu=prefix,
                                 extend_seq_lens_cpu=extend, batch_size=len(starts))


def test_decode_preserve_copies_into_the_decode_buffer():
    q = torch.arange(8, dtype=torch.float32).reshape(1, 8)
    want = q.reshape(1, 2, 4).clone()
    m = _meta(torch.empty((1, 2, 4)))
    persistent.preserve_q_before_rope(m, q, current_is_decode=True)
    q.add_(1000)
    torch.testing.assert_close(m.cur_q_before_rope, want)
    assert (m.cur_q_before_rope_local_start, m.cur_q_before_rope_local_len) == (0, 1)


def test_prefill_preserves_only_the_marked_rows():
    q = torch.arange(40, dtype=torch.float32).reshape(5, 8)
    want = q.reshape(5, 2, 4)[2:5].clone()
    m = _meta()
    persistent.preserve_q_before_rope(m, q, current_is_decode=False, forward_batch=_fb([6], [4], [5]))
    q.add_(1000)
    torch.testing.assert_close(m.cur_q_before_rope, want)
    assert (m.cur_q_before_rope_local_start, m.cur_q_before_rope_local_len) == (2, 3)


def test_prefill_without_marks_preserves_nothing():
    m = _meta()
    persistent.preserve_q_before_rope(m, torch.zeros(5, 8), current_is_decode=False,
                                      forward_batch=_fb([-1], [4], [5]))
    assert m.cur_q_before_rope is None
    assert (m.cur_q_before_rope_local_start, m.cur_q_before_rope_local_len) == (0, 0)


def test_multi_request_prefill_compacts_marked_rows():
    q = torch.arange(96, dtype=torch.float32).reshape(12, 8)
    v = q.reshape(12, 2, 4)
    want = torch.cat([v[6:9], v[11:12]]).clone()
    m = _meta()
    persistent.preserve_q_before_rope(m, q, current_is_decode=False,
                                      forward_batch=_fb([-1, 22, 32], [10, 20, 30], [4, 5, 3]))
    q.add_(1000)
    torch.testing.assert_close(m.cur_q_before_rope, want)
    assert (m.cur_q_before_rope_local_start, m.cur_q_before_rope_local_len) == (-1, 4)
    assert m.cur_q_before_rope_compacted


def test_graph_safe_prefill_keeps_the_tail_rows():
    m = _meta()
    m.prefill_q_before_rope_buf = torch.zeros(8, 2, 4)
    m.prefill_preserve_tail_tokens = 3
    q = torch.arange(40, dtype=torch.float32).reshape(5, 8)
    persistent.preserve_q_before_rope(m, q, current_is_decode=False, forward_batch=_fb([0], [0], [5]),
                                      graph_safe=True)
    torch.testing.assert_close(m.cur_q_before_rope, q.reshape(5, 2, 4)[2:])
    assert (m.cur_q_before_rope_local_start, m.cur_q_before_rope_local_len) == (2, 3)


# ------------------------------------------------------ suffix plan ----


def test_suffix_plan_vectors():
    plan = build_prefill_suffix_plan(_fb([-1, 15, 32, 0], [10, 20, 30, 7], [4, 5, 3, 2]), 4, 14)
    # request 1: mark inside its prefix -> whole chunk; request 3: mark 0 < prefix 7 -> whole chunk
    assert plan.req_indices == (1, 2, 3)
    assert plan.request_lengths == (20, 32, 7)
    assert plan.lens == (5, 1, 2) and plan.offsets == (0, 5, 6, 8) and plan.total_len == 8
    assert [s.source_start for s in plan.segments] == [4, 11, 12]
    assert plan.kv_offsets == (0, 25, 58, 67)
    kv = torch.arange(14 + 10 + 20 + 30 + 7)
    got = compact_kv_indices_by_segments(kv, plan.segments, batch_size=4)
    torch.testing.assert_close(got, torch.cat([kv[14:39], kv[39:72], kv[72:81]]))


def test_suffix_plan_needs_consistent_host_lengths():
    assert build_prefill_suffix_plan(types.SimpleNamespace(), 1, 5) is None
    assert build_prefill_suffix_plan(_fb([0], [0], [4]), 1, 5) is None  # lengths do not add up
    backend = types.SimpleNamespace(mac_prefill_cache_update_starts_current=[2],
                                    mac_extend_prefix_lens_cpu_current=[0],
                                    mac_extend_seq_lens_cpu_current=[5])
    plan = build_prefill_suffix_plan(types.SimpleNamespace(attn_backend=backend), 1, 5)
    assert plan.lens == (3,)
    assert build_prefill_suffix_plan(types.SimpleNamespace(attn_backend=backend), 1, 5,
                                     allow_backend_fallback=False) is None


# --------------------------------------------------------- hook installer ----


@pytest.fixture
def fake_module(monkeypatch):
    mod = types.ModuleType("fake_sglang_mod")

    class Backend:
        scale = 10

        def forward(self, x):
            return x + 1

        @classmethod
        def build(cls, x):
            return x * cls.scale

        @staticmethod
        def helper(x):
            return x - 1

    mod.Backend = Backend
    monkeypatch.setitem(sys.modules, "fake_sglang_mod", mod)
    return mod


def test_hooks_wrap_methods_classmethods_and_staticmethods(fake_module):
    calls = []

    def around(orig, self, x):
        calls.append("around")
        return orig(self, x) * 2

    def after(result, cls, x):
        calls.append("after")
        return result + 0.5

    def after_keep(result, x):
        return None  # keeps the original result

    specs = [hook_installer.HookSpec("fake_sglang_mod:Backend.forward", around, "around"),
             hook_installer.HookSpec("fake_sglang_mod:Backend.build", after, "after"),
             hook_installer.HookSpec("fake_sglang_mod:Backend.helper", after_keep, "after"),
             hook_installer.HookSpec("fake_sglang_mod:Backend.missing", after_keep, "after", optional=True)]
    done = hook_installer.install_hooks(specs=specs)
    assert len(done) == 3
    b = fake_module.Backend()
    assert b.forward(3) == 8 and fake_module.Backend.build(2) == 20.5 and b.helper(5) == 4
    assert isinstance(fake_module.Backend.__dict__["build"], classmethod)
    assert isinstance(fake_module.Backend.__dict__["helper"], staticmethod)
    assert hook_installer.install_hooks(specs=specs) == ()  # already wrapped
    assert b.forward(3) == 8 and calls == ["around", "after", "around"]
    assert hook_installer.is_installed()


def test_missing_targets_raise_only_in_strict_mode():
    spec = hook_installer.HookSpec("no_such_sglang_module:X.y", lambda *a: None, "after")
    with pytest.raises(ModuleNotFoundError):
        hook_installer.install_hooks(strict=True, specs=[spec])
    assert hook_installer.install_hooks(strict=False, specs=[spec]) == ()


def test_default_specs_need_sglang():
    targets = [s.target for s in hook_installer.iter_hook_specs()]
    assert "sglang.srt.layers.attention.flashinfer_backend:FlashInferAttnBackend.forward_decode" in targets
    with pytest.raises(ModuleNotFoundError):
        hook_installer.install_hooks(strict=True)


# ---------------------------------------------------- decode gates ----


def _decode_setup(**cfg_kw):
    cfg = MacSGLangConfig(enable_mac=True, **cfg_kw)
    m = persistent.MacMetadata(num_heads=8, num_kv_heads=2, head_dim=128)
    m.allocate(max_running=4, capacity=16, device="cpu")
    m.persistent_decode_ext = object()  # never reached: every case fails a gate first
    backend = types.SimpleNamespace(indices_updater_decode=types.SimpleNamespace(
        req_to_token=torch.zeros(4, 64, dtype=torch.int32)))
    fb = types.SimpleNamespace(batch_size=2)
    layer = types.SimpleNamespace(logit_cap=0, scaling=0.088, layer_id=0)
    q = torch.zeros(2, 8, 128, dtype=torch.bfloat16)
    kb = torch.zeros(10, 2, 128, dtype=torch.bfloat16)
    return cfg, m, backend, fb, layer, q, kb, torch.zeros(2, dtype=torch.int64)


@pytest.mark.parametrize("case", ["coop_off", "layout", "candidate", "dtype", "head_dim", "batch", "group",
                                  "logit_cap", "kv_scale", "r2t_dtype", "context", "not_ready"])
def test_persistent_decode_gates_fall_back(case):
    kw = {"coop_off": dict(mac_persistent_coop=False), "layout": dict(mac_persistent_cache_layout="head_major"),
          "candidate": dict(mac_persistent_candidate_mode="all")}.get(case, {})
    cfg, m, backend, fb, layer, q, kb, loc = _decode_setup(**kw)
    vb = kb
    if case == "dtype":
        q = q.float()
    elif case == "head_dim":
        q = torch.zeros(2, 8, 64, dtype=torch.bfloat16)
    elif case == "batch":
        fb.batch_size = 3
    elif case == "group":
        q = torch.zeros(2, 32, 128, dtype=torch.bfloat16)
        kb = vb = torch.zeros(10, 2, 128, dtype=torch.bfloat16)
        q = torch.zeros(2, 18, 128, dtype=torch.bfloat16)  # 18 / 2 = 9 > 8
    elif case == "logit_cap":
        layer.logit_cap = 30.0
    elif case == "kv_scale":
        layer.k_scale_float = 1.0
    elif case == "r2t_dtype":
        backend.indices_updater_decode.req_to_token = torch.zeros(4, 64, dtype=torch.int64)
    elif case == "context":
        m.cur_kv_len = cfg.mac_persistent_max_context + 1
    elif case == "not_ready":
        m.req_ids_host = [0, 1]
        m.mac_cache_ready_host = [True, False, True, True]
    assert persistent.try_persistent_decode(backend, fb, cfg, m, q, kb, vb, loc, layer) is None


def test_workspace_sizes_follow_the_reference_rule():
    cfg, m, backend, *_ = _decode_setup(mac_front_sink_tokens=40, mac_persistent_max_context=4096)
    ws = persistent.ensure_persistent_workspace(backend, m, cfg, batch_size=2)
    assert list(ws) == list(persistent.WORKSPACE_ORDER)
    # max_running = max(batch, ring rows) = 4; tiles = 4096/32 + ceil(40/32) = 130
    assert ws["partial_rect_o"].shape == (4, 2, 130, 4, 128) and ws["partial_rect_o"].dtype == torch.float32
    assert ws["partial_rect_reduced_lse"].shape == (4, 2, 5, 4)
    assert ws["match_dist"].shape == (4, 8, 16)  # ceil(512 / 32) match tiles
    assert ws["complete_task_go"].shape == (4 * 8 * 130,) and ws["task_counts"].shape == (9,)
    assert ws["partial_tail_o"].shape == (4, 2, 8, 4, 128)  # ceil(256 / 32)
    assert persistent.ensure_persistent_workspace(backend, m, cfg, batch_size=2) is ws
    cfg.mac_persistent_partial_fp32 = False
    ws2 = persistent.ensure_persistent_workspace(backend, m, cfg, batch_size=2)
    assert ws2 is not ws and ws2["partial_rect_o"].dtype == torch.bfloat16


def test_decode_hook_passes_through_when_mac_is_off():
    seen = {}

    def original(self, q, k, v, layer, fb, save_kv_cache=True):
        seen["save"] = save_kv_cache
        return "sglang"

    layer = types.SimpleNamespace(mac_config=MacSGLangConfig(enable_mac=False))
    assert persistent.flashinfer_forward_decode_around(original, object(), None, None, None, layer,
                                                       types.SimpleNamespace()) == "sglang"
    assert seen["save"] is True


def test_mode_ids():
    assert persistent.candidate_mode_id("exclude_recent_right") == 1
    assert persistent.candidate_mode_id("last_M") == 0
    assert [persistent.bench_mode_id(x) for x in ("off", "synthetic-head", "synthetic_group")] == [0, 1, 2]


def _ejection_meta(rows=6):
    meta = persistent.MacMetadata(8, 2, 128)
    meta.mac_cache_ready_host = [True] * rows  # host mirror only: no device vectors
    meta.req_ids_host = None
    return meta


def test_low_hit_ejection_policy(monkeypatch):
    """flashinfer_hooks.py:1500-1543: off unless the threshold is set; a step
    with at least the threshold's share of non-hit groups takes its requests
    off the MAC path (not ready, and not marked ready again) until their next
    prefill; the minimum-context switch keeps short requests in."""
    reqs = torch.tensor([1, 4], dtype=torch.int32)
    past = torch.tensor([500, 900], dtype=torch.int32)
    ws = {"group_mode": torch.tensor([[0, 1], [2, 1]], dtype=torch.int32)}  # 3 of 4 groups without a hit
    meta = _ejection_meta()
    monkeypatch.delenv("MAC_ADAPTIVE_LOW_HIT_EJECT_THRESHOLD", raising=False)
    assert not persistent.eject_low_hit_requests(meta, ws, 2, reqs, past)  # off by default
    monkeypatch.setenv("MAC_ADAPTIVE_LOW_HIT_EJECT_THRESHOLD", "0.8")
    assert not persistent.eject_low_hit_requests(meta, ws, 2, reqs, past)  # 0.75 < 0.8
    monkeypatch.setenv("MAC_ADAPTIVE_LOW_HIT_EJECT_THRESHOLD", "0.75")
    monkeypatch.setenv("MAC_ADAPTIVE_LOW_HIT_EJECT_MIN_KV", "600")
    assert not persistent.eject_low_hit_requests(meta, ws, 2, reqs, past)  # request 1 holds 500 < 600
    monkeypatch.delenv("MAC_ADAPTIVE_LOW_HIT_EJECT_MIN_KV")
    assert persistent.eject_low_hit_requests(meta, ws, 2, reqs, past)
    assert meta.mac_low_hit_ejected_host == [False, True, False, False, True, False]
    assert meta.mac_cache_ready_host == [True, False, True, True, False, True]
    persistent.mark_persistent_ready(meta, reqs)  # a later ring update does not bring them back
    assert meta.mac_cache_ready_host[1] is False and meta.mac_cache_ready_host[4] is False
    meta.req_ids_host = [1, 4]
    assert not persistent.persistent_ready(meta, reqs)
    meta.req_ids_host = None
    persistent.clear_low_hit_ejection(meta, [4])  # request 4 is prefilled again
    persistent.mark_persistent_ready(meta, torch.tensor([4], dtype=torch.int32))
    assert meta.mac_cache_ready_host[4] is True and meta.mac_cache_ready_host[1] is False


def test_rocm_extend_ring_rows_are_the_last_capacity_rows():
    """The ROCm extend hook computes the full prefill state only for the rows
    the ring keeps: the scheduler's marked suffix (every row without marks),
    cut to its last M rows, at the absolute positions the ring indexes them
    by; the preserved pre-RoPE rows are found for every layout the attention
    hook leaves (all rows, the plan's rows compacted, a tail)."""
    import types

    from mac_attention.integrations.sglang import model_hooks

    M = 4
    fb = types.SimpleNamespace(extend_seq_lens_cpu=[10, 3, 6], extend_prefix_lens_cpu=[5, 0, 2],
                               mac_prefill_cache_update_starts=[7, -1, 2])
    plan, kept = model_hooks._ring_rows(fb, 3, 19, M)
    # request 0: marked from position 7 = chunk row 2 (rows 2..9), last 4 -> rows 6..9 at positions 11..14
    # request 1: unmarked (-1) -> no rows; request 2: from position 2 = chunk row 0 (6 rows) -> last 4
    assert kept == [(0, 6, 11, 4, 15), (2, 15, 4, 4, 8)]
    fb_nomarks = types.SimpleNamespace(extend_seq_lens_cpu=[10, 3], extend_prefix_lens_cpu=[5, 0])
    plan2, kept2 = model_hooks._ring_rows(fb_nomarks, 2, 13, M)
    assert plan2 is None and kept2 == [(0, 6, 11, 4, 15), (1, 10, 0, 3, 3)]
    meta = types.SimpleNamespace(cur_q_before_rope=torch.zeros(19, 1, 1), cur_q_before_rope_compacted=False,
                                 cur_q_before_rope_local_start=0)
    assert model_hooks._src_rows(meta, plan, kept, 19) == [6, 7, 8, 9, 15, 16, 17, 18]
    # compacted in plan order: request 0's 8 marked rows, then request 2's 6
    meta.cur_q_before_rope = torch.zeros(14, 1, 1)
    meta.cur_q_before_rope_compacted = True
    assert model_hooks._src_rows(meta, plan, kept, 19) == [4, 5, 6, 7, 10, 11, 12, 13]
    # a preserved tail of the last 5 chunk rows cannot serve request 0's rows
    meta.cur_q_before_rope = torch.zeros(5, 1, 1)
    meta.cur_q_before_rope_local_start = 14
    assert model_hooks._src_rows(meta, plan, kept, 19) is None
    assert model_hooks._src_rows(meta, plan, [kept[1]], 19) == [1, 2, 3, 4]
