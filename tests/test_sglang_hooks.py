"""The SGLang hook set against stand-in SGLang modules (SGLang is not
installed here): every target the serving path needs is wrapped, the
scheduler's ring marks travel to the forward batch, the plugin entry point
registers with SGLang's hook registry (or wraps in place without one), and
scheduler processes install the hooks themselves.  Reference behaviour:
hook_installer.py:46-372, schedule_hooks.py:8-66, child_process.py:1-21,
plugin.py:37-69, pyproject.toml:27-28."""

import enum
import os
import sys
import types

import pytest
import torch

import sglang_standin
from helpers import REPO
from mac_attention.integrations.sglang import child_process, hook_installer, plugin, schedule_hooks

REQUIRED = {
    "sglang.srt.server_args:ServerArgs.add_cli_args",
    "sglang.srt.server_args:ServerArgs.from_cli_args",
    "sglang.srt.server_args:ServerArgs.__post_init__",
    "sglang.srt.managers.schedule_batch:ScheduleBatch.prepare_for_extend",
    "sglang.srt.managers.schedule_batch:ScheduleBatch.mix_with_running",
    "sglang.srt.managers.schedule_batch:ScheduleBatch.get_model_worker_batch",
    "sglang.srt.model_executor.forward_batch_info:ForwardBatch.init_new",
    "sglang.srt.models.llama:LlamaAttention.__init__",
    "sglang.srt.models.llama:LlamaAttention.forward",
    "sglang.srt.models.llama:LlamaModel.forward",
    "sglang.srt.layers.attention.flashinfer_backend:FlashInferAttnBackend.__init__",
    "sglang.srt.layers.attention.flashinfer_backend:FlashInferAttnBackend.init_forward_metadata",
    "sglang.srt.layers.attention.flashinfer_backend:FlashInferAttnBackend.forward_extend",
    "sglang.srt.layers.attention.flashinfer_backend:FlashInferAttnBackend.forward_decode",
}
ROCM = {f"sglang.srt.layers.attention.{m}:{c}.{attr}"
        for m, c in (("triton_backend", "TritonAttnBackend"), ("aiter_backend", "AiterAttnBackend"))
        for attr in ("__init__", "init_forward_metadata", "forward_extend", "forward_decode",
                     "init_forward_metadata_capture_cuda_graph", "init_forward_metadata_replay_cuda_graph")}
GRAPH = {f"sglang.srt.layers.attention.flashinfer_backend:FlashInferAttnBackend.{attr}"
         for attr in ("init_forward_metadata_capture_cuda_graph", "init_forward_metadata_replay_cuda_graph")}
CHILD_SITES = {
    "sglang.srt.entrypoints.engine:run_scheduler_process",
    "sglang.srt.entrypoints.http_server:run_scheduler_process",
    "sglang.srt.managers.data_parallel_controller:run_scheduler_process",
    "sglang.srt.entrypoints.engine:Engine.run_scheduler_process_func",
    "sglang.srt.entrypoints.http_server:launch_server.run_scheduler_process_func",
    "sglang.srt.managers.data_parallel_controller:run_data_parallel_controller_process.run_scheduler_process_func",
}


@pytest.fixture
def sg(monkeypatch):
    monkeypatch.setattr(hook_installer, "_INSTALLED", [])
    for k in [k for k in os.environ if k.startswith(("MAC_", "ENABLE_MAC"))]:
        monkeypatch.delenv(k)
    return sglang_standin.install(monkeypatch)


def test_install_wraps_every_serving_target(sg):
    done = set(hook_installer.install_hooks(strict=True))
    assert REQUIRED <= done, REQUIRED - done
    assert ROCM <= done, ROCM - done  # the ROCm attention backends this SGLang has
    assert GRAPH <= done, GRAPH - done
    assert CHILD_SITES <= done, CHILD_SITES - done
    assert not any("qwen" in t for t in done)  # optional classes this SGLang lacks are skipped
    assert getattr(sg.LlamaAttention.forward, "__mac_attention_hooked__", False)
    assert hook_installer.install_hooks(strict=True) == ()  # idempotent
    assert hook_installer.is_installed()


def test_rocm_backends_are_optional(monkeypatch):
    """An SGLang without the ROCm attention backends (a CUDA build) installs
    every required hook and skips theirs."""
    monkeypatch.setattr(hook_installer, "_INSTALLED", [])
    sglang_standin.install(monkeypatch, rocm=False)
    done = set(hook_installer.install_hooks(strict=True))
    assert REQUIRED <= done and not done & ROCM


def test_scheduler_process_installs_hooks_then_runs_sglang(sg, monkeypatch):
    hook_installer.install_hooks(strict=True)
    installs = []
    real = hook_installer.install_hooks
    monkeypatch.setattr(hook_installer, "install_hooks", lambda *a, **k: installs.append(1) or real(*a, **k))
    assert sg.http.launch_server("args") == "scheduler ran"
    assert sg.dpc.run_data_parallel_controller_process("args") == "scheduler ran"
    assert sg.engine.Engine.run_scheduler_process_func is child_process.run_scheduler_process_with_mac_hooks
    assert sg.engine.run_scheduler_process is child_process.run_scheduler_process_with_mac_hooks
    ran = [c for c in sg.calls if isinstance(c, tuple) and c[0] == "run_scheduler_process"]
    assert ran == [("run_scheduler_process", ("args",), {})] * 2
    assert installs == [1, 1]  # each scheduler process installed the hooks before SGLang's scheduler ran


def test_plugin_registers_with_sglang_hook_registry(sg, monkeypatch):
    registered = []

    class HookType(enum.Enum):
        AROUND = "around"
        AFTER = "after"

    class HookRegistry:
        @staticmethod
        def register(target, hook, kind):
            registered.append((target, hook, kind))

    mod = types.ModuleType("sglang.srt.plugins.hook_registry")
    mod.HookRegistry, mod.HookType = HookRegistry, HookType
    monkeypatch.setitem(sys.modules, "sglang.srt.plugins", types.ModuleType("sglang.srt.plugins"))
    monkeypatch.setitem(sys.modules, "sglang.srt.plugins.hook_registry", mod)
    plugin.register_plugin()
    targets = {t for t, _, _ in registered}
    assert REQUIRED <= targets and ROCM <= targets and not any("qwen" in t for t in targets)
    kinds = {t: k for t, _, k in registered}
    assert kinds["sglang.srt.models.llama:LlamaAttention.forward"] is HookType.AROUND
    assert kinds["sglang.srt.server_args:ServerArgs.__post_init__"] is HookType.AFTER
    assert not hook_installer.is_installed()  # the registry wraps; nothing was patched in place
    assert not getattr(sg.LlamaAttention.forward, "__mac_attention_hooked__", False)


def test_plugin_without_registry_wraps_in_place(sg):
    plugin.register_plugin()
    assert getattr(sg.LlamaAttention.forward, "__mac_attention_hooked__", False)
    assert hook_installer.is_installed()


def test_plugin_does_not_register_twice_after_a_launcher_installed(sg, monkeypatch):
    hook_installer.install_hooks(strict=True)
    called = []
    mod = types.ModuleType("sglang.srt.plugins.hook_registry")
    mod.HookRegistry = types.SimpleNamespace(register=lambda *a: called.append(a))
    mod.HookType = types.SimpleNamespace(AROUND=1, AFTER=2)
    monkeypatch.setitem(sys.modules, "sglang.srt.plugins", types.ModuleType("sglang.srt.plugins"))
    monkeypatch.setitem(sys.modules, "sglang.srt.plugins.hook_registry", mod)
    plugin.register_plugin()
    assert called == []


def test_ring_marks_travel_from_scheduler_to_forward_batch(sg, monkeypatch):
    monkeypatch.setenv("MAC_ATTENTION_ENABLE", "1")
    monkeypatch.setenv("MAC_LOOKBACK_TOKENS_LEFT", "16")
    hook_installer.install_hooks(strict=True)
    reqs = [types.SimpleNamespace(origin_input_ids=[0] * n) for n in (100, 10, 40)]
    batch = sg.ScheduleBatch(reqs, prefix_lens=[0, 0, 30], seq_lens=torch.tensor([60, 10, 40]))
    batch.prepare_for_extend()
    # request 0: ring keeps [84, 100), not in this chunk; 1: all of [0, 10); 2: [30, 40)
    assert batch.mac_prefill_cache_update_starts == [-1, 0, 30]
    running = sg.ScheduleBatch([types.SimpleNamespace(origin_input_ids=[0])] * 2, [], [])
    batch.mix_with_running(running)
    assert batch.mac_prefill_cache_update_starts == [-1, 0, 30, -1, -1]
    worker = batch.get_model_worker_batch()
    assert worker.mac_prefill_cache_update_starts == [-1, 0, 30, -1, -1]
    fb = sg.ForwardBatch.init_new(worker, model_runner=None)
    assert fb.mac_prefill_cache_update_starts == [-1, 0, 30, -1, -1]


def test_marks_rule():
    assert schedule_hooks.ring_update_starts([100, 100, 5], [0, 90, 0], [50, 100, 5], 16) == [-1, 90, 0]


def test_mac_off_leaves_batches_unmarked_and_attention_unchanged(sg):
    hook_installer.install_hooks(strict=True)
    batch = sg.ScheduleBatch([types.SimpleNamespace(origin_input_ids=[0] * 8)], [0], [8])
    batch.prepare_for_extend()
    assert batch.mac_prefill_cache_update_starts is None
    ident = lambda x: (x, None)  # noqa: E731
    attn = sg.LlamaAttention(2, 1, 4, ident, lambda pos, q, k: (q, k), lambda q, k, v, fb: q, ident)
    x = torch.arange(16.0).view(1, 16)
    out = attn.forward(torch.zeros(1, dtype=torch.long), x, types.SimpleNamespace())
    assert torch.equal(out, x[:, :8])
    assert "LlamaAttention.forward (SGLang's own)" in sg.calls


def test_pyproject_declares_the_plugin_entry_point():
    import tomli

    with open(os.path.join(REPO, "pyproject.toml"), "rb") as f:
        meta = tomli.load(f)
    eps = meta["project"]["entry-points"]["sglang.srt.plugins"]
    assert eps == {"mac_attention": "mac_attention.integrations.sglang.plugin:register_plugin"}
    mod_name, fn = eps["mac_attention"].split(":")
    __import__(mod_name)
    assert callable(getattr(sys.modules[mod_name], fn))


def test_backend_keeps_ring_marks_for_static_graph_batches(sg, monkeypatch):
    """init_forward_metadata copies the marks onto the backend; a forward batch
    that lost them (piecewise CUDA-graph replay) plans the same ring rows
    (flashinfer_hooks.py:703-735)."""
    from mac_attention.integrations.sglang.prefill_suffix import build_prefill_suffix_plan

    monkeypatch.setenv("MAC_ATTENTION_ENABLE", "1")
    hook_installer.install_hooks(strict=True)
    backend = sg.FlashInferAttnBackend()
    live = sg.ForwardBatch(batch_size=3, mac_prefill_cache_update_starts=[-1, 0, 30],
                           extend_prefix_lens_cpu=[0, 0, 30], extend_seq_lens_cpu=[60, 10, 10])
    backend.init_forward_metadata(live)
    assert "FlashInferAttnBackend.init_forward_metadata (SGLang's own)" in sg.calls
    assert backend.mac_prefill_cache_update_starts_current == [-1, 0, 30]
    want = build_prefill_suffix_plan(live, 3, 80, allow_backend_fallback=False)
    static = sg.ForwardBatch(batch_size=3, attn_backend=backend)
    got = build_prefill_suffix_plan(static, 3, 80)
    assert want is not None and got is not None
    assert (got.offsets, got.kv_offsets, got.req_indices, got.request_lengths) == \
        (want.offsets, want.kv_offsets, want.req_indices, want.request_lengths)
    assert build_prefill_suffix_plan(static, 3, 80, allow_backend_fallback=False) is None


def test_batch_state_is_computed_once_per_forward(sg):
    """The model forward's batch state (request ids, lengths, new tokens) is
    built once and shared by every layer (llama_hooks.py:1852-1876)."""
    from mac_attention.integrations.sglang import model_hooks
    from sglang_standin import ForwardMode

    cpu = torch.device("cpu")
    fb = sg.ForwardBatch(batch_size=2, req_pool_indices=torch.tensor([5, 2]), seq_lens=torch.tensor([9, 4]),
                         forward_mode=ForwardMode(decode=True), seq_lens_cpu=torch.tensor([9, 4]))
    st = model_hooks.batch_state(fb, cpu, fresh=True)  # the model forward
    assert model_hooks.batch_state(fb, cpu) is st  # its layers
    fb.seq_lens = torch.tensor([10, 5])  # the next forward on the same object rebuilds it
    assert model_hooks.batch_state(fb, cpu, fresh=True)["seq"].tolist() == [10, 5]
    assert model_hooks.batch_state(sg.ForwardBatch(**{k: v for k, v in vars(fb).items()
                                                      if k != "_mac_batch_state"}), cpu) is not st
    assert st["req_ids"].dtype == torch.int32 and st["req_ids"].tolist() == [5, 2]
    assert st["cur"].tolist() == [1, 1] and st["seq_host"] == [9, 4] and st["req_ids_host"] == [5, 2]
    ext = sg.ForwardBatch(batch_size=2, req_pool_indices=torch.tensor([1, 3]), seq_lens=torch.tensor([20, 7]),
                          forward_mode=ForwardMode(decode=False), extend_seq_lens=torch.tensor([12, 7]))
    assert model_hooks.batch_state(ext, cpu)["cur"].tolist() == [12, 7]


def test_model_forward_hook_passes_through(sg, monkeypatch):
    monkeypatch.setenv("MAC_ATTENTION_ENABLE", "1")
    hook_installer.install_hooks(strict=True)
    ident = lambda x: (x, None)  # noqa: E731
    attn = sg.LlamaAttention(2, 1, 4, ident, lambda pos, q, k: (q, k), lambda q, k, v, fb: q, ident)
    model = sg.LlamaModel([attn])
    x = torch.arange(16.0).view(1, 16)
    out = model.forward(None, torch.zeros(1, dtype=torch.long), types.SimpleNamespace(batch_size=1), input_embeds=x)
    assert torch.equal(out, x[:, :8])  # CPU tensors: SGLang's own forward, no MAC state
    assert "LlamaModel.forward (SGLang's own)" in sg.calls


@pytest.mark.parametrize("backend_name", ["FlashInferAttnBackend", "TritonAttnBackend"])
def test_decode_graph_replays_skip_backend_metadata_when_every_layer_is_mac(sg, monkeypatch, backend_name):
    """flashinfer_hooks.py:660-700, :835-899: a decode graph captured with the
    MAC step in every layer replays without the backend's metadata update;
    one layer on the backend's own decode, a prefill graph, or the switch
    off, and the backend's update runs."""
    from mac_attention.integrations.sglang import persistent

    monkeypatch.setenv("MAC_ATTENTION_ENABLE", "1")
    hook_installer.install_hooks(strict=True)
    backend = getattr(sg, backend_name)()
    assert backend.mac_config.enable_mac
    decode, prefill = sglang_standin.ForwardMode(True), sglang_standin.ForwardMode(False)
    fb = types.SimpleNamespace(batch_size=4)
    monkeypatch.setattr(persistent, "is_graph_capturing", lambda: True)

    def capture(bs, mode, paths):
        backend.init_forward_metadata_capture_cuda_graph(bs, bs, None, None, None, mode, None)
        for p in paths:  # what each layer's decode hook captured
            persistent.record_decode_graph_capture(backend, types.SimpleNamespace(batch_size=bs), persistent=p)

    def replayed(bs, mode):
        n = len(sg.calls)
        backend.init_forward_metadata_replay_cuda_graph(bs, None, None, 0, None, mode, None)
        return (f"{backend_name}.init_forward_metadata_replay_cuda_graph", bs) in sg.calls[n:]

    capture(4, decode, [True] * 3)
    assert not replayed(4, decode)  # every layer MAC: the backend's update is skipped
    capture(8, decode, [True, False, True])
    assert replayed(8, decode)  # a layer fell back: the backend's metadata is needed
    assert replayed(16, decode)  # never captured here
    capture(4, prefill, [True])
    assert replayed(4, prefill)
    capture(4, decode, [True, True])  # a new capture of the same size starts afresh
    assert not replayed(4, decode)
    monkeypatch.setenv("MAC_CUDAGRAPH_SKIP_FLASHINFER_REPLAY_METADATA", "0")
    assert replayed(4, decode)
    assert (f"{backend_name}.init_forward_metadata_capture_cuda_graph", 4) in sg.calls
    del fb
