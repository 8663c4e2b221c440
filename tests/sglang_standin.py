"""Small stand-ins for the SGLang classes and functions the MAC hooks wrap.

SGLang is not installed in this image.  ``install(monkeypatch)`` registers
fresh modules under the real SGLang module names (``sglang.srt...``) with
classes that have the attributes and call structure the hooks rely on:
ServerArgs, ScheduleBatch, ForwardBatch, LlamaAttention (qkv projection,
rotary embedding, RadixAttention, output projection), FlashInferAttnBackend
(its own extend / decode are recorded so a test can tell whether the MAC
path took over), the ROCm backends TritonAttnBackend and AiterAttnBackend
(their own extend writes the chunk's K/V and runs a prefill attention the
test supplies, without lse; their own decode must not run) and the
scheduler-process launch sites.  The numeric parts (projections, RoPE, the
paged prefill wrapper, the ROCm backends' prefill attention) are supplied by
the GPU test.
"""

from __future__ import annotations

import sys
import types


class ForwardMode:
    def __init__(self, decode: bool):
        self.decode = decode

    def is_decode_or_idle(self):
        return self.decode


def _module(monkeypatch, name):
    mod = types.ModuleType(name)
    monkeypatch.setitem(sys.modules, name, mod)
    parent, _, leaf = name.rpartition(".")
    if parent:
        monkeypatch.setattr(sys.modules[parent], leaf, mod, raising=False)
    return mod


def install(monkeypatch, rocm: bool = True):
    """Registers the stand-in modules (the ROCm attention backends' modules
    only with ``rocm``); returns them by short name."""
    mods = {}
    for name in ("sglang", "sglang.srt", "sglang.srt.managers", "sglang.srt.model_executor", "sglang.srt.models",
                 "sglang.srt.layers", "sglang.srt.layers.attention", "sglang.srt.entrypoints"):
        mods[name] = _module(monkeypatch, name)
    calls = []

    server_args = _module(monkeypatch, "sglang.srt.server_args")

    class ServerArgs:
        def __init__(self, **kw):
            self.__dict__.update(kw)
            self.__post_init__()

        def __post_init__(self):
            calls.append("ServerArgs.__post_init__")

        @staticmethod
        def add_cli_args(parser):
            parser.add_argument("--model-path", default="m")

        @classmethod
        def from_cli_args(cls, args):
            return cls(model_path=args.model_path)

    server_args.ServerArgs = ServerArgs

    sched = _module(monkeypatch, "sglang.srt.managers.schedule_batch")

    class ScheduleBatch:
        def __init__(self, reqs, prefix_lens, seq_lens):
            self.reqs, self.prefix_lens, self.seq_lens = reqs, prefix_lens, seq_lens

        def prepare_for_extend(self):
            calls.append("prepare_for_extend")

        def mix_with_running(self, running_batch):
            self.reqs = self.reqs + running_batch.reqs

        def batch_size(self):
            return len(self.reqs)

        def get_model_worker_batch(self):
            return types.SimpleNamespace(reqs=self.reqs)

    sched.ScheduleBatch = ScheduleBatch

    fbi = _module(monkeypatch, "sglang.srt.model_executor.forward_batch_info")

    class ForwardBatch:
        def __init__(self, **kw):
            self.__dict__.update(kw)

        @classmethod
        def init_new(cls, batch, model_runner):
            return cls(source=batch)

    fbi.ForwardBatch = ForwardBatch
    fbi.ForwardMode = ForwardMode

    llama = _module(monkeypatch, "sglang.srt.models.llama")

    class LlamaAttention:
        def __init__(self, num_heads, num_kv_heads, head_dim, qkv_proj, rotary_emb, attn, o_proj):
            self.num_heads, self.num_kv_heads, self.head_dim = num_heads, num_kv_heads, head_dim
            self.q_size, self.kv_size = num_heads * head_dim, num_kv_heads * head_dim
            self.qkv_proj, self.rotary_emb, self.attn, self.o_proj = qkv_proj, rotary_emb, attn, o_proj

        def forward(self, positions, hidden_states, forward_batch):
            calls.append("LlamaAttention.forward (SGLang's own)")
            qkv, _ = self.qkv_proj(hidden_states)
            q, k, v = qkv.split([self.q_size, self.kv_size, self.kv_size], dim=-1)
            q, k = self.rotary_emb(positions, q, k)
            out, _ = self.o_proj(self.attn(q, k, v, forward_batch))
            return out

    llama.LlamaAttention = LlamaAttention

    class LlamaModel:
        def __init__(self, layers):
            self.layers = layers

        def forward(self, input_ids, positions, forward_batch, input_embeds=None):
            calls.append("LlamaModel.forward (SGLang's own)")
            h = input_embeds
            for layer in self.layers:
                h = layer.forward(positions, h, forward_batch)
            return h

    llama.LlamaModel = LlamaModel

    fi = _module(monkeypatch, "sglang.srt.layers.attention.flashinfer_backend")

    class FlashInferAttnBackend:
        def __init__(self, **kw):
            self.__dict__.update(kw)
            self.num_wrappers = 1

        def _get_wrapper_idx(self, layer):
            return 0

        def init_forward_metadata(self, forward_batch):
            calls.append("FlashInferAttnBackend.init_forward_metadata (SGLang's own)")
            self.forward_metadata = types.SimpleNamespace(use_ragged=False, forward_batch=forward_batch)

        def forward_extend(self, q, k, v, layer, forward_batch, save_kv_cache=True):
            calls.append("FlashInferAttnBackend.forward_extend (SGLang's own)")
            raise AssertionError("the MAC extend path was expected")

        def forward_decode(self, q, k, v, layer, forward_batch, save_kv_cache=True):
            calls.append("FlashInferAttnBackend.forward_decode (SGLang's own)")
            raise AssertionError("the MAC decode path was expected")

        def init_forward_metadata_capture_cuda_graph(self, bs, num_tokens, req_pool_indices, seq_lens,
                                                     encoder_lens, forward_mode, spec_info):
            calls.append(("FlashInferAttnBackend.init_forward_metadata_capture_cuda_graph", bs))

        def init_forward_metadata_replay_cuda_graph(self, bs, req_pool_indices, seq_lens, seq_lens_sum,
                                                    encoder_lens, forward_mode, spec_info, seq_lens_cpu=None):
            calls.append(("FlashInferAttnBackend.init_forward_metadata_replay_cuda_graph", bs))

    fi.FlashInferAttnBackend = FlashInferAttnBackend

    rocm_backends = {}
    for module, cls_name in (("sglang.srt.layers.attention.triton_backend", "TritonAttnBackend"),
                             ("sglang.srt.layers.attention.aiter_backend", "AiterAttnBackend")):
        if not rocm:
            break
        mod = _module(monkeypatch, module)

        def make(cls_name=cls_name):
            class RocmAttnBackend:
                """SGLang's ROCm backends keep the request-to-token table as
                ``req_to_token`` and return no lse from forward_extend."""

                def __init__(self, **kw):
                    self.__dict__.update(kw)

                def init_forward_metadata(self, forward_batch):
                    calls.append(f"{cls_name}.init_forward_metadata (SGLang's own)")
                    self.forward_metadata = types.SimpleNamespace(forward_batch=forward_batch)

                def forward_extend(self, q, k, v, layer, forward_batch, save_kv_cache=True):
                    calls.append(f"{cls_name}.forward_extend (SGLang's own)")
                    if save_kv_cache:
                        forward_batch.token_to_kv_pool.set_kv_buffer(layer, forward_batch.out_cache_loc, k, v,
                                                                     layer.k_scale, layer.v_scale)
                    return self.prefill_attention(q, layer, forward_batch)

                def forward_decode(self, q, k, v, layer, forward_batch, save_kv_cache=True):
                    calls.append(f"{cls_name}.forward_decode (SGLang's own)")
                    raise AssertionError("the MAC decode path was expected")

                def init_forward_metadata_capture_cuda_graph(self, bs, num_tokens, req_pool_indices, seq_lens,
                                                             encoder_lens, forward_mode, spec_info):
                    calls.append((f"{cls_name}.init_forward_metadata_capture_cuda_graph", bs))

                def init_forward_metadata_replay_cuda_graph(self, bs, req_pool_indices, seq_lens, seq_lens_sum,
                                                            encoder_lens, forward_mode, spec_info,
                                                            seq_lens_cpu=None):
                    calls.append((f"{cls_name}.init_forward_metadata_replay_cuda_graph", bs))

            RocmAttnBackend.__name__ = RocmAttnBackend.__qualname__ = cls_name
            return RocmAttnBackend

        rocm_backends[cls_name] = make()
        setattr(mod, cls_name, rocm_backends[cls_name])

    scheduler = _module(monkeypatch, "sglang.srt.managers.scheduler")

    def run_scheduler_process(*args, **kwargs):
        calls.append(("run_scheduler_process", args, kwargs))
        return "scheduler ran"

    scheduler.run_scheduler_process = run_scheduler_process
    engine = _module(monkeypatch, "sglang.srt.entrypoints.engine")
    engine.run_scheduler_process = run_scheduler_process

    class Engine:
        run_scheduler_process_func = staticmethod(run_scheduler_process)

    engine.Engine = Engine
    http = _module(monkeypatch, "sglang.srt.entrypoints.http_server")
    http.run_scheduler_process = run_scheduler_process

    def launch_server(server_args, run_scheduler_process_func=run_scheduler_process):
        return run_scheduler_process_func(server_args)

    http.launch_server = launch_server
    dpc = _module(monkeypatch, "sglang.srt.managers.data_parallel_controller")
    dpc.run_scheduler_process = run_scheduler_process

    def run_data_parallel_controller_process(server_args, *, run_scheduler_process_func=run_scheduler_process):
        return run_scheduler_process_func(server_args)

    dpc.run_data_parallel_controller_process = run_data_parallel_controller_process
    return types.SimpleNamespace(ServerArgs=ServerArgs, ScheduleBatch=ScheduleBatch, ForwardBatch=ForwardBatch,
                                 LlamaAttention=LlamaAttention, LlamaModel=LlamaModel,
                                 FlashInferAttnBackend=FlashInferAttnBackend,
                                 TritonAttnBackend=rocm_backends.get("TritonAttnBackend"),
                                 AiterAttnBackend=rocm_backends.get("AiterAttnBackend"),
                                 engine=engine, http=http, dpc=dpc, scheduler=scheduler, calls=calls)
