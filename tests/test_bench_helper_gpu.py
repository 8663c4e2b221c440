"""mac_bench_stream_read (the streaming-read measurement helper behind
bench.py's `stream_read` leg) reads every 16-byte word it is given: each
32-bit word is XORed into exactly one workgroup's sink entry, so the XOR of
the sink equals the XOR of the words.  Also its argument checks."""

import ctypes

import numpy as np
import pytest

torch = pytest.importorskip("torch")

pytestmark = pytest.mark.gpu


def _lib():
    from mac_attention.integrations.sglang import bridge

    return bridge.load_bench_library()


@pytest.mark.parametrize("nbytes,sink_len", [(16, 1), (64 << 20, 37), ((8 << 20) + 48, 300), ((256 << 20) + 16, 2048)])
def test_stream_read_reads_every_word(nbytes, sink_len):
    lib = _lib()
    rng = np.random.default_rng(nbytes % 1000 + sink_len)
    words = rng.integers(0, 2**32, nbytes // 4, dtype=np.uint64).astype(np.uint32)
    src = torch.from_numpy(words.view(np.int32)).cuda()
    sink = torch.zeros(sink_len, dtype=torch.int32, device="cuda")
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    print(f"stream_read {nbytes} bytes, sink {sink_len}", flush=True)
    rc = lib.mac_bench_stream_read(ctypes.c_void_p(src.data_ptr()), ctypes.c_int64(nbytes),
                                   ctypes.c_void_p(sink.data_ptr()), ctypes.c_int32(sink_len), stream)
    assert rc == 0, lib.mac_bench_last_error()
    torch.cuda.synchronize()
    got = np.bitwise_xor.reduce(sink.cpu().numpy().view(np.uint32))  # entries past the grid stay 0
    assert int(got) == int(np.bitwise_xor.reduce(words[: (nbytes // 16) * 4]))


def test_stream_read_rejects_bad_arguments():
    lib = _lib()
    src = torch.zeros(64, dtype=torch.int32, device="cuda")
    sink = torch.zeros(4, dtype=torch.int32, device="cuda")
    s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    p, q = ctypes.c_void_p(src.data_ptr()), ctypes.c_void_p(sink.data_ptr())
    assert lib.mac_bench_stream_read(p, ctypes.c_int64(8), q, ctypes.c_int32(4), s) != 0          # < 16 bytes
    assert lib.mac_bench_stream_read(p, ctypes.c_int64(256), q, ctypes.c_int32(0), s) != 0        # empty sink
    assert lib.mac_bench_stream_read(ctypes.c_void_p(src.data_ptr() + 4), ctypes.c_int64(128), q,
                                     ctypes.c_int32(4), s) != 0                                   # misaligned
    assert lib.mac_bench_stream_read(None, ctypes.c_int64(256), q, ctypes.c_int32(4), s) != 0
