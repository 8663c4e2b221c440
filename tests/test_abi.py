"""The C-ABI library loads, exports every entry point include/*.h declares,
matches the binding's struct layout, and rejects bad arguments with a message
(CPU only: no kernel is launched)."""

import ctypes
import os
import re
import subprocess

import pytest

from helpers import REPO

HEADER = os.path.join(REPO, "include", "mac_attention_amd.h")
BENCH_HEADER = os.path.join(REPO, "include", "mac_bench.h")
NOALLOC_HEADER = os.path.join(REPO, "include", "mac_noalloc.h")


def _declared(header=HEADER, api="MAC_API"):
    text = open(header).read()
    return re.findall(api + r"\s+[\w\s\*]+?\b(mac_\w+)\s*\(", text)


@pytest.fixture(scope="module")
def bridge():
    from mac_attention.integrations.sglang import bridge as b

    if not os.path.exists(b.LIB_PATH):
        pytest.fail(f"{b.LIB_PATH} is not built; run __graft_entry__.build()")
    return b


def test_library_exports_every_declared_symbol(bridge):
    names = _declared()
    assert len(names) >= 8
    lib = bridge.load_library()
    for n in names:
        assert hasattr(lib, n), n
    assert set(names) == set(bridge.EXPORTED_SYMBOLS)
    nm = subprocess.run(["nm", "-D", "--defined-only", bridge.LIB_PATH], capture_output=True,
                        text=True, check=True).stdout
    exported = {l.split()[-1] for l in nm.splitlines() if " T " in l}
    assert exported == set(names)
    assert lib.mac_abi_version() == bridge.ABI_VERSION


def test_measurement_library_is_separate(bridge):
    """The measurement helpers (streaming read, per-kernel timed decode step)
    live in libmac_bench.so, not in the decode library, and it exports
    exactly what include/mac_bench.h declares -- none of the decode
    library's entry points, although it compiles the decode source too."""
    names = _declared(BENCH_HEADER, "MAC_BENCH_API")
    assert set(names) == set(bridge.BENCH_EXPORTED_SYMBOLS)
    lib = bridge.load_bench_library()
    for n in names:
        assert hasattr(lib, n), n
    nm = subprocess.run(["nm", "-D", "--defined-only", bridge.BENCH_LIB_PATH], capture_output=True,
                        text=True, check=True).stdout
    assert {l.split()[-1] for l in nm.splitlines() if " T " in l} == set(names)
    assert not set(names) & set(bridge.EXPORTED_SYMBOLS)


def test_noalloc_library_is_separate(bridge):
    """The no-allocation entry point and its static device array live in
    libmac_noalloc.so (so only processes that load it reserve the array),
    which exports exactly what include/mac_noalloc.h declares and links
    against libmac_hip.so in its own directory."""
    names = _declared(NOALLOC_HEADER)
    assert set(names) == set(bridge.NOALLOC_EXPORTED_SYMBOLS)
    lib = bridge.load_noalloc_library()
    for n in names:
        assert hasattr(lib, n), n
    nm = subprocess.run(["nm", "-D", "--defined-only", bridge.NOALLOC_LIB_PATH], capture_output=True,
                        text=True, check=True).stdout
    assert {l.split()[-1] for l in nm.splitlines() if " T " in l} == set(names)
    assert not set(names) & set(bridge.EXPORTED_SYMBOLS)
    needed = subprocess.run(["readelf", "-d", bridge.NOALLOC_LIB_PATH], capture_output=True, text=True,
                            check=True).stdout
    assert "libmac_hip.so" in needed and "$ORIGIN" in needed
    # no device array in the decode library
    syms = subprocess.run(["nm", bridge.LIB_PATH], capture_output=True, text=True, check=True).stdout
    assert "scratch" not in syms
    a = bridge.MacDecodeArgs()
    a.struct_size = ctypes.sizeof(a)
    a.abi_version = bridge.ABI_VERSION
    a.N, a.Hq, a.Hkv, a.D, a.M, a.R, a.max_context = 200, 32, 8, 128, 32, 200, 1024
    assert lib.mac_persistent_decode_bf16_noalloc(ctypes.byref(a), None) == 1
    assert b"at most 4096 query heads" in lib.mac_noalloc_last_error()
    a.N, a.M = 4, 4096
    assert lib.mac_persistent_decode_bf16_noalloc(ctypes.byref(a), None) == 1
    assert b"rings of at most 2048" in lib.mac_noalloc_last_error()


@pytest.mark.parametrize("struct", ["MacDecodeArgs", "MacWindowAttentionArgs", "MacRectifyArgs"])
def test_struct_layout_matches_header(bridge, tmp_path, struct):
    cls = getattr(bridge, struct)
    fields = [f[0] for f in cls._fields_]
    src = ['#include <stdio.h>', '#include <stddef.h>', '#include "mac_attention_amd.h"',
           'int main(void) {', f'printf("size %zu\\n", sizeof({struct}));']
    for f in fields:
        src.append(f'printf("{f} %zu\\n", offsetof({struct}, {f}));')
    src.append("return 0; }")
    c = tmp_path / "layout.c"
    c.write_text("\n".join(src))
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-I", os.path.dirname(HEADER), str(c), "-o", str(exe)], check=True)
    out = dict(l.split() for l in subprocess.run([str(exe)], capture_output=True, text=True,
                                                  check=True).stdout.splitlines())
    assert int(out["size"]) == ctypes.sizeof(cls)
    for f in fields:
        assert int(out[f]) == getattr(cls, f).offset, f


def test_bad_arguments_return_error_and_message(bridge):
    lib = bridge.load_library()
    a = bridge.MacDecodeArgs()
    a.struct_size = ctypes.sizeof(a) + 8
    a.abi_version = bridge.ABI_VERSION
    assert lib.mac_persistent_decode_bf16(ctypes.byref(a), None) == 1
    assert b"size/version mismatch" in lib.mac_last_error()
    a.struct_size = ctypes.sizeof(a)
    a.N, a.Hq, a.Hkv, a.D, a.M, a.R = 1, 32, 8, 64, 8, 1
    assert lib.mac_persistent_decode_bf16(ctypes.byref(a), None) == 1
    assert b"D=128" in lib.mac_last_error()
    a.D, a.Hkv = 128, 3
    assert lib.mac_persistent_decode_bf16(ctypes.byref(a), None) == 1
    assert b"divisible" in lib.mac_last_error()
    a.Hkv, a.Hq = 2, 32
    assert lib.mac_persistent_decode_bf16(ctypes.byref(a), None) == 1
    assert b"group size" in lib.mac_last_error()
    assert lib.mac_mark_persistent_ready(None, None, None, None, 0, 4, None) == 0
    assert lib.mac_mark_persistent_ready(None, None, None, None, 2, 4, None) == 1
    assert b"NULL" in lib.mac_last_error()


def test_prefill_entry_points_reject_bad_arguments(bridge):
    lib = bridge.load_library()
    assert lib.mac_update_then_downdate_bf16_inplace(None, None, 0, None, None, 5, 4, 128, None) == 1
    assert b"lse2 must be float32, bfloat16, or float16" in lib.mac_last_error()
    assert lib.mac_update_then_downdate_bf16_inplace(None, None, 0, None, None, 0, 0, 128, None) == 0
    w = bridge.MacWindowAttentionArgs()
    w.struct_size = ctypes.sizeof(w)
    w.abi_version = bridge.ABI_VERSION
    w.B, w.Hq, w.Hkv, w.D = 1, 8, 2, 64
    assert lib.mac_prefill_window_attention_bf16(ctypes.byref(w), None) == 1
    assert b"head_dim must be 128" in lib.mac_last_error()
    r = bridge.MacRectifyArgs()
    r.struct_size = ctypes.sizeof(r) - 4
    assert lib.mac_prefill_rectify_update_cache_bf16(ctypes.byref(r), None) == 1
    assert b"struct_size mismatch" in lib.mac_last_error()


def _pointers(args, base=0x10000):
    """Every pointer field of an argument struct set to its own 256-byte
    aligned dummy address (validation fails before anything is read)."""
    for i, (name, typ) in enumerate(args._fields_):
        if typ is ctypes.c_void_p:
            setattr(args, name, base + 256 * i)


def test_entry_points_reject_misaligned_pointers(bridge):
    """The kernels move rows with 16-byte (and 8-/4-byte) vector accesses: a
    misaligned pointer is refused with a message, before any GPU work."""
    lib = bridge.load_library()
    a = bridge.MacDecodeArgs()
    a.struct_size, a.abi_version = ctypes.sizeof(a), bridge.ABI_VERSION
    a.N, a.Hq, a.Hkv, a.D, a.M, a.R = 1, 8, 2, 128, 8, 1
    a.workspace_rows, a.tile_tokens, a.match_tile_slots, a.max_match_tiles = 1, 256, 8, 1
    a.max_context, a.max_tiles_context, a.complete_task_len = 1024, 4, 64
    a.req_to_token_rows, a.req_to_token_stride = 1, 1024
    for field, offset, msg in (("k_buffer", 8, b"16-byte aligned"), ("query_cache", 4, b"16-byte aligned"),
                               ("out", 2, b"4-byte aligned"), ("partial_o", 4, b"8-byte aligned")):
        _pointers(a)
        setattr(a, field, getattr(a, field) + offset)
        assert lib.mac_persistent_decode_bf16(ctypes.byref(a), None) == 1, field
        assert msg in lib.mac_last_error(), (field, lib.mac_last_error())
    w = bridge.MacWindowAttentionArgs()
    w.struct_size, w.abi_version = ctypes.sizeof(w), bridge.ABI_VERSION
    w.B, w.Hq, w.Hkv, w.D, w.total_q, w.pool_tokens, w.kv_indices_len = 1, 8, 2, 128, 4, 16, 4
    for field in ("q", "v_buffer", "out"):
        _pointers(w)
        setattr(w, field, getattr(w, field) + 2)
        assert lib.mac_prefill_window_attention_bf16(ctypes.byref(w), None) == 1, field
        assert b"16-byte aligned" in lib.mac_last_error(), (field, lib.mac_last_error())
    r = bridge.MacRectifyArgs()
    r.struct_size, r.abi_version = ctypes.sizeof(r), bridge.ABI_VERSION
    r.B, r.Hq, r.Hkv, r.D, r.total_q, r.pool_tokens, r.kv_indices_len = 1, 8, 2, 128, 4, 16, 4
    r.M, r.R, r.semantic_pos_ahead, r.request_length_len = 4, 1, 8, 1
    for field in ("o_full", "src_q", "q_post_cache"):
        _pointers(r)
        setattr(r, field, getattr(r, field) + 8)
        assert lib.mac_prefill_rectify_update_cache_bf16(ctypes.byref(r), None) == 1, field
        assert b"16-byte aligned" in lib.mac_last_error(), (field, lib.mac_last_error())


def test_binding_rejects_host_tensors(bridge):
    torch = pytest.importorskip("torch")
    ext = bridge.PersistentDecodeExtension(bridge.load_library())
    q = torch.zeros(1, 8, 128, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="q_post must be CUDA"):
        ext.mac_persistent_decode_bf16(q, *([None] * 67))
