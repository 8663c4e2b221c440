"""Builds the libraries for gfx950 with hipcc (no CMake, no JIT):

* libmac_hip.so -- the product: decode step, ring-cache ops, prefill
  rectification, decode RoPE;
* libmac_noalloc.so -- the decode step with its workspaces in a static device
  array (linked against libmac_hip.so; only processes that load it reserve
  the array);
* libmac_bench.so -- measurement helpers (streaming read; the decode step
  timed kernel by kernel, from the same decode source with its C ABI hidden).
"""

from __future__ import annotations

import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(HERE)
SOURCES = [os.path.join(HERE, "csrc", f) for f in ("mac_decode.hip", "mac_cache_ops.hip", "mac_prefill.hip", "mac_rope.hip")]
OUTPUT = os.path.join(HERE, "libmac_hip.so")
NOALLOC_SOURCES = [os.path.join(HERE, "csrc", "mac_noalloc.hip")]
NOALLOC_OUTPUT = os.path.join(HERE, "libmac_noalloc.so")
BENCH_SOURCES = [os.path.join(HERE, "csrc", "mac_bench.hip"), os.path.join(HERE, "csrc", "mac_decode.hip")]
BENCH_OUTPUT = os.path.join(HERE, "libmac_bench.so")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    # keep the compiler from forming packed-fp32 VALU ops (some of their forms
    # have given wrong results on the target machines, without any error)
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-fvisibility=hidden",
    # MFMA accumulators in VGPRs: the online-softmax rescale then works on
    # them in place instead of copying them through AGPRs every block
    "-mllvm", "-amdgpu-mfma-vgpr-form",
    "-I", os.path.join(REPO, "include"),
    "-I", os.path.join(HERE, "csrc"),
]


def _hipcc(sources: list[str], output: str, verbose: bool, extra: list[str] | None = None) -> str:
    cmd = [HIPCC, *FLAGS, *sources, "-o", output, *(extra or [])]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    noise = "'-packed-fp32-ops' is not a recognized feature"
    err = "\n".join(l for l in res.stderr.splitlines() if noise not in l)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed ({res.returncode}):\n{err}")
    if verbose and err.strip():
        print(err, file=sys.stderr)
    return output


def build(verbose: bool = False) -> str:
    """All three libraries; returns the decode library's path."""
    from concurrent.futures import ThreadPoolExecutor

    with ThreadPoolExecutor(max_workers=2) as pool:
        # the decode library's C ABI stays hidden in the measurement library
        bench = pool.submit(_hipcc, BENCH_SOURCES, BENCH_OUTPUT, verbose, ["-DMAC_API="])
        _hipcc(SOURCES, OUTPUT, verbose)
        _hipcc(NOALLOC_SOURCES, NOALLOC_OUTPUT, verbose, ["-L" + HERE, "-lmac_hip", "-Wl,-rpath,$ORIGIN"])
        bench.result()
    return OUTPUT


if __name__ == "__main__":
    print(build(verbose=True))
