// mac_bench.hip -- libmac_bench.so, measurement helpers for MI355X (gfx950):
// the rate a plain streaming read of HBM reaches on this GPU, as context for
// the decode kernels' fractions of the 8 TB/s nameplate, and the decode step
// timed kernel by kernel with HIP events (mac_decode.hip is compiled into
// this library as well, with its C ABI hidden).  Not part of the decode path,
// so built as a library of its own.

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdarg>
#include <cstdint>
#include <cstdio>

#include "mac_bench.h"

namespace {

thread_local char g_bench_err[256] = "";

int bench_fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_bench_err, sizeof(g_bench_err), fmt, ap);
  va_end(ap);
  return code;
}

typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));

// Grid-stride read of n16 16-byte words with the non-temporal policy (as the
// decode kernels stream K/V), eight loads in flight per lane; one XOR per
// workgroup goes to `sink` so the loads are not dead code.
__global__ void __launch_bounds__(256) stream_read_kernel(const u32x4_t* __restrict__ src, int64_t n16,
                                                          uint32_t* __restrict__ sink) {
  constexpr int kUnroll = 8;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  uint32_t acc = 0;
  int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  for (; i + (kUnroll - 1) * stride < n16; i += kUnroll * stride) {
    u32x4_t w[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) w[u] = __builtin_nontemporal_load(src + i + u * stride);
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) acc ^= w[u][0] ^ w[u][1] ^ w[u][2] ^ w[u][3];
  }
  for (; i < n16; i += stride) {
    const u32x4_t w = __builtin_nontemporal_load(src + i);
    acc ^= w[0] ^ w[1] ^ w[2] ^ w[3];
  }
  __shared__ uint32_t s_acc[256];
  s_acc[threadIdx.x] = acc;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint32_t x = 0;
    for (int t = 0; t < 256; ++t) x ^= s_acc[t];
    sink[blockIdx.x] = x;
  }
}

}  // namespace

extern "C" int mac_bench_stream_read(const void* src, int64_t bytes, uint32_t* sink, int32_t sink_len,
                                     void* stream) {
  if (src == nullptr || sink == nullptr || bytes < 16 || sink_len <= 0 ||
      (reinterpret_cast<uintptr_t>(src) & 15) != 0)
    return bench_fail(1, "mac_bench_stream_read: invalid arguments");
  int dev = 0, cus = 256;
  if (hipGetDevice(&dev) == hipSuccess) {
    int v = 0;
    if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && v > 0) cus = v;
  }
  const int grid = std::min(sink_len, cus * 8);
  hipLaunchKernelGGL(stream_read_kernel, dim3(grid), dim3(256), 0, static_cast<hipStream_t>(stream),
                     static_cast<const u32x4_t*>(src), bytes / 16, sink);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return bench_fail(2, "stream_read_kernel: %s", hipGetErrorString(e));
  g_bench_err[0] = '\0';
  return 0;
}

namespace mac {
int decode_impl(const MacDecodeArgs* a, void* stream_ptr, hipEvent_t* ev);  // mac_decode.hip
}
extern "C" const char* mac_last_error(void);  // mac_decode.hip (not exported from this library)

extern "C" int mac_bench_decode_timed(const MacDecodeArgs* a, void* stream, float* ms) {
  if (ms == nullptr) return bench_fail(MAC_ERR_INVALID_ARGUMENT, "ms must not be NULL");
  hipEvent_t ev[4];
  for (int i = 0; i < 4; ++i) {
    const hipError_t e = hipEventCreate(&ev[i]);
    if (e != hipSuccess) {
      for (int j = 0; j < i; ++j) (void)hipEventDestroy(ev[j]);
      return bench_fail(MAC_ERR_HIP, "hipEventCreate: %s", hipGetErrorString(e));
    }
  }
  int rc = mac::decode_impl(a, stream, ev);
  if (rc != MAC_OK) {
    bench_fail(rc, "%s", mac_last_error());
  } else {
    hipError_t e = hipEventSynchronize(ev[3]);
    for (int i = 0; i < 3 && e == hipSuccess; ++i) e = hipEventElapsedTime(&ms[i], ev[i], ev[i + 1]);
    if (e != hipSuccess) rc = bench_fail(MAC_ERR_HIP, "event timing: %s", hipGetErrorString(e));
  }
  for (int i = 0; i < 4; ++i) (void)hipEventDestroy(ev[i]);
  if (rc == MAC_OK) g_bench_err[0] = '\0';
  return rc;
}

extern "C" const char* mac_bench_last_error(void) { return g_bench_err; }
