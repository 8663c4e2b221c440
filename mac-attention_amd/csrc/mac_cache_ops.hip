// mac_cache_ops.hip -- MAC ring-cache maintenance ops for MI355X (gfx950).
//
//  * prefill_update_cache: copies the last min(len, M) prefill rows of each
//    batch row (pre-RoPE q, prefix attention output, lse) into the request's
//    ring at (L_before + start + i) % M and bumps request_length
//    (PREFILL:201-269).  One workgroup per kept row; the bump is a second
//    launch, so every copy of a batch row reads the same L_before.
//  * mark / invalidate / update_request_state: per-request readiness and
//    length metadata (PREFILL:271-320).

#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>

#include "mac_attention_amd.h"

namespace mac {
int fail(int code, const char* fmt, ...);
}  // namespace mac

namespace {

constexpr int kThreads = 256;

struct PrefillParams {
  uint16_t* q_cache;
  uint16_t* attn_cache;
  float* lse_cache;
  uint16_t* q_post_cache;
  const uint16_t* src_q;
  const uint16_t* src_attn;
  const float* src_lse;
  int32_t* request_length;
  const int32_t* req_ids;
  const int32_t* offsets;
  const int32_t* lens;
  int R, M, H, D, B, src_rows;
  int by_batch;
  int vec16;  // rows move as 16-byte vectors (H D % 8 == 0, every row buffer 16-byte aligned)
};

// Validity of batch row b and its kept rows [start, ni) (PREFILL:201-230):
// false when it has nothing to copy or names a request or source range
// outside the buffers.
__device__ __forceinline__ bool prefill_row(const PrefillParams& p, int b, int& req, int& ni, int& start) {
  req = p.req_ids[b];
  ni = p.lens[b];
  const int off = p.offsets[b];
  start = ni > p.M ? ni - p.M : 0;
  return ni > 0 && p.M > 0 && req >= 0 && req < p.R && off >= 0 && off + ni <= p.src_rows;
}

// Kept row i of batch row b: copies source row
// offsets[b] + start + i (q and attention output: H * D bf16 each, lse: H
// floats) to ring slot (L_before + start + i) % M.  Every load of a round is
// issued before its stores.
__device__ __forceinline__ void copy_prefill_row(const PrefillParams& p, int b, int i) {
  int req, ni, start;
  if (!prefill_row(p, b, req, ni, start) || i >= ni - start) return;
  int before = p.by_batch ? p.request_length[b] : p.request_length[req];
  if (before < 0) before = 0;
  const int dst = static_cast<int>((static_cast<int64_t>(before) + start + i) % p.M);
  const int64_t drow = static_cast<int64_t>(req) * p.M + dst;
  const int64_t srow = static_cast<int64_t>(p.offsets[b]) + start + i;
  const int64_t row = static_cast<int64_t>(p.H) * p.D;
  const int tid = threadIdx.x;
  if (p.vec16) {
    const int64_t n16 = row / 8;
    const uint4* sq = reinterpret_cast<const uint4*>(p.src_q + srow * row);
    const uint4* sa = reinterpret_cast<const uint4*>(p.src_attn + srow * row);
    uint4* dq = reinterpret_cast<uint4*>(p.q_cache + drow * row);
    uint4* da = reinterpret_cast<uint4*>(p.attn_cache + drow * row);
    for (int64_t e = tid; e < n16; e += 2 * kThreads) {
      const bool two = e + kThreads < n16;
      const uint4 q0 = sq[e], a0 = sa[e];
      uint4 q1 = q0, a1 = a0;
      if (two) {
        q1 = sq[e + kThreads];
        a1 = sa[e + kThreads];
      }
      dq[e] = q0;
      da[e] = a0;
      if (two) {
        dq[e + kThreads] = q1;
        da[e + kThreads] = a1;
      }
    }
  } else {
    for (int64_t e = tid; e < row; e += kThreads) {
      const uint16_t q = p.src_q[srow * row + e], a = p.src_attn[srow * row + e];
      p.q_cache[drow * row + e] = q;
      p.attn_cache[drow * row + e] = a;
    }
  }
  for (int h = tid; h < p.H; h += kThreads) p.lse_cache[drow * p.H + h] = p.src_lse[srow * p.H + h];
  if (p.q_post_cache != nullptr) {
    // bf16 quiet NaN marks rows whose post-RoPE query is unknown (PREFILL:251-262)
    uint16_t* qp = p.q_post_cache + drow * row;
    for (int64_t e = tid; e < row; e += kThreads) qp[e] = 0x7fc0;
  }
}

// One workgroup per (kept row, batch row).  request_length is bumped
// afterwards by bump_length_kernel, so every workgroup of a batch row reads
// the same L_before.
__global__ void __launch_bounds__(kThreads) prefill_update_cache_kernel(PrefillParams p) {
  const int i = blockIdx.x;
  for (int b = blockIdx.y; b < p.B; b += gridDim.y) copy_prefill_row(p, b, i);
}

// request_length[req] += lens[b] for the valid batch rows (indexed-by-request
// form only), after every copy has read the old length.
__global__ void bump_length_kernel(PrefillParams p) {
  const int b = blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= p.B) return;
  int req, ni, start;
  if (prefill_row(p, b, req, ni, start)) atomicAdd(&p.request_length[req], ni);
}

__global__ void mark_ready_kernel(uint8_t* ready, int64_t* cache_epoch, const int64_t* request_epoch,
                                  const int32_t* req_ids, int B, int R) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= B) return;
  const int req = req_ids[i];
  if (req < 0 || req >= R) return;
  cache_epoch[req] = request_epoch[req];
  ready[req] = 1;
}

__global__ void invalidate_ready_kernel(uint8_t* ready, int64_t* cache_epoch, int64_t* request_epoch,
                                        const int32_t* req_ids, int B, int R) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= B) return;
  const int req = req_ids[i];
  if (req < 0 || req >= R) return;
  ready[req] = 0;
  cache_epoch[req] = -1;
  request_epoch[req] += 1;
}

__global__ void update_request_state_kernel(int32_t* req_len, int32_t* match_req_len, int32_t* cache_lens,
                                            const int32_t* req_ids, const int32_t* seq_lens,
                                            const int32_t* cur_lens, int B, int R) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= B) return;
  int32_t c = seq_lens[i] - cur_lens[i];
  if (c < 0) c = 0;
  cache_lens[i] = c;
  const int req = req_ids[i];
  if (req < 0 || req >= R) return;
  req_len[req] = seq_lens[i];
  match_req_len[req] = c;
}

}  // namespace

#define REQUIRE(cond, ...) \
  do {                     \
    if (!(cond)) return mac::fail(MAC_ERR_INVALID_ARGUMENT, __VA_ARGS__); \
  } while (0)

#define HIP_OK(call)                                                                      \
  do {                                                                                    \
    hipError_t e_ = (call);                                                               \
    if (e_ != hipSuccess) return mac::fail(MAC_ERR_HIP, "%s: %s", #call, hipGetErrorString(e_)); \
  } while (0)

extern "C" int mac_prefill_update_cache(void* q_cache, void* attn_cache, float* lse_cache,
                                        int32_t* request_length, int32_t request_length_len,
                                        const int32_t* req_ids, int32_t B, const void* src_q,
                                        const void* src_attn, const float* src_lse, int32_t src_rows,
                                        const int32_t* offsets, const int32_t* lens, int32_t R,
                                        int32_t capacity, int32_t num_heads, int32_t head_dim,
                                        void* q_post_cache, void* stream) {
  // PREFILL:324-327: nothing to do for an empty batch or a zero-capacity ring
  if (capacity <= 0 || B == 0) return MAC_OK;
  REQUIRE(R > 0, "R must be > 0");
  REQUIRE(B > 0 && num_heads > 0 && head_dim > 0 && src_rows >= 0, "invalid sizes");
  REQUIRE(request_length_len == R || request_length_len == B, "request_length must be [R] or [B]");
  REQUIRE(q_cache && attn_cache && lse_cache && request_length && req_ids && offsets && lens &&
              (src_rows == 0 || (src_q && src_attn && src_lse)),
          "a required pointer is NULL");
  PrefillParams p{};
  p.q_cache = static_cast<uint16_t*>(q_cache);
  p.attn_cache = static_cast<uint16_t*>(attn_cache);
  p.lse_cache = lse_cache;
  p.q_post_cache = static_cast<uint16_t*>(q_post_cache);
  p.src_q = static_cast<const uint16_t*>(src_q);
  p.src_attn = static_cast<const uint16_t*>(src_attn);
  p.src_lse = src_lse;
  p.request_length = request_length;
  p.req_ids = req_ids;
  p.offsets = offsets;
  p.lens = lens;
  p.R = R;
  p.M = capacity;
  p.H = num_heads;
  p.D = head_dim;
  p.B = B;
  p.src_rows = src_rows;
  p.by_batch = request_length_len == B ? 1 : 0;
  auto aligned16 = [](const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15) == 0; };
  p.vec16 = (static_cast<int64_t>(num_heads) * head_dim) % 8 == 0 && aligned16(q_cache) && aligned16(attn_cache) &&
            aligned16(src_q) && aligned16(src_attn);
  hipStream_t st = static_cast<hipStream_t>(stream);
  hipLaunchKernelGGL(prefill_update_cache_kernel, dim3(capacity, B < 65535 ? B : 65535), dim3(kThreads), 0, st, p);
  HIP_OK(hipGetLastError());
  if (!p.by_batch) {
    hipLaunchKernelGGL(bump_length_kernel, dim3((B + kThreads - 1) / kThreads), dim3(kThreads), 0, st, p);
    HIP_OK(hipGetLastError());
  }
  return MAC_OK;
}

extern "C" int mac_mark_persistent_ready(uint8_t* ready, int64_t* cache_epoch, const int64_t* request_epoch,
                                         const int32_t* req_ids, int32_t B, int32_t R, void* stream) {
  if (B == 0) return MAC_OK;
  REQUIRE(B > 0 && R >= 0, "invalid sizes");
  REQUIRE(ready && cache_epoch && request_epoch && req_ids, "a required pointer is NULL");
  hipLaunchKernelGGL(mark_ready_kernel, dim3((B + 127) / 128), dim3(128), 0, static_cast<hipStream_t>(stream),
                     ready, cache_epoch, request_epoch, req_ids, B, R);
  HIP_OK(hipGetLastError());
  return MAC_OK;
}

extern "C" int mac_invalidate_persistent_ready(uint8_t* ready, int64_t* cache_epoch, int64_t* request_epoch,
                                               const int32_t* req_ids, int32_t B, int32_t R, void* stream) {
  if (B == 0) return MAC_OK;
  REQUIRE(B > 0 && R >= 0, "invalid sizes");
  REQUIRE(ready && cache_epoch && request_epoch && req_ids, "a required pointer is NULL");
  hipLaunchKernelGGL(invalidate_ready_kernel, dim3((B + 127) / 128), dim3(128), 0,
                     static_cast<hipStream_t>(stream), ready, cache_epoch, request_epoch, req_ids, B, R);
  HIP_OK(hipGetLastError());
  return MAC_OK;
}

extern "C" int mac_update_request_state(int32_t* req_len, int32_t* match_req_len, int32_t* cache_lens,
                                        const int32_t* req_ids, const int32_t* seq_lens, const int32_t* cur_lens,
                                        int32_t B, int32_t R, void* stream) {
  if (B == 0) return MAC_OK;
  REQUIRE(B > 0 && R >= 0, "invalid sizes");
  REQUIRE(req_len && match_req_len && cache_lens && req_ids && seq_lens && cur_lens,
          "a required pointer is NULL");
  hipLaunchKernelGGL(update_request_state_kernel, dim3((B + 127) / 128), dim3(128), 0,
                     static_cast<hipStream_t>(stream), req_len, match_req_len, cache_lens, req_ids, seq_lens,
                     cur_lens, B, R);
  HIP_OK(hipGetLastError());
  return MAC_OK;
}
