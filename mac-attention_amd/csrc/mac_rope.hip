// mac_rope.hip -- fused decode RoPE + pre-RoPE query preserve + KV scatter
// for MI355X (gfx950).
//
// For every decode token n (position positions[n], pool row cache_locs[n]):
//   q_pre[n]                 <- q[n]                  (pre-RoPE copy, all dims)
//   q[n], k[n] (in place)    <- RoPE(q[n]), RoPE(k[n]) on the first rotary_dim dims
//   k_buffer[cache_locs[n]]  <- RoPE(k[n]);  v_buffer[cache_locs[n]] <- v[n]
// RoPE of a pair (x0, x1) with c = cos_sin[pos][i], s = cos_sin[pos][half + i]:
//   (x0 c - x1 s, x1 c + x0 s) in fp32, rounded to bf16; the pair is
//   (i, i + half) in NeoX style, (2i, 2i + 1) otherwise
// (mac_decode_rope_preserve.cu:36-156).
//
// One workgroup per token.  The fast kernel moves 16-byte vectors: a RoPE
// unit is the two 16-byte chunks that hold 8 complete pairs (dims [8j, 8j+8)
// and [half+8j, ...) for NeoX, [16j, 16j+16) otherwise), so each lane rotates
// 8 pairs with 2 loads and 3 or 4 stores; pass-through dims and V move as
// plain 16-byte copies.  Shapes the vectors do not fit (rotary_dim not a
// multiple of 16, odd strides or misaligned views) take an element-wise
// kernel with the same results.

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>

#include "mac_attention_amd.h"
#include "mac_common.h"

namespace mac {
int fail(int code, const char* fmt, ...);
}  // namespace mac

namespace {

using namespace mac;

struct RopeParams {
  uint16_t* q;
  uint16_t* k;
  const uint16_t* v;
  uint16_t* q_pre;
  uint16_t* k_buffer;
  uint16_t* v_buffer;
  const float* cs;
  const void* positions;
  const void* cache_locs;
  int64_t q_stride0, k_stride0, v_stride0, cs_stride0;
  int64_t cs_rows, pool_tokens;
  int Hq, Hkv, D, rot;
  int pos_i64, loc_i64, neox;
};

__device__ __forceinline__ int64_t load_index(const void* p, int is_i64, int64_t n) {
  return is_i64 ? static_cast<const int64_t*>(p)[n] : static_cast<const int32_t*>(p)[n];
}

// Position row of the cos/sin table; out-of-range positions are clamped into
// the table (the reference reads outside it).
__device__ __forceinline__ const float* cs_row(const RopeParams& p, int64_t n) {
  int64_t pos = load_index(p.positions, p.pos_i64, n);
  pos = pos < 0 ? 0 : (pos >= p.cs_rows ? p.cs_rows - 1 : pos);
  return p.cs + pos * p.cs_stride0;
}

__device__ __forceinline__ void rotate(float x0, float x1, float c, float s, uint16_t& y0, uint16_t& y1) {
  y0 = f32_to_bf16(x0 * c - x1 * s);
  y1 = f32_to_bf16(x1 * c + x0 * s);
}

__device__ __forceinline__ uint32_t pack2(uint16_t lo, uint16_t hi) {
  return static_cast<uint32_t>(lo) | (static_cast<uint32_t>(hi) << 16);
}

__device__ __forceinline__ uint4 pack8(const uint16_t* r) {
  return make_uint4(pack2(r[0], r[1]), pack2(r[2], r[3]), pack2(r[4], r[5]), pack2(r[6], r[7]));
}

// Rotates the 8 pairs held by chunks a (first) and b (second) of one head.
__device__ __forceinline__ void rope_unit(const RopeParams& p, const float* cs, int j, uint4& a, uint4& b) {
  const int half = p.rot >> 1;
  float fa[8], fb[8];
  unpack8(a, fa);
  unpack8(b, fb);
  uint16_t ra[8], rb[8];
  if (p.neox) {
    // pair e: (dim 8j+e in a, dim half+8j+e in b)
#pragma unroll
    for (int e = 0; e < 8; ++e) rotate(fa[e], fb[e], cs[8 * j + e], cs[half + 8 * j + e], ra[e], rb[e]);
  } else {
    // pairs 8j..8j+3 in a, 8j+4..8j+7 in b, each (even, odd) adjacent
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      rotate(fa[2 * e], fa[2 * e + 1], cs[8 * j + e], cs[half + 8 * j + e], ra[2 * e], ra[2 * e + 1]);
      rotate(fb[2 * e], fb[2 * e + 1], cs[8 * j + 4 + e], cs[half + 8 * j + 4 + e], rb[2 * e], rb[2 * e + 1]);
    }
  }
  a = pack8(ra);
  b = pack8(rb);
}

__device__ __forceinline__ void unit_dims(const RopeParams& p, int j, int& da, int& db) {
  if (p.neox) {
    da = 8 * j;
    db = (p.rot >> 1) + 8 * j;
  } else {
    da = 16 * j;
    db = 16 * j + 8;
  }
}

__global__ void __launch_bounds__(256) rope_vec_kernel(RopeParams p) {
  const int64_t n = blockIdx.x;
  const int D = p.D;
  const int ru = p.rot / 16;        // rope units per head
  const int pc = (D - p.rot) / 8;   // pass-through chunks per head
  const int vc = D / 8;
  const int q_units = p.Hq * ru, k_units = p.Hkv * ru;
  const int q_pass = p.Hq * pc, k_pass = p.Hkv * pc, v_units = p.Hkv * vc;
  const int total = q_units + k_units + q_pass + k_pass + v_units;
  const float* cs = cs_row(p, n);
  const int64_t loc = load_index(p.cache_locs, p.loc_i64, n);
  const bool loc_ok = loc >= 0 && loc < p.pool_tokens;
  uint16_t* qn = p.q + n * p.q_stride0;
  uint16_t* kn = p.k + n * p.k_stride0;
  const uint16_t* vn = p.v + n * p.v_stride0;
  uint16_t* qp = p.q_pre + n * static_cast<int64_t>(p.Hq) * D;
  uint16_t* kb = p.k_buffer + loc * static_cast<int64_t>(p.Hkv) * D;
  uint16_t* vb = p.v_buffer + loc * static_cast<int64_t>(p.Hkv) * D;
  for (int t = threadIdx.x; t < total; t += blockDim.x) {
    if (t < q_units) {
      const int h = t / ru, j = t - h * ru;
      int da, db;
      unit_dims(p, j, da, db);
      uint16_t* base = qn + h * D;
      uint4 a = *reinterpret_cast<const uint4*>(base + da);
      uint4 b = *reinterpret_cast<const uint4*>(base + db);
      *reinterpret_cast<uint4*>(qp + h * D + da) = a;
      *reinterpret_cast<uint4*>(qp + h * D + db) = b;
      rope_unit(p, cs, j, a, b);
      *reinterpret_cast<uint4*>(base + da) = a;
      *reinterpret_cast<uint4*>(base + db) = b;
      continue;
    }
    int u = t - q_units;
    if (u < k_units) {
      const int h = u / ru, j = u - h * ru;
      int da, db;
      unit_dims(p, j, da, db);
      uint16_t* base = kn + h * D;
      uint4 a = *reinterpret_cast<const uint4*>(base + da);
      uint4 b = *reinterpret_cast<const uint4*>(base + db);
      rope_unit(p, cs, j, a, b);
      *reinterpret_cast<uint4*>(base + da) = a;
      *reinterpret_cast<uint4*>(base + db) = b;
      if (loc_ok) {
        *reinterpret_cast<uint4*>(kb + h * D + da) = a;
        *reinterpret_cast<uint4*>(kb + h * D + db) = b;
      }
      continue;
    }
    u -= k_units;
    if (u < q_pass) {
      const int h = u / pc, c = u - h * pc;
      const int d = p.rot + 8 * c;
      *reinterpret_cast<uint4*>(qp + h * D + d) = *reinterpret_cast<const uint4*>(qn + h * D + d);
      continue;
    }
    u -= q_pass;
    if (u < k_pass) {
      const int h = u / pc, c = u - h * pc;
      const int d = p.rot + 8 * c;
      if (loc_ok) *reinterpret_cast<uint4*>(kb + h * D + d) = *reinterpret_cast<const uint4*>(kn + h * D + d);
      continue;
    }
    u -= k_pass;
    {
      const int h = u / vc, c = u - h * vc;
      if (loc_ok) *reinterpret_cast<uint4*>(vb + h * D + 8 * c) = *reinterpret_cast<const uint4*>(vn + h * D + 8 * c);
    }
  }
}

// Element-wise form for shapes the vector kernel does not cover.
__global__ void __launch_bounds__(256) rope_scalar_kernel(RopeParams p) {
  const int64_t n = blockIdx.x;
  const int D = p.D, half = p.rot >> 1, pass = D - p.rot;
  const int total = p.Hq * half + p.Hkv * half + p.Hq * pass + p.Hkv * pass + p.Hkv * D;
  const float* cs = cs_row(p, n);
  const int64_t loc = load_index(p.cache_locs, p.loc_i64, n);
  const bool loc_ok = loc >= 0 && loc < p.pool_tokens;
  uint16_t* qn = p.q + n * p.q_stride0;
  uint16_t* kn = p.k + n * p.k_stride0;
  const uint16_t* vn = p.v + n * p.v_stride0;
  uint16_t* qp = p.q_pre + n * static_cast<int64_t>(p.Hq) * D;
  uint16_t* kb = p.k_buffer + loc * static_cast<int64_t>(p.Hkv) * D;
  uint16_t* vb = p.v_buffer + loc * static_cast<int64_t>(p.Hkv) * D;
  for (int t = threadIdx.x; t < total; t += blockDim.x) {
    int u = t;
    const bool is_q = u < p.Hq * half;
    if (is_q || u < p.Hq * half + p.Hkv * half) {
      if (!is_q) u -= p.Hq * half;
      const int h = u / half, i = u - h * half;
      const int d0 = p.neox ? i : 2 * i, d1 = p.neox ? i + half : 2 * i + 1;
      uint16_t* base = (is_q ? qn : kn) + h * D;
      const uint16_t x0 = base[d0], x1 = base[d1];
      uint16_t y0, y1;
      rotate(bf16_to_f32(x0), bf16_to_f32(x1), cs[i], cs[half + i], y0, y1);
      base[d0] = y0;
      base[d1] = y1;
      if (is_q) {
        qp[h * D + d0] = x0;
        qp[h * D + d1] = x1;
      } else if (loc_ok) {
        kb[h * D + d0] = y0;
        kb[h * D + d1] = y1;
      }
      continue;
    }
    u -= p.Hq * half + p.Hkv * half;
    if (u < p.Hq * pass) {
      const int h = u / pass, d = p.rot + (u - h * pass);
      qp[h * D + d] = qn[h * D + d];
      continue;
    }
    u -= p.Hq * pass;
    if (u < p.Hkv * pass) {
      const int h = u / pass, d = p.rot + (u - h * pass);
      if (loc_ok) kb[h * D + d] = kn[h * D + d];
      continue;
    }
    u -= p.Hkv * pass;
    if (loc_ok) vb[u] = vn[u];
  }
}

bool aligned16(const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15) == 0; }

}  // namespace

#define REQUIRE(cond, ...) \
  do {                     \
    if (!(cond)) return mac::fail(MAC_ERR_INVALID_ARGUMENT, __VA_ARGS__); \
  } while (0)

extern "C" int mac_decode_rope_preserve_q_bf16(void* q, int64_t q_stride0, void* k, int64_t k_stride0,
                                               const void* v, int64_t v_stride0, void* q_pre, int64_t q_pre_rows,
                                               void* k_buffer, void* v_buffer, int64_t pool_tokens,
                                               const float* cos_sin_cache, int64_t cos_sin_rows,
                                               int64_t cos_sin_stride0, int32_t rotary_dim, const void* positions,
                                               int32_t positions_is_i64, const void* cache_locs,
                                               int32_t cache_locs_is_i64, int64_t N, int32_t Hq, int32_t Hkv,
                                               int32_t head_dim, int32_t is_neox, void* stream) {
  REQUIRE(N >= 0 && N <= INT32_MAX, "bad batch size");
  if (N == 0) return MAC_OK;
  REQUIRE(head_dim > 0 && Hq > 0 && Hkv > 0, "invalid head_dim");
  REQUIRE(rotary_dim > 0 && rotary_dim <= head_dim && (rotary_dim % 2) == 0, "invalid rotary_dim");
  REQUIRE(q_pre_rows >= N, "q_pre shape mismatch");
  REQUIRE(cos_sin_rows > 0 && cos_sin_stride0 >= rotary_dim, "cos_sin_cache shape mismatch");
  REQUIRE(q_stride0 >= static_cast<int64_t>(Hq) * head_dim && k_stride0 >= static_cast<int64_t>(Hkv) * head_dim &&
              v_stride0 >= static_cast<int64_t>(Hkv) * head_dim,
          "q/k/v row stride smaller than the row");
  REQUIRE(q && k && v && q_pre && k_buffer && v_buffer && cos_sin_cache && positions && cache_locs,
          "null pointer argument");
  RopeParams p{};
  p.q = static_cast<uint16_t*>(q);
  p.k = static_cast<uint16_t*>(k);
  p.v = static_cast<const uint16_t*>(v);
  p.q_pre = static_cast<uint16_t*>(q_pre);
  p.k_buffer = static_cast<uint16_t*>(k_buffer);
  p.v_buffer = static_cast<uint16_t*>(v_buffer);
  p.cs = cos_sin_cache;
  p.positions = positions;
  p.cache_locs = cache_locs;
  p.q_stride0 = q_stride0;
  p.k_stride0 = k_stride0;
  p.v_stride0 = v_stride0;
  p.cs_stride0 = cos_sin_stride0;
  p.cs_rows = cos_sin_rows;
  p.pool_tokens = pool_tokens;
  p.Hq = Hq;
  p.Hkv = Hkv;
  p.D = head_dim;
  p.rot = rotary_dim;
  p.pos_i64 = positions_is_i64 != 0;
  p.loc_i64 = cache_locs_is_i64 != 0;
  p.neox = is_neox != 0;
  const bool vec = rotary_dim % 16 == 0 && head_dim % 8 == 0 && q_stride0 % 8 == 0 && k_stride0 % 8 == 0 &&
                   v_stride0 % 8 == 0 && aligned16(q) && aligned16(k) && aligned16(v) && aligned16(q_pre) &&
                   aligned16(k_buffer) && aligned16(v_buffer);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (vec)
    hipLaunchKernelGGL(rope_vec_kernel, dim3(static_cast<unsigned>(N)), dim3(256), 0, s, p);
  else
    hipLaunchKernelGGL(rope_scalar_kernel, dim3(static_cast<unsigned>(N)), dim3(256), 0, s, p);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return mac::fail(MAC_ERR_HIP, "rope launch: %s", hipGetErrorString(e));
  return MAC_OK;
}
