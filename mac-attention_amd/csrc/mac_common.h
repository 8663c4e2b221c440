// mac_common.h -- device helpers shared by the gfx950 MAC kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mac {

constexpr int kHeadDim = 128;      // the only head size the reference supports (DECODE:5081)
constexpr int kMaxGroup = 8;       // largest GQA group (DECODE:5086, kMaxWarps)
constexpr int kBlock = 256;        // threads per workgroup for every decode kernel
constexpr int kWaves = kBlock / 64;
constexpr int kMaxPlanBuckets = 4096;  // entries per class of the task planner's LDS offset table

// bf16 <-> f32.  A 32-bit word holds two bf16 values, low element first.
__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }
__device__ __forceinline__ float bf16_to_f32(uint16_t b) {
  return __uint_as_float(static_cast<uint32_t>(b) << 16);
}
// Round to nearest even; NaN stays NaN.  gfx950's conversion instruction
// (one VALU op, two values when the compiler pairs them) in place of the
// bit arithmetic.
__device__ __forceinline__ uint16_t f32_to_bf16(float f) { return __builtin_bit_cast(uint16_t, static_cast<__bf16>(f)); }
// Two values in one v_cvt_pk_bf16_f32: a in the low half, b in the high.
__device__ __forceinline__ uint32_t pack2_bf16(float a, float b) {
  typedef __bf16 bf16x2_v __attribute__((ext_vector_type(2)));
  const bf16x2_v v = {static_cast<__bf16>(a), static_cast<__bf16>(b)};
  return __builtin_bit_cast(uint32_t, v);
}

__device__ __forceinline__ void unpack8(const uint4& w, float* f) {
  f[0] = bf16_lo(w.x); f[1] = bf16_hi(w.x);
  f[2] = bf16_lo(w.y); f[3] = bf16_hi(w.y);
  f[4] = bf16_lo(w.z); f[5] = bf16_hi(w.z);
  f[6] = bf16_lo(w.w); f[7] = bf16_hi(w.w);
}

// DPP lane exchange within a row of 16 lanes.
template <int kCtrl>
__device__ __forceinline__ float dpp(float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), kCtrl, 0xf, 0xf, false));
}
// Sum over the 16 lanes of a DPP row; every lane of the row receives the total.
__device__ __forceinline__ float row16_sum(float x) {
  x += dpp<0xB1>(x);   // quad_perm [1,0,3,2]
  x += dpp<0x4E>(x);   // quad_perm [2,3,0,1]
  x += dpp<0x141>(x);  // row_half_mirror
  x += dpp<0x140>(x);  // row_mirror
  return x;
}

// Sum over the 8 lanes of a DPP half-row; every lane of it receives the total.
__device__ __forceinline__ float row8_sum(float x) {
  x += dpp<0xB1>(x);   // quad_perm [1,0,3,2]
  x += dpp<0x4E>(x);   // quad_perm [2,3,0,1]
  x += dpp<0x141>(x);  // row_half_mirror
  return x;
}

typedef __bf16 bf16x4_t __attribute__((ext_vector_type(4)));
// gfx950 transposing LDS read (ds_read_b64_tr_b16).  Every lane passes the
// address of four consecutive 16-bit elements; in each group of 16 lanes,
// lane i receives element (i & 3) of the vectors of lanes 4e + (i >> 2),
// e = 0..3.  With lane j pointing at row r0 + (j >> 2), columns c0 + 4 (j & 3)
// of a row-major tile, lane i gets column c0 + i of rows r0 .. r0 + 3: the
// transposed 4 x 16 block, as an MFMA operand wants it.
__device__ __forceinline__ bf16x4_t lds_read_tr16(const uint16_t* p) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4bf16((__attribute__((address_space(3))) bf16x4_t*)(p));
}

// Maximum of finite or infinite floats (no NaN operands): one
// v_maximum3_f32 (IEEE maximum, which needs no quieting of its operands,
// unlike fmaxf's, for which the compiler adds a v_max per operand that may
// come from an MFMA).  Not inline assembly: the compiler does not model an
// inline-assembly instruction's wait for a matrix-core result it reads (the
// window kernel's row maxima read the score MFMA's registers directly), so
// such an instruction could read them before the MFMA had written them.
__device__ __forceinline__ float max3_nonan(float a, float b, float c) {
  return __builtin_elementwise_maximum(__builtin_elementwise_maximum(a, b), c);
}
__device__ __forceinline__ float max8_nonan(const float (&x)[8]) {
  return max3_nonan(max3_nonan(x[0], x[1], x[2]), max3_nonan(x[3], x[4], x[5]), max3_nonan(x[6], x[7], x[7]));
}

// Max and sum over the four lanes l, l ^ 16, l ^ 32, l ^ 48 (one column of
// an MFMA result tile) with gfx950's row-swapping VALU permutes: no LDS
// round trip, so no wait on the wave's outstanding LDS reads.
// v_permlane16_swap(x, x) leaves rows (r, r ^ 1) of x in its two results;
// v_permlane32_swap(x, x) leaves rows (r, r ^ 2).  quad_max takes no NaN
// operands (max3_nonan).
__device__ __forceinline__ float quad_max(float x) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  const float y = max3_nonan(__uint_as_float(a[0]), __uint_as_float(a[1]), __uint_as_float(a[1]));
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(y), __float_as_uint(y), false, false);
  return max3_nonan(__uint_as_float(b[0]), __uint_as_float(b[1]), __uint_as_float(b[1]));
}
__device__ __forceinline__ float quad_sum(float x) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  const float y = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(y), __float_as_uint(y), false, false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

// Marks a loaded value as used here: code depending on it cannot be hoisted
// above this point (the compiler would otherwise unpack a loop-invariant
// load right after issuing it, and the in-order vmcnt wait for it would also
// wait for nothing else in flight).
__device__ __forceinline__ void pin_vgpr(uint4& w) {
  asm volatile("" : "+v"(w.x), "+v"(w.y), "+v"(w.z), "+v"(w.w));
}
__device__ __forceinline__ void pin_vgpr(int& x) { asm volatile("" : "+v"(x)); }

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }
__device__ __forceinline__ float fast_log2(float x) { return __builtin_amdgcn_logf(x); }

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
// Finite "minus infinity" for running maxima: exp2(kNegBig - finite) == 0 and
// exp2(kNegBig - kNegBig) == 1, so empty states merge without NaNs.
constexpr float kNegBig = -1.0e30f;

__host__ __device__ __forceinline__ int ceil_div(int a, int b) { return (a + b - 1) / b; }

// DECODE:713-716
__device__ __forceinline__ int cache_end_for_pos(int p, int s) {
  int e = p + 1 - s;
  return e > 0 ? e : 0;
}

// DECODE:798-807
__device__ __forceinline__ int ring_slot_to_pos(int past_len, int m, int slot) {
  if (past_len < m) return slot;
  int order = slot - past_len % m;
  if (order < 0) order += m;
  return past_len - m + order;
}

// DECODE:837-848
__device__ __forceinline__ int pos_to_ring_slot(int past_len, int m, int pos) {
  if (past_len < m) return pos;
  int slot = pos - (past_len - m) + past_len % m;
  if (slot >= m) slot -= m;
  if (slot < 0) slot += m;
  return slot;
}

// DECODE:809-811: smaller distance wins, ties go to the smaller logical position.
__device__ __forceinline__ bool better_pair(float d, int pos, float best_d, int best_pos) {
  return d < best_d || (d == best_d && pos < best_pos);
}

}  // namespace mac
