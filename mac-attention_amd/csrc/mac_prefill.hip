// mac_prefill.hip -- prefill rectification for MI355X (gfx950).
//
// A ring entry at logical position p holds the attention state of the query
// of p over the keys [0, E), E = p + 1 - S (S = semantic_pos_ahead), so that a
// later decode step that matches it only has to add the band [E, now).  The
// prefill attention computes the state over [0, p + 1); the reference removes
// the trailing window [E, p + 1) with a second, windowed FlashInfer pass and a
// log-sum-exp "downdate" (flashinfer_hooks.py:2436-2482,
// mac_merge_downdate_cache.cu:116-288).  This file provides:
//
//  * downdate_kernel: the reference's downdate op on its own (any head_dim,
//    f32/bf16/f16 lse), for callers that keep the reference's three calls.
//  * window_kernel<HPW, false>: causal sliding-window attention over a
//    ragged batch with a page-size-1 KV pool (the windowed FlashInfer pass).
//  * window_kernel<HPW, true>: the fused form.  Only the rows the ring keeps
//    (the last min(len, M) of each request) are computed; for them the window
//    state never leaves registers: it is downdated from the full state and
//    stored straight into the ring with the pre-RoPE query, followed by the
//    request_length bump (bump_kernel).
//
// Both forms run S^T[key][row] = K Q^T and O^T[d][row] += V^T P^T on
// v_mfma_f32_16x16x32_bf16 as the decode kernel does, with 16 query rows in
// place of the GQA heads: the lane holding row l%16 keeps that row's softmax
// state and 32 O^T accumulators per head.  A workgroup takes 16 rows of one
// request and several query heads of one KV head; its four waves share
// double-buffered LDS K/V tiles of 32 keys.  The layouts are described above
// window_kernel.

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>

#include <algorithm>
#include <climits>
#include <cmath>

#include "mac_attention_amd.h"
#include "mac_common.h"

namespace mac {
int fail(int code, const char* fmt, ...);
}  // namespace mac

namespace {

typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));

using namespace mac;

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ bf16x8_t as_bf16x8(const uint4& w) { return __builtin_bit_cast(bf16x8_t, w); }

// ------------------------------------------------------------- downdate ----

// Control scalars of the downdate (MERGE:148-176), fp32 as in the reference
// so that its branch decisions are reproduced.
struct Downdate {
  float lse;    // new natural-log lse (-inf: nothing left)
  float t;      // weight of the removed state
  float scale;  // renormalisation
};

__device__ __forceinline__ Downdate downdate_control(float l1, float l2) {
  const float diff = l2 - l1;
  const bool last_block = fabsf(expm1f(diff)) <= 1e-7f;
  const bool invalid = diff > 0.0f && !last_block;
  Downdate d;
  if (last_block) {
    d.lse = -INFINITY;
    d.t = 0.0f;
    d.scale = 0.0f;
  } else if (invalid) {
    d.lse = l1;
    d.t = 0.0f;
    d.scale = 1.0f;
  } else {
    d.lse = l1 + logf(fmaxf(1.0f - expf(diff) + 1e-7f, 1e-30f));
    d.t = expf(diff);
    d.scale = expf(l1 - d.lse);
  }
  return d;
}

__device__ __forceinline__ float load_lse(const void* p, int dtype, int64_t i) {
  if (dtype == MAC_DTYPE_F32) return static_cast<const float*>(p)[i];
  const uint16_t b = static_cast<const uint16_t*>(p)[i];
  if (dtype == MAC_DTYPE_BF16) return bf16_to_f32(b);
  return static_cast<float>(__builtin_bit_cast(_Float16, b));
}

__device__ __forceinline__ void store_lse(void* p, int dtype, int64_t i, float v) {
  if (dtype == MAC_DTYPE_F32) {
    static_cast<float*>(p)[i] = v;
  } else if (dtype == MAC_DTYPE_BF16) {
    static_cast<uint16_t*>(p)[i] = f32_to_bf16(v);
  } else {
    static_cast<uint16_t*>(p)[i] = __builtin_bit_cast(uint16_t, static_cast<_Float16>(v));
  }
}

// One 16-lane row group per row; 16 rows per 256-thread workgroup.  Every
// lane reads lse2 before the group's lane 0 overwrites it (same wave, program
// order), so no row reads a half-updated lse.
__global__ void __launch_bounds__(256) downdate_kernel(const uint16_t* __restrict__ out1,
                                                       const void* __restrict__ lse1, int dt1,
                                                       uint16_t* __restrict__ out2, void* __restrict__ lse2,
                                                       int dt2, int64_t rows, int D) {
  // Each 16-lane group takes kR rows at a time (rows g, g + 16, ... of the
  // workgroup's slab) with every load issued before the math; the rows are
  // read once, so o1 and o2 move with the non-temporal policy.
  constexpr int kR = 4;
  const int sub = threadIdx.x & 15;
  const int64_t step = static_cast<int64_t>(gridDim.x) * 16 * kR;
  for (int64_t row0 = static_cast<int64_t>(blockIdx.x) * 16 * kR + (threadIdx.x >> 4); row0 < rows; row0 += step) {
    Downdate c[kR];
#pragma unroll
    for (int k = 0; k < kR; ++k) {
      const int64_t row = min(row0 + 16 * k, rows - 1);
      c[k] = downdate_control(load_lse(lse1, dt1, row), load_lse(lse2, dt2, row));
    }
    if ((D & 7) == 0) {
      for (int e = sub * 8; e < D; e += 128) {
        uint4 wa[kR], wb[kR];
#pragma unroll
        for (int k = 0; k < kR; ++k) {
          const int64_t row = min(row0 + 16 * k, rows - 1);
          wa[k] = __builtin_bit_cast(uint4, __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(out1 + row * D + e)));
          wb[k] = __builtin_bit_cast(uint4, __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(out2 + row * D + e)));
        }
#pragma unroll
        for (int k = 0; k < kR; ++k) {
          if (row0 + 16 * k >= rows) break;
          float fa[8], fb[8];
          unpack8(wa[k], fa);
          unpack8(wb[k], fb);
          uint16_t r[8];
#pragma unroll
          for (int i = 0; i < 8; ++i) r[i] = f32_to_bf16((fa[i] - c[k].t * fb[i]) * c[k].scale);
          u32x4_t w;
          w[0] = r[0] | (static_cast<uint32_t>(r[1]) << 16);
          w[1] = r[2] | (static_cast<uint32_t>(r[3]) << 16);
          w[2] = r[4] | (static_cast<uint32_t>(r[5]) << 16);
          w[3] = r[6] | (static_cast<uint32_t>(r[7]) << 16);
          __builtin_nontemporal_store(w, reinterpret_cast<u32x4_t*>(out2 + (row0 + 16 * k) * D + e));
        }
      }
    } else {
#pragma unroll
      for (int k = 0; k < kR; ++k) {
        const int64_t row = row0 + 16 * k;
        if (row >= rows) break;
        const uint16_t* a = out1 + row * D;
        uint16_t* b = out2 + row * D;
        for (int e = sub; e < D; e += 16)
          b[e] = f32_to_bf16((bf16_to_f32(a[e]) - c[k].t * bf16_to_f32(b[e])) * c[k].scale);
      }
    }
    if (sub == 0) {
#pragma unroll
      for (int k = 0; k < kR; ++k)
        if (row0 + 16 * k < rows) store_lse(lse2, dt2, row0 + 16 * k, c[k].lse);
    }
  }
}

// ------------------------------------------------------ window attention ----

constexpr int kRows = 16;    // query rows per wave
constexpr int kBlk = 32;     // keys per block
constexpr int kMaxB = 4096;  // requests handled by the in-workgroup planner

struct WindowParams {
  const uint16_t* q;  // attention queries [total_q, Hq, 128]
  const uint16_t* k;
  const uint16_t* v;
  const int32_t* qo_indptr;
  const int32_t* kv_indptr;
  const int32_t* kv_indices;
  // plain window attention
  uint16_t* out;
  float* out_lse;
  // fused rectification
  const uint16_t* src_q;
  const uint16_t* o_full;
  const float* lse_full;
  uint16_t* q_cache;
  uint16_t* attn_cache;
  float* lse_cache;
  uint16_t* q_post_cache;
  const int32_t* request_length;
  const int32_t* req_ids;
  int64_t pool_tokens;
  int64_t total_q, kv_len_total;  // rows of q, entries of kv_indices
  int B, Hq, Hkv, R, M;
  int window_left;  // plain mode: keys [pos - window_left, pos]; < 0: [0, pos]
  int S, F, sink_mode;
  int rl_by_batch;
  float q_scale;  // sm_scale * log2(e)
};

// First row of request b that a kernel computes: 0 (plain form: every row),
// or the first of the last min(len, M) rows, which the ring keeps (fused form).
template <bool kRectify>
__device__ __forceinline__ int first_row(int len, int M) {
  return kRectify ? (len > M ? len - M : 0) : 0;
}

// Rows of request b the kernel computes; 0 for requests whose query or key
// ranges fall outside the buffers the caller described, or with fewer keys
// than queries.
template <bool kRectify>
__device__ __forceinline__ int request_rows(const WindowParams& p, int b) {
  const int q0 = p.qo_indptr[b], q1 = p.qo_indptr[b + 1];
  const int k0 = p.kv_indptr[b], k1 = p.kv_indptr[b + 1];
  const int len = q1 - q0, kvlen = k1 - k0;
  const bool ok = q0 >= 0 && q1 <= p.total_q && k0 >= 0 && k1 <= p.kv_len_total && len > 0 && kvlen >= len;
  return ok ? len - first_row<kRectify>(len, p.M) : 0;
}

// Sliding-window attention for GQA groups of any size: the windowed
// FlashInfer pass (kRectify false) or the fused rectification of the rows
// the ring keeps (kRectify true: a window of S keys, optionally the front
// sink [0, min(F, E)) as a second key segment, P fed to the PV product as
// bf16 hi + lo, and the downdate and ring write as epilogue).  A workgroup takes 16 consecutive query rows of one
// request and 4 * HPW query heads of one KV head (HPW heads per wave), so
// every 32-key K/V tile it stages in LDS serves 16 rows x 4 HPW heads.  Per
// wave and block:
//  * S^T = K Q^T: the A operand (K rows) is read once and used for the
//    wave's HPW heads.  Tile t's MFMA row m = 4a + i holds key 8a + 4t + i,
//    so the lane holding row (query) col ends up with the scores of keys
//    8q .. 8q + 7 (q = lane / 16) -- consecutive keys, which is what the PV
//    product's B operand needs.
//  * O^T += V^T P^T: V stays token-major in LDS; the A operand of each
//    16-dim tile, V^T[16 dt + col][8q .. 8q + 7], is two transposing LDS
//    reads (ds_read_b64_tr_b16: in each 16-lane group, lane i receives
//    element i & 3 of the 4-element vectors of lanes 4e + (i >> 2), e < 4),
//    again shared by the wave's heads.
// LDS layouts: K chunk c (16 bytes) of key k at position c ^ (4 ((k >> 3) &
// 3) + (k & 3)) of its 256-byte row, which puts the 16 keys one A-operand
// read touches on 16 different 16-byte bank groups; V row k at byte
// 288 k + 128 (k >> 3) (rows padded to 288 bytes, each group of 8 keys a
// further 128 bytes on): a transposing read takes 32 lanes per cycle, keys
// 8a + 4h + (0..3) and 8a + 8 + 4h + (0..3) x 32 bytes, which this puts on
// the 32 different 8-byte bank pairs of the 64 banks (with the padding alone
// the two key groups collide), and its address stays an immediate offset
// per 16-dim tile.
// Key validity of a block is one 32-bit mask in LDS; a lane turns it into
// the mask of its 8 keys with the row's window bounds by shifts.  The running
// maximum is moved lazily (only when a block exceeds it by 2^8), which leaves
// the result exact and skips most accumulator rescales.

constexpr int kVRow = 18;  // 16-byte units per staged V row: 256 bytes + 32 of padding
// 16-byte position of V row k in the staged tile
__device__ __forceinline__ int v_row(int k) { return k * kVRow + 8 * (k >> 3); }
constexpr int kVTile = kBlk * kVRow + 8 * (kBlk / 8 - 1);  // 16-byte units of a staged V tile

// Residency: the one-head-per-wave window pass fits 168 VGPRs, so it runs
// three workgroups per CU (more waves per SIMD to overlap the softmax VALU
// work with the MFMAs: 7% faster at GQA-4); the others need more registers.
template <int HPW, bool kRectify>
__global__ void __launch_bounds__(256, (HPW == 1 && !kRectify) ? 3 : 2) window_kernel(WindowParams p) {
  // dynamic: s_boff[B + 1] row-block offsets, s_qo[B + 1] / s_kv[B + 1] the
  // request offsets (copies of qo_indptr / kv_indptr)
  extern __shared__ int s_dyn[];
  int* s_boff = s_dyn;
  int* s_qo = s_dyn + (p.B + 1);
  int* s_kv = s_dyn + 2 * (p.B + 1);
  __shared__ int s_part[kWaves];
  __shared__ uint4 s_k[2][kBlk * 16];  // K rows of a 32-key block (swizzled)
  __shared__ uint4 s_v[2][kVTile];  // V rows of the block (v_row layout)
  __shared__ uint32_t s_okw[2][kWaves];  // per wave: bits of its 8 keys that have a pool row

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int quad = lane >> 4;
  const int col = lane & 15;

  // ---- plan: s_boff[b] = sum over b' < b of ceil(rows(b') / 16) ----
  const int B = p.B;
  const int per = ceil_div(B, 256);
  {
    int sum = 0;
    for (int b = tid * per; b < min(B, (tid + 1) * per); ++b) {
      const int n = ceil_div(request_rows<kRectify>(p, b), kRows);
      s_boff[b] = n;  // the count until the prefix replaces it below
      sum += n;
    }
    for (int b = tid; b <= B; b += 256) {
      s_qo[b] = p.qo_indptr[b];
      s_kv[b] = p.kv_indptr[b];
    }
    // exclusive scan of the per-thread sums: inclusive within each wave by
    // lane shifts, then the four wave totals through LDS (one barrier)
    int x = sum;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const int y = __shfl_up(x, off);
      if (lane >= off) x += y;
    }
    if (lane == 63) s_part[wave] = x;
    __syncthreads();
    int acc = x - sum, total = 0;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
      if (w < wave) acc += s_part[w];
      total += s_part[w];
    }
    for (int b = tid * per; b < min(B, (tid + 1) * per); ++b) {
      const int n = s_boff[b];
      s_boff[b] = acc;
      acc += n;
    }
    if (tid == 0) s_boff[B] = total;
    __syncthreads();
  }
  const int Hq = p.Hq, Hkv = p.Hkv;
  const int G = Hq / Hkv;
  constexpr int kHeadsPerTask = 4 * HPW;
  // fused form: the full state's o rows of the task (row r, task head hh,
  // 16-byte part c at r * kOfRow + 16 hh + c; rows padded by one part)
  constexpr int kOfRow = kHeadsPerTask * 16 + 1;
  __shared__ uint4 s_of[kRectify ? kRows * kOfRow : 1];
  const int nchunks = ceil_div(G, kHeadsPerTask);
  const int total_tasks = s_boff[B] * Hkv * nchunks;
  const uint32_t row_bytes = static_cast<uint32_t>(Hkv) * kHeadDim * 2;  // one pool row of K or V
  const unsigned pool_rows = static_cast<unsigned>(min(p.pool_tokens, static_cast<int64_t>(INT_MAX)));
  // keys [pos - wl, pos] form a row's window (wl < 0: [0, pos])
  const int wl = kRectify ? p.S - 1 : p.window_left;
  const bool sink = kRectify && p.sink_mode == 1 && p.F > 0;  // the front sink [0, min(F, E)) as well
  // loader side: thread t stages 16-byte chunk t%16 of keys 2 (t/16) and 2 (t/16) + 1
  const int ld_key = 2 * (tid >> 4), ld_chunk = tid & 15;
  const int ld_pk0 = ld_key * 16 + (ld_chunk ^ (4 * ((ld_key >> 3) & 3) + (ld_key & 3)));
  const int ld_pk1 = (ld_key + 1) * 16 + (ld_chunk ^ (4 * (((ld_key + 1) >> 3) & 3) + ((ld_key + 1) & 3)));
  const int ld_pv0 = v_row(ld_key) + ld_chunk;
  const int ld_pv1 = v_row(ld_key + 1) + ld_chunk;
  // compute side: K A-operand positions (tile t, k-step s) and V^T read
  // addresses (16-dim tile dt, half h) of this lane
  int pk[2][4];
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    const int key = 8 * (col >> 2) + 4 * t + (col & 3);
    const int sw = 4 * ((key >> 3) & 3) + (key & 3);
#pragma unroll
    for (int s = 0; s < 4; ++s) pk[t][s] = key * 16 + ((4 * s + quad) ^ sw);
  }
  // V^T: lane j = col of group quad reads key 8 quad + 4 h + (j >> 2), dims
  // 16 dt + 4 (j & 3) .. + 3: element offset pv[h] + 16 dt of the V tile
  int pv[2];
#pragma unroll
  for (int h = 0; h < 2; ++h) pv[h] = v_row(8 * quad + 4 * h + (col >> 2)) * 8 + 4 * (col & 3);

  // Task order, by form (measured at config 4's prefill shape):
  //  * windowed (plain, window_left >= 0): (KV head, head chunk) major, row
  //    block minor, and within each full round of the grid XCD x (the
  //    workgroups w with w % 8 == x, as the dispatcher deals them) takes the
  //    x-th contiguous eighth of the round's tasks: the row blocks sharing a
  //    K/V row run together under one L2 (row-block order dealt round-robin
  //    put them on different XCDs and fetched each K/V row about four times);
  //  * fused: row-block order (the KV heads of a row block together), XCD
  //    eighths as above (2-3% faster than round-robin; head-major was slower);
  //  * causal (window_left < 0): row-block order dealt round-robin.  Its
  //    tasks grow with the row block, and a workgroup keeps its offset within
  //    every round, so a head-major order would give some workgroups only the
  //    longest tasks.
  const int grid = gridDim.x;
  const int eighth = grid / 8;
  const int nblocks = s_boff[B];
  const bool head_major = !kRectify && wl >= 0;
  const bool by_xcd = (kRectify || wl >= 0) && grid % 8 == 0;
  for (int task = blockIdx.x; task < total_tasks; task += grid) {
    __syncthreads();  // the previous task's waves are done with the tiles
    const int round0 = task - static_cast<int>(blockIdx.x);
    const int t = (by_xcd && round0 + grid <= total_tasks)
                      ? round0 + (static_cast<int>(blockIdx.x) % 8) * eighth + static_cast<int>(blockIdx.x) / 8
                      : task;
    int blk, hc;  // row block; KV head * nchunks + head chunk
    if (head_major) {
      hc = t / nblocks;
      blk = t - hc * nblocks;
    } else {
      blk = t / (Hkv * nchunks);
      hc = t - blk * Hkv * nchunks;
    }
    const int hkv = hc / nchunks;
    const int hg0 = kHeadsPerTask * (hc - hkv * nchunks) + HPW * wave;  // first head of this wave in the group
    int lo = 0, hi = B - 1;  // request of this row block: largest b with s_boff[b] <= blk
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (s_boff[mid] <= blk) lo = mid;
      else hi = mid - 1;
    }
    const int b = lo;
    const int len = s_qo[b + 1] - s_qo[b];
    const int kvlen = s_kv[b + 1] - s_kv[b];
    const int64_t kv_begin = s_kv[b];
    const int r_local = first_row<kRectify>(len, p.M) + kRows * (blk - s_boff[b]);
    const int nrows = min(kRows, len - r_local);
    const int pos0 = kvlen - len + r_local;
    const int pos_last = pos0 + nrows - 1;
    const bool row_ok = col < nrows;
    const int pos = pos0 + col;  // this lane's row position
    const int64_t grow = static_cast<int64_t>(s_qo[b]) + r_local + (row_ok ? col : 0);
    const int w_lo = wl < 0 ? 0 : max(pos - wl, 0);  // this row's window [w_lo, pos]
    // this request's kv_indices; entry offsets fit 32 bits (fewer than 2^30
    // entries, checked on the host), so a load is a uniform base plus a
    // 32-bit lane offset
    const char* kvi = reinterpret_cast<const char*>(p.kv_indices + kv_begin);
    auto index_at = [&](int key) -> int {  // entry of a key, clamped into the request
      return *reinterpret_cast<const int*>(kvi + min(static_cast<uint32_t>(key), static_cast<uint32_t>(kvlen - 1)) * 4u);
    };
    // The entries of the first segment's first two blocks (the loader's keys)
    // go out first, ahead of the Q rows and the epilogue's inputs: the first
    // K/V loads then wait for these entries only, not for everything issued
    // before them (the memory counter retires loads in order).
    const int seg_first = sink ? 0 : 1;
    const int lo_first = seg_first == 0 ? 0 : (wl < 0 ? 0 : max(pos0 - wl, 0));
    int pre_raw[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) pre_raw[t] = index_at(lo_first + (t >> 1) * kBlk + ld_key + (t & 1));
    __builtin_amdgcn_sched_barrier(0);  // (kept ahead of the loads below)
    // fused form: the epilogue's inputs that do not depend on the attention,
    // loaded now so that their latency hides behind it
    int req = 0, before = 0;
    float lse_full[HPW];
    if (kRectify) {
      req = p.req_ids[b];
      const bool req_ok = req >= 0 && req < p.R;
      before = p.rl_by_batch ? p.request_length[b] : p.request_length[req_ok ? req : 0];
#pragma unroll
      for (int i = 0; i < HPW; ++i) lse_full[i] = p.lse_full[grow * Hq + hkv * G + min(hg0 + i, G - 1)];
    }
    const int nheads = __builtin_amdgcn_readfirstlane(max(0, min(HPW, G - hg0)));  // heads this wave computes
    // Fused form: the task's pre-RoPE query rows (copied into the ring with
    // the q_post NaN marker) and the full state's o rows (into s_of for the
    // epilogue) -- 16 rows x kHeadsPerTask heads x 16 parts of 16 bytes,
    // kHeadsPerTask rounds of one part per thread -- move with the K/V
    // stream, so that this traffic overlaps the compute-bound key blocks
    // instead of adding an HBM-bound load round after them (every workgroup
    // runs its task in step with the others).  A round's loads go out behind
    // a block's K/V loads; its query part is stored when the next block is
    // staged, and its o part is copied straight into LDS
    // (global_load_lds_dwordx4: no registers; waited for at the next
    // block's staging and barrier).  Round k, thread t: row (16 k + t / 16) /
    // kHeadsPerTask, task head (t / 16) % kHeadsPerTask, part t % 16 -- the
    // 64 lanes of a wave take 4 heads x 16 parts of one row, a contiguous
    // 1 KiB run of s_of, which is the run a wave's copy fills.
    const int cq_hh = (tid >> 4) % kHeadsPerTask;
    const int cq_part = tid & 15;
    const int cq_h = kHeadsPerTask * (hc - hkv * nchunks) + cq_hh;  // its head in the group
    const bool cq_req = kRectify && req >= 0 && req < p.R;
    int cq = 0;               // rounds issued (uniform)
    bool cq_pending = false;  // round cq - 1 loaded, its query part not yet stored
    uint4 cq_src = make_uint4(0, 0, 0, 0);
    auto cq_row = [&](int k) { return (16 * k + (tid >> 4)) / kHeadsPerTask; };
    auto cq_issue = [&](int k) {
      const int r = min(cq_row(k), nrows - 1);  // (rows past the block: a valid address, not stored)
      const int64_t e = ((static_cast<int64_t>(s_qo[b]) + r_local + r) * Hq + hkv * G + min(cq_h, G - 1)) * kHeadDim +
                        8 * cq_part;
      cq_src = *reinterpret_cast<const uint4*>(p.src_q + e);
      // the wave's run: row (16 k + 4 wave) / kHeadsPerTask, heads from (4 wave) % kHeadsPerTask
      uint4* run = &s_of[((16 * k + 4 * wave) / kHeadsPerTask) * kOfRow + 16 * ((4 * wave) % kHeadsPerTask)];
      __builtin_amdgcn_global_load_lds(static_cast<const void*>(p.o_full + e),
                                       (__attribute__((address_space(3))) void*)(run), 16, 0, 0);
    };
    auto cq_store = [&](int k) {
      const int r = cq_row(k);
      if (cq_req && r < nrows && cq_h < G) {
        const int slot = static_cast<int>((static_cast<int64_t>(max(before, 0)) + r_local + r) % p.M);
        const int64_t e = ((static_cast<int64_t>(req) * p.M + slot) * Hq + hkv * G + cq_h) * kHeadDim + 8 * cq_part;
        *reinterpret_cast<uint4*>(p.q_cache + e) = cq_src;
        if (p.q_post_cache != nullptr)
          *reinterpret_cast<uint4*>(p.q_post_cache + e) = make_uint4(0x7fc07fc0u, 0x7fc07fc0u, 0x7fc07fc0u, 0x7fc07fc0u);
      }
    };

    // Q rows of the wave's heads (B operands): lane (quad, col) holds
    // Q[row col][8 (4s + quad) .. +8].  A lane past the block's rows reads
    // the block's first row and an absent head reads the group's first head
    // (valid data, never zeroed): every score of such a lane is masked
    // (kmask 0), an absent head is never stored, and each head keeps its own
    // softmax state.  With no select on the loaded values no wait follows
    // the loads: the Q rows and the first entries are one round of loads.
    uint4 qreg[HPW][4];
#pragma unroll
    for (int i = 0; i < HPW; ++i) {
      const int h = hkv * G + (hg0 + i < G ? hg0 + i : 0);
      const uint16_t* qp = p.q + (grow * Hq + h) * kHeadDim;
#pragma unroll
      for (int s = 0; s < 4; ++s) qreg[i][s] = *reinterpret_cast<const uint4*>(qp + 8 * (4 * s + quad));
    }

    // l[h]: the softmax row sums.  Plain form: the lane's fp32 partial sums
    // in l[h][0] (reduced over the row's four lanes at the end).  Fused form:
    // accumulated by MFMAs with an all-ones A operand over P = hi + lo (every
    // element of the lane's l[h] then holds its row's sum), off the VALU; the
    // plain form cannot do that, since its P is bf16 hi alone and the sum of
    // that is ~2^-9 off per key, beyond what its lse output allows.
    float m[HPW];
    f32x4_t acc[HPW][8], l[HPW];
#pragma unroll
    for (int i = 0; i < HPW; ++i) {
      m[i] = kNegBig;
      l[i] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int dt = 0; dt < 8; ++dt) acc[i][dt] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
    }

    const char* kbase = reinterpret_cast<const char*>(p.k + static_cast<int64_t>(hkv) * kHeadDim + ld_chunk * 8);
    const char* vbase = reinterpret_cast<const char*>(p.v + static_cast<int64_t>(hkv) * kHeadDim + ld_chunk * 8);
    bool fresh = true;  // no block computed yet: the first sets m without a rescale
    auto ld = [&](const char* base, int r) -> uint4 {  // one v_mad_u64_u32 per address
      return *reinterpret_cast<const uint4*>(base + static_cast<uint64_t>(static_cast<uint32_t>(max(r, 0))) * row_bytes);
    };
    // the loader's K/V chunks of the block in flight (rc0/rc1: their rows,
    // -1: masked) and the raw indices of the block after it
    int rc0 = -1, rc1 = -1, rn0 = 0, rn1 = 0;
    uint4 kq0 = make_uint4(0, 0, 0, 0), kq1 = kq0, vq0 = kq0, vq1 = kq0;
    {
      // the first segment's block 0 goes in flight here, right behind the Q
      // rows (issued in the segment loop, its loads would wait for every
      // load before them: the loop's entry joins the counts)
      const int hi_first = seg_first == 0 ? min(p.F, max(pos_last - wl, 0)) : pos_last + 1;
      if (hi_first > lo_first) {
        const int k0 = lo_first + ld_key;
        rc0 = (k0 < hi_first && static_cast<unsigned>(pre_raw[0]) < pool_rows) ? pre_raw[0] : -1;
        rc1 = (k0 + 1 < hi_first && static_cast<unsigned>(pre_raw[1]) < pool_rows) ? pre_raw[1] : -1;
        kq0 = ld(kbase, rc0);
        kq1 = ld(kbase, rc1);
        vq0 = ld(vbase, rc0);
        vq1 = ld(vbase, rc1);
        rn0 = pre_raw[2];
        rn1 = pre_raw[3];
      }
    }
    // segment 0: the front sink [0, min(F, w_lo)) of each row (fused form,
    // sink_mode 1); segment 1: the window [w_lo, pos]
    for (int seg = seg_first; seg < 2; ++seg) {
      const int seg_lo = seg == 0 ? 0 : (wl < 0 ? 0 : max(pos0 - wl, 0));
      const int seg_hi = seg == 0 ? min(p.F, max(pos_last - wl, 0)) : pos_last + 1;
      const int r_lo = seg == 0 ? 0 : w_lo;  // this row's keys in the segment: [r_lo, r_hi)
      const int r_hi = seg == 0 ? min(p.F, w_lo) : pos + 1;
      const int nblk = seg_hi > seg_lo ? ceil_div(seg_hi - seg_lo, kBlk) : 0;
      // The loader's key ld_key + t of block i: its kv_indices entry (the load
      // only, index clamped into the request) and, checked later, its pool row
      // (-1: masked).  An index is loaded one block before it is checked, so
      // the wait for it never includes K/V loads issued after it (the memory
      // counter retires in order).
      auto index_of = [&](int i, int t) -> int { return index_at(seg_lo + i * kBlk + ld_key + t); };
      auto row_of = [&](int i, int t, int raw) -> int {
        const int key = seg_lo + i * kBlk + ld_key + t;
        return (key < seg_hi && static_cast<unsigned>(raw) < pool_rows) ? raw : -1;
      };
      if (seg != seg_first && nblk > 0) {  // (the first segment's block 0 is in flight)
        rc0 = row_of(0, 0, index_of(0, 0));
        rc1 = row_of(0, 1, index_of(0, 1));
        kq0 = ld(kbase, rc0);
        kq1 = ld(kbase, rc1);
        vq0 = ld(vbase, rc0);
        vq1 = ld(vbase, rc1);
        rn0 = index_of(1, 0);
        rn1 = index_of(1, 1);
      }
      for (int i = 0; i < nblk; ++i) {
        const int buf = i & 1;
        // stage block i: K and V rows (V of masked keys zeroed), key validity bits
        {
          s_k[buf][ld_pk0] = kq0;
          s_k[buf][ld_pk1] = kq1;
          const uint64_t b0 = __ballot(rc0 >= 0), b1 = __ballot(rc1 >= 0);
          if ((b0 & b1) != ~0ull) {  // a masked key in the wave's rows: zero its V row (P is 0 there, V may be NaN)
            const uint32_t z0 = rc0 >= 0 ? 0xffffffffu : 0u, z1 = rc1 >= 0 ? 0xffffffffu : 0u;
            vq0 = make_uint4(vq0.x & z0, vq0.y & z0, vq0.z & z0, vq0.w & z0);
            vq1 = make_uint4(vq1.x & z1, vq1.y & z1, vq1.z & z1, vq1.w & z1);
          }
          s_v[buf][ld_pv0] = vq0;
          s_v[buf][ld_pv1] = vq1;
          if (kRectify && cq_pending) {
            cq_store(cq - 1);
            cq_pending = false;
          }
          if (lane == 0) {
            // lanes 16 r hold keys 8 wave + 2 r and 8 wave + 2 r + 1
            uint32_t bits = 0;
#pragma unroll
            for (int r = 0; r < 4; ++r)
              bits |= static_cast<uint32_t>(((b0 >> (16 * r)) & 1) | (((b1 >> (16 * r)) & 1) << 1)) << (2 * r);
            s_okw[buf][wave] = bits;
          }
        }
        __syncthreads();  // block i visible; every wave is done with block i - 2 (same buffer)
        // block i + 1 in flight while block i is computed
        if (i + 1 < nblk) {
          rc0 = row_of(i + 1, 0, rn0);
          rc1 = row_of(i + 1, 1, rn1);
          kq0 = ld(kbase, rc0);
          kq1 = ld(kbase, rc1);
          vq0 = ld(vbase, rc0);
          vq1 = ld(vbase, rc1);
          rn0 = index_of(i + 2, 0);  // clamped: harmless past the last block
          rn1 = index_of(i + 2, 1);
        }
        if (kRectify && cq < kHeadsPerTask) {
          cq_issue(cq);
          ++cq;
          cq_pending = true;
        }
        if (nheads == 0) continue;
        const int base = seg_lo + i * kBlk;

        // K A operands of both score tiles (row m = 4a + i <-> key 8a + 4t + i)
        // and V A operands of the eight 16-dim tiles, all issued up front
        uint4 ka[2][4];
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
          for (int s = 0; s < 4; ++s) ka[t][s] = s_k[buf][pk[t][s]];
        const uint16_t* vtile = reinterpret_cast<const uint16_t*>(&s_v[buf][0]);
        bf16x8_t va[8];
#pragma unroll
        for (int dt = 0; dt < 8; ++dt)
          va[dt] = __builtin_shufflevector(lds_read_tr16(vtile + pv[0] + 16 * dt), lds_read_tr16(vtile + pv[1] + 16 * dt),
                                           0, 1, 2, 3, 4, 5, 6, 7);
        // mask of the lane's keys 8 quad + e: a pool row, and inside [r_lo, r_hi)
        uint32_t kmask = s_okw[buf][quad];
        {
          const int k0 = base + 8 * quad;
          const int lo_e = min(max(r_lo - k0, 0), 8), hi_e = min(max(r_hi - k0, 0), 8);
          kmask &= ((1u << hi_e) - 1u) & ~((1u << lo_e) - 1u);
          if (!row_ok) kmask = 0;
        }
        // blocks inside every row's range with every key present need no masks
        const bool full = !__any(kmask != 0xffu);
        // raw scores of both tiles and every head, the four accumulation chains
        // interleaved (an absent head is computed but never stored)
        f32x4_t c4[HPW][2];
#pragma unroll
        for (int h = 0; h < HPW; ++h)
#pragma unroll
          for (int t = 0; t < 2; ++t) c4[h][t] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int s = 0; s < 4; ++s)
#pragma unroll
          for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int h = 0; h < HPW; ++h)
              c4[h][t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(ka[t][s]), as_bf16x8(qreg[h][s]), c4[h][t],
                                                                0, 0, 0);
        if (!full) {  // masked keys -> -inf, the lane's eight bits decoded once for all heads
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const bool keep = (kmask >> e) & 1;
#pragma unroll
            for (int h = 0; h < HPW; ++h) c4[h][e >> 2][e & 3] = keep ? c4[h][e >> 2][e & 3] : -INFINITY;
          }
        }
        bf16x8_t pb[HPW], pl[HPW];
#pragma unroll
        for (int h = 0; h < HPW; ++h) {
          // the softmax scale is applied inside exp2: m[h] is a raw score,
          // p = 2^(q_scale (s - m))
          float sv[8];
#pragma unroll
          for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int r = 0; r < 4; ++r) sv[4 * t + r] = c4[h][t][r];
          // lazy move of the reference point: p <= 2^8 stays exact in fp32.
          // The vote runs on each lane's own maximum (the four lanes of a
          // row share m[h], so any lane exceeding it is the row maximum
          // exceeding it): the row reduction is only needed when the point
          // moves.  On the first block every present key moves it (acc and
          // l are still zero, and the rescale by 2^(kNegBig - m_new) = 0
          // leaves them zero).
          float bmax = max8_nonan(sv);
          const float vote = fresh ? -INFINITY : m[h] * p.q_scale + 8.0f;
          if (__any(bmax * p.q_scale > vote)) {
            bmax = quad_max(bmax);
            const float m_new = max3_nonan(m[h], bmax, bmax);
            const float alpha = fast_exp2((m[h] - m_new) * p.q_scale);
            m[h] = m_new;
            if (kRectify) l[h] *= alpha;
            else l[h][0] *= alpha;
#pragma unroll
            for (int dt = 0; dt < 8; ++dt) acc[h][dt] *= alpha;
          }
          const float mo = -m[h] * p.q_scale;
          float psum = 0.0f;
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const float pe = fast_exp2(fmaf(sv[e], p.q_scale, mo));
            if (!kRectify) psum = e == 0 ? pe : psum + pe;  // (0 + pe = pe: no add)
            pb[h][e] = static_cast<__bf16>(pe);
            // The fused form also feeds the bf16 rounding residual of P
            // through a second MFMA (P = hi + lo, ~16 significant bits): the
            // downdate divides the window's contribution by the prefix's
            // share of the softmax mass, which amplifies any error of the
            // window state.
            if (kRectify) pl[h][e] = static_cast<__bf16>(pe - static_cast<float>(pb[h][e]));
          }
          if (!kRectify) l[h][0] += psum;
        }
        fresh = false;
        // O^T += V^T P^T (fused form: l += 1^T P^T as well)
        const bf16x8_t ones = as_bf16x8(make_uint4(0x3f803f80u, 0x3f803f80u, 0x3f803f80u, 0x3f803f80u));
#pragma unroll
        for (int h = 0; h < HPW; ++h) {
          if (kRectify) {
            l[h] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ones, pb[h], l[h], 0, 0, 0);
            l[h] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ones, pl[h], l[h], 0, 0, 0);
          }
        }
#pragma unroll
        for (int dt = 0; dt < 8; ++dt)
#pragma unroll
          for (int h = 0; h < HPW; ++h) {
            acc[h][dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(va[dt], pb[h], acc[h][dt], 0, 0, 0);
            if (kRectify) acc[h][dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(va[dt], pl[h], acc[h][dt], 0, 0, 0);
          }
      }
      if (seg == 0) __syncthreads();  // the sink's last tiles are read before the window stages into them
    }
    if (kRectify) {  // the rounds the blocks did not carry; then s_of is complete for every wave
      if (cq_pending) cq_store(cq - 1);
      for (; cq < kHeadsPerTask; ++cq) {
        cq_issue(cq);
        cq_store(cq);
      }
      __syncthreads();
    }
    if (nheads == 0 || !row_ok) continue;

    if (!kRectify) {
#pragma unroll
      for (int h = 0; h < HPW; ++h) {
        if (h >= nheads) break;
        const float lt = quad_sum(l[h][0]);
        const float inv = lt > 0.0f ? 1.0f / lt : 0.0f;
        const int hq = hkv * G + hg0 + h;
        uint16_t* op = p.out + (grow * Hq + hq) * kHeadDim + 4 * quad;
#pragma unroll
        for (int dt = 0; dt < 8; ++dt) {
          uint2 w;
          w.x = pack2_bf16(acc[h][dt][0] * inv, acc[h][dt][1] * inv);
          w.y = pack2_bf16(acc[h][dt][2] * inv, acc[h][dt][3] * inv);
          *reinterpret_cast<uint2*>(op + 16 * dt) = w;
        }
        if (quad == 0) p.out_lse[grow * Hq + hq] = lt > 0.0f ? (m[h] * p.q_scale + fast_log2(lt)) * kLn2 : -INFINITY;
      }
      continue;
    }

    // ---- fused: downdate the full state, store the ring row ----
    if (req < 0 || req >= p.R) continue;
    if (before < 0) before = 0;
    const int local = r_local + col;  // row index within the request
    const int slot = static_cast<int>((static_cast<int64_t>(before) + local) % p.M);
    const int64_t drow = static_cast<int64_t>(req) * p.M + slot;
    const bool empty = pos + 1 - p.S <= (sink ? p.F : 0);  // nothing left after the downdate
    // the full state's o of the lane's row, dims 16 dt + 4 quad .. + 3 of
    // each of the wave's heads, from s_of
    uint32_t fow[HPW][16];
    const uint2* of2 = reinterpret_cast<const uint2*>(s_of);
#pragma unroll
    for (int hh = 0; hh < HPW; ++hh) {
#pragma unroll
      for (int dt = 0; dt < 8; ++dt) {
        const uint2 f = of2[2 * (col * kOfRow + 16 * (HPW * wave + hh) + 2 * dt + (quad >> 1)) + (quad & 1)];
        fow[hh][2 * dt] = f.x;
        fow[hh][2 * dt + 1] = f.y;
      }
    }
#pragma unroll
    for (int hh = 0; hh < HPW; ++hh) {
      if (hh >= nheads) break;
      const int h = hkv * G + hg0 + hh;
      const float lt = l[hh][0];
      const float inv = lt > 0.0f ? 1.0f / lt : 0.0f;
      const float lse_w = lt > 0.0f ? (m[hh] * p.q_scale + fast_log2(lt)) * kLn2 : -INFINITY;
      Downdate c;
      if (empty) {
        c.lse = -INFINITY;
        c.t = 0.0f;
        c.scale = 0.0f;
      } else {
        c = downdate_control(lse_full[hh], lse_w);
      }
      uint16_t* ap = p.attn_cache + (drow * Hq + h) * kHeadDim + 4 * quad;
#pragma unroll
      for (int dt = 0; dt < 8; ++dt) {
        float r[4];
        const uint32_t fx = fow[hh][2 * dt], fy = fow[hh][2 * dt + 1];
        const float fo[4] = {bf16_lo(fx), bf16_hi(fx), bf16_lo(fy), bf16_hi(fy)};
#pragma unroll
        for (int i = 0; i < 4; ++i) r[i] = empty ? 0.0f : (fo[i] - c.t * (acc[hh][dt][i] * inv)) * c.scale;
        uint2 w;
        w.x = pack2_bf16(r[0], r[1]);
        w.y = pack2_bf16(r[2], r[3]);
        *reinterpret_cast<uint2*>(ap + 16 * dt) = w;
      }
      if (quad == 0) p.lse_cache[drow * Hq + h] = (p.sink_mode == 0 && p.F > 0) ? -INFINITY : c.lse;
      // (the pre-RoPE query row and the NaN marker of the unknown post-RoPE
      // row, PREFILL:251-262, went into the ring with the key blocks)
    }
  }
}

// request_length[req] += len (indexed-by-request form, after the ring rows
// were addressed with the old value) for every request the window kernel
// wrote: the validity test of request_rows, a request it skipped is not bumped.
__global__ void bump_kernel(int32_t* request_length, const int32_t* req_ids, const int32_t* qo_indptr,
                            const int32_t* kv_indptr, int64_t total_q, int64_t kv_len_total, int B, int R) {
  const int b = blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= B) return;
  const int req = req_ids[b];
  const int q0 = qo_indptr[b], q1 = qo_indptr[b + 1];
  const int k0 = kv_indptr[b], k1 = kv_indptr[b + 1];
  const int len = q1 - q0;
  const bool ok = q0 >= 0 && q1 <= total_q && k0 >= 0 && k1 <= kv_len_total && len > 0 && k1 - k0 >= len;
  if (!ok || req < 0 || req >= R) return;
  atomicAdd(&request_length[req], len);
}

// Workgroups for `tasks` wave-sized units of work (4 per workgroup), at most
// as many as are resident at once (`kernel`'s occupancy on every CU), since
// the kernels loop over their tasks.
int grid_for(int64_t tasks, const void* kernel, size_t dyn_lds = 0) {
  int dev = 0, cus = 256, per_cu = 2;
  if (hipGetDevice(&dev) == hipSuccess) {
    int v = 0;
    if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && v > 0) cus = v;
    int occ = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, kernel, 256, dyn_lds) == hipSuccess && occ > 0) per_cu = occ;
  }
  const int64_t wgs = (tasks + 3) / 4;
  return static_cast<int>(std::max<int64_t>(1, std::min<int64_t>(wgs, static_cast<int64_t>(cus) * per_cu)));
}

// Launches the window kernel over `blocks` (a bound on the 16-row blocks of
// the batch): two query heads per wave when the GQA group has more than four.
template <bool kRectify>
void launch_window(const WindowParams& p, int64_t blocks, hipStream_t stream) {
  const int G = p.Hq / p.Hkv;
  const size_t lds = 3 * sizeof(int) * (static_cast<size_t>(p.B) + 1);
  if (G <= 4) {
    const void* kern = reinterpret_cast<const void*>(&window_kernel<1, kRectify>);
    hipLaunchKernelGGL((window_kernel<1, kRectify>), dim3(grid_for(4 * blocks * p.Hkv * ceil_div(G, 4), kern, lds)),
                       dim3(256), lds, stream, p);
  } else {
    const void* kern = reinterpret_cast<const void*>(&window_kernel<2, kRectify>);
    hipLaunchKernelGGL((window_kernel<2, kRectify>), dim3(grid_for(4 * blocks * p.Hkv * ceil_div(G, 8), kern, lds)),
                       dim3(256), lds, stream, p);
  }
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

extern "C" int mac_update_then_downdate_bf16_inplace(const void* out1, const void* lse1, int32_t lse1_dtype,
                                                     void* out2, void* lse2, int32_t lse2_dtype, int64_t rows,
                                                     int32_t head_dim, void* stream) {
  REQUIRE(rows >= 0, "rows must be >= 0");
  REQUIRE(head_dim > 0, "head_dim must be > 0");
  REQUIRE(lse1_dtype >= MAC_DTYPE_F32 && lse1_dtype <= MAC_DTYPE_F16, "lse1 must be float32, bfloat16, or float16");
  REQUIRE(lse2_dtype >= MAC_DTYPE_F32 && lse2_dtype <= MAC_DTYPE_F16, "lse2 must be float32, bfloat16, or float16");
  if (rows == 0) return MAC_OK;
  REQUIRE(out1 && out2 && lse1 && lse2, "null pointer argument");
  if ((head_dim & 7) == 0)
    REQUIRE((reinterpret_cast<uintptr_t>(out1) & 15) == 0 && (reinterpret_cast<uintptr_t>(out2) & 15) == 0,
            "out tensors must be 16-byte aligned");
  const int64_t wgs = std::min<int64_t>((rows + 63) / 64, 65536);
  hipLaunchKernelGGL(downdate_kernel, dim3(static_cast<unsigned>(wgs)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), static_cast<const uint16_t*>(out1), lse1, lse1_dtype,
                     static_cast<uint16_t*>(out2), lse2, lse2_dtype, rows, head_dim);
  HIP_OK(hipGetLastError());
  return MAC_OK;
}

namespace {

// the kernels move bf16 rows with 16-byte vector accesses
bool aligned16(const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15) == 0; }

int check_window_common(int B, int Hq, int Hkv, int D, int64_t total_q, int64_t pool, const void* q,
                        const void* k, const void* v, const int32_t* qo, const int32_t* kvp, const int32_t* kvi,
                        int64_t kv_len) {
  REQUIRE(D == kHeadDim, "head_dim must be 128 (got %d)", D);
  REQUIRE(Hq > 0 && Hkv > 0 && Hq % Hkv == 0, "Hq must be a positive multiple of Hkv");
  REQUIRE(B >= 0 && B <= kMaxB, "B must be in [0, %d] (got %d)", kMaxB, B);
  REQUIRE(total_q >= 0 && total_q <= INT_MAX && pool > 0, "bad total_q / pool_tokens");
  REQUIRE(total_q * Hq <= static_cast<int64_t>(INT_MAX) * 64, "total_q too large");
  REQUIRE(q && k && v && qo && kvp && kvi, "null pointer argument");
  REQUIRE(aligned16(q) && aligned16(k) && aligned16(v), "q, k and v must be 16-byte aligned");
  // the window kernel addresses a request's kv_indices with 32-bit byte offsets
  REQUIRE(kv_len >= 0 && kv_len < (int64_t{1} << 30), "kv_indices must hold fewer than 2^30 entries");
  return MAC_OK;
}

}  // namespace

extern "C" int mac_prefill_window_attention_bf16(const MacWindowAttentionArgs* a, void* stream) {
  REQUIRE(a != nullptr, "args is NULL");
  REQUIRE(a->struct_size == sizeof(MacWindowAttentionArgs), "struct_size mismatch (%u vs %zu)", a->struct_size,
          sizeof(MacWindowAttentionArgs));
  REQUIRE(a->abi_version == MAC_ABI_VERSION, "abi_version mismatch");
  if (int rc = check_window_common(a->B, a->Hq, a->Hkv, a->D, a->total_q, a->pool_tokens, a->q, a->k_buffer,
                                   a->v_buffer, a->qo_indptr, a->kv_indptr, a->kv_indices, a->kv_indices_len))
    return rc;
  REQUIRE(a->out && a->out_lse, "out / out_lse must not be NULL");
  REQUIRE(aligned16(a->out), "out must be 16-byte aligned");
  if (a->B == 0 || a->total_q == 0) return MAC_OK;
  WindowParams p{};
  p.q = static_cast<const uint16_t*>(a->q);
  p.k = static_cast<const uint16_t*>(a->k_buffer);
  p.v = static_cast<const uint16_t*>(a->v_buffer);
  p.qo_indptr = a->qo_indptr;
  p.kv_indptr = a->kv_indptr;
  p.kv_indices = a->kv_indices;
  p.out = static_cast<uint16_t*>(a->out);
  p.out_lse = a->out_lse;
  p.pool_tokens = a->pool_tokens;
  p.total_q = a->total_q;
  p.kv_len_total = a->kv_indices_len;
  p.B = a->B;
  p.Hq = a->Hq;
  p.Hkv = a->Hkv;
  p.M = 1;
  p.window_left = a->window_left;
  p.q_scale = static_cast<float>(a->sm_scale * 1.4426950408889634);
  const int64_t blocks = (a->total_q + kRows - 1) / kRows + a->B;
  launch_window<false>(p, blocks, static_cast<hipStream_t>(stream));
  HIP_OK(hipGetLastError());
  return MAC_OK;
}

extern "C" int mac_prefill_rectify_update_cache_bf16(const MacRectifyArgs* a, void* stream) {
  REQUIRE(a != nullptr, "args is NULL");
  REQUIRE(a->struct_size == sizeof(MacRectifyArgs), "struct_size mismatch (%u vs %zu)", a->struct_size,
          sizeof(MacRectifyArgs));
  REQUIRE(a->abi_version == MAC_ABI_VERSION, "abi_version mismatch");
  if (int rc = check_window_common(a->B, a->Hq, a->Hkv, a->D, a->total_q, a->pool_tokens, a->q_post, a->k_buffer,
                                   a->v_buffer, a->qo_indptr, a->kv_indptr, a->kv_indices, a->kv_indices_len))
    return rc;
  REQUIRE(a->M > 0, "capacity (M) must be > 0");
  REQUIRE(a->R > 0, "R must be > 0");
  REQUIRE(a->semantic_pos_ahead >= 1, "semantic_pos_ahead must be >= 1 (the window is S keys)");
  REQUIRE(a->front_sink_tokens >= 0, "front_sink_tokens must be >= 0");
  REQUIRE(a->sink_mode == 0 || a->sink_mode == 1, "sink_mode must be 0 or 1");
  REQUIRE(a->request_length_len == a->R || a->request_length_len == a->B, "request_length must be [R] or [B]");
  REQUIRE(a->src_q && a->o_full && a->lse_full && a->q_cache && a->attn_cache && a->lse_cache &&
              a->request_length && a->req_ids,
          "null pointer argument");
  REQUIRE(aligned16(a->src_q) && aligned16(a->o_full) && aligned16(a->q_cache) && aligned16(a->attn_cache) &&
              (a->q_post_cache == nullptr || aligned16(a->q_post_cache)),
          "src_q, o_full, q_cache, attn_cache and q_post_cache must be 16-byte aligned");
  if (a->B == 0 || a->total_q == 0) return MAC_OK;
  WindowParams p{};
  p.q = static_cast<const uint16_t*>(a->q_post);
  p.k = static_cast<const uint16_t*>(a->k_buffer);
  p.v = static_cast<const uint16_t*>(a->v_buffer);
  p.qo_indptr = a->qo_indptr;
  p.kv_indptr = a->kv_indptr;
  p.kv_indices = a->kv_indices;
  p.src_q = static_cast<const uint16_t*>(a->src_q);
  p.o_full = static_cast<const uint16_t*>(a->o_full);
  p.lse_full = a->lse_full;
  p.q_cache = static_cast<uint16_t*>(a->q_cache);
  p.attn_cache = static_cast<uint16_t*>(a->attn_cache);
  p.lse_cache = a->lse_cache;
  p.q_post_cache = static_cast<uint16_t*>(a->q_post_cache);
  p.request_length = a->request_length;
  p.req_ids = a->req_ids;
  p.pool_tokens = a->pool_tokens;
  p.total_q = a->total_q;
  p.kv_len_total = a->kv_indices_len;
  p.B = a->B;
  p.Hq = a->Hq;
  p.Hkv = a->Hkv;
  p.R = a->R;
  p.M = a->M;
  p.S = a->semantic_pos_ahead;
  p.F = a->front_sink_tokens;
  p.sink_mode = a->sink_mode;
  // the by-batch form wins when R == B, as in mac_prefill_update_cache
  p.rl_by_batch = a->request_length_len == a->B;
  p.q_scale = static_cast<float>(a->sm_scale * 1.4426950408889634);
  const int64_t kept = std::min<int64_t>(a->total_q, static_cast<int64_t>(a->B) * a->M);
  const int64_t blocks = (kept + kRows - 1) / kRows + a->B;
  hipStream_t s = static_cast<hipStream_t>(stream);
  launch_window<true>(p, blocks, s);
  HIP_OK(hipGetLastError());
  if (!p.rl_by_batch) {
    hipLaunchKernelGGL(bump_kernel, dim3((a->B + 255) / 256), dim3(256), 0, s, a->request_length, a->req_ids,
                       a->qo_indptr, a->kv_indptr, p.total_q, p.kv_len_total, a->B, a->R);
    HIP_OK(hipGetLastError());
  }
  return MAC_OK;
}
