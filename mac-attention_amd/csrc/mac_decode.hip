// mac_decode.hip -- MAC-Attention fused decode step for MI355X (gfx950).
//
// One decode step is three kernels on the caller's stream (graph-capturable,
// no host synchronisation, no allocation):
//
//  1. match_decide  (one workgroup per (request, KV head) group)
//     Scans the request's ring of cached pre-RoPE queries for every query head
//     of the group (squared L2, best = smallest distance, ties to the smaller
//     logical position), applies the readiness gate and the optional synthetic
//     bench override, and turns the per-head results into the group's mode and
//     its KV spans: sink [0, min(F, new_end)), band [rect_begin, new_end) and
//     tail [new_end, kv_len).  Reference: DECODE:942-1099, :1101-1402.
//
//  2. span_attention  (persistent grid sized to the device's residency)
//     Every workgroup plans the same task list from the group spans: the
//     spans are cut into chunks of C tokens (C picked from the total token
//     count so that the grid gets ~12 tasks per workgroup), and workgroups
//     fetch tasks through an atomic counter.  A task streams the K/V rows of its chunk once
//     for all G query heads of the group (16 lanes per token row, 16-byte
//     loads, two tokens per row in flight plus a one-iteration prefetch),
//     masks band positions that precede a head's own band start, and keeps an
//     online log2-domain softmax per head.  The task writes one partial
//     (o, lse) per head.  Reference producers: DECODE:1870-3423.
//
//  3. merge_write  (one workgroup per group)
//     Per head: cached entry (hit heads) + band partials -> ring row at
//     past_len % M (only for ready requests) -> + sink and tail partials ->
//     out / out_lse.  Reference: DECODE:4280-4685.
//
// Workspace use (caller-owned, reference names):
//   head_*, group_mode, group_rect_begin/end, group_tail_begin/end: same
//     meaning as in the reference (DECODE:1270-1402);
//   group_rect_tiles / group_tail_tiles: number of band / tail tasks;
//   complete_task_go[g]: chunk size C_g of group g; complete_task_tile[g]:
//     number of tasks of group g (written by workgroup 0 of span_attention);
//   match_dist/pos/slot[..., 0]: best (distance, position, slot) of the scan;
//   partial_o / partial_lse: one (o, lse) partial per task and head;
//   task_counts: [0] tasks, [1] tail tasks, [3] non-hit groups whose band spans
//     more than one tile_tokens tile, [4] chunk C, [5] non-hit groups, [6]
//     full-fallback groups, [7]/[8] max band tasks of full-fallback / mixed
//     groups.

#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <mutex>
#include <tuple>

#include "mac_attention_amd.h"
#include "mac_common.h"

namespace mac {

struct Shape {
  int N, Hq, Hkv, M, R;
  int64_t pool_tokens;
  int r2t_rows, r2t_stride;
  int out_cache_loc_is_i64;
  int max_match_tiles;
  int ws_rows;
};

struct DecideParams {
  Shape s;
  const uint16_t* q_pre;
  const uint16_t* query_cache;
  const float* lse_cache;
  const int32_t* req_ids;
  const int32_t* past_lens;
  const uint8_t* cache_ready;
  const int64_t* cache_epoch;
  const int64_t* request_epoch;
  float* match_dist;
  int32_t* match_pos;
  int32_t* match_slot;
  int32_t* head_hit;
  int32_t* head_match_slot;
  int32_t* head_match_pos;
  int32_t* head_prefix_end;
  int32_t* head_rect_start;
  int32_t* head_new_end;
  int32_t* group_rect_begin;
  int32_t* group_rect_end;
  int32_t* group_tail_begin;
  int32_t* group_tail_end;
  int32_t* group_mode;
  int32_t* task_counter;  // zeroed here for span_attention's dynamic fetch
  int splits;             // slot ranges of the ring scan (1: scan inside match_decide)
  int probe;              // range scan: skip the second half of rows whose first half already exceeds thr_dist
  int S, F, gen_min_limit, lookback_right, candidate_mode;
  float thr_dist;
  int mixed_group_fallback;
  int bench_mode, bench_exact_quota, bench_seed, bench_miss_mask, bench_layer_id;
  float bench_hit_rate, bench_hit_rate_std, bench_skip_ratio, bench_skip_ratio_std;
  float bench_match_lag_mean, bench_match_lag_std;
};

struct AttnParams {
  Shape s;
  const uint16_t* q_post;
  const uint16_t* k_buffer;
  const uint16_t* v_buffer;
  const int32_t* req_to_token;
  const int32_t* req_ids;
  const int32_t* past_lens;
  const void* out_cache_loc;
  const int32_t* head_rect_start;
  const int32_t* group_rect_begin;
  const int32_t* group_rect_end;
  const int32_t* group_tail_end;
  const int32_t* group_mode;
  int32_t* group_rect_tiles;
  int32_t* group_tail_tiles;
  int32_t* group_chunk;   // complete_task_go
  int32_t* group_ntasks;  // complete_task_tile
  int32_t* task_counts;
  int32_t* task_counter;   // complete_task_tile[N * Hkv]; zeroed by match_decide
  void* partial_o;
  float* partial_lse;
  int partial_bf16;
  int64_t o_group_stride;  // elements of partial_o per group
  int cap;                 // task slots per group
  int F;
  int tile_tokens;  // the caller's tile size (task_counts[3] only)
  int tasks_per_wg;  // target tasks per workgroup of the plan
  int narrow_grid;                // workgroups that take tasks when a step has
  long long narrow_min_tokens;    // at least this many tokens (the others return)
  int min_chunk;     // smallest chunk of the plan (tokens)
  float q_scale;  // sm_scale * log2(e)
};

struct MergeParams {
  Shape s;
  const uint16_t* q_pre;
  uint16_t* query_cache;
  uint16_t* attn_cache;
  float* lse_cache;
  uint16_t* out;
  float* out_lse;
  const int32_t* req_ids;
  const int32_t* past_lens;
  const uint8_t* cache_ready;
  const int64_t* cache_epoch;
  const int64_t* request_epoch;
  const int32_t* head_hit;
  const int32_t* head_match_slot;
  const int32_t* group_rect_begin;
  const int32_t* group_rect_end;
  const int32_t* group_tail_end;
  const int32_t* group_chunk;
  const void* partial_o;
  const float* partial_lse;
  int partial_bf16;
  int64_t o_group_stride;
  int cap;
  int F;
};

// DECODE:221-230.  A request id outside [0, R) is never ready: its ring rows
// cannot be addressed, so it must not be matched against or written.
__device__ __forceinline__ bool request_ready(const uint8_t* ready, const int64_t* ce,
                                              const int64_t* re, int req, int R) {
  if (req < 0 || req >= R) return false;
  if (ready == nullptr) return true;
  if (ready[req] == 0) return false;
  if (ce != nullptr && re != nullptr && ce[req] != re[req]) return false;
  return true;
}

// ---------------------------------------------------------------- hashing --
// DECODE:817-835 and :375-388, used only by the synthetic bench override.
__device__ __forceinline__ uint32_t mix_u32(uint32_t x) {
  x ^= x >> 16;
  x *= 0x7feb352du;
  x ^= x >> 15;
  x *= 0x846ca68bu;
  x ^= x >> 16;
  return x;
}
__device__ __forceinline__ float uniform01_u32(uint32_t x) {
  return static_cast<float>(mix_u32(x) & 0x00ffffffu) * (1.0f / 16777216.0f);
}
__device__ __forceinline__ float pseudo_normal_u32(uint32_t x) {
  float s = uniform01_u32(x) + uniform01_u32(x ^ 0x9e3779b9u) + uniform01_u32(x ^ 0x85ebca6bu) +
            uniform01_u32(x ^ 0xc2b2ae35u);
  return (s - 2.0f) * 1.7320508075688772f;
}
__device__ __forceinline__ float clampf(float v, float lo, float hi) { return fminf(fmaxf(v, lo), hi); }

typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));

// 16-byte non-temporal (streaming) global load.
__device__ __forceinline__ uint4 load_stream16(const uint16_t* ptr) {
  return __builtin_bit_cast(uint4, __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(ptr)));
}

// =========================================================== 1. decide ====

// Lanes of a wave form four rows of 16; row r of pass p scans query head
// r + 4p of the group, lane c of the row owns dims [8c, 8c+8).  Each wave
// takes slots wave, wave+4, ... in batches of kSlotBatch whose 16-byte loads
// (of every pass) are all issued before any reduction: with one workgroup per
// group the scan of a large ring is bound by the loads each lane keeps in
// flight.
//
// Large rings are scanned by a separate launch over (group, slot range)
// (kMode 1, `splits` ranges of about kSplitSlots slots) that writes each
// range's best into tile `range` of match_dist/pos/slot; match_decide then
// reduces the tiles (kMode 2) instead of scanning.  kMode 0 scans and decides
// in one workgroup per group.
constexpr int kSplitSlots = 256;
constexpr int kLsePrefetchSlots = 64;
constexpr int kProbeSlots = 4;  // probe scan: slot pairs per lane batch and pass

template <int G, int kMode>
__global__ void __launch_bounds__(kBlock) match_decide_kernel(DecideParams p) {
  constexpr int kPasses = (G + 3) / 4;
  constexpr int kSlotBatch = 16 / kPasses;  // 16 row loads in flight per lane
  const int g = blockIdx.x;
  const int n = g / p.s.Hkv;
  const int hkv = g - n * p.s.Hkv;
  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int row = lane >> 4;
  const int c = lane & 15;
  const int M = p.s.M;
  const int Hq = p.s.Hq;

  const int P = p.past_lens[n];
  const int req = p.req_ids[n];
  const bool ready = request_ready(p.cache_ready, p.cache_epoch, p.request_epoch, req, p.s.R);
  // DECODE:974-981
  const int cand_begin = max(0, P - M);
  int cand_end = P;
  if (p.candidate_mode == 1) cand_end = max(cand_begin, P - p.lookback_right);
  const bool eligible = P >= p.gen_min_limit && cand_end > cand_begin && ready;

  __shared__ float s_d[kWaves][kMaxGroup];
  __shared__ int s_p[kWaves][kMaxGroup];
  __shared__ int s_s[kWaves][kMaxGroup];
  __shared__ float s_lse[kMaxGroup][kLsePrefetchSlots];  // lse of every slot (small rings)

  // Every load of the scan is independent of the readiness gate and of the
  // other loads (a request id outside [0, R) reads request 0's rows, and the
  // results are masked), so the kernel waits for one round of loads, not a
  // chain.  For rings of at most kLsePrefetchSlots slots the entries' lse
  // are fetched in the same round, so the decision reads them from LDS.
  const bool req_ok = req >= 0 && req < p.s.R;
  const int64_t cache_req = static_cast<int64_t>(req_ok ? req : 0) * M;
  const bool lse_in_lds = kMode == 0 && M <= kLsePrefetchSlots;
  if (lse_in_lds && wave == 0 && lane < M) {
#pragma unroll
    for (int hh = 0; hh < G; ++hh) s_lse[hh][lane] = p.lse_cache[(cache_req + lane) * Hq + hkv * G + hh];
  }

  float best_d[kPasses];
  int best_p[kPasses], best_s[kPasses];
  float q[kPasses][8];
#pragma unroll
  for (int ps = 0; ps < kPasses; ++ps) {
    best_d[ps] = INFINITY;
    best_p[ps] = INT_MAX;
    best_s[ps] = -1;
    const int hl = row + 4 * ps;
    uint4 w = make_uint4(0, 0, 0, 0);
    if (hl < G) {
      const int64_t off = (static_cast<int64_t>(n) * Hq + hkv * G + hl) * kHeadDim + c * 8;
      w = *reinterpret_cast<const uint4*>(p.q_pre + off);
    }
    unpack8(w, q[ps]);
  }

  const int per_split = ceil_div(M, p.splits);
  const int s_lo = kMode == 1 ? static_cast<int>(blockIdx.y) * per_split : 0;
  const int s_hi = kMode == 1 ? min(M, s_lo + per_split) : M;
  if (kMode == 1 && p.probe != 0) {
    // Probe scan (the reference's default, DECODE:1001-1075).  The squared
    // distance over dims [0, 64) is a lower bound of the full one, so a slot
    // whose probe exceeds thr_dist (plus a relative slack of 1e-4, far above
    // the rounding of a 128-term fp32 sum) cannot be a hit and its second
    // half-row is not fetched; every other slot gets its full distance.
    // Hit decisions are those of the full scan; only the best distance of a
    // head without a hit may differ.  Lane (row, c) takes slot 2u + (c >> 3)
    // of the batch and 16-byte chunk (c & 7) of its first half, then chunk
    // 8 + (c & 7) -- or, for a pruned slot, a chunk of its head's query row,
    // a cache hit instead of HBM traffic (no divergent loads); a batch the
    // whole wave pruned skips the second round.  Ring rows are read once per
    // step, with the non-temporal policy.
    constexpr int kProbeBatch = kProbeSlots / kPasses;  // slot pairs per lane batch
    const int half = c >> 3, cc = c & 7;
    float qa[kPasses][8], qb[kPasses][8];
#pragma unroll
    for (int ps = 0; ps < kPasses; ++ps) {
      const int hl = min(row + 4 * ps, G - 1);
      const uint16_t* qp = p.q_pre + (static_cast<int64_t>(n) * Hq + hkv * G + hl) * kHeadDim + cc * 8;
      unpack8(*reinterpret_cast<const uint4*>(qp), qa[ps]);
      unpack8(*reinterpret_cast<const uint4*>(qp + 64), qb[ps]);
    }
    const float thr_prune = p.thr_dist + fabsf(p.thr_dist) * 1e-4f + 1e-4f;
    for (int s0 = s_lo + wave; s0 < s_hi; s0 += kWaves * 2 * kProbeBatch) {
      int pos[kProbeBatch], slot[kProbeBatch];
      bool in_window[kProbeBatch];
#pragma unroll
      for (int u = 0; u < kProbeBatch; ++u) {
        slot[u] = s0 + (2 * u + half) * kWaves;
        pos[u] = ring_slot_to_pos(P, M, slot[u]);
        in_window[u] = eligible && slot[u] < s_hi && pos[u] >= cand_begin && pos[u] < cand_end;
      }
      uint4 w[kPasses][kProbeBatch];
#pragma unroll
      for (int ps = 0; ps < kPasses; ++ps) {
        const int hl = min(row + 4 * ps, G - 1);
#pragma unroll
        for (int u = 0; u < kProbeBatch; ++u) {
          const int64_t off = ((cache_req + min(slot[u], s_hi - 1)) * Hq + hkv * G + hl) * kHeadDim + cc * 8;
          w[ps][u] = load_stream16(p.query_cache + off);  // read once: no cache pollution
        }
      }
      float acc[kPasses][kProbeBatch];
      bool eval[kPasses][kProbeBatch];
#pragma unroll
      for (int ps = 0; ps < kPasses; ++ps)
#pragma unroll
        for (int u = 0; u < kProbeBatch; ++u) {
          float cf[8];
          unpack8(w[ps][u], cf);
          float a = 0.0f;
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            const float df = qa[ps][i] - cf[i];
            a = fmaf(df, df, a);
          }
          acc[ps][u] = a;
          eval[ps][u] = in_window[u] && row + 4 * ps < G && row8_sum(a) <= thr_prune;
        }
      bool any_eval = false;
#pragma unroll
      for (int ps = 0; ps < kPasses; ++ps)
#pragma unroll
        for (int u = 0; u < kProbeBatch; ++u) any_eval |= eval[ps][u];
      if (!__any(any_eval)) continue;  // the whole batch pruned (the common case): no second half-rows
#pragma unroll
      for (int ps = 0; ps < kPasses; ++ps) {
        const int hl = min(row + 4 * ps, G - 1);
#pragma unroll
        for (int u = 0; u < kProbeBatch; ++u) {
          // a pruned slot's lanes read their head's query row instead (hot in
          // the cache: every workgroup of the group reads it); the value is unused
          const uint16_t* src =
              eval[ps][u] ? p.query_cache + ((cache_req + min(slot[u], s_hi - 1)) * Hq + hkv * G + hl) * kHeadDim + 64 + cc * 8
                          : p.q_pre + (static_cast<int64_t>(n) * Hq + hkv * G + hl) * kHeadDim + cc * 8;
          w[ps][u] = load_stream16(src);
        }
      }
#pragma unroll
      for (int ps = 0; ps < kPasses; ++ps)
#pragma unroll
        for (int u = 0; u < kProbeBatch; ++u) {
          float cf[8];
          unpack8(w[ps][u], cf);
          float b = acc[ps][u];
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            const float df = qb[ps][i] - cf[i];
            b = fmaf(df, df, b);
          }
          const float d = row8_sum(b);
          if (eval[ps][u] && better_pair(d, pos[u], best_d[ps], best_p[ps])) {
            best_d[ps] = d;
            best_p[ps] = pos[u];
            best_s[ps] = slot[u];
          }
        }
    }
    // the two half-rows of lanes tracked different slots: lane c takes the
    // better of its own and lane c ^ 8's
#pragma unroll
    for (int ps = 0; ps < kPasses; ++ps) {
      const float od = __shfl_xor(best_d[ps], 8);
      const int op = __shfl_xor(best_p[ps], 8), os = __shfl_xor(best_s[ps], 8);
      if (better_pair(od, op, best_d[ps], best_p[ps])) {
        best_d[ps] = od;
        best_p[ps] = op;
        best_s[ps] = os;
      }
    }
  } else if (kMode != 2) {
    for (int s0 = s_lo + wave; s0 < s_hi; s0 += kWaves * kSlotBatch) {
      // every pass's loads of the batch are in flight before any reduction
      uint4 w[kPasses][kSlotBatch];
      int pos[kSlotBatch];
      bool in_window[kSlotBatch];
#pragma unroll
      for (int u = 0; u < kSlotBatch; ++u) {
        const int slot = s0 + u * kWaves;
        pos[u] = ring_slot_to_pos(P, M, slot);
        in_window[u] = eligible && slot < s_hi && pos[u] >= cand_begin && pos[u] < cand_end;
      }
#pragma unroll
      for (int ps = 0; ps < kPasses; ++ps) {
        const int hl = min(row + 4 * ps, G - 1);
#pragma unroll
        for (int u = 0; u < kSlotBatch; ++u) {
          const int slot = min(s0 + u * kWaves, s_hi - 1);  // past the range: re-reads its last row
          const int64_t off = ((cache_req + slot) * Hq + hkv * G + hl) * kHeadDim + c * 8;
          w[ps][u] = load_stream16(p.query_cache + off);  // ring rows are read once per step
        }
      }
#pragma unroll
      for (int ps = 0; ps < kPasses; ++ps) {
        const int hl = row + 4 * ps;
#pragma unroll
        for (int u = 0; u < kSlotBatch; ++u) {
          float cf[8];
          unpack8(w[ps][u], cf);
          float acc = 0.0f;
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            const float df = q[ps][i] - cf[i];
            acc = fmaf(df, df, acc);
          }
          acc = row16_sum(acc);
          if (in_window[u] && hl < G && better_pair(acc, pos[u], best_d[ps], best_p[ps])) {
            best_d[ps] = acc;
            best_p[ps] = pos[u];
            best_s[ps] = s0 + u * kWaves;
          }
        }
      }
    }
  }
#pragma unroll
  for (int ps = 0; ps < kPasses; ++ps) {
    const int hl = row + 4 * ps;
    if (c == 0 && hl < G) {
      s_d[wave][hl] = best_d[ps];
      s_p[wave][hl] = best_p[ps];
      s_s[wave][hl] = best_s[ps];
    }
  }
  __syncthreads();
  if (wave != 0) return;

  // ---- per-head decisions (lanes 0..G-1 of wave 0), DECODE:1147-1299 ----
  const int h = lane;
  const bool head_lane = h < G;
  const int hq = hkv * G + (head_lane ? h : 0);
  float bd = INFINITY;
  int bp = INT_MAX, bs = -1;
  if (head_lane) {
    for (int w = 0; w < kWaves; ++w) {
      if (better_pair(s_d[w][h], s_p[w][h], bd, bp)) {
        bd = s_d[w][h];
        bp = s_p[w][h];
        bs = s_s[w][h];
      }
    }
  }
  const int64_t ho = static_cast<int64_t>(n) * Hq + hq;
  const int64_t mo = ho * p.s.max_match_tiles;
  if (kMode == 1) {  // this range's best -> its tile
    if (head_lane) {
      p.match_dist[mo + blockIdx.y] = bd;
      p.match_pos[mo + blockIdx.y] = bp;
      p.match_slot[mo + blockIdx.y] = bs;
    }
    return;
  }
  if (kMode == 2) {  // best over the ranges' tiles
    if (head_lane && eligible) {
      for (int r = 0; r < p.splits; ++r) {
        const float d = p.match_dist[mo + r];
        const int ps = p.match_pos[mo + r];
        if (p.match_slot[mo + r] >= 0 && better_pair(d, ps, bd, bp)) {
          bd = d;
          bp = ps;
          bs = p.match_slot[mo + r];
        }
      }
    }
  } else if (head_lane) {
    p.match_dist[mo] = bd;
    p.match_pos[mo] = bp;
    p.match_slot[mo] = bs;
  }
  bool hit = eligible && bs >= 0 && bd < p.thr_dist;
  const int S = p.S;
  const int F = p.F;
  if (p.bench_mode != 0 || p.bench_miss_mask >= 0) {  // DECODE:1184-1269
    const int lane_i = h;
    const uint32_t unit_id = p.bench_mode == 2 ? static_cast<uint32_t>(hkv) : static_cast<uint32_t>(hq);
    const uint32_t base_key = static_cast<uint32_t>(p.bench_seed) ^
                              (static_cast<uint32_t>(p.bench_layer_id) * 0x9e3779b9u) ^
                              (static_cast<uint32_t>(P) * 0x85ebca6bu);
    const uint32_t key = base_key ^ (static_cast<uint32_t>(n) * 0xc2b2ae35u) ^ (unit_id * 0x27d4eb2fu);
    const float hit_rate = clampf(
        p.bench_hit_rate + p.bench_hit_rate_std * pseudo_normal_u32(key ^ 0x4cf5ad43u), 0.0f, 1.0f);
    if (p.bench_miss_mask >= 0) {
      const bool miss = lane_i < 30 && ((p.bench_miss_mask >> lane_i) & 1) != 0;
      hit = eligible && P > 0 && M > 0 && !miss;
    } else if (p.bench_exact_quota != 0 && p.bench_hit_rate_std == 0.0f) {
      const int unit_total = p.bench_mode == 2 ? p.s.N * p.s.Hkv : p.s.N * Hq;
      const int unit = p.bench_mode == 2 ? n * p.s.Hkv + hkv : n * Hq + hq;
      float miss_rate = fminf(fmaxf(1.0f - p.bench_hit_rate, 0.0f), 1.0f);
      int miss_units = unit_total > 0 ? static_cast<int>(floorf(miss_rate * static_cast<float>(unit_total) + 0.5f)) : 0;
      miss_units = min(max(miss_units, 0), unit_total);
      const int offset = unit_total > 0 ? static_cast<int>(base_key % static_cast<uint32_t>(unit_total)) : 0;
      int rotated = unit + offset;
      if (rotated >= unit_total) rotated -= unit_total;
      hit = eligible && P > 0 && M > 0 && !(rotated < miss_units);
    } else {
      hit = eligible && P > 0 && M > 0 && uniform01_u32(key ^ 0x165667b1u) < hit_rate;
    }
    if (hit) {
      const int max_lag = min(M, P);
      const int ne = cache_end_for_pos(P, S);
      float lag_f = p.bench_match_lag_mean + p.bench_match_lag_std * pseudo_normal_u32(key ^ 0xd3a2646cu);
      bool req_skip = false;
      if (p.bench_skip_ratio >= 0.0f) {
        req_skip = true;
        const float sr = clampf(p.bench_skip_ratio + p.bench_skip_ratio_std * pseudo_normal_u32(key ^ 0xfd7046c5u),
                                0.0f, 0.999999f);
        int tpe = static_cast<int>(roundf(sr * static_cast<float>(P)));
        if (tpe > ne - 1) tpe = ne - 1;
        if (tpe < 0) tpe = 0;
        lag_f = static_cast<float>(ne - tpe);
      }
      int lag = static_cast<int>(roundf(lag_f));
      if (lag < 1) lag = 1;
      if (req_skip) {
        if (lag > P) lag = P;
      } else if (lag > max_lag) {
        lag = max_lag;
      }
      if (max_lag <= 0 || ne <= 0) {
        hit = false;
        bp = INT_MAX;
        bs = -1;
      } else {
        bp = max(P - lag, 0);
        bs = pos_to_ring_slot(P, M, bp);
      }
    } else {
      bp = INT_MAX;
      bs = -1;
    }
  }
  int prefix_end = 0, mpos = -1, mslot = -1;
  if (hit) {
    mpos = bp;
    mslot = bs;
    prefix_end = cache_end_for_pos(mpos, S);
  }
  if (hit && F > 0 && prefix_end < F) {  // front-sink demotion, DECODE:1285-1291
    hit = false;
    mpos = mslot = -1;
    prefix_end = 0;
  }
  const int new_end = cache_end_for_pos(P, S);
  const int fs_begin = min(F, new_end);
  // DECODE:1315-1328 validity of a hit head for MAC reuse
  bool valid = false;
  if (head_lane && hit && mslot >= 0) {
    const float pl = lse_in_lds ? s_lse[h][mslot] : p.lse_cache[(static_cast<int64_t>(req) * M + mslot) * Hq + hq];
    const int clen = new_end - prefix_end;
    valid = isfinite(pl) && clen >= 0 && clen <= M;
  }
  const uint64_t vmask = __ballot(valid);
  const int valid_count = __popcll(vmask);
  int mode = MAC_GROUP_FULL_FALLBACK;
  if (valid_count == G)
    mode = MAC_GROUP_MAC_HIT;
  else if (valid_count > 0 && p.mixed_group_fallback != 0)
    mode = MAC_GROUP_MIXED;
  const bool keep = mode == MAC_GROUP_MAC_HIT || (mode == MAC_GROUP_MIXED && valid);
  int rect_start = keep ? prefix_end : fs_begin;
  if (!keep) {
    hit = false;
    mpos = mslot = -1;
    prefix_end = 0;
  }
  // group band begins at the smallest head band start
  int rb = head_lane ? rect_start : INT_MAX;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) rb = min(rb, __shfl_xor(rb, off));
  if (mode != MAC_GROUP_MAC_HIT) rb = fs_begin;
  rb = max(0, min(rb, new_end));
  if (head_lane) {
    p.head_hit[ho] = hit ? 1 : 0;
    p.head_match_slot[ho] = mslot;
    p.head_match_pos[ho] = mpos;
    p.head_prefix_end[ho] = prefix_end;
    p.head_rect_start[ho] = rect_start;
    p.head_new_end[ho] = new_end;
  }
  if (lane == 0 && g == 0) *p.task_counter = 0;
  if (lane == 0) {
    const int64_t go = static_cast<int64_t>(n) * p.s.Hkv + hkv;
    p.group_mode[go] = mode;
    p.group_rect_begin[go] = rb;
    p.group_rect_end[go] = new_end;
    p.group_tail_begin[go] = new_end;
    p.group_tail_end[go] = P + 1;
  }
}

// ========================================================= 2. attention ====

struct GroupSpans {
  int sink_end, band_begin, new_end, kv_len;
  int chunk, n_sink, n_band, n_tail;
};

__device__ __forceinline__ int group_tokens(int sink_end, int band_begin, int new_end, int kv_len) {
  return sink_end + (new_end - band_begin) + (kv_len - new_end);
}

// Chunk of a group: the launch-wide chunk, enlarged (to a multiple of 64) when
// the group would otherwise need more task slots than its workspace holds.
__device__ __forceinline__ int group_chunk(int tokens, int chunk, int cap) {
  int need = ceil_div(tokens, max(cap - 3, 1));
  need = ceil_div(need, 64) * 64;
  return max(chunk, need);
}

__device__ __forceinline__ GroupSpans load_spans(const int32_t* rect_begin, const int32_t* rect_end,
                                                 const int32_t* tail_end, int g, int F, int chunk,
                                                 int cap) {
  GroupSpans s;
  s.band_begin = rect_begin[g];
  s.new_end = rect_end[g];
  s.kv_len = tail_end[g];
  s.sink_end = min(F, s.new_end);
  s.chunk = group_chunk(group_tokens(s.sink_end, s.band_begin, s.new_end, s.kv_len), chunk, cap);
  s.n_sink = ceil_div(s.sink_end, s.chunk);
  s.n_band = ceil_div(s.new_end - s.band_begin, s.chunk);
  s.n_tail = ceil_div(s.kv_len - s.new_end, s.chunk);
  return s;
}

// Band pieces of a group that span a full chunk (the first ones; only the
// last band piece can be shorter).
__device__ __forceinline__ int full_band_pieces(const GroupSpans& s) {
  return (s.new_end - s.band_begin) / s.chunk;
}

// Block-wide exclusive scan of per-thread values (256 threads).
__device__ __forceinline__ int block_exclusive_scan(int v, int* s_tmp, int& total) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  int x = v;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    int y = __shfl_up(x, off);
    if (lane >= off) x += y;
  }
  if (lane == 63) s_tmp[wave] = x;
  __syncthreads();
  int base = 0;
  total = 0;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) {
    if (w < wave) base += s_tmp[w];
    total += s_tmp[w];
  }
  __syncthreads();
  return base + x - v;
}

// Task granularity.  Workgroups fetch tasks dynamically, so about a dozen
// tasks per workgroup bounds the end-of-kernel imbalance to a few percent,
// while a task of at least kMinChunk tokens amortises its fixed cost (plan
// lookup, Q staging, pipeline fill, partial write).
constexpr int kTasksPerWorkgroup = 12;  // default of AttnParams::tasks_per_wg
constexpr int kMinChunk = 2048;
constexpr int kMaxChunk = 16384;

// Every workgroup of span_attention derives the same task list: the chunk C
// from the total token count of all groups (kTasksPerWorkgroup tasks per
// workgroup, a multiple of 64 tokens in [kMinChunk, kMaxChunk]), then the
// tasks in two classes, largest first: class A holds the band pieces of full
// chunk length, class B everything shorter (sinks, band remainders, tails,
// and the whole bands of hit groups).  Workgroups fetch A tasks before B
// tasks, so the end of the kernel is filled with short tasks and the idle
// time of the last workgroups is bounded by a short task, not a full chunk.
// s_off[0..NG] holds the exclusive prefix sums of the per-group A counts,
// s_off[NG+1 .. 2NG+1] those of the B counts.  Workgroup 0 also publishes the
// per-group chunk and task counts for merge_write and the task counters.
__device__ void plan_tasks(const AttnParams& p, int* s_off, int* s_tmp, int& total_tasks_out,
                           int& chunk_out, int& active_wgs_out) {
  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int NG = p.s.N * p.s.Hkv;
  const int per_thread = ceil_div(NG, kBlock);
  const int g_lo = min(tid * per_thread, NG);
  const int g_hi = min(g_lo + per_thread, NG);
  long long tok = 0;
  for (int g = g_lo; g < g_hi; ++g) {
    const int ne = p.group_rect_end[g];
    tok += group_tokens(min(p.F, ne), p.group_rect_begin[g], ne, p.group_tail_end[g]);
  }
  // reduce token count (64-bit) across the block
  {
    long long x = tok;
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) x += __shfl_xor(x, off);
    __shared__ long long s_tok[kWaves];
    if (lane == 0) s_tok[wave] = x;
    __syncthreads();
    tok = 0;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) tok += s_tok[w];
    __syncthreads();
  }
  // A step with many tokens streams fastest with one workgroup per CU; a
  // small (latency-bound) one wants every resident workgroup.
  const int W = tok >= p.narrow_min_tokens ? min(static_cast<int>(gridDim.x), p.narrow_grid)
                                           : static_cast<int>(gridDim.x);
  active_wgs_out = W;
  const long long target_tasks = static_cast<long long>(p.tasks_per_wg) * W;
  int chunk = static_cast<int>((tok + target_tasks - 1) / target_tasks);
  chunk = ceil_div(max(chunk, p.min_chunk), 64) * 64;
  chunk = min(chunk, kMaxChunk);
  int* s_offb = s_off + NG + 1;
  int my_a = 0, my_b = 0;
  for (int g = g_lo; g < g_hi; ++g) {
    GroupSpans sp = load_spans(p.group_rect_begin, p.group_rect_end, p.group_tail_end, g, p.F, chunk, p.cap);
    const int na = full_band_pieces(sp);
    s_off[g] = na;
    s_offb[g] = sp.n_sink + sp.n_band + sp.n_tail - na;
    my_a += na;
    my_b += s_offb[g];
  }
  int total_a = 0, total_b = 0;
  int base_a = block_exclusive_scan(my_a, s_tmp, total_a);
  int base_b = block_exclusive_scan(my_b, s_tmp, total_b);
  for (int g = g_lo; g < g_hi; ++g) {
    const int ca = s_off[g], cb = s_offb[g];
    s_off[g] = base_a;
    s_offb[g] = total_a + base_b;
    base_a += ca;
    base_b += cb;
  }
  const int total_tasks = total_a + total_b;
  if (tid == 0) {
    s_off[NG] = total_a;
    s_offb[NG] = total_tasks;
  }
  __syncthreads();

  if (blockIdx.x == 0) {
    // descriptors for merge_write and the reference's task counters
    int nonhit = 0, ff = 0, red = 0, max_ff = 0, max_mixed = 0, tails = 0;
    for (int g = tid; g < NG; g += kBlock) {
      GroupSpans sp = load_spans(p.group_rect_begin, p.group_rect_end, p.group_tail_end, g, p.F, chunk, p.cap);
      p.group_chunk[g] = sp.chunk;
      p.group_ntasks[g] = sp.n_sink + sp.n_band + sp.n_tail;
      p.group_rect_tiles[g] = sp.n_band;
      p.group_tail_tiles[g] = sp.n_tail;
      const int mode = p.group_mode[g];
      tails += sp.n_tail;
      if (mode != MAC_GROUP_MAC_HIT) {
        ++nonhit;
        // the reference's reduce condition with its default threshold: the
        // band spans more than one tile of tile_tokens
        if (sp.new_end - sp.band_begin > p.tile_tokens) ++red;
      }
      if (mode == MAC_GROUP_FULL_FALLBACK) {
        ++ff;
        max_ff = max(max_ff, sp.n_band);
      }
      if (mode == MAC_GROUP_MIXED) max_mixed = max(max_mixed, sp.n_band);
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
      nonhit += __shfl_xor(nonhit, off);
      ff += __shfl_xor(ff, off);
      red += __shfl_xor(red, off);
      tails += __shfl_xor(tails, off);
      max_ff = max(max_ff, __shfl_xor(max_ff, off));
      max_mixed = max(max_mixed, __shfl_xor(max_mixed, off));
    }
    __shared__ int s_cnt[kWaves][6];
    if (lane == 0) {
      s_cnt[wave][0] = nonhit;
      s_cnt[wave][1] = ff;
      s_cnt[wave][2] = red;
      s_cnt[wave][3] = tails;
      s_cnt[wave][4] = max_ff;
      s_cnt[wave][5] = max_mixed;
    }
    __syncthreads();
    if (tid == 0) {
      int a[6] = {0, 0, 0, 0, 0, 0};
      for (int w = 0; w < kWaves; ++w) {
        for (int i = 0; i < 4; ++i) a[i] += s_cnt[w][i];
        a[4] = max(a[4], s_cnt[w][4]);
        a[5] = max(a[5], s_cnt[w][5]);
      }
      p.task_counts[0] = total_tasks;
      p.task_counts[1] = a[3];
      p.task_counts[2] = 0;
      p.task_counts[3] = a[2];
      p.task_counts[4] = chunk;
      p.task_counts[5] = a[0];
      p.task_counts[6] = a[1];
      p.task_counts[7] = a[4];
      p.task_counts[8] = a[5];
    }
  }

  total_tasks_out = total_tasks;
  chunk_out = chunk;
}

// Dynamic task fetch: the counter is zeroed by match_decide, which runs
// before this kernel on the same stream, so every step (and every graph
// replay) starts from task 0.  Ends with a barrier, so the previous task's
// LDS use is complete before the caller starts the next one.  (Claiming the
// next task one task ahead hides the atomic's round trip but hands two tasks
// to the first workgroups when there are about as many tasks as workgroups,
// which measured slower.)
__device__ __forceinline__ int next_task(const AttnParams& p, int& s_task) {
  __syncthreads();
  if (threadIdx.x == 0) s_task = atomicAdd(p.task_counter, 1);
  __syncthreads();
  return s_task;
}

struct TaskInfo {
  int g, j, n, hkv, a, b;
  bool band;
  int P, req;
  bool req_ok;
  int64_t cur_loc;
};

// Group, token range [a, b) and kind of task t (sink, band or tail).
__device__ __forceinline__ TaskInfo decode_task(const AttnParams& p, const int* s_off, int NG, int chunk,
                                                int t) {
  TaskInfo ti;
  const bool class_a = t < s_off[NG];
  const int* off = class_a ? s_off : s_off + NG + 1;
  int lo = 0, hi = NG - 1;  // last g with off[g] <= t
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (off[mid] <= t) lo = mid; else hi = mid - 1;
  }
  ti.g = lo;
  ti.n = lo / p.s.Hkv;
  ti.hkv = lo - ti.n * p.s.Hkv;
  const GroupSpans sp = load_spans(p.group_rect_begin, p.group_rect_end, p.group_tail_end, lo, p.F, chunk, p.cap);
  // piece index j of the group (sink pieces, band pieces, tail pieces), which
  // is also the partial's slot: class A takes the full band pieces, class B
  // the sink pieces, the band remainder and the tail pieces, in that order
  const int k = t - off[lo];
  const int na = full_band_pieces(sp);
  if (class_a)
    ti.j = sp.n_sink + k;
  else if (k < sp.n_sink)
    ti.j = k;
  else
    ti.j = k + na;
  ti.band = false;
  if (ti.j < sp.n_sink) {
    ti.a = ti.j * sp.chunk;
    ti.b = min(ti.a + sp.chunk, sp.sink_end);
  } else if (ti.j < sp.n_sink + sp.n_band) {
    ti.a = sp.band_begin + (ti.j - sp.n_sink) * sp.chunk;
    ti.b = min(ti.a + sp.chunk, sp.new_end);
    ti.band = true;
  } else {
    ti.a = sp.new_end + (ti.j - sp.n_sink - sp.n_band) * sp.chunk;
    ti.b = min(ti.a + sp.chunk, sp.kv_len);
  }
  ti.P = p.past_lens[ti.n];
  ti.req = p.req_ids[ti.n];
  ti.req_ok = ti.req >= 0 && ti.req < p.s.r2t_rows;
  ti.cur_loc = p.s.out_cache_loc_is_i64 ? static_cast<const int64_t*>(p.out_cache_loc)[ti.n]
                                        : static_cast<int64_t>(static_cast<const int32_t*>(p.out_cache_loc)[ti.n]);
  return ti;
}

// Combines the per-wave softmax states in LDS (unnormalised o, running max m
// in log2 units, sum l) into one normalised partial (o, natural-log lse) per
// head and stores it in slot j of group g.
template <int G>
__device__ __forceinline__ void write_partial(const AttnParams& p, int g, int j,
                                              const float (*s_o)[G][kHeadDim],
                                              const float (*s_ml)[G][2]) {
  const int tid = threadIdx.x;
  const int64_t slot = static_cast<int64_t>(g) * p.cap + j;
  for (int e = tid; e < G * kHeadDim; e += kBlock) {
    const int h = e / kHeadDim;
    const int d = e - h * kHeadDim;
    float mm = kNegBig;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) mm = fmaxf(mm, s_ml[w][h][0]);
    float ll = 0.0f, oo = 0.0f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
      const float sc = fast_exp2(s_ml[w][h][0] - mm);
      ll += s_ml[w][h][1] * sc;
      oo += s_o[w][h][d] * sc;
    }
    const bool nonempty = ll > 0.0f;
    const float ov = nonempty ? oo / ll : 0.0f;
    const int64_t oi = static_cast<int64_t>(g) * p.o_group_stride + (static_cast<int64_t>(j) * G + h) * kHeadDim + d;
    if (p.partial_bf16)
      static_cast<uint16_t*>(p.partial_o)[oi] = f32_to_bf16(ov);
    else
      static_cast<float*>(p.partial_o)[oi] = ov;
    if (d == 0) p.partial_lse[slot * G + h] = nonempty ? (mm + log2f(ll)) * kLn2 : -INFINITY;
  }
}

template <int G>
__global__ void __launch_bounds__(kBlock) span_attention_kernel(AttnParams p) {
  constexpr int U = 2;                 // tokens per row per iteration
  constexpr int kStep = kWaves * 4 * U;  // tokens per workgroup iteration
  extern __shared__ int s_off[];  // 2 (NG + 1) task offsets (dynamic)
  __shared__ int s_tmp[kWaves];
  __shared__ float s_o[kWaves][G][kHeadDim];
  __shared__ float s_ml[kWaves][G][2];

  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int row = lane >> 4;
  const int c = lane & 15;
  const int NG = p.s.N * p.s.Hkv;

  int total_tasks = 0, chunk = 0, active_wgs = 0;
  plan_tasks(p, s_off, s_tmp, total_tasks, chunk, active_wgs);
  if (static_cast<int>(blockIdx.x) >= active_wgs) return;

  // ---- tasks ----
  const int Hq = p.s.Hq;
  const int Hkv = p.s.Hkv;
  const int my_tok = wave * 4 + row;  // token offset inside each 16-token sub-block
  __shared__ int s_task;
  for (int t = next_task(p, s_task); t < total_tasks; t = next_task(p, s_task)) {
    const TaskInfo ti = decode_task(p, s_off, NG, chunk, t);
    const int g = ti.g, j = ti.j, n = ti.n, hkv = ti.hkv, a = ti.a, b = ti.b, P = ti.P, req = ti.req;
    const bool band = ti.band, req_ok = ti.req_ok;
    const int64_t cur_loc = ti.cur_loc;
    const int32_t* r2t = p.req_to_token + static_cast<int64_t>(req_ok ? req : 0) * p.s.r2t_stride;

    // per-head band start (positions before it are masked for that head)
    int mb[G];
    float q[G][8];
#pragma unroll
    for (int h = 0; h < G; ++h) {
      const int hq = hkv * G + h;
      mb[h] = band ? p.head_rect_start[static_cast<int64_t>(n) * Hq + hq] : 0;
      const uint4 w = *reinterpret_cast<const uint4*>(p.q_post + (static_cast<int64_t>(n) * Hq + hq) * kHeadDim + c * 8);
      unpack8(w, q[h]);
#pragma unroll
      for (int i = 0; i < 8; ++i) q[h][i] *= p.q_scale;
    }
    float m[G], l[G], o[G][8];
#pragma unroll
    for (int h = 0; h < G; ++h) {
      m[h] = kNegBig;
      l[h] = 0.0f;
#pragma unroll
      for (int i = 0; i < 8; ++i) o[h][i] = 0.0f;
    }

    auto phys_of = [&](int pos) -> int64_t {
      if (pos >= b || !req_ok) return -1;
      const int64_t ph = pos == P ? cur_loc : static_cast<int64_t>(r2t[pos]);
      return (ph >= 0 && ph < p.s.pool_tokens) ? ph : -1;
    };
    const int64_t kv_stride = static_cast<int64_t>(Hkv) * kHeadDim;
    const uint16_t* kbase = p.k_buffer + static_cast<int64_t>(hkv) * kHeadDim + c * 8;
    const uint16_t* vbase = p.v_buffer + static_cast<int64_t>(hkv) * kHeadDim + c * 8;

    int64_t ph0[U], ph1[U];
    uint4 k0[U], v0[U];
#pragma unroll
    for (int u = 0; u < U; ++u) ph0[u] = phys_of(a + u * 16 + my_tok);
#pragma unroll
    for (int u = 0; u < U; ++u) {
      k0[u] = make_uint4(0, 0, 0, 0);
      v0[u] = make_uint4(0, 0, 0, 0);
      if (ph0[u] >= 0) {
        k0[u] = *reinterpret_cast<const uint4*>(kbase + ph0[u] * kv_stride);
        v0[u] = *reinterpret_cast<const uint4*>(vbase + ph0[u] * kv_stride);
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) ph1[u] = phys_of(a + kStep + u * 16 + my_tok);

    for (int base_pos = a; base_pos < b; base_pos += kStep) {
      // prefetch the next iteration's rows and the one after's indices
      uint4 k1[U], v1[U];
      int64_t ph2[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        k1[u] = make_uint4(0, 0, 0, 0);
        v1[u] = make_uint4(0, 0, 0, 0);
        if (ph1[u] >= 0) {
          k1[u] = *reinterpret_cast<const uint4*>(kbase + ph1[u] * kv_stride);
          v1[u] = *reinterpret_cast<const uint4*>(vbase + ph1[u] * kv_stride);
        }
      }
#pragma unroll
      for (int u = 0; u < U; ++u) ph2[u] = phys_of(base_pos + 2 * kStep + u * 16 + my_tok);

      float s[G][U];
      float vf[U][8];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        float kf[8];
        unpack8(k0[u], kf);
        unpack8(v0[u], vf[u]);
        const int pos = base_pos + u * 16 + my_tok;
#pragma unroll
        for (int h = 0; h < G; ++h) {
          float acc = 0.0f;
#pragma unroll
          for (int i = 0; i < 8; ++i) acc = fmaf(q[h][i], kf[i], acc);
          acc = row16_sum(acc);
          s[h][u] = (ph0[u] >= 0 && pos >= mb[h]) ? acc : -INFINITY;
        }
      }
#pragma unroll
      for (int h = 0; h < G; ++h) {
        float mx = s[h][0];
#pragma unroll
        for (int u = 1; u < U; ++u) mx = fmaxf(mx, s[h][u]);
        const float m_new = fmaxf(m[h], mx);
        const float alpha = fast_exp2(m[h] - m_new);
        float pu[U];
        float psum = 0.0f;
#pragma unroll
        for (int u = 0; u < U; ++u) {
          pu[u] = fast_exp2(s[h][u] - m_new);
          psum += pu[u];
        }
        l[h] = fmaf(l[h], alpha, psum);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          float acc = o[h][i] * alpha;
#pragma unroll
          for (int u = 0; u < U; ++u) acc = fmaf(pu[u], vf[u][i], acc);
          o[h][i] = acc;
        }
        m[h] = m_new;
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        k0[u] = k1[u];
        v0[u] = v1[u];
        ph0[u] = ph1[u];
        ph1[u] = ph2[u];
      }
    }

    // ---- combine the four rows of the wave, then the waves ----
#pragma unroll
    for (int msk = 16; msk <= 32; msk <<= 1) {
#pragma unroll
      for (int h = 0; h < G; ++h) {
        const float mo = __shfl_xor(m[h], msk);
        const float lo2 = __shfl_xor(l[h], msk);
        const float m_new = fmaxf(m[h], mo);
        const float a1 = fast_exp2(m[h] - m_new);
        const float a2 = fast_exp2(mo - m_new);
        l[h] = l[h] * a1 + lo2 * a2;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const float oo = __shfl_xor(o[h][i], msk);
          o[h][i] = o[h][i] * a1 + oo * a2;
        }
        m[h] = m_new;
      }
    }
    if (row == 0) {
#pragma unroll
      for (int h = 0; h < G; ++h) {
#pragma unroll
        for (int i = 0; i < 8; ++i) s_o[wave][h][c * 8 + i] = o[h][i];
        if (c == 0) {
          s_ml[wave][h][0] = m[h];
          s_ml[wave][h][1] = l[h];
        }
      }
    }
    __syncthreads();
    write_partial<G>(p, g, j, s_o, s_ml);  // next_task's barrier closes the task
  }
}

// ------------------------------------------------- MFMA span attention ----
//
// Same plan and task list as span_attention_kernel.  One 64-lane wave owns a
// 32-token block at a time (waves take blocks wave, wave+4, ...):
//
//  * Loads: each 256-byte K or V row is read by 16 consecutive lanes (lane
//    l reads 16-byte chunk l%16 of the row of token 8*(l/16) + i in load i),
//    so every load instruction covers whole 128-byte lines, with the
//    non-temporal policy (the rows are read once per step).  Measured on
//    MI355X this streams ~12% faster than loading the MFMA operands straight
//    from HBM, whose layout splits lines across instructions.  The block
//    after the current one is always in flight in registers; its
//    req_to_token entries are loaded one block earlier still.
//  * The rows are staged in two 8 KiB per-wave LDS tiles, token-major.  In
//    the K tile, 16-byte chunk c of token t sits at position c ^ k_swz(t)
//    (see below), so the 16 tokens one A-operand read touches hit 16
//    different bank groups; in the V tile at c ^ 2 (t & 7), which does the
//    same for the transposing reads.
//  * S^T[t][g] = sum_d K[t][d] Q[g][d] and O^T[d][g] += sum_t V[t][d] P[g][t]
//    both run on v_mfma_f32_16x16x32_bf16.  MFMA row 4a + i of score tile t
//    is token 8a + 4t + i, so the lane holding head g = l%16 ends with the
//    scores of tokens 8q .. 8q + 7 (q = l/16): after conversion to bf16 they
//    are the B operand of the PV product as they stand, and its A operand
//    V^T[16 dt + g][8q .. 8q + 7] is two ds_read_b64_tr_b16 (gfx950's
//    transposing LDS read) of the V tile.  The lane keeps its head's softmax
//    state and 32 O^T accumulators, so the online-softmax rescale is
//    lane-local.  Heads g >= G are zero padding rows of the 16-wide MFMA.

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ bf16x8_t as_bf16x8(const uint4& w) { return __builtin_bit_cast(bf16x8_t, w); }

// K tile: 16-byte chunk c of token t at position c ^ k_swz(t) of its row.
// The S^T tiles read tokens 8a + 4t + i (a, i < 4) in one instruction; this
// swizzle puts the 16 of them on 16 different chunk positions.
__device__ __forceinline__ int k_swz(int t) { return 4 * ((t >> 3) & 3) + (t & 3); }

constexpr int kMfmaBlk = 32;  // tokens per wave block

// One task of the MFMA kernel: the four waves of the workgroup take its
// blocks in turn and combine their softmax states through LDS.  (A function
// of its own, called once per task, so the compiler recomputes the LDS
// addresses per task instead of holding them across the task loop: the
// registers go to the block loop, which measured 2% faster for steps of many
// short tasks.)
template <int G>
__device__ __forceinline__ void mfma_task(const AttnParams& p, const TaskInfo& ti,
                                          uint4 (*s_k)[kMfmaBlk * 16], uint4 (*s_v)[kMfmaBlk * 16],
                                          uint4* s_q, float (*s_ml)[G][2]) {
  constexpr int kBlk = kMfmaBlk;
  // the per-wave o of the task epilogue reuses the K tiles
  auto s_o = reinterpret_cast<float (*)[G][kHeadDim]>(&s_k[0][0]);
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform (scalar) control flow
  const int lane = tid & 63;
  const int quad = lane >> 4;  // lane / 16
  const int col = lane & 15;   // lane % 16
  const int Hq = p.s.Hq;
  const int Hkv = p.s.Hkv;
  const int64_t kv_stride = static_cast<int64_t>(Hkv) * kHeadDim;
  const bool head_ok = col < G;
  const uint16_t* vtile = reinterpret_cast<const uint16_t*>(&s_v[wave][0]);
  // load-side token of load i for this lane: 8*quad + i; chunk: col
  {
    const int n = ti.n, hkv = ti.hkv, a = ti.a, b = ti.b, P = ti.P;
    const int32_t* r2t = p.req_to_token + static_cast<int64_t>(ti.req_ok ? ti.req : 0) * p.s.r2t_stride;
    const uint16_t* kbase = p.k_buffer + static_cast<int64_t>(hkv) * kHeadDim + col * 8;
    const uint16_t* vbase = p.v_buffer + static_cast<int64_t>(hkv) * kHeadDim + col * 8;

    // Q of the group's heads (rows g >= G zero), staged once per task; lane
    // (quad, col) reads Q[col][8*(4s+quad) .. +8] as the B operand of k-step s.
    int head_begin = 0;
    {
      const int64_t qoff = static_cast<int64_t>(n) * Hq * kHeadDim + static_cast<int64_t>(hkv) * G * kHeadDim;
      for (int e = tid; e < 16 * 16; e += kBlock) {
        const int g = e >> 4, c = e & 15;
        uint4 w = make_uint4(0, 0, 0, 0);
        if (g < G) w = *reinterpret_cast<const uint4*>(p.q_post + qoff + g * kHeadDim + c * 8);
        s_q[e] = w;
      }
      if (ti.band && head_ok) head_begin = p.head_rect_start[static_cast<int64_t>(n) * Hq + hkv * G + col];
      __syncthreads();
    }
    // Physical rows: raw_row() only issues the req_to_token load (index
    // clamped into the row); phys_ok() checks it one block later, so waiting
    // for it never drains the K/V loads issued after it.  -1 = masked token.
    const int r2t_last = max(min(P, p.s.r2t_stride) - 1, 0);
    const int cur_row = (ti.cur_loc >= 0 && ti.cur_loc < p.s.pool_tokens) ? static_cast<int>(ti.cur_loc) : -1;
    const unsigned pool_rows = static_cast<unsigned>(min(p.s.pool_tokens, static_cast<int64_t>(INT_MAX)));
    auto raw_row = [&](int pos) -> int { return r2t[min(max(pos, 0), r2t_last)]; };
    auto phys_ok = [&](int pos, int raw) -> int {
      const int ph = pos == P ? cur_row : raw;
      return (pos < b && ti.req_ok && static_cast<unsigned>(ph) < pool_rows) ? ph : -1;
    };
    auto block_base = [&](int k) { return a + (wave + kWaves * k) * kBlk; };  // k-th block of this wave

    float m = kNegBig, l = 0.0f;
    f32x4_t acc[8];
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) acc[dt] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};

    uint4 kr[8], vr[8];  // rows of tokens 8*quad + i, chunk col (current block)
    int ph[8];           // checked rows of the current block
    int raw[8];          // raw rows of the next block
    auto issue = [&](const int (&rows)[8]) {
#pragma unroll
      for (int i = 0; i < 8; ++i) vr[i] = load_stream16(vbase + static_cast<int64_t>(max(rows[i], 0)) * kv_stride);
#pragma unroll
      for (int i = 0; i < 8; ++i) kr[i] = load_stream16(kbase + static_cast<int64_t>(max(rows[i], 0)) * kv_stride);
    };
    {
      const int b0 = block_base(0), b1 = block_base(1);
#pragma unroll
      for (int i = 0; i < 8; ++i) ph[i] = phys_ok(b0 + 8 * quad + i, raw_row(b0 + 8 * quad + i));
#pragma unroll
      for (int i = 0; i < 8; ++i) raw[i] = raw_row(b1 + 8 * quad + i);
      __builtin_amdgcn_sched_barrier(0);
      issue(ph);
      __builtin_amdgcn_sched_barrier(0);
    }

    const int nblk = ceil_div(b - a, kBlk);
    const int my_blocks = wave < nblk ? ceil_div(nblk - wave, kWaves) : 0;
    for (int k = 0; k < my_blocks; ++k) {
      const int base = block_base(k);
      const int b1 = block_base(k + 1), b2 = block_base(k + 2);
      int nph[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) nph[i] = phys_ok(b1 + 8 * quad + i, raw[i]);
#pragma unroll
      for (int i = 0; i < 8; ++i) raw[i] = raw_row(b2 + 8 * quad + i);
      __builtin_amdgcn_sched_barrier(0);
      // token validity of this block: bit t set if token t has a row
      uint32_t vmask = 0;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const uint64_t bal = __ballot(ph[i] >= 0);
#pragma unroll
        for (int r = 0; r < 4; ++r) vmask |= static_cast<uint32_t>((bal >> (16 * r)) & 1) << (8 * r + i);
      }
      // stage K and V rows (V of masked tokens zeroed) into the wave's tiles
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int tok = 8 * quad + i;
        const uint32_t keep = ph[i] >= 0 ? 0xffffffffu : 0u;
        uint4 w = vr[i];
        w.x &= keep;
        w.y &= keep;
        w.z &= keep;
        w.w &= keep;
        s_k[wave][tok * 16 + (col ^ k_swz(tok))] = kr[i];
        s_v[wave][tok * 16 + (col ^ (2 * (tok & 7)))] = w;
      }
      __builtin_amdgcn_sched_barrier(0);
      // the next block's rows go in flight while this block is computed
#pragma unroll
      for (int i = 0; i < 8; ++i) ph[i] = nph[i];
      issue(ph);
      __builtin_amdgcn_sched_barrier(0);
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

      // S^T = K Q^T for the block's 32 tokens
      f32x4_t st[2];
#pragma unroll
      for (int tile = 0; tile < 2; ++tile) {
        f32x4_t c4 = {0.0f, 0.0f, 0.0f, 0.0f};
        const int tok = 8 * (col >> 2) + 4 * tile + (col & 3);  // MFMA row col of this tile
#pragma unroll
        for (int s = 0; s < 4; ++s)
          c4 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(s_k[wave][tok * 16 + ((4 * s + quad) ^ k_swz(tok))]),
                                                      as_bf16x8(s_q[col * 16 + 4 * s + quad]), c4, 0, 0, 0);
        st[tile] = c4;
      }

      // scale, mask, online softmax (lane-local except the block max)
      float sv[8];
      float bmax = kNegBig;
#pragma unroll
      for (int tile = 0; tile < 2; ++tile) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int tok = 8 * quad + 4 * tile + r;
          const bool ok = head_ok && ((vmask >> tok) & 1) && base + tok >= head_begin;
          const float x = ok ? st[tile][r] * p.q_scale : -INFINITY;
          sv[4 * tile + r] = x;
          bmax = fmaxf(bmax, x);
        }
      }
      bmax = quad_max(bmax);
      // Lazy rescale: the reference point m only moves when the block max
      // exceeds it by more than kRescaleSlack (log2 units), so most blocks
      // skip the 32-accumulator rescale; p <= 2^kRescaleSlack stays exact in
      // fp32 and well inside bf16 range.
      constexpr float kRescaleSlack = 8.0f;
      if (__any(bmax > m + kRescaleSlack)) {
        const float m_new = fmaxf(m, bmax);
        const float alpha = fast_exp2(m - m_new);
        m = m_new;
        l *= alpha;
#pragma unroll
        for (int dt = 0; dt < 8; ++dt) acc[dt] *= alpha;
      }
      bf16x8_t pb;
      float psum = 0.0f;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float pe = fast_exp2(sv[e] - m);
        psum += pe;
        pb[e] = static_cast<__bf16>(pe);
      }
      l += psum;
      // O^T += V^T P^T: the A operand V^T[16 dt + col][tokens 8 quad .. +8]
      // is two transposing reads of tokens 8 quad + 4 h + (col >> 2), dims
      // 16 dt + 4 (col & 3) .. +3 (16-byte chunk 2 dt + ((col & 3) >> 1))
#pragma unroll
      for (int dt = 0; dt < 8; ++dt) {
        bf16x4_t part[2];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const int t = 8 * quad + 4 * h + (col >> 2);
          const int c = (2 * dt + ((col & 3) >> 1)) ^ (2 * (t & 7));
          part[h] = lds_read_tr16(vtile + t * 128 + c * 8 + (col & 1) * 4);
        }
        const bf16x8_t va = __builtin_shufflevector(part[0], part[1], 0, 1, 2, 3, 4, 5, 6, 7);
        acc[dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(va, pb, acc[dt], 0, 0, 0);
      }
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
    }

    l = quad_sum(l);
    // ---- wave result -> LDS (over the K tiles), then combine the four waves ----
    __syncthreads();  // every wave is done with its K tile
    if (head_ok) {
#pragma unroll
      for (int dt = 0; dt < 8; ++dt)
#pragma unroll
        for (int r = 0; r < 4; ++r) s_o[wave][col][16 * dt + 4 * quad + r] = acc[dt][r];
      if (quad == 0) {
        s_ml[wave][col][0] = m;
        s_ml[wave][col][1] = l;
      }
    }
    __syncthreads();
    write_partial<G>(p, ti.g, ti.j, s_o, s_ml);  // next_task's barrier closes the task
  }
}

template <int G>
__global__ void __launch_bounds__(kBlock, 2) span_attention_mfma_kernel(AttnParams p) {
  extern __shared__ int s_off[];  // 2 (NG + 1) task offsets (dynamic)
  __shared__ int s_tmp[kWaves];
  __shared__ uint4 s_k[kWaves][kMfmaBlk * 16];
  __shared__ uint4 s_v[kWaves][kMfmaBlk * 16];
  __shared__ uint4 s_q[16 * 16];
  __shared__ float s_ml[kWaves][G][2];
  static_assert(sizeof(float) * kWaves * G * kHeadDim <= sizeof(uint4) * kWaves * kMfmaBlk * 16, "s_o alias");

  const int NG = p.s.N * p.s.Hkv;
  int total_tasks = 0, chunk = 0, active_wgs = 0;
  plan_tasks(p, s_off, s_tmp, total_tasks, chunk, active_wgs);
  if (static_cast<int>(blockIdx.x) >= active_wgs) return;

  __shared__ int s_task;
  for (int t = next_task(p, s_task); t < total_tasks; t = next_task(p, s_task))
    mfma_task<G>(p, decode_task(p, s_off, NG, chunk, t), s_k, s_v, s_q, s_ml);
}

// ============================================================ 3. merge ====

// One workgroup per (group, query head); lane l of every wave owns dims
// 2l, 2l+1.  The partials are split over the four waves (eight loads in
// flight at a time) and loaded in one pass, so a full-fallback group with
// hundreds of partials is merged in a fraction of the serial latency; the
// four wave states are combined through LDS.  Per head (DECODE:4280-4685):
// ring state = cached entry (hit heads) (+) band partials -> ring row (ready
// requests only); out / out_lse = ring state (+) sink and tail partials.  An empty partial (lse = -inf) has weight 0,
// the reference's skip rule (DECODE:866-890).
struct MergeState {
  float lse;   // natural log; -inf = empty
  float o[2];  // normalised output of the owned dims
};

__device__ __forceinline__ void merge_into(MergeState& st, float lse2, float o0, float o1) {
  if (!isfinite(lse2)) return;
  if (!isfinite(st.lse)) {
    st.lse = lse2;
    st.o[0] = o0;
    st.o[1] = o1;
    return;
  }
  const float mx = fmaxf(st.lse, lse2);
  const float w1 = __expf(st.lse - mx), w2 = __expf(lse2 - mx);
  const float inv = 1.0f / (w1 + w2);
  st.o[0] = (w1 * st.o[0] + w2 * o0) * inv;
  st.o[1] = (w1 * st.o[1] + w2 * o1) * inv;
  st.lse = mx + __logf(w1 + w2);
}

template <int G>
__global__ void __launch_bounds__(kBlock) merge_write_kernel(MergeParams p) {
  constexpr int kBatch = 8;
  const int g = blockIdx.x;
  const int h = blockIdx.y;
  const int n = g / p.s.Hkv;
  const int hkv = g - n * p.s.Hkv;
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int d0 = 2 * lane;
  const int M = p.s.M;
  const int Hq = p.s.Hq;
  const int hq = hkv * G + h;
  const int64_t ho = static_cast<int64_t>(n) * Hq + hq;
  const int P = p.past_lens[n];
  const int req = p.req_ids[n];
  const bool ready = request_ready(p.cache_ready, p.cache_epoch, p.request_epoch, req, p.s.R);
  const int dest = P % M;

  const int band_begin = p.group_rect_begin[g];
  const int new_end = p.group_rect_end[g];
  const int kv_len = p.group_tail_end[g];
  const int sink_end = min(p.F, new_end);
  const int chunk = p.group_chunk[g];
  const int n_sink = ceil_div(sink_end, chunk);
  const int n_band = ceil_div(new_end - band_begin, chunk);
  const int n_tail = ceil_div(kv_len - new_end, chunk);

  __shared__ float s_o[2][kWaves][kHeadDim];
  __shared__ float s_l[2][kWaves];

  auto load_partial = [&](int j, float& lse2, float& o0, float& o1) {
    const int64_t slot = static_cast<int64_t>(g) * p.cap + j;
    lse2 = p.partial_lse[slot * G + h];
    const int64_t oi = static_cast<int64_t>(g) * p.o_group_stride + (static_cast<int64_t>(j) * G + h) * kHeadDim + d0;
    if (p.partial_bf16) {
      const uint32_t w = *reinterpret_cast<const uint32_t*>(static_cast<const uint16_t*>(p.partial_o) + oi);
      o0 = bf16_lo(w);
      o1 = bf16_hi(w);
    } else {
      const float2 v = *reinterpret_cast<const float2*>(static_cast<const float*>(p.partial_o) + oi);
      o0 = v.x;
      o1 = v.y;
    }
  };

  // One pass over all partials of the group (wave w takes j = w, w + 4, ...,
  // eight loads in flight at a time): band partials into `ring` (on top of
  // the cached entry), sink and tail partials into `rest`.
  MergeState ring{-INFINITY, {0.0f, 0.0f}}, rest{-INFINITY, {0.0f, 0.0f}};
  // The cached entry of a hit head (wave 0): its lse and o are loaded
  // together here and merged after the partials, so the partial loads are
  // issued without waiting for them.  A non-finite lse is skipped.
  float entry_lse = -INFINITY;
  uint32_t entry_o = 0;
  const int mslot = p.head_match_slot[ho];
  if (wave == 0 && p.head_hit[ho] != 0 && mslot >= 0 && req >= 0 && req < p.s.R) {
    const int64_t rowi = (static_cast<int64_t>(req) * M + mslot) * Hq + hq;
    entry_lse = p.lse_cache[rowi];
    entry_o = *reinterpret_cast<const uint32_t*>(p.attn_cache + rowi * kHeadDim + d0);
  }
  // this wave's partials of [j0, j1) into `st`, eight loads in flight; wave
  // (first + k) % 4 takes j0 + k, so that consecutive ranges continue the
  // rotation instead of all starting on wave 0
  auto merge_range = [&](MergeState& st, int j0, int j1, int first) {
    for (int jb = j0 + ((wave - first) & (kWaves - 1)); jb < j1; jb += kWaves * kBatch) {
      float pl[kBatch], p0[kBatch], p1[kBatch];
#pragma unroll
      for (int u = 0; u < kBatch; ++u) {
        const int j = jb + kWaves * u;
        load_partial(j < j1 ? j : j0, pl[u], p0[u], p1[u]);
        if (j >= j1) pl[u] = -INFINITY;
      }
#pragma unroll
      for (int u = 0; u < kBatch; ++u) merge_into(st, pl[u], p0[u], p1[u]);
    }
  };
  merge_range(ring, n_sink, n_sink + n_band, 0);
  merge_range(rest, n_sink + n_band, n_sink + n_band + n_tail, n_band);
  merge_range(rest, 0, n_sink, n_band + n_tail);
  merge_into(ring, entry_lse, bf16_lo(entry_o), bf16_hi(entry_o));
  // the four waves' states, combined by wave 0 (which also read the entry:
  // the entry read precedes the ring write below in the same lanes)
  s_o[0][wave][d0] = ring.o[0];
  s_o[0][wave][d0 + 1] = ring.o[1];
  s_o[1][wave][d0] = rest.o[0];
  s_o[1][wave][d0 + 1] = rest.o[1];
  if (lane == 0) {
    s_l[0][wave] = ring.lse;
    s_l[1][wave] = rest.lse;
  }
  __syncthreads();
  if (wave != 0) return;
#pragma unroll
  for (int w = 1; w < kWaves; ++w) {
    merge_into(ring, s_l[0][w], s_o[0][w][d0], s_o[0][w][d0 + 1]);
    merge_into(rest, s_l[1][w], s_o[1][w][d0], s_o[1][w][d0 + 1]);
  }

  if (ready && P >= 0) {  // ring row at past_len % M (a negative past_len has no ring slot)
    const int64_t rowi = (static_cast<int64_t>(req) * M + dest) * Hq + hq;
    const bool valid = isfinite(ring.lse);
    *reinterpret_cast<uint32_t*>(p.query_cache + rowi * kHeadDim + d0) =
        *reinterpret_cast<const uint32_t*>(p.q_pre + ho * kHeadDim + d0);
    const uint32_t packed = valid ? (static_cast<uint32_t>(f32_to_bf16(ring.o[0])) |
                                     (static_cast<uint32_t>(f32_to_bf16(ring.o[1])) << 16))
                                  : 0u;
    *reinterpret_cast<uint32_t*>(p.attn_cache + rowi * kHeadDim + d0) = packed;
    if (lane == 0) p.lse_cache[rowi] = valid ? ring.lse : -INFINITY;
  }
  merge_into(ring, rest.lse, rest.o[0], rest.o[1]);
  const bool valid = isfinite(ring.lse);
  const uint32_t packed = valid ? (static_cast<uint32_t>(f32_to_bf16(ring.o[0])) |
                                   (static_cast<uint32_t>(f32_to_bf16(ring.o[1])) << 16))
                                : 0u;
  *reinterpret_cast<uint32_t*>(p.out + ho * kHeadDim + d0) = packed;
  if (p.out_lse != nullptr && lane == 0) p.out_lse[ho] = valid ? ring.lse : -INFINITY;
}

// ============================================================ host side ====

thread_local char g_err[512] = "";

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

#define MAC_REQUIRE(cond, ...) \
  do {                         \
    if (!(cond)) return fail(MAC_ERR_INVALID_ARGUMENT, __VA_ARGS__); \
  } while (0)

#define MAC_HIP(call)                                                               \
  do {                                                                              \
    hipError_t e_ = (call);                                                         \
    if (e_ != hipSuccess) return fail(MAC_ERR_HIP, "%s: %s", #call, hipGetErrorString(e_)); \
  } while (0)

// MAC_AMD_ATTN_IMPL=valu selects the VALU span-attention kernel; the default
// is the MFMA kernel.  Read once per process.
// Target tasks per workgroup (MAC_AMD_TASKS_PER_WG, read once; 4..64).
int tasks_per_wg() {
  static const int v = [] {
    const char* e = std::getenv("MAC_AMD_TASKS_PER_WG");
    const int x = e != nullptr ? std::atoi(e) : kTasksPerWorkgroup;
    return x < 4 ? 4 : (x > 64 ? 64 : x);
  }();
  return v;
}

// Smallest plan chunk in tokens (MAC_AMD_MIN_CHUNK, read once; 256..16384).
int min_chunk() {
  static const int v = [] {
    const char* e = std::getenv("MAC_AMD_MIN_CHUNK");
    const int x = e != nullptr ? std::atoi(e) : kMinChunk;
    return x < 256 ? 256 : (x > kMaxChunk ? kMaxChunk : x);
  }();
  return v;
}

// MAC_PERSISTENT_MATCH_EARLY_EXIT (the reference's knob, DECODE:5202; read
// once, default on): probe-pruned ring scan for rings split over ranges.
int match_probe() {
  static const int v = [] {
    const char* e = std::getenv("MAC_PERSISTENT_MATCH_EARLY_EXIT");
    return (e != nullptr && std::atoi(e) == 0) ? 0 : 1;
  }();
  return v;
}

// Tokens from which a step runs one span-attention workgroup per CU
// (MAC_AMD_NARROW_TOKENS, read once; default 8M tokens, 4 GB of K/V).
long long narrow_min_tokens() {
  static const long long v = [] {
    const char* e = std::getenv("MAC_AMD_NARROW_TOKENS");
    return e != nullptr ? std::atoll(e) : (8LL << 20);
  }();
  return v;
}

int attn_impl() {
  static const int impl = [] {
    const char* e = std::getenv("MAC_AMD_ATTN_IMPL");
    return (e != nullptr && std::strcmp(e, "valu") == 0) ? 0 : 1;
  }();
  return impl;
}

template <int G>
void* attn_kernel_ptr(int impl) {
  return impl ? reinterpret_cast<void*>(&span_attention_mfma_kernel<G>)
              : reinterpret_cast<void*>(&span_attention_kernel<G>);
}

// Compute units of the device and resident span-attention workgroups per CU
// for a given kernel and dynamic LDS size, cached per process.
std::mutex g_dev_mu;
std::map<std::tuple<int, int, int, size_t>, int> g_blocks_per_cu;
std::map<int, int> g_cus;

int attn_residency(int dev, int G, int impl, size_t dyn_lds, int* cus, int* per_cu) {
  std::lock_guard<std::mutex> lk(g_dev_mu);
  auto ci = g_cus.find(dev);
  if (ci == g_cus.end()) {
    int n = 0;
    MAC_HIP(hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev));
    ci = g_cus.emplace(dev, n).first;
  }
  const auto key = std::make_tuple(dev, G, impl, dyn_lds);
  auto bi = g_blocks_per_cu.find(key);
  if (bi == g_blocks_per_cu.end()) {
    void* fn = nullptr;
    switch (G) {
      case 1: fn = attn_kernel_ptr<1>(impl); break;
      case 2: fn = attn_kernel_ptr<2>(impl); break;
      case 3: fn = attn_kernel_ptr<3>(impl); break;
      case 4: fn = attn_kernel_ptr<4>(impl); break;
      case 5: fn = attn_kernel_ptr<5>(impl); break;
      case 6: fn = attn_kernel_ptr<6>(impl); break;
      case 7: fn = attn_kernel_ptr<7>(impl); break;
      default: fn = attn_kernel_ptr<8>(impl); break;
    }
    int blocks = 0;
    MAC_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(&blocks, fn, kBlock, dyn_lds));
    bi = g_blocks_per_cu.emplace(key, blocks > 0 ? blocks : 1).first;
  }
  *cus = ci->second;
  *per_cu = bi->second;
  return MAC_OK;
}

template <int G>
int launch_all(const DecideParams& dp, const AttnParams& ap, const MergeParams& mp, int attn_grid,
               int impl, hipStream_t stream, hipEvent_t* ev) {
  const int NG = dp.s.N * dp.s.Hkv;
  if (ev) MAC_HIP(hipEventRecord(ev[0], stream));
  if (dp.splits > 1) {
    hipLaunchKernelGGL((match_decide_kernel<G, 1>), dim3(NG, dp.splits), dim3(kBlock), 0, stream, dp);
    MAC_HIP(hipGetLastError());
    hipLaunchKernelGGL((match_decide_kernel<G, 2>), dim3(NG), dim3(kBlock), 0, stream, dp);
  } else {
    hipLaunchKernelGGL((match_decide_kernel<G, 0>), dim3(NG), dim3(kBlock), 0, stream, dp);
  }
  MAC_HIP(hipGetLastError());
  if (ev) MAC_HIP(hipEventRecord(ev[1], stream));
  const size_t plan_lds = 2 * sizeof(int) * (static_cast<size_t>(NG) + 1);
  if (impl)
    hipLaunchKernelGGL(span_attention_mfma_kernel<G>, dim3(attn_grid), dim3(kBlock), plan_lds, stream, ap);
  else
    hipLaunchKernelGGL(span_attention_kernel<G>, dim3(attn_grid), dim3(kBlock), plan_lds, stream, ap);
  MAC_HIP(hipGetLastError());
  if (ev) MAC_HIP(hipEventRecord(ev[2], stream));
  hipLaunchKernelGGL(merge_write_kernel<G>, dim3(NG, G), dim3(kBlock), 0, stream, mp);
  MAC_HIP(hipGetLastError());
  if (ev) MAC_HIP(hipEventRecord(ev[3], stream));
  return MAC_OK;
}

}  // namespace mac

using namespace mac;

extern "C" const char* mac_last_error(void) { return g_err; }
extern "C" int mac_abi_version(void) { return MAC_ABI_VERSION; }

namespace mac {
int decode_impl(const MacDecodeArgs* a, void* stream_ptr, hipEvent_t* ev);
}

extern "C" int mac_persistent_decode_bf16(const MacDecodeArgs* a, void* stream_ptr) {
  return mac::decode_impl(a, stream_ptr, nullptr);
}

extern "C" int mac_persistent_decode_bf16_timed(const MacDecodeArgs* a, void* stream_ptr, float* ms) {
  g_err[0] = '\0';
  MAC_REQUIRE(ms != nullptr, "ms must not be NULL");
  hipEvent_t ev[4];
  for (int i = 0; i < 4; ++i) MAC_HIP(hipEventCreate(&ev[i]));
  int rc = mac::decode_impl(a, stream_ptr, ev);
  if (rc == MAC_OK) {
    hipError_t e = hipEventSynchronize(ev[3]);
    for (int i = 0; i < 3 && e == hipSuccess; ++i) e = hipEventElapsedTime(&ms[i], ev[i], ev[i + 1]);
    if (e != hipSuccess) rc = fail(MAC_ERR_HIP, "event timing: %s", hipGetErrorString(e));
  }
  for (int i = 0; i < 4; ++i) (void)hipEventDestroy(ev[i]);
  return rc;
}

int mac::decode_impl(const MacDecodeArgs* a, void* stream_ptr, hipEvent_t* ev) {
  g_err[0] = '\0';
  MAC_REQUIRE(a != nullptr, "args must not be NULL");
  MAC_REQUIRE(a->struct_size == sizeof(MacDecodeArgs) && a->abi_version == MAC_ABI_VERSION,
              "MacDecodeArgs size/version mismatch (got %u/%u, library expects %zu/%d)",
              a->struct_size, a->abi_version, sizeof(MacDecodeArgs), MAC_ABI_VERSION);
  const int N = a->N, Hq = a->Hq, Hkv = a->Hkv, D = a->D, M = a->M;
  // checks mirror DECODE:5031-5153
  MAC_REQUIRE(D == kHeadDim, "persistent decode v1 supports D=128 only");
  MAC_REQUIRE(Hkv > 0 && Hq % Hkv == 0, "Hq must be divisible by Hkv");
  const int G = Hq / Hkv;
  MAC_REQUIRE(G > 0 && G <= kMaxGroup, "unsupported GQA group size");
  MAC_REQUIRE(N >= 0, "batch must be non-negative");
  MAC_REQUIRE(M > 0, "query_cache capacity M must be positive");
  MAC_REQUIRE(a->R > 0, "query_cache must hold at least one request");
  MAC_REQUIRE(a->workspace_rows >= N, "group_mode workspace too small");
  MAC_REQUIRE(a->tile_tokens > 0 && a->match_tile_slots > 0, "tile sizes must be positive");
  MAC_REQUIRE(a->max_match_tiles >= (M + a->match_tile_slots - 1) / a->match_tile_slots && a->max_match_tiles > 0,
              "match workspace too small");
  MAC_REQUIRE(a->max_tiles_context >= (a->max_context + a->tile_tokens - 1) / a->tile_tokens,
              "rect workspace too small");
  MAC_REQUIRE(a->max_tiles_context >= 4,
              "rect workspace too small: this build needs at least 4 partial slots per group");
  MAC_REQUIRE(a->semantic_pos_ahead >= 0, "semantic_pos_ahead must be non-negative");
  MAC_REQUIRE(a->bench_mode == 0 || a->bench_mode == 1 || a->bench_mode == 2,
              "unsupported synthetic MAC bench mode");
  MAC_REQUIRE(static_cast<int64_t>(N) * Hkv <= kMaxPlanGroups,
              "N * Hkv = %lld exceeds the %d groups one launch can plan", static_cast<long long>(N) * Hkv,
              kMaxPlanGroups);
  MAC_REQUIRE(a->complete_task_len >= static_cast<int64_t>(N) * Hkv + 1, "complete task workspace too small");
  MAC_REQUIRE(a->req_to_token_rows > 0 && a->req_to_token_stride >= 0, "req_to_token must be 2-D");
  if (N == 0) return MAC_OK;
  MAC_REQUIRE(a->q_post && a->q_pre && a->k_buffer && a->v_buffer && a->req_to_token && a->req_ids &&
                  a->past_lens && a->out_cache_loc && a->query_cache && a->attn_cache && a->lse_cache &&
                  a->out && a->match_dist && a->match_pos && a->match_slot && a->head_hit &&
                  a->head_match_slot && a->head_match_pos && a->head_prefix_end && a->head_rect_start &&
                  a->head_new_end && a->group_rect_begin && a->group_rect_end && a->group_rect_tiles &&
                  a->group_tail_begin && a->group_tail_end && a->group_tail_tiles && a->group_mode &&
                  a->complete_task_go && a->complete_task_tile && a->task_counts && a->partial_o &&
                  a->partial_lse,
              "a required pointer is NULL");

  hipStream_t stream = static_cast<hipStream_t>(stream_ptr);
  int dev = 0;
  MAC_HIP(hipGetDevice(&dev));
  int cus = 0, per_cu = 0;
  const int impl = attn_impl();
  const size_t plan_lds = 2 * sizeof(int) * (static_cast<size_t>(N) * Hkv + 1);
  int rc = attn_residency(dev, G, impl, plan_lds, &cus, &per_cu);
  if (rc != MAC_OK) return rc;

  Shape s{};
  s.N = N;
  s.Hq = Hq;
  s.Hkv = Hkv;
  s.M = M;
  s.R = a->R;
  s.pool_tokens = a->pool_tokens;
  s.r2t_rows = a->req_to_token_rows;
  s.r2t_stride = a->req_to_token_stride;
  s.out_cache_loc_is_i64 = a->out_cache_loc_is_i64 ? 1 : 0;
  s.max_match_tiles = a->max_match_tiles;
  s.ws_rows = a->workspace_rows;

  // group_* arrays are indexed n * Hkv + hkv; head_* arrays n * Hq + hq.
  DecideParams dp{};
  dp.s = s;
  dp.q_pre = static_cast<const uint16_t*>(a->q_pre);
  dp.query_cache = static_cast<const uint16_t*>(a->query_cache);
  dp.lse_cache = a->lse_cache;
  dp.req_ids = a->req_ids;
  dp.past_lens = a->past_lens;
  dp.cache_ready = a->cache_ready;
  dp.cache_epoch = a->cache_ready ? a->cache_epoch : nullptr;
  dp.request_epoch = a->cache_ready ? a->request_epoch : nullptr;
  dp.match_dist = a->match_dist;
  dp.match_pos = a->match_pos;
  dp.match_slot = a->match_slot;
  dp.head_hit = a->head_hit;
  dp.head_match_slot = a->head_match_slot;
  dp.head_match_pos = a->head_match_pos;
  dp.head_prefix_end = a->head_prefix_end;
  dp.head_rect_start = a->head_rect_start;
  dp.head_new_end = a->head_new_end;
  dp.group_rect_begin = a->group_rect_begin;
  dp.group_rect_end = a->group_rect_end;
  dp.group_tail_begin = a->group_tail_begin;
  dp.group_tail_end = a->group_tail_end;
  dp.group_mode = a->group_mode;
  dp.task_counter = a->complete_task_tile + static_cast<int64_t>(N) * Hkv;
  // rings of more than two ranges of kSplitSlots slots are scanned by a
  // separate (group, range) launch, one match tile per range
  dp.splits = std::max(1, std::min(a->max_match_tiles, ceil_div(M, kSplitSlots)));
  dp.probe = match_probe();
  if (dp.splits < 3) dp.splits = 1;
  dp.S = a->semantic_pos_ahead;
  dp.F = a->front_sink_tokens > 0 ? a->front_sink_tokens : 0;
  dp.gen_min_limit = a->gen_min_limit;
  dp.lookback_right = a->lookback_right;
  dp.candidate_mode = a->candidate_mode;
  {
    const float thr = static_cast<float>(a->threshold);
    dp.thr_dist = 2.0f * static_cast<float>(D) * (1.0f - thr) * (1.0f - thr);  // DECODE:5342
  }
  dp.mixed_group_fallback = a->mixed_group_fallback;
  dp.bench_mode = a->bench_mode;
  dp.bench_exact_quota = a->bench_exact_quota;
  dp.bench_seed = a->bench_seed;
  dp.bench_miss_mask = a->bench_miss_mask;
  dp.bench_layer_id = a->bench_layer_id;
  dp.bench_hit_rate = static_cast<float>(a->bench_hit_rate);
  dp.bench_hit_rate_std = static_cast<float>(a->bench_hit_rate_std);
  dp.bench_skip_ratio = static_cast<float>(a->bench_skip_ratio);
  dp.bench_skip_ratio_std = static_cast<float>(a->bench_skip_ratio_std);
  dp.bench_match_lag_mean = static_cast<float>(a->bench_match_lag_mean);
  dp.bench_match_lag_std = static_cast<float>(a->bench_match_lag_std);

  const int cap = a->max_tiles_context;
  const int64_t o_group_stride = static_cast<int64_t>(cap) * G * kHeadDim;

  AttnParams ap{};
  ap.s = s;
  ap.q_post = static_cast<const uint16_t*>(a->q_post);
  ap.k_buffer = static_cast<const uint16_t*>(a->k_buffer);
  ap.v_buffer = static_cast<const uint16_t*>(a->v_buffer);
  ap.req_to_token = a->req_to_token;
  ap.req_ids = a->req_ids;
  ap.past_lens = a->past_lens;
  ap.out_cache_loc = a->out_cache_loc;
  ap.head_rect_start = a->head_rect_start;
  ap.group_rect_begin = a->group_rect_begin;
  ap.group_rect_end = a->group_rect_end;
  ap.group_tail_end = a->group_tail_end;
  ap.group_mode = a->group_mode;
  ap.group_rect_tiles = a->group_rect_tiles;
  ap.group_tail_tiles = a->group_tail_tiles;
  ap.group_chunk = a->complete_task_go;
  ap.group_ntasks = a->complete_task_tile;
  ap.task_counts = a->task_counts;
  ap.task_counter = dp.task_counter;
  ap.partial_o = a->partial_o;
  ap.partial_lse = a->partial_lse;
  ap.partial_bf16 = a->partial_o_is_bf16 ? 1 : 0;
  ap.o_group_stride = o_group_stride;
  ap.cap = cap;
  ap.F = dp.F;
  ap.q_scale = static_cast<float>(a->sm_scale) * kLog2e;
  ap.tile_tokens = a->tile_tokens;
  ap.tasks_per_wg = tasks_per_wg();
  ap.min_chunk = min_chunk();
  ap.narrow_grid = impl ? cus : INT_MAX;  // the VALU kernel is instruction-bound: every resident workgroup
  ap.narrow_min_tokens = narrow_min_tokens();

  MergeParams mp{};
  mp.s = s;
  mp.q_pre = dp.q_pre;
  mp.query_cache = static_cast<uint16_t*>(a->query_cache);
  mp.attn_cache = static_cast<uint16_t*>(a->attn_cache);
  mp.lse_cache = a->lse_cache;
  mp.out = static_cast<uint16_t*>(a->out);
  mp.out_lse = a->out_lse;
  mp.req_ids = a->req_ids;
  mp.past_lens = a->past_lens;
  mp.cache_ready = dp.cache_ready;
  mp.cache_epoch = dp.cache_epoch;
  mp.request_epoch = dp.request_epoch;
  mp.head_hit = a->head_hit;
  mp.head_match_slot = a->head_match_slot;
  mp.group_rect_begin = a->group_rect_begin;
  mp.group_rect_end = a->group_rect_end;
  mp.group_tail_end = a->group_tail_end;
  mp.group_chunk = a->complete_task_go;
  mp.partial_o = a->partial_o;
  mp.partial_lse = a->partial_lse;
  mp.partial_bf16 = ap.partial_bf16;
  mp.o_group_stride = o_group_stride;
  mp.cap = cap;
  mp.F = dp.F;

  // Persistent grid: what the device keeps resident, but no more workgroups
  // than the largest task count the caller's max_context allows.
  const int NG = N * Hkv;
  const long long max_tokens = static_cast<long long>(a->max_context) + dp.F + 1;
  const long long max_tasks = static_cast<long long>(NG) * ((max_tokens + 63) / 64 + 3);
  long long grid = static_cast<long long>(cus) * per_cu;
  if (grid > max_tasks) grid = max_tasks;
  if (grid < 1) grid = 1;

  switch (G) {
    case 1: return launch_all<1>(dp, ap, mp, static_cast<int>(grid), impl, stream, ev);
    case 2: return launch_all<2>(dp, ap, mp, static_cast<int>(grid), impl, stream, ev);
    case 3: return launch_all<3>(dp, ap, mp, static_cast<int>(grid), impl, stream, ev);
    case 4: return launch_all<4>(dp, ap, mp, static_cast<int>(grid), impl, stream, ev);
    case 5: return launch_all<5>(dp, ap, mp, static_cast<int>(grid), impl, stream, ev);
    case 6: return launch_all<6>(dp, ap, mp, static_cast<int>(grid), impl, stream, ev);
    case 7: return launch_all<7>(dp, ap, mp, static_cast<int>(grid), impl, stream, ev);
    default: return launch_all<8>(dp, ap, mp, static_cast<int>(grid), impl, stream, ev);
  }
}
