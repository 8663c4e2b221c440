// mac_decode.hip -- MAC-Attention fused decode step for MI355X (gfx950).
//
// One decode step is three kernels on the caller's stream (four for rings
// scanned in slot ranges; graph-capturable, no host synchronisation, no
// allocation):
//
//  1. match_decide  (one workgroup per (request, KV head) group, four or
//     eight waves; for rings of three or more 256-slot ranges, a range-split
//     probe scan over (group, range) workgroups, then the decision kernel)
//     Scans the request's ring of cached pre-RoPE queries for every query head
//     of the group (squared L2, best = smallest distance, ties to the smaller
//     logical position), applies the readiness gate and the optional synthetic
//     bench override, and turns the per-head results into the group's mode and
//     its KV spans: sink [0, min(F, new_end)), band [rect_begin, new_end) and
//     tail [new_end, kv_len).  A short group (at most fuse_tokens tokens: in
//     practice the all-hit groups, whose band is at most the ring capacity) is
//     finished here when the short-group rule says so (short_group: its
//     attention, the merge with the cached entry, the ring row and out).
//     Reference: DECODE:942-1099, :1101-1402.
//
//  2. span_attention  (persistent grid sized to the device's residency)
//     Every workgroup plans the same task list from the group spans: the long
//     groups' spans are cut into chunks of C tokens (C picked from the total
//     token count so that the grid gets ~12 tasks per workgroup; the last
//     quarter of a long band in half chunks where the partial slots allow),
//     a short group left to this kernel is one task, and workgroups claim
//     tasks through an atomic counter, full chunks first.  A task streams its
//     K/V rows in 32-token blocks for all G query heads of the group (S^T =
//     K Q^T and O^T += V^T P^T on v_mfma_f32_16x16x32_bf16, the blocks dealt
//     to four waves, an online log2-domain softmax per head) and writes one
//     partial (o, lse) per head.  Reference producers: DECODE:1870-3423.
//
//  3. merge_write  (one workgroup per (group, query head); those of groups
//     already finished return at once; one more workgroup counts)
//     Per head: cached entry (hit heads) + band partials -> ring row at
//     past_len % M (only for ready requests) -> + sink and tail partials ->
//     out / out_lse.  The counting workgroup writes the per-group task
//     descriptors and the step's counters.  Reference: DECODE:4280-4685.
//
// Workspace use (caller-owned, reference names):
//   head_*, group_mode, group_rect_begin/end, group_tail_begin/end: same
//     meaning as in the reference (DECODE:1270-1402);
//   group_rect_tiles / group_tail_tiles: number of band / tail tasks;
//   complete_task_go[g]: chunk size C_g of group g; complete_task_tile[g]:
//     number of tasks of group g (written by merge_write's counting
//     workgroup);
//     complete_task_go[NG + g]: 1 if match_decide finished group g;
//     complete_task_go[2 NG]: 1 if any group was left to span_attention;
//     complete_task_go[2 NG + 2 .. + 4]: the previous step's short groups,
//     long groups and tokens / 64 (step_fuse_rule);
//     complete_task_tile[NG]: span_attention's task counter (NG = N Hkv);
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

// No multiply-add contraction in this file: every product and sum rounds on
// its own, so the same expression gives the same bits in every kernel it is
// inlined into (a short group computed by match_decide and by span_attention
// must agree bit for bit).
#pragma clang fp contract(off)

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
  // groups of at most fuse_tokens tokens are finished by match_decide itself
  // (attention, merge, ring row, out); group_fused[g] tells the later kernels
  int fuse_tokens;
  int32_t* group_fused;
  int32_t* long_groups;  // set to 1 by every group left to span_attention
  // The previous step's counts for the short-group rule (step_fuse_rule;
  // NULL: every short group is finished here)
  const uint32_t* fuse_sync;
  int fuse_cus;                // span_attention's workgroups in narrow mode
  long long narrow_min_tokens;  // span_attention's narrow-mode threshold
  const uint16_t* q_post;
  const uint16_t* k_buffer;
  const uint16_t* v_buffer;
  const int32_t* req_to_token;
  const void* out_cache_loc;
  uint16_t* ring_q;  // query_cache (written for finished groups)
  uint16_t* attn_cache;
  float* ring_lse;   // lse_cache
  uint16_t* out;
  float* out_lse;
  float q_scale;  // sm_scale * log2(e)
  int64_t* phase_cycles;  // stamps (debug_enabled >= 2), else NULL
  int stamp_first;        // this launch records the step's first stamp
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
  int32_t* task_counts;   // [0] tasks and [4] the plan's chunk (workgroup 0)
  int32_t* task_counter;   // complete_task_tile[N * Hkv]; zeroed by match_decide
  void* partial_o;
  float* partial_lse;
  int partial_bf16;
  int64_t o_group_stride;  // elements of partial_o per group
  int cap;                 // task slots per group
  int F;
  int tasks_per_wg;  // target tasks per workgroup of the plan
  int narrow_grid;                // workgroups that take tasks when a step has
  long long narrow_min_tokens;    // at least this many tokens (the others return)
  int min_chunk;     // smallest chunk of the plan (tokens)
  float q_scale;  // sm_scale * log2(e)
  const int32_t* group_fused;  // groups match_decide finished (no tasks here)
  const int32_t* long_groups;  // 0: match_decide finished every group
  int fuse_tokens;             // a group of at most fuse_tokens tokens is short (0: none)
  int plan_bucket;             // groups per entry of the plan's LDS offset table
  int64_t* phase_cycles;
  // short groups match_decide left here (one task each, short_group)
  const uint16_t* q_pre;
  uint16_t* ring_q;
  uint16_t* attn_cache;
  float* lse_cache;
  uint16_t* out;
  float* out_lse;
  const uint8_t* cache_ready;
  const int64_t* cache_epoch;
  const int64_t* request_epoch;
  const int32_t* head_hit;
  const int32_t* head_match_slot;
  int R;
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
  const void* partial_o;
  const float* partial_lse;
  int partial_bf16;
  int64_t o_group_stride;
  int cap;
  int F;
  const int32_t* group_fused;
  int32_t* long_groups;  // cleared here for the next step
  int64_t* phase_cycles;
  int fuse_tokens;  // short groups (at most this many tokens) have no partials: skipped
  // the counting workgroup's outputs (publish_counts)
  const int32_t* group_mode;
  int32_t* group_chunk_out;  // complete_task_go
  int32_t* group_ntasks;     // complete_task_tile
  int32_t* group_rect_tiles;
  int32_t* group_tail_tiles;
  int32_t* task_counts;      // [0] and [4] come from span_attention
  uint32_t* fuse_sync;       // the next step's short-group rule (NULL: no rule)
  int tile_tokens;
};

// Whether this step's short groups are finished here.  Finishing a short
// group in this kernel takes it out of span_attention and merge_write but
// adds its stream to this kernel, which runs before them: worth it when no
// group is long (span_attention and merge_write then have nothing to do), or
// when span_attention runs one workgroup per CU and the short groups' band
// and tail tasks would need more than one round of them.  Otherwise they are
// left to span_attention, where they fill the workgroups that finish their
// long tasks first.  The counts the rule needs are the whole step's, which a
// workgroup cannot know when it decides (a device-wide count and wait, or
// even just counting with atomics on shared words, cost more than the rule
// saves), so it reads the previous step's, which merge_write's counting
// workgroup leaves in fuse_sync: [0] short groups, [1] long groups, [2]
// tokens / 64.
// Decode steps of a batch change slowly, so the previous step's counts are
// the usual case.  The rule only moves work between kernels: both run a short
// group through short_group with the same states, combine order and merges,
// so its results are the same bits either way, and a step's results do not
// depend on the steps before it (MAC_AMD_FUSE_POLICY pins the choice, for
// measurements).
__device__ __forceinline__ int step_fuse_rule(const DecideParams& p, const uint32_t (&c)[3]) {
  const uint32_t n_short = c[0], n_long = c[1];
  const long long all_tokens = static_cast<long long>(c[2]) << 6;
  // counts of a different batch shape (or none yet: a workspace's first
  // step) are no history: short groups are finished here
  if (n_short + n_long != static_cast<uint32_t>(p.s.N) * static_cast<uint32_t>(p.s.Hkv)) return 1;
  if (n_long == 0) return 1;
  return (all_tokens >= p.narrow_min_tokens && 2ll * n_short > p.fuse_cus) ? 1 : 0;
}

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

// threadIdx.x behind an empty asm statement: the addresses derived from it
// inside a task body are then computed per task instead of being hoisted out
// of span_attention's task loop and held in registers across every task.
__device__ __forceinline__ int task_tid() {
  int t = static_cast<int>(threadIdx.x);
  asm volatile("" : "+v"(t));
  return t;
}

// 16-byte non-temporal (streaming) global load.
__device__ __forceinline__ uint4 load_stream16(const uint16_t* ptr) {
  return __builtin_bit_cast(uint4, __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(ptr)));
}


// ------------------------------------------------- MFMA block stream ----
//
// The K/V stream both attention paths share (span_attention for long spans,
// match_decide for groups it finishes itself).  One 64-lane wave owns a
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
//  * The rows are staged in two 8 KiB per-wave LDS tiles, token-major, with
//    XOR-swizzled 16-byte chunks (k_swz / v_swz below) so that the operand
//    reads of the MFMAs hit distinct banks.
//  * S^T[t][g] = sum_d K[t][d] Q[g][d] and O^T[d][g] += sum_t V[t][d] P[g][t]
//    both run on v_mfma_f32_16x16x32_bf16.  MFMA row 4a + i of score tile t
//    is token 8a + 4t + i, so the lane holding head g = l%16 ends with the
//    scores of tokens 8q .. 8q + 7 (q = l/16): after conversion to bf16 they
//    are the B operand of the PV product as they stand, and its A operand
//    V^T[16 dt + g][8q .. 8q + 7] is two ds_read_b64_tr_b16 (gfx950's
//    transposing LDS read) of the V tile.  The lane keeps its head's softmax
//    state and 32 O^T accumulators, so the online-softmax rescale is
//    lane-local.  Heads g >= G are zero padding rows of the 16-wide MFMA.
//  * The Q operand (B of the score MFMAs) is read from LDS into registers
//    once per stream: read per block, its 16 lanes of a quarter-wave hit one
//    bank group (the rows are 256 bytes apart).

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ bf16x8_t as_bf16x8(const uint4& w) { return __builtin_bit_cast(bf16x8_t, w); }

// K tile: 16-byte chunk c of token t at position c ^ k_swz(t) of its row.
// The S^T tiles read tokens 8a + 4t + i (a, i < 4) in one instruction; this
// swizzle puts the 16 of them on 16 different chunk positions.
__device__ __forceinline__ int k_swz(int t) { return 4 * ((t >> 3) & 3) + (t & 3); }
// V tile: chunk c of token t at c ^ v_swz(t).  One transposing read covers,
// per 32-lane half, tokens 16h' + 4h + (0..3) and 16h' + 8 + 4h + (0..3)
// (two quarter-waves) at two chunk bases and two 8-byte halves: with bit 3 of
// the token in the swizzle the 32 lanes read 32 different 8-byte bank pairs
// of the 64 banks.
__device__ __forceinline__ int v_swz(int t) { return 2 * ((t & 3) | ((t >> 1) & 4)); }

constexpr int kMfmaBlk = 32;  // tokens per wave block
constexpr int kVirtualWaves = 4;  // a stream's blocks are dealt to four virtual waves
constexpr int kTileU4 = kMfmaBlk * 16;  // uint4 per K or V tile

// Softmax state of one lane: its head's running max m (log2 units) and sum l
// and the 32 O^T accumulators (dims 16 dt + 4 quad + r).
struct WaveState {
  f32x4_t acc[8];
  float m, l;
};

__device__ __forceinline__ void state_reset(WaveState& s) {
#pragma unroll
  for (int dt = 0; dt < 8; ++dt) s.acc[dt] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
  s.m = kNegBig;
  s.l = 0.0f;
}

// Per-lane constants of the K/V stream of one (request, KV head).
struct KvStream {
  const int32_t* r2t;     // req_to_token row of the request
  int r2t_last;           // last column that may be read
  int r2t_cols;           // positions at or past it (other than P) have no row
  int P;                  // position of the current token (pool row cur_row)
  int cur_row;            // out_cache_loc of the request, -1 if outside the pool
  unsigned pool_rows;
  bool req_ok;
  const uint16_t* kbase;  // K / V row base of the KV head + this lane's chunk
  const uint16_t* vbase;
  int64_t kv_stride;      // elements between consecutive pool rows

  // req_to_token entry of a position (index clamped into the row)
  __device__ __forceinline__ int raw_row(int pos) const { return r2t[min(max(pos, 0), r2t_last)]; }
  // Checked pool row of position pos of a range ending at `end`, given its
  // raw entry: -1 = masked (past the range, outside the pool, or at a
  // position the req_to_token row does not reach).
  __device__ __forceinline__ int row_of(int pos, int end, int raw) const {
    const bool cur = pos == P;
    const int ph = cur ? cur_row : raw;
    return (pos < end && req_ok && (cur || pos < r2t_cols) && static_cast<unsigned>(ph) < pool_rows) ? ph : -1;
  }
  __device__ __forceinline__ uint4 k_chunk(int row) const {
    return load_stream16(kbase + static_cast<int64_t>(max(row, 0)) * kv_stride);
  }
  __device__ __forceinline__ uint4 v_chunk(int row) const {
    return load_stream16(vbase + static_cast<int64_t>(max(row, 0)) * kv_stride);
  }
};


__device__ __forceinline__ KvStream make_stream(const int32_t* req_to_token, int r2t_rows, int r2t_stride,
                                                int req, int P, int64_t cur_loc, int64_t pool_tokens,
                                                const uint16_t* k_buffer, const uint16_t* v_buffer,
                                                int Hkv, int hkv, int col) {
  KvStream ks;
  ks.req_ok = req >= 0 && req < r2t_rows;
  ks.r2t = req_to_token + static_cast<int64_t>(ks.req_ok ? req : 0) * r2t_stride;
  ks.r2t_last = max(min(P, r2t_stride) - 1, 0);
  ks.r2t_cols = r2t_stride;
  ks.P = P;
  ks.cur_row = (cur_loc >= 0 && cur_loc < pool_tokens) ? static_cast<int>(cur_loc) : -1;
  ks.pool_rows = static_cast<unsigned>(min(pool_tokens, static_cast<int64_t>(INT_MAX)));
  ks.kv_stride = static_cast<int64_t>(Hkv) * kHeadDim;
  ks.kbase = k_buffer + static_cast<int64_t>(hkv) * kHeadDim + col * 8;
  ks.vbase = v_buffer + static_cast<int64_t>(hkv) * kHeadDim + col * 8;
  return ks;
}

// Up to three token ranges, each cut into 32-token blocks from its begin;
// blocks are numbered across them: [0, first1) range 0, [first1, first2)
// range 1, [first2, nblk) range 2.  Range 0 applies the per-head start mask
// (the band of a group whose heads start at different positions).
struct BlockList {
  int begin0, end0, first1;
  int begin1, end1, first2;
  int begin2, end2, nblk;
};

__device__ __forceinline__ BlockList one_range(int a, int b) {
  BlockList bl;
  const int nb = ceil_div(max(b - a, 0), kMfmaBlk);
  bl.begin0 = a;
  bl.end0 = b;
  bl.first1 = bl.first2 = bl.nblk = nb;
  bl.begin1 = bl.end1 = bl.begin2 = bl.end2 = b;
  return bl;
}

// First position and end of block v (blocks past the last one are empty).
__device__ __forceinline__ void block_span(const BlockList& bl, int v, int& base, int& end) {
  if (v < bl.first1) {
    base = bl.begin0 + v * kMfmaBlk;
    end = bl.end0;
  } else if (v < bl.first2) {
    base = bl.begin1 + (v - bl.first1) * kMfmaBlk;
    end = bl.end1;
  } else {
    base = bl.begin2 + (v - bl.first2) * kMfmaBlk;
    end = bl.end2;
  }
}

// Streams one virtual wave's blocks of `bl` into `st`; qb: this lane's Q
// operands (k-steps 0..3).  Blocks are dealt to four virtual waves, vw
// taking every fourth one, so that the states a computation ends with do not
// depend on how many hardware waves run it.  One class (kTwoClass false):
// blocks vw, vw + 4, ... of the list; range 0 is masked per head from
// head_begin on (a band piece), ranges 1 and 2 are not.  Two classes: blocks
// [0, first2) (ranges 0 and 1: sink and tail) are the rest class and end in
// `st`; blocks [first2, nblk) (range 2: the band, masked per head) are the
// ring class and end in `ring`; each class is dealt to the virtual waves
// separately (rest block j and band block j both go to virtual wave j % 4),
// and do_rest / do_ring select the classes this hardware wave streams (a
// four-wave workgroup streams both, rest first; an eight-wave one gives each
// class its own four waves).  pre0/pre1 (when not NULL): the req_to_token
// entries of the wave's first two rest blocks, loaded by the caller.
template <int G, bool kTwoClass>
__device__ __forceinline__ void stream_blocks(const KvStream& ks, const BlockList& bl, int head_begin,
                                              float q_scale, const bf16x8_t (&qb)[4], uint4* s_kw,
                                              uint4* s_vw, WaveState& st, WaveState& ring, int vw,
                                              bool do_rest = true, bool do_ring = true,
                                              const int* pre0 = nullptr, const int* pre1 = nullptr) {
  const int lane = task_tid() & 63;
  const int quad = lane >> 4;
  const int col = lane & 15;
  const bool head_ok = col < G;
  const uint16_t* vtile = reinterpret_cast<const uint16_t*>(s_vw);
  constexpr int kV = kVirtualWaves;
  auto share = [&](int nb) { return nb > vw ? (nb - vw + kV - 1) / kV : 0; };
  const int rest_end = kTwoClass ? bl.first2 : bl.nblk;
  const int n_rest = do_rest ? share(rest_end) : 0;
  const int n_ring = (kTwoClass && do_ring) ? share(bl.nblk - bl.first2) : 0;
  const int my_blocks = n_rest + n_ring;
  // list index of this wave's k-th block (past its last: an empty block)
  auto vidx = [&](int k) -> int {
    if (k < n_rest) return vw + kV * k;
    if (k < my_blocks) return bl.first2 + vw + kV * (k - n_rest);
    return bl.nblk + kV * (k - my_blocks);
  };

  // raw_row() only issues the req_to_token load; phys_ok() checks it one
  // block later, so waiting for it never drains the K/V loads issued after it.
  auto raw_row = [&](int pos) -> int { return ks.raw_row(pos); };
  auto phys_ok = [&](int pos, int end, int raw) -> int { return ks.row_of(pos, end, raw); };

  uint4 kr[8], vr[8];  // rows of tokens 8*quad + i, chunk col (next block)
  int ph[8];           // checked rows of the block in flight
  int raw[8];          // raw rows of the block after it
  auto issue = [&](const int (&rows)[8]) {
#pragma unroll
    for (int i = 0; i < 8; ++i) vr[i] = ks.v_chunk(rows[i]);
#pragma unroll
    for (int i = 0; i < 8; ++i) kr[i] = ks.k_chunk(rows[i]);
  };
  {
    int b0, e0, b1, e1;
    block_span(bl, vidx(0), b0, e0);
    block_span(bl, vidx(1), b1, e1);
    const bool use0 = pre0 != nullptr && n_rest > 0;
    const bool use1 = pre1 != nullptr && n_rest > 1;
#pragma unroll
    for (int i = 0; i < 8; ++i) ph[i] = phys_ok(b0 + 8 * quad + i, e0, use0 ? pre0[i] : raw_row(b0 + 8 * quad + i));
#pragma unroll
    for (int i = 0; i < 8; ++i) raw[i] = use1 ? pre1[i] : raw_row(b1 + 8 * quad + i);
    __builtin_amdgcn_sched_barrier(0);
    issue(ph);
    __builtin_amdgcn_sched_barrier(0);
  }

  bool switched = false;
  for (int k = 0; k < my_blocks; ++k) {
    const int v = vidx(k);
    if (kTwoClass && !switched && k == n_rest) {  // sink and tail done: st -> ring for the band
      ring = st;
      state_reset(st);
      switched = true;
    }
    int base, end_unused, b1, e1, b2, e2;
    block_span(bl, v, base, end_unused);
    block_span(bl, vidx(k + 1), b1, e1);
    block_span(bl, vidx(k + 2), b2, e2);
    const int hb = (kTwoClass ? v >= bl.first2 : v < bl.first1) ? head_begin : 0;
    int nph[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) nph[i] = phys_ok(b1 + 8 * quad + i, e1, raw[i]);
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
      s_kw[tok * 16 + (col ^ k_swz(tok))] = kr[i];
      s_vw[tok * 16 + (col ^ v_swz(tok))] = w;
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
    f32x4_t sc[2];
#pragma unroll
    for (int tile = 0; tile < 2; ++tile) {
      f32x4_t c4 = {0.0f, 0.0f, 0.0f, 0.0f};
      const int tok = 8 * (col >> 2) + 4 * tile + (col & 3);  // MFMA row col of this tile
#pragma unroll
      for (int s = 0; s < 4; ++s)
        c4 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(s_kw[tok * 16 + ((4 * s + quad) ^ k_swz(tok))]),
                                                    qb[s], c4, 0, 0, 0);
      sc[tile] = c4;
    }

    // scale, mask, online softmax (lane-local except the block max)
    float sv[8];
    float bmax = kNegBig;
#pragma unroll
    for (int tile = 0; tile < 2; ++tile) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int tok = 8 * quad + 4 * tile + r;
        const bool ok = head_ok && ((vmask >> tok) & 1) && base + tok >= hb;
        const float x = ok ? sc[tile][r] * q_scale : -INFINITY;
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
    if (__any(bmax > st.m + kRescaleSlack)) {
      const float m_new = fmaxf(st.m, bmax);
      const float alpha = fast_exp2(st.m - m_new);
      st.m = m_new;
      st.l *= alpha;
#pragma unroll
      for (int dt = 0; dt < 8; ++dt) st.acc[dt] *= alpha;
    }
    // P goes to the PV product as bf16 hi + lo (two MFMAs per tile): the
    // probabilities keep ~16 mantissa bits, so long spans accumulate the
    // bf16 rounding of V only, not that of P as well.
    bf16x8_t pb, pl;
    float psum = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float pe = fast_exp2(sv[e] - st.m);
      psum += pe;
      pb[e] = static_cast<__bf16>(pe);
      pl[e] = static_cast<__bf16>(pe - static_cast<float>(pb[e]));
    }
    st.l += psum;
    // O^T += V^T P^T: the A operand V^T[16 dt + col][tokens 8 quad .. +8]
    // is two transposing reads of tokens 8 quad + 4 h + (col >> 2), dims
    // 16 dt + 4 (col & 3) .. +3 (16-byte chunk 2 dt + ((col & 3) >> 1))
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) {
      bf16x4_t part[2];
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int t = 8 * quad + 4 * h + (col >> 2);
        const int c = (2 * dt + ((col & 3) >> 1)) ^ v_swz(t);
        part[h] = lds_read_tr16(vtile + t * 128 + c * 8 + (col & 1) * 4);
      }
      const bf16x8_t va = __builtin_shufflevector(part[0], part[1], 0, 1, 2, 3, 4, 5, 6, 7);
      st.acc[dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(va, pb, st.acc[dt], 0, 0, 0);
      st.acc[dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(va, pl, st.acc[dt], 0, 0, 0);
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
  }
  if (kTwoClass) {  // st: band blocks (if any), ring: sink and tail -> swap
    if (switched) {
      const WaveState t = st;
      st = ring;
      ring = t;
    } else {
      state_reset(ring);
    }
  }
  st.l = quad_sum(st.l);
  if (kTwoClass) ring.l = quad_sum(ring.l);
}

// This lane's Q operands of the score MFMAs from the 16 x 128 Q tile in LDS
// (rows g >= G zero): k-step s reads Q[col][8 (4 s + quad) .. + 8].
__device__ __forceinline__ void load_q_operands(const uint4* s_q, bf16x8_t (&qb)[4]) {
  const int lane = task_tid() & 63;
  const int quad = lane >> 4, col = lane & 15;
#pragma unroll
  for (int s = 0; s < 4; ++s) qb[s] = as_bf16x8(s_q[col * 16 + 4 * s + quad]);
}

// Stores this lane's part of virtual wave vw's state into the LDS combine
// area: so[vw][head][dim] (row pitch kOPitch floats), sml[vw][head] = (m, l).
constexpr int kOPitch = kHeadDim + 4;  // padded: lanes of different heads hit different banks
template <int G>
__device__ __forceinline__ void state_to_lds(const WaveState& st, float* so, float* sml, int wave) {
  const int lane = task_tid() & 63;
  const int quad = lane >> 4, col = lane & 15;
  if (col < G) {
    float* row = so + (wave * G + col) * kOPitch;
#pragma unroll
    for (int dt = 0; dt < 8; ++dt)
#pragma unroll
      for (int r = 0; r < 4; ++r) row[16 * dt + 4 * quad + r] = st.acc[dt][r];
    if (quad == 0) {
      sml[(wave * G + col) * 2] = st.m;
      sml[(wave * G + col) * 2 + 1] = st.l;
    }
  }
}

// Normalised (o[d], o[d+1], natural-log lse) of head h from the four wave
// states in LDS; lse = -inf and o = 0 for an empty state.
template <int G, int W = kWaves>
__device__ __forceinline__ void combine_waves(const float* so, const float* sml, int h, int d, float& o0,
                                              float& o1, float& lse) {
  float mm = kNegBig;
#pragma unroll
  for (int w = 0; w < W; ++w) mm = fmaxf(mm, sml[(w * G + h) * 2]);
  float ll = 0.0f, a0 = 0.0f, a1 = 0.0f;
#pragma unroll
  for (int w = 0; w < W; ++w) {
    const float sc = fast_exp2(sml[(w * G + h) * 2] - mm);
    ll += sml[(w * G + h) * 2 + 1] * sc;
    a0 += so[(w * G + h) * kOPitch + d] * sc;
    a1 += so[(w * G + h) * kOPitch + d + 1] * sc;
  }
  const bool nonempty = ll > 0.0f;
  const float inv = nonempty ? 1.0f / ll : 0.0f;
  o0 = a0 * inv;
  o1 = a1 * inv;
  lse = nonempty ? (mm + log2f(ll)) * kLn2 : -INFINITY;
}

// LSE merge of (lse2, o0, o1) into st (natural log).  An operand with a
// non-finite lse is empty and skipped (DECODE:866-890).
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

__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
  return pack2_bf16(a, b);
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
// complete_task_go / _tile entries beyond 2 N Hkv: the long-group flag, one
// spare, the previous step's counts for the short-group rule, one spare
constexpr int kTaskExtra = 6;
constexpr int kLsePrefetchSlots = 64;
constexpr int kProbeSlots = 4;  // probe scan: slot pairs per lane batch and pass

// Per-head decisions and group spans of group g (wave 0; lanes 0..G-1 own a
// head each), DECODE:1147-1402.  Publishes in LDS what short_group needs:
// per head its band start, the slot of a reusable cached entry (-1: none)
// and that entry's lse; the group's band begin, new_end and whether
// match_decide finishes the group itself.
template <int G, int kMode, int W = kWaves>
__device__ __forceinline__ void decide_group(const DecideParams& p, const float (*s_d)[kMaxGroup],
                                             const int (*s_p)[kMaxGroup], const int (*s_s)[kMaxGroup],
                                             const float (*s_lse)[kLsePrefetchSlots], bool lse_in_lds, int g,
                                             int n, int hkv, int P, int req, bool eligible,
                                             const uint32_t (&rule_counts)[3], int* s_rect,
                                             int* s_mslot, float* s_entry, int* s_span) {
  const int lane = threadIdx.x & 63;
  const int M = p.s.M;
  const int Hq = p.s.Hq;
  const int h = lane;
  const bool head_lane = h < G;
  const int hq = hkv * G + (head_lane ? h : 0);
  float bd = INFINITY;
  int bp = INT_MAX, bs = -1;
  if (head_lane) {
    for (int w = 0; w < W; ++w) {
      if (better_pair(s_d[w][h], s_p[w][h], bd, bp)) {
        bd = s_d[w][h];
        bp = s_p[w][h];
        bs = s_s[w][h];
      }
    }
  }
  if (!eligible) {  // the readiness gate and the candidate window, applied after the scan
    bd = INFINITY;
    bp = INT_MAX;
    bs = -1;
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
  float pl = -INFINITY;
  if (head_lane && hit && mslot >= 0) {
    pl = lse_in_lds ? s_lse[h][mslot] : p.lse_cache[(static_cast<int64_t>(req) * M + mslot) * Hq + hq];
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
  // a group of few tokens is finished by this kernel (no tasks, no merge)
  const long long tokens = static_cast<long long>(fs_begin) + (new_end - rb) + max(P + 1 - new_end, 0);
  const bool is_short = p.fuse_tokens > 0 && tokens <= p.fuse_tokens;
  int fused = is_short ? 1 : 0;
  if (is_short && p.fuse_sync != nullptr) fused = step_fuse_rule(p, rule_counts);
  if (head_lane) {
    s_rect[h] = rect_start;
    s_mslot[h] = hit ? mslot : -1;
    s_entry[h] = hit ? pl : -INFINITY;
  }
  if (lane == 0) {
    const int64_t go = static_cast<int64_t>(n) * p.s.Hkv + hkv;
    p.group_mode[go] = mode;
    p.group_rect_begin[go] = rb;
    p.group_rect_end[go] = new_end;
    p.group_tail_begin[go] = new_end;
    p.group_tail_end[go] = P + 1;
    p.group_fused[g] = fused;
    if (!fused) *p.long_groups = 1;
    s_span[0] = rb;
    s_span[1] = new_end;
    s_span[2] = fused;
  }
}

// The decision-independent part of a group's blocks: sink [0, min(F,
// new_end)) as range 0 and tail [new_end, P + 1) as range 1 (range 2 empty).
__device__ __forceinline__ BlockList rest_blocks(int P, int new_end, int F) {
  BlockList bl;
  const int sink_end = min(F, new_end);
  bl.begin0 = 0;
  bl.end0 = sink_end;
  bl.first1 = ceil_div(max(sink_end, 0), kMfmaBlk);
  bl.begin1 = new_end;
  bl.end1 = P + 1;
  bl.first2 = bl.first1 + ceil_div(max(P + 1 - new_end, 0), kMfmaBlk);
  bl.begin2 = bl.end2 = new_end;
  bl.nblk = bl.first2;
  return bl;
}

// What a short group's computation reads and writes besides its K/V stream.
struct ShortCtx {
  const uint16_t* q_pre;
  uint16_t* ring_q;      // query_cache
  uint16_t* attn_cache;  // cached entries in, ring rows out
  float* ring_lse;       // lse_cache
  uint16_t* out;
  float* out_lse;
  int Hq, M, R, F;
  float q_scale;
};

// The short-group computation (a group of at most fuse_tokens tokens: in
// practice the hit groups, whose band is at most the ring capacity, and short
// requests): its sink, tail and band are streamed by four virtual waves
// (stream_blocks' two-class deal), the virtual waves' states are combined in
// LDS, and the merge of DECODE:4280-4685 follows in place -- ring state =
// band (+) cached entry -> ring row at past_len % M (ready requests only);
// out = ring state (+) sink and tail -- with no partials and no merge
// launch.  match_decide runs it for the groups it finishes (four or eight
// hardware waves), span_attention as one task (four): the states, the
// combine order and the merges are the same in every case, so a group's
// results are bit for bit the same wherever it runs.
//   s_rect / s_mslot / s_entry: per head its band start, the slot of a
//   reusable cached entry (-1: none) and that entry's lse (LDS);
//   s_kv: 2 x W K/V tiles (the combine area afterwards); s_q: 16 x 16 uint4;
//   s_ml: [2][4][G][2] floats; pre: req_to_token entries of the wave's first
//   two rest blocks (or NULL).
template <int G, int W, bool kSeq>
__device__ __forceinline__ void short_group(const ShortCtx& c, int n, int hkv, int P, int req, bool ready,
                                            int band_begin, int new_end, const int* s_rect, const int* s_mslot,
                                            const float* s_entry, uint4 qpost_w, const KvStream& ks,
                                            const int (*pre)[8], uint4* s_kv, uint4* s_q, float* s_ml) {
  static_assert(W == kVirtualWaves || W == 2 * kVirtualWaves, "four or eight waves");
  static_assert(!kSeq || W == kVirtualWaves, "the sequential form runs on four waves");
  constexpr int kV = kVirtualWaves;
  constexpr int kPairs = (G * 64 + (W * 64) - 1) / (W * 64);  // dim pairs per thread in the epilogue
  const int tid = task_tid();
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int vw = wave & (kV - 1);
  const int col = tid & 15;
  const int Hq = c.Hq;
  const int M = c.M;
  const bool req_ok = req >= 0 && req < c.R;

  if (tid < 16 * 16) s_q[tid] = qpost_w;
  // the cached entries (hit heads) and the pre-RoPE query rows of the
  // epilogue, in flight during the stream
  uint32_t ent[kPairs], qpre[kPairs];
#pragma unroll
  for (int i = 0; i < kPairs; ++i) {
    const int e = tid + i * (W * 64);
    ent[i] = 0;
    qpre[i] = 0;
    if (e < G * 64) {
      const int h = e >> 6, d0 = 2 * (e & 63), hq = hkv * G + h;
      const int ms = s_mslot[h];
      if (ms >= 0 && req_ok)
        ent[i] = *reinterpret_cast<const uint32_t*>(c.attn_cache +
                                                    ((static_cast<int64_t>(req) * M + ms) * Hq + hq) * kHeadDim + d0);
      qpre[i] = *reinterpret_cast<const uint32_t*>(c.q_pre + (static_cast<int64_t>(n) * Hq + hq) * kHeadDim + d0);
    }
  }
  __syncthreads();
  bf16x8_t qb[4];
  load_q_operands(s_q, qb);

  // blocks: sink [0, min(F, new_end)), tail [new_end, P + 1), band [band_begin, new_end)
  BlockList bl = rest_blocks(P, new_end, c.F);
  bl.begin2 = band_begin;
  bl.end2 = new_end;
  bl.nblk = bl.first2 + ceil_div(max(new_end - band_begin, 0), kMfmaBlk);
  float* so = reinterpret_cast<float*>(s_kv);
  float* so_rest = so + kV * G * kOPitch;
  float* sml_rest = s_ml + kV * G * 2;
  const int head_begin = col < G ? s_rect[col] : 0;
  uint4* s_kw = s_kv + wave * kTileU4;
  uint4* s_vw = s_kv + (W + wave) * kTileU4;
  float rg[kPairs][3];  // the ring class combined: (o[d0], o[d0 + 1], lse) of each pair
  if constexpr (kSeq) {
    // one state at a time: the band (the ring class), combined into
    // registers, then the sink and tail (the rest class).  Each class's
    // blocks go to the same virtual waves, in the same order, as in the
    // two-class stream, and the band's and the rest's block lists number
    // their blocks as its ranges 2 and 0, 1 do.
    WaveState st, unused;
    state_reset(st);
    stream_blocks<G, false>(ks, one_range(band_begin, new_end), head_begin, c.q_scale, qb, s_kw, s_vw, st,
                            unused, vw);
    __syncthreads();  // every wave is done with its tiles
    state_to_lds<G>(st, so, s_ml, vw);
    __syncthreads();
#pragma unroll
    for (int i = 0; i < kPairs; ++i) {
      const int e = tid + i * (W * 64);
      rg[i][0] = rg[i][1] = 0.0f;
      rg[i][2] = -INFINITY;
      if (e < G * 64) combine_waves<G, kV>(so, s_ml, e >> 6, 2 * (e & 63), rg[i][0], rg[i][1], rg[i][2]);
    }
    __syncthreads();  // the combine area is the tiles again
    BlockList rl;  // sink as range 1, tail as range 2 (range 0, the masked one, empty)
    rl.begin0 = rl.end0 = 0;
    rl.first1 = 0;
    rl.begin1 = bl.begin0;
    rl.end1 = bl.end0;
    rl.first2 = bl.first1;
    rl.begin2 = bl.begin1;
    rl.end2 = bl.end1;
    rl.nblk = bl.first2;
    state_reset(st);
    stream_blocks<G, false>(ks, rl, 0, c.q_scale, qb, s_kw, s_vw, st, unused, vw, true, true,
                            pre != nullptr ? pre[0] : nullptr, pre != nullptr ? pre[1] : nullptr);
    __syncthreads();
    state_to_lds<G>(st, so_rest, sml_rest, vw);
    __syncthreads();
  } else {
    WaveState rest, ring;
    state_reset(rest);
    state_reset(ring);
    const bool do_rest = W == kV || wave < kV;
    const bool do_ring = W == kV || wave >= kV;
    stream_blocks<G, true>(ks, bl, head_begin, c.q_scale, qb, s_kw, s_vw, rest, ring, vw, do_rest, do_ring,
                           pre != nullptr ? pre[0] : nullptr, pre != nullptr ? pre[1] : nullptr);
    __syncthreads();  // every wave is done with its tiles
    if (do_ring) state_to_lds<G>(ring, so, s_ml, vw);
    if (do_rest) state_to_lds<G>(rest, so_rest, sml_rest, vw);
    __syncthreads();
#pragma unroll
    for (int i = 0; i < kPairs; ++i) {
      const int e = tid + i * (W * 64);
      rg[i][0] = rg[i][1] = 0.0f;
      rg[i][2] = -INFINITY;
      if (e < G * 64) combine_waves<G, kV>(so, s_ml, e >> 6, 2 * (e & 63), rg[i][0], rg[i][1], rg[i][2]);
    }
  }

  const int dest = P % M;
#pragma unroll
  for (int i = 0; i < kPairs; ++i) {
    const int e = tid + i * (W * 64);
    if (e >= G * 64) break;
    const int h = e >> 6, d0 = 2 * (e & 63), hq = hkv * G + h;
    const int64_t ho = static_cast<int64_t>(n) * Hq + hq;
    MergeState st{-INFINITY, {0.0f, 0.0f}};
    float o0, o1, l;
    merge_into(st, rg[i][2], rg[i][0], rg[i][1]);
    merge_into(st, s_entry[h], bf16_lo(ent[i]), bf16_hi(ent[i]));
    if (ready && P >= 0) {  // ring row (a negative past_len has no ring slot)
      const int64_t rowi = (static_cast<int64_t>(req) * M + dest) * Hq + hq;
      const bool valid = isfinite(st.lse);
      *reinterpret_cast<uint32_t*>(c.ring_q + rowi * kHeadDim + d0) = qpre[i];
      *reinterpret_cast<uint32_t*>(c.attn_cache + rowi * kHeadDim + d0) = valid ? pack_bf16x2(st.o[0], st.o[1]) : 0u;
      if (d0 == 0) c.ring_lse[rowi] = valid ? st.lse : -INFINITY;
    }
    combine_waves<G, kV>(so_rest, sml_rest, h, d0, o0, o1, l);
    merge_into(st, l, o0, o1);
    const bool valid = isfinite(st.lse);
    *reinterpret_cast<uint32_t*>(c.out + ho * kHeadDim + d0) = valid ? pack_bf16x2(st.o[0], st.o[1]) : 0u;
    if (c.out_lse != nullptr && d0 == 0) c.out_lse[ho] = valid ? st.lse : -INFINITY;
  }
}

template <int G, int kMode, int W = kWaves>
__global__ void __launch_bounds__(W * 64, W == kWaves ? 2 : 1) match_decide_kernel(DecideParams p) {
  constexpr int kPasses = (G + 3) / 4;
  // 16 row loads in flight per lane with four waves (eight with eight, which
  // cover as many slots per batch)
  constexpr int kSlotBatch = 16 / kPasses * kWaves / W;
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
  // The words the decision reads besides the scan's results -- the readiness
  // gate and the previous step's counts for the short-group rule -- are
  // loaded here, with the scan's round, and used only after the scan.  They
  // are vector loads (`zero` is a vector register the compiler cannot see
  // through) from always-valid addresses, with no branch: a uniform load
  // would be moved to a scalar register at once, and a branch on a pointer
  // would join the loaded value before its use, either of which waits for
  // the load before the scan's loads are issued.
  int zero = 0;
  asm volatile("" : "+v"(zero));
  const bool req_in = req >= 0 && req < p.s.R;
  const int req_c = req_in ? req : 0;
  const bool have_ready = p.cache_ready != nullptr;
  const bool have_epochs = have_ready && p.cache_epoch != nullptr && p.request_epoch != nullptr;
  const bool have_rule = kMode != 1 && p.fuse_sync != nullptr;
  const void* any_valid = p.q_pre;  // (8-byte aligned, at least 32 bytes)
  const uint8_t* ready_at = have_ready ? p.cache_ready + req_c : static_cast<const uint8_t*>(any_valid);
  const int64_t* epoch_c_at = have_epochs ? p.cache_epoch + req_c : static_cast<const int64_t*>(any_valid);
  const int64_t* epoch_r_at = have_epochs ? p.request_epoch + req_c : static_cast<const int64_t*>(any_valid);
  const uint32_t* rule_at = have_rule ? p.fuse_sync : static_cast<const uint32_t*>(any_valid);
  const uint32_t ready_word = ready_at[zero];
  const int64_t epoch_c = epoch_c_at[zero], epoch_r = epoch_r_at[zero];
  uint32_t rule_counts[3];
#pragma unroll
  for (int i = 0; i < 3; ++i) rule_counts[i] = rule_at[i + zero];
  // DECODE:974-981; the readiness gate is applied after the scan
  const int cand_begin = max(0, P - M);
  int cand_end = P;
  if (p.candidate_mode == 1) cand_end = max(cand_begin, P - p.lookback_right);
  const bool cand_ok = P >= p.gen_min_limit && cand_end > cand_begin;

  __shared__ float s_d[W][kMaxGroup];
  __shared__ int s_p[W][kMaxGroup];
  __shared__ int s_s[W][kMaxGroup];
  __shared__ float s_lse[kMaxGroup][kLsePrefetchSlots];  // lse of every slot (small rings)

  // Every load of the scan is independent of the readiness gate and of the
  // other loads (a request id outside [0, R) reads request 0's rows, and the
  // results are masked), so the kernel waits for one round of loads, not a
  // chain.  For rings of at most kLsePrefetchSlots slots the entries' lse
  // are fetched in the same round, so the decision reads them from LDS.
  float best_d[kPasses];
  int best_p[kPasses], best_s[kPasses];
  uint4 qw[kPasses];  // this lane's chunk of its heads' pre-RoPE queries, unpacked where used
#pragma unroll
  for (int ps = 0; ps < kPasses; ++ps) {
    best_d[ps] = INFINITY;
    best_p[ps] = INT_MAX;
    best_s[ps] = -1;
    const int hl = row + 4 * ps;
    qw[ps] = make_uint4(0, 0, 0, 0);
    if (kMode != 2 && hl < G) {
      const int64_t off = (static_cast<int64_t>(n) * Hq + hkv * G + hl) * kHeadDim + c * 8;
      qw[ps] = *reinterpret_cast<const uint4*>(p.q_pre + off);
    }
  }

  if (p.phase_cycles != nullptr && p.stamp_first && g == 0 && tid == 0 && blockIdx.y == 0)
    p.phase_cycles[0] = static_cast<int64_t>(wall_clock64());
  // the post-RoPE query tile of a group this kernel may finish (rows g >= G
  // zero), loaded with the scan's round
  // Loads a group this kernel may finish needs (issued unconditionally and
  // consumed only after the decision, so that no wait for them precedes the
  // scan's loads): the post-RoPE query tile (rows >= G zeroed when stored),
  // the current token's pool row (as two 32-bit words) and the req_to_token
  // entries of this wave's first two sink / tail blocks.
  uint4 qpost_w = make_uint4(0, 0, 0, 0);
  int cur_lo = -1, cur_hi = -1;
  int pre[2][8];
  KvStream ks{};
  if constexpr (kMode != 1) {
    qpost_w = *reinterpret_cast<const uint4*>(
        p.q_post + (static_cast<int64_t>(n) * Hq + hkv * G + min(tid >> 4, G - 1)) * kHeadDim + (tid & 15) * 8);
    const int32_t* ocl = static_cast<const int32_t*>(p.out_cache_loc);
    const int64_t w0 = p.s.out_cache_loc_is_i64 ? 2 * static_cast<int64_t>(n) : n;
    cur_lo = ocl[w0];
    cur_hi = ocl[p.s.out_cache_loc_is_i64 ? w0 + 1 : w0];
    ks = make_stream(p.req_to_token, p.s.r2t_rows, p.s.r2t_stride, req, P, -1, p.s.pool_tokens, p.k_buffer,
                     p.v_buffer, p.s.Hkv, hkv, c);
    // (rest blocks of the wave's virtual wave; an eight-wave workgroup's
    // waves 4..7 stream the band only)
    const BlockList rblk = rest_blocks(P, cache_end_for_pos(P, p.S), p.F);
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      int base, end;
      block_span(rblk, (wave & (kVirtualWaves - 1)) + kVirtualWaves * u, base, end);
#pragma unroll
      for (int i = 0; i < 8; ++i) pre[u][i] = (W == kVirtualWaves || wave < kVirtualWaves) ? ks.raw_row(base + 8 * row + i) : 0;
    }
  }
  const bool req_ok = req >= 0 && req < p.s.R;
  const int64_t cache_req = static_cast<int64_t>(req_ok ? req : 0) * M;
  const bool lse_in_lds = kMode == 0 && M <= kLsePrefetchSlots;
  float lse_reg[G];  // stored to s_lse once the scan's loads are in flight
  if (lse_in_lds && wave == 0 && lane < M) {
#pragma unroll
    for (int hh = 0; hh < G; ++hh) lse_reg[hh] = p.lse_cache[(cache_req + lane) * Hq + hkv * G + hh];
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
    uint4 qaw[kPasses], qbw[kPasses];  // unpacked where used
#pragma unroll
    for (int ps = 0; ps < kPasses; ++ps) {
      const int hl = min(row + 4 * ps, G - 1);
      const uint16_t* qp = p.q_pre + (static_cast<int64_t>(n) * Hq + hkv * G + hl) * kHeadDim + cc * 8;
      qaw[ps] = *reinterpret_cast<const uint4*>(qp);
      qbw[ps] = *reinterpret_cast<const uint4*>(qp + 64);
    }
    const float thr_prune = p.thr_dist + fabsf(p.thr_dist) * 1e-4f + 1e-4f;
    for (int s0 = s_lo + wave; s0 < s_hi; s0 += W * 2 * kProbeBatch) {
      int pos[kProbeBatch], slot[kProbeBatch];
      bool in_window[kProbeBatch];
#pragma unroll
      for (int u = 0; u < kProbeBatch; ++u) {
        slot[u] = s0 + (2 * u + half) * W;
        pos[u] = ring_slot_to_pos(P, M, slot[u]);
        in_window[u] = cand_ok && slot[u] < s_hi && pos[u] >= cand_begin && pos[u] < cand_end;
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
#pragma unroll
      for (int ps = 0; ps < kPasses; ++ps) {
        pin_vgpr(qaw[ps]);
        pin_vgpr(qbw[ps]);
      }
      float acc[kPasses][kProbeBatch];
      bool eval[kPasses][kProbeBatch];
#pragma unroll
      for (int ps = 0; ps < kPasses; ++ps)
#pragma unroll
        for (int u = 0; u < kProbeBatch; ++u) {
          float cf[8], qa[8];
          unpack8(w[ps][u], cf);
          unpack8(qaw[ps], qa);
          float a = 0.0f;
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            const float df = qa[i] - cf[i];
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
          float cf[8], qb[8];
          unpack8(w[ps][u], cf);
          unpack8(qbw[ps], qb);
          float b = acc[ps][u];
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            const float df = qb[i] - cf[i];
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
    // every pass's loads of a batch are in flight before any reduction
    auto scan_batch = [&](int s0) {
      uint4 w[kPasses][kSlotBatch];
      int pos[kSlotBatch];
      bool in_window[kSlotBatch];
#pragma unroll
      for (int u = 0; u < kSlotBatch; ++u) {
        const int slot = s0 + u * W;
        pos[u] = ring_slot_to_pos(P, M, slot);
        in_window[u] = cand_ok && slot < s_hi && pos[u] >= cand_begin && pos[u] < cand_end;
      }
#pragma unroll
      for (int ps = 0; ps < kPasses; ++ps) {
        const int hl = min(row + 4 * ps, G - 1);
#pragma unroll
        for (int u = 0; u < kSlotBatch; ++u) {
          const int slot = min(s0 + u * W, s_hi - 1);  // past the range: re-reads its last row
          const int64_t off = ((cache_req + slot) * Hq + hkv * G + hl) * kHeadDim + c * 8;
          w[ps][u] = load_stream16(p.query_cache + off);  // ring rows are read once per step
        }
      }
      uint4 qv[kPasses];  // unpacked only once the ring loads are issued
#pragma unroll
      for (int ps = 0; ps < kPasses; ++ps) {
        qv[ps] = qw[ps];
        pin_vgpr(qv[ps]);
      }
#pragma unroll
      for (int ps = 0; ps < kPasses; ++ps) {
        const int hl = row + 4 * ps;
#pragma unroll
        for (int u = 0; u < kSlotBatch; ++u) {
          float cf[8], q[8];
          unpack8(w[ps][u], cf);
          unpack8(qv[ps], q);
          float acc = 0.0f;
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            const float df = q[i] - cf[i];
            acc = fmaf(df, df, acc);
          }
          acc = row16_sum(acc);
          if (in_window[u] && hl < G && better_pair(acc, pos[u], best_d[ps], best_p[ps])) {
            best_d[ps] = acc;
            best_p[ps] = pos[u];
            best_s[ps] = s0 + u * W;
          }
        }
      }
    };
    // A ring that one batch per wave covers (32 slots with G = 8, 64 with
    // G <= 4) is scanned without a loop: the queries' unpacking then cannot
    // be hoisted in front of the ring loads, where its wait would hold them.
    if (s_hi - s_lo <= W * kSlotBatch) {
      scan_batch(s_lo + wave);
    } else {
      for (int s0 = s_lo + wave; s0 < s_hi; s0 += W * kSlotBatch) scan_batch(s0);
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
  if (lse_in_lds && wave == 0 && lane < M) {
#pragma unroll
    for (int hh = 0; hh < G; ++hh) s_lse[hh][lane] = lse_reg[hh];
  }
  // DECODE:221-230, request_ready's rule on the words loaded at the start
  const bool ready = req_in && (!have_ready || (ready_word != 0 && (!have_epochs || epoch_c == epoch_r)));
  const bool eligible = cand_ok && ready;
  __syncthreads();
  if (kMode != 1 && p.phase_cycles != nullptr && g == 0 && tid == 0)
    p.phase_cycles[1] = static_cast<int64_t>(wall_clock64());
  __shared__ int s_rect[kMaxGroup], s_mslot[kMaxGroup];
  __shared__ float s_entry[kMaxGroup];
  __shared__ int s_span[3];  // band begin, new_end, fused
  if (wave == 0) decide_group<G, kMode, W>(p, s_d, s_p, s_s, s_lse, lse_in_lds, g, n, hkv, P, req, eligible,
                                        rule_counts, s_rect, s_mslot, s_entry, s_span);
  if constexpr (kMode != 1) {
    __syncthreads();
    if (s_span[2] == 0) return;
    pin_vgpr(cur_lo);  // combined here, not where they are loaded
    pin_vgpr(cur_hi);
    const int64_t cl = p.s.out_cache_loc_is_i64
                           ? static_cast<int64_t>((static_cast<uint64_t>(static_cast<uint32_t>(cur_hi)) << 32) |
                                                  static_cast<uint32_t>(cur_lo))
                           : static_cast<int64_t>(cur_lo);
    ks.cur_row = (cl >= 0 && cl < p.s.pool_tokens) ? static_cast<int>(cl) : -1;
    if ((tid >> 4) >= G) qpost_w = make_uint4(0, 0, 0, 0);
    __shared__ uint4 s_kv[2][W][kTileU4];  // K and V tiles; the combine area afterwards
    __shared__ uint4 s_q[16 * 16];
    __shared__ float s_ml[2][kVirtualWaves][G][2];
    static_assert(sizeof(float) * 2 * kVirtualWaves * G * kOPitch <= sizeof(s_kv), "combine area");
    const ShortCtx sc{p.q_pre, p.ring_q, p.attn_cache, p.ring_lse, p.out, p.out_lse, p.s.Hq, p.s.M, p.s.R, p.F,
                      p.q_scale};
    short_group<G, W, false>(sc, n, hkv, P, req, ready, s_span[0], s_span[1], s_rect, s_mslot, s_entry, qpost_w, ks, pre,
                      &s_kv[0][0][0], s_q, &s_ml[0][0][0][0]);
  }
}

// ========================================================= 2. attention ====

struct GroupSpans {
  int sink_end, band_begin, new_end, kv_len;
  int chunk, n_sink, n_band, n_tail;
  int n_full;  // band pieces of a full chunk (the first ones)
  int piece2;  // length of the band pieces after them
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

// Band pieces: a band of at least kTierChunks full chunks ends in pieces of
// half a chunk (a multiple of 64 tokens) covering its last quarter, when its
// group's pieces still fit `cap` partial slots; other bands are cut into full
// chunks and one shorter remainder.  Span attention fetches the full pieces
// first and the shorter ones after them, so the last tasks of a step are
// short and the workgroups end close together.
constexpr int kTierChunks = 4;

__device__ __forceinline__ void band_layout(GroupSpans& s, int cap) {
  const int len = s.new_end - s.band_begin;
  s.n_full = len / s.chunk;
  s.piece2 = s.chunk;
  s.n_band = ceil_div(len, s.chunk);
  if (s.n_full >= kTierChunks) {
    const int half = ((s.chunk >> 1) + 63) & ~63;
    const int f = (len - len / 4) / s.chunk;
    const int n = f + ceil_div(len - f * s.chunk, half);
    if (s.n_sink + n + s.n_tail <= cap) {
      s.n_full = f;
      s.piece2 = half;
      s.n_band = n;
    }
  }
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
  s.n_tail = ceil_div(s.kv_len - s.new_end, s.chunk);
  band_layout(s, cap);
  return s;
}

// Band pieces of a group that span a full chunk (the first ones).
__device__ __forceinline__ int full_band_pieces(const GroupSpans& s) { return s.n_full; }

// A group of at most fuse_tokens tokens is short: its whole computation is
// short_group, wherever it runs (the same rule as match_decide's).
__device__ __forceinline__ bool group_is_short(const GroupSpans& s, int fuse_tokens) {
  return fuse_tokens > 0 && group_tokens(s.sink_end, s.band_begin, s.new_end, s.kv_len) <= fuse_tokens;
}

// Tasks of a group in class A (full band pieces) and class B (the rest): a
// group match_decide finished has none, a short group one class-B task.
__device__ __forceinline__ void group_task_counts(const GroupSpans& s, bool fused, int fuse_tokens, int& na,
                                                  int& nb) {
  const bool shrt = group_is_short(s, fuse_tokens);
  na = (fused || shrt) ? 0 : full_band_pieces(s);
  nb = fused ? 0 : (shrt ? 1 : s.n_sink + s.n_band + s.n_tail - na);
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
// lookup, Q staging, pipeline fill, partial write) and keeps a long group's
// partials few enough for merge_write to fetch in one or two rounds.
constexpr int kTasksPerWorkgroup = 12;  // default of AttnParams::tasks_per_wg
constexpr int kMinChunk = 3072;
constexpr int kMaxChunk = 16384;
constexpr int kFuseTokens = 1024;  // default of DecideParams::fuse_tokens

// Every workgroup of span_attention derives the same task list: the chunk C
// from the total token count of all groups (kTasksPerWorkgroup tasks per
// workgroup, a multiple of 64 tokens in [kMinChunk, kMaxChunk]), then the
// tasks in two classes, largest first: class A holds the band pieces of full
// chunk length, class B everything shorter (sinks, band remainders, tails,
// and the whole bands of hit groups).  Workgroups fetch A tasks before B
// tasks, so the end of the kernel is filled with short tasks and the idle
// time of the last workgroups is bounded by a short task, not a full chunk.
// s_off[0..NB] holds the exclusive prefix sums of the A counts of buckets of
// plan_bucket consecutive groups (NB buckets; one group per bucket for up to
// kMaxPlanBuckets groups), s_off[NB+1 .. 2NB+1] those of the B counts;
// decode_task finds a task's bucket in the table and its group from the
// bucket's spans.  Workgroup 0 also publishes the chunk and the task count.
__device__ void plan_tasks(const AttnParams& p, int* s_off, int* s_tmp, int& total_tasks_out,
                           int& chunk_out, int& active_wgs_out) {
  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int NG = p.s.N * p.s.Hkv;
  const int gpb = p.plan_bucket;
  const int NB = ceil_div(NG, gpb);  // offset-table entries per class
  const int per_thread = ceil_div(NB, kBlock) * gpb;  // whole buckets per thread
  const int g_lo = min(tid * per_thread, NG);
  const int g_hi = min(g_lo + per_thread, NG);
  // match_decide finished every group: only workgroup 0 stays, to publish
  // the chunk and the task count
  const bool any_long = *p.long_groups != 0;
  if (!any_long && blockIdx.x != 0) {
    total_tasks_out = 0;
    chunk_out = 0;
    active_wgs_out = 0;
    return;
  }
  long long tok = 0;
  for (int g = g_lo; any_long && g < g_hi; ++g) {  // (all four loads in one round)
    const int fused = p.group_fused[g];  // finished by match_decide
    const int ne = p.group_rect_end[g];
    const int t = group_tokens(min(p.F, ne), p.group_rect_begin[g], ne, p.group_tail_end[g]);
    tok += fused != 0 ? 0 : t;
  }
  // reduce token count (64-bit) across the block
  if (any_long) {
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
  if (tok == 0 && blockIdx.x != 0) {  // nothing to attend: only workgroup 0 publishes the counters
    total_tasks_out = 0;
    chunk_out = 0;
    active_wgs_out = 0;
    return;
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
  if (tok == 0) {  // nothing to attend (only workgroup 0 is here): publish an empty plan
    if (tid == 0) {
      p.task_counts[0] = 0;
      p.task_counts[4] = chunk;
    }
    total_tasks_out = 0;
    chunk_out = chunk;
    return;
  }
  // Offset table: entry b of class A (s_off) / class B (s_offb) is the
  // first task of bucket b (groups b gpb .. b gpb + gpb - 1; one group per
  // bucket unless the batch has more groups than the table has entries).
  int* s_offb = s_off + NB + 1;
  int my_a = 0, my_b = 0;
  for (int g = g_lo; tok > 0 && g < g_hi; ++g) {
    GroupSpans sp = load_spans(p.group_rect_begin, p.group_rect_end, p.group_tail_end, g, p.F, chunk, p.cap);
    int na, nb;
    group_task_counts(sp, p.group_fused[g] != 0, p.fuse_tokens, na, nb);
    const int b = g / gpb;
    if (g % gpb == 0) {
      s_off[b] = 0;
      s_offb[b] = 0;
    }
    s_off[b] += na;
    s_offb[b] += nb;
    my_a += na;
    my_b += nb;
  }
  int total_a = 0, total_b = 0;
  int base_a = block_exclusive_scan(my_a, s_tmp, total_a);
  int base_b = block_exclusive_scan(my_b, s_tmp, total_b);
  for (int b = g_lo / gpb; tok > 0 && b * gpb < g_hi; ++b) {
    const int ca = s_off[b], cb = s_offb[b];
    s_off[b] = base_a;
    s_offb[b] = total_a + base_b;
    base_a += ca;
    base_b += cb;
  }
  const int total_tasks = total_a + total_b;
  if (tid == 0) {
    s_off[NB] = total_a;
    s_offb[NB] = total_tasks;
  }
  __syncthreads();

  if (blockIdx.x == 0 && tid == 0) {
    // the plan's chunk, from which merge_write derives every group's chunk,
    // and the task total (the reference's counters [4] and [0]; the others
    // are counted by merge_write's workgroup 0, off this kernel's critical path)
    p.task_counts[0] = total_tasks;
    p.task_counts[4] = chunk;
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
  bool shrt;  // the whole short group (short_group)
  int P, req;
  bool req_ok;
  int64_t cur_loc;
};

// Group, token range [a, b) and kind of task t (sink, band or tail).
__device__ __forceinline__ TaskInfo decode_task(const AttnParams& p, const int* s_off, int NG, int chunk,
                                                int t) {
  TaskInfo ti;
  const int gpb = p.plan_bucket;
  const int NB = ceil_div(NG, gpb);
  const bool class_a = t < s_off[NB];
  const int* off = class_a ? s_off : s_off + NB + 1;
  int lo = 0, hi = NB - 1;  // last bucket b with off[b] <= t
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (off[mid] <= t) lo = mid; else hi = mid - 1;
  }
  // the group of the bucket that holds task t (its earlier groups' counts
  // come from their spans)
  int k = t - off[lo];
  int g = lo * gpb;
  GroupSpans sp = load_spans(p.group_rect_begin, p.group_rect_end, p.group_tail_end, g, p.F, chunk, p.cap);
  for (; g + 1 < min((lo + 1) * gpb, NG); ++g) {
    int na, nb;
    group_task_counts(sp, p.group_fused[g] != 0, p.fuse_tokens, na, nb);
    const int cnt = class_a ? na : nb;
    if (k < cnt) break;
    k -= cnt;
    sp = load_spans(p.group_rect_begin, p.group_rect_end, p.group_tail_end, g + 1, p.F, chunk, p.cap);
  }
  ti.g = g;
  ti.n = g / p.s.Hkv;
  ti.hkv = g - ti.n * p.s.Hkv;
  // piece index j of the group (sink pieces, band pieces, tail pieces), which
  // is also the partial's slot: class A takes the full band pieces, class B
  // the sink pieces, the band remainder and the tail pieces, in that order
  ti.shrt = !class_a && group_is_short(sp, p.fuse_tokens);
  const int na = full_band_pieces(sp);
  if (ti.shrt)
    ti.j = 0;
  else if (class_a)
    ti.j = sp.n_sink + k;
  else if (k < sp.n_sink)
    ti.j = k;
  else
    ti.j = k + na;
  ti.band = false;
  if (ti.shrt) {
    ti.a = sp.band_begin;
    ti.b = sp.new_end;
  } else if (ti.j < sp.n_sink) {
    ti.a = ti.j * sp.chunk;
    ti.b = min(ti.a + sp.chunk, sp.sink_end);
  } else if (ti.j < sp.n_sink + sp.n_band) {
    const int k2 = ti.j - sp.n_sink;  // band piece: n_full of a chunk, then of piece2
    ti.a = k2 < sp.n_full ? sp.band_begin + k2 * sp.chunk
                          : sp.band_begin + sp.n_full * sp.chunk + (k2 - sp.n_full) * sp.piece2;
    ti.b = min(ti.a + (k2 < sp.n_full ? sp.chunk : sp.piece2), sp.new_end);
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

// ------------------------------------------------- MFMA span attention ----
//
// A task is one range of the block stream above (band pieces mask each
// head's positions before its own band start).  The four waves' states are
// combined through LDS into one normalised partial per head.
template <int G>
__device__ __forceinline__ void mfma_task(const AttnParams& p, const TaskInfo& ti, uint4 (*s_kv)[kWaves][kTileU4],
                                          uint4* s_q, float (*s_ml)[G][2]) {
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int col = tid & 15;
  const int n = ti.n, hkv = ti.hkv;
  // Q of the group's heads (rows g >= G zero), staged once per task
  {
    const int64_t qoff = (static_cast<int64_t>(n) * p.s.Hq + hkv * G) * kHeadDim;
    const int g = tid >> 4, c = tid & 15;
    uint4 w = make_uint4(0, 0, 0, 0);
    if (g < G) w = *reinterpret_cast<const uint4*>(p.q_post + qoff + g * kHeadDim + c * 8);
    s_q[tid] = w;
  }
  const int head_begin =
      (ti.band && col < G) ? p.head_rect_start[static_cast<int64_t>(n) * p.s.Hq + hkv * G + col] : 0;
  __syncthreads();
  bf16x8_t qb[4];
  load_q_operands(s_q, qb);
  const KvStream ks = make_stream(p.req_to_token, p.s.r2t_rows, p.s.r2t_stride, ti.req, ti.P, ti.cur_loc,
                                  p.s.pool_tokens, p.k_buffer, p.v_buffer, p.s.Hkv, hkv, col);
  WaveState st, unused;
  state_reset(st);
  stream_blocks<G, false>(ks, one_range(ti.a, ti.b), head_begin, p.q_scale, qb, &s_kv[0][wave][0],
                          &s_kv[1][wave][0], st, unused, wave);
  // ---- wave results -> LDS (over the tiles), then combine the four waves ----
  __syncthreads();  // every wave is done with its tiles
  float* so = reinterpret_cast<float*>(&s_kv[0][0][0]);
  state_to_lds<G>(st, so, &s_ml[0][0][0], wave);
  __syncthreads();
  const int64_t slot = static_cast<int64_t>(ti.g) * p.cap + ti.j;
  for (int e = tid; e < G * 64; e += kBlock) {
    const int h = e >> 6, d0 = 2 * (e & 63);
    float o0, o1, l;
    combine_waves<G>(so, &s_ml[0][0][0], h, d0, o0, o1, l);
    const int64_t oi = static_cast<int64_t>(ti.g) * p.o_group_stride + (static_cast<int64_t>(ti.j) * G + h) * kHeadDim + d0;
    if (p.partial_bf16)
      *reinterpret_cast<uint32_t*>(static_cast<uint16_t*>(p.partial_o) + oi) = pack_bf16x2(o0, o1);
    else
      *reinterpret_cast<float2*>(static_cast<float*>(p.partial_o) + oi) = make_float2(o0, o1);
    if (d0 == 0) p.partial_lse[slot * G + h] = l;
  }
  // next_task's barrier closes the task
}

// A short group left to this kernel: the whole group as one task, computed by
// short_group exactly as match_decide computes the groups it finishes (the
// same four virtual waves, combine and merges), so that where a short group
// runs never changes its results.  Writes out, out_lse and the ring row.
template <int G>
__device__ __forceinline__ void short_task(const AttnParams& p, const TaskInfo& ti, uint4* s_kv, uint4* s_q,
                                           float* s_ml, int* s_rect, int* s_mslot, float* s_entry) {
  const int tid = task_tid();
  const int n = ti.n, hkv = ti.hkv;
  const int Hq = p.s.Hq;
  const bool ready = request_ready(p.cache_ready, p.cache_epoch, p.request_epoch, ti.req, p.R);
  if (tid < G) {
    const int64_t ho = static_cast<int64_t>(n) * Hq + hkv * G + tid;
    const int hit = p.head_hit[ho];
    const int ms = p.head_match_slot[ho];
    const bool reuse = hit != 0 && ms >= 0 && ti.req >= 0 && ti.req < p.R;
    s_rect[tid] = p.head_rect_start[ho];
    s_mslot[tid] = hit != 0 ? ms : -1;
    s_entry[tid] = reuse ? p.lse_cache[(static_cast<int64_t>(ti.req) * p.s.M + ms) * Hq + hkv * G + tid] : -INFINITY;
  }
  uint4 qpost_w = make_uint4(0, 0, 0, 0);
  if ((tid >> 4) < G)
    qpost_w = *reinterpret_cast<const uint4*>(p.q_post + (static_cast<int64_t>(n) * Hq + hkv * G + (tid >> 4)) * kHeadDim +
                                              (tid & 15) * 8);
  const KvStream ks = make_stream(p.req_to_token, p.s.r2t_rows, p.s.r2t_stride, ti.req, ti.P, ti.cur_loc,
                                  p.s.pool_tokens, p.k_buffer, p.v_buffer, p.s.Hkv, hkv, tid & 15);
  const ShortCtx sc{p.q_pre, p.ring_q, p.attn_cache, p.lse_cache, p.out, p.out_lse, Hq, p.s.M, p.R, p.F, p.q_scale};
  __syncthreads();  // s_rect / s_mslot / s_entry
  short_group<G, kVirtualWaves, true>(sc, n, hkv, ti.P, ti.req, ready, ti.a, ti.b, s_rect, s_mslot, s_entry, qpost_w, ks,
                                nullptr, s_kv, s_q, s_ml);
}

template <int G>
__global__ void __launch_bounds__(kBlock, 2) span_attention_mfma_kernel(AttnParams p) {
  extern __shared__ int s_off[];  // 2 (NB + 1) bucket task offsets (dynamic)
  __shared__ int s_tmp[kWaves];
  __shared__ uint4 s_kv[2][kWaves][kTileU4];
  __shared__ uint4 s_q[16 * 16];
  __shared__ float s_ml[2][kWaves][G][2];
  __shared__ int s_rect[kMaxGroup], s_mslot[kMaxGroup];
  __shared__ float s_entry[kMaxGroup];
  static_assert(sizeof(float) * 2 * kWaves * G * kOPitch <= sizeof(s_kv), "combine area");
  static_assert(kWaves == kVirtualWaves, "a short task runs short_group on four waves");

  if (p.phase_cycles != nullptr && blockIdx.x == 0 && threadIdx.x == 0)
    p.phase_cycles[2] = static_cast<int64_t>(wall_clock64());
  const int NG = p.s.N * p.s.Hkv;
  int total_tasks = 0, chunk = 0, active_wgs = 0;
  plan_tasks(p, s_off, s_tmp, total_tasks, chunk, active_wgs);
  if (p.phase_cycles != nullptr && blockIdx.x == 0 && threadIdx.x == 0)
    p.phase_cycles[3] = static_cast<int64_t>(wall_clock64());
  if (static_cast<int>(blockIdx.x) >= active_wgs || total_tasks == 0) return;

  __shared__ int s_task;
  for (int t = next_task(p, s_task); t < total_tasks; t = next_task(p, s_task)) {
    const TaskInfo ti = decode_task(p, s_off, NG, chunk, t);
    if (ti.shrt)
      short_task<G>(p, ti, &s_kv[0][0][0], s_q, &s_ml[0][0][0][0], s_rect, s_mslot, s_entry);
    else
      mfma_task<G>(p, ti, s_kv, s_q, s_ml[0]);
  }
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
// The per-group descriptors (chunk, task, band and tail task counts) and the
// reference's task counters of the step (DECODE:1406-1530), counted by one
// extra workgroup of merge_write, where they overlap that launch instead of
// delaying span_attention's end; also the step's counts for the next step's
// short-group rule (step_fuse_rule) and the cleared long-group flag.
__device__ void publish_counts(const MergeParams& p) {
  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int NG = p.s.N * p.s.Hkv;
  const int chunk = p.task_counts[4];
  if (tid == 0) *p.long_groups = 0;  // read by span_attention, set again by match_decide
  int nonhit = 0, ff = 0, red = 0, max_ff = 0, max_mixed = 0, tails = 0, shorts = 0, longs = 0;
  uint32_t units = 0;  // tokens / 64 of all groups, for the next step's short-group rule
  for (int g = tid; g < NG; g += kBlock) {
    GroupSpans sp = load_spans(p.group_rect_begin, p.group_rect_end, p.group_tail_end, g, p.F, chunk, p.cap);
    const bool fused = p.group_fused[g] != 0;
    const int mode = p.group_mode[g];
    const int t = group_tokens(sp.sink_end, sp.band_begin, sp.new_end, sp.kv_len);
    const bool shrt = p.fuse_tokens > 0 && t <= p.fuse_tokens;
    if (t <= p.fuse_tokens) ++shorts;
    else ++longs;
    units += static_cast<uint32_t>((t + 63) >> 6);
    const int na = (fused || shrt) ? 0 : full_band_pieces(sp);
    const int nb = fused ? 0 : (shrt ? 1 : sp.n_sink + sp.n_band + sp.n_tail - na);
    p.group_chunk_out[g] = sp.chunk;
    p.group_ntasks[g] = na + nb;
    p.group_rect_tiles[g] = sp.n_band;
    p.group_tail_tiles[g] = sp.n_tail;
    if (!fused && !shrt) tails += sp.n_tail;
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
    shorts += __shfl_xor(shorts, off);
    longs += __shfl_xor(longs, off);
    units += __shfl_xor(units, off);
    max_ff = max(max_ff, __shfl_xor(max_ff, off));
    max_mixed = max(max_mixed, __shfl_xor(max_mixed, off));
  }
  __shared__ int s_cnt[kWaves][9];
  if (lane == 0) {
    s_cnt[wave][0] = nonhit;
    s_cnt[wave][1] = ff;
    s_cnt[wave][2] = red;
    s_cnt[wave][3] = tails;
    s_cnt[wave][4] = max_ff;
    s_cnt[wave][5] = max_mixed;
    s_cnt[wave][6] = shorts;
    s_cnt[wave][7] = longs;
    s_cnt[wave][8] = static_cast<int>(units);
  }
  __syncthreads();
  if (tid == 0) {
    int a[6] = {0, 0, 0, 0, 0, 0};
    uint32_t f[3] = {0, 0, 0};
    for (int w = 0; w < kWaves; ++w) {
      for (int i = 0; i < 4; ++i) a[i] += s_cnt[w][i];
      a[4] = max(a[4], s_cnt[w][4]);
      a[5] = max(a[5], s_cnt[w][5]);
      for (int i = 0; i < 3; ++i) f[i] += static_cast<uint32_t>(s_cnt[w][6 + i]);
    }
    if (p.fuse_sync != nullptr) {
      for (int i = 0; i < 3; ++i) p.fuse_sync[i] = f[i];
    }
    p.task_counts[1] = a[3];
    p.task_counts[2] = 0;
    p.task_counts[3] = a[2];
    p.task_counts[5] = a[0];
    p.task_counts[6] = a[1];
    p.task_counts[7] = a[4];
    p.task_counts[8] = a[5];
  }
}

// One workgroup per (group, query head) -- blockIdx.x = group + 1; the
// workgroups of blockIdx.x = 0 count (publish_counts, y = 0) or return.
template <int G>
__global__ void __launch_bounds__(kBlock) merge_write_kernel(MergeParams p) {
  constexpr int kBatch = 8;
  if (blockIdx.x == 0) {
    if (blockIdx.y == 0) publish_counts(p);
    return;
  }
  const int g = blockIdx.x - 1;
  const int h = blockIdx.y;
  const int n = g / p.s.Hkv;
  const int hkv = g - n * p.s.Hkv;
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int d0 = 2 * lane;
  const bool stamp = p.phase_cycles != nullptr && g == 0 && h == 0 && tid == 0;
  if (stamp) p.phase_cycles[4] = static_cast<int64_t>(wall_clock64());
  // the group's descriptors are loaded with its finished flag (one round of
  // loads, not two; a finished group does not use them)
  const int M = p.s.M;
  const int Hq = p.s.Hq;
  const int hq = hkv * G + h;
  const int64_t ho = static_cast<int64_t>(n) * Hq + hq;
  const int fused = p.group_fused[g];
  const int P = p.past_lens[n];
  const int req = p.req_ids[n];
  const int band_begin = p.group_rect_begin[g];
  const int new_end = p.group_rect_end[g];
  const int kv_len = p.group_tail_end[g];
  const int plan_chunk = p.task_counts[4];
  const int hit = p.head_hit[ho];
  const int mslot = p.head_match_slot[ho];
  const int sink_end = min(p.F, new_end);
  const int tokens = group_tokens(sink_end, band_begin, new_end, kv_len);
  const bool shrt = p.fuse_tokens > 0 && tokens <= p.fuse_tokens;
  if (fused != 0 || shrt) {  // finished by match_decide or by a short task
    if (stamp) p.phase_cycles[5] = static_cast<int64_t>(wall_clock64());
    return;
  }
  const int chunk = group_chunk(tokens, plan_chunk, p.cap);  // as span_attention's plan derives it
  const bool ready = request_ready(p.cache_ready, p.cache_epoch, p.request_epoch, req, p.s.R);
  const int dest = P % M;
  // the group's pieces, as span_attention's plan cuts them
  GroupSpans sp;
  sp.sink_end = sink_end;
  sp.band_begin = band_begin;
  sp.new_end = new_end;
  sp.kv_len = kv_len;
  sp.chunk = chunk;
  sp.n_sink = ceil_div(sink_end, chunk);
  sp.n_tail = ceil_div(kv_len - new_end, chunk);
  band_layout(sp, p.cap);
  const int n_sink = sp.n_sink, n_band = sp.n_band, n_tail = sp.n_tail;

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
  if (wave == 0 && hit != 0 && mslot >= 0 && req >= 0 && req < p.s.R) {
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
    const uint32_t packed = valid ? pack2_bf16(ring.o[0], ring.o[1]) : 0u;
    *reinterpret_cast<uint32_t*>(p.attn_cache + rowi * kHeadDim + d0) = packed;
    if (lane == 0) p.lse_cache[rowi] = valid ? ring.lse : -INFINITY;
  }
  merge_into(ring, rest.lse, rest.o[0], rest.o[1]);
  const bool valid = isfinite(ring.lse);
  const uint32_t packed = valid ? pack2_bf16(ring.o[0], ring.o[1]) : 0u;
  *reinterpret_cast<uint32_t*>(p.out + ho * kHeadDim + d0) = packed;
  if (p.out_lse != nullptr && lane == 0) p.out_lse[ho] = valid ? ring.lse : -INFINITY;
  if (stamp) p.phase_cycles[5] = static_cast<int64_t>(wall_clock64());
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

// Tokens up to which match_decide finishes a group itself
// (MAC_AMD_FUSE_TOKENS, read per call like the reference's switches; 0
// sends every group through span_attention and merge_write).  Results do not
// depend on it beyond rounding.
int fuse_tokens() {
  const char* e = std::getenv("MAC_AMD_FUSE_TOKENS");
  const int x = e != nullptr ? std::atoi(e) : kFuseTokens;
  return x < 0 ? 0 : x;
}

template <int G>
void* attn_kernel_ptr() {
  return reinterpret_cast<void*>(&span_attention_mfma_kernel<G>);
}

// Compute units of the device and resident span-attention workgroups per CU
// for a given kernel and dynamic LDS size, cached per process.
std::mutex g_dev_mu;
std::map<std::tuple<int, int, size_t>, int> g_blocks_per_cu;
std::map<int, int> g_cus;

int attn_residency(int dev, int G, size_t dyn_lds, int* cus, int* per_cu) {
  std::lock_guard<std::mutex> lk(g_dev_mu);
  auto ci = g_cus.find(dev);
  if (ci == g_cus.end()) {
    int n = 0;
    MAC_HIP(hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev));
    ci = g_cus.emplace(dev, n).first;
  }
  const auto key = std::make_tuple(dev, G, dyn_lds);
  auto bi = g_blocks_per_cu.find(key);
  if (bi == g_blocks_per_cu.end()) {
    void* fn = nullptr;
    switch (G) {
      case 1: fn = attn_kernel_ptr<1>(); break;
      case 2: fn = attn_kernel_ptr<2>(); break;
      case 3: fn = attn_kernel_ptr<3>(); break;
      case 4: fn = attn_kernel_ptr<4>(); break;
      case 5: fn = attn_kernel_ptr<5>(); break;
      case 6: fn = attn_kernel_ptr<6>(); break;
      case 7: fn = attn_kernel_ptr<7>(); break;
      default: fn = attn_kernel_ptr<8>(); break;
    }
    int blocks = 0;
    MAC_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(&blocks, fn, kBlock, dyn_lds));
    bi = g_blocks_per_cu.emplace(key, blocks > 0 ? blocks : 1).first;
  }
  *cus = ci->second;
  *per_cu = bi->second;
  return MAC_OK;
}

// Waves per match_decide workgroup when a step has at most one group per CU
// (MAC_AMD_MATCH_WAVES, read per call: 8, the default, or 4; the two give the
// same bits: the blocks go to four virtual waves either way).
int match_waves() {
  const char* e = std::getenv("MAC_AMD_MATCH_WAVES");
  return (e != nullptr && std::atoi(e) == 4) ? 4 : 8;
}

// MAC_AMD_FUSE_POLICY (read per call): "auto" (default) applies
// step_fuse_rule; "always" finishes every short group in match_decide.
bool fuse_policy_always() {
  const char* e = std::getenv("MAC_AMD_FUSE_POLICY");
  return e != nullptr && std::strcmp(e, "always") == 0;
}

template <int G>
int launch_all(const DecideParams& dp, const AttnParams& ap, const MergeParams& mp, int attn_grid,
               hipStream_t stream, hipEvent_t* ev) {
  const int NG = dp.s.N * dp.s.Hkv;
  if (ev) MAC_HIP(hipEventRecord(ev[0], stream));
  if (dp.splits > 1) {
    hipLaunchKernelGGL((match_decide_kernel<G, 1>), dim3(NG, dp.splits), dim3(kBlock), 0, stream, dp);
    MAC_HIP(hipGetLastError());
    DecideParams dp2 = dp;
    dp2.stamp_first = 0;  // the range scan recorded the step's start
    hipLaunchKernelGGL((match_decide_kernel<G, 2>), dim3(NG), dim3(kBlock), 0, stream, dp2);
  } else if (NG <= dp.fuse_cus && match_waves() == 8) {
    // at most one group per CU: eight waves per group stream a finished
    // group's blocks in half the rounds
    hipLaunchKernelGGL((match_decide_kernel<G, 0, 8>), dim3(NG), dim3(8 * 64), 0, stream, dp);
  } else {
    hipLaunchKernelGGL((match_decide_kernel<G, 0>), dim3(NG), dim3(kBlock), 0, stream, dp);
  }
  MAC_HIP(hipGetLastError());
  if (ev) MAC_HIP(hipEventRecord(ev[1], stream));
  const size_t plan_lds = 2 * sizeof(int) * (static_cast<size_t>(ceil_div(NG, ap.plan_bucket)) + 1);
  hipLaunchKernelGGL(span_attention_mfma_kernel<G>, dim3(attn_grid), dim3(kBlock), plan_lds, stream, ap);
  MAC_HIP(hipGetLastError());
  if (ev) MAC_HIP(hipEventRecord(ev[2], stream));
  hipLaunchKernelGGL(merge_write_kernel<G>, dim3(NG + 1, G), dim3(kBlock), 0, stream, mp);
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
  MAC_REQUIRE(static_cast<int64_t>(N) * Hkv <= INT_MAX / 2, "N * Hkv = %lld groups is too many",
              static_cast<long long>(N) * Hkv);
  MAC_REQUIRE(a->complete_task_len >= 2 * static_cast<int64_t>(N) * Hkv + kTaskExtra,
              "complete task workspace too small");
  MAC_REQUIRE(a->debug_enabled < 2 || a->phase_cycles == nullptr || a->phase_cycles_len >= 6,
              "phase_cycles must have at least 6 elements");
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
  // the kernels move these with 16-, 8- and 4-byte vector accesses
  auto aligned = [](const void* ptr, uintptr_t n) { return (reinterpret_cast<uintptr_t>(ptr) & (n - 1)) == 0; };
  MAC_REQUIRE(aligned(a->q_post, 16) && aligned(a->q_pre, 16) && aligned(a->k_buffer, 16) &&
                  aligned(a->v_buffer, 16) && aligned(a->query_cache, 16),
              "q_post, q_pre, k_buffer, v_buffer and query_cache must be 16-byte aligned");
  MAC_REQUIRE(aligned(a->attn_cache, 4) && aligned(a->out, 4) && aligned(a->partial_o, 8),
              "attn_cache and out must be 4-byte aligned, partial_o 8-byte aligned");

  hipStream_t stream = static_cast<hipStream_t>(stream_ptr);
  int dev = 0;
  MAC_HIP(hipGetDevice(&dev));
  int cus = 0, per_cu = 0;
  // The planner's LDS table has one entry per bucket of plan_bucket groups
  // (one group per entry up to kMaxPlanBuckets groups).
  const int plan_bucket = ceil_div(N * Hkv, kMaxPlanBuckets);
  const size_t plan_lds = 2 * sizeof(int) * (static_cast<size_t>(ceil_div(N * Hkv, plan_bucket)) + 1);
  int rc = attn_residency(dev, G, plan_lds, &cus, &per_cu);
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
  int64_t* stamps = a->debug_enabled >= 2 ? a->phase_cycles : nullptr;
  dp.fuse_tokens = fuse_tokens();
  dp.group_fused = a->complete_task_go + static_cast<int64_t>(N) * Hkv;
  dp.long_groups = a->complete_task_go + 2 * static_cast<int64_t>(N) * Hkv;
  dp.fuse_sync = (dp.fuse_tokens > 0 && !fuse_policy_always())
                     ? reinterpret_cast<uint32_t*>(a->complete_task_go + 2 * static_cast<int64_t>(N) * Hkv + 2)
                     : nullptr;
  dp.fuse_cus = cus;
  dp.narrow_min_tokens = narrow_min_tokens();
  dp.q_post = static_cast<const uint16_t*>(a->q_post);
  dp.k_buffer = static_cast<const uint16_t*>(a->k_buffer);
  dp.v_buffer = static_cast<const uint16_t*>(a->v_buffer);
  dp.req_to_token = a->req_to_token;
  dp.out_cache_loc = a->out_cache_loc;
  dp.ring_q = static_cast<uint16_t*>(a->query_cache);
  dp.attn_cache = static_cast<uint16_t*>(a->attn_cache);
  dp.ring_lse = a->lse_cache;
  dp.out = static_cast<uint16_t*>(a->out);
  dp.out_lse = a->out_lse;
  dp.q_scale = static_cast<float>(a->sm_scale) * kLog2e;
  dp.phase_cycles = stamps;
  dp.stamp_first = 1;

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
  ap.task_counts = a->task_counts;
  ap.task_counter = dp.task_counter;
  ap.partial_o = a->partial_o;
  ap.partial_lse = a->partial_lse;
  ap.partial_bf16 = a->partial_o_is_bf16 ? 1 : 0;
  ap.o_group_stride = o_group_stride;
  ap.cap = cap;
  ap.F = dp.F;
  ap.q_scale = static_cast<float>(a->sm_scale) * kLog2e;
  ap.tasks_per_wg = tasks_per_wg();
  ap.min_chunk = min_chunk();
  ap.narrow_grid = cus;
  ap.narrow_min_tokens = narrow_min_tokens();
  ap.group_fused = dp.group_fused;
  ap.fuse_tokens = dp.fuse_tokens;
  ap.plan_bucket = plan_bucket;
  ap.long_groups = dp.long_groups;
  ap.phase_cycles = stamps;
  ap.q_pre = dp.q_pre;
  ap.ring_q = dp.ring_q;
  ap.attn_cache = dp.attn_cache;
  ap.lse_cache = a->lse_cache;
  ap.out = dp.out;
  ap.out_lse = dp.out_lse;
  ap.cache_ready = dp.cache_ready;
  ap.cache_epoch = dp.cache_epoch;
  ap.request_epoch = dp.request_epoch;
  ap.head_hit = a->head_hit;
  ap.head_match_slot = a->head_match_slot;
  ap.R = a->R;

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
  mp.partial_o = a->partial_o;
  mp.partial_lse = a->partial_lse;
  mp.partial_bf16 = ap.partial_bf16;
  mp.o_group_stride = o_group_stride;
  mp.cap = cap;
  mp.F = dp.F;
  mp.group_fused = dp.group_fused;
  mp.long_groups = dp.long_groups;
  mp.phase_cycles = stamps;
  mp.fuse_tokens = dp.fuse_tokens;
  mp.group_mode = a->group_mode;
  mp.group_chunk_out = a->complete_task_go;
  mp.group_ntasks = a->complete_task_tile;
  mp.group_rect_tiles = a->group_rect_tiles;
  mp.group_tail_tiles = a->group_tail_tiles;
  mp.task_counts = a->task_counts;
  mp.fuse_sync = const_cast<uint32_t*>(dp.fuse_sync);
  mp.tile_tokens = a->tile_tokens;

  // Persistent grid: what the device keeps resident, but no more workgroups
  // than the largest task count the caller's max_context allows.
  const int NG = N * Hkv;
  const long long max_tokens = static_cast<long long>(a->max_context) + dp.F + 1;
  const long long max_tasks = static_cast<long long>(NG) * ((max_tokens + 63) / 64 + 3);
  long long grid = static_cast<long long>(cus) * per_cu;
  if (grid > max_tasks) grid = max_tasks;
  if (grid < 1) grid = 1;

  switch (G) {
    case 1: return launch_all<1>(dp, ap, mp, static_cast<int>(grid), stream, ev);
    case 2: return launch_all<2>(dp, ap, mp, static_cast<int>(grid), stream, ev);
    case 3: return launch_all<3>(dp, ap, mp, static_cast<int>(grid), stream, ev);
    case 4: return launch_all<4>(dp, ap, mp, static_cast<int>(grid), stream, ev);
    case 5: return launch_all<5>(dp, ap, mp, static_cast<int>(grid), stream, ev);
    case 6: return launch_all<6>(dp, ap, mp, static_cast<int>(grid), stream, ev);
    case 7: return launch_all<7>(dp, ap, mp, static_cast<int>(grid), stream, ev);
    default: return launch_all<8>(dp, ap, mp, static_cast<int>(grid), stream, ev);
  }
}
