/*
 * mac_attention_amd.h -- C ABI of the MI355X (gfx950) MAC-Attention decode
 * library (libmac_hip.so).
 *
 * Every entry point takes plain pointers, sizes and scalars; no framework
 * types cross this boundary.  All device pointers must be device memory of the
 * current HIP device; `stream` is a hipStream_t passed as void* (NULL = the
 * null stream).  No entry point allocates device memory or synchronises the
 * host, so every call may be captured into a hipGraph.
 *
 * Alignment: tensors of 128-element bf16 rows that the kernels move with
 * 16-byte vector accesses (decode: q_post, q_pre, k_buffer, v_buffer,
 * query_cache; window attention: q, k_buffer, v_buffer, out; rectification:
 * those of the window plus src_q, o_full, q_cache, attn_cache,
 * q_post_cache) must start on a 16-byte boundary, the decode step's
 * attn_cache and out on 4 bytes and partial_o on 8; a misaligned pointer is
 * refused with MAC_ERR_INVALID_ARGUMENT.  Framework allocations and row
 * views of them always qualify.
 *
 * Return value: 0 on success, otherwise a MAC_ERR_* code; mac_last_error()
 * then returns a NUL-terminated message for the calling thread.
 *
 * Reference paths are relative to the reference repository root.  "DECODE"
 * stands for attention/src/mac_attention/integrations/sglang/csrc/
 * mac_decode_persistent.cu, "PREFILL" for .../csrc/mac_prefill_update_cache.cu,
 * "MERGE" for .../csrc/mac_merge_downdate_cache.cu, "ROPE" for
 * .../csrc/mac_decode_rope_preserve.cu and "HOOKS" for
 * attention/src/mac_attention/integrations/sglang/flashinfer_hooks.py.
 */
#ifndef MAC_ATTENTION_AMD_H_
#define MAC_ATTENTION_AMD_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MAC_ABI_VERSION 2

#ifndef MAC_API
#if defined(__GNUC__)
#define MAC_API __attribute__((visibility("default")))
#else
#define MAC_API
#endif
#endif

enum {
  MAC_OK = 0,
  MAC_ERR_INVALID_ARGUMENT = 1, /* shape/size/parameter check failed */
  MAC_ERR_HIP = 2,              /* a HIP runtime call failed */
  MAC_ERR_UNSUPPORTED = 3       /* valid input outside what this build supports */
};

/* Group modes written to group_mode (DECODE:41-43). */
enum { MAC_GROUP_MAC_HIT = 0, MAC_GROUP_FULL_FALLBACK = 1, MAC_GROUP_MIXED = 2 };

/*
 * Arguments of one fused MAC decode step.  Field order follows the 68
 * positional arguments of the reference's Python binding
 * mac_persistent_decode_bf16 (DECODE:4962-5030); tensor arguments become a
 * pointer plus the sizes the reference reads from tensor shapes.
 *
 * Tensors (row-major, contiguous):
 *   q_post, q_pre      bf16 [N, Hq, D]        post-/pre-RoPE decode queries
 *   k_buffer, v_buffer bf16 [pool_tokens, Hkv, D]  paged KV pool
 *   req_to_token       i32  [req_to_token_rows, req_to_token_stride]
 *   req_ids, past_lens i32  [>= N]
 *   out_cache_loc      i32 or i64 [>= N] (out_cache_loc_is_i64)
 *   query_cache, attn_cache bf16 [R, M, Hq, D]; lse_cache f32 [R, M, Hq]
 *   out                bf16 [N, Hq, D]; out_lse f32 [N, Hq] or NULL
 * Workspaces (caller-owned, any content on entry):
 *   match_dist f32, match_pos/match_slot i32 [N, Hq, max_match_tiles]
 *   head_* i32 [N, Hq]; group_* i32 [N, Hkv] (leading dimension may exceed N)
 *   complete_task_go/tile i32 [complete_task_len >= 2 N Hkv + 6]
 *   task_counts i32 [>= 9]
 *   partial_o (f32, or bf16 if partial_o_is_bf16) [>= N, Hkv, max_tiles_context, G, D]
 *   partial_lse f32 [>= N, Hkv, max_tiles_context, G]
 * Readiness gate (DECODE:208-230): cache_ready (u8/bool [R]) NULL disables the
 * gate; cache_epoch/request_epoch (i64 [R]) are compared only when both are
 * non-NULL.
 */
typedef struct MacDecodeArgs {
  uint32_t struct_size; /* sizeof(MacDecodeArgs) */
  uint32_t abi_version; /* MAC_ABI_VERSION */

  const void* q_post;
  const void* q_pre;
  const void* k_buffer;
  const void* v_buffer;
  const int32_t* req_to_token;
  const int32_t* req_ids;
  const int32_t* past_lens;
  const void* out_cache_loc;
  void* query_cache;
  void* attn_cache;
  float* lse_cache;
  void* out;
  float* out_lse;

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
  int32_t* group_rect_tiles;
  int32_t* group_tail_begin;
  int32_t* group_tail_end;
  int32_t* group_tail_tiles;
  int32_t* group_mode;
  int32_t* complete_task_go;
  int32_t* complete_task_tile;
  int32_t* task_counts;
  void* partial_o;
  float* partial_lse;

  const uint8_t* cache_ready;
  const int64_t* cache_epoch;
  const int64_t* request_epoch;

  /* shapes */
  int32_t N, Hq, Hkv, D;
  int32_t M, R;
  int64_t pool_tokens;
  int32_t req_to_token_rows, req_to_token_stride;
  int32_t out_cache_loc_is_i64;
  int32_t max_match_tiles;
  int32_t max_tiles_context; /* partial_o / partial_lse dim 2 */
  int32_t partial_o_is_bf16;
  int64_t complete_task_len; /* numel of complete_task_go and complete_task_tile */
  int32_t workspace_rows;    /* leading dim of head_/group_ workspaces (>= N) */

  /* scalar arguments, same meaning as the reference */
  int32_t max_context;
  int32_t tile_tokens;
  int32_t match_tile_slots;
  int32_t semantic_pos_ahead;
  int32_t front_sink_tokens;
  int32_t gen_min_limit;
  int32_t lookback_right;
  int32_t candidate_mode;
  double threshold;
  double sm_scale;
  int32_t debug_enabled;
  int32_t bench_mode;
  double bench_hit_rate;
  double bench_hit_rate_std;
  double bench_skip_ratio;
  double bench_skip_ratio_std;
  double bench_match_lag_mean;
  double bench_match_lag_std;
  int32_t bench_seed;
  int32_t bench_miss_mask;
  int32_t bench_layer_id;
  /* Result-affecting switches the reference reads from the environment:
   * MAC_PERSISTENT_MIXED_GROUP_FALLBACK (DECODE:5229, default 1) and
   * MAC_BENCH_EXACT_QUOTA (DECODE:5334, default 1). */
  int32_t mixed_group_fallback;
  int32_t bench_exact_quota;
  /* The reference's phase_cycles workspace (DECODE:4751-4929), i64
   * [phase_cycles_len >= 6] or NULL.  With debug_enabled >= 2 the step
   * stores s_memrealtime stamps (the 100 MHz device clock, comparable across
   * kernels and compute units) in [0..5]: [0] the step starts, [1] the ring
   * scan of the first group is done, [2] every group is decided (the
   * span-attention kernel starts), [3] its task plan is ready, [4] every
   * span is attended (the merge kernel starts), [5] the first group's merge
   * is written.  Otherwise the array is not touched. */
  int64_t* phase_cycles;
  int32_t phase_cycles_len;
} MacDecodeArgs;

/* Replaces mac_persistent_decode_bf16 (DECODE:4962-5524, pybind DECODE:5526-5529).
 * Writes out/out_lse, one ring row per (request, query head) at past_len % M
 * (skipped for requests failing the readiness gate), and the decision
 * workspaces head_hit ([3] in the reference's workspace list), head_match_pos
 * ([5]), group_mode ([15]) and task_counts ([22]). */
MAC_API int mac_persistent_decode_bf16(const MacDecodeArgs* args, void* stream);

/* The same step for callers that cannot allocate (no reference counterpart)
 * is mac_persistent_decode_bf16_noalloc in libmac_noalloc.so, declared in
 * mac_noalloc.h. */

/* Replaces mac_prefill_update_cache (PREFILL:324-372, pybind PREFILL:500-502).
 * q_cache/attn_cache bf16 [R, M, H, D]; lse_cache f32 [R, M, H];
 * request_length i32 [request_length_len] with request_length_len == R
 * (indexed by request, bumped by lens[b]) or == B (indexed by batch row, not
 * bumped; this form wins when R == B, as in the reference); src_q/src_attn bf16
 * [src_rows, H, D]; src_lse f32 [src_rows, H]; offsets i32 [B+1]; lens i32 [B];
 * q_post_cache bf16 [R, M, H, D] or NULL (rows written get bf16 NaN 0x7fc0). */
MAC_API int mac_prefill_update_cache(void* q_cache, void* attn_cache, float* lse_cache,
                             int32_t* request_length, int32_t request_length_len,
                             const int32_t* req_ids, int32_t B, const void* src_q,
                             const void* src_attn, const float* src_lse, int32_t src_rows,
                             const int32_t* offsets, const int32_t* lens, int32_t R,
                             int32_t capacity, int32_t num_heads, int32_t head_dim,
                             void* q_post_cache, void* stream);

/* Replaces mac_mark_persistent_ready (PREFILL:374-409):
 * cache_epoch[req] = request_epoch[req]; ready[req] = 1 for req in req_ids[0:B]. */
MAC_API int mac_mark_persistent_ready(uint8_t* ready, int64_t* cache_epoch,
                              const int64_t* request_epoch, const int32_t* req_ids, int32_t B,
                              int32_t R, void* stream);

/* Replaces mac_invalidate_persistent_ready (PREFILL:411-446):
 * ready[req] = 0; cache_epoch[req] = -1; request_epoch[req] += 1. */
MAC_API int mac_invalidate_persistent_ready(uint8_t* ready, int64_t* cache_epoch,
                                    int64_t* request_epoch, const int32_t* req_ids, int32_t B,
                                    int32_t R, void* stream);

/* Replaces mac_update_request_state (PREFILL:448-497):
 * cache_lens[i] = max(seq_lens[i] - cur_lens[i], 0); req_len[req] = seq_lens[i];
 * match_req_len[req] = cache_lens[i]. */
MAC_API int mac_update_request_state(int32_t* req_len, int32_t* match_req_len, int32_t* cache_lens,
                             const int32_t* req_ids, const int32_t* seq_lens,
                             const int32_t* cur_lens, int32_t B, int32_t R, void* stream);

/* ------------------------------------------------ prefill rectification --- */

/* Element types of lse tensors for mac_update_then_downdate_bf16_inplace. */
enum { MAC_DTYPE_F32 = 0, MAC_DTYPE_BF16 = 1, MAC_DTYPE_F16 = 2 };

/* Replaces mac_update_then_downdate_bf16_inplace (MERGE:320-401, kernel
 * MERGE:116-288).  out1/out2 bf16 [rows, head_dim]; lse1/lse2 [rows] of type
 * lse1_dtype/lse2_dtype (MAC_DTYPE_*), natural log.  Removes the state
 * (out2, lse2) from the state (out1, lse1) and writes the result into
 * out2/lse2:
 *   |expm1(lse2 - lse1)| <= 1e-7 -> lse2 = -inf, out2 = 0 (nothing left);
 *   lse2 > lse1 otherwise        -> lse2 = lse1, out2 = out1 (no-op);
 *   else r = lse1 + log(max(1 - e^(lse2-lse1) + 1e-7, 1e-30)),
 *        out2 = (out1 - e^(lse2-lse1) out2) e^(lse1 - r), lse2 = r. */
MAC_API int mac_update_then_downdate_bf16_inplace(const void* out1, const void* lse1, int32_t lse1_dtype,
                                                 void* out2, void* lse2, int32_t lse2_dtype,
                                                 int64_t rows, int32_t head_dim, void* stream);

/*
 * Causal sliding-window attention over a ragged batch with a page-size-1 KV
 * pool: the windowed prefill pass the reference runs through FlashInfer's
 * paged prefill wrapper with window_left = semantic_pos_ahead - 1
 * (HOOKS:2436-2466).  Request b owns query rows [qo_indptr[b], qo_indptr[b+1])
 * and keys kv_indices[kv_indptr[b] .. kv_indptr[b+1]); query row i of the
 * request sits at position kv_len - qo_len + i and attends to the keys at
 * positions [pos - window_left, pos] (window_left < 0: [0, pos]).  Requests
 * whose ranges are not within [0, total_q) / [0, kv_indices_len), or with
 * kv_len < qo_len, are skipped (their rows are not written); keys whose pool
 * row is outside [0, pool_tokens) are masked.
 *   q        bf16 [total_q, Hq, 128]
 *   k_buffer, v_buffer bf16 [pool_tokens, Hkv, 128]
 *   out      bf16 [total_q, Hq, 128]
 *   out_lse  f32  [total_q, Hq], NATURAL log (FlashInfer returns log2; the
 *            reference multiplies it by ln 2 right after, HOOKS:2467)
 */
typedef struct MacWindowAttentionArgs {
  uint32_t struct_size; /* sizeof(MacWindowAttentionArgs) */
  uint32_t abi_version; /* MAC_ABI_VERSION */
  const void* q;
  const void* k_buffer;
  const void* v_buffer;
  const int32_t* qo_indptr;  /* [B+1] */
  const int32_t* kv_indptr;  /* [B+1] */
  const int32_t* kv_indices; /* [kv_indptr[B]] pool rows */
  void* out;
  float* out_lse;
  int64_t total_q;
  int64_t pool_tokens;
  int64_t kv_indices_len; /* entries of kv_indices */
  int32_t B, Hq, Hkv, D;
  int32_t window_left;
  double sm_scale;
} MacWindowAttentionArgs;

MAC_API int mac_prefill_window_attention_bf16(const MacWindowAttentionArgs* args, void* stream);

/*
 * Fused prefill rectification + ring update: the composition
 *   window attention (above, window_left = S - 1)
 *   -> mac_update_then_downdate_bf16_inplace(o_full, lse_full, window)
 *   -> mac_prefill_update_cache (offsets = qo_indptr, lens = its differences)
 * of HOOKS:2436-2482, computed only for the rows the ring keeps (the last
 * min(len_b, M) rows of each request; PREFILL:201-269 drops the others).
 * Row i at position p gets the prefix state over [0, E), E = p + 1 - S, as
 * full (o_full, lse_full) minus the window [E, p + 1); E <= 0 gives the empty
 * state (o = 0, lse = -inf) exactly.
 * front_sink_tokens F > 0:
 *   sink_mode 0: as the reference (HOOKS:2205-2215), rows are written with
 *                lse = -inf (never matched; o = full minus window);
 *   sink_mode 1: the sink [0, min(F, E)) is removed as well, giving the state
 *                over [min(F, E), E) that decode-written rows hold
 *                (DECODE:4280-4685), with finite lse.
 *   q_post       bf16 [total_q, Hq, 128]  queries of the attention (post-RoPE)
 *   src_q        bf16 [total_q, Hq, 128]  rows stored as ring queries (pre-RoPE)
 *   o_full       bf16 [total_q, Hq, 128], lse_full f32 [total_q, Hq] (natural log):
 *                full causal prefill attention of the same rows
 *   ring tensors, request_length, req_ids, q_post_cache: as in
 *                mac_prefill_update_cache (request_length read before any bump;
 *                bumped by len_b in the indexed-by-request form).
 */
typedef struct MacRectifyArgs {
  uint32_t struct_size; /* sizeof(MacRectifyArgs) */
  uint32_t abi_version; /* MAC_ABI_VERSION */
  const void* q_post;
  const void* src_q;
  const void* o_full;
  const float* lse_full;
  const void* k_buffer;
  const void* v_buffer;
  const int32_t* qo_indptr;
  const int32_t* kv_indptr;
  const int32_t* kv_indices;
  void* q_cache;
  void* attn_cache;
  float* lse_cache;
  void* q_post_cache; /* NULL allowed */
  int32_t* request_length;
  const int32_t* req_ids;
  int64_t total_q;
  int64_t pool_tokens;
  int64_t kv_indices_len; /* entries of kv_indices */
  int32_t request_length_len;
  int32_t B, R, M, Hq, Hkv, D;
  int32_t semantic_pos_ahead;
  int32_t front_sink_tokens;
  int32_t sink_mode;
  double sm_scale;
} MacRectifyArgs;

MAC_API int mac_prefill_rectify_update_cache_bf16(const MacRectifyArgs* args, void* stream);

/* ------------------------------------------------- decode RoPE + scatter --- */

/* Replaces mac_decode_rope_preserve_q_bf16 (ROPE:174-269, kernel ROPE:36-156).
 * For each decode token n < N (position positions[n], pool row cache_locs[n]):
 * q_pre[n] = q[n] (all head_dim dims, before RoPE); q[n] and k[n] get RoPE on
 * their first rotary_dim dims in place; k_buffer[cache_locs[n]] = RoPE(k[n]);
 * v_buffer[cache_locs[n]] = v[n].  RoPE of pair (x0, x1) with c =
 * cos_sin[pos][i], s = cos_sin[pos][rotary_dim/2 + i] is (x0 c - x1 s,
 * x1 c + x0 s) in fp32 rounded to bf16; pairs are (i, i + rotary_dim/2) when
 * is_neox, else (2i, 2i+1).
 *   q bf16 [N, Hq*head_dim] with row stride q_stride0 (elements), likewise k, v
 *   q_pre bf16 [q_pre_rows >= N, Hq, head_dim]; k_buffer/v_buffer bf16
 *   [pool_tokens, Hkv, head_dim]; cos_sin_cache f32 [cos_sin_rows, >= rotary_dim]
 *   with row stride cos_sin_stride0; positions / cache_locs i32 or i64 [>= N].
 * Positions outside the table are clamped into it and pool rows outside
 * [0, pool_tokens) are not written (the reference does not check either). */
MAC_API int mac_decode_rope_preserve_q_bf16(void* q, int64_t q_stride0, void* k, int64_t k_stride0,
                                            const void* v, int64_t v_stride0, void* q_pre, int64_t q_pre_rows,
                                            void* k_buffer, void* v_buffer, int64_t pool_tokens,
                                            const float* cos_sin_cache, int64_t cos_sin_rows,
                                            int64_t cos_sin_stride0, int32_t rotary_dim, const void* positions,
                                            int32_t positions_is_i64, const void* cache_locs,
                                            int32_t cache_locs_is_i64, int64_t N, int32_t Hq, int32_t Hkv,
                                            int32_t head_dim, int32_t is_neox, void* stream);

/* Message of the last failed call on this thread ("" if none).  No reference
 * counterpart: the reference raises through TORCH_CHECK instead. */
MAC_API const char* mac_last_error(void);

/* ABI version of the loaded library (MAC_ABI_VERSION it was built with).  No
 * reference counterpart. */
MAC_API int mac_abi_version(void);

#ifdef __cplusplus
}
#endif

#endif /* MAC_ATTENTION_AMD_H_ */
