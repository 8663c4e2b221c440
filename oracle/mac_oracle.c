/*
 * mac_oracle.c -- CPU restatement of MAC-Attention's fused decode step and of
 * its ring-cache maintenance ops.
 *
 * TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load this library, and only as the checker
 * (or the timed CPU baseline).  The product path never calls it.
 *
 * Every function cites the reference file:line whose behaviour it restates.
 * Paths are relative to the reference repository root; "DECODE" abbreviates
 * attention/src/mac_attention/integrations/sglang/csrc/mac_decode_persistent.cu
 * and "PREFILL" abbreviates .../csrc/mac_prefill_update_cache.cu.
 *
 * Arithmetic:
 *  - match distances are accumulated in double (exact for bf16 inputs), then
 *    compared against the float32 threshold distance the reference computes
 *    (DECODE:5342);
 *  - span attention and log-sum-exp merges run in double; values that the
 *    reference stores as bf16 (out, attn_cache rows) are rounded to bf16 with
 *    round-to-nearest-even at the same points the reference rounds them.
 *  The GPU kernels accumulate in fp32, so values are compared under a
 *  tolerance and integer decisions exactly (apart from distances that sit
 *  within rounding of the threshold, which the tests report).
 *
 * Parity pins (tests/test_oracle_*.py): every known-answer case of the
 * reference's tests/tools (planted exact matches, wraparound ties, short
 * context, all-miss, mixed groups, front-sink exclusion, two-step recurrence)
 * plus closed forms: exact softmax attention over [0, kv_len) computed by a
 * separate numpy routine, merge associativity, and brute-force ring
 * addressing.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define EXPORT __attribute__((visibility("default")))

enum { MODE_MAC_HIT = 0, MODE_FULL_FALLBACK = 1, MODE_MIXED = 2 };

/* ---------------------------------------------------------------- bf16 --- */

static double bf16_to_d(uint16_t b) {
  uint32_t u = ((uint32_t)b) << 16;
  float f;
  memcpy(&f, &u, 4);
  return (double)f;
}

/* Round-to-nearest-even float -> bf16 (NaN kept quiet). */
static uint16_t f_to_bf16(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x007fffffu)) return (uint16_t)((u >> 16) | 0x40);
  uint32_t lsb = (u >> 16) & 1u;
  u += 0x7fffu + lsb;
  return (uint16_t)(u >> 16);
}

static uint16_t d_to_bf16(double d) { return f_to_bf16((float)d); }

/* --------------------------------------------------- ring addressing ---- */

/* DECODE:798-807 ring_slot_to_pos */
EXPORT int mac_oracle_ring_slot_to_pos(int past_len, int M, int slot) {
  if (past_len < M) return slot;
  int base = past_len - M;
  int tail = past_len % M;
  int order = slot - tail;
  if (order < 0) order += M;
  return base + order;
}

/* DECODE:837-848 pos_to_ring_slot */
EXPORT int mac_oracle_pos_to_ring_slot(int past_len, int M, int pos) {
  if (past_len < M) return pos;
  int base = past_len - M;
  int tail = past_len % M;
  int slot = (pos - base) + tail;
  if (slot >= M) slot -= M;
  if (slot < 0) slot += M;
  return slot;
}

/* DECODE:713-716 cache_end_for_pos */
static int cache_end_for_pos(int p, int S) {
  int e = p + 1 - S;
  return e > 0 ? e : 0;
}

/* ------------------------------------------------ synthetic bench hash -- */

/* DECODE:817-835 mix_u32 / uniform01_u32 / pseudo_normal_u32 */
static uint32_t mix_u32(uint32_t x) {
  x ^= x >> 16;
  x *= 0x7feb352du;
  x ^= x >> 15;
  x *= 0x846ca68bu;
  x ^= x >> 16;
  return x;
}
static float uniform01_u32(uint32_t x) {
  return (float)(mix_u32(x) & 0x00ffffffu) * (1.0f / 16777216.0f);
}
static float pseudo_normal_u32(uint32_t x) {
  float s = uniform01_u32(x) + uniform01_u32(x ^ 0x9e3779b9u) + uniform01_u32(x ^ 0x85ebca6bu) +
            uniform01_u32(x ^ 0xc2b2ae35u);
  return (s - 2.0f) * 1.7320508075688772f;
}
static float clampf_(float v, float lo, float hi) { return fminf(fmaxf(v, lo), hi); }

/* DECODE:375-388 bench_target_miss_units */
static int bench_target_miss_units(float hit_rate, float hit_rate_std, int exact_quota,
                                   int unit_total) {
  if (unit_total <= 0) return 0;
  float miss_rate = 1.0f - hit_rate;
  miss_rate = fminf(fmaxf(miss_rate, 0.0f), 1.0f);
  int miss;
  if (exact_quota && hit_rate_std == 0.0f)
    miss = (int)floorf(miss_rate * (float)unit_total + 0.5f);
  else
    miss = (int)ceilf(miss_rate * (float)unit_total);
  if (miss < 0) miss = 0;
  if (miss > unit_total) miss = unit_total;
  return miss;
}

/* ------------------------------------------------------------- args ---- */

typedef struct {
  /* shapes */
  int N, Hq, Hkv, D, M, R, req_to_token_stride;
  /* inputs (bf16 as raw uint16) */
  const uint16_t* q_post;   /* [N,Hq,D] */
  const uint16_t* q_pre;    /* [N,Hq,D] */
  const uint16_t* k_buffer; /* [pool,Hkv,D] */
  const uint16_t* v_buffer; /* [pool,Hkv,D] */
  const int32_t* req_to_token;
  const int32_t* req_ids;
  const int32_t* past_lens;
  const int64_t* out_cache_loc; /* widened to int64 by the wrapper */
  /* ring caches (updated in place) */
  uint16_t* query_cache; /* [R,M,Hq,D] */
  uint16_t* attn_cache;  /* [R,M,Hq,D] */
  float* lse_cache;      /* [R,M,Hq] */
  /* readiness gate (NULL = every request ready) */
  const uint8_t* cache_ready;
  const int64_t* cache_epoch;
  const int64_t* request_epoch;
  /* outputs */
  uint16_t* out;   /* [N,Hq,D] */
  float* out_lse;  /* [N,Hq] or NULL */
  /* decision outputs, [N,Hq] */
  int32_t* head_hit;
  int32_t* head_match_slot;
  int32_t* head_match_pos;
  int32_t* head_prefix_end;
  int32_t* head_rect_start;
  int32_t* head_new_end;
  double* head_best_dist; /* best distance of the scan (before any override), inf if none */
  /* decision outputs, [N,Hkv] */
  int32_t* group_mode;
  int32_t* group_rect_begin;
  int32_t* group_rect_end;
  int32_t* group_tail_begin;
  int32_t* group_tail_end;
  /* scalars */
  int semantic_pos_ahead, front_sink_tokens, gen_min_limit, lookback_right, candidate_mode;
  float threshold, sm_scale;
  int mixed_group_fallback;
  int bench_mode, bench_exact_quota, bench_seed, bench_miss_mask, bench_layer_id;
  float bench_hit_rate, bench_hit_rate_std, bench_skip_ratio, bench_skip_ratio_std;
  float bench_match_lag_mean, bench_match_lag_std;
} MacOracleDecodeArgs;

/* DECODE:221-230 request_persistent_ready */
static int request_ready(const MacOracleDecodeArgs* a, int req) {
  if (a->cache_ready == NULL) return 1;
  if (req < 0 || req >= a->R) return 0;
  if (a->cache_ready[req] == 0) return 0;
  if (a->cache_epoch != NULL && a->request_epoch != NULL &&
      a->cache_epoch[req] != a->request_epoch[req])
    return 0;
  return 1;
}

/* --------------------------------------------------- span attention ---- */

typedef struct {
  double o[128];
  double lse; /* -inf == empty */
} State;

static void state_empty(State* s, int D) {
  for (int i = 0; i < D; ++i) s->o[i] = 0.0;
  s->lse = -INFINITY;
}

/* DECODE:866-890 merge_scalar, tests/test_mac_persistent_decode.py:31-51 _merge:
 * an invalid (non-finite) other is skipped; an invalid state takes other. */
static void state_merge(State* s, const State* o, int D) {
  if (!isfinite(o->lse)) return;
  if (!isfinite(s->lse)) {
    *s = *o;
    return;
  }
  double m = s->lse > o->lse ? s->lse : o->lse;
  double w1 = exp(s->lse - m), w2 = exp(o->lse - m);
  double den = w1 + w2;
  for (int i = 0; i < D; ++i) s->o[i] = (w1 * s->o[i] + w2 * o->o[i]) / den;
  s->lse = m + log(den);
}

/* DECODE:850-864 physical_token */
static int64_t physical_token(const MacOracleDecodeArgs* a, int n, int req, int pos, int past_len) {
  if (pos == past_len) return a->out_cache_loc[n];
  return (int64_t)a->req_to_token[(int64_t)req * a->req_to_token_stride + pos];
}

/* Exact softmax attention of one query head over logical positions [b, e)
 * (tests/test_mac_persistent_decode.py:9-28 _ref_attention; the kernel's
 * producers DECODE:1870-3423 compute the same quantity tile by tile). */
static void span_attention(const MacOracleDecodeArgs* a, int n, int req, int past_len, int hq,
                           int b, int e, State* st, double* logits_scratch) {
  const int D = a->D;
  state_empty(st, D);
  if (e <= b) return;
  const int G = a->Hq / a->Hkv;
  const int hkv = hq / G;
  const uint16_t* q = a->q_post + ((int64_t)n * a->Hq + hq) * D;
  double qd[128];
  for (int i = 0; i < D; ++i) qd[i] = bf16_to_d(q[i]);
  double m = -INFINITY;
  for (int pos = b; pos < e; ++pos) {
    int64_t phys = physical_token(a, n, req, pos, past_len);
    const uint16_t* kr = a->k_buffer + (phys * a->Hkv + hkv) * D;
    double dot = 0.0;
    for (int i = 0; i < D; ++i) dot += qd[i] * bf16_to_d(kr[i]);
    double s = dot * (double)a->sm_scale;
    logits_scratch[pos - b] = s;
    if (s > m) m = s;
  }
  double den = 0.0;
  for (int pos = b; pos < e; ++pos) {
    double w = exp(logits_scratch[pos - b] - m);
    logits_scratch[pos - b] = w;
    den += w;
  }
  for (int pos = b; pos < e; ++pos) {
    int64_t phys = physical_token(a, n, req, pos, past_len);
    const uint16_t* vr = a->v_buffer + (phys * a->Hkv + hkv) * D;
    double w = logits_scratch[pos - b] / den;
    for (int i = 0; i < D; ++i) st->o[i] += w * bf16_to_d(vr[i]);
  }
  st->lse = m + log(den);
}

/* ------------------------------------------------------ decode step ---- */

/*
 * One decode step: match scan (DECODE:942-1099, tile reduce :1147-1174),
 * per-head decisions (:1175-1299), group modes and spans (:1305-1402),
 * span attention, merge + ring write (:4280-4685).
 *
 * Returns 0 on success, a negative code on bad arguments.
 */
EXPORT int mac_oracle_decode(const MacOracleDecodeArgs* a) {
  const int N = a->N, Hq = a->Hq, Hkv = a->Hkv, D = a->D, M = a->M;
  if (N < 0 || Hkv <= 0 || Hq % Hkv != 0 || D <= 0 || D > 128 || M <= 0) return -1;
  const int G = Hq / Hkv;
  const int S = a->semantic_pos_ahead;
  const int F = a->front_sink_tokens > 0 ? a->front_sink_tokens : 0;
  /* DECODE:5342 threshold distance, float32 arithmetic */
  const float thr_dist = 2.0f * (float)D * (1.0f - a->threshold) * (1.0f - a->threshold);

  /* All ring reads see the caches as they were at entry; writes are applied at
   * the end (each (req, dest_slot, hq) row is written by exactly one head). */
  const size_t ring_rows = (size_t)a->R * M * Hq;
  uint16_t* qc0 = (uint16_t*)malloc(ring_rows * D * 2);
  uint16_t* ac0 = (uint16_t*)malloc(ring_rows * D * 2);
  float* lc0 = (float*)malloc(ring_rows * 4);
  int max_past = 0;
  for (int n = 0; n < N; ++n)
    if (a->past_lens[n] > max_past) max_past = a->past_lens[n];
  double* scratch = (double*)malloc(sizeof(double) * ((size_t)max_past + 2 + (S < 0 ? -S : 0)));
  State* st = (State*)malloc(sizeof(State));
  State* tmp = (State*)malloc(sizeof(State));
  if (!qc0 || !ac0 || !lc0 || !scratch || !st || !tmp) {
    free(qc0); free(ac0); free(lc0); free(scratch); free(st); free(tmp);
    return -2;
  }
  memcpy(qc0, a->query_cache, ring_rows * D * 2);
  memcpy(ac0, a->attn_cache, ring_rows * D * 2);
  memcpy(lc0, a->lse_cache, ring_rows * 4);

  for (int n = 0; n < N; ++n) {
    const int P = a->past_lens[n];
    const int kv_len = P + 1;
    const int req = a->req_ids[n];
    const int ready = request_ready(a, req);
    /* DECODE:974-981 candidate window and eligibility */
    const int cand_begin = P - M > 0 ? P - M : 0;
    int cand_end = P;
    if (a->candidate_mode == 1) {
      cand_end = P - a->lookback_right;
      if (cand_end < cand_begin) cand_end = cand_begin;
    }
    const int eligible = P >= a->gen_min_limit && cand_end > cand_begin && ready;
    const int new_end = cache_end_for_pos(P, S);
    int fs_begin = F < new_end ? F : new_end; /* DECODE:719-724 clamp_front_sink_end */

    for (int hq = 0; hq < Hq; ++hq) {
      /* ---- match scan: squared L2 over the candidate slots ---- */
      double best_d = INFINITY;
      int best_p = INT32_MAX, best_s = -1;
      if (eligible) {
        const uint16_t* qp = a->q_pre + ((int64_t)n * Hq + hq) * D;
        for (int slot = 0; slot < M; ++slot) {
          int pos = mac_oracle_ring_slot_to_pos(P, M, slot);
          if (pos < cand_begin || pos >= cand_end) continue;
          const uint16_t* cr = qc0 + (((int64_t)req * M + slot) * Hq + hq) * D;
          double d = 0.0;
          for (int i = 0; i < D; ++i) {
            double df = bf16_to_d(qp[i]) - bf16_to_d(cr[i]);
            d += df * df;
          }
          /* DECODE:809-811 better_pair: smaller distance, tie -> smaller pos */
          if (d < best_d || (d == best_d && pos < best_p)) {
            best_d = d;
            best_p = pos;
            best_s = slot;
          }
        }
      }
      const int64_t ho = (int64_t)n * Hq + hq;
      if (a->head_best_dist) a->head_best_dist[ho] = best_d;
      int hit = eligible && best_s >= 0 && best_d < (double)thr_dist;

      /* ---- synthetic bench override, DECODE:1184-1269 ---- */
      if (a->bench_mode != 0 || a->bench_miss_mask >= 0) {
        int hkv = hq / G;
        int lane_i = hq - hkv * G;
        uint32_t unit_id = a->bench_mode == 2 ? (uint32_t)hkv : (uint32_t)hq;
        uint32_t base_key = (uint32_t)a->bench_seed ^ ((uint32_t)a->bench_layer_id * 0x9e3779b9u) ^
                            ((uint32_t)P * 0x85ebca6bu);
        uint32_t key = base_key ^ ((uint32_t)n * 0xc2b2ae35u) ^ (unit_id * 0x27d4eb2fu);
        float hit_rate = clampf_(
            a->bench_hit_rate + a->bench_hit_rate_std * pseudo_normal_u32(key ^ 0x4cf5ad43u), 0.0f,
            1.0f);
        if (a->bench_miss_mask >= 0) {
          int synth_miss = lane_i >= 0 && lane_i < 30 && ((a->bench_miss_mask >> lane_i) & 1);
          hit = eligible && P > 0 && M > 0 && !synth_miss;
        } else if (a->bench_exact_quota && a->bench_hit_rate_std == 0.0f) {
          int unit_total = a->bench_mode == 2 ? N * Hkv : N * Hq;
          int unit = a->bench_mode == 2 ? n * Hkv + hkv : n * Hq + hq;
          int miss_units = bench_target_miss_units(a->bench_hit_rate, a->bench_hit_rate_std,
                                                   a->bench_exact_quota, unit_total);
          int offset = unit_total > 0 ? (int)(base_key % (uint32_t)unit_total) : 0;
          int rotated = unit + offset;
          if (rotated >= unit_total) rotated -= unit_total;
          hit = eligible && P > 0 && M > 0 && !(rotated < miss_units);
        } else {
          hit = eligible && P > 0 && M > 0 && uniform01_u32(key ^ 0x165667b1u) < hit_rate;
        }
        if (hit) {
          int max_lag = M < P ? M : P;
          int ne = cache_end_for_pos(P, S);
          float lag_f = a->bench_match_lag_mean +
                        a->bench_match_lag_std * pseudo_normal_u32(key ^ 0xd3a2646cu);
          int req_skip = 0;
          if (a->bench_skip_ratio >= 0.0f) {
            req_skip = 1;
            float sr = clampf_(a->bench_skip_ratio +
                                   a->bench_skip_ratio_std * pseudo_normal_u32(key ^ 0xfd7046c5u),
                               0.0f, 0.999999f);
            int tpe = (int)roundf(sr * (float)P);
            if (tpe > ne - 1) tpe = ne - 1;
            if (tpe < 0) tpe = 0;
            lag_f = (float)(ne - tpe);
          }
          int lag = (int)roundf(lag_f);
          if (lag < 1) lag = 1;
          if (req_skip) {
            if (lag > P) lag = P;
          } else if (lag > max_lag) {
            lag = max_lag;
          }
          if (max_lag <= 0 || ne <= 0) {
            hit = 0;
            best_p = INT32_MAX;
            best_s = -1;
          } else {
            best_p = P - lag;
            if (best_p < 0) best_p = 0;
            best_s = mac_oracle_pos_to_ring_slot(P, M, best_p);
            best_d = 0.0;
          }
        } else {
          best_p = INT32_MAX;
          best_s = -1;
          best_d = INFINITY;
        }
      }

      /* ---- per-head span decision, DECODE:1270-1299 ---- */
      int prefix_end = 0, rect_start = 0, mpos = -1, mslot = -1;
      if (hit) {
        mpos = best_p;
        mslot = best_s;
        prefix_end = cache_end_for_pos(mpos, S);
        rect_start = prefix_end;
      }
      if (hit && F > 0 && prefix_end < F) { /* front-sink demotion */
        hit = 0;
        mpos = mslot = -1;
        prefix_end = rect_start = 0;
      }
      a->head_hit[ho] = hit;
      a->head_match_slot[ho] = mslot;
      a->head_match_pos[ho] = mpos;
      a->head_prefix_end[ho] = prefix_end;
      a->head_rect_start[ho] = rect_start;
      a->head_new_end[ho] = new_end;
    }

    /* ---- group validity, mode and spans, DECODE:1305-1402 ---- */
    for (int hkv = 0; hkv < Hkv; ++hkv) {
      int valid_count = 0, complete_begin = INT32_MAX;
      int valid[64];
      for (int li = 0; li < G; ++li) {
        int hq = hkv * G + li;
        int64_t ho = (int64_t)n * Hq + hq;
        int slot = a->head_match_slot[ho];
        int v = a->head_hit[ho] != 0 && slot >= 0 && a->head_new_end[ho] == new_end;
        int clen = a->head_new_end[ho] - a->head_rect_start[ho];
        if (v) {
          float pl = lc0[((int64_t)req * M + slot) * Hq + hq];
          v = isfinite(pl) && clen >= 0 && clen <= M;
        }
        valid[li] = v;
        if (v) {
          ++valid_count;
          if (a->head_rect_start[ho] < complete_begin) complete_begin = a->head_rect_start[ho];
        }
      }
      int mode = MODE_FULL_FALLBACK;
      if (valid_count == G)
        mode = MODE_MAC_HIT;
      else if (valid_count > 0 && a->mixed_group_fallback)
        mode = MODE_MIXED;
      if (mode != MODE_MAC_HIT) {
        complete_begin = fs_begin;
        for (int li = 0; li < G; ++li) {
          if (mode == MODE_MIXED && valid[li]) continue;
          int64_t ho = (int64_t)n * Hq + hkv * G + li;
          a->head_hit[ho] = 0;
          a->head_match_slot[ho] = -1;
          a->head_match_pos[ho] = -1;
          a->head_prefix_end[ho] = 0;
          a->head_rect_start[ho] = fs_begin;
          a->head_new_end[ho] = new_end;
        }
      }
      if (complete_begin > new_end) complete_begin = new_end;
      if (complete_begin < 0) complete_begin = 0;
      int64_t go = (int64_t)n * Hkv + hkv;
      a->group_mode[go] = mode;
      a->group_rect_begin[go] = complete_begin;
      a->group_rect_end[go] = new_end;
      a->group_tail_begin[go] = new_end;
      a->group_tail_end[go] = kv_len;
    }

    /* ---- span attention, merge, ring write, DECODE:4280-4685 ---- */
    const int dest = P % M;
    for (int hq = 0; hq < Hq; ++hq) {
      int64_t ho = (int64_t)n * Hq + hq;
      int hit = a->head_hit[ho];
      int mslot = a->head_match_slot[ho];
      int hb = a->head_rect_start[ho], he = a->head_new_end[ho];
      state_empty(st, D);
      if (hit && mslot >= 0) {
        int64_t row = ((int64_t)req * M + mslot) * Hq + hq;
        float pl = lc0[row];
        if (isfinite(pl)) {
          for (int i = 0; i < D; ++i) st->o[i] = bf16_to_d(ac0[row * D + i]);
          st->lse = (double)pl;
        }
      }
      /* band [head_rect_start, new_end) joins the stored state */
      span_attention(a, n, req, P, hq, hb, he, tmp, scratch);
      state_merge(st, tmp, D);
      if (ready) {
        int64_t row = ((int64_t)req * M + dest) * Hq + hq;
        const uint16_t* qp = a->q_pre + ho * D;
        int valid = isfinite(st->lse);
        for (int i = 0; i < D; ++i) {
          a->query_cache[row * D + i] = qp[i];
          a->attn_cache[row * D + i] = valid ? d_to_bf16(st->o[i]) : 0;
        }
        a->lse_cache[row] = valid ? (float)st->lse : -INFINITY;
      }
      /* sink [0, min(F, head_rect_start, new_end)) is output-only (DECODE:726-731) */
      int sink_end = F < he ? F : he;
      if (sink_end > hb) sink_end = hb;
      if (sink_end < 0) sink_end = 0;
      span_attention(a, n, req, P, hq, 0, sink_end, tmp, scratch);
      state_merge(st, tmp, D);
      /* tail [new_end, kv_len) */
      span_attention(a, n, req, P, hq, new_end, kv_len, tmp, scratch);
      state_merge(st, tmp, D);
      int valid = isfinite(st->lse);
      for (int i = 0; i < D; ++i) a->out[ho * D + i] = valid ? d_to_bf16(st->o[i]) : 0;
      if (a->out_lse) a->out_lse[ho] = valid ? (float)st->lse : -INFINITY;
    }
  }
  free(qc0);
  free(ac0);
  free(lc0);
  free(scratch);
  free(st);
  free(tmp);
  return 0;
}

/* Exact attention of one head over [b, e) for the tests' closed-form checks:
 * writes o (double[D]) and returns lse. */
EXPORT double mac_oracle_span_attention(const MacOracleDecodeArgs* a, int n, int hq, int b, int e,
                                        double* o_out) {
  State* s = (State*)malloc(sizeof(State));
  int P = a->past_lens[n];
  int len = e > b ? e - b : 1;
  double* scratch = (double*)malloc(sizeof(double) * (size_t)len);
  span_attention(a, n, a->req_ids[n], P, hq, b, e, s, scratch);
  for (int i = 0; i < a->D; ++i) o_out[i] = s->o[i];
  double l = s->lse;
  free(s);
  free(scratch);
  return l;
}

/* ------------------------------------------- ring-cache maintenance ---- */

/*
 * PREFILL:201-269 mac_prefill_update_cache_kernel.  For each batch row b with
 * Ni = lens[b] > 0: keep the last min(Ni, M) rows of the source range starting
 * at offsets[b], writing row i of the kept range to slot (L_before+start+i)%M.
 * L_before = request_length[b] when request_length has one entry per batch row
 * (then it is not bumped), else request_length[req] (bumped by Ni).
 * q_post_cache rows (if given) are filled with the bf16 NaN 0x7fc0.
 */
EXPORT int mac_oracle_prefill_update_cache(uint16_t* q_cache, uint16_t* attn_cache,
                                           float* lse_cache, int32_t* request_length,
                                           int request_length_len, const int32_t* req_ids, int B,
                                           const uint16_t* src_q, const uint16_t* src_attn,
                                           const float* src_lse, int src_rows,
                                           const int32_t* offsets, const int32_t* lens, int R,
                                           int M, int H, int D, uint16_t* q_post_cache) {
  if (M <= 0 || B == 0) return 0;
  const int by_batch = request_length_len == B;
  const size_t row = (size_t)H * D;
  /* all reads of request_length happen before any bump (the GPU kernel's
   * blocks read theirs concurrently with the single-thread bump at the end). */
  int32_t* before = (int32_t*)malloc(sizeof(int32_t) * (size_t)B);
  for (int b = 0; b < B; ++b) {
    int req = req_ids[b];
    before[b] = 0;
    if (by_batch)
      before[b] = request_length[b];
    else if (req >= 0 && req < R)
      before[b] = request_length[req];
  }
  for (int b = 0; b < B; ++b) {
    int req = req_ids[b];
    int Ni = lens[b];
    if (Ni <= 0) continue;
    if (req < 0 || req >= R) continue;
    int start = Ni > M ? Ni - M : 0;
    int keep = Ni - start;
    int base_off = offsets[b];
    if (base_off < 0 || base_off + Ni > src_rows) continue;
    int L = before[b] < 0 ? 0 : before[b];
    int base_dest = (int)(((int64_t)L + start) % M);
    for (int i = 0; i < keep; ++i) {
      int dst = base_dest + i;
      if (dst >= M) dst -= M;
      size_t drow = (size_t)req * M + dst;
      size_t srow = (size_t)base_off + start + i;
      memcpy(q_cache + drow * row, src_q + srow * row, row * 2);
      memcpy(attn_cache + drow * row, src_attn + srow * row, row * 2);
      memcpy(lse_cache + drow * H, src_lse + srow * H, (size_t)H * 4);
      if (q_post_cache)
        for (size_t j = 0; j < row; ++j) q_post_cache[drow * row + j] = 0x7fc0;
    }
    if (!by_batch) request_length[req] += Ni;
  }
  free(before);
  return 0;
}

/* PREFILL:271-283 */
EXPORT void mac_oracle_mark_ready(uint8_t* ready, int64_t* cache_epoch,
                                  const int64_t* request_epoch, const int32_t* req_ids, int B,
                                  int R) {
  for (int i = 0; i < B; ++i) {
    int req = req_ids[i];
    if (req < 0 || req >= R) continue;
    cache_epoch[req] = request_epoch[req];
    ready[req] = 1;
  }
}

/* PREFILL:285-298 */
EXPORT void mac_oracle_invalidate_ready(uint8_t* ready, int64_t* cache_epoch,
                                        int64_t* request_epoch, const int32_t* req_ids, int B,
                                        int R) {
  for (int i = 0; i < B; ++i) {
    int req = req_ids[i];
    if (req < 0 || req >= R) continue;
    ready[req] = 0;
    cache_epoch[req] = -1;
    request_epoch[req] += 1;
  }
}

/* PREFILL:300-320 */
EXPORT void mac_oracle_update_request_state(int32_t* req_len, int32_t* match_req_len,
                                            int32_t* cache_lens, const int32_t* req_ids,
                                            const int32_t* seq_lens, const int32_t* cur_lens,
                                            int B, int R) {
  for (int i = 0; i < B; ++i) {
    int32_t c = seq_lens[i] - cur_lens[i];
    if (c < 0) c = 0;
    cache_lens[i] = c;
    int req = req_ids[i];
    if (req < 0 || req >= R) continue;
    req_len[req] = seq_lens[i];
    match_req_len[req] = c;
  }
}

/* ------------------------------------------- prefill rectification ---- */

static float lse_in(const void* p, int dtype, int64_t i) {
  if (dtype == 0) return ((const float*)p)[i];
  uint16_t b = ((const uint16_t*)p)[i];
  if (dtype == 1) return (float)bf16_to_d(b);
  /* IEEE half */
  uint32_t s = (uint32_t)(b >> 15), e = (uint32_t)((b >> 10) & 31), m = (uint32_t)(b & 1023);
  float v;
  if (e == 0) v = ldexpf((float)m, -24);
  else if (e == 31) v = m ? NAN : INFINITY;
  else v = ldexpf((float)(m | 1024), (int)e - 25);
  return s ? -v : v;
}

static uint16_t f_to_half(float f) {
  /* round to nearest even via float arithmetic on the scaled mantissa */
  uint32_t u;
  memcpy(&u, &f, 4);
  uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
  float a = fabsf(f);
  if (isnan(f)) return (uint16_t)(sign | 0x7e00u);
  if (a >= 65520.0f) return (uint16_t)(sign | 0x7c00u);
  if (a < ldexpf(1.0f, -14)) { /* subnormal: multiple of 2^-24 */
    float q = nearbyintf(ldexpf(a, 24));
    return (uint16_t)(sign | (uint16_t)q);
  }
  int ex;
  float fr = frexpf(a, &ex); /* a = fr * 2^ex, fr in [0.5, 1) */
  float mant = nearbyintf(ldexpf(fr, 11)); /* 11 significant bits */
  if (mant >= 2048.0f) { mant = 1024.0f; ex += 1; }
  int he = ex - 1 + 15;
  if (he >= 31) return (uint16_t)(sign | 0x7c00u);
  return (uint16_t)(sign | (uint16_t)(he << 10) | ((uint16_t)mant - 1024u));
}

static void lse_out(void* p, int dtype, int64_t i, float v) {
  if (dtype == 0) ((float*)p)[i] = v;
  else if (dtype == 1) ((uint16_t*)p)[i] = f_to_bf16(v);
  else ((uint16_t*)p)[i] = f_to_half(v);
}

/* Downdate control of MERGE:148-176: returns 0 = nothing left, 1 = no-op
 * (keep state 1), 2 = regular, with t = e^(l2-l1) and r the new lse.  The
 * branch tests run in float32 as in the reference so that decisions match. */
static int downdate_control(float l1, float l2, double* t, double* r) {
  float diff = l2 - l1;
  float em1 = expm1f(diff);
  int last_block = fabsf(em1) <= 1e-7f;
  int invalid = (diff > 0.0f) && !last_block;
  if (last_block) return 0;
  if (invalid) return 1;
  double dd = (double)l2 - (double)l1;
  double one_minus = 1.0 - exp(dd);
  double x = one_minus + 1e-7;
  if (x < 1e-30) x = 1e-30;
  *r = (double)l1 + log(x);
  *t = exp(dd);
  return 2;
}

/*
 * MERGE:116-288 (kernel) and MERGE:320-401 (binding): in-place downdate of
 * (out2, lse2) from (out1, lse1), rows x D, bf16 outputs, lse of dtype codes
 * 0 = f32, 1 = bf16, 2 = f16.
 */
EXPORT void mac_oracle_update_then_downdate(const uint16_t* out1, const void* lse1, int lse1_dtype,
                                            uint16_t* out2, void* lse2, int lse2_dtype,
                                            int64_t rows, int D) {
  for (int64_t g = 0; g < rows; ++g) {
    float l1 = lse_in(lse1, lse1_dtype, g), l2 = lse_in(lse2, lse2_dtype, g);
    double t = 0.0, r = 0.0;
    int c = downdate_control(l1, l2, &t, &r);
    const uint16_t* a = out1 + g * D;
    uint16_t* b = out2 + g * D;
    if (c == 0) {
      /* scale 0: (o1 - 0 * o2) * 0 */
      for (int i = 0; i < D; ++i) b[i] = d_to_bf16((bf16_to_d(a[i]) - 0.0 * bf16_to_d(b[i])) * 0.0);
      lse_out(lse2, lse2_dtype, g, -INFINITY);
    } else if (c == 1) {
      for (int i = 0; i < D; ++i) b[i] = d_to_bf16(bf16_to_d(a[i]));
      lse_out(lse2, lse2_dtype, g, l1);
    } else {
      double scale = exp((double)l1 - r);
      for (int i = 0; i < D; ++i) b[i] = d_to_bf16((bf16_to_d(a[i]) - t * bf16_to_d(b[i])) * scale);
      lse_out(lse2, lse2_dtype, g, (float)r);
    }
  }
}

/* Exact attention of one query row over the key positions [lo, hi) of
 * request b (page size 1: position j is pool row kv_indices[kv_begin + j]),
 * merged into st.  Natural-log lse. */
static void window_state(const uint16_t* q, const uint16_t* k_buffer, const uint16_t* v_buffer,
                         const int32_t* kv_indices, int64_t kv_begin, int Hkv, int hkv, int D,
                         int lo, int hi, double sm_scale, State* st, double* logits) {
  State w;
  state_empty(&w, D);
  if (hi > lo) {
    double qd[128];
    for (int i = 0; i < D; ++i) qd[i] = bf16_to_d(q[i]);
    double m = -INFINITY;
    for (int j = lo; j < hi; ++j) {
      int64_t row = kv_indices[kv_begin + j];
      const uint16_t* kr = k_buffer + (row * Hkv + hkv) * D;
      double dot = 0.0;
      for (int i = 0; i < D; ++i) dot += qd[i] * bf16_to_d(kr[i]);
      logits[j - lo] = dot * sm_scale;
      if (logits[j - lo] > m) m = logits[j - lo];
    }
    double sum = 0.0;
    for (int i = 0; i < D; ++i) w.o[i] = 0.0;
    for (int j = lo; j < hi; ++j) {
      double p = exp(logits[j - lo] - m);
      sum += p;
      int64_t row = kv_indices[kv_begin + j];
      const uint16_t* vr = v_buffer + (row * Hkv + hkv) * D;
      for (int i = 0; i < D; ++i) w.o[i] += p * bf16_to_d(vr[i]);
    }
    for (int i = 0; i < D; ++i) w.o[i] /= sum;
    w.lse = m + log(sum);
  }
  state_merge(st, &w, D);
}

/*
 * Causal sliding-window prefill attention over a ragged batch with a
 * page-size-1 pool (the FlashInfer call of HOOKS:2436-2466 with
 * window_left = S - 1): query row i of request b sits at position
 * kv_len - qo_len + i and attends to [pos - window_left, pos]
 * (window_left < 0: [0, pos]).  out bf16, out_lse natural log.
 */
EXPORT void mac_oracle_window_attention(const uint16_t* q, const uint16_t* k_buffer,
                                        const uint16_t* v_buffer, const int32_t* qo_indptr,
                                        const int32_t* kv_indptr, const int32_t* kv_indices, int B,
                                        int Hq, int Hkv, int D, int window_left, double sm_scale,
                                        uint16_t* out, float* out_lse) {
  const int G = Hq / Hkv;
  int maxkv = 1;
  for (int b = 0; b < B; ++b)
    if (kv_indptr[b + 1] - kv_indptr[b] > maxkv) maxkv = kv_indptr[b + 1] - kv_indptr[b];
  double* logits = (double*)malloc(sizeof(double) * (size_t)maxkv);
  State* st = (State*)malloc(sizeof(State));
  for (int b = 0; b < B; ++b) {
    int qlen = qo_indptr[b + 1] - qo_indptr[b];
    int kvlen = kv_indptr[b + 1] - kv_indptr[b];
    for (int i = 0; i < qlen; ++i) {
      int pos = kvlen - qlen + i;
      int lo = window_left < 0 ? 0 : pos - window_left;
      if (lo < 0) lo = 0;
      int64_t row = (int64_t)qo_indptr[b] + i;
      for (int h = 0; h < Hq; ++h) {
        state_empty(st, D);
        window_state(q + (row * Hq + h) * D, k_buffer, v_buffer, kv_indices, kv_indptr[b], Hkv,
                     h / G, D, lo, pos + 1, sm_scale, st, logits);
        for (int d = 0; d < D; ++d) out[(row * Hq + h) * D + d] = d_to_bf16(st->o[d]);
        out_lse[row * Hq + h] = (float)st->lse;
      }
    }
  }
  free(st);
  free(logits);
}

/*
 * Fused rectification + ring update: for the rows the ring keeps (the last
 * min(len_b, M) rows of request b, PREFILL:201-269), the prefix state over
 * [0, E) (sink_mode 1: [min(F, E), E)), E = pos + 1 - S, obtained as the full
 * causal state (o_full, lse_full) minus the window [E, pos + 1) (and the sink)
 * with the downdate of MERGE:148-176, then stored like mac_prefill_update_cache
 * with offsets = qo_indptr.  The composition is HOOKS:2436-2482; sink_mode 0
 * with F > 0 writes lse = -inf as HOOKS:2205-2215 does.  E <= 0 (or E <= F
 * in sink_mode 1) leaves nothing: o = 0, lse = -inf.
 */
EXPORT void mac_oracle_rectify_update_cache(
    const uint16_t* q_post, const uint16_t* src_q, const uint16_t* o_full, const float* lse_full,
    const uint16_t* k_buffer, const uint16_t* v_buffer, const int32_t* qo_indptr,
    const int32_t* kv_indptr, const int32_t* kv_indices, uint16_t* q_cache, uint16_t* attn_cache,
    float* lse_cache, uint16_t* q_post_cache, int32_t* request_length, int request_length_len,
    const int32_t* req_ids, int B, int R, int M, int Hq, int Hkv, int D, int S, int F,
    int sink_mode, double sm_scale, int64_t total_q, int64_t kv_indices_len) {
  if (M <= 0 || B <= 0) return;
  const int G = Hq / Hkv;
  const int by_batch = request_length_len == B;
  const size_t rowsz = (size_t)Hq * D;
  int maxkv = 1;
  for (int b = 0; b < B; ++b)
    if (kv_indptr[b + 1] - kv_indptr[b] > maxkv) maxkv = kv_indptr[b + 1] - kv_indptr[b];
  double* logits = (double*)malloc(sizeof(double) * (size_t)maxkv);
  State* st = (State*)malloc(sizeof(State));
  int32_t* before = (int32_t*)malloc(sizeof(int32_t) * (size_t)B);
  for (int b = 0; b < B; ++b) {
    int req = req_ids[b];
    before[b] = 0;
    if (by_batch) before[b] = request_length[b];
    else if (req >= 0 && req < R) before[b] = request_length[req];
  }
  for (int b = 0; b < B; ++b) {
    int req = req_ids[b];
    int Ni = qo_indptr[b + 1] - qo_indptr[b];
    if (Ni <= 0 || req < 0 || req >= R) continue;
    int kvlen = kv_indptr[b + 1] - kv_indptr[b];
    /* a request whose query or key ranges fall outside the buffers the
     * caller described, or with fewer keys than queries, is skipped whole:
     * no ring row and no request_length bump (as the window pass skips it) */
    if (qo_indptr[b] < 0 || qo_indptr[b + 1] > total_q || kv_indptr[b] < 0 ||
        kv_indptr[b + 1] > kv_indices_len || kvlen < Ni)
      continue;
    int start = Ni > M ? Ni - M : 0;
    int L = before[b] < 0 ? 0 : before[b];
    int base_dest = (int)(((int64_t)L + start) % M);
    for (int i = start; i < Ni; ++i) {
      int dst = base_dest + (i - start);
      if (dst >= M) dst -= M;
      size_t drow = (size_t)req * M + dst;
      int64_t srow = (int64_t)qo_indptr[b] + i;
      int pos = kvlen - Ni + i;
      int E = pos + 1 - S;
      int floor_e = (sink_mode == 1 && F > 0) ? F : 0;
      for (int h = 0; h < Hq; ++h) {
        double o[128];
        double lse;
        if (E <= floor_e) {
          for (int d = 0; d < D; ++d) o[d] = 0.0;
          lse = -INFINITY;
        } else {
          state_empty(st, D);
          const uint16_t* qh = q_post + (srow * Hq + h) * D;
          window_state(qh, k_buffer, v_buffer, kv_indices, kv_indptr[b], Hkv, h / G, D, E, pos + 1,
                       sm_scale, st, logits);
          if (sink_mode == 1 && F > 0)
            window_state(qh, k_buffer, v_buffer, kv_indices, kv_indptr[b], Hkv, h / G, D, 0,
                         F < E ? F : E, sm_scale, st, logits);
          float l1 = lse_full[srow * Hq + h], l2 = (float)st->lse;
          const uint16_t* of = o_full + (srow * Hq + h) * D;
          double t = 0.0, r = 0.0;
          int c = downdate_control(l1, l2, &t, &r);
          if (c == 0) {
            for (int d = 0; d < D; ++d) o[d] = 0.0;
            lse = -INFINITY;
          } else if (c == 1) {
            for (int d = 0; d < D; ++d) o[d] = bf16_to_d(of[d]);
            lse = l1;
          } else {
            double scale = exp((double)l1 - r);
            for (int d = 0; d < D; ++d) o[d] = (bf16_to_d(of[d]) - t * st->o[d]) * scale;
            lse = r;
          }
          if (sink_mode == 0 && F > 0) lse = -INFINITY;
        }
        for (int d = 0; d < D; ++d) attn_cache[drow * rowsz + (size_t)h * D + d] = d_to_bf16(o[d]);
        lse_cache[drow * Hq + h] = (float)lse;
      }
      memcpy(q_cache + drow * rowsz, src_q + (size_t)srow * rowsz, rowsz * 2);
      if (q_post_cache)
        for (size_t j = 0; j < rowsz; ++j) q_post_cache[drow * rowsz + j] = 0x7fc0;
    }
    if (!by_batch) request_length[req] += Ni;
  }
  free(before);
  free(st);
  free(logits);
}

/* -------------------------------------------- decode RoPE + scatter ---- */

/*
 * ROPE:36-156 decode_rope_preserve_kernel.  q/k rows have row strides
 * q_stride0/k_stride0/v_stride0 (elements); positions and cache_locs are
 * int64 here.  The rotation is evaluated in double and rounded once to bf16
 * through float (the GPU evaluates it in fp32: results may differ by one bf16
 * ulp on values next to a rounding boundary).  Positions outside the table
 * are clamped, pool rows outside [0, pool) skipped.
 */
EXPORT void mac_oracle_rope_preserve(uint16_t* q, int64_t q_stride0, uint16_t* k, int64_t k_stride0,
                                     const uint16_t* v, int64_t v_stride0, uint16_t* q_pre,
                                     uint16_t* k_buffer, uint16_t* v_buffer, int64_t pool,
                                     const float* cs, int64_t cs_rows, int64_t cs_stride0, int rot,
                                     const int64_t* positions, const int64_t* cache_locs, int64_t N,
                                     int Hq, int Hkv, int D, int neox) {
  const int half = rot / 2;
  for (int64_t n = 0; n < N; ++n) {
    int64_t pos = positions[n];
    if (pos < 0) pos = 0;
    if (pos >= cs_rows) pos = cs_rows - 1;
    const float* c = cs + pos * cs_stride0;
    int64_t loc = cache_locs[n];
    int loc_ok = loc >= 0 && loc < pool;
    for (int pass = 0; pass < 2; ++pass) {
      int H = pass == 0 ? Hq : Hkv;
      uint16_t* row = pass == 0 ? q + n * q_stride0 : k + n * k_stride0;
      for (int h = 0; h < H; ++h) {
        uint16_t* x = row + (int64_t)h * D;
        if (pass == 0)
          for (int d = 0; d < D; ++d) q_pre[(n * Hq + h) * D + d] = x[d];
        for (int i = 0; i < half; ++i) {
          int d0 = neox ? i : 2 * i, d1 = neox ? i + half : 2 * i + 1;
          double x0 = bf16_to_d(x[d0]), x1 = bf16_to_d(x[d1]);
          double cc = c[i], ss = c[half + i];
          x[d0] = d_to_bf16(x0 * cc - x1 * ss);
          x[d1] = d_to_bf16(x1 * cc + x0 * ss);
        }
        if (pass == 1 && loc_ok)
          for (int d = 0; d < D; ++d) k_buffer[(loc * Hkv + h) * D + d] = x[d];
      }
    }
    if (loc_ok)
      for (int h = 0; h < Hkv; ++h)
        for (int d = 0; d < D; ++d)
          v_buffer[(loc * Hkv + h) * D + d] = v[n * v_stride0 + (int64_t)h * D + d];
  }
}
