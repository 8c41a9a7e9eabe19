/*
 * CPU ORACLE for the hi-rocm batched token sampler -- TEST INFRASTRUCTURE ONLY.
 *
 * This file is the checker, never the product: only tests/, the smoke check and
 * bench.py's cpu_baseline leg load it.  The HIP library under hi_amd/csrc never
 * links, calls or falls back to it.
 *
 * It restates, in plain C, the reference's CPU sampler and the device paths the
 * reference keeps on the GPU, so that the HIP kernels can be compared id-for-id:
 *
 *   hro_argmax_total        crates/hi-cuda/src/gpu.rs:739-751   (argmax_host)
 *   hro_argmax_ieee         crates/hi-cuda/src/kernels.cu:7153-7186 (block_argmax_last)
 *   hro_argmax_finite_lane  crates/hi-cuda/src/kernels.cu:7775-7801 (finite max/argmax
 *                           of sample_last_token_row, 256-thread strided scan + tree)
 *   hro_ranked_sample       crates/hi-cuda/src/gpu.rs:753-900
 *                           (sample_host_ranked_logits_with_uniform), windowed form
 *   hro_ranked_sample_brute crates/hi-cuda/src/gpu.rs:29505-29580
 *                           (reference_ranked_sample, the full-sort test baseline)
 *   hro_temp_only_sample    crates/hi-cuda/src/kernels.cu:7803-7867 (temperature-only
 *                           inverse CDF over 256 contiguous chunks, index order)
 *   hro_process_row         extension stages that the reference does not define for
 *                           the CUDA path: allowed-token mask, repetition penalty
 *                           (crates/hi-mlx/src/generate.rs:60-70 semantics),
 *                           OpenAI frequency/presence penalties, min-p, logprobs.
 *   hro_sample_rows         the whole per-row routing of
 *                           select_batched_last_token_per_row (gpu.rs:15810-15967)
 *                           with the extension stages, one call per batch.
 *
 * Arithmetic follows the reference exactly: f32 IEEE ops, sequential f32 folds
 * in the reference's order, glibc expf (what Rust's f32::exp lowers to on
 * Linux).  Build with -ffp-contract=off so no fused multiply-add changes a
 * rounding.  Logprobs (an extension) are computed in double.
 */
#include <float.h>
#include <math.h>
#include <pthread.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

typedef struct hro_row_params {
  float temperature;        /* <= 0 or non-finite: greedy */
  float top_p;              /* >= 1 or non-finite: no nucleus cut */
  float min_p;              /* <= 0 or non-finite: off */
  float repetition_penalty; /* |p - 1| <= FLT_EPSILON, <= 0 or non-finite: off */
  float frequency_penalty;  /* non-finite: off */
  float presence_penalty;   /* non-finite: off */
  int32_t top_k;            /* <= 0: unset */
  uint32_t eos_id;          /* token for a row whose mask allows nothing finite */
  uint32_t flags;           /* HRO_FLAG_* */
  uint32_t reserved;
} hro_row_params;

#define HRO_FLAG_REP_ONCE 1u /* repetition penalty once per distinct token */

/* Sampler outcome classes, reported per row for test bookkeeping. */
enum { HRO_GREEDY = 0, HRO_RANKED = 1, HRO_TEMP_ONLY = 2, HRO_EOS = 3, HRO_FALLBACK = 4 };

/* ------------------------------------------------------------------------- */
/* total order helpers                                                       */

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

/* Key whose signed comparison is Rust's f32::total_cmp. */
static inline int32_t total_key(float f) {
  int32_t i = (int32_t)f2u(f);
  return i ^ (int32_t)(((uint32_t)(i >> 31)) >> 1);
}

static inline int is_finite_f(float f) { return isfinite(f) != 0; }

/* gpu.rs:739-751: max_by(total_cmp), ties resolve to the lower index. */
int64_t hro_argmax_total(const float* x, int64_t n) {
  if (n <= 0) return -1;
  int64_t best = 0;
  int32_t bk = total_key(x[0]);
  for (int64_t i = 1; i < n; ++i) {
    int32_t k = total_key(x[i]);
    if (k > bk) { bk = k; best = i; }
  }
  return best;
}

/* kernels.cu:7153-7186: IEEE '>' scan from -inf, the lowest index wins ties,
 * NaN never wins; a row with nothing above -inf yields 0. */
int64_t hro_argmax_ieee(const float* x, int64_t n) {
  float best = -INFINITY;
  int64_t bi = 0;
  for (int64_t i = 0; i < n; ++i) {
    if (x[i] > best) { best = x[i]; bi = i; }
  }
  return bi;
}

/* kernels.cu:7775-7801, restated literally: 256 lanes, lane t scans indices
 * t, t+256, ... and keeps the first finite value that is strictly larger than
 * its running maximum (start -inf, argmax 0); then a tree over the lanes with
 * strides 128, 64, ..., 1, where slot t takes slot t+s only when that value is
 * strictly larger.  On tied maxima this prefers the smallest 8-bit bit
 * reversal of (idx mod 256), then the smallest idx.  With no finite value the
 * result is 0 and *max_out is -inf. */
int64_t hro_argmax_finite_lane(const float* x, int64_t n, float* max_out) {
  float lmax[256];
  int64_t larg[256];
  for (int t = 0; t < 256; ++t) {
    lmax[t] = -INFINITY;
    larg[t] = 0;
    for (int64_t i = t; i < n; i += 256) {
      const float v = x[i];
      if (is_finite_f(v) && v > lmax[t]) { lmax[t] = v; larg[t] = i; }
    }
  }
  for (int s = 128; s > 0; s >>= 1) {
    for (int t = 0; t < s; ++t) {
      if (lmax[t + s] > lmax[t]) { lmax[t] = lmax[t + s]; larg[t] = larg[t + s]; }
    }
  }
  if (max_out) *max_out = lmax[0];
  return larg[0];
}

/* ------------------------------------------------------------------------- */
/* ranked sampler (gpu.rs:753-900)                                           */

typedef struct { int64_t idx; float w; } ranked_t;

/* by_rank (gpu.rs:794-796): weight descending by total_cmp, then index asc. */
static inline int rank_less(const ranked_t* a, const ranked_t* b) {
  int32_t ka = total_key(a->w), kb = total_key(b->w);
  if (ka != kb) return ka > kb;
  return a->idx < b->idx;
}
static int rank_cmp(const void* pa, const void* pb) {
  const ranked_t* a = pa; const ranked_t* b = pb;
  if (rank_less(a, b)) return -1;
  if (rank_less(b, a)) return 1;
  return 0;
}

/* Partial selection standing in for Rust's select_nth_unstable_by: afterwards
 * v[0..k) holds the k first elements of the rank order (in any order).  The
 * comparator is a total order, so the selected set is unique. */
static void select_first_k(ranked_t* v, int64_t n, int64_t k) {
  int64_t lo = 0, hi = n - 1;
  uint64_t state = 0x9E3779B97F4A7C15ull;
  while (lo < hi) {
    state = state * 6364136223846793005ull + 1442695040888963407ull;
    int64_t p = lo + (int64_t)((state >> 33) % (uint64_t)(hi - lo + 1));
    ranked_t pivot = v[p];
    v[p] = v[hi]; v[hi] = pivot;
    int64_t store = lo;
    for (int64_t i = lo; i < hi; ++i) {
      if (rank_less(&v[i], &pivot)) { ranked_t t = v[i]; v[i] = v[store]; v[store] = t; ++store; }
    }
    ranked_t t = v[store]; v[store] = v[hi]; v[hi] = t;
    if (store == k) return;
    if (store < k) lo = store + 1; else hi = store - 1;
  }
}

/* Rust's f32 Sum: a sequential fold from -0.0. */
static float fold_sum(const float* w, int64_t n, int64_t stride) {
  float acc = -0.0f;
  for (int64_t i = 0; i < n; ++i) acc += w[i * stride];
  return acc;
}

typedef struct hro_ranked_info {
  int32_t path;            /* HRO_RANKED or HRO_FALLBACK */
  int64_t n_candidates;    /* nucleus size after top-k / top-p / min-p */
  float total;             /* normaliser (gpu.rs:834-838) */
  float candidate_total;   /* gpu.rs:874-881 */
  float max_scaled;
  double cdf_margin;       /* distance of the clamped uniform to the nearest CDF
                              boundary around the pick, in uniform units */
  double cutoff_margin;    /* |cum_p at the last candidate - top_p| (top-p rows) */
} hro_ranked_info;

/*
 * gpu.rs:753-900, restated step for step, with one extension: min_p (> 0)
 * zeroes every weight below min_p before ranking (the maximum weight is 1, so
 * this is p_i < min_p * p_max).  min_p = 0 reproduces the reference exactly.
 * Returns the token, or -1 for empty logits.
 */
int64_t hro_ranked_sample(const float* logits, int64_t n, float temperature, float top_p,
                          int32_t top_k, float min_p, float sample, hro_ranked_info* info) {
  hro_ranked_info dummy;
  if (!info) info = &dummy;
  memset(info, 0, sizeof(*info));
  info->path = HRO_FALLBACK;
  if (n <= 0) return -1;
  if (!is_finite_f(temperature) || temperature <= 0.0f) return hro_argmax_total(logits, n);

  float* w = malloc((size_t)n * sizeof(float));
  float mx = -INFINITY;
  for (int64_t i = 0; i < n; ++i) {
    w[i] = is_finite_f(logits[i]) ? logits[i] / temperature : -INFINITY;
    mx = fmaxf(mx, w[i]);
  }
  info->max_scaled = mx;
  if (!is_finite_f(mx)) { free(w); return hro_argmax_total(logits, n); }
  for (int64_t i = 0; i < n; ++i) w[i] = expf(w[i] - mx);
  if (is_finite_f(min_p) && min_p > 0.0f) {
    float mp = min_p > 1.0f ? 1.0f : min_p;
    for (int64_t i = 0; i < n; ++i) if (w[i] < mp) w[i] = 0.0f;
  }

  float cutoff = is_finite_f(top_p) ? (top_p < 0.0f ? 0.0f : (top_p > 1.0f ? 1.0f : top_p)) : 1.0f;
  ranked_t* ranked = malloc((size_t)n * sizeof(ranked_t));
  for (int64_t i = 0; i < n; ++i) { ranked[i].idx = i; ranked[i].w = w[i]; }
  const int64_t WINDOW = 1024; /* TOP_P_PREFILTER_WINDOW, gpu.rs:806 */
  int64_t ranked_len = n;
  int64_t ordered_len;
  int have_k = top_k > 0;
  int64_t k_keep = have_k ? ((int64_t)top_k < n ? (int64_t)top_k : n) : 0;
  if (have_k) {
    if (k_keep < n) { select_first_k(ranked, n, k_keep); ranked_len = k_keep; }
    qsort(ranked, (size_t)ranked_len, sizeof(ranked_t), rank_cmp);
    ordered_len = ranked_len;
  } else if (cutoff < 1.0f && WINDOW < n) {
    select_first_k(ranked, n, WINDOW);
    qsort(ranked, (size_t)WINDOW, sizeof(ranked_t), rank_cmp);
    ordered_len = WINDOW;
  } else {
    qsort(ranked, (size_t)n, sizeof(ranked_t), rank_cmp);
    ordered_len = n;
  }

  float total;
  if (have_k) {
    total = -0.0f;
    for (int64_t i = 0; i < ranked_len; ++i) total += ranked[i].w;
  } else {
    total = fold_sum(w, n, 1);
  }
  info->total = total;
  if (total <= 0.0f || !is_finite_f(total)) { free(w); free(ranked); return hro_argmax_total(logits, n); }

  int64_t n_cand = 0; /* candidates are a prefix-with-gaps of ranked[]: record positions */
  int64_t* cand = malloc((size_t)(ranked_len > 0 ? ranked_len : 1) * sizeof(int64_t));
  float cum_p = 0.0f;
  int covered = ordered_len == ranked_len;
  for (int64_t i = 0; i < ordered_len; ++i) {
    if (ranked[i].w <= 0.0f) continue;
    cand[n_cand++] = i;
    cum_p += ranked[i].w / total;
    if (cutoff < 1.0f && cum_p >= cutoff) { covered = 1; break; }
  }
  if (!covered) {
    qsort(ranked, (size_t)ranked_len, sizeof(ranked_t), rank_cmp);
    n_cand = 0;
    cum_p = 0.0f;
    for (int64_t i = 0; i < ranked_len; ++i) {
      if (ranked[i].w <= 0.0f) continue;
      cand[n_cand++] = i;
      cum_p += ranked[i].w / total;
      if (cutoff < 1.0f && cum_p >= cutoff) break;
    }
  }
  info->cutoff_margin = fabs((double)cum_p - (double)cutoff);
  if (n_cand == 0) { free(w); free(ranked); free(cand); return hro_argmax_total(logits, n); }

  float ct = -0.0f;
  for (int64_t j = 0; j < n_cand; ++j) ct += ranked[cand[j]].w;
  info->candidate_total = ct;
  info->n_candidates = n_cand;
  if (ct <= 0.0f || !is_finite_f(ct)) { free(w); free(ranked); free(cand); return hro_argmax_total(logits, n); }

  float u = is_finite_f(sample) ? (sample < 0.0f ? 0.0f : (sample > 0.99999994f ? 0.99999994f : sample)) : 0.0f;
  float target = u * ct;
  float cum = 0.0f, prev = 0.0f;
  int64_t pick = ranked[cand[n_cand - 1]].idx;
  int64_t pick_j = n_cand - 1;
  for (int64_t j = 0; j < n_cand; ++j) {
    prev = cum;
    cum += ranked[cand[j]].w;
    if (target < cum) { pick = ranked[cand[j]].idx; pick_j = j; break; }
  }
  if (pick_j == n_cand - 1 && !(target < cum)) prev = cum; /* fell through */
  {
    double lo = (double)prev / (double)ct, hi = (double)cum / (double)ct;
    double a = fabs((double)u - lo), b = fabs((double)u - hi);
    info->cdf_margin = a < b ? a : b;
  }
  info->path = HRO_RANKED;
  free(w); free(ranked); free(cand);
  return pick;
}

/* gpu.rs:29505-29580: the reference test's brute-force baseline (always a full
 * sort), extended with the same min_p rule as hro_ranked_sample. */
int64_t hro_ranked_sample_brute(const float* logits, int64_t n, float temperature, float top_p,
                                int32_t top_k, float min_p, float sample) {
  float* w = malloc((size_t)n * sizeof(float));
  float mx = -INFINITY;
  for (int64_t i = 0; i < n; ++i) {
    w[i] = is_finite_f(logits[i]) ? logits[i] / temperature : -INFINITY;
    mx = fmaxf(mx, w[i]);
  }
  for (int64_t i = 0; i < n; ++i) w[i] = expf(w[i] - mx);
  if (is_finite_f(min_p) && min_p > 0.0f) {
    float mp = min_p > 1.0f ? 1.0f : min_p;
    for (int64_t i = 0; i < n; ++i) if (w[i] < mp) w[i] = 0.0f;
  }
  ranked_t* r = malloc((size_t)n * sizeof(ranked_t));
  for (int64_t i = 0; i < n; ++i) { r[i].idx = i; r[i].w = w[i]; }
  qsort(r, (size_t)n, sizeof(ranked_t), rank_cmp);
  int64_t len = n;
  int have_k = top_k > 0;
  if (have_k && (int64_t)top_k < len) len = top_k;
  float cutoff = is_finite_f(top_p) ? (top_p < 0.0f ? 0.0f : (top_p > 1.0f ? 1.0f : top_p)) : 1.0f;
  float total = -0.0f;
  if (have_k) { for (int64_t i = 0; i < len; ++i) total += r[i].w; }
  else { for (int64_t i = 0; i < n; ++i) total += w[i]; }
  int64_t nc = 0; float cum = 0.0f;
  for (int64_t i = 0; i < len; ++i) {
    if (r[i].w <= 0.0f) continue;
    r[nc++] = r[i];
    cum += r[i].w / total;
    if (cutoff < 1.0f && cum >= cutoff) break;
  }
  float ct = -0.0f;
  for (int64_t i = 0; i < nc; ++i) ct += r[i].w;
  float u = is_finite_f(sample) ? (sample < 0.0f ? 0.0f : (sample > 0.99999994f ? 0.99999994f : sample)) : 0.0f;
  float target = u * ct, c = 0.0f;
  int64_t out = nc > 0 ? r[nc - 1].idx : -1;
  for (int64_t i = 0; i < nc; ++i) { c += r[i].w; if (target < c) { out = r[i].idx; break; } }
  free(w); free(r);
  return out;
}

/* ------------------------------------------------------------------------- */
/* temperature-only inverse CDF (kernels.cu:7803-7867)                        */

static inline float temp_weight(float logit, float temperature, float max_scaled) {
  if (!is_finite_f(logit)) return 0.0f;            /* kernels.cu:7241-7243 */
  float scaled = logit / temperature;
  if (!is_finite_f(scaled)) return 0.0f;           /* kernels.cu:7245-7247 */
  return expf(scaled - max_scaled);                /* kernels.cu:7249, glibc expf */
}

/* The reference device path for sampled rows that have neither top_k nor a
 * top_p below 1: 256 contiguous chunks, per-chunk sequential f32 sums, a serial
 * chunk prefix, then the owning chunk rescans from its exclusive prefix.  The
 * reference evaluates CUDA expf here; this restatement (and the HIP kernel)
 * use the glibc-exact weight instead. */
int64_t hro_temp_only_sample(const float* logits, int64_t n, float temperature, float sample) {
  float lmax;
  int64_t argmax = hro_argmax_finite_lane(logits, n, &lmax);
  if (!is_finite_f(temperature) || temperature <= 0.0f) return argmax;
  float max_scaled = lmax / temperature;
  if (!is_finite_f(max_scaled)) return argmax;
  float u = is_finite_f(sample) ? fminf(fmaxf(sample, 0.0f), 0.99999994f) : 0.0f;
  const int64_t T = 256;
  int64_t chunk = (n + T - 1) / T;
  float csum[256], prefix[256];
  for (int64_t t = 0; t < T; ++t) {
    int64_t start = t * chunk, end = start + chunk < n ? start + chunk : n;
    float s = 0.0f;
    for (int64_t i = start; i < end; ++i) s += temp_weight(logits[i], temperature, max_scaled);
    csum[t] = s;
  }
  float acc = 0.0f;
  for (int64_t t = 0; t < T; ++t) { prefix[t] = acc; acc += csum[t]; }
  float total = acc;
  if (total <= 0.0f || !is_finite_f(total)) return argmax;
  float target = u * total;
  uint32_t token = 0xFFFFFFFFu;
  for (int64_t t = 0; t < T; ++t) {
    int64_t start = t * chunk, end = start + chunk < n ? start + chunk : n;
    float lo = prefix[t], hi = lo + csum[t];
    if (start < end && target >= lo && (target < hi || t == T - 1)) {
      float c = lo;
      int64_t chosen = -1;
      for (int64_t i = start; i < end; ++i) {
        float wv = temp_weight(logits[i], temperature, max_scaled);
        if (wv <= 0.0f) continue;
        chosen = i;
        c += wv;
        if (target < c) break;
      }
      if (chosen >= 0 && (uint32_t)chosen < token) token = (uint32_t)chosen;
    }
  }
  return token != 0xFFFFFFFFu ? (int64_t)token : argmax;
}

/* ------------------------------------------------------------------------- */
/* extension stages (mask, penalties) and the per-row router                  */

/* Widen bf16 to f32: exact. */
static inline float bf16_to_f32(uint16_t h) { uint32_t u = (uint32_t)h << 16; float f; memcpy(&f, &u, 4); return f; }

/*
 * Processed logits for one row, in stage order:
 *   1. allowed-token mask: a clear bit (LSB-first in 32-bit words) gives -inf;
 *   2. repetition penalty p for a token seen c > 0 times:
 *        l = l < 0 ? l * p : l / p, applied c times in f32
 *        (crates/hi-mlx/src/generate.rs:60-70, once per history occurrence),
 *        once if HRO_FLAG_REP_ONCE; off when |p - 1| <= FLT_EPSILON
 *        (generate.rs:60) or p is not finite and > 0;
 *   3. frequency and presence penalties (OpenAI form), for c > 0:
 *        l = l - f * c; l = l - presence  (separate f32 roundings, no FMA).
 * History entries are (id, count) pairs; ids >= n are ignored; repeated ids add.
 * Returns 1 when at least one processed logit is finite.
 */
int hro_process_row(const float* raw, int64_t n, const hro_row_params* p,
                    const uint32_t* hist_ids, const uint32_t* hist_counts, int64_t hist_len,
                    const uint32_t* mask_words, float* out) {
  for (int64_t i = 0; i < n; ++i) out[i] = raw[i];
  if (mask_words) {
    for (int64_t i = 0; i < n; ++i)
      if (!((mask_words[i >> 5] >> (i & 31)) & 1u)) out[i] = -INFINITY;
  }
  if (hist_len > 0) {
    uint32_t* cnt = calloc((size_t)n, sizeof(uint32_t));
    for (int64_t h = 0; h < hist_len; ++h)
      if ((int64_t)hist_ids[h] < n) cnt[hist_ids[h]] += hist_counts[h];
    float rp = p->repetition_penalty;
    int rep_on = is_finite_f(rp) && rp > 0.0f && fabsf(rp - 1.0f) > FLT_EPSILON;
    float fp = is_finite_f(p->frequency_penalty) ? p->frequency_penalty : 0.0f;
    float pp = is_finite_f(p->presence_penalty) ? p->presence_penalty : 0.0f;
    for (int64_t i = 0; i < n; ++i) {
      uint32_t c = cnt[i];
      if (c == 0) continue;
      float l = out[i];
      if (rep_on) {
        uint32_t reps = (p->flags & HRO_FLAG_REP_ONCE) ? 1u : c;
        for (uint32_t r = 0; r < reps; ++r) l = l < 0.0f ? l * rp : l / rp;
      }
      float fc = fp * (float)c;
      l = l - fc;
      l = l - pp;
      out[i] = l;
    }
    free(cnt);
  }
  for (int64_t i = 0; i < n; ++i) if (is_finite_f(out[i])) return 1;
  return 0;
}

/* gpu.rs:731-738 extended with min_p: sampled rows that need a ranking. */
static int needs_rank(const hro_row_params* p) {
  return is_finite_f(p->temperature) && p->temperature > 0.0f &&
         ((is_finite_f(p->top_p) && p->top_p < 1.0f) || p->top_k > 0 ||
          (is_finite_f(p->min_p) && p->min_p > 0.0f));
}

/* Logprobs over the processed, temperature-scaled distribution before any
 * truncation: lp_i = (s_i - max) - ln(sum_j exp(s_j - max)), in double.
 * Entries are the first n_lp of the rank order (weight desc, index asc);
 * missing entries are (UINT32_MAX, -inf). */
static void row_logprobs(const float* l, int64_t n, float t_eff, int n_lp, int64_t token,
                         float* out_lp, uint32_t* out_ids, float* out_token_lp) {
  float* s = malloc((size_t)n * sizeof(float));
  float mx = -INFINITY;
  for (int64_t i = 0; i < n; ++i) { s[i] = is_finite_f(l[i]) ? l[i] / t_eff : -INFINITY; mx = fmaxf(mx, s[i]); }
  for (int j = 0; j < n_lp; ++j) { out_lp[j] = -INFINITY; out_ids[j] = 0xFFFFFFFFu; }
  if (!is_finite_f(mx)) { if (out_token_lp) *out_token_lp = -INFINITY; free(s); return; }
  double sum = 0.0;
  for (int64_t i = 0; i < n; ++i) sum += exp((double)s[i] - (double)mx);
  double lse = log(sum);
  if (n_lp > 0) {
    ranked_t* r = malloc((size_t)n * sizeof(ranked_t));
    for (int64_t i = 0; i < n; ++i) { r[i].idx = i; r[i].w = expf(s[i] - mx); }
    int64_t m = n_lp < n ? n_lp : n;
    if (m < n) select_first_k(r, n, m);
    qsort(r, (size_t)m, sizeof(ranked_t), rank_cmp);
    for (int64_t j = 0; j < m; ++j) {
      out_ids[j] = (uint32_t)r[j].idx;
      out_lp[j] = (float)(((double)s[r[j].idx] - (double)mx) - lse);
    }
    free(r);
  }
  if (out_token_lp)
    *out_token_lp = (token >= 0 && token < n) ? (float)(((double)s[token] - (double)mx) - lse) : -INFINITY;
  free(s);
}

typedef struct hro_batch {
  const void* logits;          /* [B][row_stride] f32 or bf16 */
  int dtype;                   /* 0 = f32, 1 = bf16 */
  int64_t batch, vocab, row_stride;
  const hro_row_params* params;   /* [B] */
  const float* uniforms;          /* [B] */
  const uint32_t* hist_offsets;   /* [B+1] or NULL */
  const uint32_t* hist_ids;
  const uint32_t* hist_counts;
  const uint32_t* mask_words;     /* [B][ceil(V/32)] or NULL */
  int n_logprobs;
  uint32_t* out_tokens;           /* [B] */
  float* out_logprobs;            /* [B][n_logprobs] or NULL */
  uint32_t* out_logprob_ids;      /* [B][n_logprobs] or NULL */
  float* out_token_logprobs;      /* [B] or NULL */
  int32_t* out_path;              /* [B] or NULL: HRO_* class per row */
  double* out_cdf_margin;         /* [B] or NULL */
  double* out_cutoff_margin;      /* [B] or NULL */
  int64_t* out_n_candidates;      /* [B] or NULL */
} hro_batch;

static void sample_one_row(const hro_batch* b, int64_t row, float* l) {
  int64_t V = b->vocab;
  const hro_row_params* p = &b->params[row];
  if (b->dtype == 1) {
    const uint16_t* src = (const uint16_t*)b->logits + row * b->row_stride;
    for (int64_t i = 0; i < V; ++i) l[i] = bf16_to_f32(src[i]);
  } else {
    const float* src = (const float*)b->logits + row * b->row_stride;
    memcpy(l, src, (size_t)V * sizeof(float));
  }
  int64_t h0 = 0, h1 = 0;
  if (b->hist_offsets) { h0 = b->hist_offsets[row]; h1 = b->hist_offsets[row + 1]; }
  const uint32_t* mask = b->mask_words ? b->mask_words + row * ((V + 31) / 32) : NULL;
  int any_finite = hro_process_row(l, V, p, b->hist_ids ? b->hist_ids + h0 : NULL,
                                   b->hist_counts ? b->hist_counts + h0 : NULL, h1 - h0, mask, l);
  int64_t token;
  int32_t path;
  double cdf_margin = INFINITY, cutoff_margin = INFINITY;
  int64_t n_cand = 0;
  int greedy = !(is_finite_f(p->temperature) && p->temperature > 0.0f);
  if (mask && !any_finite) {
    token = p->eos_id;
    path = HRO_EOS;
  } else if (greedy) {
    token = hro_argmax_ieee(l, V);
    path = HRO_GREEDY;
  } else if (needs_rank(p)) {
    hro_ranked_info info;
    token = hro_ranked_sample(l, V, p->temperature, p->top_p, p->top_k, p->min_p, b->uniforms[row], &info);
    path = info.path;
    cdf_margin = info.cdf_margin;
    cutoff_margin = info.cutoff_margin;
    n_cand = info.n_candidates;
  } else {
    token = hro_temp_only_sample(l, V, p->temperature, b->uniforms[row]);
    path = HRO_TEMP_ONLY;
  }
  b->out_tokens[row] = (uint32_t)token;
  if (b->out_path) b->out_path[row] = path;
  if (b->out_cdf_margin) b->out_cdf_margin[row] = cdf_margin;
  if (b->out_cutoff_margin) b->out_cutoff_margin[row] = cutoff_margin;
  if (b->out_n_candidates) b->out_n_candidates[row] = n_cand;
  if (b->n_logprobs > 0 || b->out_token_logprobs) {
    int nl = b->n_logprobs > 0 ? b->n_logprobs : 0;
    float* lp = b->out_logprobs ? b->out_logprobs + row * nl : NULL;
    uint32_t* ids = b->out_logprob_ids ? b->out_logprob_ids + row * nl : NULL;
    float tok_lp;
    if (path == HRO_EOS) {
      for (int j = 0; j < nl; ++j) { if (lp) lp[j] = -INFINITY; if (ids) ids[j] = 0xFFFFFFFFu; }
      tok_lp = 0.0f;
    } else {
      float* tmp_lp = malloc((size_t)(nl > 0 ? nl : 1) * sizeof(float));
      uint32_t* tmp_ids = malloc((size_t)(nl > 0 ? nl : 1) * sizeof(uint32_t));
      row_logprobs(l, V, greedy ? 1.0f : p->temperature, nl, token, tmp_lp, tmp_ids, &tok_lp);
      for (int j = 0; j < nl; ++j) { if (lp) lp[j] = tmp_lp[j]; if (ids) ids[j] = tmp_ids[j]; }
      free(tmp_lp); free(tmp_ids);
    }
    if (b->out_token_logprobs) b->out_token_logprobs[row] = tok_lp;
  }
}

typedef struct { const hro_batch* b; int64_t r0, r1; } job_t;
static void* run_job(void* arg) {
  job_t* j = arg;
  float* l = malloc((size_t)j->b->vocab * sizeof(float));
  for (int64_t r = j->r0; r < j->r1; ++r) sample_one_row(j->b, r, l);
  free(l);
  return NULL;
}

/* Whole batch, rows split over n_threads (1 = the reference's serial host loop,
 * gpu.rs:15716-15732).  Returns 0, or 1 for bad arguments. */
int hro_sample_rows(const hro_batch* b, int n_threads) {
  if (!b || !b->logits || !b->params || !b->uniforms || !b->out_tokens || b->batch <= 0 ||
      b->vocab <= 0 || b->row_stride < b->vocab || (b->dtype != 0 && b->dtype != 1))
    return 1;
  if (n_threads < 1) n_threads = 1;
  if (n_threads > b->batch) n_threads = (int)b->batch;
  if (n_threads == 1) {
    job_t j = {b, 0, b->batch};
    run_job(&j);
    return 0;
  }
  pthread_t* th = malloc(sizeof(pthread_t) * (size_t)n_threads);
  job_t* jobs = malloc(sizeof(job_t) * (size_t)n_threads);
  for (int t = 0; t < n_threads; ++t) {
    jobs[t].b = b;
    jobs[t].r0 = b->batch * t / n_threads;
    jobs[t].r1 = b->batch * (t + 1) / n_threads;
    pthread_create(&th[t], NULL, run_job, &jobs[t]);
  }
  for (int t = 0; t < n_threads; ++t) pthread_join(th[t], NULL);
  free(th); free(jobs);
  return 0;
}

/* glibc expf, exported so tests can compare the device weight function with
 * the host library bit for bit. */
void hro_expf_array(const float* x, float* y, int64_t n) {
  for (int64_t i = 0; i < n; ++i) y[i] = expf(x[i]);
}

/* Parallel exhaustive helper: count x in the bit range [lo, hi] where
 * expf(x) differs from ref(x) given as a table of results for that range. */
int64_t hro_expf_count_mismatch(uint32_t lo_bits, const uint32_t* dev_bits, int64_t n) {
  int64_t bad = 0;
  for (int64_t i = 0; i < n; ++i) {
    uint32_t u = lo_bits + (uint32_t)i;
    float x; memcpy(&x, &u, 4);
    float y = expf(x);
    if (f2u(y) != dev_bits[i]) ++bad;
  }
  return bad;
}

/* Sequential f32 fold exactly as Rust's Sum (used by tests of the device fold). */
float hro_fold_f32(const float* x, int64_t n) { return fold_sum(x, n, 1); }

/* ---- DSV4 indexer block selection -------------------------------------
 * Follows the host's indexer_select_math, crates/hi-cuda/src/dsv4_cpu.rs:
 * 3258-3270 (and the test's host_select, dsv4_gpu.rs:7260-7275): sort
 * (index, score) by score with f32::total_cmp descending, then index
 * ascending; take min(top_k, n); sort the taken indices ascending.
 * total_cmp order is the unsigned order of the key below. */
static uint32_t hro_total_key(float x) {
  uint32_t u;
  memcpy(&u, &x, 4);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

typedef struct { uint32_t key; int32_t idx; } hro_scored;

static int hro_rank_cmp(const void* a, const void* b) {
  const hro_scored* x = (const hro_scored*)a;
  const hro_scored* y = (const hro_scored*)b;
  if (x->key != y->key) return x->key > y->key ? -1 : 1;
  return x->idx < y->idx ? -1 : (x->idx > y->idx);
}

static int hro_int_cmp(const void* a, const void* b) {
  const int32_t x = *(const int32_t*)a, y = *(const int32_t*)b;
  return x < y ? -1 : (x > y);
}

/* Returns take (the entries written to sel), or -1 for bad arguments or no
 * memory.  marks[b] = 1 for a kept block, else 0. */
int64_t hro_indexer_select(const float* scores, int64_t n, int64_t top_k, uint8_t* marks,
                           int32_t* sel) {
  if (n <= 0 || top_k <= 0) return -1;
  const int64_t take = top_k < n ? top_k : n;
  hro_scored* r = (hro_scored*)malloc((size_t)n * sizeof(hro_scored));
  if (r == NULL) return -1;
  for (int64_t i = 0; i < n; ++i) {
    r[i].key = hro_total_key(scores[i]);
    r[i].idx = (int32_t)i;
  }
  qsort(r, (size_t)n, sizeof(hro_scored), hro_rank_cmp);
  memset(marks, 0, (size_t)n);
  for (int64_t i = 0; i < take; ++i) {
    sel[i] = r[i].idx;
    marks[r[i].idx] = 1;
  }
  free(r);
  qsort(sel, (size_t)take, sizeof(int32_t), hro_int_cmp);
  return take;
}

/* ---- MoE router top-k (kernels.cu:536-684 moe_topk_router_kernel) ----
 * The reference's per-row loops restated literally, one row at a time,
 * with glibc expf in place of CUDA's expf (which cannot be reproduced
 * here).  scores [rows][experts]; ids u32 / weights f32 [rows][top_k];
 * bias f32[experts] or NULL. */
void hro_moe_router(const float* scores, uint32_t* output_ids, float* output_weights,
                    const float* selection_bias, int rows, int experts, int top_k, int norm_topk,
                    int gating_sigmoid, float weights_scale) {
  for (int row = 0; row < rows; ++row) {
    const float* row_scores = scores + (int64_t)row * experts;
    uint32_t* row_ids = output_ids + (int64_t)row * top_k;
    float* row_weights = output_weights + (int64_t)row * top_k;
    if (gating_sigmoid) {
      /* kernels.cu:556-604 */
      float previous_key = INFINITY;
      int previous_id = -1;
      float selected_sum = 0.0f;
      for (int rank = 0; rank < top_k; ++rank) {
        int best_id = -1;
        float best_key = -INFINITY, best_weight = 0.0f;
        for (int expert = 0; expert < experts; ++expert) {
          float score = 1.0f / (1.0f + expf(-row_scores[expert]));
          if (!isfinite(score)) score = 0.0f;
          float key = score;
          if (selection_bias != NULL) key += selection_bias[expert];
          const int eligible = previous_id < 0 || key < previous_key ||
                               (key == previous_key && expert > previous_id);
          if (!eligible) continue;
          if (best_id < 0 || key > best_key || (key == best_key && expert < best_id)) {
            best_id = expert;
            best_key = key;
            best_weight = score;
          }
        }
        if (best_id < 0) {
          best_id = rank < experts ? rank : experts - 1;
          best_key = -INFINITY;
          best_weight = 0.0f;
        }
        row_ids[rank] = (uint32_t)best_id;
        row_weights[rank] = best_weight;
        selected_sum += best_weight;
        previous_id = best_id;
        previous_key = best_key;
      }
      if (norm_topk && top_k > 1 && selected_sum > 1.0e-7f && isfinite(selected_sum))
        for (int rank = 0; rank < top_k; ++rank) row_weights[rank] /= selected_sum;
      if (weights_scale != 1.0f)
        for (int rank = 0; rank < top_k; ++rank) row_weights[rank] *= weights_scale;
      continue;
    }
    /* kernels.cu:606-684 */
    float max_score = -INFINITY;
    for (int expert = 0; expert < experts; ++expert)
      if (row_scores[expert] > max_score) max_score = row_scores[expert];
    float denom = 0.0f;
    int fallback = !isfinite(max_score);
    if (!fallback) {
      for (int expert = 0; expert < experts; ++expert) denom += expf(row_scores[expert] - max_score);
      fallback = denom <= 0.0f || !isfinite(denom);
    }
    if (fallback) {
      const float weight = (norm_topk && top_k > 1) ? 1.0f / (float)top_k : 1.0f / (float)experts;
      for (int rank = 0; rank < top_k; ++rank) {
        row_ids[rank] = (uint32_t)rank;
        row_weights[rank] = weight;
      }
      continue;
    }
    float previous_weight = INFINITY;
    int previous_id = -1;
    float selected_sum = 0.0f;
    for (int rank = 0; rank < top_k; ++rank) {
      int best_id = -1;
      float best_weight = -1.0f;
      for (int expert = 0; expert < experts; ++expert) {
        float weight = expf(row_scores[expert] - max_score) / denom;
        if (!isfinite(weight)) weight = 0.0f;
        const int eligible = previous_id < 0 || weight < previous_weight ||
                             (weight == previous_weight && expert > previous_id);
        if (!eligible) continue;
        if (best_id < 0 || weight > best_weight || (weight == best_weight && expert < best_id)) {
          best_id = expert;
          best_weight = weight;
        }
      }
      if (best_id < 0) {
        best_id = rank < experts ? rank : experts - 1;
        best_weight = 0.0f;
      }
      row_ids[rank] = (uint32_t)best_id;
      row_weights[rank] = best_weight;
      selected_sum += best_weight;
      previous_id = best_id;
      previous_weight = best_weight;
    }
    if (norm_topk && top_k > 1 && selected_sum > 1.0e-7f && isfinite(selected_sum))
      for (int rank = 0; rank < top_k; ++rank) row_weights[rank] /= selected_sum;
    if (weights_scale != 1.0f)
      for (int rank = 0; rank < top_k; ++rank) row_weights[rank] *= weights_scale;
  }
}

/* ---- greedy speculative verification (gpu.rs:10725-10762) ----
 * argmax_rows (gpu.rs:6421-6434) per verify row, then the accepted prefix.
 * logits [batch][K+1][V]; draft [batch][K]; draft_len[batch] or NULL;
 * greedy / out_tokens [batch][K+1]; out_count[batch]. */
void hro_spec_verify_greedy(const float* logits, int batch, int K, int V, const uint32_t* draft,
                            const int32_t* draft_len, uint32_t* greedy, uint32_t* out_tokens,
                            int32_t* out_count) {
  for (int b = 0; b < batch; ++b) {
    for (int r = 0; r <= K; ++r) {
      const float* row = logits + ((int64_t)b * (K + 1) + r) * V;
      int64_t best = 0;
      float best_val = row[0];
      for (int64_t idx = 0; idx < V; ++idx) {
        if (row[idx] > best_val) {
          best_val = row[idx];
          best = idx;
        }
      }
      greedy[(int64_t)b * (K + 1) + r] = (uint32_t)best;
    }
    int k = draft_len ? draft_len[b] : K;
    if (k < 0) k = 0;
    if (k > K) k = K;
    const uint32_t* g = greedy + (int64_t)b * (K + 1);
    int accepted = k;
    for (int i = 0; i < k; ++i) {
      if (draft[(int64_t)b * K + i] != g[i]) {
        accepted = i;
        break;
      }
    }
    for (int i = 0; i <= accepted; ++i) out_tokens[(int64_t)b * (K + 1) + i] = g[i];
    out_count[b] = accepted + 1;
  }
}
