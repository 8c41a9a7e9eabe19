// hi-rocm batched token sampler: CDNA4 (gfx950) kernels.
//
// Per decode step the logits [B, V] stay in HBM; two kernels produce one
// token id (and optional logprobs) per row:
//
//   scan_chunks   grid (ceil(V/8192), B) x 256 threads.  One streaming pass
//                 over the row's logits with 128-bit loads: allowed-token
//                 mask, penalties from an LDS count table built from the
//                 row's history, temperature, then per-chunk statistics
//                 (max, three argmax variants, online log-sum-exp) and the
//                 chunk's exact top-k' candidates (LDS radix select).
//   finish_rows   grid B x 1024 threads.  Merges the chunk candidates,
//                 ranks them with the glibc-exact weight function and runs
//                 the reference's sequential f32 folds and inverse-CDF draw
//                 (crates/hi-cuda/src/gpu.rs:753-900) on device.
//
// Rows without top-k (top-p / min-p only, temperature-only) and rows with
// top_k > 1024 additionally keep their scaled logits in the workspace and are
// finished from there (several passes, served mostly by L2/MALL).
//
// All arithmetic that decides a token mirrors the reference bit for bit:
// IEEE f32 division and addition in the reference's order, no contraction
// (this file is built with -ffp-contract=off), and exact_expf() equal to
// host glibc expf.  Selections use integer radix histograms only, so results
// are deterministic run to run.
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <float.h>

#include "hi_rocm.h"
#include "exact_expf.h"
#include "sampler_internal.h"

namespace hi_rocm {

// --------------------------------------------------------------------------
// small helpers

__device__ __forceinline__ bool finitef_(float x) {
  return (__float_as_uint(x) & 0x7f800000u) != 0x7f800000u;
}

// Order-preserving unsigned key of a float (NaN never occurs here).
__device__ __forceinline__ uint32_t okey(float f) {
  uint32_t u = __float_as_uint(f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ float okey_inv(uint32_t k) {
  uint32_t u = (k & 0x80000000u) ? (k & 0x7fffffffu) : ~k;
  return __uint_as_float(u);
}

// Rust's f32::total_cmp as a signed key (gpu.rs:744).
__device__ __forceinline__ int32_t total_key(float f) {
  int32_t i = (int32_t)__float_as_uint(f);
  return i ^ (int32_t)(((uint32_t)(i >> 31)) >> 1);
}

// Candidate key: scaled-logit key high, inverted index low, so a larger
// 64-bit value ranks first (value desc, index asc).
__device__ __forceinline__ uint64_t cand_key(uint32_t key, uint32_t idx) {
  return ((uint64_t)key << 32) | (uint64_t)(0xffffffffu - idx);
}
__device__ __forceinline__ uint32_t cand_idx(uint64_t c) { return 0xffffffffu - (uint32_t)c; }
__device__ __forceinline__ uint32_t cand_skey(uint64_t c) { return (uint32_t)(c >> 32); }

// Rank key of the reference order (weight desc by total_cmp, index asc);
// weights are >= +0 so their bits order like the floats.
__device__ __forceinline__ uint64_t rank_key(float w, uint32_t idx) {
  return ((uint64_t)__float_as_uint(w) << 32) | (uint64_t)(0xffffffffu - idx);
}

__device__ __forceinline__ float bf16_to_f32(uint16_t h) { return __uint_as_float((uint32_t)h << 16); }

// ---- parameters ----------------------------------------------------------

__device__ RowCfg load_cfg(const ParamsView& pv, int row, int V, int n_lp, int need_lse) {
  RowCfg c;
  c.min_p = 0.f; c.rep = 1.f; c.freq = 0.f; c.pres = 0.f; c.eos = 0u; c.flags = 0u;
  if (pv.mode == kParamsRows) {
    const hi_rocm_row_params p = pv.rows[row];
    c.T = p.temperature; c.top_p = p.top_p; c.min_p = p.min_p;
    c.rep = p.repetition_penalty; c.freq = p.frequency_penalty; c.pres = p.presence_penalty;
    c.top_k = p.top_k; c.eos = p.eos_id; c.flags = p.flags;
  } else if (pv.mode == kParamsSoA) {
    c.T = pv.temps[row]; c.top_p = pv.top_ps[row]; c.top_k = pv.top_ks[row];
  } else {
    c.T = pv.T; c.top_p = pv.top_p; c.top_k = pv.top_k;
  }
  const bool greedy = !(finitef_(c.T) && c.T > 0.f);
  const bool minp_on = finitef_(c.min_p) && c.min_p > 0.f;
  // gpu.rs:731-738, extended with min_p.
  const bool ranked = !greedy && ((finitef_(c.top_p) && c.top_p < 1.f) || c.top_k > 0 || minp_on);
  c.cls = greedy ? kGreedy : (ranked ? (c.top_k > 0 ? kTopK : kTopP) : kTempOnly);
  c.k_eff = c.cls == kTopK ? min(c.top_k, V) : 0;
  c.t_eff = greedy ? 1.f : c.T;
  c.cutoff = finitef_(c.top_p) ? (c.top_p < 0.f ? 0.f : (c.top_p > 1.f ? 1.f : c.top_p)) : 1.f;
  c.min_p = minp_on ? fminf(c.min_p, 1.f) : 0.f;
  c.rep_on = finitef_(c.rep) && c.rep > 0.f && fabsf(c.rep - 1.f) > FLT_EPSILON;
  c.freq = finitef_(c.freq) ? c.freq : 0.f;
  c.pres = finitef_(c.pres) ? c.pres : 0.f;
  c.wide = c.cls == kTopK && c.k_eff > kFast;
  c.k_sel = (c.cls == kTopK && !c.wide) ? max(c.k_eff, n_lp) : n_lp;
  // Logprobs need the normaliser to ~1e-7 relative: the largest terms are
  // summed in double from the candidates, so every chunk keeps a few.
  if (need_lse) c.k_sel = max(c.k_sel, kLseTop);
  if (c.k_sel > V) c.k_sel = V;
  c.store_s = c.cls == kTopP || c.cls == kTempOnly || c.wide;
  return c;
}

__device__ __forceinline__ float row_uniform(const ParamsView& pv, int row) {
  return pv.uniforms ? pv.uniforms[row] : pv.uniform_value;
}

// Stage 2 and 3 of the processed logit (the mask is applied by the caller):
// repetition penalty per occurrence (crates/hi-mlx/src/generate.rs:60-70),
// then frequency and presence penalties as separate f32 roundings.
__device__ __forceinline__ float apply_penalties(float l, uint32_t cnt, const RowCfg& c) {
  if (cnt == 0u) return l;
  if (c.rep_on) {
    const uint32_t reps = (c.flags & HI_ROCM_FLAG_REP_ONCE) ? 1u : cnt;
    for (uint32_t r = 0; r < reps; ++r) l = l < 0.f ? l * c.rep : l / c.rep;
  }
  const float fc = c.freq * (float)cnt;
  l = l - fc;
  l = l - c.pres;
  return l;
}

// ---- block-level reductions ------------------------------------------------

template <int NT>
__device__ __forceinline__ uint32_t block_sum_u32(uint32_t v, uint32_t* red) {
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  __syncthreads();
  if (lane == 0) red[wid] = v;
  __syncthreads();
  uint32_t s = 0;
  for (int i = 0; i < NT / 64; ++i) s += red[i];
  return s;
}

template <int NT>
__device__ __forceinline__ float block_sum_f32(float v, float* red) {
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  __syncthreads();
  if (lane == 0) red[wid] = v;
  __syncthreads();
  float s = 0.f;
  for (int i = 0; i < NT / 64; ++i) s += red[i];
  return s;
}

template <int NT>
__device__ __forceinline__ double block_sum_f64(double v, double* red) {
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  __syncthreads();
  if (lane == 0) red[wid] = v;
  __syncthreads();
  double s = 0.0;
  for (int i = 0; i < NT / 64; ++i) s += red[i];
  return s;
}

template <int NT>
__device__ __forceinline__ uint32_t block_max_u32(uint32_t v, uint32_t* red) {
  for (int o = 32; o > 0; o >>= 1) v = max(v, (uint32_t)__shfl_xor(v, o, 64));
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  __syncthreads();
  if (lane == 0) red[wid] = v;
  __syncthreads();
  uint32_t s = 0;
  for (int i = 0; i < NT / 64; ++i) s = max(s, red[i]);
  return s;
}

template <int NT>
__device__ __forceinline__ uint64_t block_min_u64(uint64_t v, uint64_t* red) {
  for (int o = 32; o > 0; o >>= 1) {
    const uint64_t t = ((uint64_t)(uint32_t)__shfl_xor((int)(uint32_t)(v >> 32), o, 64) << 32) |
                       (uint64_t)(uint32_t)__shfl_xor((int)(uint32_t)v, o, 64);
    if (t < v) v = t;
  }
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  __syncthreads();
  if (lane == 0) red[wid] = v;
  __syncthreads();
  uint64_t s = red[0];
  for (int i = 1; i < NT / 64; ++i) s = red[i] < s ? red[i] : s;
  return s;
}

// Exclusive prefix sum over the block in thread order; *total gets the sum.
template <int NT>
__device__ __forceinline__ uint32_t block_excl_scan_u32(uint32_t v, uint32_t* red, uint32_t* total) {
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  uint32_t inc = v;
  for (int o = 1; o < 64; o <<= 1) {
    uint32_t t = __shfl_up(inc, o, 64);
    if (lane >= o) inc += t;
  }
  __syncthreads();
  if (lane == 63) red[wid] = inc;
  __syncthreads();
  uint32_t before = 0, tot = 0;
  for (int i = 0; i < NT / 64; ++i) {
    if (i < wid) before += red[i];
    tot += red[i];
  }
  *total = tot;
  return before + inc - v;
}

// Chunk / row statistics merge (associative, order independent).
__device__ __forceinline__ void stat_merge(ChunkStat& a, const ChunkStat& b) {
  a.max_s = fmaxf(a.max_s, b.max_s);
  if (b.am_ieee_i != 0xffffffffu &&
      (a.am_ieee_i == 0xffffffffu || b.am_ieee_v > a.am_ieee_v ||
       (b.am_ieee_v == a.am_ieee_v && b.am_ieee_i < a.am_ieee_i))) {
    a.am_ieee_v = b.am_ieee_v; a.am_ieee_i = b.am_ieee_i;
  }
  if (b.am_tot_i != 0xffffffffu &&
      (a.am_tot_i == 0xffffffffu || b.am_tot_k > a.am_tot_k ||
       (b.am_tot_k == a.am_tot_k && b.am_tot_i < a.am_tot_i))) {
    a.am_tot_k = b.am_tot_k; a.am_tot_i = b.am_tot_i;
  }
  if (b.am_fin_i != 0xffffffffu) {
    bool take = a.am_fin_i == 0xffffffffu || b.am_fin_v > a.am_fin_v;
    if (!take && b.am_fin_v == a.am_fin_v) {
      const uint32_t ra = a.am_fin_i & 255u, rb = b.am_fin_i & 255u;
      take = rb < ra || (rb == ra && b.am_fin_i < a.am_fin_i);
    }
    if (take) { a.am_fin_v = b.am_fin_v; a.am_fin_i = b.am_fin_i; }
  }
  a.any_finite |= b.any_finite;
}

__device__ __forceinline__ void stat_init(ChunkStat& s) {
  s.max_s = -__builtin_inff();
  s.am_ieee_v = -__builtin_inff(); s.am_ieee_i = 0xffffffffu;
  s.am_tot_k = 0; s.am_tot_i = 0xffffffffu;
  s.am_fin_v = -__builtin_inff(); s.am_fin_i = 0xffffffffu;
  s.any_finite = 0u;
  s.lse_m = -__builtin_inff(); s.lse_sum = 0.f;
  s.n_cand = 0u; s.trunc = 0u; s.unkept_key = 0u; s.pad0 = 0u;
  s.min_kept = 0ull;
}

__device__ __forceinline__ ChunkStat stat_shfl_xor(const ChunkStat& s, int o) {
  ChunkStat r;
  r.max_s = __shfl_xor(s.max_s, o, 64);
  r.am_ieee_v = __shfl_xor(s.am_ieee_v, o, 64); r.am_ieee_i = __shfl_xor(s.am_ieee_i, o, 64);
  r.am_tot_k = __shfl_xor(s.am_tot_k, o, 64); r.am_tot_i = __shfl_xor(s.am_tot_i, o, 64);
  r.am_fin_v = __shfl_xor(s.am_fin_v, o, 64); r.am_fin_i = __shfl_xor(s.am_fin_i, o, 64);
  r.any_finite = __shfl_xor(s.any_finite, o, 64);
  r.lse_m = __shfl_xor(s.lse_m, o, 64); r.lse_sum = __shfl_xor(s.lse_sum, o, 64);
  r.n_cand = 0u; r.trunc = 0u; r.unkept_key = 0u; r.pad0 = 0u; r.min_kept = 0ull;
  return r;
}

// Reduce a per-thread ChunkStat over the block; the result is valid in all threads.
template <int NT>
__device__ __forceinline__ ChunkStat block_stat(ChunkStat s, ChunkStat* red) {
  for (int o = 32; o > 0; o >>= 1) {
    ChunkStat t = stat_shfl_xor(s, o);
    stat_merge(s, t);
  }
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  __syncthreads();
  if (lane == 0) red[wid] = s;
  __syncthreads();
  ChunkStat r = red[0];
  for (int i = 1; i < NT / 64; ++i) stat_merge(r, red[i]);
  return r;
}

// ---- element access -------------------------------------------------------

__device__ __forceinline__ float load_raw(const void* base, int dtype, int64_t off) {
  if (dtype == HI_ROCM_DTYPE_BF16) return bf16_to_f32(((const uint16_t*)base)[off]);
  return ((const float*)base)[off];
}

// Processed logit of a single token (mask + penalties), computed by the whole
// block: the count is reduced over the row's history.  Used off the hot path.
template <int NT>
__device__ float processed_single(const SampleArgs& a, int row, const RowCfg& c, uint32_t idx,
                                  uint32_t* red) {
  uint32_t cnt = 0;
  if (a.hoff) {
    const uint32_t h0 = a.hoff[row], h1 = a.hoff[row + 1];
    for (uint32_t h = h0 + threadIdx.x; h < h1; h += NT)
      if (a.hids[h] == idx) cnt += a.hcnt[h];
  }
  cnt = block_sum_u32<NT>(cnt, red);
  const int64_t rbase = (int64_t)row * a.row_stride;
  float l = load_raw(a.logits, a.dtype, rbase + idx);
  if (a.mask && !((a.mask[(int64_t)row * a.mask_words + (idx >> 5)] >> (idx & 31u)) & 1u))
    l = -__builtin_inff();
  return apply_penalties(l, cnt, c);
}

// ==========================================================================
// Kernel 1: streaming chunk scan
// ==========================================================================

struct ScanShared {
  uint32_t cnt[kChunk];   // history counts of the chunk (32 KB)
  uint32_t key[kChunk];   // scaled-logit keys of the chunk (32 KB)
  uint32_t hist[4096];    // radix histogram (16 KB)
  ChunkStat red[kScanThreads / 64];
  uint32_t redu[kScanThreads / 64];
  uint64_t red64[kScanThreads / 64];
  float redf[kScanThreads / 64];
  uint32_t sel_digit, sel_above, sel_cnt, counter;
};

__global__ void __launch_bounds__(kScanThreads) scan_chunks_kernel(SampleArgs a) {
  __shared__ ScanShared sh;
  const int row = blockIdx.y;
  const int chunk = blockIdx.x;
  const int tid = threadIdx.x;
  const int V = a.V;
  const int c0 = chunk * kChunk;
  const int c1 = min(c0 + kChunk, V);
  const int len = c1 - c0;
  const RowCfg cfg = load_cfg(a.pv, row, V, a.n_lp, a.need_lse);

  // History counts for this chunk, in LDS.
  bool pen = false;
  uint32_t h0 = 0, h1 = 0;
  if (a.hoff) { h0 = a.hoff[row]; h1 = a.hoff[row + 1]; pen = h1 > h0; }
  if (pen) {
    for (int i = tid; i < kChunk; i += kScanThreads) sh.cnt[i] = 0u;
    __syncthreads();
    for (uint32_t h = h0 + tid; h < h1; h += kScanThreads) {
      const uint32_t id = a.hids[h];
      if (id >= (uint32_t)c0 && id < (uint32_t)c1) atomicAdd(&sh.cnt[id - c0], a.hcnt[h]);
    }
    __syncthreads();
  }

  const int64_t rbase = (int64_t)row * a.row_stride;
  const uint32_t* mrow = a.mask ? a.mask + (int64_t)row * a.mask_words : nullptr;
  const bool need_keys = cfg.k_sel > 0;
  float* srow = cfg.store_s ? a.ws_s + (int64_t)row * V : nullptr;

  ChunkStat st;
  stat_init(st);

  #pragma unroll 1
  for (int j = 0; j < kScanVec; ++j) {
    const int e0 = c0 + (j * kScanThreads + tid) * 4;
    if (e0 >= c1) break;
    float raw[4];
    if (a.vec_ok && e0 + 3 < c1) {
      if (a.dtype == HI_ROCM_DTYPE_BF16) {
        const uint2 v = *(const uint2*)((const uint16_t*)a.logits + rbase + e0);
        raw[0] = __uint_as_float(v.x << 16); raw[1] = __uint_as_float(v.x & 0xffff0000u);
        raw[2] = __uint_as_float(v.y << 16); raw[3] = __uint_as_float(v.y & 0xffff0000u);
      } else {
        const float4 v = *(const float4*)((const float*)a.logits + rbase + e0);
        raw[0] = v.x; raw[1] = v.y; raw[2] = v.z; raw[3] = v.w;
      }
    } else {
      #pragma unroll
      for (int q = 0; q < 4; ++q) raw[q] = (e0 + q < c1) ? load_raw(a.logits, a.dtype, rbase + e0 + q) : 0.f;
    }
    const uint32_t mword = mrow ? mrow[e0 >> 5] : 0xffffffffu;
    float sv[4];
    #pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int e = e0 + q;
      if (e >= c1) { sv[q] = -__builtin_inff(); continue; }
      float l = raw[q];
      if (!((mword >> (e & 31)) & 1u)) l = -__builtin_inff();
      if (pen) l = apply_penalties(l, sh.cnt[e - c0], cfg);
      const bool fin = finitef_(l);
      const float s = fin ? l / cfg.t_eff : -__builtin_inff();
      sv[q] = s;
      st.max_s = fmaxf(st.max_s, s);
      if (l > st.am_ieee_v) { st.am_ieee_v = l; st.am_ieee_i = (uint32_t)e; }
      const int32_t tk = total_key(l);
      if (st.am_tot_i == 0xffffffffu || tk > st.am_tot_k) { st.am_tot_k = tk; st.am_tot_i = (uint32_t)e; }
      if (fin) {
        st.any_finite = 1u;
        if (st.am_fin_i == 0xffffffffu || l > st.am_fin_v ||
            (l == st.am_fin_v && ((uint32_t)e & 255u) < (st.am_fin_i & 255u))) {
          st.am_fin_v = l; st.am_fin_i = (uint32_t)e;
        }
      }
      if (need_keys) sh.key[e - c0] = okey(s);
    }
    if (srow) {
      if (e0 + 3 < c1 && (V & 3) == 0) {
        *(float4*)(srow + e0) = make_float4(sv[0], sv[1], sv[2], sv[3]);
      } else {
        for (int q = 0; q < 4; ++q) if (e0 + q < c1) srow[e0 + q] = sv[q];
      }
    }
  }

  ChunkStat bs = block_stat<kScanThreads>(st, sh.red);

  // Exact top-k' of the chunk by (scaled logit desc, index asc).
  uint64_t* cand = a.cand + ((int64_t)row * a.n_chunks + chunk) * kFast;
  if (need_keys) {
    __syncthreads();
    const int k = cfg.k_sel;
    if (len <= k) {
      for (int i = tid; i < len; i += kScanThreads) cand[i] = cand_key(sh.key[i], (uint32_t)(c0 + i));
      bs.n_cand = (uint32_t)len; bs.trunc = 0u;
    } else {
      // 48-bit composite: key << 16 | (0xffff - local index); unique per item.
      uint64_t prefix = 0;
      uint32_t remaining = (uint32_t)k;
      for (int pass = 0; pass < 4; ++pass) {
        const int shift = 36 - 12 * pass;
        for (int b = tid; b < 4096; b += kScanThreads) sh.hist[b] = 0u;
        __syncthreads();
        const uint64_t hi_pref = prefix >> (shift + 12);
        for (int i = tid; i < len; i += kScanThreads) {
          const uint64_t comp = ((uint64_t)sh.key[i] << 16) | (uint64_t)(0xffffu - (uint32_t)i);
          if ((comp >> (shift + 12)) == hi_pref) atomicAdd(&sh.hist[(comp >> shift) & 4095u], 1u);
        }
        __syncthreads();
        // thread t owns bins 4095-16t down to 4080-16t
        uint32_t loc[16];
        uint32_t lsum = 0;
        #pragma unroll
        for (int q = 0; q < 16; ++q) { loc[q] = sh.hist[4095 - 16 * tid - q]; lsum += loc[q]; }
        uint32_t tot;
        const uint32_t above = block_excl_scan_u32<kScanThreads>(lsum, sh.redu, &tot);
        if (above < remaining && remaining <= above + lsum) {
          uint32_t acc = above;
          for (int q = 0; q < 16; ++q) {
            if (remaining <= acc + loc[q]) {
              sh.sel_digit = 4095u - 16u * tid - q; sh.sel_above = acc; sh.sel_cnt = loc[q];
              break;
            }
            acc += loc[q];
          }
        }
        __syncthreads();
        prefix |= (uint64_t)sh.sel_digit << shift;
        remaining -= sh.sel_above;
        const bool done = sh.sel_cnt == remaining;
        __syncthreads();
        if (done) break;
      }
      const uint64_t thr = prefix;
      if (tid == 0) sh.counter = 0u;
      __syncthreads();
      uint32_t unkept = 0u;
      uint64_t minkept = ~0ull;
      float rest = 0.f;  // sum of exp(s - chunk max) over elements not kept
      const bool rest_on = a.need_lse && finitef_(bs.max_s);
      for (int i = tid; i < len; i += kScanThreads) {
        const uint32_t kk = sh.key[i];
        const uint64_t comp = ((uint64_t)kk << 16) | (uint64_t)(0xffffu - (uint32_t)i);
        if (comp >= thr) {
          const uint32_t pos = atomicAdd(&sh.counter, 1u);
          const uint64_t ck = cand_key(kk, (uint32_t)(c0 + i));
          if (pos < (uint32_t)kFast) cand[pos] = ck;
          if (ck < minkept) minkept = ck;
        } else {
          unkept = max(unkept, kk);
          if (rest_on) rest += __expf(okey_inv(kk) - bs.max_s);
        }
      }
      bs.lse_m = bs.max_s;
      bs.lse_sum = block_sum_f32<kScanThreads>(rest, sh.redf);
      const uint64_t mk = block_min_u64<kScanThreads>(minkept, sh.red64);
      const uint32_t um = block_max_u32<kScanThreads>(unkept, sh.redu);
      bs.n_cand = (uint32_t)k;
      bs.trunc = 1u;
      bs.unkept_key = um;
      bs.min_kept = mk;
    }
  }
  if (tid == 0) a.stats[(int64_t)row * a.n_chunks + chunk] = bs;
}

// ==========================================================================
// Kernel 2: per-row finish
// ==========================================================================

constexpr int kFinBuf = 8192;  // u64 LDS entries

struct FinShared {
  uint64_t buf[kFinBuf];       // 64 KB: candidates / rank keys / tiles
  uint32_t hist[4096];         // 16 KB
  uint64_t mass[2048];         // 16 KB (top-p path)
  uint32_t aux[2048];          //  8 KB (fill counters, per-thread sums)
  float fa[kFast];             //  4 KB: weights in rank order
  float fb[kFast];             //  4 KB: q = w / total
  uint32_t pay[kFast];         //  4 KB: scaled-logit keys riding with sh.buf
  ChunkStat red[kFinThreads / 64];
  uint32_t redu[kFinThreads / 64];
  double redd[kFinThreads / 64];
  uint32_t sel_digit, sel_above, sel_cnt, counter, n_ext, token, flag;
  float fval0, fval1;
  uint64_t thr;
};

// Top-`k` threshold over a set of unique 64-bit keys produced by get(j)
// for j < n (invalid slots return 0 and are never selected because k never
// exceeds the number of valid non-zero keys).  Returns T with exactly k keys
// >= T.  8-bit MSD radix descent with early exit.
template <typename Get>
__device__ uint64_t block_select64(FinShared& sh, int n, uint32_t k, Get get) {
  const int tid = threadIdx.x;
  uint64_t prefix = 0;
  uint32_t remaining = k;
  for (int pass = 0; pass < 8; ++pass) {
    const int shift = 56 - 8 * pass;
    for (int b = tid; b < 256; b += kFinThreads) sh.hist[b] = 0u;
    __syncthreads();
    for (int j = tid; j < n; j += kFinThreads) {
      bool valid;
      const uint64_t x = get(j, valid);
      if (!valid) continue;
      if (pass == 0 || (x >> (shift + 8)) == (prefix >> (shift + 8)))
        atomicAdd(&sh.hist[(x >> shift) & 255u], 1u);
    }
    __syncthreads();
    if (tid < 64) {
      // each lane of wave 0 owns 4 bins, highest bins first
      uint32_t loc[4], lsum = 0;
      #pragma unroll
      for (int q = 0; q < 4; ++q) { loc[q] = sh.hist[255 - 4 * tid - q]; lsum += loc[q]; }
      uint32_t inc = lsum;
      for (int o = 1; o < 64; o <<= 1) {
        const uint32_t t = __shfl_up(inc, o, 64);
        if (tid >= o) inc += t;
      }
      const uint32_t above = inc - lsum;
      if (above < remaining && remaining <= above + lsum) {
        uint32_t acc = above;
        for (int q = 0; q < 4; ++q) {
          if (remaining <= acc + loc[q]) {
            sh.sel_digit = 255u - 4u * tid - q; sh.sel_above = acc; sh.sel_cnt = loc[q];
            break;
          }
          acc += loc[q];
        }
      }
    }
    __syncthreads();
    prefix |= (uint64_t)sh.sel_digit << shift;
    remaining -= sh.sel_above;
    const bool done = sh.sel_cnt == remaining;
    __syncthreads();
    if (done) break;
  }
  return prefix;
}

// Bitonic sort of sh.buf[0..n2) in descending order, carrying sh.pay along
// (n2 a power of two <= kFast).
__device__ void lds_sort_desc(FinShared& sh, int n2) {
  for (int k = 2; k <= n2; k <<= 1) {
    for (int j = k >> 1; j > 0; j >>= 1) {
      for (int i = threadIdx.x; i < n2; i += kFinThreads) {
        const int ixj = i ^ j;
        if (ixj > i) {
          const uint64_t x = sh.buf[i], y = sh.buf[ixj];
          const bool desc = (i & k) == 0;
          if (desc ? (x < y) : (x > y)) {
            sh.buf[i] = y; sh.buf[ixj] = x;
            const uint32_t t = sh.pay[i]; sh.pay[i] = sh.pay[ixj]; sh.pay[ixj] = t;
          }
        }
      }
      __syncthreads();
    }
  }
}

// Bitonic sort of a global array (descending), used by the wide paths.
__device__ void global_sort_desc(uint64_t* g, int n2) {
  for (int k = 2; k <= n2; k <<= 1) {
    for (int j = k >> 1; j > 0; j >>= 1) {
      for (int i = threadIdx.x; i < n2; i += kFinThreads) {
        const int ixj = i ^ j;
        if (ixj > i) {
          const uint64_t x = g[i], y = g[ixj];
          const bool desc = (i & k) == 0;
          if (desc ? (x < y) : (x > y)) { g[i] = y; g[ixj] = x; }
        }
      }
      __syncthreads();
    }
  }
}

__device__ __forceinline__ int next_pow2(int x) {
  int p = 1;
  while (p < x) p <<= 1;
  return p;
}

// Merge the chunk candidates of `row` into the exact first `kk` entries of
// the reference rank order (weight desc, index asc).  On return (all
// threads): sh.buf[0..kk) holds rank keys in order, sh.pay[0..kk) the
// matching scaled-logit keys, and the function returns kk (0 if the row max
// is not finite).  M is the row max of s.
__device__ int rank_candidates(FinShared& sh, const SampleArgs& a, int row, const RowCfg& cfg,
                               int kk_req, float M) {
  const int tid = threadIdx.x;
  const int nch = a.n_chunks;
  const ChunkStat* stats = a.stats + (int64_t)row * nch;
  const uint64_t* cand = a.cand + (int64_t)row * nch * kFast;
  if (!finitef_(M) || kk_req <= 0) return 0;
  int n_total = 0;
  for (int c = 0; c < nch; ++c) n_total += (int)stats[c].n_cand;
  const int kk = min(kk_req, n_total);
  // 1. select top-kk candidates by (key desc, index asc)
  const int span = nch * kFast;
  auto get_cand = [&](int j, bool& valid) -> uint64_t {
    const int c = j / kFast, s = j - c * kFast;
    valid = (uint32_t)s < stats[c].n_cand;
    return valid ? cand[j] : 0ull;
  };
  uint64_t thr = 0;
  if (kk < n_total) thr = block_select64(sh, span, (uint32_t)kk, get_cand);
  if (tid == 0) sh.counter = 0u;
  __syncthreads();
  for (int j = tid; j < span; j += kFinThreads) {
    bool valid;
    const uint64_t x = get_cand(j, valid);
    if (valid && x >= thr) {
      const uint32_t p = atomicAdd(&sh.counter, 1u);
      if (p < (uint32_t)kFast) sh.buf[p] = x;
    }
  }
  __syncthreads();
  // 2. weights; the smallest selected weight (the kk-th) is w_b
  uint32_t wmin_bits = 0xffffffffu;
  for (int i = tid; i < kk; i += kFinThreads) {
    const uint64_t x = sh.buf[i];
    const float s = okey_inv(cand_skey(x));
    const float w = exact_expf(s - M);
    const uint32_t idx = cand_idx(x);
    sh.buf[i] = rank_key(w, idx);
    sh.pay[i] = cand_skey(x);
    wmin_bits = min(wmin_bits, __float_as_uint(w));
  }
  // block min via max of complement
  const uint32_t wb_bits = ~block_max_u32<kFinThreads>(~wmin_bits, sh.redu);
  const float w_b = __uint_as_float(wb_bits);
  // 3. tie extension: elements outside the selection with the same weight
  if (tid == 0) sh.n_ext = 0u;
  __syncthreads();
  uint64_t* ext = a.ws_list + (int64_t)row * a.list_stride;
  uint32_t* ext_aux = (uint32_t*)(a.ws_w + (int64_t)row * a.V);
  const int64_t ext_cap = a.V;
  if (w_b > 0.f) {
    // (a) candidates not selected
    if (kk < n_total) {
      for (int j = tid; j < span; j += kFinThreads) {
        bool valid;
        const uint64_t x = get_cand(j, valid);
        if (!valid || x >= thr) continue;
        const float w = exact_expf(okey_inv(cand_skey(x)) - M);
        if (w == w_b) {
          const uint32_t p = atomicAdd(&sh.n_ext, 1u);
          if (p < ext_cap) { ext[p] = rank_key(w, cand_idx(x)); ext_aux[p] = cand_skey(x); }
        }
      }
    }
    // (b) elements a chunk did not keep
    for (int c = 0; c < nch; ++c) {
      const ChunkStat cs = stats[c];
      if (!cs.trunc) continue;
      if (exact_expf(okey_inv(cs.unkept_key) - M) != w_b) continue;
      // Recompute the chunk's scaled logits (rare path).
      const int c0 = c * kChunk, c1 = min(c0 + kChunk, a.V);
      uint32_t* cnt = (uint32_t*)sh.hist;  // 4096 u32 reused as two halves below
      // counts for the chunk, two 4096-element halves
      for (int half = 0; half < 2; ++half) {
        const int b0 = c0 + half * 4096, b1 = min(b0 + 4096, c1);
        if (b0 >= b1) break;
        __syncthreads();
        for (int i = tid; i < 4096; i += kFinThreads) cnt[i] = 0u;
        __syncthreads();
        if (a.hoff) {
          const uint32_t h0 = a.hoff[row], h1 = a.hoff[row + 1];
          for (uint32_t h = h0 + tid; h < h1; h += kFinThreads) {
            const uint32_t id = a.hids[h];
            if (id >= (uint32_t)b0 && id < (uint32_t)b1) atomicAdd(&cnt[id - b0], a.hcnt[h]);
          }
        }
        __syncthreads();
        const int64_t rbase = (int64_t)row * a.row_stride;
        for (int e = b0 + tid; e < b1; e += kFinThreads) {
          float l = load_raw(a.logits, a.dtype, rbase + e);
          if (a.mask && !((a.mask[(int64_t)row * a.mask_words + (e >> 5)] >> (e & 31)) & 1u))
            l = -__builtin_inff();
          l = apply_penalties(l, cnt[e - b0], cfg);
          const float s = finitef_(l) ? l / cfg.t_eff : -__builtin_inff();
          const uint64_t ck = cand_key(okey(s), (uint32_t)e);
          if (ck >= cs.min_kept) continue;  // kept by the chunk: already a candidate
          const float w = exact_expf(s - M);
          if (w == w_b) {
            const uint32_t p = atomicAdd(&sh.n_ext, 1u);
            if (p < ext_cap) { ext[p] = rank_key(w, (uint32_t)e); ext_aux[p] = okey(s); }
          }
        }
      }
      __syncthreads();
    }
  }
  __syncthreads();
  const uint32_t n_ext = min(sh.n_ext, (uint32_t)(ext_cap - kk));
  if (n_ext > 0) {
    // Union of selection and extension, then the top-kk by rank key.
    const int n_all = kk + (int)n_ext;
    // move the selection behind the extension in the global list
    for (int i = tid; i < kk; i += kFinThreads) { ext[n_ext + i] = sh.buf[i]; ext_aux[n_ext + i] = sh.pay[i]; }
    __syncthreads();
    auto get_ext = [&](int j, bool& valid) -> uint64_t { valid = true; return ext[j]; };
    const uint64_t t2 = block_select64(sh, n_all, (uint32_t)kk, get_ext);
    if (tid == 0) sh.counter = 0u;
    __syncthreads();
    for (int j = tid; j < n_all; j += kFinThreads) {
      const uint64_t x = ext[j];
      if (x >= t2) {
        const uint32_t p = atomicAdd(&sh.counter, 1u);
        if (p < (uint32_t)kFast) {
          sh.buf[p] = x;
          sh.pay[p] = ext_aux[j];
        }
      }
    }
    __syncthreads();
  }
  // 4. sort the kk rank keys (pad with 0, which sorts last)
  const int n2 = next_pow2(kk);
  for (int i = kk + tid; i < n2; i += kFinThreads) sh.buf[i] = 0ull;
  __syncthreads();
  lds_sort_desc(sh, n2);
  return kk;
}

__device__ __forceinline__ float clamp_uniform(float u) {
  // gpu.rs:882-886
  return finitef_(u) ? (u < 0.f ? 0.f : (u > 0.99999994f ? 0.99999994f : u)) : 0.f;
}

// Reference steps 7-10 (gpu.rs:831-899) over the first `k` entries of the rank
// order held in sh.buf (top-k rows).  Returns the token or 0xffffffff for
// "fall back to argmax_host".
__device__ uint32_t draw_topk(FinShared& sh, const RowCfg& cfg, int k, float u) {
  const int tid = threadIdx.x;
  for (int i = tid; i < k; i += kFinThreads) {
    const float w = __uint_as_float((uint32_t)(sh.buf[i] >> 32));
    sh.fa[i] = (w < cfg.min_p) ? 0.f : w;
  }
  __syncthreads();
  if (tid == 0) {
    float total = -0.0f;
    for (int i = 0; i < k; ++i) total += sh.fa[i];
    sh.fval0 = total;
  }
  __syncthreads();
  const float total = sh.fval0;
  if (total <= 0.f || !finitef_(total)) return 0xffffffffu;
  for (int i = tid; i < k; i += kFinThreads) sh.fb[i] = sh.fa[i] / total;
  __syncthreads();
  if (tid == 0) {
    float cum_p = 0.f;
    int m_end = 0;  // candidates are entries [0, m_end) with positive weight
    bool any = false;
    for (int i = 0; i < k; ++i) {
      if (sh.fa[i] <= 0.f) continue;
      any = true;
      m_end = i + 1;
      cum_p += sh.fb[i];
      if (cfg.cutoff < 1.f && cum_p >= cfg.cutoff) break;
    }
    uint32_t tok = 0xffffffffu;
    if (any) {
      float ct = -0.0f;
      for (int i = 0; i < m_end; ++i) if (sh.fa[i] > 0.f) ct += sh.fa[i];
      if (ct > 0.f && finitef_(ct)) {
        const float target = clamp_uniform(u) * ct;
        float cum = 0.f;
        int last = -1, pick = -1;
        for (int i = 0; i < m_end; ++i) {
          if (sh.fa[i] <= 0.f) continue;
          last = i;
          cum += sh.fa[i];
          if (target < cum) { pick = i; break; }
        }
        if (pick < 0) pick = last;
        tok = 0xffffffffu - (uint32_t)sh.buf[pick];
      }
    }
    sh.token = tok;
  }
  __syncthreads();
  return sh.token;
}

// Serial f32 fold of a global float array in index order (Rust's Sum: a
// fold from -0.0), by thread 0, staged through LDS tiles.  Result valid in
// all threads.
__device__ float fold_global(FinShared& sh, const float* x, int n) {
  float* tile = (float*)sh.buf;
  const int T = kFinBuf * 2;  // floats per tile
  float acc = -0.0f;          // meaningful in thread 0 only
  for (int t0 = 0; t0 < n; t0 += T) {
    const int m = min(T, n - t0);
    __syncthreads();
    for (int i = threadIdx.x; i < m; i += kFinThreads) tile[i] = x[t0 + i];
    __syncthreads();
    if (threadIdx.x == 0)
      for (int i = 0; i < m; ++i) acc += tile[i];
  }
  __syncthreads();
  if (threadIdx.x == 0) sh.fval0 = acc;
  __syncthreads();
  const float r = sh.fval0;
  __syncthreads();
  return r;
}

// Rows without top-k (or with top_k > 1024): the whole distribution is
// re-read from the workspace (ws_s holds the scaled logits).
__device__ uint32_t draw_wide(FinShared& sh, const SampleArgs& a, int row, const RowCfg& cfg,
                              float M, float u) {
  const int tid = threadIdx.x;
  const int V = a.V;
  const float* srow = a.ws_s + (int64_t)row * V;
  float* wrow = a.ws_w + (int64_t)row * V;
  uint64_t* list = a.ws_list + (int64_t)row * a.list_stride;
  // weights (min-p applied), histogram of positive weights over 2048 bins
  for (int b = tid; b < 2048; b += kFinThreads) { sh.hist[b] = 0u; sh.mass[b] = 0ull; }
  __syncthreads();
  for (int i = tid; i < V; i += kFinThreads) {
    float w = exact_expf(srow[i] - M);
    if (w < cfg.min_p) w = 0.f;
    wrow[i] = w;
    if (w > 0.f) {
      const uint32_t b = __float_as_uint(w) >> 19;
      atomicAdd(&sh.hist[b], 1u);
      atomicAdd((unsigned long long*)&sh.mass[b], (unsigned long long)((double)w * 1099511627776.0));
    }
  }
  __syncthreads();
  const bool wide_k = cfg.cls == kTopK;
  float total = 0.f;
  if (!wide_k) {
    total = fold_global(sh, wrow, V);  // gpu.rs:837: vocab-order sum
    if (total <= 0.f || !finitef_(total)) return 0xffffffffu;
  }
  // boundary bin of the superset
  if (tid == 0) {
    uint64_t all_mass = 0;
    uint32_t all_cnt = 0;
    for (int b = 0; b < 2048; ++b) { all_mass += sh.mass[b]; all_cnt += sh.hist[b]; }
    int bstar = 0;
    if (wide_k) {
      uint32_t c = 0;
      for (int b = 2047; b >= 0; --b) { c += sh.hist[b]; if (c >= (uint32_t)cfg.k_eff) { bstar = b; break; } }
    } else if (cfg.cutoff < 1.f) {
      const double need = fmin(1.0, (double)cfg.cutoff + 0.02) * (double)all_mass;
      uint64_t c = 0;
      for (int b = 2047; b >= 0; --b) { c += sh.mass[b]; if ((double)c >= need) { bstar = b; break; } }
    }
    sh.flag = (uint32_t)bstar;
    (void)all_cnt;
  }
  __syncthreads();
  int bstar = (int)sh.flag;
  uint32_t tok = 0xffffffffu;
  for (int attempt = 0; attempt < 2; ++attempt) {
    // offsets of bins >= bstar in descending bin order
    __syncthreads();
    if (tid == 0) {
      uint32_t off = 0;
      for (int b = 2047; b >= 0; --b) {
        sh.aux[b] = off;
        if (b >= bstar) off += sh.hist[b];
      }
      sh.counter = off;
    }
    __syncthreads();
    const int n_sup = (int)sh.counter;
    for (int i = tid; i < V; i += kFinThreads) {
      const float w = wrow[i];
      if (w > 0.f) {
        const int b = (int)(__float_as_uint(w) >> 19);
        if (b >= bstar) list[atomicAdd(&sh.aux[b], 1u)] = rank_key(w, (uint32_t)i);
      }
    }
    __syncthreads();
    const int n2 = next_pow2(max(n_sup, 1));
    for (int i = n_sup + tid; i < n2; i += kFinThreads) list[i] = 0ull;
    __syncthreads();
    global_sort_desc(list, n2);
    // serial walk over the sorted superset (thread 0), tiles through LDS
    if (wide_k) {
      const int k = min(cfg.k_eff, n_sup);  // zero-weight entries add nothing
      if (tid == 0) {
        float t = -0.0f;
        for (int i = 0; i < k; ++i) t += __uint_as_float((uint32_t)(list[i] >> 32));
        sh.fval0 = t;
      }
      __syncthreads();
      total = sh.fval0;
      if (total <= 0.f || !finitef_(total)) return 0xffffffffu;
      if (tid == 0) {
        float cum_p = 0.f;
        int m_end = 0;
        for (int i = 0; i < k; ++i) {
          const float w = __uint_as_float((uint32_t)(list[i] >> 32));
          m_end = i + 1;
          cum_p += w / total;
          if (cfg.cutoff < 1.f && cum_p >= cfg.cutoff) break;
        }
        float ct = -0.0f;
        for (int i = 0; i < m_end; ++i) ct += __uint_as_float((uint32_t)(list[i] >> 32));
        uint32_t r = 0xffffffffu;
        if (m_end > 0 && ct > 0.f && finitef_(ct)) {
          const float target = clamp_uniform(u) * ct;
          float cum = 0.f;
          int pick = m_end - 1;
          for (int i = 0; i < m_end; ++i) {
            cum += __uint_as_float((uint32_t)(list[i] >> 32));
            if (target < cum) { pick = i; break; }
          }
          r = 0xffffffffu - (uint32_t)list[pick];
        }
        sh.token = r;
        sh.flag = 1u;
      }
      __syncthreads();
      return sh.token;
    }
    if (tid == 0) {
      float cum_p = 0.f;
      int m_end = 0;
      bool reached = false;
      for (int i = 0; i < n_sup; ++i) {
        const float w = __uint_as_float((uint32_t)(list[i] >> 32));
        m_end = i + 1;
        cum_p += w / total;
        if (cfg.cutoff < 1.f && cum_p >= cfg.cutoff) { reached = true; break; }
      }
      const bool complete = bstar == 0;
      if (!reached && !complete) {
        sh.flag = 0xffffffffu;  // superset too small: retry with every positive weight
      } else {
        float ct = -0.0f;
        for (int i = 0; i < m_end; ++i) ct += __uint_as_float((uint32_t)(list[i] >> 32));
        uint32_t r = 0xffffffffu;
        if (m_end > 0 && ct > 0.f && finitef_(ct)) {
          const float target = clamp_uniform(u) * ct;
          float cum = 0.f;
          int pick = m_end - 1;
          for (int i = 0; i < m_end; ++i) {
            cum += __uint_as_float((uint32_t)(list[i] >> 32));
            if (target < cum) { pick = i; break; }
          }
          r = 0xffffffffu - (uint32_t)list[pick];
        }
        sh.token = r;
        sh.flag = 1u;
      }
    }
    __syncthreads();
    if (sh.flag != 0xffffffffu) { tok = sh.token; break; }
    bstar = 0;
  }
  return tok;
}

// Temperature-only rows: kernels.cu:7803-7867 with the exact weight function.
__device__ uint32_t draw_temp_only(FinShared& sh, const SampleArgs& a, int row, float M, float u,
                                   uint32_t argmax_fin) {
  const int tid = threadIdx.x;
  const int V = a.V;
  const float* srow = a.ws_s + (int64_t)row * V;
  const int chunk = (V + 255) / 256;
  float* csum = sh.fa;       // 256 used
  float* prefix = sh.fb;     // 256 used
  if (tid < 256) {
    const int start = tid * chunk, end = min(start + chunk, V);
    float s = 0.f;
    for (int i = start; i < end; ++i) s += exact_expf(srow[i] - M);
    csum[tid] = s;
  }
  __syncthreads();
  if (tid == 0) {
    float acc = 0.f;
    for (int j = 0; j < 256; ++j) { prefix[j] = acc; acc += csum[j]; }
    sh.fval0 = acc;
    sh.token = 0xffffffffu;
  }
  __syncthreads();
  const float total = sh.fval0;
  if (total <= 0.f || !finitef_(total)) return argmax_fin;
  const float uu = finitef_(u) ? fminf(fmaxf(u, 0.f), 0.99999994f) : 0.f;
  const float target = uu * total;
  if (tid < 256) {
    const int start = tid * chunk, end = min(start + chunk, V);
    const float lo = prefix[tid];
    const float hi = lo + csum[tid];
    if (start < end && target >= lo && (target < hi || tid == 255)) {
      float cum = lo;
      int chosen = -1;
      for (int i = start; i < end; ++i) {
        const float w = exact_expf(srow[i] - M);
        if (w <= 0.f) continue;
        chosen = i;
        cum += w;
        if (target < cum) break;
      }
      if (chosen >= 0) atomicMin(&sh.token, (uint32_t)chosen);
    }
  }
  __syncthreads();
  return sh.token != 0xffffffffu ? sh.token : argmax_fin;
}

__global__ void __launch_bounds__(kFinThreads) finish_rows_kernel(SampleArgs a) {
  __shared__ FinShared sh;
  const int row = blockIdx.x;
  const int tid = threadIdx.x;
  const int V = a.V;
  const RowCfg cfg = load_cfg(a.pv, row, V, a.n_lp, a.need_lse);

  // Row statistics from the chunk statistics.
  ChunkStat st;
  stat_init(st);
  for (int c = tid; c < a.n_chunks; c += kFinThreads) stat_merge(st, a.stats[(int64_t)row * a.n_chunks + c]);
  const ChunkStat rs = block_stat<kFinThreads>(st, sh.red);
  const float M = rs.max_s;
  const uint32_t am_ieee = rs.am_ieee_i == 0xffffffffu ? 0u : rs.am_ieee_i;
  const uint32_t am_tot = rs.am_tot_i == 0xffffffffu ? 0u : rs.am_tot_i;
  const uint32_t am_fin = rs.am_fin_i == 0xffffffffu ? 0u : rs.am_fin_i;
  const float u = row_uniform(a.pv, row);

  const bool eos = a.mask && !rs.any_finite;
  uint32_t token;
  int ranked_k = 0;  // entries of sh.buf that are in rank order
  if (eos) {
    token = cfg.eos;
  } else if (cfg.cls == kGreedy) {
    token = a.pv.greedy_rule == kGreedyFiniteLane ? am_fin : am_ieee;
  } else if (cfg.cls == kTopK && !cfg.wide) {
    if (!finitef_(M)) {
      token = am_tot;
    } else {
      ranked_k = rank_candidates(sh, a, row, cfg, cfg.k_sel, M);
      token = draw_topk(sh, cfg, cfg.k_eff, u);
      if (token == 0xffffffffu) token = am_tot;
    }
  } else if (cfg.cls == kTempOnly) {
    token = finitef_(M) ? draw_temp_only(sh, a, row, M, u, am_fin) : am_fin;
  } else {
    if (!finitef_(M)) {
      token = am_tot;
    } else {
      token = draw_wide(sh, a, row, cfg, M, u);
      if (token == 0xffffffffu) token = am_tot;
    }
  }
  if (tid == 0) a.out_tokens[row] = token;

  // Logprobs of the processed distribution (extension).
  if (a.n_lp > 0 || a.out_token_lp) {
    __syncthreads();
    const int N = a.n_lp;
    if (eos || !finitef_(M)) {
      for (int j = tid; j < N; j += kFinThreads) {
        a.out_lp[(int64_t)row * N + j] = -__builtin_inff();
        a.out_lp_ids[(int64_t)row * N + j] = 0xffffffffu;
      }
      if (tid == 0 && a.out_token_lp) a.out_token_lp[row] = eos ? 0.f : -__builtin_inff();
      return;
    }
    if (N > 0 && ranked_k < N) ranked_k = rank_candidates(sh, a, row, cfg, N, M);
    // log of the normaliser relative to M (lse = M + log_sum): the kept
    // candidates of every chunk in double, the rest from each chunk's sum.
    double part = 0.0;
    {
      const int nch = a.n_chunks;
      const ChunkStat* stats = a.stats + (int64_t)row * nch;
      const uint64_t* cand = a.cand + (int64_t)row * nch * kFast;
      for (int c = 0; c < nch; ++c) {
        const uint32_t nc = stats[c].n_cand;
        for (uint32_t j = tid; j < nc; j += kFinThreads)
          part += exp((double)okey_inv(cand_skey(cand[(int64_t)c * kFast + j])) - (double)M);
      }
      for (int c = tid; c < nch; c += kFinThreads) {
        const ChunkStat cs = stats[c];
        if (cs.lse_sum > 0.f) part += (double)cs.lse_sum * exp((double)cs.lse_m - (double)M);
      }
    }
    const double log_sum = log(block_sum_f64<kFinThreads>(part, sh.redd));
    for (int j = tid; j < N; j += kFinThreads) {
      float lp = -__builtin_inff();
      uint32_t id = 0xffffffffu;
      if (j < ranked_k) {
        id = 0xffffffffu - (uint32_t)sh.buf[j];
        const float s = okey_inv(sh.pay[j]);
        lp = (float)(((double)s - (double)M) - log_sum);
      }
      a.out_lp_ids[(int64_t)row * N + j] = id;
      a.out_lp[(int64_t)row * N + j] = lp;
    }
    if (a.out_token_lp) {
      if (tid == 0) sh.flag = 0u;
      __syncthreads();
      for (int j = tid; j < ranked_k; j += kFinThreads) {
        if (0xffffffffu - (uint32_t)sh.buf[j] == token) { sh.flag = 1u; sh.fval1 = okey_inv(sh.pay[j]); }
      }
      __syncthreads();
      float s;
      if (sh.flag) {
        s = sh.fval1;
      } else {
        const float l = processed_single<kFinThreads>(a, row, cfg, token < (uint32_t)V ? token : 0u, sh.redu);
        s = finitef_(l) ? l / cfg.t_eff : -__builtin_inff();
      }
      if (tid == 0)
        a.out_token_lp[row] = token < (uint32_t)V ? (float)(((double)s - (double)M) - log_sum) : -__builtin_inff();
    }
  }
}

// ==========================================================================
// Argmax kernels for the reference's argmax launchers (no workspace)
// ==========================================================================

__global__ void __launch_bounds__(1024) argmax_rows_kernel(const float* logits, uint32_t* out,
                                                           int B, int64_t row_stride,
                                                           int64_t row_offset, int cols,
                                                           int vec_ok) {
  __shared__ float sv[16];
  __shared__ uint32_t si[16];
  const int row = blockIdx.x;
  const float* r = logits + row_offset + (int64_t)row * row_stride;
  float best = -__builtin_inff();
  uint32_t bi = 0xffffffffu;
  if (vec_ok) {
    const int n4 = cols >> 2;
    for (int i = threadIdx.x; i < n4; i += 1024) {
      const float4 v = ((const float4*)r)[i];
      const float x[4] = {v.x, v.y, v.z, v.w};
      #pragma unroll
      for (int q = 0; q < 4; ++q) if (x[q] > best) { best = x[q]; bi = (uint32_t)(4 * i + q); }
    }
    for (int i = 4 * n4 + threadIdx.x; i < cols; i += 1024)
      if (r[i] > best) { best = r[i]; bi = (uint32_t)i; }
  } else {
    for (int i = threadIdx.x; i < cols; i += 1024)
      if (r[i] > best) { best = r[i]; bi = (uint32_t)i; }
  }
  for (int o = 32; o > 0; o >>= 1) {
    const float ov = __shfl_xor(best, o, 64);
    const uint32_t oi = __shfl_xor(bi, o, 64);
    if (oi != 0xffffffffu && (bi == 0xffffffffu || ov > best || (ov == best && oi < bi))) { best = ov; bi = oi; }
  }
  if ((threadIdx.x & 63) == 0) { sv[threadIdx.x >> 6] = best; si[threadIdx.x >> 6] = bi; }
  __syncthreads();
  if (threadIdx.x == 0) {
    float b = sv[0];
    uint32_t i0 = si[0];
    for (int w = 1; w < 16; ++w) {
      if (si[w] != 0xffffffffu && (i0 == 0xffffffffu || sv[w] > b || (sv[w] == b && si[w] < i0))) { b = sv[w]; i0 = si[w]; }
    }
    out[row] = i0 == 0xffffffffu ? 0u : i0;
  }
}

// ==========================================================================
// Debug kernels
// ==========================================================================

__global__ void debug_expf_kernel(const float* x, float* y, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) y[i] = exact_expf(x[i]);
}

// Processed logits and per-chunk max of s (stats[.].max_s) for the debug export.
__global__ void __launch_bounds__(kScanThreads) debug_processed_kernel(SampleArgs a, float* out_proc) {
  __shared__ uint32_t cnt[kChunk];
  __shared__ ChunkStat red[kScanThreads / 64];
  const int row = blockIdx.y, chunk = blockIdx.x, tid = threadIdx.x;
  const int V = a.V, c0 = chunk * kChunk, c1 = min(c0 + kChunk, V);
  const RowCfg cfg = load_cfg(a.pv, row, V, 0, 0);
  bool pen = false;
  uint32_t h0 = 0, h1 = 0;
  if (a.hoff) { h0 = a.hoff[row]; h1 = a.hoff[row + 1]; pen = h1 > h0; }
  if (pen) {
    for (int i = tid; i < kChunk; i += kScanThreads) cnt[i] = 0u;
    __syncthreads();
    for (uint32_t h = h0 + tid; h < h1; h += kScanThreads) {
      const uint32_t id = a.hids[h];
      if (id >= (uint32_t)c0 && id < (uint32_t)c1) atomicAdd(&cnt[id - c0], a.hcnt[h]);
    }
    __syncthreads();
  }
  ChunkStat st;
  stat_init(st);
  const int64_t rbase = (int64_t)row * a.row_stride;
  for (int e = c0 + tid; e < c1; e += kScanThreads) {
    float l = load_raw(a.logits, a.dtype, rbase + e);
    if (a.mask && !((a.mask[(int64_t)row * a.mask_words + (e >> 5)] >> (e & 31)) & 1u)) l = -__builtin_inff();
    if (pen) l = apply_penalties(l, cnt[e - c0], cfg);
    out_proc[(int64_t)row * V + e] = l;
    const float s = finitef_(l) ? l / cfg.t_eff : -__builtin_inff();
    st.max_s = fmaxf(st.max_s, s);
  }
  const ChunkStat bs = block_stat<kScanThreads>(st, red);
  if (tid == 0) a.stats[(int64_t)row * a.n_chunks + chunk] = bs;
}

__global__ void __launch_bounds__(1024) debug_probs_kernel(SampleArgs a, const float* proc, float* out_probs) {
  __shared__ double dred[16];
  __shared__ float fred[16];
  const int row = blockIdx.x, tid = threadIdx.x, V = a.V;
  const RowCfg cfg = load_cfg(a.pv, row, V, 0, 0);
  float M = -__builtin_inff();
  for (int c = tid; c < a.n_chunks; c += 1024) M = fmaxf(M, a.stats[(int64_t)row * a.n_chunks + c].max_s);
  for (int o = 32; o > 0; o >>= 1) M = fmaxf(M, __shfl_xor(M, o, 64));
  if ((tid & 63) == 0) fred[tid >> 6] = M;
  __syncthreads();
  M = fred[0];
  for (int w = 1; w < 16; ++w) M = fmaxf(M, fred[w]);
  double sum = 0.0;
  const float* pr = proc + (int64_t)row * V;
  if (finitef_(M)) {
    for (int i = tid; i < V; i += 1024) {
      const float l = pr[i];
      const float s = finitef_(l) ? l / cfg.t_eff : -__builtin_inff();
      sum += exp((double)s - (double)M);
    }
  }
  for (int o = 32; o > 0; o >>= 1) sum += __shfl_xor(sum, o, 64);
  if ((tid & 63) == 0) dred[tid >> 6] = sum;
  __syncthreads();
  sum = 0.0;
  for (int w = 0; w < 16; ++w) sum += dred[w];
  for (int i = tid; i < V; i += 1024) {
    const float l = pr[i];
    const float s = finitef_(l) ? l / cfg.t_eff : -__builtin_inff();
    out_probs[(int64_t)row * V + i] = finitef_(M) ? (float)(exp((double)s - (double)M) / sum) : 0.f;
  }
}

// --------------------------------------------------------------------------
// launch wrappers (called from the host API)

hipError_t launch_sample(const SampleArgs& a, hipStream_t stream) {
  dim3 g1(a.n_chunks, a.B);
  hipLaunchKernelGGL(scan_chunks_kernel, g1, dim3(kScanThreads), 0, stream, a);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(finish_rows_kernel, dim3(a.B), dim3(kFinThreads), 0, stream, a);
  return hipGetLastError();
}

hipError_t launch_argmax(const float* logits, uint32_t* out, int B, int64_t row_stride,
                         int64_t row_offset, int cols, hipStream_t stream) {
  const int vec_ok = (((uintptr_t)(logits + row_offset) & 15u) == 0) && (row_stride % 4 == 0);
  hipLaunchKernelGGL(argmax_rows_kernel, dim3(B), dim3(1024), 0, stream, logits, out, B, row_stride,
                     row_offset, cols, vec_ok);
  return hipGetLastError();
}

hipError_t launch_debug_expf(const float* x, float* y, int64_t n, hipStream_t stream) {
  const int64_t blocks = (n + 255) / 256;
  hipLaunchKernelGGL(debug_expf_kernel, dim3((unsigned)blocks), dim3(256), 0, stream, x, y, n);
  return hipGetLastError();
}

hipError_t launch_debug_distribution(const SampleArgs& a, float* out_proc, float* out_probs,
                                     hipStream_t stream) {
  dim3 g1(a.n_chunks, a.B);
  hipLaunchKernelGGL(debug_processed_kernel, g1, dim3(kScanThreads), 0, stream, a, out_proc);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(debug_probs_kernel, dim3(a.B), dim3(1024), 0, stream, a, (const float*)out_proc, out_probs);
  return hipGetLastError();
}

}  // namespace hi_rocm
