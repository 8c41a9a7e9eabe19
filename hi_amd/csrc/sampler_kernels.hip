// hi-rocm batched token sampler: CDNA4 (gfx950) kernels.
//
// Two kernels per decode step.  Logits [B, V] stay in HBM; the scan grid is
// (chunks per row, B) workgroups of 256 threads (4 wave64s):
//
//   scan   every workgroup streams one chunk of one row exactly once with
//          128-bit loads, all issued before any use (4 KiB per wave in
//          flight; 4096-logit chunks, 1024 when the batch is small).  Per element: allowed-token mask, penalties from an LDS
//          count table built from the row's history, temperature.  The
//          workgroup then reduces its statistics (max, three argmax
//          variants) and selects the chunk's exact top-k' by (scaled logit
//          desc, index asc): a bound from the per-thread maxima pre-filters
//          the chunk to about 1.3 k' elements, and an 8-bit LDS radix
//          descent finishes the selection.
//   finish a second launch, one workgroup per row, merges the chunk
//          candidates, ranks them with the glibc-exact weight function and
//          runs the reference's sequential f32 folds and inverse-CDF draw
//          (crates/hi-cuda/src/gpu.rs:753-900).
//
// Rows without top-k (top-p / min-p only, temperature-only) and rows with
// top_k > 1024 also keep their scaled logits in the workspace; their finish
// re-reads the row from there (served mostly by L2 / MALL).
//
// Every operation that decides a token mirrors the reference bit for bit:
// IEEE f32 division and addition in the reference's order, no contraction
// (the library is built with -ffp-contract=off), and exact_expf() equal to
// host glibc expf.  Selections use integer histograms and prefix scans in a
// fixed order, so results are deterministic run to run.
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <float.h>
#include <stddef.h>

#include "hi_rocm.h"
#include "exact_expf.h"
#include "sampler_internal.h"

namespace hi_rocm {

constexpr int NT = kScanThreads;  // threads of the fused kernel
constexpr int kBuf = 1024;        // ranked entries held in LDS
constexpr int kGather = 4096;     // candidates of a row gathered into LDS
constexpr int kBufCap = 2048;     // running chunk candidates held in LDS
constexpr int kHashCap = 1024;    // distinct history tokens per chunk held in LDS
constexpr int kBins = 1024;       // weight histogram of the wide paths (w bits >> 20)

// --------------------------------------------------------------------------
// small helpers

__device__ __forceinline__ bool finitef_(float x) {
  return (__float_as_uint(x) & 0x7f800000u) != 0x7f800000u;
}

// Order-preserving unsigned key of a float (NaN never occurs here).
__device__ __forceinline__ uint32_t okey(float f) {
  const uint32_t u = __float_as_uint(f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ float okey_inv(uint32_t k) {
  const uint32_t u = (k & 0x80000000u) ? (k & 0x7fffffffu) : ~k;
  return __uint_as_float(u);
}

// Key of a processed logit: its order key, non-finite values as -inf
// (gpu.rs:767-777 maps them to -inf before ranking).
constexpr uint32_t kKeyNegInf = 0x007fffffu;  // okey(-inf)
__device__ __forceinline__ uint32_t lkey(float l) { return finitef_(l) ? okey(l) : kKeyNegInf; }

// Scaled logit s = l / t_eff of a key (gpu.rs:767-777); the key of -inf
// decodes to -inf and t_eff is positive, so no case needs a branch.
__device__ __forceinline__ float key_to_s(uint32_t key, float t_eff) {
  return okey_inv(key) / t_eff;
}

// Rust's f32::total_cmp as a signed key (gpu.rs:744).
__device__ __forceinline__ int32_t total_key(float f) {
  const int32_t i = (int32_t)__float_as_uint(f);
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
// weights are >= +0, so their bits order like the floats.
__device__ __forceinline__ uint64_t rank_key(float w, uint32_t idx) {
  return ((uint64_t)__float_as_uint(w) << 32) | (uint64_t)(0xffffffffu - idx);
}
__device__ __forceinline__ float rank_w(uint64_t r) { return __uint_as_float((uint32_t)(r >> 32)); }

// Chunk-local composite (48 bits): key << 16 | (0xffff - local index).
__device__ __forceinline__ uint64_t local_comp(uint32_t key, uint32_t li) {
  return ((uint64_t)key << 16) | (uint64_t)(0xffffu - li);
}

__device__ __forceinline__ float bf16_to_f32(uint16_t h) { return __uint_as_float((uint32_t)h << 16); }

__device__ __forceinline__ float clamp_uniform(float u) {
  // gpu.rs:882-886
  return finitef_(u) ? (u < 0.f ? 0.f : (u > 0.99999994f ? 0.99999994f : u)) : 0.f;
}

__device__ __forceinline__ int next_pow2(int x) {
  int p = 1;
  while (p < x) p <<= 1;
  return p;
}

// ---- parameters ----------------------------------------------------------

__device__ __forceinline__ RowCfg load_cfg(const ParamsView& pv, int row, int V, int n_lp, int need_lse) {
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
  c.wide = c.cls == kTopK && c.k_eff > kLeanK;
  c.k_sel = (c.cls == kTopK && !c.wide) ? max(c.k_eff, n_lp) : n_lp;
  // Logprobs need the normaliser to ~1e-7 relative: its largest terms are
  // summed in double from the candidates, so every chunk keeps a few.
  if (need_lse) c.k_sel = max(c.k_sel, kLseTop);
  if (c.k_sel > V) c.k_sel = V;
  c.store_s = c.cls == kTopP || c.cls == kTempOnly || c.wide;
  return c;
}

__device__ __forceinline__ float row_uniform(const ParamsView& pv, int row) {
  return pv.uniforms ? pv.uniforms[row] : pv.uniform_value;
}

// Stages 2 and 3 of the processed logit (the mask is applied by the caller):
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

// ---- block-level reductions (wave64 shuffles, then LDS) -------------------

template <int N>
__device__ __forceinline__ uint32_t block_sum_u32(uint32_t v, uint32_t* red) {
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  __syncthreads();
  if (lane == 0) red[wid] = v;
  __syncthreads();
  uint32_t s = 0;
  for (int i = 0; i < N / 64; ++i) s += red[i];
  return s;
}

template <int N>
__device__ __forceinline__ float block_sum_f32(float v, float* red) {
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  __syncthreads();
  if (lane == 0) red[wid] = v;
  __syncthreads();
  float s = 0.f;
  for (int i = 0; i < N / 64; ++i) s += red[i];
  return s;
}

template <int N>
__device__ __forceinline__ double block_sum_f64(double v, double* red) {
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  __syncthreads();
  if (lane == 0) red[wid] = v;
  __syncthreads();
  double s = 0.0;
  for (int i = 0; i < N / 64; ++i) s += red[i];
  return s;
}

template <int N>
__device__ __forceinline__ uint32_t block_max_u32(uint32_t v, uint32_t* red) {
  for (int o = 32; o > 0; o >>= 1) v = max(v, (uint32_t)__shfl_xor(v, o, 64));
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  __syncthreads();
  if (lane == 0) red[wid] = v;
  __syncthreads();
  uint32_t s = 0;
  for (int i = 0; i < N / 64; ++i) s = max(s, red[i]);
  return s;
}

__device__ __forceinline__ uint64_t shfl_xor_u64(uint64_t v, int o) {
  const uint32_t hi = (uint32_t)__shfl_xor((int)(uint32_t)(v >> 32), o, 64);
  const uint32_t lo = (uint32_t)__shfl_xor((int)(uint32_t)v, o, 64);
  return ((uint64_t)hi << 32) | lo;
}

template <int N>
__device__ __forceinline__ uint64_t block_max_u64(uint64_t v, uint64_t* red) {
  for (int o = 32; o > 0; o >>= 1) {
    const uint64_t t = shfl_xor_u64(v, o);
    if (t > v) v = t;
  }
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  __syncthreads();
  if (lane == 0) red[wid] = v;
  __syncthreads();
  uint64_t s = red[0];
  for (int i = 1; i < N / 64; ++i) s = red[i] > s ? red[i] : s;
  return s;
}

template <int N>
__device__ __forceinline__ uint64_t block_min_u64(uint64_t v, uint64_t* red) {
  return ~block_max_u64<N>(~v, red);
}

// Exclusive prefix sum over the block in thread order; *total gets the sum.
template <int N>
__device__ __forceinline__ uint32_t block_excl_scan_u32(uint32_t v, uint32_t* red, uint32_t* total) {
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  uint32_t inc = v;
  for (int o = 1; o < 64; o <<= 1) {
    const uint32_t t = __shfl_up(inc, o, 64);
    if (lane >= o) inc += t;
  }
  __syncthreads();
  if (lane == 63) red[wid] = inc;
  __syncthreads();
  uint32_t before = 0, tot = 0;
  for (int i = 0; i < N / 64; ++i) {
    if (i < wid) before += red[i];
    tot += red[i];
  }
  *total = tot;
  return before + inc - v;
}

// ---- chunk statistics ------------------------------------------------------

// Associative, order-independent merge of two statistics records.
__device__ __forceinline__ void stat_merge(ChunkStat& a, const ChunkStat& b) {
  a.max_l = fmaxf(a.max_l, b.max_l);
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
  s.max_l = -__builtin_inff();
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
  stat_init(r);
  r.max_l = __shfl_xor(s.max_l, o, 64);
  r.am_ieee_v = __shfl_xor(s.am_ieee_v, o, 64); r.am_ieee_i = __shfl_xor(s.am_ieee_i, o, 64);
  r.am_tot_k = __shfl_xor(s.am_tot_k, o, 64); r.am_tot_i = __shfl_xor(s.am_tot_i, o, 64);
  r.am_fin_v = __shfl_xor(s.am_fin_v, o, 64); r.am_fin_i = __shfl_xor(s.am_fin_i, o, 64);
  r.any_finite = __shfl_xor(s.any_finite, o, 64);
  return r;
}

// Reduce a per-thread statistics record over the block (valid in all threads).
template <int N>
__device__ __forceinline__ ChunkStat block_stat(ChunkStat s, ChunkStat* red) {
  for (int o = 32; o > 0; o >>= 1) {
    const ChunkStat t = stat_shfl_xor(s, o);
    stat_merge(s, t);
  }
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  __syncthreads();
  if (lane == 0) red[wid] = s;
  __syncthreads();
  ChunkStat r = red[0];
  for (int i = 1; i < N / 64; ++i) stat_merge(r, red[i]);
  return r;
}

// ---- element access -------------------------------------------------------

__device__ __forceinline__ float load_raw(const void* base, int dtype, int64_t off) {
  if (dtype == HI_ROCM_DTYPE_BF16) return bf16_to_f32(((const uint16_t*)base)[off]);
  return ((const float*)base)[off];
}

__device__ __forceinline__ bool allowed(const SampleArgs& a, int row, uint32_t idx) {
  return !a.mask || ((a.mask[(int64_t)row * a.mask_words + (idx >> 5)] >> (idx & 31u)) & 1u);
}

// Processed logit of one token (mask + penalties), computed by the whole
// block: its history count is reduced over the row's history list.
template <int N>
__device__ __forceinline__ float processed_single(const SampleArgs& a, int row, const RowCfg& c, uint32_t idx,
                                  uint32_t* red) {
  uint32_t cnt = 0;
  if (a.hoff) {
    const uint32_t h0 = a.hoff[row], h1 = a.hoff[row + 1];
    for (uint32_t h = h0 + threadIdx.x; h < h1; h += N)
      if (a.hids[h] == idx) cnt += a.hcnt[h];
  }
  cnt = block_sum_u32<N>(cnt, red);
  float l = load_raw(a.logits, a.dtype, (int64_t)row * a.row_stride + idx);
  if (!allowed(a, row, idx)) l = -__builtin_inff();
  return apply_penalties(l, cnt, c);
}

// ---- radix selection ------------------------------------------------------

// Threshold T such that exactly k of the block's items (unique keys of
// `bits` bits, a multiple of 8) are >= T.  for_each(cb) calls cb(key) for
// every item the calling thread owns.  8-bit MSD descent with early exit;
// hist has 256 entries, sel 3.
template <typename ForEach>
__device__ __forceinline__ uint64_t radix_select_top(uint32_t* hist, uint32_t* sel, uint32_t k, int bits,
                                     ForEach for_each) {
  const int tid = threadIdx.x;
  uint64_t prefix = 0;
  uint32_t remaining = k;
  for (int shift = bits - 8; shift >= 0; shift -= 8) {
    for (int b = tid; b < 256; b += NT) hist[b] = 0u;
    __syncthreads();
    const int hs = shift + 8;
    const uint64_t hp = hs >= 64 ? 0ull : (prefix >> hs);
    for_each([&](uint64_t x) {
      if (hs >= 64 || (x >> hs) == hp) atomicAdd(&hist[(uint32_t)(x >> shift) & 255u], 1u);
    });
    __syncthreads();
    if (tid < 64) {
      // lane l owns bins 255-4l .. 252-4l (descending)
      uint32_t loc[4], lsum = 0;
      #pragma unroll
      for (int q = 0; q < 4; ++q) { loc[q] = hist[255 - 4 * tid - q]; lsum += loc[q]; }
      uint32_t inc = lsum;
      for (int o = 1; o < 64; o <<= 1) {
        const uint32_t t = __shfl_up(inc, o, 64);
        if (tid >= o) inc += t;
      }
      const uint32_t above = inc - lsum;
      if (above < remaining && remaining <= above + lsum) {
        uint32_t acc = above;
        #pragma unroll
        for (int q = 0; q < 4; ++q) {
          if (remaining <= acc + loc[q] && acc < remaining) {
            sel[0] = 255u - 4u * tid - q; sel[1] = acc; sel[2] = loc[q];
          }
          acc += loc[q];
        }
      }
    }
    __syncthreads();
    prefix |= (uint64_t)sel[0] << shift;
    remaining -= sel[1];
    const bool done = sel[2] == remaining;
    __syncthreads();
    if (done) break;
  }
  return prefix;
}

// ==========================================================================
// LDS layouts
// ==========================================================================

struct ScanLds {
  uint64_t cbuf[kBufCap];     // running candidates (48-bit local composites)
  uint32_t U[kBuf];           // per-thread top-j keys of the first tile
  uint32_t hist[256];
  ChunkStat red[NT / 64];
  uint32_t redu[NT / 64];
  uint64_t red64[NT / 64];
  float redf[NT / 64];
  uint32_t sel[4];
  uint32_t bound, count, hovf;
  // when the batch has histories: bitmap[chunk / 32], hash keys[kHashCap],
  // hash counts[kHashCap] follow
};

struct FinLds {
  uint64_t cbig[kGather];     // gathered candidates (32 KiB) -- also a fold tile
  uint64_t buf[kBuf];         // selected candidates / rank keys
  uint32_t pay[kBuf];         // scaled-logit keys riding with buf
  float fa[kBuf];             // weights in rank order
  float fb[kBuf];             // w / total
  uint32_t hist[kBins];
  uint64_t mass[kBins];
  uint32_t aux[kBins];
  ChunkStat red[NT / 64];
  uint32_t redu[NT / 64];
  double redd[NT / 64];
  uint64_t red64[NT / 64];
  uint32_t sel[4];
  uint32_t counter, n_ext, token, flag;
  float fval0, fval1;
};
constexpr int kTileFloats = kGather * 2;  // floats of the fold tile (cbig)


// ==========================================================================
// Finish phase (one workgroup per row)
// ==========================================================================

// Candidates of `row` (written by the chunks): visit every (chunk, slot).
// Chunk c kept min(k_sel, its length) candidates, so the slots are known
// without reading the chunk records; one flat parallel loop.
template <typename F>
__device__ __forceinline__ void for_each_candidate(const SampleArgs& a, int row, int k_sel, F f) {
  const int nch = a.n_chunks;
  const uint64_t* cand = a.cand + (int64_t)row * nch * kFast;
  const int last_len = a.V - (nch - 1) * a.chunk;
  const int n_full = min(k_sel, a.chunk);
  const int n_last = min(k_sel, last_len);
  const int span = (nch - 1) * n_full + n_last;
  for (int j = threadIdx.x; j < span; j += NT) {
    const int c = n_full > 0 ? j / n_full : 0;
    const int s = j - c * n_full;
    f(cand[(int64_t)c * kFast + s]);
  }
}

// Descending sort of fs.buf[0..n) carrying fs.pay; n <= kBuf.
__device__ __forceinline__ void sort_ranked(FinLds& fs, int n) {
  const int tid = threadIdx.x;
  if (n <= NT) {
    // rank by counting (keys are unique), then scatter
    uint64_t x = 0;
    uint32_t p = 0, r = 0;
    if (tid < n) {
      x = fs.buf[tid];
      p = fs.pay[tid];
      for (int j = 0; j < n; ++j) r += fs.buf[j] > x;
    }
    __syncthreads();
    if (tid < n) { fs.buf[r] = x; fs.pay[r] = p; }
    __syncthreads();
    return;
  }
  const int n2 = next_pow2(n);
  for (int i = n + tid; i < n2; i += NT) { fs.buf[i] = 0ull; fs.pay[i] = 0u; }
  __syncthreads();
  for (int k = 2; k <= n2; k <<= 1) {
    for (int j = k >> 1; j > 0; j >>= 1) {
      for (int i = tid; i < n2; i += NT) {
        const int ixj = i ^ j;
        if (ixj > i) {
          const uint64_t x = fs.buf[i], y = fs.buf[ixj];
          const bool desc = (i & k) == 0;
          if (desc ? (x < y) : (x > y)) {
            fs.buf[i] = y; fs.buf[ixj] = x;
            const uint32_t t = fs.pay[i]; fs.pay[i] = fs.pay[ixj]; fs.pay[ixj] = t;
          }
        }
      }
      __syncthreads();
    }
  }
}

// Number of candidates the chunks of `row` wrote: chunk c keeps
// min(k_sel, its length), so it is known without reading the records.
__device__ __forceinline__ int candidate_count(const SampleArgs& a, int k_sel) {
  const int last_len = a.V - (a.n_chunks - 1) * a.chunk;
  return (a.n_chunks - 1) * min(k_sel, a.chunk) + min(k_sel, last_len);
}

// The exact first `kk` entries of the reference rank order (weight desc,
// index asc) of `row`.  On return fs.buf[0..kk) holds rank keys in order and
// fs.pay[0..kk) the scaled-logit keys; returns kk.  M is the row max of s.
// When lse_part is not null, it receives this thread's share of
// sum(exp(s - M)) over every candidate (double).
__device__ __forceinline__ int rank_candidates(FinLds& fs, const SampleArgs& a, int row, const RowCfg& cfg,
                               int kk_req, float M, double* lse_part) {
  const int tid = threadIdx.x;
  const int nch = a.n_chunks;
  const ChunkStat* stats = a.stats + (int64_t)row * nch;
  const int n_total = candidate_count(a, cfg.k_sel);
  const int kk = min(kk_req, n_total);
  if (kk <= 0) return 0;
  auto s_of = [&](uint64_t x) { return key_to_s(cand_skey(x), cfg.t_eff); };
  double part = 0.0;
  // 1. candidates into LDS: all of them when they fit, else those at or above
  //    t0, the largest chunk cut (the kk-th composite is at least every
  //    truncated chunk's smallest kept composite)
  uint64_t t0 = 0;
  uint64_t below_max = 0;  // largest candidate left out of LDS
  int n_u;
  bool in_lds = true;
  if (n_total <= kGather) {
    int j = 0;
    for_each_candidate(a, row, cfg.k_sel, [&](uint64_t x) {
      fs.cbig[tid + j * NT] = x;
      ++j;
      if (lse_part) part += exp((double)s_of(x) - (double)M);
    });
    n_u = n_total;
  } else {
    for (int c = tid; c < nch; c += NT)
      if (stats[c].trunc && stats[c].min_kept > t0) t0 = stats[c].min_kept;
    t0 = block_max_u64<NT>(t0, fs.red64);
    uint32_t nu = 0;
    for_each_candidate(a, row, cfg.k_sel, [&](uint64_t x) {
      nu += x >= t0;
      if (x < t0 && x > below_max) below_max = x;
      if (lse_part) part += exp((double)s_of(x) - (double)M);
    });
    n_u = (int)block_sum_u32<NT>(nu, fs.redu);
    below_max = block_max_u64<NT>(below_max, fs.red64);
    in_lds = n_u <= kGather;
    if (in_lds) {
      if (tid == 0) fs.counter = 0u;
      __syncthreads();
      for_each_candidate(a, row, cfg.k_sel, [&](uint64_t x) {
        if (x >= t0) fs.cbig[atomicAdd(&fs.counter, 1u)] = x;
      });
    }
  }
  __syncthreads();
  if (lse_part) *lse_part = part;
  // 2. the kk largest
  uint64_t thr = 0;
  if (in_lds) {
    if (n_u > kk) {
      thr = radix_select_top(fs.hist, fs.sel, (uint32_t)kk, 64, [&](auto cb) {
        for (int i = tid; i < n_u; i += NT) cb(fs.cbig[i]);
      });
    }
    uint64_t umax = 0;  // largest unselected
    if (tid == 0) fs.counter = 0u;
    __syncthreads();
    for (int i = tid; i < n_u; i += NT) {
      const uint64_t x = fs.cbig[i];
      if (x >= thr) fs.buf[atomicAdd(&fs.counter, 1u)] = x;
      else if (x > umax) umax = x;
    }
    below_max = max(below_max, block_max_u64<NT>(umax, fs.red64));
  } else {
    // rare: more than kGather candidates above t0; select over global memory
    thr = radix_select_top(fs.hist, fs.sel, (uint32_t)kk, 64, [&](auto cb) {
      for_each_candidate(a, row, cfg.k_sel, [&](uint64_t x) { if (x >= t0) cb(x); });
    });
    if (tid == 0) fs.counter = 0u;
    __syncthreads();
    uint64_t umax = 0;
    for_each_candidate(a, row, cfg.k_sel, [&](uint64_t x) {
      if (x >= thr && x >= t0) {
        const uint32_t p = atomicAdd(&fs.counter, 1u);
        if (p < (uint32_t)kBuf) fs.buf[p] = x;
      } else if (x > umax) {
        umax = x;
      }
    });
    below_max = max(below_max, block_max_u64<NT>(umax, fs.red64));
  }
  thr = thr > t0 ? thr : t0;
  // 3. weights; the smallest selected weight is w_b
  uint32_t wmin_bits = 0xffffffffu;
  for (int i = tid; i < kk; i += NT) {
    const uint64_t x = fs.buf[i];
    const float sx = s_of(x);
    const float w = exact_expf(sx - M);
    fs.buf[i] = rank_key(w, cand_idx(x));
    fs.pay[i] = okey(sx);
    wmin_bits = min(wmin_bits, __float_as_uint(w));
  }
  const float w_b = __uint_as_float(~block_max_u32<NT>(~wmin_bits, fs.redu));
  // 4. tie extension: elements outside the selection with weight w_b can
  //    still belong to the first kk of the rank order (lower index)
  if (tid == 0) fs.n_ext = 0u;
  __syncthreads();
  uint64_t* ext = a.ws_list + (int64_t)row * a.list_stride;
  uint32_t* ext_aux = reinterpret_cast<uint32_t*>(a.ws_w + (int64_t)row * a.V);
  const int64_t ext_cap = a.V;
  auto add_ext = [&](float w, uint32_t idx, float sx) {
    const uint32_t p = atomicAdd(&fs.n_ext, 1u);
    if (p < ext_cap) { ext[p] = rank_key(w, idx); ext_aux[p] = okey(sx); }
  };
  if (w_b > 0.f) {
    // (a) unselected candidates: weights are monotone in the key, so only if
    //     the largest of them ties
    if (below_max != 0 && exact_expf(s_of(below_max) - M) == w_b) {
      if (in_lds) {
        for (int i = tid; i < n_u; i += NT) {
          const uint64_t x = fs.cbig[i];
          if (x >= thr) continue;
          const float sx = s_of(x);
          const float w = exact_expf(sx - M);
          if (w == w_b) add_ext(w, cand_idx(x), sx);
        }
      }
      if (!in_lds || t0 != 0) {
        for_each_candidate(a, row, cfg.k_sel, [&](uint64_t x) {
          if (x >= thr || (in_lds && x >= t0)) return;  // selected, or seen in LDS
          const float sx = s_of(x);
          const float w = exact_expf(sx - M);
          if (w == w_b) add_ext(w, cand_idx(x), sx);
        });
      }
    }
    // (b) elements a truncated chunk did not keep (rare: recompute the
    //     chunk); chunks are checked NT at a time
    for (int cb = 0; cb < nch; cb += NT) {
      if (tid == 0) fs.counter = 0u;
      __syncthreads();
      {
        const int c = cb + tid;
        if (c < nch) {
          const ChunkStat cs = stats[c];
          if (cs.trunc && exact_expf(key_to_s(cs.unkept_key, cfg.t_eff) - M) == w_b)
            fs.aux[atomicAdd(&fs.counter, 1u)] = (uint32_t)c;
        }
      }
      __syncthreads();
      const uint32_t n_flag = fs.counter;
      for (uint32_t f = 0; f < n_flag; ++f) {
        const int c = (int)fs.aux[f];
        const ChunkStat cs = stats[c];
        const int c0 = c * a.chunk, c1 = min(c0 + a.chunk, a.V);
        const int64_t rbase = (int64_t)row * a.row_stride;
        uint32_t h0 = 0, h1 = 0;
        if (a.hoff) { h0 = a.hoff[row]; h1 = a.hoff[row + 1]; }
        for (int e = c0 + tid; e < c1; e += NT) {
          float l = load_raw(a.logits, a.dtype, rbase + e);
          if (!allowed(a, row, (uint32_t)e)) l = -__builtin_inff();
          uint32_t cnt = 0;
          for (uint32_t h = h0; h < h1; ++h) if (a.hids[h] == (uint32_t)e) cnt += a.hcnt[h];
          l = apply_penalties(l, cnt, cfg);
          const uint32_t kl = lkey(l);
          if (cand_key(kl, (uint32_t)e) >= cs.min_kept) continue;  // already a candidate
          const float sx = key_to_s(kl, cfg.t_eff);
          const float w = exact_expf(sx - M);
          if (w == w_b) add_ext(w, (uint32_t)e, sx);
        }
      }
      __syncthreads();
    }
  }
  __syncthreads();
  const uint32_t n_ext = min(fs.n_ext, (uint32_t)(ext_cap - kk));
  if (n_ext > 0) {
    // union of selection and extension, then its first kk by rank key
    const int n_all = kk + (int)n_ext;
    for (int i = tid; i < kk; i += NT) { ext[n_ext + i] = fs.buf[i]; ext_aux[n_ext + i] = fs.pay[i]; }
    __syncthreads();
    const uint64_t t2 = radix_select_top(fs.hist, fs.sel, (uint32_t)kk, 64, [&](auto cb) {
      for (int j = tid; j < n_all; j += NT) cb(ext[j]);
    });
    if (tid == 0) fs.counter = 0u;
    __syncthreads();
    for (int j = tid; j < n_all; j += NT) {
      const uint64_t x = ext[j];
      if (x >= t2) {
        const uint32_t p = atomicAdd(&fs.counter, 1u);
        if (p < (uint32_t)kBuf) { fs.buf[p] = x; fs.pay[p] = ext_aux[j]; }
      }
    }
    __syncthreads();
  }
  sort_ranked(fs, kk);
  return kk;
}

// Reference steps 7-10 (gpu.rs:831-899) over the first k entries of the rank
// order in fs.buf (top-k rows).  Returns the token, or 0xffffffff for "fall
// back to argmax_host".
__device__ __forceinline__ uint32_t draw_topk(FinLds& fs, const RowCfg& cfg, int k, float u) {
  const int tid = threadIdx.x;
  for (int i = tid; i < k; i += NT) {
    const float w = rank_w(fs.buf[i]);
    fs.fa[i] = (w < cfg.min_p) ? 0.f : w;
  }
  __syncthreads();
  if (tid == 0) {
    float total = -0.0f;  // gpu.rs:834-836: kept mass in rank order
    for (int i = 0; i < k; ++i) total += fs.fa[i];
    fs.fval0 = total;
  }
  __syncthreads();
  const float total = fs.fval0;
  if (total <= 0.f || !finitef_(total)) return 0xffffffffu;
  for (int i = tid; i < k; i += NT) fs.fb[i] = fs.fa[i] / total;
  __syncthreads();
  if (tid == 0) {
    float cum_p = 0.f;
    int m_end = 0;  // candidates: positive weights in [0, m_end)
    bool any = false;
    for (int i = 0; i < k; ++i) {
      if (fs.fa[i] <= 0.f) continue;
      any = true;
      m_end = i + 1;
      cum_p += fs.fb[i];
      if (cfg.cutoff < 1.f && cum_p >= cfg.cutoff) break;
    }
    uint32_t tok = 0xffffffffu;
    if (any) {
      float ct = -0.0f;
      for (int i = 0; i < m_end; ++i) if (fs.fa[i] > 0.f) ct += fs.fa[i];
      if (ct > 0.f && finitef_(ct)) {
        const float target = clamp_uniform(u) * ct;
        float cum = 0.f;
        int last = -1, pick = -1;
        for (int i = 0; i < m_end; ++i) {
          if (fs.fa[i] <= 0.f) continue;
          last = i;
          cum += fs.fa[i];
          if (target < cum) { pick = i; break; }
        }
        if (pick < 0) pick = last;
        tok = cand_idx(fs.buf[pick]);
      }
    }
    fs.token = tok;
  }
  __syncthreads();
  return fs.token;
}

// Serial f32 fold of a global float array in index order (Rust's Sum: a fold
// from -0.0), by thread 0, staged through LDS tiles.  Valid in all threads.
__device__ __forceinline__ float fold_global(FinLds& fs, const float* x, int n) {
  float* tile = reinterpret_cast<float*>(fs.cbig);
  float acc = -0.0f;  // meaningful in thread 0 only
  for (int t0 = 0; t0 < n; t0 += kTileFloats) {
    const int m = min(kTileFloats, n - t0);
    __syncthreads();
    for (int i = threadIdx.x; i < m; i += NT) tile[i] = x[t0 + i];
    __syncthreads();
    if (threadIdx.x == 0)
      for (int i = 0; i < m; ++i) acc += tile[i];
  }
  __syncthreads();
  if (threadIdx.x == 0) fs.fval0 = acc;
  __syncthreads();
  const float r = fs.fval0;
  __syncthreads();
  return r;
}

// Bitonic sort of a global array (descending) by one workgroup.
__device__ __forceinline__ void global_sort_desc(uint64_t* g, int n2) {
  for (int k = 2; k <= n2; k <<= 1) {
    for (int j = k >> 1; j > 0; j >>= 1) {
      for (int i = threadIdx.x; i < n2; i += NT) {
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

// Rows without top-k (or with top_k > 1024): the distribution is re-read from
// the workspace (ws_s holds the scaled logits).  Returns the token or
// 0xffffffff for the argmax fallback.
__device__ __forceinline__ uint32_t draw_wide(FinLds& fs, const SampleArgs& a, int row, const RowCfg& cfg,
                              float M, float u) {
  const int tid = threadIdx.x;
  const int V = a.V;
  const float* srow = a.ws_s + (int64_t)row * V;
  float* wrow = a.ws_w + (int64_t)row * V;
  uint64_t* list = a.ws_list + (int64_t)row * a.list_stride;
  for (int b = tid; b < kBins; b += NT) { fs.hist[b] = 0u; fs.mass[b] = 0ull; }
  __syncthreads();
  for (int i = tid; i < V; i += NT) {
    float w = exact_expf(srow[i] - M);
    if (w < cfg.min_p) w = 0.f;
    wrow[i] = w;
    if (w > 0.f) {
      const uint32_t b = __float_as_uint(w) >> 20;
      atomicAdd(&fs.hist[b], 1u);
      atomicAdd((unsigned long long*)&fs.mass[b], (unsigned long long)((double)w * 1099511627776.0));
    }
  }
  __syncthreads();
  const bool wide_k = cfg.cls == kTopK;
  float total = 0.f;
  if (!wide_k) {
    total = fold_global(fs, wrow, V);  // gpu.rs:837: vocab-order sum
    if (total <= 0.f || !finitef_(total)) return 0xffffffffu;
  }
  if (tid == 0) {
    uint64_t all_mass = 0;
    for (int b = 0; b < kBins; ++b) all_mass += fs.mass[b];
    int bstar = 0;
    if (wide_k) {
      uint32_t c = 0;
      for (int b = kBins - 1; b >= 0; --b) { c += fs.hist[b]; if (c >= (uint32_t)cfg.k_eff) { bstar = b; break; } }
    } else if (cfg.cutoff < 1.f) {
      // superset holding the nucleus with margin (verified below)
      const double need = fmin(1.0, (double)cfg.cutoff + 0.02) * (double)all_mass;
      uint64_t c = 0;
      for (int b = kBins - 1; b >= 0; --b) { c += fs.mass[b]; if ((double)c >= need) { bstar = b; break; } }
    }
    fs.flag = (uint32_t)bstar;
  }
  __syncthreads();
  int bstar = (int)fs.flag;
  uint32_t tok = 0xffffffffu;
  for (int attempt = 0; attempt < 2; ++attempt) {
    __syncthreads();
    if (tid == 0) {
      uint32_t off = 0;
      for (int b = kBins - 1; b >= 0; --b) {
        fs.aux[b] = off;
        if (b >= bstar) off += fs.hist[b];
      }
      fs.counter = off;
    }
    __syncthreads();
    const int n_sup = (int)fs.counter;
    for (int i = tid; i < V; i += NT) {
      const float w = wrow[i];
      if (w > 0.f) {
        const int b = (int)(__float_as_uint(w) >> 20);
        if (b >= bstar) list[atomicAdd(&fs.aux[b], 1u)] = rank_key(w, (uint32_t)i);
      }
    }
    __syncthreads();
    const int n2 = next_pow2(max(n_sup, 1));
    for (int i = n_sup + tid; i < n2; i += NT) list[i] = 0ull;
    __syncthreads();
    global_sort_desc(list, n2);
    if (tid == 0) {
      int k = n_sup;
      if (wide_k) {
        k = min(cfg.k_eff, n_sup);  // zero-weight entries add nothing
        float t = -0.0f;
        for (int i = 0; i < k; ++i) t += rank_w(list[i]);
        total = t;
      }
      uint32_t r = 0xffffffffu;
      uint32_t flag = 1u;
      if (total > 0.f && finitef_(total)) {
        float cum_p = 0.f;
        int m_end = 0;
        bool reached = false;
        for (int i = 0; i < k; ++i) {
          m_end = i + 1;
          cum_p += rank_w(list[i]) / total;
          if (cfg.cutoff < 1.f && cum_p >= cfg.cutoff) { reached = true; break; }
        }
        if (!wide_k && !reached && bstar != 0) {
          flag = 0xffffffffu;  // superset too small: retry with every positive weight
        } else {
          float ct = -0.0f;
          for (int i = 0; i < m_end; ++i) ct += rank_w(list[i]);
          if (m_end > 0 && ct > 0.f && finitef_(ct)) {
            const float target = clamp_uniform(u) * ct;
            float cum = 0.f;
            int pick = m_end - 1;
            for (int i = 0; i < m_end; ++i) {
              cum += rank_w(list[i]);
              if (target < cum) { pick = i; break; }
            }
            r = cand_idx(list[pick]);
          }
        }
      }
      fs.token = r;
      fs.flag = flag;
    }
    __syncthreads();
    if (fs.flag != 0xffffffffu) { tok = fs.token; break; }
    bstar = 0;
  }
  return tok;
}

// Temperature-only rows: kernels.cu:7803-7867 with the exact weight function.
// 256 contiguous chunks, one per thread of the (256-thread) workgroup.
__device__ __forceinline__ uint32_t draw_temp_only(FinLds& fs, const SampleArgs& a, int row, float M, float u,
                                   uint32_t argmax_fin) {
  static_assert(NT == 256, "the reference's temperature-only path uses 256 chunks");
  const int tid = threadIdx.x;
  const int V = a.V;
  const float* srow = a.ws_s + (int64_t)row * V;
  const int chunk = (V + 255) / 256;
  float* csum = fs.fa;
  float* prefix = fs.fb;
  {
    const int start = tid * chunk, end = min(start + chunk, V);
    float s = 0.f;
    for (int i = start; i < end; ++i) s += exact_expf(srow[i] - M);
    csum[tid] = s;
  }
  __syncthreads();
  if (tid == 0) {
    float acc = 0.f;
    for (int j = 0; j < 256; ++j) { prefix[j] = acc; acc += csum[j]; }
    fs.fval0 = acc;
    fs.token = 0xffffffffu;
  }
  __syncthreads();
  const float total = fs.fval0;
  if (total <= 0.f || !finitef_(total)) return argmax_fin;
  const float uu = finitef_(u) ? fminf(fmaxf(u, 0.f), 0.99999994f) : 0.f;
  const float target = uu * total;
  {
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
      if (chosen >= 0) atomicMin(&fs.token, (uint32_t)chosen);
    }
  }
  __syncthreads();
  return fs.token != 0xffffffffu ? fs.token : argmax_fin;
}

// argmax_host (gpu.rs:739-751, total_cmp, lowest index) over the processed
// logits of the row.  Only needed when no scaled logit is finite (or l / T
// overflows), so the row is re-read here, 4096 logits at a time, with an LDS
// count table for the penalties.
__device__ __forceinline__ uint32_t row_argmax_total(FinLds& fs, const SampleArgs& a, int row,
                                                     const RowCfg& cfg) {
  const int tid = threadIdx.x;
  const int V = a.V;
  constexpr int T = 4096;
  static_assert(kGather * 2 >= T, "count table fits cbig");
  uint32_t* cnt = reinterpret_cast<uint32_t*>(fs.cbig);
  uint32_t h0 = 0, h1 = 0;
  if (a.hoff) { h0 = a.hoff[row]; h1 = a.hoff[row + 1]; }
  const int64_t rbase = (int64_t)row * a.row_stride;
  uint64_t best = 0ull;  // (total key biased) << 32 | (0xffffffff - index)
  for (int t0 = 0; t0 < V; t0 += T) {
    const int t1 = min(t0 + T, V);
    __syncthreads();
    for (int i = tid; i < T; i += NT) cnt[i] = 0u;
    __syncthreads();
    for (uint32_t h = h0 + tid; h < h1; h += NT) {
      const uint32_t id = a.hids[h];
      if (id >= (uint32_t)t0 && id < (uint32_t)t1) atomicAdd(&cnt[id - t0], a.hcnt[h]);
    }
    __syncthreads();
    for (int e = t0 + tid; e < t1; e += NT) {
      float l = load_raw(a.logits, a.dtype, rbase + e);
      if (!allowed(a, row, (uint32_t)e)) l = -__builtin_inff();
      l = apply_penalties(l, cnt[e - t0], cfg);
      const uint64_t v = ((uint64_t)((uint32_t)total_key(l) ^ 0x80000000u) << 32) |
                         (uint64_t)(0xffffffffu - (uint32_t)e);
      best = v > best ? v : best;
    }
  }
  best = block_max_u64<NT>(best, fs.red64);
  return 0xffffffffu - (uint32_t)best;
}

__device__ __forceinline__ void finish_row(FinLds& fs, const SampleArgs& a, int row, const RowCfg& cfg) {
  const int tid = threadIdx.x;
  const int V = a.V;
  ChunkStat st;
  stat_init(st);
  for (int c = tid; c < a.n_chunks; c += NT) stat_merge(st, a.stats[(int64_t)row * a.n_chunks + c]);
  const ChunkStat rs = block_stat<NT>(st, fs.red);
  // row max of s = l / T: division is monotone, so it is max(l) / T
  const float M = finitef_(rs.max_l) ? rs.max_l / cfg.t_eff : -__builtin_inff();
  const uint32_t am_ieee = rs.am_ieee_i == 0xffffffffu ? 0u : rs.am_ieee_i;
  const uint32_t am_fin = rs.am_fin_i == 0xffffffffu ? 0u : rs.am_fin_i;
  const float u = row_uniform(a.pv, row);

  const bool eos = a.mask && !rs.any_finite;
  uint32_t token;
  int ranked_k = 0;  // entries of fs.buf in rank order
  double lse_part = 0.0;  // this thread's share of sum(exp(s - M)) over the candidates
  bool have_part = false;
  if (eos) {
    token = cfg.eos;
  } else if (cfg.cls == kGreedy) {
    token = a.pv.greedy_rule == kGreedyFiniteLane ? am_fin : am_ieee;
  } else if (!finitef_(M)) {
    token = cfg.cls == kTempOnly ? am_fin : row_argmax_total(fs, a, row, cfg);
  } else if (cfg.cls == kTopK && !cfg.wide) {
    ranked_k = rank_candidates(fs, a, row, cfg, cfg.k_sel, M, a.need_lse ? &lse_part : nullptr);
    have_part = a.need_lse != 0;
    token = draw_topk(fs, cfg, cfg.k_eff, u);
    if (token == 0xffffffffu) token = row_argmax_total(fs, a, row, cfg);
  } else if (cfg.cls == kTempOnly) {
    token = draw_temp_only(fs, a, row, M, u, am_fin);
  } else {
    token = draw_wide(fs, a, row, cfg, M, u);
    if (token == 0xffffffffu) token = row_argmax_total(fs, a, row, cfg);
  }
  if (tid == 0) a.out_tokens[row] = token;
  if (a.n_lp <= 0 && !a.out_token_lp) return;

  // Logprobs of the processed distribution (extension).
  __syncthreads();
  const int N = a.n_lp;
  if (eos || !finitef_(M)) {
    for (int j = tid; j < N; j += NT) {
      a.out_lp[(int64_t)row * N + j] = -__builtin_inff();
      a.out_lp_ids[(int64_t)row * N + j] = 0xffffffffu;
    }
    if (tid == 0 && a.out_token_lp) a.out_token_lp[row] = eos ? 0.f : -__builtin_inff();
    return;
  }
  if (N > 0 && ranked_k < N) {
    ranked_k = rank_candidates(fs, a, row, cfg, N, M, have_part ? nullptr : &lse_part);
    have_part = true;
  }
  // log of the normaliser relative to M: the kept candidates of every chunk
  // in double, the rest from each chunk's sum over the elements it dropped
  if (!have_part) {
    for_each_candidate(a, row, cfg.k_sel, [&](uint64_t x) {
      lse_part += exp((double)key_to_s(cand_skey(x), cfg.t_eff) - (double)M);
    });
  }
  double part = lse_part;
  for (int c = tid; c < a.n_chunks; c += NT) {
    const ChunkStat cs = a.stats[(int64_t)row * a.n_chunks + c];
    if (cs.lse_sum > 0.f) part += (double)cs.lse_sum * exp((double)cs.lse_m - (double)M);
  }
  const double log_sum = log(block_sum_f64<NT>(part, fs.redd));
  for (int j = tid; j < N; j += NT) {
    float lp = -__builtin_inff();
    uint32_t id = 0xffffffffu;
    if (j < ranked_k) {
      id = cand_idx(fs.buf[j]);
      lp = (float)(((double)okey_inv(fs.pay[j]) - (double)M) - log_sum);
    }
    a.out_lp_ids[(int64_t)row * N + j] = id;
    a.out_lp[(int64_t)row * N + j] = lp;
  }
  if (a.out_token_lp) {
    if (tid == 0) fs.flag = 0u;
    __syncthreads();
    for (int j = tid; j < ranked_k; j += NT)
      if (cand_idx(fs.buf[j]) == token) { fs.flag = 1u; fs.fval1 = okey_inv(fs.pay[j]); }
    __syncthreads();
    float s;
    if (fs.flag) {
      s = fs.fval1;
    } else {
      const float l = processed_single<NT>(a, row, cfg, token < (uint32_t)V ? token : 0u, fs.redu);
      s = finitef_(l) ? l / cfg.t_eff : -__builtin_inff();
    }
    if (tid == 0)
      a.out_token_lp[row] = token < (uint32_t)V ? (float)(((double)s - (double)M) - log_sum) : -__builtin_inff();
  }
}

// ==========================================================================
// The scan kernel: one pass over the logits
// ==========================================================================

// Online sum of exp(s - m) with a running maximum m (for the log-sum-exp of
// the elements a chunk does not keep).
struct RestAcc {
  float m, sum;
  __device__ __forceinline__ void init() { m = -__builtin_inff(); sum = 0.f; }
  __device__ __forceinline__ void add(float s) {
    if (!finitef_(s)) return;
    if (sum == 0.f) { m = s; sum = 1.f; }
    else if (s > m) { sum = sum * __expf(m - s) + 1.f; m = s; }
    else sum += __expf(s - m);
  }
};

// Per-chunk running selection state (kept in registers, uniform over the
// workgroup): tau is a 48-bit local composite below which no element can be
// among the chunk's top k.
struct SelState {
  uint64_t tau;
  uint32_t unkept;  // largest key known not to be kept
  RestAcc rest;
  bool rest_on;
  float t_eff;
};

__device__ __forceinline__ void reject_key(SelState& ss, uint32_t key) {
  ss.unkept = max(ss.unkept, key);
  if (ss.rest_on) ss.rest.add(key_to_s(key, ss.t_eff));
}
__device__ __forceinline__ void reject(SelState& ss, uint64_t comp) {
  reject_key(ss, (uint32_t)(comp >> 16));
}

// Keep the k largest composites of the LDS buffer; raises tau and rejects
// the others.  All threads call it.
__device__ __forceinline__ void compact_buffer(ScanLds& sh, SelState& ss, uint32_t k) {
  const int tid = threadIdx.x;
  const uint32_t n = sh.count;
  if (n <= k) return;
  const uint64_t thr = radix_select_top(sh.hist, sh.sel, k, 48, [&](auto cb) {
    for (uint32_t i = tid; i < n; i += NT) cb(sh.cbuf[i]);
  });
  constexpr int PER = kBufCap / NT;
  uint64_t v[PER];
  uint32_t keep = 0;
  #pragma unroll
  for (int r = 0; r < PER; ++r) {
    const uint32_t i = r * NT + tid;
    v[r] = i < n ? sh.cbuf[i] : 0ull;
    if (i < n) {
      if (v[r] >= thr) ++keep;
      else reject(ss, v[r]);
    }
  }
  uint32_t total;
  uint32_t pos = block_excl_scan_u32<NT>(keep, sh.redu, &total);  // has barriers
  #pragma unroll
  for (int r = 0; r < PER; ++r) {
    const uint32_t i = r * NT + tid;
    if (i < n && v[r] >= thr) sh.cbuf[pos++] = v[r];
  }
  if (thr > ss.tau) ss.tau = thr;
  __syncthreads();
  if (tid == 0) sh.count = total;
  __syncthreads();
}

// Append NI items per thread to the running selection.  Item i has scaled-
// logit key key[i] (0 = no item) and local index li_of(i).  Items below tau
// are rejected, the rest go to the LDS buffer.  The caller guarantees that
// NI * NT <= kBufCap - k, so after one compaction (which leaves at most k
// entries) every batch fits.
template <int NI, typename LiOf>
__device__ __forceinline__ void append_batch(ScanLds& sh, SelState& ss, uint32_t k,
                                             const uint32_t (&key)[NI], LiOf li_of) {
  static_assert(NI * NT + kFast <= kBufCap, "a batch must fit after compaction");
  uint32_t mine = 0;
  #pragma unroll
  for (int i = 0; i < NI; ++i) mine += key[i] != 0u && local_comp(key[i], li_of(i)) >= ss.tau;
  uint32_t total;
  uint32_t off = block_excl_scan_u32<NT>(mine, sh.redu, &total);
  if (sh.count + total > (uint32_t)kBufCap) {
    compact_buffer(sh, ss, k);
    mine = 0;
    #pragma unroll
    for (int i = 0; i < NI; ++i) mine += key[i] != 0u && local_comp(key[i], li_of(i)) >= ss.tau;
    off = block_excl_scan_u32<NT>(mine, sh.redu, &total);
  }
  const uint32_t base = sh.count;
  #pragma unroll
  for (int i = 0; i < NI; ++i) {
    if (key[i] == 0u) continue;
    const uint64_t c = local_comp(key[i], li_of(i));
    if (c >= ss.tau) sh.cbuf[base + off++] = c;
    else reject(ss, c);
  }
  __syncthreads();
  if (threadIdx.x == 0) sh.count = base + total;
  __syncthreads();
}

template <int VEC>
__device__ __forceinline__ void load_tile(const SampleArgs& a, int64_t rbase, int tb, int c1,
                                          float (&raw)[VEC * 4]) {
  const int tid = threadIdx.x;
  if (a.dtype == HI_ROCM_DTYPE_BF16) {
    #pragma unroll
    for (int j = 0; j < VEC; ++j) {
      const int e0 = tb + (j * NT + tid) * 4;
      if (a.vec_ok && e0 + 3 < c1) {
        const uint2 v = *(const uint2*)((const uint16_t*)a.logits + rbase + e0);
        raw[4 * j + 0] = __uint_as_float(v.x << 16); raw[4 * j + 1] = __uint_as_float(v.x & 0xffff0000u);
        raw[4 * j + 2] = __uint_as_float(v.y << 16); raw[4 * j + 3] = __uint_as_float(v.y & 0xffff0000u);
      } else {
        #pragma unroll
        for (int q = 0; q < 4; ++q) raw[4 * j + q] = (e0 + q < c1) ? load_raw(a.logits, a.dtype, rbase + e0 + q) : 0.f;
      }
    }
  } else {
    #pragma unroll
    for (int j = 0; j < VEC; ++j) {
      const int e0 = tb + (j * NT + tid) * 4;
      if (a.vec_ok && e0 + 3 < c1) {
        const float4 v = *(const float4*)((const float*)a.logits + rbase + e0);
        raw[4 * j + 0] = v.x; raw[4 * j + 1] = v.y; raw[4 * j + 2] = v.z; raw[4 * j + 3] = v.w;
      } else {
        #pragma unroll
        for (int q = 0; q < 4; ++q) raw[4 * j + q] = (e0 + q < c1) ? load_raw(a.logits, a.dtype, rbase + e0 + q) : 0.f;
      }
    }
  }
}

// Which statistics a row needs from the scan (uniform per row).
struct StatNeeds {
  bool ieee;  // greedy rows: block_argmax_last
  bool fin;   // temperature-only rows and the finite-lane greedy rule
};

__device__ __forceinline__ StatNeeds stat_needs(const RowCfg& c, const ParamsView& pv) {
  StatNeeds n;
  n.ieee = c.cls == kGreedy && pv.greedy_rule == kGreedyIeee;
  n.fin = c.cls == kTempOnly || (c.cls == kGreedy && pv.greedy_rule == kGreedyFiniteLane);
  return n;
}

// Statistics update for one processed logit l at index e.  The maximum is
// tracked on the order key of l (non-finite l maps to the key of -inf),
// which also tells whether any finite value exists.
__device__ __forceinline__ void stat_add(ChunkStat& st, const StatNeeds& nd, uint32_t& maxkey,
                                         float l, uint32_t kl, uint32_t e) {
  maxkey = max(maxkey, kl);
  if (nd.ieee && l > st.am_ieee_v) { st.am_ieee_v = l; st.am_ieee_i = e; }
  if (nd.fin && finitef_(l) &&
      (st.am_fin_i == 0xffffffffu || l > st.am_fin_v ||
       (l == st.am_fin_v && (e & 255u) < (st.am_fin_i & 255u)))) {
    st.am_fin_v = l; st.am_fin_i = e;
  }
}


// History count of token `id` from the chunk's LDS hash (linear probing);
// `found` is false when the hash overflowed before the token was inserted.
__device__ __forceinline__ uint32_t hash_count(const uint32_t* hkey, const uint32_t* hcnt,
                                               uint32_t id, bool& found) {
  uint32_t slot = (id * 2654435761u) & (kHashCap - 1);
  for (int p = 0; p < kHashCap; ++p) {
    const uint32_t kk = hkey[slot];
    if (kk == id) { found = true; return hcnt[slot]; }
    if (kk == 0xffffffffu) break;
    slot = (slot + 1) & (kHashCap - 1);
  }
  found = false;
  return 0u;
}

// Block reduction of (min u64, max u32, f32 sum): the chunk's smallest kept
// candidate, largest dropped key and dropped log-sum-exp mass.
__device__ __forceinline__ void block_tail3(uint64_t& mn, uint32_t& mx, float& sum, ScanLds& sh) {
  uint64_t a = ~mn;
  for (int o = 32; o > 0; o >>= 1) {
    const uint64_t t = shfl_xor_u64(a, o);
    a = t > a ? t : a;
    mx = max(mx, (uint32_t)__shfl_xor(mx, o, 64));
    sum += __shfl_xor(sum, o, 64);
  }
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  __syncthreads();
  if (lane == 0) { sh.red64[wid] = a; sh.redu[wid] = mx; sh.redf[wid] = sum; }
  __syncthreads();
  a = sh.red64[0]; mx = sh.redu[0]; sum = sh.redf[0];
  for (int i = 1; i < NT / 64; ++i) {
    a = sh.red64[i] > a ? sh.red64[i] : a;
    mx = max(mx, sh.redu[i]);
    sum += sh.redf[i];
  }
  mn = ~a;
}

// ==========================================================================
// Lean scan path (every row class when at most kLeanK logprobs are asked)
// ==========================================================================
//
// Every wave keeps its own running top-(k+1) of the elements it streams, in
// its own LDS buffer, with a wave-uniform threshold: an element below the
// threshold costs a compare, survivors are appended with ballot/mbcnt, and a
// buffer that passes its limit is compacted by a wave-level radix select.
// No workgroup barrier runs inside the tile loop.  At the end wave 0 merges
// the four per-wave sets into the range's top k.  Selection entries are the
// 64-bit candidate keys (scaled-logit key, inverted index).

constexpr int kLeanVec = 2;                     // float4 loads per thread per tile
constexpr int kWaveCap = 1024;                  // per-wave buffer entries
constexpr int kWaveMaxLim = kWaveCap - kLeanVec * 4 * 64;  // a tile's survivors fit above the limit
static_assert(kLeanK + 1 <= kWaveMaxLim, "a compacted buffer is below the limit");
constexpr uint32_t kChunkHistCap = 1024;        // distinct history tokens counted in LDS per chunk
constexpr uint32_t kRowHistCap = 4096;          // ... per row (row kernel)

template <int NW>
struct LeanLds {
  uint64_t wbuf[NW][kWaveCap];
  uint32_t whist[NW][256];
  uint32_t wcount[NW];
  uint32_t wmax[NW];
  float wbv[NW];
  uint32_t wbi[NW];
  float wrest[NW];
  float wlref[NW];
  float wfv[NW];
  uint32_t wfi[NW];
};

// Orders this wave's LDS accesses (a wave executes its LDS operations in
// order; this keeps the compiler from moving them across the point).
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Number of set bits of m below the calling lane.
__device__ __forceinline__ uint32_t lanes_below(uint64_t m) {
  return __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
}

// Up to NS LDS arrays of candidate keys, read as one list.
template <int NS>
struct Segs {
  const uint64_t* p[NS];
  uint32_t n[NS];
  int ns;
};

// Threshold T such that exactly `need` of the listed entries (unique keys)
// are >= T, for 1 <= need <= the number of entries.  8-bit MSD descent with
// early exit over a 256-bin LDS histogram owned by the wave.
template <int NS>
__device__ __forceinline__ uint64_t wave_select(const Segs<NS>& sg, uint32_t need, uint32_t* hist) {
  const uint32_t lane = threadIdx.x & 63u;
  uint64_t prefix = 0;
  uint32_t remaining = need;
  #pragma unroll 1
  for (int shift = 56; shift >= 0; shift -= 8) {
    wave_lds_sync();
    *reinterpret_cast<uint4*>(hist + 4 * lane) = make_uint4(0u, 0u, 0u, 0u);
    wave_lds_sync();
    const int hs = shift + 8;
    const uint64_t hp = hs >= 64 ? 0ull : (prefix >> hs);
    #pragma unroll
    for (int sgi = 0; sgi < NS; ++sgi) {
      if (sgi >= sg.ns) break;
      const uint64_t* p = sg.p[sgi];
      const uint32_t n = sg.n[sgi];
      #pragma unroll 2
      for (uint32_t i = lane; i < n; i += 64u) {
        const uint64_t x = p[i];
        if (hs >= 64 || (x >> hs) == hp) atomicAdd(&hist[(uint32_t)(x >> shift) & 255u], 1u);
      }
    }
    wave_lds_sync();
    // lane l owns bins 255-4l, 254-4l, 253-4l, 252-4l (descending)
    const uint4 h = *reinterpret_cast<const uint4*>(hist + 252 - 4 * lane);
    const uint32_t cs[4] = {h.w, h.z, h.y, h.x};
    const uint32_t lsum = cs[0] + cs[1] + cs[2] + cs[3];
    uint32_t inc = lsum;
    #pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const uint32_t t = (uint32_t)__shfl_up((int)inc, o, 64);
      if (lane >= (uint32_t)o) inc += t;
    }
    uint32_t acc = inc - lsum, d = 0, da = 0, dc = 0;
    #pragma unroll
    for (int q = 0; q < 4; ++q) {
      if (acc < remaining && remaining <= acc + cs[q]) { d = 255u - 4u * lane - (uint32_t)q; da = acc; dc = cs[q]; }
      acc += cs[q];
    }
    const uint64_t who = __ballot(inc - lsum < remaining && remaining <= inc);
    const int src = __ffsll((unsigned long long)who) - 1;
    d = (uint32_t)__builtin_amdgcn_readlane((int)d, src);
    da = (uint32_t)__builtin_amdgcn_readlane((int)da, src);
    dc = (uint32_t)__builtin_amdgcn_readlane((int)dc, src);
    prefix |= (uint64_t)d << shift;
    remaining -= da;
    if (dc == remaining) break;
  }
  return prefix;
}

// Rest of the normaliser over the elements a range does not keep, per lane:
// sum of 2^((l - lref) * a2) with a2 = log2(e) / T and a wave-uniform
// reference lref that only grows (the value of the current threshold key).
struct LseRest {
  float sum, lref, a2;
  __device__ __forceinline__ void add(float l) { sum += exp2f((l - lref) * a2); }
  __device__ __forceinline__ void add_key(uint32_t key) {
    if (key > kKeyNegInf) add(okey_inv(key));
  }
  __device__ __forceinline__ void move_ref(uint32_t tk) {
    if (tk <= kKeyNegInf) return;
    const float nl = okey_inv(tk);
    if (finitef_(lref)) sum *= exp2f((lref - nl) * a2);
    else sum = 0.f;
    lref = nl;
  }
};

// Running per-wave selection of the top k1 candidate keys.
struct WaveSel {
  uint64_t* buf;
  uint32_t* hist;
  uint32_t count;   // entries in buf (wave-uniform)
  uint32_t k1;      // entries a compaction keeps
  uint32_t lim;     // compaction trigger
  uint64_t tau;     // keys below tau are not among the wave's top k1
  uint32_t tk;      // scaled-logit key threshold: max(1, tau >> 32)
};

// Compact the wave's buffer to its top k1 (in place, in order) and raise
// the threshold.
__device__ __forceinline__ void wave_compact(WaveSel& ws, LseRest& rest, bool lse) {
  const uint32_t lane = threadIdx.x & 63u;
  const uint32_t n = ws.count;
  if (n <= ws.k1) return;
  Segs<1> sg;
  sg.p[0] = ws.buf;
  sg.n[0] = n;
  sg.ns = 1;
  const uint64_t thr = wave_select(sg, ws.k1, ws.hist);
  if (thr > ws.tau) ws.tau = thr;
  ws.tk = max(1u, (uint32_t)(ws.tau >> 32));
  if (lse) rest.move_ref(ws.tk);
  wave_lds_sync();
  uint32_t pos = 0;
  // entry i moves to a position <= i, and a block of 64 is read before any
  // of its writes, so the compaction can run in place
  #pragma unroll 1
  for (uint32_t b = 0; b < n; b += 64u) {
    const uint32_t i = b + lane;
    const bool valid = i < n;
    const uint64_t x = valid ? ws.buf[i] : 0ull;
    const bool keep = valid && x >= thr;
    const uint64_t m = __ballot(keep);
    if (keep) ws.buf[pos + lanes_below(m)] = x;
    else if (lse && valid) rest.add_key(cand_skey(x));
    pos += (uint32_t)__popcll(m);
  }
  ws.count = pos;
}

// History tokens of [base, base + len) as seen by the lean path: bit li of
// `bitmap` marks token base + li, prefix[w] counts the marked tokens of the
// words below w, and cnts[r] is the summed count of the marked token of rank
// r (for r < cap; higher ranks are counted from the global list).
struct HistView {
  const uint32_t* bitmap;
  const uint32_t* prefix;
  uint32_t* cnts;         // counts by rank; the lean pass then keeps keys there
  const uint32_t* ids;    // ids[r]: the marked token of rank r (r < min(distinct, cap))
  uint32_t cap;
  uint32_t distinct;      // marked tokens
  uint32_t h0, h1;
  bool on;
  bool ovf;               // more marked tokens than cap
};

// LDS bytes of a HistView over `len` tokens with `cap` counted tokens
// (bitmap, prefix, counts + a zero slot, ids, 16 reduction words).
__host__ __device__ constexpr size_t hist_lds_bytes(int len, uint32_t cap) {
  return (size_t)2 * ((len + 31) / 32) * 4 + (size_t)(2 * cap + 1) * 4 + 64;
}

// Builds the HistView of row `row` over [base, base + len) in `mem`.  All
// NTH threads of the workgroup call it.
template <int NTH>
__device__ __forceinline__ HistView stage_history_rank(const SampleArgs& a, int row, int base, int len,
                                                       uint32_t cap, uint32_t* mem) {
  const int tid = threadIdx.x;
  const int W = (len + 31) / 32;
  uint32_t* bitmap = mem;
  uint32_t* prefix = mem + W;
  uint32_t* cnts = mem + 2 * W;   // cap counts, then a zero slot at cnts[cap]
  uint32_t* ids = cnts + cap + 1;
  uint32_t* red = ids + cap;
  HistView hv;
  hv.bitmap = bitmap; hv.prefix = prefix; hv.cnts = cnts; hv.ids = ids; hv.cap = cap;
  hv.distinct = 0u;
  hv.h0 = a.hoff[row];
  hv.h1 = a.hoff[row + 1];
  hv.on = hv.h1 > hv.h0;
  hv.ovf = false;
  if (!hv.on) return hv;
  const uint32_t h0 = hv.h0, h1 = hv.h1;
  for (int i = tid; i < W; i += NTH) bitmap[i] = 0u;
  __syncthreads();
  constexpr int PER = 8;
  const bool one = h1 - h0 <= (uint32_t)(NTH * PER);
  uint32_t hid[PER], cs[PER];
  for (uint32_t hb = h0; hb < h1; hb += NTH * PER) {
    #pragma unroll
    for (int r = 0; r < PER; ++r) {  // independent loads first
      const uint32_t h = hb + r * NTH + tid;
      hid[r] = h < h1 ? a.hids[h] : 0xffffffffu;
      cs[r] = h < h1 ? a.hcnt[h] : 0u;
    }
    #pragma unroll
    for (int r = 0; r < PER; ++r) {
      const uint32_t li = hid[r] - (uint32_t)base;
      if (hid[r] >= (uint32_t)base && li < (uint32_t)len) atomicOr(&bitmap[li >> 5], 1u << (li & 31u));
    }
  }
  __syncthreads();
  // exclusive prefix of the per-word popcounts
  const int PW = (W + NTH - 1) / NTH;
  uint32_t loc = 0;
  for (int i = 0; i < PW; ++i) {
    const int w = tid * PW + i;
    if (w < W) loc += (uint32_t)__popc(bitmap[w]);
  }
  uint32_t total;
  uint32_t run = block_excl_scan_u32<NTH>(loc, red, &total);
  for (int i = 0; i < PW; ++i) {
    const int w = tid * PW + i;
    if (w < W) { prefix[w] = run; run += (uint32_t)__popc(bitmap[w]); }
  }
  const uint32_t nz = min(total, cap);
  hv.ovf = total > cap;
  hv.distinct = total;
  for (uint32_t i = tid; i < nz; i += NTH) cnts[i] = 0u;
  if (tid == 0) cnts[cap] = 0u;
  __syncthreads();
  for (uint32_t hb = h0; hb < h1; hb += NTH * PER) {
    if (!one) {
      #pragma unroll
      for (int r = 0; r < PER; ++r) {
        const uint32_t h = hb + r * NTH + tid;
        hid[r] = h < h1 ? a.hids[h] : 0xffffffffu;
        cs[r] = h < h1 ? a.hcnt[h] : 0u;
      }
    }
    #pragma unroll
    for (int r = 0; r < PER; ++r) {
      const uint32_t li = hid[r] - (uint32_t)base;
      if (hid[r] >= (uint32_t)base && li < (uint32_t)len) {
        const uint32_t w = li >> 5;
        const uint32_t rank = prefix[w] + (uint32_t)__popc(bitmap[w] & ((1u << (li & 31u)) - 1u));
        if (rank < cap) {
          atomicAdd(&cnts[rank], cs[r]);
          ids[rank] = (uint32_t)base + li;  // every occurrence writes the same id
        }
      }
    }
  }
  __syncthreads();
  return hv;
}

// History count of the marked token e of rank `rank`.  OVF: the table may
// not hold every marked token; the others are counted from the global list.
template <bool OVF>
__device__ __forceinline__ uint32_t hist_count(const SampleArgs& a, const HistView& hv, uint32_t e,
                                               uint32_t rank) {
  if (!OVF || rank < hv.cap) return hv.cnts[rank];
  uint32_t cnt = 0u;
  for (uint32_t h = hv.h0; h < hv.h1; ++h) if (a.hids[h] == e) cnt += a.hcnt[h];
  return cnt;
}

// f(x) with x - lref <= 0 relevant only where `use` holds (0 elsewhere).
__device__ __forceinline__ float masked_exp2(bool use, float v) { return use ? exp2f(v) : 0.f; }

// Range-checked loads of one row (byte offsets at or past the range read
// as zero; nothing faults).
typedef int i32x4_t __attribute__((ext_vector_type(4)));
typedef int i32x2_t __attribute__((ext_vector_type(2)));
constexpr int kBufferConfig = 0x00020000;  // raw buffer, 32-bit data (gfx9 family)

struct RowBuf {
  __amdgpu_buffer_rsrc_t logits, mask;
};

// Range [c0, c1) of `row` (c0 a multiple of 32).
template <int DT, bool MASK>
__device__ __forceinline__ RowBuf row_buf(const SampleArgs& a, int row, int c0, int c1) {
  RowBuf rb;
  const int esize = DT == HI_ROCM_DTYPE_BF16 ? 2 : 4;
  const char* base = (const char*)a.logits + ((int64_t)row * a.row_stride + c0) * esize;
  rb.logits = __builtin_amdgcn_make_buffer_rsrc((void*)base, (short)0, (c1 - c0) * esize, kBufferConfig);
  if (MASK)
    rb.mask = __builtin_amdgcn_make_buffer_rsrc((void*)(a.mask + (int64_t)row * a.mask_words + (c0 >> 5)),
                                                (short)0, ((c1 - c0 + 31) >> 5) * 4, kBufferConfig);
  return rb;
}

// One tile at offset tr from the range start (element tr + (j * NTH + tid)
// * 4 + q in x[4 * j + q]); needs 16-byte (f32) or 8-byte (bf16) aligned
// rows.
template <int NTH, int VEC, int DT, bool MASK>
__device__ __forceinline__ void buf_load(const RowBuf& rb, int tr, float (&x)[VEC * 4], uint32_t (&mw)[VEC]) {
  const int tid = threadIdx.x;
  #pragma unroll
  for (int j = 0; j < VEC; ++j) {
    const int e0 = tr + (j * NTH + tid) * 4;
    if (DT == HI_ROCM_DTYPE_BF16) {
      const i32x2_t v = __builtin_amdgcn_raw_buffer_load_b64(rb.logits, e0 * 2, 0, 0);
      x[4 * j + 0] = __uint_as_float((uint32_t)v.x << 16); x[4 * j + 1] = __uint_as_float((uint32_t)v.x & 0xffff0000u);
      x[4 * j + 2] = __uint_as_float((uint32_t)v.y << 16); x[4 * j + 3] = __uint_as_float((uint32_t)v.y & 0xffff0000u);
    } else {
      const i32x4_t v = __builtin_amdgcn_raw_buffer_load_b128(rb.logits, e0 * 4, 0, 0);
      x[4 * j + 0] = __int_as_float(v.x); x[4 * j + 1] = __int_as_float(v.y);
      x[4 * j + 2] = __int_as_float(v.z); x[4 * j + 3] = __int_as_float(v.w);
    }
    if (MASK) mw[j] = (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(rb.mask, (e0 >> 5) * 4, 0, 0);
  }
}

// Argmax merges: IEEE '>' with ties to the lower index (kernels.cu:7153-7186),
// and the finite-lane rule of kernels.cu:7775-7801 (ties to the lower
// index modulo 256, then the lower index).
__device__ __forceinline__ void merge_ieee(float& v, uint32_t& i, float ov, uint32_t oi) {
  if (oi != 0xffffffffu && (i == 0xffffffffu || ov > v || (ov == v && oi < i))) { v = ov; i = oi; }
}
__device__ __forceinline__ void merge_fin(float& v, uint32_t& i, float ov, uint32_t oi) {
  if (oi == 0xffffffffu) return;
  bool take = i == 0xffffffffu || ov > v;
  if (!take && ov == v) {
    const uint32_t ra = i & 255u, rb = oi & 255u;
    take = rb < ra || (rb == ra && oi < i);
  }
  if (take) { v = ov; i = oi; }
}

// Per-wave results written before the workgroup barrier of the merge.
struct WaveOut {
  uint32_t count, maxkey;
  float bv;
  uint32_t bi;
  float fv;
  uint32_t fi;
  float rest, lref;
};

template <int NW>
__device__ __forceinline__ void wave_results(LeanLds<NW>& L, int wid, WaveOut o, bool ieee, bool fin,
                                             bool lse) {
  #pragma unroll
  for (int s = 32; s > 0; s >>= 1) {
    o.maxkey = max(o.maxkey, (uint32_t)__shfl_xor((int)o.maxkey, s, 64));
    if (ieee) merge_ieee(o.bv, o.bi, __shfl_xor(o.bv, s, 64), (uint32_t)__shfl_xor((int)o.bi, s, 64));
    if (fin) merge_fin(o.fv, o.fi, __shfl_xor(o.fv, s, 64), (uint32_t)__shfl_xor((int)o.fi, s, 64));
    if (lse) o.rest += __shfl_xor(o.rest, s, 64);
  }
  if ((threadIdx.x & 63) == 0) {
    L.wcount[wid] = o.count;
    L.wmax[wid] = o.maxkey;
    L.wbv[wid] = o.bv;
    L.wbi[wid] = o.bi;
    L.wfv[wid] = o.fv;
    L.wfi[wid] = o.fi;
    L.wrest[wid] = o.rest;
    L.wlref[wid] = o.lref;
  }
}

// Per-wave state of the lean pass.
struct LeanState {
  WaveSel ws;
  LseRest rest;
  uint32_t maxkey;
  float bv, fv;
  uint32_t bi, fi;
};

// Constant context of the lean pass over [c0, c1) of `row`.
struct LeanCtx {
  const SampleArgs* a;
  const RowCfg* cfg;
  const HistView* hv;
  float* srow;      // scaled logits for the finish, or null
  int c0, c1, len;
  uint32_t k;       // candidates to keep (k_sel)
  bool ieee, fin, lse, rep_once;
};

// One tile of the lean pass: mask, penalties, keys, statistics, survivors.
// cur holds the tile's logits (element tb + (j * NTH + tid) * 4 + q in
// cur[4 * j + q]); first: the range's first tile.
template <int NTH, int VEC, bool MASK, bool OVF>
__device__ __forceinline__ void lean_tile(const LeanCtx& x, LeanState& st, float (&cur)[VEC * 4],
                                          const uint32_t (&mw)[VEC], int tb, bool first) {
  constexpr int TILE = NTH * VEC * 4;
  constexpr int E = VEC * 4;
  const SampleArgs& a = *x.a;
  const RowCfg& cfg = *x.cfg;
  const HistView& hv = *x.hv;
  const int tid = threadIdx.x;
  const uint32_t lane = (uint32_t)tid & 63u;
  const int c0 = x.c0, c1 = x.c1;
  const bool full = tb + TILE <= c1;
  WaveSel& ws = st.ws;
  if (MASK) {
    #pragma unroll
    for (int j = 0; j < VEC; ++j) {
      const int e0 = tb + (j * NTH + tid) * 4;
      const uint32_t nib = mw[j] >> (e0 & 31);
      #pragma unroll
      for (int q = 0; q < 4; ++q) if (!((nib >> q) & 1u)) cur[4 * j + q] = -__builtin_inff();
    }
  }
  // elements this tile does not stream: past the range, and (without OVF)
  // history tokens, which the lean pass handles on their own
  uint32_t drop[VEC];
  bool anyd = false;
  #pragma unroll
  for (int j = 0; j < VEC; ++j) {
    const int e0 = tb + (j * NTH + tid) * 4;
    drop[j] = full ? 0u : (e0 + 3 < c1 ? 0u : (0xfu << max(0, min(4, c1 - e0))) & 0xfu);
  }
  if (hv.on) {
    uint32_t wb[VEC];
    bool anyf = false;
    #pragma unroll
    for (int j = 0; j < VEC; ++j) {
      const uint32_t li0 = (uint32_t)(tb - c0 + (j * NTH + tid) * 4);
      wb[j] = li0 < (uint32_t)x.len ? hv.bitmap[li0 >> 5] : 0u;
      anyf |= ((wb[j] >> (li0 & 31u)) & 15u) != 0u;
    }
    if (!OVF) {
      #pragma unroll
      for (int j = 0; j < VEC; ++j) {
        const uint32_t li0 = (uint32_t)(tb - c0 + (j * NTH + tid) * 4);
        drop[j] |= (wb[j] >> (li0 & 31u)) & 15u;
      }
    } else if (__ballot(anyf) != 0ull) {
      // counts of the marked elements; the others read the zero slot
      // cnts[cap] (tokens of rank >= cap count from the global list)
      const uint32_t W = (uint32_t)(x.len + 31) >> 5;
      uint32_t cnt[E];
      uint32_t most = 0u;
      #pragma unroll
      for (int j = 0; j < VEC; ++j) {
        const uint32_t li0 = (uint32_t)(tb - c0 + (j * NTH + tid) * 4);
        const uint32_t sh = li0 & 31u;
        const uint32_t nib = (wb[j] >> sh) & 15u;
        const uint32_t base = hv.prefix[min(li0 >> 5, W - 1u)] + (uint32_t)__popc(wb[j] & ((1u << sh) - 1u));
        #pragma unroll
        for (int q = 0; q < 4; ++q) {
          const bool m = (nib >> q) & 1u;
          const uint32_t r = base + (uint32_t)__popc(nib & ((1u << q) - 1u));
          cnt[4 * j + q] = m ? hist_count<true>(a, hv, (uint32_t)c0 + li0 + (uint32_t)q, r) : 0u;
          most = max(most, cnt[4 * j + q]);
        }
      }
      // repetition penalty once per occurrence (or once), then the
      // frequency and presence penalties (apply_penalties, element-wise)
      if (cfg.rep_on) {
        const uint32_t reps = x.rep_once ? min(most, 1u) : most;
        #pragma unroll 1
        for (uint32_t rr = 0; rr < reps; ++rr) {
          #pragma unroll
          for (int i = 0; i < E; ++i) {
            const uint32_t ci = x.rep_once ? min(cnt[i], 1u) : cnt[i];
            const float y = cur[i] < 0.f ? cur[i] * cfg.rep : cur[i] / cfg.rep;
            cur[i] = rr < ci ? y : cur[i];
          }
        }
      }
      #pragma unroll
      for (int i = 0; i < E; ++i) {
        const float fc = cfg.freq * (float)cnt[i];
        const float y = (cur[i] - fc) - cfg.pres;
        cur[i] = cnt[i] != 0u ? y : cur[i];
      }
    }
  }
  #pragma unroll
  for (int j = 0; j < VEC; ++j) anyd |= drop[j] != 0u;
  uint32_t key[E];
  #pragma unroll
  for (int i = 0; i < E; ++i) key[i] = lkey(cur[i]);
  if (__ballot(anyd) != 0ull) {
    #pragma unroll
    for (int i = 0; i < E; ++i) {
      const bool dr = (drop[i >> 2] >> (i & 3)) & 1u;
      key[i] = dr ? 0u : key[i];
      cur[i] = dr ? -__builtin_inff() : cur[i];
    }
  }
  #pragma unroll
  for (int i = 0; i < E; ++i) st.maxkey = max(st.maxkey, key[i]);
  if (x.ieee) {
    #pragma unroll
    for (int i = 0; i < E; ++i) {
      const bool g = cur[i] > st.bv;
      st.bv = g ? cur[i] : st.bv;
      st.bi = g ? (uint32_t)(tb + ((i >> 2) * NTH + tid) * 4 + (i & 3)) : st.bi;
    }
  }
  if (x.fin) {
    // within a lane indices grow, so a tie keeps the earlier index unless
    // the new one has the smaller residue modulo 256
    #pragma unroll
    for (int i = 0; i < E; ++i) {
      const uint32_t e = (uint32_t)(tb + ((i >> 2) * NTH + tid) * 4 + (i & 3));
      const bool g = finitef_(cur[i]) &&
                     (st.fi == 0xffffffffu || cur[i] > st.fv || (cur[i] == st.fv && (e & 255u) < (st.fi & 255u)));
      st.fv = g ? cur[i] : st.fv;
      st.fi = g ? e : st.fi;
    }
  }
  if (x.srow) {
    // scaled logits s = l / T for the finish (non-finite -> -inf)
    #pragma unroll
    for (int j = 0; j < VEC; ++j) {
      const int e0 = tb + (j * NTH + tid) * 4;
      float sv[4];
      #pragma unroll
      for (int q = 0; q < 4; ++q) sv[q] = key_to_s(key[4 * j + q] ? key[4 * j + q] : kKeyNegInf, cfg.t_eff);
      if (full && (a.V & 3) == 0) {
        *(float4*)(x.srow + e0) = make_float4(sv[0], sv[1], sv[2], sv[3]);
      } else {
        #pragma unroll
        for (int q = 0; q < 4; ++q) if (e0 + q < c1) x.srow[e0 + q] = sv[q];
      }
    }
  }
  if (x.k == 0u) return;
  if (first && ws.k1 <= 256u) {
    // bound from this wave's first tile: the k1-th largest of the per-lane
    // top-jt keys, rounded down to 16 bits (at least k1 of the wave's
    // elements are at or above it)
    const int jt = (int)((ws.k1 + 63u) >> 6);
    uint32_t t4[4] = {0u, 0u, 0u, 0u};
    if (jt == 1) {
      #pragma unroll
      for (int i = 0; i < E; ++i) t4[0] = max(t4[0], key[i]);
    } else {
      #pragma unroll
      for (int i = 0; i < E; ++i) {
        uint32_t v = key[i];
        #pragma unroll
        for (int r = 0; r < 4; ++r) {
          const uint32_t hi = max(t4[r], v);
          v = min(t4[r], v);
          t4[r] = hi;
        }
      }
    }
    uint32_t prefix = 0u;
    #pragma unroll 1
    for (int bit = 31; bit >= 16; --bit) {
      const uint32_t probe = prefix | (1u << bit);
      uint32_t c = 0u;
      #pragma unroll
      for (int r = 0; r < 4; ++r)
        if (r < jt) c += (uint32_t)__popcll(__ballot(t4[r] >= probe));
      if (c >= ws.k1) prefix = probe;
    }
    if (prefix > 1u) {
      ws.tau = (uint64_t)prefix << 32;
      ws.tk = prefix;
      if (x.lse) st.rest.move_ref(ws.tk);
    }
  }
  // survivors of the tile (<= 64 * E entries: count <= lim before, so they
  // fit); compact when the buffer passes its limit
  uint64_t m[E];
  uint64_t any = 0ull;
  #pragma unroll
  for (int i = 0; i < E; ++i) { m[i] = __ballot(key[i] >= ws.tk); any |= m[i]; }
  if (x.lse) {
    // the elements below the threshold leave the selection here
    float add = 0.f;
    #pragma unroll
    for (int i = 0; i < E; ++i)
      add += masked_exp2(key[i] < ws.tk && key[i] > kKeyNegInf, (cur[i] - st.rest.lref) * st.rest.a2);
    st.rest.sum += add;
  }
  if (any != 0ull) {
    #pragma unroll
    for (int i = 0; i < E; ++i) {
      if (key[i] >= ws.tk)
        ws.buf[ws.count + lanes_below(m[i])] = cand_key(key[i], (uint32_t)(tb + ((i >> 2) * NTH + tid) * 4 + (i & 3)));
      ws.count += (uint32_t)__popcll(m[i]);
    }
    if (ws.count > ws.lim) wave_compact(ws, st.rest, x.lse);
  }
}

// Tiles t0 + d .. t0 + D - 1 of one pipeline round: process buffer d, then
// load tile t0 + d + D into it (past the range the loads read zeros).
template <int d, int NTH, int VEC, int D, int DT, bool MASK, bool OVF>
__device__ __forceinline__ void lean_round(const LeanCtx& x, LeanState& st, const RowBuf& rb,
                                           float (&tl)[D][VEC * 4], uint32_t (&tmw)[D][VEC], int t0) {
  constexpr int TILE = NTH * VEC * 4;
  const int tb = x.c0 + (t0 + d) * TILE;
  lean_tile<NTH, VEC, MASK, OVF>(x, st, tl[d], tmw[d], tb, d == 0 && t0 == 0);
  buf_load<NTH, VEC, DT, MASK>(rb, tb - x.c0 + D * TILE, tl[d], tmw[d]);
  if constexpr (d + 1 < D) lean_round<d + 1, NTH, VEC, D, DT, MASK, OVF>(x, st, rb, tl, tmw, t0);
}

// Streams [c0, c1) of `row` in tiles of NTH * VEC * 4 logits with D tiles of
// loads in flight per thread: tl[d] holds tile d on entry (the caller issues
// those loads first).  Writes the range's record to stats[slot] and its
// candidates to cand[slot * kFast ...].  Every thread returns after the
// workgroup barrier.
template <int NTH, int VEC, int D, int DT, bool MASK, bool OVF>
__device__ __forceinline__ void scan_lean(const SampleArgs& a, const RowCfg& cfg, LeanLds<NTH / 64>& L,
                                          const RowBuf& rb,
                                          float (&tl)[D][VEC * 4], uint32_t (&tmw)[D][VEC],
                                          const HistView& hv, int row, int64_t slot, int c0, int c1) {
  constexpr int TILE = NTH * VEC * 4;
  constexpr int NW = NTH / 64;
  const int tid = threadIdx.x;
  const uint32_t lane = (uint32_t)tid & 63u;
  const int wid = tid >> 6;
  LeanCtx x;
  x.a = &a; x.cfg = &cfg; x.hv = &hv;
  x.srow = cfg.store_s ? a.ws_s + (int64_t)row * a.V : nullptr;
  x.c0 = c0; x.c1 = c1; x.len = c1 - c0;
  x.k = (uint32_t)cfg.k_sel;
  x.ieee = cfg.cls == kGreedy && a.pv.greedy_rule == kGreedyIeee;
  x.fin = cfg.cls == kTempOnly || (cfg.cls == kGreedy && a.pv.greedy_rule == kGreedyFiniteLane);
  x.lse = a.need_lse != 0;
  x.rep_once = (cfg.flags & HI_ROCM_FLAG_REP_ONCE) != 0u;
  const uint32_t k = x.k;
  const bool ieee = x.ieee, fin = x.fin;
  const int len = x.len;
  const int ntiles = (len + TILE - 1) / TILE;

  LeanState st;
  WaveSel& ws = st.ws;
  ws.buf = L.wbuf[wid];
  ws.hist = L.whist[wid];
  ws.count = 0u;
  ws.k1 = k + 1u;
  ws.lim = min((uint32_t)kWaveMaxLim, ws.k1 + max(ws.k1, 192u));
  ws.tau = 0ull;
  ws.tk = 1u;
  LseRest& rest = st.rest;
  rest.sum = 0.f;
  rest.lref = -__builtin_inff();
  rest.a2 = 1.4426950408889634f / cfg.t_eff;
  st.maxkey = 0u;
  st.bv = -__builtin_inff(); st.fv = -__builtin_inff();
  st.bi = 0xffffffffu; st.fi = 0xffffffffu;

  // history tokens (without OVF the tiles skip them): gather each marked
  // token's logit, apply the mask and the penalties exactly, and enter it
  // like a streamed element; its key replaces its count in hv.cnts
  float pbv = -__builtin_inff(), pfv = -__builtin_inff();
  uint32_t pbi = 0xffffffffu, pfi = 0xffffffffu;
  if (!OVF && hv.on) {
    const uint32_t nd = hv.distinct;
    #pragma unroll 1
    for (uint32_t r0 = (uint32_t)wid * 64u; r0 < nd; r0 += NTH) {
      const uint32_t r = r0 + lane;
      const bool v = r < nd;
      const uint32_t e = v ? hv.ids[r] : (uint32_t)c0;
      const uint32_t off = e - (uint32_t)c0;
      float l;
      if (DT == HI_ROCM_DTYPE_BF16)
        l = __uint_as_float((uint32_t)(uint16_t)__builtin_amdgcn_raw_buffer_load_b16(rb.logits, off * 2, 0, 0) << 16);
      else
        l = __int_as_float(__builtin_amdgcn_raw_buffer_load_b32(rb.logits, off * 4, 0, 0));
      if (MASK) {
        const uint32_t w = (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(rb.mask, (off >> 5) * 4, 0, 0);
        if (!((w >> (off & 31u)) & 1u)) l = -__builtin_inff();
      }
      l = apply_penalties(l, v ? hv.cnts[r] : 0u, cfg);
      const uint32_t key = v ? lkey(l) : 0u;
      if (v) hv.cnts[r] = key;
      l = v ? l : -__builtin_inff();
      st.maxkey = max(st.maxkey, key);
      if (ieee && l > -__builtin_inff()) merge_ieee(pbv, pbi, l, e);
      if (fin && finitef_(l)) merge_fin(pfv, pfi, l, e);
      if (k > 0u) {
        const uint64_t m = __ballot(key >= ws.tk);
        if (key >= ws.tk) ws.buf[ws.count + lanes_below(m)] = cand_key(key, e);
        ws.count += (uint32_t)__popcll(m);
        if (ws.count > ws.lim) wave_compact(ws, rest, x.lse);
      }
    }
  }

  #pragma unroll 1
  for (int t0 = 0; t0 < ntiles; t0 += D) lean_round<0, NTH, VEC, D, DT, MASK, OVF>(x, st, rb, tl, tmw, t0);

  uint32_t maxkey = st.maxkey;
  float bv = st.bv, fv = st.fv;
  uint32_t bi = st.bi, fi = st.fi;
  merge_ieee(bv, bi, pbv, pbi);
  merge_fin(fv, fi, pfv, pfi);
  if (k > 0u) wave_compact(ws, rest, x.lse);
  {
    WaveOut o;
    o.count = ws.count; o.maxkey = maxkey; o.bv = bv; o.bi = bi; o.fv = fv; o.fi = fi;
    o.rest = rest.sum; o.lref = rest.lref;
    wave_results(L, wid, o, ieee, fin, x.lse);
  }
  __syncthreads();
  if (!OVF && hv.on && x.srow) {
    // the tiles stored -inf for the history tokens; store their s now
    for (uint32_t r = (uint32_t)tid; r < hv.distinct; r += NTH) x.srow[hv.ids[r]] = key_to_s(hv.cnts[r], cfg.t_eff);
  }
  if (wid != 0) return;

  // wave 0: merge the per-wave sets into the range's top k
  ChunkStat bs;
  stat_init(bs);
  maxkey = 0u;
  #pragma unroll
  for (int w = 0; w < NW; ++w) maxkey = max(maxkey, L.wmax[w]);
  bs.max_l = maxkey > kKeyNegInf ? okey_inv(maxkey) : -__builtin_inff();
  bs.any_finite = maxkey > kKeyNegInf ? 1u : 0u;
  if (ieee) {
    #pragma unroll
    for (int w = 0; w < NW; ++w) merge_ieee(bs.am_ieee_v, bs.am_ieee_i, L.wbv[w], L.wbi[w]);
  }
  if (fin) {
    #pragma unroll
    for (int w = 0; w < NW; ++w) merge_fin(bs.am_fin_v, bs.am_fin_i, L.wfv[w], L.wfi[w]);
  }
  if (k > 0u) {
    Segs<NW> sg;
    uint32_t total = 0u;
    #pragma unroll
    for (int w = 0; w < NW; ++w) { sg.p[w] = L.wbuf[w]; sg.n[w] = L.wcount[w]; total += sg.n[w]; }
    sg.ns = NW;
    uint64_t thr = 0ull;
    if (total > k) thr = wave_select(sg, k, L.whist[0]);
    // the dropped mass relative to the range max
    const float lmax = bs.max_l;
    float part = 0.f;
    const bool LSE = x.lse;
    if (LSE && finitef_(lmax)) {
      #pragma unroll
      for (int w = 0; w < NW; ++w)
        if (L.wrest[w] > 0.f && finitef_(L.wlref[w]))
          part += L.wrest[w] * exp2f((L.wlref[w] - lmax) * rest.a2);
    }
    float lane_part = 0.f;
    uint64_t* cand = a.cand + slot * kFast;
    uint32_t pos = 0u, unkept = 0u;
    uint64_t minkept = ~0ull;
    #pragma unroll
    for (int w = 0; w < NW; ++w) {
      const uint32_t n = sg.n[w];
      #pragma unroll 1
      for (uint32_t b = 0; b < n; b += 64u) {
        const uint32_t i = b + lane;
        const bool valid = i < n;
        const uint64_t x = valid ? sg.p[w][i] : 0ull;
        const bool keep = valid && x >= thr;
        const uint64_t m = __ballot(keep);
        if (keep) {
          cand[pos + lanes_below(m)] = x;
          minkept = x < minkept ? x : minkept;
        } else if (valid) {
          const uint32_t kv = cand_skey(x);
          unkept = max(unkept, kv);
          if (LSE && finitef_(lmax) && kv > kKeyNegInf) lane_part += exp2f((okey_inv(kv) - lmax) * rest.a2);
        }
        pos += (uint32_t)__popcll(m);
      }
    }
    #pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
      const uint64_t t = shfl_xor_u64(minkept, o);
      minkept = t < minkept ? t : minkept;
      unkept = max(unkept, (uint32_t)__shfl_xor((int)unkept, o, 64));
      if (LSE) lane_part += __shfl_xor(lane_part, o, 64);
    }
    bs.n_cand = pos;
    bs.trunc = len > (int)k ? 1u : 0u;
    bs.min_kept = minkept;
    bs.unkept_key = unkept;
    bs.lse_m = finitef_(lmax) ? lmax / cfg.t_eff : -__builtin_inff();
    bs.lse_sum = LSE ? part + lane_part : 0.f;
  }
  if (lane == 0u) a.stats[slot] = bs;
}

// The general per-chunk pass (top-p, min-p, temperature-only and wide rows,
// the finite-lane greedy rule, large logprob counts): block-level running
// selection, scaled logits stored for the finish.
template <int VEC, int TILES>
__device__ __forceinline__ void scan_generic(const SampleArgs& a, const RowCfg& cfg, ScanLds& sh,
                                             const float (&tile0)[VEC * 4],
                                             const uint32_t* bitmap, const uint32_t* hkey,
                                             const uint32_t* hcnt, bool pen, uint32_t h0, uint32_t h1,
                                             int row, int chunk, int c0, int c1) {
  constexpr int TILE = NT * VEC * 4;
  constexpr int E = VEC * 4;
  const int tid = threadIdx.x;
  const int V = a.V;
  const int len = c1 - c0;
  const int64_t rbase = (int64_t)row * a.row_stride;
  const uint32_t* mrow = a.mask ? a.mask + (int64_t)row * a.mask_words : nullptr;
  float* srow = cfg.store_s ? a.ws_s + (int64_t)row * V : nullptr;
  const uint32_t k = (uint32_t)cfg.k_sel;

  float cur[E];
  #pragma unroll
  for (int i = 0; i < E; ++i) cur[i] = tile0[i];
  if (tid == 0) sh.count = 0u;
  __syncthreads();

  SelState ss;
  ss.tau = 0ull;
  ss.unkept = 0u;
  ss.rest.init();
  ss.rest_on = a.need_lse != 0;
  ss.t_eff = cfg.t_eff;
  ChunkStat st;
  stat_init(st);
  const StatNeeds nd = stat_needs(cfg, a.pv);
  uint32_t maxkey = 0u;

  #pragma unroll 1
  for (int t = 0; t < TILES; ++t) {
    const int tb = c0 + t * TILE;
    if (tb >= c1) break;
    float nxt[E];
    if (t + 1 < TILES && tb + TILE < c1) load_tile<VEC>(a, rbase, tb + TILE, c1, nxt);
    uint32_t key[E];  // 0: no element (past the end)
    #pragma unroll
    for (int j = 0; j < VEC; ++j) {
      const int e0 = tb + (j * NT + tid) * 4;
      const uint32_t mword = (mrow && e0 < c1) ? mrow[e0 >> 5] : 0xffffffffu;
      uint32_t flags = 0u;
      if (pen && e0 < c1) flags = (bitmap[(e0 - c0) >> 5] >> ((e0 - c0) & 31)) & 15u;
      #pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int e = e0 + q;
        float l = cur[4 * j + q];
        if (!((mword >> (e & 31)) & 1u)) l = -__builtin_inff();
        if ((flags >> q) & 1u) {
          bool found;
          uint32_t cnt = hash_count(hkey, hcnt, (uint32_t)e, found);
          if (!found) {  // the hash overflowed: count from the global list (slow)
            cnt = 0u;
            for (uint32_t h = h0; h < h1; ++h) if (a.hids[h] == (uint32_t)e) cnt += a.hcnt[h];
          }
          l = apply_penalties(l, cnt, cfg);
        }
        const uint32_t kl = lkey(l);
        const bool in = e < c1;
        if (in) stat_add(st, nd, maxkey, l, kl, (uint32_t)e);
        key[4 * j + q] = in ? kl : 0u;
      }
      if (srow) {
        float sv[4];
        #pragma unroll
        for (int q = 0; q < 4; ++q) sv[q] = key[4 * j + q] ? key_to_s(key[4 * j + q], cfg.t_eff) : -__builtin_inff();
        if (e0 + 3 < c1 && (V & 3) == 0) {
          *(float4*)(srow + e0) = make_float4(sv[0], sv[1], sv[2], sv[3]);
        } else {
          for (int q = 0; q < 4; ++q) if (e0 + q < c1) srow[e0 + q] = sv[q];
        }
      }
    }
    if (k > 0) {
      if (t == 0 && len > (int)k) {
        // bound from the first tile: the k-th largest of the per-thread
        // top-j keys, rounded down to 16 bits (k or more real elements are
        // at or above it)
        const int jt = ((int)k + NT - 1) / NT;  // 1..4
        uint32_t t4[4] = {0u, 0u, 0u, 0u};
        #pragma unroll
        for (int i = 0; i < E; ++i) {
          uint32_t x = key[i];
          #pragma unroll
          for (int r = 0; r < 4; ++r) {
            const uint32_t hi = max(t4[r], x);
            x = min(t4[r], x);
            t4[r] = hi;
          }
        }
        for (int r = 0; r < jt; ++r) sh.U[r * NT + tid] = t4[r];
        __syncthreads();
        if (tid < 64) {
          const int nr = jt * NT / 64;
          uint32_t prefix = 0u;
          for (int bit = 31; bit >= 16; --bit) {
            const uint32_t probe = prefix | (1u << bit);
            uint32_t c = 0;
            for (int r = 0; r < nr; ++r) c += (uint32_t)__popcll(__ballot(sh.U[r * 64 + tid] >= probe));
            if (c >= k) prefix = probe;
          }
          if (tid == 0) sh.bound = prefix;
        }
        __syncthreads();
        ss.tau = (uint64_t)sh.bound << 16;
      }
      const uint32_t li0 = (uint32_t)(tb - c0);
      auto li_of = [&](int i) { return li0 + (uint32_t)(((i >> 2) * NT + tid) * 4 + (i & 3)); };
      // fast path: the whole tile's survivors fit the buffer (one scan).
      // Survivors are compared on the key alone (a superset of the
      // composite test; the extra entries are dropped at compaction).
      const uint32_t tk = (uint32_t)(ss.tau >> 16);
      uint32_t mine = 0;
      #pragma unroll
      for (int i = 0; i < E; ++i) mine += key[i] >= tk && key[i] != 0u;
      uint32_t total;
      uint32_t off = block_excl_scan_u32<NT>(mine, sh.redu, &total);
      if (sh.count + total <= (uint32_t)kBufCap) {
        const uint32_t base = sh.count;
        #pragma unroll
        for (int i = 0; i < E; ++i) {
          if (key[i] == 0u) continue;
          if (key[i] >= tk) sh.cbuf[base + off++] = local_comp(key[i], li_of(i));
          else reject_key(ss, key[i]);
        }
        __syncthreads();
        if (tid == 0) sh.count = base + total;
        __syncthreads();
      } else {
        // one float4 column (NT * 4 items) at a time, so each batch fits
        #pragma unroll
        for (int j = 0; j < VEC; ++j) {
          const uint32_t kj[4] = {key[4 * j], key[4 * j + 1], key[4 * j + 2], key[4 * j + 3]};
          const uint32_t lij = li0 + (uint32_t)((j * NT + tid) * 4);
          append_batch<4>(sh, ss, k, kj, [&](int q) { return lij + (uint32_t)q; });
        }
      }
    }
    #pragma unroll
    for (int i = 0; i < E; ++i) cur[i] = nxt[i];
  }

  st.max_l = maxkey > kKeyNegInf ? okey_inv(maxkey) : -__builtin_inff();
  st.any_finite = maxkey > kKeyNegInf ? 1u : 0u;
  ChunkStat bs = block_stat<NT>(st, sh.red);
  uint64_t* cand = a.cand + ((int64_t)row * a.n_chunks + chunk) * kFast;
  if (k > 0) {
    // the chunk's exact top-k: select in the buffer, emit in thread order
    compact_buffer(sh, ss, k);
    const uint32_t n = sh.count;
    constexpr int PER = kBufCap / NT;
    uint32_t mine = 0;
    #pragma unroll
    for (int r = 0; r < PER; ++r) mine += (uint32_t)(r * NT + tid) < n;
    uint32_t total;
    uint32_t pos = block_excl_scan_u32<NT>(mine, sh.redu, &total);
    uint64_t minkept = ~0ull;
    #pragma unroll
    for (int r = 0; r < PER; ++r) {
      const uint32_t i = r * NT + tid;
      if (i >= n) continue;
      const uint64_t v = sh.cbuf[i];
      const uint32_t li = 0xffffu - (uint32_t)(v & 0xffffu);
      const uint64_t ck = cand_key((uint32_t)(v >> 16), (uint32_t)c0 + li);
      if (pos < (uint32_t)kFast) cand[pos] = ck;
      ++pos;
      minkept = ck < minkept ? ck : minkept;
    }
    const float mc = finitef_(bs.max_l) ? bs.max_l / cfg.t_eff : -__builtin_inff();
    float part = (ss.rest_on && ss.rest.sum > 0.f && finitef_(mc)) ? ss.rest.sum * __expf(ss.rest.m - mc) : 0.f;
    uint32_t unkept = ss.unkept;
    block_tail3(minkept, unkept, part, sh);
    bs.n_cand = min(total, (uint32_t)kFast);
    bs.trunc = len > (int)k ? 1u : 0u;
    bs.min_kept = minkept;
    bs.unkept_key = unkept;
    bs.lse_m = mc;
    bs.lse_sum = part;
  }
  if (tid == 0) a.stats[(int64_t)row * a.n_chunks + chunk] = bs;
}

// History tokens of the chunk [c0, c1) for the general pass: an LDS bitmap
// of the tokens present and an (id -> summed count) hash with linear
// probing.  All threads call it.
template <int CH>
__device__ __forceinline__ void stage_history_hash(const SampleArgs& a, uint32_t h0, uint32_t h1, int c0,
                                                   int c1, uint32_t* bitmap, uint32_t* hkey, uint32_t* hcnt) {
  const int tid = threadIdx.x;
  for (int i = tid; i < CH / 32; i += NT) bitmap[i] = 0u;
  for (int i = tid; i < kHashCap; i += NT) { hkey[i] = 0xffffffffu; hcnt[i] = 0u; }
  __syncthreads();
  for (uint32_t hb = h0; hb < h1; hb += NT * 8) {
    uint32_t ids[8], cnts[8];
    #pragma unroll
    for (int r = 0; r < 8; ++r) {  // independent loads first
      const uint32_t h = hb + r * NT + tid;
      ids[r] = h < h1 ? a.hids[h] : 0xffffffffu;
      cnts[r] = h < h1 ? a.hcnt[h] : 0u;
    }
    #pragma unroll
    for (int r = 0; r < 8; ++r) {
      const uint32_t id = ids[r];
      if (id < (uint32_t)c0 || id >= (uint32_t)c1) continue;
      const uint32_t li = id - (uint32_t)c0;
      atomicOr(&bitmap[li >> 5], 1u << (li & 31u));
      // a token that finds no free slot is counted from the global list
      // when it is looked up (hash_count reports it as not found)
      uint32_t slot = (id * 2654435761u) & (kHashCap - 1);
      for (int probe = 0; probe < kHashCap; ++probe) {
        const uint32_t prev = atomicCAS(&hkey[slot], 0xffffffffu, id);
        if (prev == 0xffffffffu || prev == id) {
          atomicAdd(&hcnt[slot], cnts[r]);
          break;
        }
        slot = (slot + 1) & (kHashCap - 1);
      }
    }
  }
  __syncthreads();
}

// LDS of the scan kernels.
constexpr int kRowThreads = 512;  // row kernel: 8 waves stream, the first 4 finish
size_t lean_chunk_lds_bytes(int chunk, bool hist) {
  return ((sizeof(LeanLds<NT / 64>) + 15) & ~(size_t)15) + (hist ? hist_lds_bytes(chunk, kChunkHistCap) : 0);
}
size_t generic_chunk_lds_bytes(int chunk, bool hist) {
  return ((sizeof(ScanLds) + 15) & ~(size_t)15) +
         (hist ? (size_t)chunk / 8 + 2 * kHashCap * sizeof(uint32_t) : 0);
}
constexpr size_t kRowUnionBytes =
    ((sizeof(FinLds) > sizeof(LeanLds<kRowThreads / 64>) ? sizeof(FinLds) : sizeof(LeanLds<kRowThreads / 64>)) + 15) &
    ~(size_t)15;
size_t row_lds_bytes(int V, bool hist) {
  return kRowUnionBytes + (hist ? hist_lds_bytes(V, kRowHistCap) : 0);
}
constexpr size_t kMaxLds = 160 * 1024;  // LDS per workgroup on gfx950

template <int NTH, int VEC, int D, int DT, bool MASK>
__device__ __forceinline__ void scan_lean_dispatch(const SampleArgs& a, const RowCfg& cfg, LeanLds<NTH / 64>& L,
                                                   const RowBuf& rb, float (&tl)[D][VEC * 4],
                                                   uint32_t (&tmw)[D][VEC], const HistView& hv, int row,
                                                   int64_t slot, int c0, int c1) {
  if (hv.on && hv.ovf) scan_lean<NTH, VEC, D, DT, MASK, true>(a, cfg, L, rb, tl, tmw, hv, row, slot, c0, c1);
  else scan_lean<NTH, VEC, D, DT, MASK, false>(a, cfg, L, rb, tl, tmw, hv, row, slot, c0, c1);
}

// One workgroup per (chunk, row): the lean pass over a chunk, finished by
// finish_kernel.  Used when a row's history table does not fit the row
// kernel's LDS.
template <int VEC, int TILES, int DT, bool MASK>
__global__ void __launch_bounds__(NT) scan_kernel(SampleArgs a) {
  extern __shared__ __align__(16) unsigned char lds_raw[];
  constexpr int CH = NT * VEC * 4 * TILES;
  static_assert(CH <= 65536, "chunk");
  const int row = blockIdx.y;
  const int chunk = blockIdx.x;
  const int c0 = chunk * CH;
  const int c1 = min(c0 + CH, a.V);
  // every load of the chunk is issued first, so that the parameter and
  // history reads below overlap them
  const RowBuf rb = row_buf<DT, MASK>(a, row, c0, c1);
  float tl[TILES][VEC * 4];
  uint32_t tmw[TILES][VEC];
  #pragma unroll
  for (int t = 0; t < TILES; ++t) buf_load<NT, VEC, DT, MASK>(rb, t * NT * VEC * 4, tl[t], tmw[t]);
  const RowCfg cfg = load_cfg(a.pv, row, a.V, a.n_lp, a.need_lse);
  HistView hv;
  hv.on = false;
  hv.ovf = false;
  if (a.hoff)
    hv = stage_history_rank<NT>(a, row, c0, c1 - c0, kChunkHistCap,
                                reinterpret_cast<uint32_t*>(lds_raw + ((sizeof(LeanLds<NT / 64>) + 15) & ~(size_t)15)));
  scan_lean_dispatch<NT, VEC, TILES, DT, MASK>(a, cfg, *reinterpret_cast<LeanLds<NT / 64>*>(lds_raw), rb, tl, tmw,
                                               hv, row, (int64_t)row * a.n_chunks + chunk, c0, c1);
}

// One workgroup per row: kRowThreads threads stream the whole row with D
// tiles of loads in flight per thread; then the waves past the first four
// end (a barrier waits only for the waves still running) and the first four
// finish the row in place (the row is one chunk for the finish code).
template <int VEC, int D, int DT, bool MASK>
__global__ void __launch_bounds__(kRowThreads) row_kernel(SampleArgs a) {
  extern __shared__ __align__(16) unsigned char lds_raw[];
  constexpr int NTH = kRowThreads;
  constexpr int TILE = NTH * VEC * 4;
  const int row = blockIdx.x;
  const int V = a.V;
  const RowBuf rb = row_buf<DT, MASK>(a, row, 0, V);
  float tl[D][VEC * 4];
  uint32_t tmw[D][VEC];
  #pragma unroll
  for (int t = 0; t < D; ++t) buf_load<NTH, VEC, DT, MASK>(rb, t * TILE, tl[t], tmw[t]);
  const RowCfg cfg = load_cfg(a.pv, row, V, a.n_lp, a.need_lse);
  HistView hv;
  hv.on = false;
  hv.ovf = false;
  if (a.hoff)
    hv = stage_history_rank<NTH>(a, row, 0, V, kRowHistCap, reinterpret_cast<uint32_t*>(lds_raw + kRowUnionBytes));
  scan_lean_dispatch<NTH, VEC, D, DT, MASK>(a, cfg, *reinterpret_cast<LeanLds<NTH / 64>*>(lds_raw), rb, tl, tmw,
                                            hv, row, row, 0, V);
  if (threadIdx.x >= NT) return;
  __syncthreads();  // the row's record and candidates are visible to the workgroup
  finish_row(*reinterpret_cast<FinLds*>(lds_raw), a, row, cfg);
}

// The general pass with a block-level running selection of up to kFast
// candidates per chunk: used when more than kLeanK logprobs are requested.
template <int VEC, int TILES>
__global__ void __launch_bounds__(NT) scan_generic_kernel(SampleArgs a) {
  extern __shared__ __align__(16) unsigned char lds_raw[];
  constexpr int CH = NT * VEC * 4 * TILES;
  static_assert(CH <= 65536, "local indices are 16-bit");
  uint32_t* bitmap = reinterpret_cast<uint32_t*>(lds_raw + ((sizeof(ScanLds) + 15) & ~(size_t)15));
  uint32_t* hkey = bitmap + CH / 32;
  uint32_t* hcnt = hkey + kHashCap;
  const int row = blockIdx.y;
  const int chunk = blockIdx.x;
  const int c0 = chunk * CH;
  const int c1 = min(c0 + CH, a.V);
  float tile0[VEC * 4];
  load_tile<VEC>(a, (int64_t)row * a.row_stride, c0, c1, tile0);
  const RowCfg cfg = load_cfg(a.pv, row, a.V, a.n_lp, a.need_lse);
  bool pen = false;
  uint32_t h0 = 0, h1 = 0;
  if (a.hoff) { h0 = a.hoff[row]; h1 = a.hoff[row + 1]; pen = h1 > h0; }
  if (pen) stage_history_hash<CH>(a, h0, h1, c0, c1, bitmap, hkey, hcnt);
  scan_generic<VEC, TILES>(a, cfg, *reinterpret_cast<ScanLds*>(lds_raw), tile0, bitmap, hkey, hcnt,
                           pen, h0, h1, row, chunk, c0, c1);
}

// One workgroup per row: merge the row's chunk results and draw.  A separate
// launch: the kernel boundary makes every chunk's results visible to the
// finishing workgroup on any XCD without a device-scope fence per chunk.
__global__ void __launch_bounds__(NT) finish_kernel(SampleArgs a) {
  __shared__ FinLds fs;
  const int row = blockIdx.x;
  const RowCfg cfg = load_cfg(a.pv, row, a.V, a.n_lp, a.need_lse);
  finish_row(fs, a, row, cfg);
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

// Processed logits and per-chunk max of s (kept in stats[.].max_l) for the
// debug export.
__global__ void __launch_bounds__(NT) debug_processed_kernel(SampleArgs a, float* out_proc) {
  __shared__ uint32_t cnt[kChunk];
  __shared__ ChunkStat red[NT / 64];
  const int row = blockIdx.y, chunk = blockIdx.x, tid = threadIdx.x;
  const int V = a.V, c0 = chunk * kChunk, c1 = min(c0 + kChunk, V);
  const RowCfg cfg = load_cfg(a.pv, row, V, 0, 0);
  bool pen = false;
  uint32_t h0 = 0, h1 = 0;
  if (a.hoff) { h0 = a.hoff[row]; h1 = a.hoff[row + 1]; pen = h1 > h0; }
  if (pen) {
    for (int i = tid; i < kChunk; i += NT) cnt[i] = 0u;
    __syncthreads();
    for (uint32_t h = h0 + tid; h < h1; h += NT) {
      const uint32_t id = a.hids[h];
      if (id >= (uint32_t)c0 && id < (uint32_t)c1) atomicAdd(&cnt[id - c0], a.hcnt[h]);
    }
    __syncthreads();
  }
  ChunkStat st;
  stat_init(st);
  const int64_t rbase = (int64_t)row * a.row_stride;
  for (int e = c0 + tid; e < c1; e += NT) {
    float l = load_raw(a.logits, a.dtype, rbase + e);
    if (!allowed(a, row, (uint32_t)e)) l = -__builtin_inff();
    if (pen) l = apply_penalties(l, cnt[e - c0], cfg);
    out_proc[(int64_t)row * V + e] = l;
    const float s = finitef_(l) ? l / cfg.t_eff : -__builtin_inff();
    st.max_l = fmaxf(st.max_l, s);
  }
  const ChunkStat bs = block_stat<NT>(st, red);
  if (tid == 0) a.stats[(int64_t)row * a.n_chunks + chunk] = bs;
}

__global__ void __launch_bounds__(1024) debug_probs_kernel(SampleArgs a, const float* proc, float* out_probs) {
  __shared__ double dred[16];
  __shared__ float fred[16];
  const int row = blockIdx.x, tid = threadIdx.x, V = a.V;
  const RowCfg cfg = load_cfg(a.pv, row, V, 0, 0);
  float M = -__builtin_inff();
  for (int c = tid; c < a.n_chunks; c += 1024) M = fmaxf(M, a.stats[(int64_t)row * a.n_chunks + c].max_l);
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

bool row_mode(int V, int n_lp, int vec_ok, bool hist) {
  return n_lp <= kLeanK && vec_ok && row_lds_bytes(V, hist) <= kMaxLds;
}

int choose_chunk(int B, int V, int n_lp, int vec_ok, bool hist) {
  // one workgroup per row when the row fits the row kernel's LDS;
  // otherwise chunks: fewer, larger ones when the batch alone fills the GPU
  if (row_mode(V, n_lp, vec_ok, hist)) return V;
  const long wg_large = (long)B * ((V + kChunk - 1) / kChunk);
  return wg_large >= 512 ? kChunk : kChunkSmall;
}

// Dynamic LDS above 64 KiB needs the kernel's attribute raised once.
template <typename K>
hipError_t allow_lds(K kernel, size_t bytes) {
  if (bytes <= 65536) return hipSuccess;
  return hipFuncSetAttribute((const void*)kernel, hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes);
}

hipError_t launch_chunked(const SampleArgs& a, hipStream_t stream) {
  const bool hist = a.hoff != nullptr;
  const bool large = a.chunk == kChunk;
  dim3 grid(a.n_chunks, a.B);
  if (a.n_lp > kLeanK || !a.vec_ok) {
    if (large)
      hipLaunchKernelGGL((scan_generic_kernel<kVecLarge, kTilesLarge>), grid, dim3(NT),
                         generic_chunk_lds_bytes(kChunk, hist), stream, a);
    else
      hipLaunchKernelGGL((scan_generic_kernel<kVecSmall, 1>), grid, dim3(NT),
                         generic_chunk_lds_bytes(kChunkSmall, hist), stream, a);
  } else {
    constexpr int TL = kChunk / (NT * kLeanVec * 4);
    constexpr int TS = kChunkSmall / (NT * kLeanVec * 4);
    static_assert(TL * NT * kLeanVec * 4 == kChunk && TS * NT * kLeanVec * 4 == kChunkSmall, "chunk sizes");
    const size_t lds = lean_chunk_lds_bytes(large ? kChunk : kChunkSmall, hist);
#define HI_ROCM_LAUNCH_LEAN(DT, M)                                                                   \
  do {                                                                                              \
    if (large) hipLaunchKernelGGL((scan_kernel<kLeanVec, TL, DT, M>), grid, dim3(NT), lds, stream, a); \
    else hipLaunchKernelGGL((scan_kernel<kLeanVec, TS, DT, M>), grid, dim3(NT), lds, stream, a);       \
  } while (0)
    if (a.dtype == HI_ROCM_DTYPE_BF16) {
      if (a.mask) HI_ROCM_LAUNCH_LEAN(HI_ROCM_DTYPE_BF16, true);
      else HI_ROCM_LAUNCH_LEAN(HI_ROCM_DTYPE_BF16, false);
    } else {
      if (a.mask) HI_ROCM_LAUNCH_LEAN(HI_ROCM_DTYPE_F32, true);
      else HI_ROCM_LAUNCH_LEAN(HI_ROCM_DTYPE_F32, false);
    }
#undef HI_ROCM_LAUNCH_LEAN
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(finish_kernel, dim3(a.B), dim3(NT), 0, stream, a);
  return hipGetLastError();
}

constexpr int kRowDepth = 4;  // tiles of loads in flight per thread

template <int DT, bool MASK>
hipError_t launch_row_t(const SampleArgs& a, hipStream_t stream) {
  const size_t lds = row_lds_bytes(a.V, a.hoff != nullptr);
  auto kern = row_kernel<kLeanVec, kRowDepth, DT, MASK>;
  hipError_t e = allow_lds(kern, lds);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(kern, dim3(a.B), dim3(kRowThreads), lds, stream, a);
  return hipGetLastError();
}

hipError_t launch_sample(const SampleArgs& a, hipStream_t stream) {
  if (a.n_chunks == 1 && a.chunk == a.V && row_mode(a.V, a.n_lp, a.vec_ok, a.hoff != nullptr)) {
    if (a.dtype == HI_ROCM_DTYPE_BF16)
      return a.mask ? launch_row_t<HI_ROCM_DTYPE_BF16, true>(a, stream) : launch_row_t<HI_ROCM_DTYPE_BF16, false>(a, stream);
    return a.mask ? launch_row_t<HI_ROCM_DTYPE_F32, true>(a, stream) : launch_row_t<HI_ROCM_DTYPE_F32, false>(a, stream);
  }
  return launch_chunked(a, stream);
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
  dim3 g1((a.V + kChunk - 1) / kChunk, a.B);
  SampleArgs b = a;
  b.n_chunks = (int)g1.x;
  hipLaunchKernelGGL(debug_processed_kernel, g1, dim3(NT), 0, stream, b, out_proc);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(debug_probs_kernel, dim3(a.B), dim3(1024), 0, stream, b, (const float*)out_proc, out_probs);
  return hipGetLastError();
}

}  // namespace hi_rocm
