// The wide pass of top-p rows: device code of the chunked path's finish
// kernel (sampler_chunked.hip), also reached from the select pass.
#pragma once
#include "sampler_select.h"

namespace hi_rocm {

// ==========================================================================
// Wide pass: top-p rows without a top-k bound (gpu.rs:820-899 with
// top_k unset), chunk-parallel
// ==========================================================================
//
// The reference walks such a row's whole rank order with three sequential
// f32 folds: the normaliser over every weight in vocabulary order
// (gpu.rs:837), then cum_p += w / total in rank order up to the cutoff
// (:843-856), then the candidate total and the inverse CDF (:874-899).  Here
// the select pass leaves the scaled logits s in ws_s and a mass histogram
// per chunk (WideStat); then one workgroup per (chunk, row):
//   1. merges the row's chunk maxima (M) and histograms (wide_row_stats,
//      every workgroup of the row alike): a conservative
//      weight bound w_lo such that the weights >= w_lo hold at least
//      cutoff + kWideMargin of the mass (every weight of the nucleus is
//      >= w_lo unless the f32 folds differ from exact sums by more than the
//      margin, which the finish detects), and the predicted sum before the
//      chunk;
//   2. computes its weights w = expf(s - M) exactly (min-p zeros them),
//      plans its part of the vocabulary-order fold (fold_plan: segments of
//      one predicted binade and boundary terms) and writes the plan;
//   3. counts its weights >= w_lo by distinct value in an LDS hash: the
//      rank order only needs each distinct weight's multiplicity (equal
//      weights rank by index, and the folds do not see indices);
//   4. bumps the row's counter; the last workgroup finishes the row:
//      chains the chunk plans into the exact normaliser (refolding a chunk
//      whose prediction missed), merges the chunks' runs, sorts them
//      (weight descending), folds cum_p, the candidate total and the CDF
//      over the runs with the closed forms for equal terms, and finds the
//      drawn index among the equal weights of the drawn run.
// Rows whose chunks took the select pass's exact path, whose tables
// overflow, or whose nucleus is not inside the superset take finish_row.

constexpr float kWideMargin = 0.005f;  // extra probability mass of the superset
constexpr int kWideChunkHash = 2048;   // distinct superset weights per chunk
constexpr int kWideFinHash = 2048;     // distinct superset weights per row
constexpr int kWideRunCap = kWideFinHash;
constexpr int kWideBatch = 64;         // chunk plans the chain holds in LDS at a time
constexpr int kWideGBins = 64;         // threshold bins (binades of w below M)

// Per-wave slots of the chunk work's workgroup scans and reductions.
struct WideScanLds {
  fold::Map wmap[NT / 64];
  uint32_t wcnt[NT / 64];
  fold::Map wmap3[3][NT / 64];  // block_map_scan3
};
// LDS of a (chunk, row) workgroup; the chunk's weights follow at
// wide_w_off.
struct WideChunkLds {
  WideScanLds fl;
  uint64_t exptab[32];                   // exact_expf's table (wide_row_stats copies it)
  unsigned long long gmass[kWideGBins];  // wide_row_stats
  unsigned long long predfx, ownfx;
  float w_lo;
  uint32_t hkey[kWideChunkHash];
  uint32_t hcnt[kWideChunkHash];
  uint32_t hmin[kWideChunkHash];
  fold::Map exm[NT];  // the full path's block maps before each block, in the predicted binade
  uint32_t nrun, ovf, last, fu;
  float fend;
  int x_ws, x_we;  // window 0 of the full path
};
constexpr size_t kWideChunkHead = (sizeof(WideChunkLds) + 15) & ~(size_t)15;
// Weights sit in LDS with one pad word per 16, so that threads reading
// their own 16 consecutive terms hit distinct banks.
__host__ __device__ inline int wide_pad(int i) { return i + (i >> 4); }
__host__ __device__ inline size_t wide_w_bytes(int chunk) { return (size_t)wide_pad(chunk) * 4 + 16; }
__host__ __device__ inline size_t wide_w_off(int) { return kWideChunkHead; }
__host__ __device__ inline size_t wide_chunk_lds(int chunk) { return kWideChunkHead + wide_w_bytes(chunk); }

// LDS of the row finish.  Its phases reuse one union: the chain (chunk
// plans, and the refold arrays past them), the merge (hash table and sort
// keys), the draw (runs in rank order and the fold values before them).
struct WideFinLds {
  fold::WgLds<NT> fl;
  union {
    struct {
      ChunkFold batch[kWideBatch];
    } ch;
    struct {
      uint32_t hkey[kWideFinHash];
      uint32_t hcnt[kWideFinHash];
      uint32_t hmin[kWideFinHash];
      uint64_t sortk[kWideRunCap];
    } mg;
    struct {
      float rx[kWideRunCap];   // weight of run r (rank order)
      uint32_t rm[kWideRunCap];  // its multiplicity
      uint32_t ri[kWideRunCap];  // its smallest index
      float st[kWideRunCap];   // cum_p before run r
      float st2[kWideRunCap];  // candidate weight sum before run r
    } fo;
    uint32_t cntc[kWideRunCap];  // the drawn weight's multiplicity per chunk
  } u;
  uint8_t pe[kWideRunCap + 4];
  uint32_t noff[NT + 1];
  uint32_t cnt, fail_c, rsel, csel, tok, fu;
  float acc, acc2;
};
// The refold's weights start past the whole struct: the refold runs in the
// middle of the chain, which still needs the batch of chunk plans and the
// fields after the union.
__host__ __device__ inline size_t wide_fin_w_off() { return (sizeof(WideFinLds) + 15) & ~(size_t)15; }
__host__ __device__ inline size_t wide_fin_lds(int chunk) {
  const size_t r = wide_fin_w_off() + wide_w_bytes(chunk);
  return r > sizeof(WideFinLds) ? r : sizeof(WideFinLds);
}

__device__ __forceinline__ uint32_t wide_hash(uint32_t key, int log2n) {
  return (key * 0x9E3779B1u) >> (32 - log2n);
}

// Inserts `count` copies of weight bits `key` with smallest index `idx`
// into an LDS table of 2^log2n slots (key 0 = empty; weights here are > 0).
// Returns false when the table is full.
__device__ __forceinline__ bool wide_insert(uint32_t* hkey, uint32_t* hcnt, uint32_t* hmin, int log2n,
                                            uint32_t key, uint32_t count, uint32_t idx) {
  const uint32_t mask = (1u << log2n) - 1u;
  uint32_t h = wide_hash(key, log2n);
  for (uint32_t probe = 0; probe <= mask; ++probe, h = (h + 1u) & mask) {
    const uint32_t old = atomicCAS(&hkey[h], 0u, key);
    if (old == 0u || old == key) {
      atomicAdd(&hcnt[h], count);
      atomicMin(&hmin[h], idx);
      return true;
    }
  }
  return false;
}

// The first kWidePre * NT scaled logits of a chunk (the whole of a
// 4096-logit chunk), loaded by wide_row_stats behind its own loads, so that
// their latency hides behind the statistics.
constexpr int kWidePre = 16;
__device__ __forceinline__ void wide_preload(const float* s, int len, float (&pre)[kWidePre]) {
  #pragma unroll
  for (int k = 0; k < kWidePre; ++k) {
    const int i = k * NT + (int)threadIdx.x;
    pre[k] = i < len ? s[i] : -__builtin_inff();
  }
}

// Step 1, by every workgroup of a top-p row's chunk work: the row max of s
// (M), the superset bound w_lo and the predicted fold value before this
// workgroup's chunk, from the chunks' statistics the select pass wrote
// (WideStat).  The masses use approximate exp; they only size the superset
// and predict binades.  valid = 0: a chunk's statistics were not written by
// this call's pass, or no logit is finite (the row takes finish_row).  The
// row's finishing workgroup clears the chunks' valid flags afterwards.
struct WideRowStats {
  float M, w_lo;
  uint32_t valid;
  double pred;  // the predicted fold value before the chunk
  double mass;  // the chunk's predicted mass
};
__device__ __forceinline__ WideRowStats wide_row_stats(WideChunkLds& L, const SampleArgs& a, int row, int chunk,
                                                      const RowCfg& cfg, float (&pre)[kWidePre]) {
  const int tid = threadIdx.x;
  const int nch = a.n_chunks;
  const ChunkStat* stats = a.stats + (int64_t)row * nch;
  const WideStat* wst = a.wstat + (int64_t)row * nch;
  // the loads of the first kU * NT (chunk, bin) items go out with those of
  // the chunk maxima
  constexpr int kU = 8;
  float hv0[kU], ms0[kU];
  {
    const int items0 = nch * kWideBins;
    #pragma unroll
    for (int k = 0; k < kU; ++k) {
      const int it = k * NT + tid;
      hv0[k] = 0.f;
      ms0[k] = 0.f;
      if (it < items0) {
        const WideStat& ws = wst[it / kWideBins];
        hv0[k] = ws.hist[it % kWideBins];
        ms0[k] = ws.ms;
      }
    }
  }
  // the chunk maxima and valid flags (chunks tid, tid + NT, ...): the first
  // round goes out with the loads above; then the chunk's scaled logits,
  // behind all of them, so that waiting for the statistics' loads does not
  // wait for these
  float ml0 = 0.f;
  uint32_t v0 = 1u;
  if (tid < nch) {
    ml0 = stats[tid].max_l;
    v0 = wst[tid].valid;
  }
  {
    const int c0 = chunk * a.chunk;
    wide_preload(a.ws_s + (int64_t)row * a.V + c0, min(a.chunk, a.V - c0), pre);
  }
  uint32_t mk = tid < nch ? okey(ml0) : 0u, bad = tid < nch ? v0 ^ 1u : 0u;
  for (int c = tid + NT; c < nch; c += NT) {
    mk = max(mk, okey(stats[c].max_l));
    bad |= wst[c].valid ^ 1u;
  }
  if (tid < kWideGBins) L.gmass[tid] = 0ull;
  if (tid == 0) { L.predfx = 0ull; L.ownfx = 0ull; }
  if (tid < 32) L.exptab[tid] = exp2_tab32((uint32_t)tid);
  mk = block_max_u32<NT>(mk, L.fl.wcnt);
  bad = block_max_u32<NT>(bad, L.fl.wcnt);
  const float ml = okey_inv(mk);
  const float M = finitef_(ml) ? ml / cfg.t_eff : -__builtin_inff();
  if (!finitef_(M) || bad) return WideRowStats{M, 0.f, 0u, 0.0, 0.0};
  // chunk masses relative to M, in fixed point (2^-32): per binade of their
  // lower end (for w_lo) and, for the chunks before this one and for this
  // one, their sums (the prediction): each thread adds its bins' shares,
  // then one wave reduction and an atomic per wave (integer sums, exact in
  // any order)
  static_assert(kWideBins == 32, "a chunk's bins are one half of a wave");
  static_assert(kWideGBins == 64, "one bin per lane");
  const int items = nch * kWideBins;
  unsigned long long bef = 0ull, own = 0ull;
  for (int base = 0; base < items; base += kU * NT) {
    float hv[kU], msv[kU];
    #pragma unroll
    for (int k = 0; k < kU; ++k) {
      const int it = base + k * NT + tid;
      hv[k] = hv0[k];
      msv[k] = ms0[k];
      if (base != 0) {
        hv[k] = 0.f;
        if (it < items) {
          const WideStat& ws = wst[it / kWideBins];
          hv[k] = ws.hist[it % kWideBins];
          msv[k] = ws.ms;
        }
      }
    }
    #pragma unroll
    for (int k = 0; k < kU; ++k) {
      const int it = base + k * NT + tid;
      const int j = it % kWideBins;
      const float lb = (M - msv[k]) * 1.4426950408889634f;  // log2 of M's weight over the chunk max's
      const float m = hv[k] * __builtin_amdgcn_exp2f(-lb);
      const bool pos = it < items && m > 0.f;
      const unsigned long long fx = pos ? (unsigned long long)((double)m * 4294967296.0) : 0ull;
      if (pos) {
        int g = j == kWideBins - 1 ? kWideGBins - 1 : (int)floorf((float)(j + 1) + lb);
        g = g < kWideGBins ? g : kWideGBins - 1;
        atomicAdd(&L.gmass[g], fx);
      }
      const int c = it / kWideBins;
      bef += c < chunk ? fx : 0ull;
      own += c == chunk ? fx : 0ull;
    }
  }
  bef = wave_reduce64(bef, 0ull, [](uint64_t x, uint64_t y) { return x + y; });
  own = wave_reduce64(own, 0ull, [](uint64_t x, uint64_t y) { return x + y; });
  if ((tid & 63) == 0) {
    if (bef != 0ull) atomicAdd(&L.predfx, bef);
    if (own != 0ull) atomicAdd(&L.ownfx, own);
  }
  __syncthreads();
  // w_lo: the first binade bin where the masses from the top reach the
  // cutoff plus the margin (one wave over the 64 bins)
  if (tid < 64) {
    const int lane = tid;
    // inclusive prefix sum over the lanes (DPP row shifts and broadcasts;
    // lanes with no source add zero)
    unsigned long long inc = L.gmass[lane];
    auto up = [&](auto ctl) {
      constexpr int C = decltype(ctl)::c, RM = decltype(ctl)::rm;
      constexpr bool BC = decltype(ctl)::bc;
      inc += ((unsigned long long)dpp32<C, RM, BC>(0u, (uint32_t)(inc >> 32)) << 32) | dpp32<C, RM, BC>(0u, (uint32_t)inc);
    };
    up(fold::DppStep<kDppShr1, 0xf, true>{});
    up(fold::DppStep<kDppShr1 + 1, 0xf, true>{});
    up(fold::DppStep<kDppShr1 + 3, 0xf, true>{});
    up(fold::DppStep<kDppShr1 + 7, 0xf, true>{});
    up(fold::DppStep<kDppBcast15, 0xa, false>{});
    up(fold::DppStep<kDppBcast31, 0xc, false>{});
    const unsigned long long tot = ((unsigned long long)(uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(inc >> 32), 63) << 32) |
                                   (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)inc, 63);
    const double frac = (double)cfg.cutoff + (double)kWideMargin;
    float w_lo = 0.f;
    if (cfg.cutoff < 1.f && frac < 1.0) {
      const unsigned long long target = (unsigned long long)(frac * (double)tot);
      const uint64_t hit = __ballot(lane < kWideGBins - 1 && inc >= target);
      if (hit != 0ull) w_lo = __builtin_ldexpf(1.f, -(__ffsll((unsigned long long)hit)));
    }
    if (lane == 0) L.w_lo = fmaxf(w_lo, cfg.min_p);
  }
  __syncthreads();
  const WideRowStats r = WideRowStats{M, L.w_lo, 1u, (double)L.predfx * (1.0 / 4294967296.0),
                                      (double)L.ownfx * (1.0 / 4294967296.0)};
  __syncthreads();  // L is reused by the chunk work
  return r;
}

// w[wide_pad(i)] = wg[i] = the weight of scaled logit s[i] (exact expf, its
// table read from LDS; min-p zeros it), i < len; the first kWidePre * NT
// come in `pre`, the rest are loaded here (all of a thread's loads of a
// block issued before any is used).
__device__ __forceinline__ void wide_weights(const float* s, int len, float M, float min_p, float* w,
                                             const uint64_t* tab, float* wg, const float (&pre)[kWidePre]) {
  const Exp2TabLds et{tab};
  #pragma unroll
  for (int k = 0; k < kWidePre; ++k) {
    const int i = k * NT + (int)threadIdx.x;
    float x = exact_expf_t(pre[k] - M, et);
    x = x < min_p ? 0.f : x;  // min-p: excluded like a zero weight
    if (i < len) {
      w[wide_pad(i)] = x;
      wg[i] = x;
    }
  }
  constexpr int kB = 8;
  for (int base = kWidePre * NT; base < len; base += kB * NT) {
    float v[kB];
    #pragma unroll
    for (int k = 0; k < kB; ++k) {
      const int i = base + k * NT + (int)threadIdx.x;
      v[k] = i < len ? s[i] : -__builtin_inff();
    }
    #pragma unroll
    for (int k = 0; k < kB; ++k) {
      const int i = base + k * NT + (int)threadIdx.x;
      float x = exact_expf_t(v[k] - M, et);
      x = x < min_p ? 0.f : x;  // min-p: excluded like a zero weight
      if (i < len) {
        w[wide_pad(i)] = x;
        wg[i] = x;
      }
    }
  }
}

// Map of one term in binade e (exact_fold.h): n ulps, plus one above half
// an ulp, plus one on an exact half when that makes the sum even.
__device__ __forceinline__ fold::Map term_map(float x, int e) {
  const fold::Inc c = fold::classify(x, e);
  const uint32_t base = c.n + (c.cls == 2u ? 1u : 0u);
  const uint32_t odd = c.n & 1u;
  fold::Map m;
  m.t0 = base + ((c.cls == 1u && odd) ? 1u : 0u);
  m.t1 = base + ((c.cls == 1u && !odd) ? 1u : 0u);
  return m;
}

// f(x) for the terms x = w[wide_pad(r)], r in [r0, r1), in order.  The LDS
// loads of 16 terms are issued together (a loop of single loads waits out
// the LDS latency on every term).  Past r1 the terms read as -0.0, which a
// fold and a map treat as no term at all: x + -0.0 == x for every x, and
// term_map(-0.0, e) is the identity.
template <typename F>
__device__ __forceinline__ void wide_terms(const float* w, int r0, int r1, F f) {
  for (int g = r0; g < r1; g += 16) {
    float t[16];
    #pragma unroll
    for (int k = 0; k < 16; ++k) t[k] = g + k < r1 ? w[wide_pad(g + k)] : -0.0f;
    #pragma unroll
    for (int k = 0; k < 16; ++k) f(t[k]);
  }
}

// Exclusive scan of maps over the workgroup in thread order; *tot gets the
// composition of all.  Two barriers.
__device__ __forceinline__ fold::Map block_map_scan(fold::Map m, fold::Map* wm, fold::Map* tot) {
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  const fold::Map inc = fold::wave_map_scan(m);
  const fold::Map ex = fold::wave_map_prev(inc);
  __syncthreads();
  if (lane == 63) wm[wid] = inc;
  __syncthreads();
  fold::Map before = fold::map_identity(), all = fold::map_identity();
  #pragma unroll
  for (int w = 0; w < NT / 64; ++w) {
    if (w < wid) before = fold::compose(before, wm[w]);
    all = fold::compose(all, wm[w]);
  }
  *tot = all;
  return fold::compose(before, ex);
}

// block_map_scan of three maps at once (one pair of barriers); returns the
// exclusive scans of m0 and m1, and the totals of all three.
__device__ __forceinline__ void block_map_scan3(fold::Map m0, fold::Map m1, fold::Map m2, fold::Map (*wm)[NT / 64],
                                                fold::Map& ex0, fold::Map& ex1, fold::Map* tot) {
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  const fold::Map i0 = fold::wave_map_scan(m0), i1 = fold::wave_map_scan(m1), i2 = fold::wave_map_scan(m2);
  const fold::Map e0 = fold::wave_map_prev(i0), e1 = fold::wave_map_prev(i1);
  __syncthreads();
  if (lane == 63) {
    wm[0][wid] = i0;
    wm[1][wid] = i1;
    wm[2][wid] = i2;
  }
  __syncthreads();
  fold::Map b0 = fold::map_identity(), b1 = b0, a0 = b0, a1 = b0, a2 = b0;
  #pragma unroll
  for (int w = 0; w < NT / 64; ++w) {
    if (w < wid) {
      b0 = fold::compose(b0, wm[0][w]);
      b1 = fold::compose(b1, wm[1][w]);
    }
    a0 = fold::compose(a0, wm[0][w]);
    a1 = fold::compose(a1, wm[1][w]);
    a2 = fold::compose(a2, wm[2][w]);
  }
  tot[0] = a0;
  tot[1] = a1;
  tot[2] = a2;
  ex0 = fold::compose(b0, e0);
  ex1 = fold::compose(b1, e1);
}

// The exact sequential f32 fold of w[wide_pad(0 .. len)) (LDS) from a0, by
// the workgroup.  Thread t holds a block of consecutive terms; in the
// current binade every block is one map, so a scan gives each block's
// exact start until the first block whose terms leave the binade.  That
// thread adds its terms (and, while crossings come close together, the
// next blocks' terms) as real f32 additions, and the scan resumes after
// them in the new binade.  Returns the sum (uniform).
__device__ __forceinline__ float exact_chunk_fold(const float* w, int len, float a0, fold::Map* wm, float* shf,
                                                  uint32_t* red) {
  constexpr int kSeqBlocks = 4;  // blocks one thread adds after a crossing
  const int tid = threadIdx.x;
  const int J = (len + NT - 1) / NT;
  const int r0 = min(tid * J, len), r1 = min(r0 + J, len);
  float a = a0;
  int pos = 0;
  while (pos < NT) {
    const int e = fold::binade(a);
    const uint32_t A = fold::to_A(a);
    fold::Map m = fold::map_identity();
    if (tid >= pos) wide_terms(w, r0, r1, [&](float x) { m = fold::compose(m, term_map(x, e)); });
    fold::Map tot;
    const fold::Map ex = block_map_scan(m, wm, &tot);
    const uint32_t p = A & 1u;
    if ((uint64_t)A + fold::apply(tot, p) < fold::kTop) {
      a = fold::from_A(A + fold::apply(tot, p), e);
      break;
    }
    const uint64_t At = (uint64_t)A + fold::apply(ex, p);
    const bool cross = tid >= pos && (At >= fold::kTop || At + fold::apply(m, (uint32_t)At & 1u) >= fold::kTop);
    uint32_t first = ~block_max_u32<NT>(cross ? ~(uint32_t)tid : 0u, red);
    if (first == 0xffffffffu) first = (uint32_t)pos;  // (not reached: the total leaves the binade)
    if (tid == (int)first) {
      // At < kTop: the blocks before this one stayed in the binade
      float x = fold::from_A((uint32_t)At, e);
      const int stop = min(len, (tid + kSeqBlocks) * J);
      wide_terms(w, r0, stop, [&](float t) { x = fold::fadd(x, t); });
      shf[0] = x;
    }
    __syncthreads();
    a = shf[0];
    pos = (int)first + kSeqBlocks;
    __syncthreads();
  }
  return a;
}

// Whether a chunk predicted to start at S and add `mass` stays well inside
// the binade of S (0.1% margins, far above the predictions' errors).
__device__ __forceinline__ bool wide_one_binade(double S, double mass) {
  const int ep = fold::binade((float)S);
  return ep > 1 && fold::binade((float)(S * 0.999)) == ep && fold::binade((float)((S + mass) * 1.001)) == ep;
}

// Steps 2-3 for one (chunk, row), with the row's M, w_lo, the chunk's
// predicted start S and its predicted mass.
__device__ __forceinline__ void wide_chunk_work(WideChunkLds& L, unsigned char* lds_raw, const SampleArgs& a, int row, int chunk,
                                const RowCfg& cfg, float M, float w_lo, double S, double mass,
                                const float (&pre)[kWidePre]) {
  const int tid = threadIdx.x;
  const int c0 = chunk * a.chunk;
  const int len = min(a.chunk, a.V - c0);
  float* w = reinterpret_cast<float*>(lds_raw + wide_w_off(a.chunk));
  const float* srow = a.ws_s + (int64_t)row * a.V + c0;
  // the weights, in LDS and (for the finish's exact refolds) in ws_w
  wide_weights(srow, len, M, cfg.min_p, w, L.exptab, a.ws_w + (int64_t)row * a.V + c0, pre);
  for (int h = tid; h < kWideChunkHash; h += NT) { L.hkey[h] = 0u; L.hcnt[h] = 0u; L.hmin[h] = 0xffffffffu; }
  if (tid == 0) { L.nrun = 0u; L.ovf = 0u; }
  __syncthreads();
  // the chunk's part of the vocabulary-order fold: chunk 0 starts from the
  // known -0.0 and folds exactly; the others give their maps in the
  // binades around the predicted start
  ChunkFold* cf = a.wfold + (int64_t)row * a.n_chunks + chunk;
  if (chunk == 0) {
    const float end = exact_chunk_fold(w, len, -0.0f, L.fl.wmap, &L.fend, L.fl.wcnt);
    if (tid == 0) { cf->has_end = 1u; cf->end = end; cf->e0 = 1u; cf->nw = 0u; cf->flags = 0u; }
  } else if (wide_one_binade(S, mass)) {
    // predicted start and end well inside one binade ep (0.1% margins): the
    // chunk's map in ep alone; a chain that finds the start elsewhere, or
    // the sum leaving ep, refolds the chunk
    const int ep = fold::binade((float)S);
    const int J = (len + NT - 1) / NT;
    const int r0 = min(tid * J, len), r1 = min(r0 + J, len);
    fold::Map m1 = fold::map_identity();
    wide_terms(w, r0, r1, [&](float x) { m1 = fold::compose(m1, term_map(x, ep)); });
    fold::Map t1;
    block_map_scan(m1, L.fl.wmap, &t1);
    if (tid == 0) {
      cf->has_end = 0u;
      cf->e0 = (uint32_t)(ep - 1);
      cf->map[1] = t1;
      cf->flags = 2u;
      cf->nw = 0u;
    }
  } else {
    const int ep = fold::binade((float)S);
    const int e0 = ep > 1 ? ep - 1 : 1;
    const int J = (len + NT - 1) / NT;
    const int r0 = min(tid * J, len), r1 = min(r0 + J, len);
    fold::Map m0 = fold::map_identity(), m1 = m0, m2 = m0;
    wide_terms(w, r0, r1, [&](float x) {
      m0 = fold::compose(m0, term_map(x, e0));
      m1 = fold::compose(m1, term_map(x, e0 + 1));
      m2 = fold::compose(m2, term_map(x, e0 + 2));
    });
    // each thread's block maps, for the finish's crossing search
    fold::Map* bm = a.wbmap + ((int64_t)row * a.n_chunks + chunk) * 3 * NT;
    bm[tid] = m0;
    bm[NT + tid] = m1;
    bm[2 * NT + tid] = m2;
    if (tid == 0) L.x_ws = -1;
    fold::Map tt[3], ex0, ex1;
    block_map_scan3(m0, m1, m2, L.fl.wmap3, ex0, ex1, tt);
    if (tid == 0) {
      cf->has_end = 0u;
      cf->e0 = (uint32_t)e0;
      cf->map[0] = tt[0];
      cf->map[1] = tt[1];
      cf->map[2] = tt[2];
      cf->flags = 15u;
    }
    // the predicted crossings: from the predicted start, the block, then
    // the term, where the fold leaves its binade; the chunk records a window
    // of terms around each (up to kCrossWins) and the maps of the segments
    // between them, so that the chain crosses with a few real additions
    // (wide_chain_cross).
    const int kx = ep - e0;  // 0 or 1: ep's maps
    {
      const fold::Map ex = kx == 0 ? ex0 : ex1;
      L.exm[tid] = ex;
    }
    __syncthreads();
    int p0 = 0, ec = ep, nw = 0;
    uint32_t Ac = fold::to_A((float)S);
    // window 0, all of it by the wave holding the one block that leaves ep
    // (the predicted values rise, so only one block can): the term that
    // leaves (the block's terms one a lane, a scan of their maps), the
    // window around it, the map of the segment before the window (the scan
    // up to the window's block, then that block's terms before the window,
    // again one a lane) and the predicted value after the window (a DPP
    // chain of real additions)
    {
      const fold::Map mb = kx == 0 ? m0 : m1;
      const fold::Map ex = L.exm[tid];
      const uint64_t Ab = (uint64_t)Ac + fold::apply(ex, Ac & 1u);
      const uint64_t bal = __ballot(r0 < r1 && Ab < fold::kTop && Ab + fold::apply(mb, (uint32_t)Ab & 1u) >= fold::kTop);
      if (bal != 0ull) {
        static_assert(kSelChunkLarge / NT <= 64, "a block's terms fit one wave");
        const int lane = tid & 63;
        const int l = __ffsll((unsigned long long)bal) - 1;
        const int rc0 = ((tid & ~63) + l) * J;
        const int nc = min(rc0 + J, len) - rc0;
        const uint32_t Ablk = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)Ab, l);
        const fold::Map mt = lane < nc ? term_map(w[wide_pad(rc0 + lane)], ec) : fold::map_identity();
        const fold::Map it = fold::wave_map_scan(mt);
        const uint64_t cr = __ballot(lane < nc && (uint64_t)Ablk + fold::apply(it, Ablk & 1u) >= fold::kTop);
        const int tstar = rc0 + __ffsll((unsigned long long)cr) - 1;  // (cr != 0: the block leaves ep)
        const int ws = max(0, min(tstar - kCrossTerms / 2, len - kCrossTerms));
        const int we = min(len, ws + kCrossTerms);
        const int tb = ws / J;
        const int np = ws - tb * J;  // the window block's terms before the window
        const fold::Map mp = lane < np ? term_map(w[wide_pad(tb * J + lane)], ec) : fold::map_identity();
        const fold::Map ip = fold::wave_map_scan(mp);
        const fold::Map head = fold::Map{(uint32_t)__builtin_amdgcn_readlane((int)ip.t0, 63),
                                         (uint32_t)__builtin_amdgcn_readlane((int)ip.t1, 63)};
        const fold::Map sg = fold::compose(L.exm[tb], head);
        const uint64_t A1 = (uint64_t)Ac + fold::apply(sg, Ac & 1u);
        const float v0 = A1 < fold::kTop ? fold::from_A((uint32_t)A1, ec) : __builtin_nanf("");
        const int nw0 = we - ws;
        const float tl = lane < nw0 ? w[wide_pad(ws + lane)] : 0.f;
        const float f = wave_fold_f32(tl, v0, nw0);
        const float v = __uint_as_float((uint32_t)__builtin_amdgcn_readlane((int)__float_as_uint(f), nw0 - 1));
        if (lane == 0) {
          L.fend = v;
          L.x_ws = ws;
          L.x_we = we;
          cf->be[0] = (uint32_t)ec;
          cf->wn[0] = (uint32_t)nw0;
          cf->seg[0] = sg;
        }
      }
    }
    __syncthreads();
    {
      const int ws = L.x_ws;
      if (ws >= 0) {
        const int we = L.x_we;
        if (tid < we - ws) cf->term[0][tid] = w[wide_pad(ws + tid)];
        const float v = L.fend;
        nw = 1;
        p0 = we;
        ec = fold::binade(v);
        Ac = fold::to_A(v);
        if (!finitef_(v)) nw = 0;  // the prediction left the binade before the window
      }
    }
    // the rest of the chunk from p0 in binade ec: the threads' maps of
    // their terms from p0 on, and their scan.  The total is the last
    // segment, unless the fold leaves ec again: then window 1 (found as
    // window 0, by the wave holding the block that leaves) and the last
    // segment after it.
    if (nw == 1) {
      const int q0 = max(r0, p0);
      // a block wholly after p0 in one of the three binades: its map above
      const int kc = ec - e0;
      fold::Map mb = fold::map_identity();
      if (r0 >= p0 && kc >= 0 && kc < 3)
        mb = kc == 0 ? m0 : (kc == 1 ? m1 : m2);
      else
        wide_terms(w, q0, r1, [&](float x) { mb = fold::compose(mb, term_map(x, ec)); });
      fold::Map tot;
      const fold::Map ex = block_map_scan(mb, L.fl.wmap, &tot);
      if ((uint64_t)Ac + fold::apply(tot, Ac & 1u) < fold::kTop) {
        if (tid == 0) {
          cf->be[1] = (uint32_t)ec;
          cf->seg[1] = tot;
        }
      } else {
        if (tid == 0) L.x_ws = -1;
        L.exm[tid] = ex;  // (window 0's reads of exm ended at the barrier after it)
        __syncthreads();
        const uint64_t Ab = (uint64_t)Ac + fold::apply(ex, Ac & 1u);
        const uint64_t bal = __ballot(q0 < r1 && Ab < fold::kTop && Ab + fold::apply(mb, (uint32_t)Ab & 1u) >= fold::kTop);
        if (bal != 0ull) {
          const int lane = tid & 63;
          const int l = __ffsll((unsigned long long)bal) - 1;
          const int tc = (tid & ~63) + l;
          const int rc0 = max(tc * J, p0);
          const int nc = min(tc * J + J, len) - rc0;
          const uint32_t Ablk = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)Ab, l);
          const fold::Map mt = lane < nc ? term_map(w[wide_pad(rc0 + lane)], ec) : fold::map_identity();
          const fold::Map it = fold::wave_map_scan(mt);
          const uint64_t cr = __ballot(lane < nc && (uint64_t)Ablk + fold::apply(it, Ablk & 1u) >= fold::kTop);
          const int tstar = rc0 + __ffsll((unsigned long long)cr) - 1;
          const int ws = max(p0, min(tstar - kCrossTerms / 2, len - kCrossTerms));
          const int we = min(len, ws + kCrossTerms);
          const int tb = ws / J;
          const int hb = max(tb * J, p0);  // the window block's first term from p0 on
          const int np = ws - hb;
          const fold::Map mp = lane < np ? term_map(w[wide_pad(hb + lane)], ec) : fold::map_identity();
          const fold::Map ip = fold::wave_map_scan(mp);
          const fold::Map head = fold::Map{(uint32_t)__builtin_amdgcn_readlane((int)ip.t0, 63),
                                           (uint32_t)__builtin_amdgcn_readlane((int)ip.t1, 63)};
          const fold::Map sg = fold::compose(L.exm[tb], head);
          const uint64_t A1 = (uint64_t)Ac + fold::apply(sg, Ac & 1u);
          const float v0 = A1 < fold::kTop ? fold::from_A((uint32_t)A1, ec) : __builtin_nanf("");
          const int nw1 = we - ws;
          const float tl = lane < nw1 ? w[wide_pad(ws + lane)] : 0.f;
          const float f = wave_fold_f32(tl, v0, nw1);
          const float v = __uint_as_float((uint32_t)__builtin_amdgcn_readlane((int)__float_as_uint(f), nw1 - 1));
          if (lane == 0) {
            L.fend = v;
            L.x_ws = ws;
            L.x_we = we;
            cf->be[1] = (uint32_t)ec;
            cf->wn[1] = (uint32_t)nw1;
            cf->seg[1] = sg;
          }
        }
        __syncthreads();
        const int ws = L.x_ws;
        nw = 0;  // (no block leaves: not reached, the total leaves ec)
        if (ws >= 0) {
          const int we = L.x_we;
          if (tid < we - ws) cf->term[1][tid] = w[wide_pad(ws + tid)];
          const float v = L.fend;
          nw = finitef_(v) ? 2 : 0;  // (not finite: the prediction left the binade before the window)
          p0 = we;
          ec = fold::binade(v);
          Ac = fold::to_A(v);
        }
        if (nw == 2) {
          // the last segment [p0, len) in binade ec
          const int q2 = max(r0, p0);
          fold::Map ms = fold::map_identity();
          wide_terms(w, q2, r1, [&](float x) { ms = fold::compose(ms, term_map(x, ec)); });
          fold::Map sg;
          block_map_scan(ms, L.fl.wmap, &sg);
          if (tid == 0) {
            cf->be[2] = (uint32_t)ec;
            cf->seg[2] = sg;
          }
        }
      }
    }
    if (tid == 0) cf->nw = (uint32_t)nw;
  }
  // the superset's distinct weights
  constexpr int kLog2 = 11;
  static_assert((1 << kLog2) == kWideChunkHash, "hash size");
  bool full = false;
  for (int base = 0; base < len; base += 16 * NT) {
    float v[16];
    #pragma unroll
    for (int k = 0; k < 16; ++k) {
      const int i = base + k * NT + tid;
      v[k] = i < len ? w[wide_pad(i)] : 0.f;
    }
    #pragma unroll
    for (int k = 0; k < 16; ++k) {
      const int i = base + k * NT + tid;
      if (v[k] > 0.f && v[k] >= w_lo)
        full |= !wide_insert(L.hkey, L.hcnt, L.hmin, kLog2, __float_as_uint(v[k]), 1u, (uint32_t)i);
    }
  }
  if (full) L.ovf = 1u;
  __syncthreads();
  uint64_t* out = a.ws_list + (int64_t)row * a.list_stride + (int64_t)chunk * a.chunk;
  for (int h = tid; h < kWideChunkHash; h += NT) {
    const uint32_t k = L.hkey[h];
    if (k != 0u) {
      const uint32_t p = atomicAdd(&L.nrun, 1u);
      out[p] = ((uint64_t)k << 32) | ((uint64_t)L.hcnt[h] << 16) | (uint64_t)L.hmin[h];
    }
  }
  __syncthreads();
  if (tid == 0) cf->nruns = L.ovf ? kFoldNone : L.nrun;
}

// The exact fold value after chunk c's weights, from `acc` before them:
// reads the chunk's weights back (the chain's path when a chunk's sum
// leaves its binades).  All threads call it.
__device__ __forceinline__ float wide_refold(WideFinLds& F, unsigned char* lds_raw, const SampleArgs& a, int row,
                                             int c, float acc) {
  const int c0 = c * a.chunk;
  const int len = min(a.chunk, a.V - c0);
  float* w = reinterpret_cast<float*>(lds_raw + wide_fin_w_off());
  const float* wg = a.ws_w + (int64_t)row * a.V + c0;
  constexpr int kB = 8;
  for (int base = 0; base < len; base += kB * NT) {
    float v[kB];
    #pragma unroll
    for (int k = 0; k < kB; ++k) {
      const int i = base + k * NT + (int)threadIdx.x;
      v[k] = i < len ? wg[i] : 0.f;
    }
    #pragma unroll
    for (int k = 0; k < kB; ++k) {
      const int i = base + k * NT + (int)threadIdx.x;
      if (i < len) w[wide_pad(i)] = v[k];
    }
  }
  __syncthreads();
  return exact_chunk_fold(w, len, acc, F.fl.wmap, &F.acc2, F.fl.wcnt);
}

// The exact fold value after chunk c's weights from the exact value `acc`
// before them, when the chunk's sum leaves the binade it starts in: wave 0
// finds the crossing block from the chunk's stored block maps (a scan of the
// maps over the blocks; block b holds the chunk's terms [b * J, b * J + J),
// J = ceil(len / NT)), adds that block's terms one by one as real f32
// additions, and repeats in the new binade.  Returns kNone's float bits
// (NaN) when a binade falls outside the three stored ones; the caller then
// refolds the chunk.  Wave 0 only; the result is in lane 0 and every lane.
__device__ __forceinline__ float wide_cross_wave(const SampleArgs& a, int row, int c, float acc, bool& ok) {
  constexpr int PB = NT / 64;  // blocks per lane
  const int lane = threadIdx.x & 63;
  const ChunkFold cf = a.wfold[(int64_t)row * a.n_chunks + c];
  ok = (cf.flags & 8u) != 0u;  // a one-binade chunk stores no block maps: refold it
  if (!ok) return acc;
  const fold::Map* bm = a.wbmap + ((int64_t)row * a.n_chunks + c) * 3 * NT;
  const int c0 = c * a.chunk;
  const int len = min(a.chunk, a.V - c0);
  const int J = (len + NT - 1) / NT;
  const float* wg = a.ws_w + (int64_t)row * a.V + c0;
  float x = acc;
  int bstart = 0;
  ok = true;
  while (bstart < NT) {
    const int ey = fold::binade(x);
    const int k = ey - (int)cf.e0;
    if (k < 0 || k >= 3) { ok = false; return x; }
    // this lane's blocks 4 * lane .. (those before bstart count as identity)
    fold::Map bl[PB];
    fold::Map mine = fold::map_identity();
    #pragma unroll
    for (int q = 0; q < PB; ++q) {
      const int b = PB * lane + q;
      bl[q] = b >= bstart ? bm[k * NT + b] : fold::map_identity();
      mine = fold::compose(mine, bl[q]);
    }
    const fold::Map inc = fold::wave_map_scan(mine);
    const fold::Map ex = fold::wave_map_prev(inc);
    const uint32_t A = fold::to_A(x), p = A & 1u;
    const uint64_t cross = __ballot((uint64_t)A + fold::apply(inc, p) >= fold::kTop);
    if (cross == 0ull) {
      const fold::Map all = {(uint32_t)__builtin_amdgcn_readlane((int)inc.t0, 63),
                             (uint32_t)__builtin_amdgcn_readlane((int)inc.t1, 63)};
      return fold::from_A(A + fold::apply(all, p), ey);
    }
    const int fl = __ffsll((unsigned long long)cross) - 1;
    // in lane fl: the block where the sum leaves the binade, and the value before it
    uint32_t Ab = A + fold::apply(ex, p);  // A before this lane's blocks (< kTop: earlier lanes stayed)
    int blk = PB * lane + PB - 1;
    bool found = false;
    #pragma unroll
    for (int q = 0; q < PB; ++q) {
      const uint32_t t = fold::apply(bl[q], Ab & 1u);
      if (!found && (uint64_t)Ab + t >= fold::kTop) { blk = PB * lane + q; found = true; }
      if (!found) Ab += t;
    }
    blk = __builtin_amdgcn_readlane(blk, fl);
    Ab = (uint32_t)__builtin_amdgcn_readlane((int)Ab, fl);
    // the crossing block's terms as real additions (lane 0; the rest wait)
    float y = fold::from_A(Ab, ey);
    if (lane == 0) {
      const int r0 = min(blk * J, len), r1 = min(r0 + J, len);
      for (int r = r0; r < r1; ++r) y = fold::fadd(y, wg[r]);
    }
    x = __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(y), 0));
    bstart = blk + 1;
  }
  return x;
}

// The chain's step over a chunk whose fold leaves the binade it starts in,
// from the chunk's crossing record (in LDS): x (exact, in binade be[0]),
// then per window the segment before it by its map and the window's terms
// as real additions, then the last segment by its map.  False when the
// record does not apply (x is not in binade be[0], or the fold leaves a
// binade outside a window, or lands in another binade than predicted).
// Wave-uniform: every lane of the calling wave gets the same.
__device__ __forceinline__ bool wide_chain_cross(const ChunkFold& cf, float x, float& y) {
  const int lane = (int)(threadIdx.x & 63u);
  const int nw = (int)cf.nw;
  if (nw == 0 || (uint32_t)fold::binade(x) != cf.be[0]) return false;
  float v = x;
  for (int wdx = 0; wdx < nw; ++wdx) {
    const int e = (int)cf.be[wdx];
    const uint32_t A = fold::to_A(v);
    const uint64_t A1 = (uint64_t)A + fold::apply(cf.seg[wdx], A & 1u);
    if (A1 >= fold::kTop) return false;
    v = fold::from_A((uint32_t)A1, e);
    // the window's terms, one per lane, folded onto v in lane order
    const int n = (int)cf.wn[wdx];
    const float tl = lane < n ? cf.term[wdx][lane] : 0.f;
    const float f = wave_fold_f32(tl, v, n);
    v = __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(f), n - 1));
    if ((uint32_t)fold::binade(v) != cf.be[wdx + 1]) return false;
  }
  const uint32_t A = fold::to_A(v);
  const uint64_t A1 = (uint64_t)A + fold::apply(cf.seg[nw], A & 1u);
  if (A1 >= fold::kTop) return false;
  y = fold::from_A((uint32_t)A1, (int)cf.be[nw]);
  return true;
}

// The chain over chunks c .. cb + nb - 1 of the batch in LDS (nb <= 64),
// from the exact value x before chunk c, by one wave, lane i holding chunk
// c + i.  While the fold stays in one binade e the chunks' maps in e
// compose, so one scan over the lanes gives the value after every chunk up
// to the first whose map in e is not stored or leaves e; that chunk steps
// by its crossing record, and the scan resumes after it in the new binade.
// Returns the value after the last chunk it could step over and sets fail
// to the first chunk it could not (0xffffffff: none).
__device__ __forceinline__ float wide_wave_chain(const ChunkFold* batch, int cb, int nb, int c, float x,
                                                 uint32_t& fail) {
  const int lane = (int)(threadIdx.x & 63u);
  const int hi = c - cb + lane;
  const bool live = hi < nb;
  const ChunkFold& h = batch[live ? hi : 0];
  const int h_e0 = (int)h.e0;
  const uint32_t h_flags = h.flags;
  const bool h_end = live && h.has_end != 0u;
  const fold::Map hm0 = h.map[0], hm1 = h.map[1], hm2 = h.map[2];
  const uint32_t h_endv = __float_as_uint(h.end);
  fail = 0xffffffffu;
  int i0 = 0;  // the first lane (chunk c + i0) not yet stepped over
  const int n = cb + nb - c;
  while (i0 < n) {
    if (__builtin_amdgcn_readlane((int)h_end, i0)) {  // chunk 0, from -0.0
      x = __uint_as_float((uint32_t)__builtin_amdgcn_readlane((int)h_endv, i0));
      ++i0;
      continue;
    }
    const int e = fold::binade(x);
    const uint32_t A = fold::to_A(x);
    // this lane's map in binade e (saturated: not stored, or past the chunks)
    const int k = e - h_e0;
    const bool ok_l = lane >= i0 && lane < n && !h_end && k >= 0 && k < 3 && ((h_flags >> k) & 1u);
    fold::Map m = k == 0 ? hm0 : (k == 1 ? hm1 : hm2);
    if (!ok_l) m = fold::Map{fold::kSat, fold::kSat};
    if (lane < i0) m = fold::map_identity();
    // inclusive scan over the lanes: the increment after each chunk
    const fold::Map inc = fold::wave_map_scan(m);
    const uint64_t Ai = (uint64_t)A + fold::apply(inc, A & 1u);
    const uint64_t bad = __ballot(lane >= i0 && lane < n && Ai >= fold::kTop);
    if (bad == 0ull) {
      const uint32_t Al = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)Ai, n - 1);
      return fold::from_A(Al, e);
    }
    const int f = __ffsll((unsigned long long)bad) - 1;  // the first chunk that does not step in e
    if (f > i0) x = fold::from_A((uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)Ai, f - 1), e);
    float y = x;
    if (__builtin_amdgcn_readlane((int)h_end, f) || !wide_chain_cross(batch[c - cb + f], x, y)) {
      fail = (uint32_t)(c + f);
      return x;
    }
    x = y;
    i0 = f + 1;
  }
  return x;
}

// Calls f(c, e) for every superset run entry e of chunk c of `row`, in
// parallel: chunks in blocks of NT, their run counts scanned into offsets
// (a row of at most NT chunks whose offsets noff already holds passes their
// total as `ready_tot`, and the scan is skipped).
template <typename F>
__device__ __forceinline__ void wide_for_each_run(WideFinLds& W, const SampleArgs& a, int row, F f,
                                                  int ready_tot = -1) {
  const int tid = threadIdx.x;
  const int nch = a.n_chunks;
  const ChunkFold* folds = a.wfold + (int64_t)row * nch;
  for (int cb = 0; cb < nch; cb += NT) {
    uint32_t tot = (uint32_t)ready_tot;
    if (ready_tot < 0) {
      const int c = cb + tid;
      const uint32_t n = c < nch ? folds[c].nruns : 0u;
      const uint32_t off = block_excl_scan_u32<NT>(n, W.fl.wcnt, &tot);
      W.noff[tid] = off;
      if (tid == 0) W.noff[NT] = tot;
      __syncthreads();
    }
    // kU entries a thread: every load issued before the first is used
    constexpr int kU = 8;
    for (uint32_t base = 0; base < tot; base += kU * NT) {
      uint64_t v[kU];
      int cc[kU];
      // the last block whose offset is <= p, by a search of fixed steps
      // (the kU searches interleave; a data-dependent loop would run them
      // one after another, each step an LDS round trip)
      int lo[kU];
      #pragma unroll
      for (int k = 0; k < kU; ++k) lo[k] = 0;
      #pragma unroll
      for (int st = NT / 2; st >= 1; st >>= 1) {
        #pragma unroll
        for (int k = 0; k < kU; ++k) {
          const uint32_t p = base + (uint32_t)(k * NT + tid);
          lo[k] = W.noff[lo[k] + st] <= p ? lo[k] + st : lo[k];
        }
      }
      #pragma unroll
      for (int k = 0; k < kU; ++k) {
        const uint32_t p = base + (uint32_t)(k * NT + tid);
        cc[k] = -1;
        if (p < tot) {
          const uint64_t* src = a.ws_list + (int64_t)row * a.list_stride + (int64_t)(cb + lo[k]) * a.chunk;
          cc[k] = cb + lo[k];
          v[k] = src[p - W.noff[lo[k]]];
        }
      }
      #pragma unroll
      for (int k = 0; k < kU; ++k)
        if (cc[k] >= 0) f(cc[k], v[k]);
    }
    __syncthreads();
  }
}

// Step 4: the row finish by the last workgroup.  Returns the token, or
// 0xffffffff when the row must take finish_row (nothing written); `path`
// gets the WidePath code.
__device__ __forceinline__ uint32_t wide_finish(unsigned char* lds_raw, const SampleArgs& a, int row, const RowCfg& cfg, float M,
                                float w_lo, uint32_t& path) {
  WideFinLds& F = *reinterpret_cast<WideFinLds*>(lds_raw);
  const int tid = threadIdx.x;
  const int nch = a.n_chunks;
  const ChunkFold* folds = a.wfold + (int64_t)row * nch;

  // the merge's input (every chunk's superset runs, step c), loaded before
  // the chain so that its latency hides behind it: rows of more than kPreMin
  // entries a thread and up to kPreU (C2's bf16 rows: 3.6K entries; the merge
  // 11.6 -> 5 us), each with its chunk (a search of fixed steps over the
  // chunks' offsets in noff, which the chain leaves alone); rows of fewer
  // entries merge after the chain, where the early loads would delay the
  // chain's own more than they save
  constexpr int kPreU = 16, kPreMin = 4;
  uint64_t pv[kPreU];
  int pc[kPreU];
  bool pre_ok = nch <= NT;
  int ready_tot = -1;  // noff's total, when the merge can reuse it
  if (pre_ok) {
    uint32_t n = tid < nch ? folds[tid].nruns : 0u;
    n = n == kFoldNone ? 0u : n;  // (the row fails on the chunk's overflow below)
    uint32_t tot;
    const uint32_t off = block_excl_scan_u32<NT>(n, F.fl.wcnt, &tot);
    F.noff[tid] = off;
    if (tid == 0) F.noff[NT] = tot;
    __syncthreads();
    ready_tot = (int)tot;
    pre_ok = tot > (uint32_t)(kPreMin * NT) && tot <= (uint32_t)(kPreU * NT);
    if (pre_ok) {
      int lo[kPreU];
      #pragma unroll
      for (int k = 0; k < kPreU; ++k) lo[k] = 0;
      #pragma unroll
      for (int st = NT / 2; st >= 1; st >>= 1) {
        #pragma unroll
        for (int k = 0; k < kPreU; ++k) {
          const uint32_t p = (uint32_t)(k * NT + tid);
          lo[k] = F.noff[lo[k] + st] <= p ? lo[k] + st : lo[k];
        }
      }
      #pragma unroll
      for (int k = 0; k < kPreU; ++k) {
        const uint32_t p = (uint32_t)(k * NT + tid);
        pc[k] = -1;
        pv[k] = 0ull;
        if (p < tot) {
          pc[k] = lo[k];
          pv[k] = a.ws_list[(int64_t)row * a.list_stride + (int64_t)lo[k] * a.chunk + (p - F.noff[lo[k]])];
        }
      }
    }
  }

  // a. the normaliser: the chunk plans chained in vocabulary order
  //    (Rust's Sum folds from -0.0)
  float acc = -0.0f;
  bool ovf = false;
  for (int cb = 0; cb < nch; cb += kWideBatch) {
    const int nb = min(kWideBatch, nch - cb);
    {
      // 16-byte copies, every load of a thread issued before its stores
      static_assert(sizeof(ChunkFold) % 16 == 0, "ChunkFold in 16-byte pieces");
      const uint4* src = reinterpret_cast<const uint4*>(folds + cb);
      uint4* dst = reinterpret_cast<uint4*>(F.u.ch.batch);
      const int n4 = nb * (int)(sizeof(ChunkFold) / 16);
      constexpr int kU = 8;
      for (int base = 0; base < n4; base += kU * NT) {
        uint4 v[kU];
        #pragma unroll
        for (int k = 0; k < kU; ++k) {
          const int i = base + k * NT + tid;
          if (i < n4) v[k] = src[i];
        }
        #pragma unroll
        for (int k = 0; k < kU; ++k) {
          const int i = base + k * NT + tid;
          if (i < n4) dst[i] = v[k];
        }
      }
    }
    __syncthreads();
    for (int i = tid; i < nb; i += NT)
      if (F.u.ch.batch[i].nruns == kFoldNone) ovf = true;
    int c = cb;
    while (c < cb + nb) {
      if (tid < 64) {
        uint32_t fail;
        const float x = wide_wave_chain(F.u.ch.batch, cb, nb, c, acc, fail);
        if (tid == 0) {
          F.acc = x;
          F.fail_c = fail;
        }
      }
      __syncthreads();
      acc = F.acc;
      const uint32_t fail = F.fail_c;
      __syncthreads();
      if (fail == 0xffffffffu) break;
      // the chunk whose sum leaves its binade: the crossing from the block
      // maps (wave 0), else an exact refold of its weights
      if (tid < 64) {
        bool okw = true;
        const float y = wide_cross_wave(a, row, (int)fail, acc, okw);
        if (tid == 0) { F.acc = y; F.fail_c = okw ? 1u : 0u; }
      }
      __syncthreads();
      const bool crossed = F.fail_c != 0u;
      const float ycross = F.acc;
      __syncthreads();
      acc = crossed ? ycross : wide_refold(F, lds_raw, a, row, (int)fail, acc);
      c = (int)fail + 1;
    }
    __syncthreads();
  }
  ovf = __syncthreads_or(ovf);
  const float total = acc;
  if (tid == 0) a.wtot[2 * row] = total;
  path = kWideTotal;
  if (!(total > 0.f) || !finitef_(total)) return 0xffffffffu;  // argmax_host fallback (finish_row)
  path = kWideChunkFull;
  if (ovf) return 0xffffffffu;
  path = kWideMergeFull;

  // c. merge the chunks' runs by weight
  constexpr int kLog2 = 11;
  static_assert((1 << kLog2) == kWideFinHash, "hash size");
  for (int h = tid; h < kWideFinHash; h += NT) {
    F.u.mg.hkey[h] = 0u;
    F.u.mg.hcnt[h] = 0u;
    F.u.mg.hmin[h] = 0xffffffffu;
  }
  if (tid == 0) F.cnt = 0u;
  __syncthreads();
  bool full = false;
  auto insert = [&](int c, uint64_t e) {
    full |= !wide_insert(F.u.mg.hkey, F.u.mg.hcnt, F.u.mg.hmin, kLog2, (uint32_t)(e >> 32),
                         (uint32_t)(e >> 16) & 0xffffu, (uint32_t)(c * a.chunk) + ((uint32_t)e & 0xffffu));
  };
  if (pre_ok) {
    #pragma unroll
    for (int k = 0; k < kPreU; ++k)
      if (pc[k] >= 0) insert(pc[k], pv[k]);
  } else {
    wide_for_each_run(F, a, row, insert, ready_tot);
  }
  if (__syncthreads_or(full)) return 0xffffffffu;
  path = kWideDrawFail;
  // d. distinct weights, descending: the table's used slots compacted in
  //    order of (thread, slot) (thread t holds slots q * NT + t: their
  //    count, then a block scan of the counts), then ranked
  {
    constexpr int kSl = kWideFinHash / NT;
    uint32_t hk[kSl];
    uint32_t nu = 0u;
    #pragma unroll
    for (int q = 0; q < kSl; ++q) {
      hk[q] = F.u.mg.hkey[q * NT + tid];
      nu += hk[q] != 0u ? 1u : 0u;
    }
    uint32_t tot;
    uint32_t o = block_excl_scan_u32<NT>(nu, F.fl.wcnt, &tot);
    #pragma unroll
    for (int q = 0; q < kSl; ++q)
      if (hk[q] != 0u) F.u.mg.sortk[o++] = ((uint64_t)hk[q] << 32) | (uint64_t)(q * NT + tid);
    if (tid == 0) F.cnt = tot;
  }
  __syncthreads();
  const int R = (int)F.cnt;
  if (R == 0) return 0xffffffffu;
  if (R <= NT) {
    block_sort_desc<1>(F.u.mg.sortk, R);
  } else if (R <= 2 * NT) {
    block_sort_desc<2>(F.u.mg.sortk, R);
  } else if (R <= 4 * NT) {
    block_sort_desc<4>(F.u.mg.sortk, R);
  } else {
    const int n2 = next_pow2(R);
    for (int i = R + tid; i < n2; i += NT) F.u.mg.sortk[i] = 0ull;
    __syncthreads();
    for (int k = 2; k <= n2; k <<= 1) {
      for (int j = k >> 1; j > 0; j >>= 1) {
        for (int i = tid; i < n2; i += NT) {
          const int ixj = i ^ j;
          if (ixj > i) {
            const uint64_t x = F.u.mg.sortk[i], y = F.u.mg.sortk[ixj];
            const bool desc = (i & k) == 0;
            if (desc ? (x < y) : (x > y)) { F.u.mg.sortk[i] = y; F.u.mg.sortk[ixj] = x; }
          }
        }
        __syncthreads();
      }
    }
  }
  {
    // runs in rank order: read everything first, the arrays overlap
    constexpr int kPer = kWideRunCap / NT;
    float rx[kPer];
    uint32_t rm[kPer], ri[kPer];
    #pragma unroll
    for (int q = 0; q < kPer; ++q) {
      const int r = q * NT + tid;
      if (r < R) {
        const uint64_t k = F.u.mg.sortk[r];
        const uint32_t h = (uint32_t)k;
        rx[q] = __uint_as_float((uint32_t)(k >> 32));
        rm[q] = F.u.mg.hcnt[h];
        ri[q] = F.u.mg.hmin[h];
      }
    }
    __syncthreads();
    #pragma unroll
    for (int q = 0; q < kPer; ++q) {
      const int r = q * NT + tid;
      if (r < R) { F.u.fo.rx[r] = rx[q]; F.u.fo.rm[r] = rm[q]; F.u.fo.ri[r] = ri[q]; }
    }
    __syncthreads();
  }

  // e. cum_p += w / total in rank order (from 0.0), up to the cutoff
  auto q_of = [&](int r) { return F.u.fo.rx[r] / total; };
  auto m_of = [&](int r) { return F.u.fo.rm[r]; };
  const float cum_end = fold::fold_runs<NT>(F.fl, F.pe, R, 0.0f, q_of, m_of,
                                            [&](int r, float v) { F.u.fo.st[r] = v; });
  __syncthreads();
  int rstar = R - 1;
  uint32_t cstar = F.u.fo.rm[R - 1];
  if (cfg.cutoff < 1.f) {
    uint32_t first = 0xffffffffu;
    for (int r = tid; r < R; r += NT) {
      const float end = r + 1 < R ? F.u.fo.st[r + 1] : cum_end;
      if (end >= cfg.cutoff) first = min(first, (uint32_t)r);
    }
    first = ~block_max_u32<NT>(~first, F.fl.wcnt);
    if (first == 0xffffffffu) {
      // the cutoff is not reached inside the superset: that is the whole
      // nucleus only when the superset holds every positive weight
      if (w_lo > cfg.min_p) {
        path = kWideNoCutoff;
        return 0xffffffffu;
      }
    } else {
      rstar = (int)first;
      cstar = fold::run_find<false>(F.u.fo.st[rstar], q_of(rstar), F.u.fo.rm[rstar], cfg.cutoff, nullptr);
      if (cstar == fold::kNone) return 0xffffffffu;
    }
  }
  // f. the candidate total: the weights of the ranks before m_end (from -0.0)
  auto m2_of = [&](int r) { return r == rstar ? cstar : F.u.fo.rm[r]; };
  const float ct = fold::fold_runs<NT>(F.fl, F.pe, rstar + 1, -0.0f, [&](int r) { return F.u.fo.rx[r]; }, m2_of,
                                       [&](int r, float v) { F.u.fo.st2[r] = v; });
  __syncthreads();
  if (tid == 0) a.wtot[2 * row + 1] = ct;
  if (!(ct > 0.f) || !finitef_(ct)) return 0xffffffffu;
  // g. the inverse CDF: the first rank whose running weight passes target
  const float target = clamp_uniform(cfg.u) * ct;
  uint32_t pr = 0xffffffffu;
  for (int r = tid; r <= rstar; r += NT) {
    const float end = r < rstar ? F.u.fo.st2[r + 1] : ct;
    if (target < end) pr = min(pr, (uint32_t)r);
  }
  pr = ~block_max_u32<NT>(~pr, F.fl.wcnt);
  int rp = rstar;
  uint32_t cp = cstar;  // gpu.rs:899: the last candidate
  if (pr != 0xffffffffu) {
    const uint32_t c = fold::run_find<true>(F.u.fo.st2[pr], F.u.fo.rx[pr], m2_of((int)pr), target, nullptr);
    if (c != fold::kNone) { rp = (int)pr; cp = c; }
  }
  // h. the drawn index: the cp-th smallest index among the weights equal
  //    to the run's (equal weights rank by index)
  const uint32_t first_idx = F.u.fo.ri[rp];
  path = kWideDone;
  if (cp == 1u) return first_idx;
  const uint32_t key = __float_as_uint(F.u.fo.rx[rp]);
  __syncthreads();
  for (int c = tid; c < kWideRunCap; c += NT) F.u.cntc[c] = 0u;
  __syncthreads();
  if (nch > kWideRunCap) {
    path = kWideDrawFail;
    return 0xffffffffu;
  }
  wide_for_each_run(F, a, row, [&](int c, uint64_t e) {
    if ((uint32_t)(e >> 32) == key) F.u.cntc[c] = (uint32_t)(e >> 16) & 0xffffu;
  });
  if (tid < 64) {
    // the chunk holding the cp-th match: an inclusive scan of the chunks'
    // match counts over the lanes, 64 chunks at a time
    uint32_t seen = 0u, csel = 0xffffffffu, rsel = 0u;
    for (int cb = 0; cb < nch; cb += 64) {
      const int c = cb + tid;
      const uint32_t k = c < nch ? F.u.cntc[c] : 0u;
      const uint32_t inc = wave_incl_scan_u32(k);
      const uint64_t hit = __ballot(k != 0u && seen + inc >= cp);
      if (hit != 0ull) {
        const int l = __ffsll((unsigned long long)hit) - 1;
        const uint32_t before = seen + (uint32_t)__builtin_amdgcn_readlane((int)(inc - k), l);
        csel = (uint32_t)(cb + l);
        rsel = cp - before;
        break;
      }
      seen += (uint32_t)__builtin_amdgcn_readlane((int)inc, 63);
    }
    if (tid == 0) {
      F.csel = csel;
      F.rsel = rsel;
      F.tok = 0xffffffffu;
      F.cnt = 0u;
    }
  }
  __syncthreads();
  const uint32_t csel = F.csel, want = F.rsel;
  if (csel == 0xffffffffu) {
    path = kWideDrawFail;
    return 0xffffffffu;
  }
  // the want-th weight equal to key in chunk csel, in index order: the
  // chunk's weights (ws_w, written by its chunk work) in blocks of kE
  // consecutive ones per thread, all loads in flight at once; a thread's
  // count of matches before it by a scan over the threads
  const int c0 = (int)csel * a.chunk;
  const int len = min(a.chunk, a.V - c0);
  const float* wrow = a.ws_w + (int64_t)row * a.V + c0;
  constexpr int kE = 16;
  for (int base = 0; base < len; base += kE * NT) {
    const int i0 = base + tid * kE;
    uint32_t eqm = 0u;
    #pragma unroll
    for (int q = 0; q < kE; ++q) {
      const int i = i0 + q;
      const float x = i < len ? wrow[i] : 0.f;
      eqm |= (i < len && __float_as_uint(x) == key ? 1u : 0u) << q;
    }
    const uint32_t nm = (uint32_t)__popc(eqm);
    uint32_t tot;
    const uint32_t before = F.cnt + block_excl_scan_u32<NT>(nm, F.fl.wcnt, &tot);
    if (before < want && before + nm >= want) {
      uint32_t m = eqm;
      for (uint32_t r = want - before; r > 1u; --r) m &= m - 1u;  // drop the matches before the wanted one
      F.tok = (uint32_t)(c0 + i0 + __ffs(m) - 1);
    }
    __syncthreads();
    if (tid == 0) F.cnt += tot;
    __syncthreads();
    if (F.tok != 0xffffffffu) break;
  }
  if (F.tok == 0xffffffffu) path = kWideDrawFail;
  return F.tok;
}

// A whole row by one workgroup of NT threads, any row class: the select
// pass over kRowGeneralChunk-logit chunks in turn, then the chunked path's
// finish (finish_lean, else finish_row).  The workspace must hold the
// records of ceil(V / kRowGeneralChunk) chunks per row (general_layout);
// lds_raw must hold SelLds (plus the history table when a.hoff is given)
// and FinLds.
template <bool MASK>
__device__ __forceinline__ void general_row_path(SampleArgs& a, int row, unsigned char* lds_raw) {
  a.chunk = kRowGeneralChunk;
  a.n_chunks = (a.V + kRowGeneralChunk - 1) / kRowGeneralChunk;
  const RowCfg cfg = load_cfg(a.pv, row, a.V, a.n_lp, a.need_lse);
  for (int c = 0; c < a.n_chunks; ++c) {
    select_chunk<HI_ROCM_DTYPE_F32, kRowGeneralChunk / NT / 4, MASK>(a, row, c, lds_raw);
    __syncthreads();
  }
  if (threadIdx.x == 0) a.diag[row] = kRowPathGeneral;
  FinLds& fs = *reinterpret_cast<FinLds*>(lds_raw);
  if (finish_lean(fs, a, row, cfg)) return;
  __syncthreads();
  finish_row(fs, a, row, cfg);
}

}  // namespace hi_rocm
