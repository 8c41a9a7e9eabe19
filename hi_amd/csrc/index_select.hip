// Exact top-k block selection for the DeepSeek-V4 sparse-attention indexer
// (the select of crates/hi-cuda/src/kernels.cu:2610-2707, driven from
// crates/hi-cuda/src/dsv4_gpu.rs:4569 once per indexer layer).
//
// Semantics (the host's indexer_select_math, dsv4_cpu.rs:3258-3270): rank
// the n scores by Rust's f32 total_cmp descending, the lower index first
// on equal keys, keep the first take = min(top_k, n), and emit their indices
// in ascending order.  marks[b] = 1 for a kept block, 0 otherwise.
//
// One workgroup of 1024 threads (16 waves):
//  1. Radix descent over the 32-bit total-order key, 8 bits per pass: each
//     wave histograms the keys that share the prefix found so far into its
//     own 256 LDS bins; wave 0 sums the 16 histograms and, by a suffix scan
//     across its lanes (4 bins each), finds the bin that holds the take-th
//     largest key.  A pass whose bin is taken whole ends the descent (at
//     most 4 passes).  The result is a prefix P over the top 32-s bits and
//     the quota q of keys with that prefix to keep: every key whose prefix
//     is above P is kept (take - q of them), and of those equal to P the q
//     of lowest index.
//  2. Each wave owns a contiguous span of the scores.  It counts, with
//     ballots, its keys above P and equal to P; after one barrier every
//     wave knows how many of each lie before its span.
//  3. Each wave walks its span again, 64 scores a step: a key equal to P
//     is kept while its rank among equal keys (earlier waves, earlier steps,
//     lower lanes) is below q; a kept score's output slot is the number of
//     kept scores before it.  marks and the output are written in the same
//     walk, so the output comes out in ascending index order by
//     construction.
// Every decision is an integer compare or count, so the result does not
// depend on timing; the reference's serial thread-0 tie fill and compaction
// are replaced by the ballot ranks of steps 2-3.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "sampler_internal.h"
#include "wave_ops.h"

namespace hi_rocm {
hipError_t ensure_lds(const void* fn, size_t bytes);
}

namespace hi_rocm {
namespace {

constexpr int kSelThreads = 1024;
constexpr int kSelWaves = kSelThreads / 64;
constexpr int kSelBins = 256;

// f32 -> a key whose unsigned order is Rust's f32::total_cmp order
// (-NaN < -inf < ... < -0 < +0 < ... < +inf < +NaN).
__device__ __forceinline__ uint32_t total_key(float x) {
  const uint32_t u = __float_as_uint(x);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

struct SelLds {
  uint32_t hist[kSelWaves][kSelBins];
  uint32_t span_gt[kSelWaves];
  uint32_t span_eq[kSelWaves];
  uint32_t digit;  // the bin holding the take-th largest key
  uint32_t above;  // keys in the bins above it
  uint32_t count;  // keys in it
};

__global__ void __launch_bounds__(kSelThreads)
index_select_kernel(const float* __restrict__ scores, int n, int take, uint8_t* __restrict__ marks,
                    int32_t* __restrict__ sel) {
  __shared__ SelLds L;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wid = tid >> 6;
  const uint64_t below = (1ull << lane) - 1ull;

  // 1. radix descent
  uint32_t prefix = 0u;  // the chosen bins so far
  int shift = 32;        // key bits below the prefix
  uint32_t need = (uint32_t)take;
  for (int pass = 0; pass < 4; ++pass) {
    const int dshift = 24 - 8 * pass;
    for (int i = tid; i < kSelWaves * kSelBins; i += kSelThreads) (&L.hist[0][0])[i] = 0u;
    __syncthreads();
    uint32_t* h = L.hist[wid];
    for (int i = tid; i < n; i += kSelThreads) {
      const uint32_t k = total_key(scores[i]);
      if (pass == 0 || (k >> (dshift + 8)) == prefix) atomicAdd(&h[(k >> dshift) & 255u], 1u);
    }
    __syncthreads();
    if (wid == 0) {
      uint32_t c[4];
      uint32_t tot = 0u;
      #pragma unroll
      for (int q = 0; q < 4; ++q) {
        uint32_t s = 0u;
        #pragma unroll
        for (int w = 0; w < kSelWaves; ++w) s += L.hist[w][lane * 4 + q];
        c[q] = s;
        tot += s;
      }
      uint32_t incl = tot;
      #pragma unroll
      for (int off = 1; off < 64; off <<= 1) {
        const uint32_t y = __shfl_up(incl, off);
        if (lane >= off) incl += y;
      }
      uint32_t above = __shfl(incl, 63) - incl;  // keys in the bins of higher lanes
      #pragma unroll
      for (int q = 3; q >= 0; --q) {
        if (above < need && above + c[q] >= need) {
          L.digit = (uint32_t)(lane * 4 + q);
          L.above = above;
          L.count = c[q];
        }
        above += c[q];
      }
    }
    __syncthreads();
    const uint32_t d = L.digit;
    need -= L.above;
    const bool whole = L.count == need;
    prefix = (prefix << 8) | d;
    shift = dshift;
    __syncthreads();  // L is rewritten by the next pass
    if (whole) break;
  }

  // 2. per-wave counts over contiguous spans
  const int span = (((n + kSelWaves - 1) / kSelWaves) + 63) & ~63;
  const int s0 = wid * span;
  const int s1 = min(n, s0 + span);
  uint32_t gt = 0u, eq = 0u;
  for (int i0 = s0; i0 < s1; i0 += 64) {
    const int i = i0 + lane;
    const uint32_t hi = i < s1 ? total_key(scores[i]) >> shift : 0u;
    const bool in = i < s1;
    gt += (uint32_t)__popcll(__ballot(in && hi > prefix));
    eq += (uint32_t)__popcll(__ballot(in && hi == prefix));
  }
  if (lane == 0) {
    L.span_gt[wid] = gt;
    L.span_eq[wid] = eq;
  }
  __syncthreads();
  uint32_t gt_before = 0u, eq_before = 0u;
  #pragma unroll
  for (int w = 0; w < kSelWaves; ++w) {
    gt_before += w < wid ? L.span_gt[w] : 0u;
    eq_before += w < wid ? L.span_eq[w] : 0u;
  }

  // 3. marks and ascending output
  uint32_t eq_run = eq_before;
  uint32_t pos_run = gt_before + min(eq_before, need);
  for (int i0 = s0; i0 < s1; i0 += 64) {
    const int i = i0 + lane;
    const bool in = i < s1;
    const uint32_t hi = in ? total_key(scores[i]) >> shift : 0u;
    const bool is_gt = in && hi > prefix;
    const bool is_eq = in && hi == prefix;
    const uint64_t eqm = __ballot(is_eq);
    const bool keep = is_gt || (is_eq && eq_run + (uint32_t)__popcll(eqm & below) < need);
    const uint64_t km = __ballot(keep);
    const uint32_t slot = pos_run + (uint32_t)__popcll(km & below);
    if (keep && slot < (uint32_t)take) sel[slot] = i;
    if (in) marks[i] = keep ? 1u : 0u;
    eq_run += (uint32_t)__popcll(eqm);
    pos_run += (uint32_t)__popcll(km);
  }
}

// The same three steps with every key held in registers: wave w owns the
// contiguous span [w * 64 * PER, (w + 1) * 64 * PER), lane l its elements
// span + j * 64 + l (j < PER), loaded once with all loads in flight (the
// loop form above reloads the scores on every pass and waits on each load).
// The descent takes 12, 10 and 10 bits: float keys crowd into few values of
// their top 8 bits (sign and exponent), and lanes of one wave adding to the
// same LDS bin are serialised, so the first digit reaches 3 mantissa bits
// into one shared 4096-bin histogram.  For n <= 1024 * PER.
constexpr int kRegBins = 4096;

struct RegSelLds {
  uint32_t hist[kRegBins];
  uint32_t wsum[kSelWaves];
  uint32_t span_gt[kSelWaves];
  uint32_t span_eq[kSelWaves];
  uint32_t digit, above, count;
};

// The bin of hist[0, 1024 * BPT) that holds the need-th largest key
// (thread t owns bins [t * BPT, t * BPT + BPT)), with the keys in the bins
// above it and in it.  Ends with a barrier; every thread reads the result.
template <int BPT>
__device__ __forceinline__ void reg_find_bin(RegSelLds& L, uint32_t need) {
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  uint32_t c[BPT], tot = 0u;
  #pragma unroll
  for (int q = 0; q < BPT; ++q) {
    c[q] = L.hist[tid * BPT + q];
    tot += c[q];
  }
  uint32_t sfx = tot;  // this lane and the lanes above it in the wave
  #pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const uint32_t y = (uint32_t)__shfl_down((int)sfx, (unsigned)d, 64);
    if (lane + d < 64) sfx += y;
  }
  if (lane == 0) L.wsum[wid] = sfx;
  __syncthreads();
  uint32_t above = sfx - tot;
  for (int w = wid + 1; w < kSelWaves; ++w) above += L.wsum[w];
  #pragma unroll
  for (int q = BPT - 1; q >= 0; --q) {
    if (above < need && above + c[q] >= need) {
      L.digit = (uint32_t)(tid * BPT + q);
      L.above = above;
      L.count = c[q];
    }
    above += c[q];
  }
  __syncthreads();
}

template <int PER>
__global__ void __launch_bounds__(kSelThreads)
index_select_reg_kernel(const float* __restrict__ scores, int n, int take, uint8_t* __restrict__ marks,
                        int32_t* __restrict__ sel, int vec) {
  static_assert(PER % 4 == 0, "four consecutive elements per lane and group");
  constexpr int G = PER / 4;  // groups of 256 elements per wave
  __shared__ RegSelLds L;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wid = tid >> 6;
  const int s0 = wid * 64 * PER;
  // lane l holds elements s0 + g * 256 + 4 * l + q, q < 4 (16-byte loads
  // and 4-byte mark stores when `vec`: aligned pointers and n a multiple of
  // 4; otherwise element by element)
  uint32_t key[PER];
  if (vec) {
    // every load issued before any is used: out-of-range groups load
    // element 0 and are masked afterwards
    float4 v[G];
    #pragma unroll
    for (int g = 0; g < G; ++g) {
      const int i0 = s0 + g * 256 + 4 * lane;
      v[g] = *reinterpret_cast<const float4*>(scores + (i0 < n ? i0 : 0));
    }
    #pragma unroll
    for (int g = 0; g < G; ++g) {
      const bool in = s0 + g * 256 + 4 * lane < n;
      key[4 * g + 0] = in ? total_key(v[g].x) : 0u;
      key[4 * g + 1] = in ? total_key(v[g].y) : 0u;
      key[4 * g + 2] = in ? total_key(v[g].z) : 0u;
      key[4 * g + 3] = in ? total_key(v[g].w) : 0u;
    }
  } else {
    float v[PER];
    #pragma unroll
    for (int j = 0; j < PER; ++j) {
      const int i = s0 + (j >> 2) * 256 + 4 * lane + (j & 3);
      v[j] = scores[i < n ? i : 0];
    }
    #pragma unroll
    for (int j = 0; j < PER; ++j) key[j] = s0 + (j >> 2) * 256 + 4 * lane + (j & 3) < n ? total_key(v[j]) : 0u;
  }
  auto idx = [&](int j) { return s0 + (j >> 2) * 256 + 4 * lane + (j & 3); };
  // 1. radix descent over bits [31:20], [19:10], [9:0] (keys past n never count)
  uint32_t prefix = 0u;
  int shift = 32;
  uint32_t need = (uint32_t)take;
  #pragma unroll 1
  for (int pass = 0; pass < 3; ++pass) {
    const int dshift = pass == 0 ? 20 : (pass == 1 ? 10 : 0);
    const uint32_t dmask = pass == 0 ? 4095u : 1023u;
    const int nb = pass == 0 ? kRegBins : 1024;
    for (int i = tid; i < nb; i += kSelThreads) L.hist[i] = 0u;
    __syncthreads();
    #pragma unroll
    for (int j = 0; j < PER; ++j)
      if (idx(j) < n && (pass == 0 || (key[j] >> shift) == prefix)) atomicAdd(&L.hist[(key[j] >> dshift) & dmask], 1u);
    __syncthreads();
    if (pass == 0) reg_find_bin<kRegBins / kSelThreads>(L, need);
    else reg_find_bin<1>(L, need);
    const uint32_t d = L.digit;
    need -= L.above;
    const bool whole = L.count == need;
    prefix = pass == 0 ? d : ((prefix << 10) | d);
    shift = dshift;
    __syncthreads();  // L is rewritten by the next pass
    if (whole) break;
  }
  // 2. per-wave counts (per-lane counters, one reduction)
  uint32_t gt = 0u, eq = 0u;
  #pragma unroll
  for (int j = 0; j < PER; ++j) {
    const bool in = idx(j) < n;
    const uint32_t hi = key[j] >> shift;
    gt += (in && hi > prefix) ? 1u : 0u;
    eq += (in && hi == prefix) ? 1u : 0u;
  }
  uint32_t packed = (eq << 16) | gt;  // per lane <= PER each
  #pragma unroll
  for (int o = 32; o > 0; o >>= 1) packed += (uint32_t)__shfl_xor((int)packed, o, 64);
  if (lane == 0) {
    L.span_gt[wid] = packed & 0xffffu;
    L.span_eq[wid] = packed >> 16;
  }
  __syncthreads();
  uint32_t gt_run = 0u, eq_run = 0u;
  #pragma unroll
  for (int w = 0; w < kSelWaves; ++w) {
    gt_run += w < wid ? L.span_gt[w] : 0u;
    eq_run += w < wid ? L.span_eq[w] : 0u;
  }
  // 3. marks and ascending output, a group of 256 elements at a time: the
  //    (greater, equal) counts before each element come from one exclusive
  //    scan of the lanes' packed counts
  #pragma unroll
  for (int g = 0; g < G; ++g) {
    uint32_t cg = 0u, ce = 0u;
    bool is_gt[4], is_eq[4];
    #pragma unroll
    for (int q = 0; q < 4; ++q) {
      const bool in = idx(4 * g + q) < n;
      const uint32_t hi = key[4 * g + q] >> shift;
      is_gt[q] = in && hi > prefix;
      is_eq[q] = in && hi == prefix;
      cg += is_gt[q] ? 1u : 0u;
      ce += is_eq[q] ? 1u : 0u;
    }
    const uint32_t mine = (ce << 16) | cg;
    const uint32_t incl = wave_incl_scan_u32(mine);
    const uint32_t excl = incl - mine;
    uint32_t G0 = gt_run + (excl & 0xffffu), E0 = eq_run + (excl >> 16);
    uint32_t mk = 0u;
    #pragma unroll
    for (int q = 0; q < 4; ++q) {
      const bool keep = is_gt[q] || (is_eq[q] && E0 < need);
      const uint32_t slot = G0 + min(E0, need);
      if (keep && slot < (uint32_t)take) sel[slot] = idx(4 * g + q);
      mk |= (keep ? 1u : 0u) << (8 * q);
      G0 += is_gt[q] ? 1u : 0u;
      E0 += is_eq[q] ? 1u : 0u;
    }
    const int i0 = idx(4 * g);
    if (vec && i0 < n) {
      *reinterpret_cast<uint32_t*>(marks + i0) = mk;
    } else {
      #pragma unroll
      for (int q = 0; q < 4; ++q)
        if (i0 + q < n) marks[i0 + q] = (uint8_t)(mk >> (8 * q));
    }
    const uint32_t tot = (uint32_t)__builtin_amdgcn_readlane((int)incl, 63);
    gt_run += tot & 0xffffu;
    eq_run += tot >> 16;
  }
}

// --------------------------------------------------------------------------
// Many workgroups (n above kMultiMinN): three kernels over spans of
// kSpan = 4096 scores, one span per workgroup of 1024 threads (4 scores a
// thread), with a small workspace:
//  1. multi_hist_kernel: each workgroup histograms its span's top 12 key
//     bits in LDS and adds the nonzero bins into one global histogram.
//  2. multi_cand_kernel: every workgroup reads the global histogram and
//     finds, as the one-workgroup kernel does, the bin b1 that holds the
//     take-th largest key, the keys above it and the keys in it (E); it
//     writes its counts of keys above b1 and in b1, and its keys in b1 to
//     its own candidate region as 64-bit composites: the low 20 key bits,
//     then the complement of the index (larger composite = higher rank).
//  3. multi_out_kernel: every workgroup reads b1 and the spans' counts,
//     gathers the candidates (into LDS when they fit), selects the q1-th
//     largest composite T (radix select; over global memory when E >
//     kCandLds), counts the keys kept before its span, and writes its marks
//     and its part of the ascending output; it then clears its slice of the
//     histogram.
// The histogram is zero between calls.  Every decision is
// an integer compare or count, as in the one-workgroup kernels, so the
// result is the same.
constexpr int kSpan = 4096;
constexpr int kMultiBins = 4096;  // top 12 key bits
constexpr int kCandLds = 8192;    // candidates the output kernel holds in LDS
constexpr int kMultiMaxG = kSelThreads;  // spans: one per thread of a workgroup

struct MultiWs {
  uint32_t* hist;   // [kMultiBins], zero between calls
  uint32_t* cnt;    // [G][2]: keys above b1 and in b1 per span; then b1 and the keys above it
  uint64_t* cand;   // [G][kSpan]: each span's candidates
};

// The span's scores as keys, 4 consecutive ones per thread (index
// g * kSpan + 4 * tid + q); keys past n are 0 (the callers test the index).
__device__ __forceinline__ void span_keys(const float* scores, int n, int g, int vec, uint32_t (&key)[4]) {
  const int i0 = g * kSpan + 4 * (int)threadIdx.x;
  if (vec && i0 + 3 < n) {
    const float4 v = *reinterpret_cast<const float4*>(scores + i0);
    key[0] = total_key(v.x); key[1] = total_key(v.y); key[2] = total_key(v.z); key[3] = total_key(v.w);
  } else {
    #pragma unroll
    for (int q = 0; q < 4; ++q) key[q] = i0 + q < n ? total_key(scores[i0 + q]) : 0u;
  }
}

__device__ __forceinline__ uint64_t composite(uint32_t key, uint32_t i) {
  return ((uint64_t)(key & 0xfffffu) << 32) | (uint64_t)(0xffffffffu - i);
}

__global__ void __launch_bounds__(kSelThreads) multi_hist_kernel(const float* __restrict__ scores, int n, int vec,
                                                                 MultiWs ws) {
  __shared__ uint32_t hist[kMultiBins];
  const int g = blockIdx.x, tid = threadIdx.x;
  uint32_t key[4];
  span_keys(scores, n, g, vec, key);
  for (int i = tid; i < kMultiBins; i += kSelThreads) hist[i] = 0u;
  __syncthreads();
  const int i0 = g * kSpan + 4 * tid;
  #pragma unroll
  for (int q = 0; q < 4; ++q)
    if (i0 + q < n) atomicAdd(&hist[key[q] >> 20], 1u);
  __syncthreads();
  for (int i = tid; i < kMultiBins; i += kSelThreads)
    if (hist[i] != 0u) atomicAdd(&ws.hist[i], hist[i]);
}

__global__ void __launch_bounds__(kSelThreads) multi_cand_kernel(const float* __restrict__ scores, int n, int take,
                                                                 int vec, MultiWs ws) {
  __shared__ RegSelLds L;
  __shared__ uint32_t wgt[kSelWaves];
  const int g = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int G = (int)gridDim.x;
  uint32_t key[4];
  span_keys(scores, n, g, vec, key);
  constexpr int BPT = kMultiBins / kSelThreads;
  #pragma unroll
  for (int q = 0; q < BPT; ++q) L.hist[tid * BPT + q] = ws.hist[tid * BPT + q];
  __syncthreads();
  reg_find_bin<BPT>(L, (uint32_t)take);
  const uint32_t b1 = L.digit;
  const int i0 = g * kSpan + 4 * tid;
  uint32_t gt = 0u, ne = 0u;
  #pragma unroll
  for (int q = 0; q < 4; ++q) {
    const bool in = i0 + q < n;
    gt += (in && (key[q] >> 20) > b1) ? 1u : 0u;
    ne += (in && (key[q] >> 20) == b1) ? 1u : 0u;
  }
  // candidate places in the span's region: an exclusive scan of the
  // per-thread counts (both counts packed, each at most kSpan)
  const uint32_t packed = (ne << 16) | gt;
  const uint32_t incl = wave_incl_scan_u32(packed);
  if (lane == 63) wgt[wid] = incl;
  __syncthreads();
  uint32_t before = 0u, tot = 0u;
  #pragma unroll
  for (int w = 0; w < kSelWaves; ++w) {
    before += w < wid ? wgt[w] : 0u;
    tot += wgt[w];
  }
  uint32_t at = (before + incl - packed) >> 16;
  uint64_t* cand = ws.cand + (int64_t)g * kSpan;
  #pragma unroll
  for (int q = 0; q < 4; ++q)
    if (i0 + q < n && (key[q] >> 20) == b1) cand[at++] = composite(key[q], (uint32_t)(i0 + q));
  if (tid == 0) {
    ws.cnt[2 * g] = tot & 0xffffu;
    ws.cnt[2 * g + 1] = tot >> 16;
    if (g == 0) {
      // for the output kernel, whose workgroups clear the histogram
      ws.cnt[2 * G] = b1;
      ws.cnt[2 * G + 1] = L.above;
    }
  }
}

// LDS of the output kernel.
struct OutLds {
  RegSelLds r;
  uint32_t bins[256];
  uint32_t eoff[kMultiMaxG + 1];  // candidates before span h
  uint64_t red64[kSelWaves];
  uint64_t cand[kCandLds];
  uint32_t gt_before;
  uint32_t digit, above, count;
};

// The need-th largest of the distinct values item(0 .. m-1) below 2^52
// (1 <= need <= m), by an 8-bit radix descent (digits at bits 44, 36, ...,
// 4, 0; the last overlaps the one before, whose bits the prefix already
// fixes) that stops at a bin taken whole; every thread returns it.
template <typename Item>
__device__ __forceinline__ uint64_t block_select_u64(OutLds& L, int m, uint32_t need, Item item) {
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  uint64_t prefix = 0ull;
  int shift = 44, pshift = 64;  // this digit's lowest bit; the prefix's (64: none yet)
  for (;;) {
    for (int i = tid; i < 256; i += kSelThreads) L.bins[i] = 0u;
    __syncthreads();
    for (int i = tid; i < m; i += kSelThreads) {
      const uint64_t x = item(i);
      if (pshift == 64 || (x >> pshift) == (prefix >> pshift))
        atomicAdd(&L.bins[(uint32_t)(x >> shift) & 255u], 1u);
    }
    __syncthreads();
    if (wid == 0) {
      uint32_t c[4], tot = 0u;
      #pragma unroll
      for (int q = 0; q < 4; ++q) { c[q] = L.bins[lane * 4 + q]; tot += c[q]; }
      uint32_t incl = tot;
      #pragma unroll
      for (int off = 1; off < 64; off <<= 1) {
        const uint32_t y = __shfl_up(incl, off);
        if (lane >= off) incl += y;
      }
      uint32_t above = __shfl(incl, 63) - incl;
      #pragma unroll
      for (int q = 3; q >= 0; --q) {
        if (above < need && above + c[q] >= need) { L.digit = (uint32_t)(lane * 4 + q); L.above = above; L.count = c[q]; }
        above += c[q];
      }
    }
    __syncthreads();
    need -= L.above;
    prefix |= (uint64_t)L.digit << shift;
    const bool whole = L.count == need;
    __syncthreads();
    pshift = shift;
    if (whole || shift == 0) break;
    shift = shift > 8 ? shift - 8 : 0;
  }
  if (shift == 0) return prefix;
  // the bin's values are all kept: the threshold is the smallest of them
  uint64_t mn = ~0ull;
  for (int i = tid; i < m; i += kSelThreads) {
    const uint64_t x = item(i);
    if ((x >> shift) == (prefix >> shift) && x < mn) mn = x;
  }
  #pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const uint64_t y = ((uint64_t)(uint32_t)__shfl_xor((int)(uint32_t)(mn >> 32), o, 64) << 32) |
                       (uint32_t)__shfl_xor((int)(uint32_t)mn, o, 64);
    mn = y < mn ? y : mn;
  }
  if (lane == 0) L.red64[wid] = mn;
  __syncthreads();
  uint64_t r = ~0ull;
  #pragma unroll
  for (int w = 0; w < kSelWaves; ++w) r = L.red64[w] < r ? L.red64[w] : r;
  __syncthreads();
  return r;
}

// A span's marks and its part of the ascending output: a key is kept when
// its top 12 bits are above b1, or equal with a composite at or above T;
// kept_before keys are kept in the spans before it.
__device__ __forceinline__ void span_emit(OutLds& L, const uint32_t (&key)[4], int n, int g, int take, uint32_t b1,
                                          uint64_t T, uint32_t kept_before, int vec, uint8_t* __restrict__ marks,
                                          int32_t* __restrict__ sel) {
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int i0 = g * kSpan + 4 * tid;
  uint32_t mk = 0u, nk = 0u;
  #pragma unroll
  for (int q = 0; q < 4; ++q) {
    const uint32_t hb = key[q] >> 20;
    const bool keep = i0 + q < n && (hb > b1 || (hb == b1 && composite(key[q], (uint32_t)(i0 + q)) >= T));
    mk |= (keep ? 1u : 0u) << (8 * q);
    nk += keep ? 1u : 0u;
  }
  // slots by an exclusive scan over the threads
  const uint32_t incl = wave_incl_scan_u32(nk);
  __syncthreads();
  if (lane == 63) L.r.span_gt[wid] = incl;
  __syncthreads();
  uint32_t slot = kept_before + incl - nk;
  #pragma unroll
  for (int w = 0; w < kSelWaves; ++w) slot += w < wid ? L.r.span_gt[w] : 0u;
  #pragma unroll
  for (int q = 0; q < 4; ++q) {
    if ((mk >> (8 * q)) & 1u) {
      if (slot < (uint32_t)take) sel[slot] = i0 + q;
      ++slot;
    }
  }
  if (vec && i0 + 3 < n) {
    *reinterpret_cast<uint32_t*>(marks + i0) = mk;
  } else {
    #pragma unroll
    for (int q = 0; q < 4; ++q)
      if (i0 + q < n) marks[i0 + q] = (uint8_t)(mk >> (8 * q));
  }
}

__global__ void __launch_bounds__(kSelThreads) multi_out_kernel(const float* __restrict__ scores, int n, int take,
                                                                int vec, MultiWs ws, uint8_t* __restrict__ marks,
                                                                int32_t* __restrict__ sel) {
  extern __shared__ __align__(16) unsigned char lds_raw[];
  OutLds& L = *reinterpret_cast<OutLds*>(lds_raw);
  const int g = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int G = (int)gridDim.x;
  uint32_t key[4];
  span_keys(scores, n, g, vec, key);
  const uint32_t b1 = ws.cnt[2 * G];
  const uint32_t q1 = (uint32_t)take - ws.cnt[2 * G + 1];  // keys of bin b1 to keep (>= 1)
  // the spans' counts (one span per thread): keys above b1 before this
  // span, and the candidates' offsets in the concatenation span after span
  {
    const uint32_t c0 = tid < G ? ws.cnt[2 * tid] : 0u;
    const uint32_t c1 = tid < G ? ws.cnt[2 * tid + 1] : 0u;
    uint32_t gb = tid < g ? c0 : 0u;
    #pragma unroll
    for (int o = 32; o > 0; o >>= 1) gb += (uint32_t)__shfl_xor((int)gb, o, 64);
    const uint32_t incl = wave_incl_scan_u32(c1);
    if (lane == 63) L.r.span_eq[wid] = incl;
    if (lane == 0) L.r.span_gt[wid] = gb;
    __syncthreads();
    uint32_t eb = incl - c1;
    #pragma unroll
    for (int w = 0; w < kSelWaves; ++w) eb += w < wid ? L.r.span_eq[w] : 0u;
    if (tid < G) L.eoff[tid] = eb;
    if (tid == G - 1) L.eoff[G] = eb + c1;  // the total
    if (tid == 0) {
      uint32_t a = 0u;
      for (int w = 0; w < kSelWaves; ++w) a += L.r.span_gt[w];
      L.gt_before = a;
    }
    __syncthreads();
  }
  const uint32_t E = L.eoff[G];
  // candidate j of the concatenation: the span holding it by a binary
  // search of the offsets
  auto gitem = [&](int j) -> uint64_t {
    int lo = 0, hi = G - 1;  // the last span h with eoff[h] <= j
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (L.eoff[mid] <= (uint32_t)j) lo = mid;
      else hi = mid - 1;
    }
    return ws.cand[(int64_t)lo * kSpan + ((uint32_t)j - L.eoff[lo])];
  };
  const bool in_lds = E <= (uint32_t)kCandLds;
  if (in_lds) {
    for (int j = tid; j < (int)E; j += kSelThreads) L.cand[j] = gitem(j);
    __syncthreads();
  }
  const uint64_t T = in_lds ? block_select_u64(L, (int)E, q1, [&](int j) { return L.cand[j]; })
                            : block_select_u64(L, (int)E, q1, gitem);
  // candidates kept before this span
  uint32_t kb = 0u;
  const int eb = (int)L.eoff[g];
  for (int j = tid; j < eb; j += kSelThreads) kb += (in_lds ? L.cand[j] : gitem(j)) >= T ? 1u : 0u;
  #pragma unroll
  for (int o = 32; o > 0; o >>= 1) kb += (uint32_t)__shfl_xor((int)kb, o, 64);
  __syncthreads();
  if (lane == 0) L.r.wsum[wid] = kb;
  __syncthreads();
  uint32_t kept_before = L.gt_before;
  #pragma unroll
  for (int w = 0; w < kSelWaves; ++w) kept_before += L.r.wsum[w];
  span_emit(L, key, n, g, take, b1, T, kept_before, vec, marks, sel);
  // the histogram back to zero for the next call (only the previous kernel
  // read it)
  for (int i = g * kSelThreads + tid; i < kMultiBins; i += G * kSelThreads) ws.hist[i] = 0u;
}

}  // namespace

// Bytes of the workspace of launch_index_select_multi (0: n takes the
// one-workgroup kernels); its first kIndexHistBytes must be zero before the
// first call (the calls leave them so).
size_t index_select_ws_bytes(int n) {
  if (n <= kMultiMinN || n > kSpan * kMultiMaxG) return 0;
  const int G = (n + kSpan - 1) / kSpan;
  return kIndexHistBytes + (((size_t)(G + 1) * 2 * sizeof(uint32_t) + 255) & ~(size_t)255) +
         (size_t)G * kSpan * sizeof(uint64_t);
}

hipError_t launch_index_select_multi(const float* scores, int n, int top_k, uint8_t* marks, int32_t* sel,
                                     void* ws_mem, hipStream_t stream) {
  static_assert(kIndexHistBytes >= kMultiBins * sizeof(uint32_t), "histogram");
  const int take = top_k < n ? top_k : n;
  const int vec = ((uintptr_t)scores % 16 == 0) && ((uintptr_t)marks % 4 == 0) && (n % 4 == 0);
  const int G = (n + kSpan - 1) / kSpan;
  MultiWs ws;
  ws.hist = (uint32_t*)ws_mem;
  ws.cnt = (uint32_t*)((char*)ws_mem + kIndexHistBytes);
  ws.cand = (uint64_t*)((char*)ws.cnt + (((size_t)(G + 1) * 2 * sizeof(uint32_t) + 255) & ~(size_t)255));
  hipLaunchKernelGGL(multi_hist_kernel, dim3(G), dim3(kSelThreads), 0, stream, scores, n, vec, ws);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(multi_cand_kernel, dim3(G), dim3(kSelThreads), 0, stream, scores, n, take, vec, ws);
  e = hipGetLastError();
  if (e != hipSuccess) return e;
  const size_t lds = sizeof(OutLds);
  e = ensure_lds((const void*)multi_out_kernel, lds);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(multi_out_kernel, dim3(G), dim3(kSelThreads), lds, stream, scores, n, take, vec, ws, marks, sel);
  return hipGetLastError();
}

hipError_t launch_index_select(const float* scores, int n, int top_k, uint8_t* marks, int32_t* sel,
                               hipStream_t stream) {
  const int take = top_k < n ? top_k : n;
  const int vec = ((uintptr_t)scores % 16 == 0) && ((uintptr_t)marks % 4 == 0) && (n % 4 == 0);
  if (n <= kSelThreads * 4)
    hipLaunchKernelGGL(index_select_reg_kernel<4>, dim3(1), dim3(kSelThreads), 0, stream, scores, n, take, marks, sel,
                       vec);
  else if (n <= kSelThreads * 16)
    hipLaunchKernelGGL(index_select_reg_kernel<16>, dim3(1), dim3(kSelThreads), 0, stream, scores, n, take, marks,
                       sel, vec);
  else if (n <= kSelThreads * 64)
    hipLaunchKernelGGL(index_select_reg_kernel<64>, dim3(1), dim3(kSelThreads), 0, stream, scores, n, take, marks,
                       sel, vec);
  else
    hipLaunchKernelGGL(index_select_kernel, dim3(1), dim3(kSelThreads), 0, stream, scores, n, take, marks, sel);
  return hipGetLastError();
}

}  // namespace hi_rocm
