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

}  // namespace

hipError_t launch_index_select(const float* scores, int n, int top_k, uint8_t* marks, int32_t* sel,
                               hipStream_t stream) {
  const int take = top_k < n ? top_k : n;
  hipLaunchKernelGGL(index_select_kernel, dim3(1), dim3(kSelThreads), 0, stream, scores, n, take,
                     marks, sel);
  return hipGetLastError();
}

}  // namespace hi_rocm
