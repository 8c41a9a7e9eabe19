// MoE router top-k (the mirror of crates/hi-cuda/src/kernels.cu:536-684,
// launcher :8482-8510 hi_cuda_launch_moe_topk_router).
//
// The reference gives each row one thread that rescans every expert once
// per selected rank (top_k x experts exponentials per row).  Here one wave
// owns a row: expert e sits in lane e % 64, slot e / 64, so the scores are
// read once, coalesced, and every per-rank scan is a wave reduction.
//
// Semantics kept from the reference, step by step:
//  * softmax gating: max_score by '>' in expert order (NaN never wins); a
//    non-finite max, or a sum of exp(s - max) that is not positive and
//    finite, gives ids 0 .. k-1 with weight 1/k (normalised, k > 1) or 1/E;
//    the sum is the f32 sequential fold in expert order; weight =
//    exp(s - max) / sum, non-finite -> 0;
//  * sigmoid gating: score = 1 / (1 + exp(-s)), non-finite -> 0; the rank
//    key is score + selection_bias[e] (when given) and the weight the score;
//  * rank r takes the expert the reference's scan picks: among the experts
//    eligible after rank r-1 (key below the previous key, or equal with a
//    higher id), the scan keeps the first one and replaces it by any later
//    one with a strictly larger key -- so a NaN key at the first eligible
//    expert stays, otherwise the largest non-NaN key with the lowest id
//    wins; with no eligible expert, id = min(r, E-1) and weight 0;
//  * the selected weights' f32 sum in rank order normalises them (norm_topk,
//    k > 1, sum > 1e-7 and finite), then weights_scale multiplies them.
// The exponential is glibc's expf (exact_expf.h), as in the sampler.  The
// reference calls CUDA's expf, whose results are not reproduced here.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "exact_expf.h"
#include "hi_rocm.h"
#include "sampler_internal.h"
#include "wave_ops.h"

namespace hi_rocm {
namespace {

constexpr int kRouterWaves = 4;            // rows per workgroup
constexpr int kRouterMaxExperts = 2048;    // 32 slots of 64 lanes

__device__ __forceinline__ bool finite_f(float x) { return (__float_as_uint(x) & 0x7f800000u) != 0x7f800000u; }

// Order-preserving u32 of a non-NaN float, with -0 taken as +0 (the
// reference's comparisons do not tell them apart).
__device__ __forceinline__ uint32_t order_key(float x) {
  if (x == 0.0f) x = 0.0f;
  const uint32_t b = __float_as_uint(x);
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

__device__ __forceinline__ uint32_t wave_min_u32(uint32_t v) {
  #pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const uint32_t w = (uint32_t)__shfl_xor((int)v, o, 64);
    v = w < v ? w : v;
  }
  return v;
}
__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) {
  #pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const uint32_t hi = (uint32_t)__shfl_xor((int)(uint32_t)(v >> 32), o, 64);
    const uint32_t lo = (uint32_t)__shfl_xor((int)(uint32_t)v, o, 64);
    const uint64_t w = ((uint64_t)hi << 32) | lo;
    v = w > v ? w : v;
  }
  return v;
}
__device__ __forceinline__ float wave_max_gt(float v) {
  #pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const float w = __shfl_xor(v, o, 64);
    v = w > v ? w : v;
  }
  return v;
}

template <int PER>
__global__ void __launch_bounds__(64 * kRouterWaves)
    moe_router_kernel(const float* scores, uint32_t* out_ids, float* out_w, const float* bias, int rows, int E, int k,
                      int norm_topk, int gating_sigmoid, float weights_scale) {
  __shared__ float wsel[kRouterWaves][kRouterMaxExperts];
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int row = (int)blockIdx.x * kRouterWaves + wv;
  if (row >= rows) return;
  const float* rs = scores + (int64_t)row * E;
  uint32_t* ids = out_ids + (int64_t)row * k;
  float* ow = out_w + (int64_t)row * k;
  float* sel = wsel[wv];

  float key[PER], wt[PER];
  if (gating_sigmoid) {
    #pragma unroll
    for (int m = 0; m < PER; ++m) {
      const int e = m * 64 + lane;
      float sc = 0.f, ky = 0.f;
      if (e < E) {
        sc = 1.0f / (1.0f + exact_expf(-rs[e]));
        if (!finite_f(sc)) sc = 0.0f;
        ky = bias ? sc + bias[e] : sc;
      }
      key[m] = ky;
      wt[m] = sc;
    }
  } else {
    float x[PER];
    float mx = -__builtin_inff();
    #pragma unroll
    for (int m = 0; m < PER; ++m) {
      const int e = m * 64 + lane;
      x[m] = e < E ? rs[e] : -__builtin_inff();
      mx = x[m] > mx ? x[m] : mx;
    }
    mx = wave_max_gt(mx);
    bool fallback = !finite_f(mx);
    float denom = 0.0f;
    if (!fallback) {
      float t[PER];
      #pragma unroll
      for (int m = 0; m < PER; ++m) t[m] = m * 64 + lane < E ? exact_expf(x[m] - mx) : 0.0f;
      #pragma unroll
      for (int m = 0; m < PER; ++m) {
        const int n = min(64, E - m * 64);
        if (n > 0) {
          const float p = wave_fold_f32(t[m], denom, n);
          denom = __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(p), n - 1));
        }
      }
      fallback = !(denom > 0.0f) || !finite_f(denom);
      #pragma unroll
      for (int m = 0; m < PER; ++m) {
        float w = t[m] / denom;
        if (!finite_f(w)) w = 0.0f;
        key[m] = w;
        wt[m] = w;
      }
    }
    if (fallback) {
      const float w = (norm_topk && k > 1) ? 1.0f / (float)k : 1.0f / (float)E;
      for (int r = lane; r < k; r += 64) {
        ids[r] = (uint32_t)r;
        ow[r] = w;
      }
      return;
    }
  }

  // ranks: the reference's scan, as wave reductions
  float prev_key = __builtin_inff();
  int prev_id = -1;
  float sum = 0.0f;
  for (int r = 0; r < k; ++r) {
    uint32_t first = 0xffffffffu;
    uint64_t best = 0ull;
    #pragma unroll
    for (int m = 0; m < PER; ++m) {
      const int e = m * 64 + lane;
      const float ky = key[m];
      const bool ok = e < E && (prev_id < 0 || ky < prev_key || (ky == prev_key && e > prev_id));
      if (ok && (uint32_t)e < first) first = (uint32_t)e;
      if (ok && ky == ky) {
        const uint64_t c = ((uint64_t)order_key(ky) << 32) | (uint64_t)(0xffffffffu - (uint32_t)e);
        best = c > best ? c : best;
      }
    }
    first = wave_min_u32(first);
    int bid;
    float bkey, bw;
    if (first == 0xffffffffu) {
      bid = r < E ? r : E - 1;
      bkey = gating_sigmoid ? -__builtin_inff() : 0.0f;
      bw = 0.0f;
    } else {
      // the first eligible expert's key and weight
      const int fl = (int)(first & 63u), fm = (int)(first >> 6);
      float fk = 0.f, fw = 0.f;
      #pragma unroll
      for (int m = 0; m < PER; ++m)
        if (m == fm) { fk = key[m]; fw = wt[m]; }
      fk = __shfl(fk, fl, 64);
      fw = __shfl(fw, fl, 64);
      if (fk != fk) {
        bid = (int)first;
        bkey = fk;
        bw = fw;
      } else {
        best = wave_max_u64(best);
        bid = (int)(0xffffffffu - (uint32_t)best);
        const int bl = bid & 63, bm = bid >> 6;
        float k2 = 0.f, w2 = 0.f;
        #pragma unroll
        for (int m = 0; m < PER; ++m)
          if (m == bm) { k2 = key[m]; w2 = wt[m]; }
        bkey = __shfl(k2, bl, 64);
        bw = __shfl(w2, bl, 64);
      }
    }
    if (lane == 0) {
      ids[r] = (uint32_t)bid;
      sel[r] = bw;
    }
    sum += bw;
    prev_id = bid;
    prev_key = bkey;
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
  const bool norm = norm_topk && k > 1 && sum > 1.0e-7f && finite_f(sum);
  for (int r = lane; r < k; r += 64) {
    float w = sel[r];
    if (norm) w = w / sum;
    if (weights_scale != 1.0f) w = w * weights_scale;
    ow[r] = w;
  }
}

template <int PER>
void launch_router(const float* s, uint32_t* ids, float* w, const float* bias, int rows, int E, int k, int norm,
                   int sig, float scale, hipStream_t st) {
  const int blocks = (rows + kRouterWaves - 1) / kRouterWaves;
  hipLaunchKernelGGL(moe_router_kernel<PER>, dim3(blocks), dim3(64 * kRouterWaves), 0, st, s, ids, w, bias, rows, E, k,
                     norm, sig, scale);
}

}  // namespace
}  // namespace hi_rocm

extern "C" int hi_rocm_launch_moe_topk_router(const void* scores, void* output_ids, void* output_weights,
                                              const void* selection_bias, int rows, int experts, int top_k,
                                              int norm_topk, int gating_sigmoid, float weights_scale,
                                              void* stream) {
  // kernels.cu:8482-8495: status 1 for these
  if (scores == nullptr || output_ids == nullptr || output_weights == nullptr || rows <= 0 || experts <= 0 ||
      top_k <= 0 || top_k > experts || stream == nullptr)
    return hi_rocm::api_fail(HI_ROCM_ERR_ARGS, "hi_rocm_launch_moe_topk_router: invalid arguments");
  if (experts > hi_rocm::kRouterMaxExperts)
    return hi_rocm::api_fail(HI_ROCM_ERR_UNSUPPORTED, "hi_rocm_launch_moe_topk_router: more than 2048 experts");
  const float* s = (const float*)scores;
  uint32_t* ids = (uint32_t*)output_ids;
  float* w = (float*)output_weights;
  const float* b = (const float*)selection_bias;
  hipStream_t st = (hipStream_t)stream;
  const int per = (experts + 63) / 64;
  if (per <= 1) hi_rocm::launch_router<1>(s, ids, w, b, rows, experts, top_k, norm_topk, gating_sigmoid, weights_scale, st);
  else if (per <= 2) hi_rocm::launch_router<2>(s, ids, w, b, rows, experts, top_k, norm_topk, gating_sigmoid, weights_scale, st);
  else if (per <= 4) hi_rocm::launch_router<4>(s, ids, w, b, rows, experts, top_k, norm_topk, gating_sigmoid, weights_scale, st);
  else if (per <= 8) hi_rocm::launch_router<8>(s, ids, w, b, rows, experts, top_k, norm_topk, gating_sigmoid, weights_scale, st);
  else if (per <= 16) hi_rocm::launch_router<16>(s, ids, w, b, rows, experts, top_k, norm_topk, gating_sigmoid, weights_scale, st);
  else hi_rocm::launch_router<32>(s, ids, w, b, rows, experts, top_k, norm_topk, gating_sigmoid, weights_scale, st);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? HI_ROCM_OK : hi_rocm::api_hip_fail(e, "moe router launch");
}
