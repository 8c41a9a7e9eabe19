// Greedy speculative-decoding verification on the device (the acceptance
// of crates/hi-cuda/src/gpu.rs:10725-10762,
// speculative_greedy_next_tokens_paged_with_page_table, batched over
// requests; the rule of docs/deepseek-v4-spec-decode-plan.md:95-102).
//
// The reference copies the K + 1 verify rows of logits to the host, takes
// each row's argmax there (gpu.rs:6406-6435: best = 0, best_val = row[0],
// replaced by a later value only when strictly greater -- so a NaN at
// index 0 keeps index 0, other NaNs never win, ties keep the lower index),
// accepts draft[i] while it equals greedy[i], and emits
// greedy[0 ..= accepted] (the first mismatch's target token, or the bonus
// token after a fully accepted draft).  Here one workgroup takes each row's
// argmax in place and one thread per request then runs the acceptance, so
// only the emitted tokens and their count leave the device.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "hi_rocm.h"
#include "sampler_internal.h"

namespace hi_rocm {
namespace {

constexpr int kVerifyThreads = 1024;

// Order key of a non-NaN float with -0 taken as +0 (the reference's '>'
// does not tell them apart).
__device__ __forceinline__ uint32_t order_key0(float x) {
  if (x == 0.0f) x = 0.0f;
  const uint32_t b = __float_as_uint(x);
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

// greedy[r] for every verify row r: the row's first-maximum index by the
// host rule above.  One workgroup per row; keys (value, -index) reduce by
// max, so the result does not depend on the reduction order.
__global__ void __launch_bounds__(kVerifyThreads)
    verify_argmax_kernel(const float* logits, int64_t row_stride, int V, uint32_t* greedy) {
  __shared__ uint64_t red[kVerifyThreads / 64];
  const int r = blockIdx.x, tid = threadIdx.x;
  const float* x = logits + (int64_t)r * row_stride;
  uint64_t best = 0ull;
  for (int i = tid; i < V; i += kVerifyThreads) {
    const float v = x[i];
    if (v == v) {
      const uint64_t k = ((uint64_t)order_key0(v) << 32) | (uint64_t)(0xffffffffu - (uint32_t)i);
      best = k > best ? k : best;
    }
  }
  #pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const uint32_t hi = (uint32_t)__shfl_xor((int)(uint32_t)(best >> 32), o, 64);
    const uint32_t lo = (uint32_t)__shfl_xor((int)(uint32_t)best, o, 64);
    const uint64_t w = ((uint64_t)hi << 32) | lo;
    best = w > best ? w : best;
  }
  if ((tid & 63) == 0) red[tid >> 6] = best;
  __syncthreads();
  if (tid == 0) {
    best = 0ull;
    for (int w = 0; w < kVerifyThreads / 64; ++w) best = red[w] > best ? red[w] : best;
    const float x0 = x[0];
    // NaN at index 0, or no non-NaN value: index 0
    greedy[r] = (x0 != x0 || best == 0ull) ? 0u : 0xffffffffu - (uint32_t)best;
  }
}

// One thread per request: accepted prefix and the emitted tokens.
__global__ void verify_accept_kernel(const uint32_t* greedy, const uint32_t* draft, const int32_t* draft_len, int B,
                                     int K, uint32_t* out_tokens, int32_t* out_count) {
  const int b = (int)(blockIdx.x * blockDim.x + threadIdx.x);
  if (b >= B) return;
  const int k = draft_len ? min(max(draft_len[b], 0), K) : K;
  const uint32_t* g = greedy + (int64_t)b * (K + 1);
  const uint32_t* d = draft + (int64_t)b * K;
  int accepted = k;
  for (int i = 0; i < k; ++i) {
    if (d[i] != g[i]) {
      accepted = i;
      break;
    }
  }
  for (int i = 0; i <= accepted; ++i) out_tokens[(int64_t)b * (K + 1) + i] = g[i];
  out_count[b] = accepted + 1;
}

}  // namespace
}  // namespace hi_rocm

extern "C" int hi_rocm_spec_verify_greedy(const void* logits, int batch, int max_draft, int vocab,
                                          const void* draft_tokens, const void* draft_len, void* out_greedy,
                                          void* out_tokens, void* out_count, void* stream) {
  if (logits == nullptr || batch <= 0 || max_draft < 0 || vocab <= 0 || (max_draft > 0 && draft_tokens == nullptr) ||
      out_greedy == nullptr || out_tokens == nullptr || out_count == nullptr || stream == nullptr)
    return hi_rocm::api_fail(HI_ROCM_ERR_ARGS, "hi_rocm_spec_verify_greedy: invalid arguments");
  const int64_t rows = (int64_t)batch * (max_draft + 1);
  if (rows > INT32_MAX) return hi_rocm::api_fail(HI_ROCM_ERR_UNSUPPORTED, "hi_rocm_spec_verify_greedy: too many rows");
  hipStream_t st = (hipStream_t)stream;
  hipLaunchKernelGGL(hi_rocm::verify_argmax_kernel, dim3((unsigned)rows), dim3(hi_rocm::kVerifyThreads), 0, st,
                     (const float*)logits, (int64_t)vocab, vocab, (uint32_t*)out_greedy);
  hipLaunchKernelGGL(hi_rocm::verify_accept_kernel, dim3((unsigned)((batch + 255) / 256)), dim3(256), 0, st,
                     (const uint32_t*)out_greedy, (const uint32_t*)draft_tokens, (const int32_t*)draft_len, batch,
                     max_draft, (uint32_t*)out_tokens, (int32_t*)out_count);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? HI_ROCM_OK : hi_rocm::api_hip_fail(e, "spec verify launch");
}
