// hi-rocm: the argmax launchers' kernel and the numerics/debug kernels
// (processed distribution, expf, fold engine), with their launchers.
#include "sampler_common.h"

namespace hi_rocm {

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

// The workgroup fold of runs (fold_wg.h) on its own: out_start[r] gets the
// sequential f32 fold value before run r, *out_final the value after the
// last run.  Terms and counts are read from global memory.
__global__ void __launch_bounds__(NT) debug_fold_kernel(const float* x, const uint32_t* m, int R, float a0,
                                                        float* out_start, float* out_final) {
  extern __shared__ __align__(16) unsigned char lds_raw[];
  auto& L = *reinterpret_cast<fold::WgLds<NT>*>(lds_raw);
  uint8_t* pe = lds_raw + sizeof(fold::WgLds<NT>);
  const float fin = fold::fold_runs<NT>(
      L, pe, R, a0, [&](int r) { return x[r]; }, [&](int r) { return m[r]; },
      [&](int r, float v) { out_start[r] = v; });
  if (threadIdx.x == 0) *out_final = fin;
}

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
    // the form the row kernel uses (the branch-free one without a
    // repetition penalty), so that the check covers both
    if (pen) l = cfg.rep_on ? apply_penalties(l, cnt[e - c0], cfg) : apply_penalties_norep(l, cnt[e - c0], cfg);
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


hipError_t launch_argmax(const float* logits, uint32_t* out, int B, int64_t row_stride,
                         int64_t row_offset, int cols, hipStream_t stream) {
  const int vec_ok = (((uintptr_t)(logits + row_offset) & 15u) == 0) && (row_stride % 4 == 0);
  hipLaunchKernelGGL(argmax_rows_kernel, dim3(B), dim3(1024), 0, stream, logits, out, B, row_stride,
                     row_offset, cols, vec_ok);
  return hipGetLastError();
}

size_t debug_fold_lds(int R) { return sizeof(fold::WgLds<NT>) + (size_t)R + 1; }

hipError_t launch_debug_fold(const float* x, const uint32_t* m, int R, float a0, float* out_start,
                             float* out_final, hipStream_t stream) {
  const size_t lds = debug_fold_lds(R);
  hipError_t e = ensure_lds((const void*)debug_fold_kernel, lds);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(debug_fold_kernel, dim3(1), dim3(NT), lds, stream, x, m, R, a0, out_start, out_final);
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
