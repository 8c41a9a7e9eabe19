// hi-rocm: the general scan and the finish kernels of the chunked path
// (finish_kernel; finish_grid_kernel with the wide pass of top-p rows), and
// launch_sample, which picks the kernels of a call.
#include "sampler_wide.h"

#include <map>
#include <mutex>

namespace hi_rocm {

// LDS of the general scan kernel.
size_t generic_chunk_lds_bytes(int chunk, bool hist) {
  return ((sizeof(ScanLds) + 15) & ~(size_t)15) +
         (hist ? (size_t)chunk / 8 + 2 * kHashCap * sizeof(uint32_t) : 0);
}

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
  if (finish_lean(fs, a, row, cfg)) return;
  __syncthreads();
  finish_row(fs, a, row, cfg);
}

// the rest chunks 1 .. of each row in turn.  Top-p rows take the wide pass
// on every chunk; every other row is finished by its chunk-0 workgroup
// (finish_lean, else finish_row) and its other workgroups exit at once.
// Workgroups go to the XCDs and their shader engines round-robin by linear
// id, so the B finishing workgroups, being consecutive, spread over the
// whole chip (on a (chunks, rows) grid they would share a few engines).
__global__ void __launch_bounds__(NT) finish_grid_kernel(SampleArgs a) {
  extern __shared__ __align__(16) unsigned char lds_raw[];
  int row = (int)blockIdx.x, chunk = 0;
  if (row >= a.B) {
    const int rest = row - a.B, per = a.n_chunks - 1;
    row = rest / per;
    chunk = 1 + rest % per;
  }
  const RowCfg cfg = load_cfg(a.pv, row, a.V, a.n_lp, a.need_lse);
  if (cfg.cls != kTopP) {
    if (chunk != 0) return;
    FinLds& fs = *reinterpret_cast<FinLds*>(lds_raw);
    if (finish_lean(fs, a, row, cfg)) return;
    __syncthreads();
    finish_row(fs, a, row, cfg);
    return;
  }
  WideChunkLds& L = *reinterpret_cast<WideChunkLds*>(lds_raw);
  float pre[kWidePre];
  const WideRowStats st = wide_row_stats(L, a, row, chunk, cfg, pre);
  const bool valid = st.valid != 0u;
  const float M = st.M, w_lo = st.w_lo;
  if (valid) wide_chunk_work(L, lds_raw, a, row, chunk, cfg, M, w_lo, st.pred, st.mass, pre);
  // the last workgroup of the row finishes it (as select_finish_kernel)
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  uint32_t* counter = a.done + row;
  if (threadIdx.x == 0) {
    __threadfence();
    L.last = atomicAdd(counter, 1u) == (uint32_t)(a.n_chunks - 1) ? 1u : 0u;
    if (L.last) {
      __threadfence();
      *counter = 0u;
    }
  }
  __syncthreads();
  if (L.last == 0u) return;
  // every workgroup of the row has read the chunks' statistics: clear their
  // valid flags, so that a chunk the next call's pass does not write is seen
  for (int c = threadIdx.x; c < a.n_chunks; c += NT) a.wstat[(int64_t)row * a.n_chunks + c].valid = 0u;
  uint32_t token = 0xffffffffu;
  uint32_t path = kWideNoStats;
  if (valid) token = wide_finish(lds_raw, a, row, cfg, M, w_lo, path);
  if (threadIdx.x == 0) a.diag[row] = path;
  __syncthreads();
  FinLds& fs = *reinterpret_cast<FinLds*>(lds_raw);
  if (token == 0xffffffffu) {
    finish_row(fs, a, row, cfg);
    return;
  }
  if (threadIdx.x == 0) a.out_tokens[row] = token;
  if (a.n_lp > 0 || a.out_token_lp) finish_logprobs(fs, a, row, cfg, token, M, false, 0);
}

size_t finish_grid_lds(int chunk) {
  size_t b = sizeof(FinLds);
  b = b > wide_chunk_lds(chunk) ? b : wide_chunk_lds(chunk);
  b = b > wide_fin_lds(chunk) ? b : wide_fin_lds(chunk);
  return (b + 15) & ~(size_t)15;
}

// --------------------------------------------------------------------------
// launch wrappers (called from the host API)

bool select_mode(int n_lp, int vec_ok) { return n_lp <= kLeanK && vec_ok; }

int choose_chunk(int B, int V, int n_lp, int vec_ok, bool hist) {
  (void)hist;
  if (select_mode(n_lp, vec_ok)) {
    const long wg_large = (long)B * ((V + kSelChunkLarge - 1) / kSelChunkLarge);
    return wg_large >= 1024 ? kSelChunkLarge : kSelChunkSmall;
  }
  const long wg_large = (long)B * ((V + kChunk - 1) / kChunk);
  return wg_large >= 512 ? kChunk : kChunkSmall;
}

// Raises a kernel's dynamic LDS limit to at least `bytes` on the current
// device (once per device and size; the attribute is per device).
hipError_t ensure_lds(const void* fn, size_t bytes) {
  static std::mutex mu;
  static std::map<std::pair<const void*, int>, size_t> done;
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  std::lock_guard<std::mutex> lock(mu);
  size_t& have = done[{fn, dev}];
  if (have >= bytes) return hipSuccess;
  e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes);
  if (e == hipSuccess) have = bytes;
  return e;
}

hipError_t record(const LaunchEvents* le, int i, hipStream_t stream) {
  return le ? hipEventRecord(le->ev[i], stream) : hipSuccess;
}

hipError_t launch_chunked(const SampleArgs& a, hipStream_t stream, const LaunchEvents* le) {
  const bool hist = a.hoff != nullptr;
  dim3 grid(a.n_chunks, a.B);
  hipError_t e = record(le, 0, stream);
  if (e != hipSuccess) return e;
  if (a.chunk == kChunk)
    hipLaunchKernelGGL((scan_generic_kernel<kVecLarge, kTilesLarge>), grid, dim3(NT),
                       generic_chunk_lds_bytes(kChunk, hist), stream, a);
  else
    hipLaunchKernelGGL((scan_generic_kernel<kVecSmall, 1>), grid, dim3(NT),
                       generic_chunk_lds_bytes(kChunkSmall, hist), stream, a);
  e = hipGetLastError();
  if (e == hipSuccess) e = record(le, 1, stream);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(finish_kernel, dim3(a.B), dim3(NT), 0, stream, a);
  e = hipGetLastError();
  return e == hipSuccess ? record(le, 2, stream) : e;
}

hipError_t launch_sample(const SampleArgs& a, hipStream_t stream, const LaunchEvents* le) {
  if (!select_mode(a.n_lp, a.vec_ok) || (a.chunk != kSelChunkLarge && a.chunk != kSelChunkSmall))
    return launch_chunked(a, stream, le);
  hipError_t e = record(le, 0, stream);
  if (e != hipSuccess) return e;
  if (row_kernel_fits(a)) {
    e = launch_rows(a, stream);
    if (e == hipSuccess) e = record(le, 1, stream);
    return e == hipSuccess ? record(le, 2, stream) : e;
  }
  if (fused_fits(a)) {
    e = launch_fused(a, stream);
    if (e == hipSuccess) e = record(le, 1, stream);
    return e == hipSuccess ? record(le, 2, stream) : e;
  }
  e = launch_select(a, stream);
  if (e == hipSuccess) e = record(le, 1, stream);
  if (e != hipSuccess) return e;
  const int64_t n_wg = (int64_t)a.n_chunks * a.B;
  if (n_wg * NT >= ((int64_t)1 << 32)) return hipErrorInvalidConfiguration;  // 1-D grid of work-items
  const size_t lds = finish_grid_lds(a.chunk);
  e = ensure_lds((const void*)finish_grid_kernel, lds);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(finish_grid_kernel, dim3((unsigned)n_wg), dim3(NT), lds, stream, a);
  e = hipGetLastError();
  return e == hipSuccess ? record(le, 2, stream) : e;
}

}  // namespace hi_rocm
