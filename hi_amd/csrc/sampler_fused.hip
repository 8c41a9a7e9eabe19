// hi-rocm: the streaming select pass and the finish of each row in one launch
// (select_finish_kernel: the last workgroup of a row finishes it), for
// small batches, and its launcher.
#include "sampler_wide.h"

namespace hi_rocm {

// The streaming select pass and the finish in one launch, for small
// batches: the last workgroup of a row to finish its chunk (a device-scope
// counter per row) runs the row's finish.  The other workgroups' records
// and candidates are released by their fence before the counter update and
// acquired by the last one's fence after it (one thread fences for the
// workgroup, between barriers); the last one also sets the counter back to
// zero for the next launch.  No workgroup waits for another.
template <int DT, int NL, bool MASK>
__global__ void __launch_bounds__(NT) select_finish_kernel(SampleArgs a, uint32_t flag_off) {
  extern __shared__ __align__(16) unsigned char lds_raw[];
  const int row = blockIdx.y;
  select_chunk<DT, NL, MASK>(a, row, blockIdx.x, lds_raw);
  uint32_t* last = reinterpret_cast<uint32_t*>(lds_raw + flag_off);  // past both LDS layouts
  // every wave waits for its stores to reach L2 (a workgroup barrier alone
  // does not), then one device-scope fence writes them back before the
  // counter update
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  uint32_t* counter = a.done + row;
  if (threadIdx.x == 0) {
    __threadfence();
    *last = atomicAdd(counter, 1u) == (uint32_t)(a.n_chunks - 1) ? 1u : 0u;
    if (*last) {
      __threadfence();  // acquire: the caches hold no stale record or candidate
      *counter = 0u;
    }
  }
  __syncthreads();
  if (*last == 0u) return;
  FinLds& fs = *reinterpret_cast<FinLds*>(lds_raw);
  const RowCfg cfg = load_cfg(a.pv, row, a.V, a.n_lp, a.need_lse);
  if (finish_lean(fs, a, row, cfg)) return;
  __syncthreads();
  finish_row(fs, a, row, cfg);
}

bool fused_fits(const SampleArgs& a) {
  return a.done != nullptr && (long)a.B * a.n_chunks <= kFusedMaxWorkgroups;
}

template <int DT, int NL, bool MASK>
hipError_t launch_fused_t(const SampleArgs& a, hipStream_t stream) {
  constexpr int E = NL * (DT == HI_ROCM_DTYPE_BF16 ? 8 : 4);
  size_t sel = kSelHead + (a.hoff ? sel_hist_bytes(NT * E) : 0);
  size_t body = sel > sizeof(FinLds) ? sel : sizeof(FinLds);
  body = (body + 15) & ~(size_t)15;
  const size_t lds = body + 16;
  hipError_t e = ensure_lds((const void*)select_finish_kernel<DT, NL, MASK>, lds);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL((select_finish_kernel<DT, NL, MASK>), dim3(a.n_chunks, a.B), dim3(NT), lds, stream, a,
                     (uint32_t)body);
  return hipGetLastError();
}

template <int DT, bool MASK>
hipError_t launch_fused_d(const SampleArgs& a, hipStream_t stream) {
  constexpr int EPL = DT == HI_ROCM_DTYPE_BF16 ? 8 : 4;
  if (a.chunk == kSelChunkLarge) return launch_fused_t<DT, kSelChunkLarge / NT / EPL, MASK>(a, stream);
  return launch_fused_t<DT, kSelChunkSmall / NT / EPL, MASK>(a, stream);
}

hipError_t launch_fused(const SampleArgs& a, hipStream_t stream) {
  if (a.dtype == HI_ROCM_DTYPE_BF16)
    return a.mask ? launch_fused_d<HI_ROCM_DTYPE_BF16, true>(a, stream) : launch_fused_d<HI_ROCM_DTYPE_BF16, false>(a, stream);
  return a.mask ? launch_fused_d<HI_ROCM_DTYPE_F32, true>(a, stream) : launch_fused_d<HI_ROCM_DTYPE_F32, false>(a, stream);
}

}  // namespace hi_rocm
