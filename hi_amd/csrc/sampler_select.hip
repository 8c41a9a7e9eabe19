// hi-rocm: the streaming select pass over (chunk, row) workgroups
// (select_kernel) and its launcher.
#include "sampler_wide.h"

namespace hi_rocm {

// The streaming select pass: workgroup (chunk, row).  At most 128 VGPRs
// (four waves per SIMD): the 16384-logit chunks' kernels need ~160 and then
// run three workgroups per CU; held to 128 they spill ~150 bytes a lane and
// still take C4's select pass from 38.6 to 36.6 us (the 4096-logit ones
// need under 70 either way).
template <int DT, int NL, bool MASK>
__global__ void __launch_bounds__(NT, 4) select_kernel(SampleArgs a) {
  extern __shared__ __align__(16) unsigned char lds_raw[];
  const int row = blockIdx.y;
  select_chunk<DT, NL, MASK>(a, row, blockIdx.x, lds_raw);
}

template <int DT, int NL, bool MASK>
hipError_t launch_select_t(const SampleArgs& a, hipStream_t stream) {
  constexpr int E = NL * (DT == HI_ROCM_DTYPE_BF16 ? 8 : 4);
  const size_t lds = kSelHead + (a.hoff ? sel_hist_bytes(NT * E) : 0);
  hipLaunchKernelGGL((select_kernel<DT, NL, MASK>), dim3(a.n_chunks, a.B), dim3(NT), lds, stream, a);
  return hipGetLastError();
}

template <int DT, bool MASK>
hipError_t launch_select_d(const SampleArgs& a, hipStream_t stream) {
  constexpr int EPL = DT == HI_ROCM_DTYPE_BF16 ? 8 : 4;
  if (a.chunk == kSelChunkLarge) return launch_select_t<DT, kSelChunkLarge / NT / EPL, MASK>(a, stream);
  return launch_select_t<DT, kSelChunkSmall / NT / EPL, MASK>(a, stream);
}

hipError_t launch_select(const SampleArgs& a, hipStream_t stream) {
  if (a.dtype == HI_ROCM_DTYPE_BF16)
    return a.mask ? launch_select_d<HI_ROCM_DTYPE_BF16, true>(a, stream) : launch_select_d<HI_ROCM_DTYPE_BF16, false>(a, stream);
  return a.mask ? launch_select_d<HI_ROCM_DTYPE_F32, true>(a, stream) : launch_select_d<HI_ROCM_DTYPE_F32, false>(a, stream);
}

}  // namespace hi_rocm
