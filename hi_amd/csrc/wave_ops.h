// Wave-level helpers shared by the sampler and the MoE router kernels.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace hi_rocm {

// DPP controls (gfx9 encodings)
constexpr int kDppXor1 = 0xB1;         // quad_perm [1,0,3,2]
constexpr int kDppXor2 = 0x4E;         // quad_perm [2,3,0,1]
constexpr int kDppHalfMirror = 0x141;  // row_half_mirror
constexpr int kDppMirror = 0x140;      // row_mirror
constexpr int kDppShr1 = 0x111;        // row_shr:1 (+1, +3, +7 for :2, :4, :8)
constexpr int kDppBcast15 = 0x142;     // row_bcast:15
constexpr int kDppBcast31 = 0x143;     // row_bcast:31

// v moved by CTRL; lanes of rows outside ROW_MASK (or with no source lane
// when BC) get `old`.
template <int CTRL, int ROW_MASK = 0xf, bool BC = false>
__device__ __forceinline__ uint32_t dpp32(uint32_t old, uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp((int)old, (int)v, CTRL, ROW_MASK, 0xf, BC);
}

// Sequential f32 sums over the wave's lanes: lane l < n returns
// ((start + v_0) + v_1) + ... + v_l, the reference's left-to-right fold
// (gpu.rs:834-836, 851, 878, 889-896); lanes from n on hold partial sums.
// Lane 0 holds start + v_0 from the outset; each step adds v to the running
// sums moved one lane up (wave_shr:1 filling lane 0 with zero, which the
// compiler fuses into the add).  After step s lanes [0, s] hold their
// final sums and later steps leave them unchanged, so steps run in groups
// of 32 (n - 1 steps are needed): a taken branch per group costs about as
// much as five steps, so short groups cost more than the few extra steps.
// No lane's sum is -0 (the terms and `start` are not negative), so
// 0 + x == x at lane 0.
__device__ __forceinline__ float wave_fold_u(float u) {
  return __uint_as_float(dpp32<0x138, 0xf, true>(0u, __float_as_uint(u)));
}
__device__ __forceinline__ float wave_fold_f32(float v, float start, int n) {
  const float u = (threadIdx.x & 63u) == 0u ? start + v : v;
  float p = u;
  #pragma unroll 1
  for (int s = 1; s < n; s += 32) {
    #pragma unroll
    for (int i = 0; i < 32; ++i) p = wave_fold_u(p) + u;
  }
  return p;
}

// Inclusive prefix sum over the wave in lane order.
__device__ __forceinline__ uint32_t wave_incl_scan_u32(uint32_t v) {
  v += dpp32<kDppShr1, 0xf, true>(0u, v);
  v += dpp32<kDppShr1 + 1, 0xf, true>(0u, v);
  v += dpp32<kDppShr1 + 3, 0xf, true>(0u, v);
  v += dpp32<kDppShr1 + 7, 0xf, true>(0u, v);
  v += dpp32<kDppBcast15, 0xa>(0u, v);
  v += dpp32<kDppBcast31, 0xc>(0u, v);
  return v;
}

}  // namespace hi_rocm
