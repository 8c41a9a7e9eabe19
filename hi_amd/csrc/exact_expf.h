// Device single-precision exp that is bit-identical to the host glibc expf.
//
// The reference ranks tokens by f32 weights w = expf(s - max) computed with
// Rust's f32::exp (crates/hi-cuda/src/gpu.rs:786), which on Linux is glibc's
// expf.  glibc >= 2.27 implements expf with the method of ARM's
// optimized-routines (Szabolcs Nagy, 2017): reduce x*32/ln2 to k + r with a
// round-to-nearest shift, look up 2^(k/32) in a 32-entry table, evaluate a
// cubic for 2^(r/32) in double and round once to float.  On x86-64 glibc
// selects an FMA build of that code; it forms r with a fused multiply-add,
// and this port does the same (the choice changes 2 of the 2^32 results).
//
// The table below is 2^(i/32) rounded to double, minus i << 47 (so the
// exponent of 2^(k/32) can be added with one integer add).  The cubic's
// coefficients are the published ones, pre-divided by 32^3, 32^2 and 32.
// Every double operation here is correctly rounded on CDNA and on the host
// (add, mul, fma and the final conversion round to nearest even), so the
// device result equals the host result for every input.  The header builds
// for the host too (plain C++), which lets the CPU tests compare it with
// glibc on all 2^32 inputs; the GPU tests compare the device build with glibc
// on [-104, 0].
#pragma once
#include <stdint.h>
#include <string.h>

#if defined(__HIPCC__)
#include <hip/hip_runtime.h>
#define HI_ROCM_HD __host__ __device__
#else
#define HI_ROCM_HD
#endif

namespace hi_rocm {

#define HI_ROCM_EXP2_TAB32                                                                  \
  {0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full, 0x3fef9301d0125b51ull, \
   0x3fef72b83c7d517bull, 0x3fef54873168b9aaull, 0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull, \
   0x3fef06fe0a31b715ull, 0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull, \
   0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull, 0x3feea47eb03a5585ull, \
   0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull, 0x3feea11473eb0187ull, 0x3feea589994cce13ull, \
   0x3feeace5422aa0dbull, 0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull, \
   0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull, 0x3fef3720dcef9069ull, \
   0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full, 0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull}

#if defined(__HIPCC__)
__device__ __constant__ static const uint64_t kExp2Tab32Dev[32] = HI_ROCM_EXP2_TAB32;
#endif
static const uint64_t kExp2Tab32Host[32] = HI_ROCM_EXP2_TAB32;

HI_ROCM_HD inline uint64_t exp2_tab32(uint32_t i) {
#if defined(__HIP_DEVICE_COMPILE__)
  return kExp2Tab32Dev[i];
#else
  return kExp2Tab32Host[i];
#endif
}

HI_ROCM_HD inline double hr_fma(double a, double b, double c) { return __builtin_fma(a, b, c); }

// The table read through the constant copy (see exp2_tab32); kernels that
// keep a copy in LDS pass their own reader to exact_expf_t.
struct Exp2TabConst {
  HI_ROCM_HD uint64_t operator()(uint32_t i) const { return exp2_tab32(i); }
};

template <typename Tab>
HI_ROCM_HD inline float exact_expf_t(float x, const Tab& tab) {
  const double kInvLn2N = 0x1.71547652b82fep+0 * 32.0;
  const double kShift = 0x1.8p+52;
  const double kC0 = 0x1.c6af84b912394p-5 / (32.0 * 32.0 * 32.0);
  const double kC1 = 0x1.ebfce50fac4f3p-3 / (32.0 * 32.0);
  const double kC2 = 0x1.62e42ff0c52d6p-1 / 32.0;
  uint32_t ux;
  memcpy(&ux, &x, 4);
  const uint32_t abstop = (ux >> 20) & 0x7ffu;
  if (abstop >= 0x42bu) {  // |x| >= 88 or x is NaN
    if (ux == 0xff800000u) return 0.0f;
    if (abstop >= 0x7f8u) return x + x;
    if (x > 0x1.62e42ep6f) return __builtin_inff();
    if (x < -0x1.9fe368p6f) return 0.0f;
  }
  const double xd = (double)x;
  double kd = hr_fma(kInvLn2N, xd, kShift);
  uint64_t ki;
  memcpy(&ki, &kd, 8);
  kd -= kShift;
  const double r = hr_fma(kInvLn2N, xd, -kd);
  uint64_t t = tab((uint32_t)(ki & 31u));
  t += ki << 47;
  double s;
  memcpy(&s, &t, 8);
  const double z = hr_fma(kC0, r, kC1);
  const double r2 = r * r;
  double y = hr_fma(kC2, r, 1.0);
  y = hr_fma(z, r2, y);
  y = y * s;
  return (float)y;
}

HI_ROCM_HD inline float exact_expf(float x) { return exact_expf_t(x, Exp2TabConst{}); }

}  // namespace hi_rocm
