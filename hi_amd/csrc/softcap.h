// Final logit softcap, cap * tanh(x / cap) (crates/hi-cuda/src/gpu.rs:
// 23232-23249 apply_final_logit_softcap, after the LM-head projection and
// bias of gpu.rs:20999-21009).
//
// The reference evaluates tanh with CUDA's tanhf, whose results are not
// reproduced here.  This tanh is defined from operations that round the
// same way on the host and on the device (IEEE double +, -, *, / and the
// glibc-exact expf of exact_expf.h), so a host restatement gets the same
// bits: for |y| < 0.55 the Taylor series to y^21 in double (the first
// omitted term is below 7e-11 of the result), above it 1 - 2 / (e + 1)
// with e = expf(2|y|) widened to double; the result is rounded to f32 once,
// then multiplied by cap in f32, in the reference's order (x / cap, tanh,
// times cap).
#pragma once
#include <stdint.h>

#include "exact_expf.h"

namespace hi_rocm {

HI_ROCM_HD inline float softcap_tanh_f32(float y) {
  if (!(y == y)) return y;  // NaN
  const double ay = y < 0.f ? -(double)y : (double)y;
  double t;
  if (ay < 0.55) {
    const double z = ay * ay;
    double p = 18888466084.0 / 194896477400625.0;
    p = p * z + (-443861162.0 / 1856156927625.0);
    p = p * z + (6404582.0 / 10854718875.0);
    p = p * z + (-929569.0 / 638512875.0);
    p = p * z + (21844.0 / 6081075.0);
    p = p * z + (-1382.0 / 155925.0);
    p = p * z + (62.0 / 2835.0);
    p = p * z + (-17.0 / 315.0);
    p = p * z + (2.0 / 15.0);
    p = p * z + (-1.0 / 3.0);
    t = ay + ay * (p * z);
  } else if (ay < 44.0) {
    const double e = (double)exact_expf((float)(2.0 * ay));
    t = 1.0 - 2.0 / (e + 1.0);
  } else {
    t = 1.0;
  }
  const float tf = (float)t;
  return y < 0.f ? -tf : tf;
}

// cap * tanh(x / cap) for cap > 0 (the caller skips the softcap otherwise).
HI_ROCM_HD inline float softcap_f32(float x, float cap) {
  const float y = x / cap;
  return softcap_tanh_f32(y) * cap;
}

}  // namespace hi_rocm
