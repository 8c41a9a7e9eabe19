// Exact emulation of a sequential f32 fold of non-negative terms,
//   acc = fl(acc + x_0); acc = fl(acc + x_1); ...   (round to nearest even),
// in integer arithmetic, so that the fold can be split across threads.
//
// The reference sums weights this way (crates/hi-cuda/src/gpu.rs:834-838:
// the top-p normaliser; :851: the cumulative probability; :878 and
// :889-896: the candidate total and the inverse CDF).  A left-to-right f32
// fold has no parallel form in floating point, but it has one in integers:
//
//  * While acc stays in one binade (one exponent field e, ulp = 2^(e-150);
//    the zero/subnormal range shares field 1's ulp 2^-149), acc = A * ulp
//    with an integer A < 2^24, and fl(acc + x) = (A + inc) * ulp where inc
//    is x / ulp rounded to nearest: n = floor(x / ulp) plus one when the
//    remainder is above half an ulp.  On an exact half the result rounds to
//    the even A + inc, so inc depends on the parity of A.  Each term is
//    therefore a map from the start parity p to an increment t(p), and maps
//    compose associatively: (f then g)(p) = f(p) + g((p + f(p)) mod 2).
//  * The emulation is exact while A + t < 2^24.  The first term whose result
//    reaches 2^24 leaves the binade: that one term is added as a real f32
//    add, and the fold continues in the new binade.  Binade crossings are
//    few (acc only grows), so almost all terms take the integer path.
//  * m equal terms (a run) have a closed form: their increments are
//    m * s (+0/+p/-p for exact halves), and the copy at which a run leaves
//    the binade, or reaches a threshold, is found by one division.
//
// Preconditions: terms finite and >= 0 (-0 counts as +0), every partial sum
// below 2^128.  The start value may be -0 (Rust's Sum folds from -0.0):
// -0 + x == x for x > 0, and the only difference (-0 + +0 = +0) is a zero
// sum that every caller treats like +0.
//
// The scalar pieces below are __host__ __device__ so that the host tests
// can check them against a literal sequential fold.
#pragma once
#include <stdint.h>
#include <string.h>

#if defined(__HIPCC__)
#define HRF_HD __host__ __device__ __forceinline__
#else
#define HRF_HD static inline
#endif

namespace hi_rocm {
namespace fold {

constexpr uint32_t kTop = 1u << 24;  // A reaching this: the sum left the binade
constexpr uint32_t kSat = 1u << 26;  // map values saturate here (any value >= kTop crosses)
constexpr uint32_t kNone = 0xffffffffu;

HRF_HD uint32_t fbits(float f) {
#if defined(__HIP_DEVICE_COMPILE__)
  return __float_as_uint(f);
#else
  uint32_t u;
  memcpy(&u, &f, 4);
  return u;
#endif
}
HRF_HD float bfloat(uint32_t u) {
#if defined(__HIP_DEVICE_COMPILE__)
  return __uint_as_float(u);
#else
  float f;
  memcpy(&f, &u, 4);
  return f;
#endif
}

// One IEEE f32 addition, round to nearest even (the library is compiled
// with -ffp-contract=off, so this is never fused with a neighbour).
HRF_HD float fadd(float a, float b) { return a + b; }

// Binade of acc >= 0: its exponent field, at least 1.
HRF_HD int binade(float a) {
  const int e = (int)((fbits(a) & 0x7fffffffu) >> 23);
  return e < 1 ? 1 : e;
}
// acc / ulp(binade(acc)), an integer below 2^24.
HRF_HD uint32_t to_A(float a) {
  const uint32_t b = fbits(a) & 0x7fffffffu;
  return (b >> 23) ? ((b & 0x7fffffu) | 0x800000u) : b;
}
// A * 2^(e-150) for A < 2^24 in binade e (A >= 2^23 unless e == 1).
HRF_HD float from_A(uint32_t A, int e) {
  if (A < 0x800000u) return bfloat(A);  // zero / subnormal (e == 1)
  return bfloat(((uint32_t)e << 23) | (A & 0x7fffffu));
}

HRF_HD uint32_t sat(uint64_t v) { return v > kSat ? kSat : (uint32_t)v; }

// x / ulp(e): n = floor, cls 0 = below half (or exact), 1 = exactly half,
// 2 = above half.
struct Inc {
  uint32_t n;
  uint32_t cls;
};
// Both cases are computed and one is selected (no branches): d <= 0 is an
// integer number of ulps (X < 2^24, so three shifts reach kSat and X << 3
// stays below 2^27); for d >= 1 the shift is clamped to 25, where X >> 25
// is 0 and the remainder X is below the half 2^24 (a term below a quarter
// ulp adds nothing).
HRF_HD Inc classify(float x, int e) {
  const uint32_t b = fbits(x) & 0x7fffffffu;
  const int ex = (int)(b >> 23);
  const uint32_t X = ex ? ((b & 0x7fffffu) | 0x800000u) : b;
  const int d = e - (ex ? ex : 1);
  const int sh = d >= 0 ? 0 : (-d > 3 ? 3 : -d);
  const uint32_t up = X << sh;
  const int ds = d < 1 ? 1 : (d > 25 ? 25 : d);
  const uint32_t rem = X & ((1u << ds) - 1u);
  const uint32_t half = 1u << (ds - 1);
  Inc r;
  r.n = d <= 0 ? (up > kSat ? kSat : up) : X >> ds;
  r.cls = d <= 0 ? 0u : (rem < half ? 0u : (rem == half ? 1u : 2u));
  return r;
}

// Per-copy increment of a run in its binade: copy c >= 1 of m equal terms
// ends at A + c * s + delta(p), delta = 0 (no exact half), +p (half, n
// even: the first copy rounds to even, the parity is then even) or -p
// (half, n odd: every copy rounds up from an even A).
HRF_HD uint32_t steady(Inc c) {
  return c.n + ((c.cls == 2u || (c.cls == 1u && (c.n & 1u))) ? 1u : 0u);
}
HRF_HD int64_t delta(Inc c, uint32_t p) {
  return c.cls == 1u ? ((c.n & 1u) ? -(int64_t)p : (int64_t)p) : 0;
}

// Map of a run: increments t0 / t1 for start parity 0 / 1.
struct Map {
  uint32_t t0, t1;
};
HRF_HD Map map_identity() { return Map{0u, 0u}; }
HRF_HD Map run_map(Inc c, uint32_t m) {
  if (m == 0u) return map_identity();
  const uint64_t base = (uint64_t)steady(c) * m;
  Map r;
  r.t0 = sat(base);
  r.t1 = c.cls == 1u ? ((c.n & 1u) ? sat(base - 1u) : sat(base + 1u)) : r.t0;
  return r;
}
// f, then g.  Map values are at most kSat + 2 (term maps add at most two
// to a saturated count, every composition saturates), so the sums stay
// below 2^28 in 32 bits.
HRF_HD Map compose(Map f, Map g) {
  Map h;
  const uint32_t a0 = f.t0 + ((f.t0 & 1u) ? g.t1 : g.t0);
  const uint32_t a1 = f.t1 + ((f.t1 & 1u) ? g.t0 : g.t1);
  h.t0 = a0 > kSat ? kSat : a0;
  h.t1 = a1 > kSat ? kSat : a1;
  return h;
}
HRF_HD uint32_t apply(Map f, uint32_t p) { return p ? f.t1 : f.t0; }

// First copy count cc >= 1 of the run (x in binade e from A) whose result
// reaches 2^24 (leaves the binade); kNone when no copy does.
HRF_HD uint32_t cross_copy(uint32_t A, Inc c) {
  const uint64_t s = steady(c);
  const int64_t need = (int64_t)kTop - (int64_t)A - delta(c, A & 1u);  // cc * s >= need
  if (need <= (int64_t)s) return 1u;
  if (s == 0u) return kNone;
  // need <= kTop + 1 and s <= kSat + 1: the quotient is taken in 32 bits
  return ((uint32_t)need + (uint32_t)s - 1u) / (uint32_t)s;
}
// A after c >= 0 copies, all inside the binade.
HRF_HD uint32_t after_copies(uint32_t A, Inc c, uint32_t cnt) {
  if (cnt == 0u) return A;
  return (uint32_t)((int64_t)A + (int64_t)steady(c) * cnt + delta(c, A & 1u));
}

// The sequential fold of m copies of x onto a, exactly.
HRF_HD float run_walk(float a, float x, uint32_t m) {
  while (m > 0u) {
    const int e = binade(a);
    const uint32_t A = to_A(a);
    const Inc c = classify(x, e);
    const uint32_t cc = cross_copy(A, c);
    if (cc > m) return from_A(after_copies(A, c, m), e);
    a = fadd(from_A(after_copies(A, c, cc - 1u), e), x);
    m -= cc;
  }
  return a;
}

// The first copy count c in [1, m] after which the fold of copies of x onto
// a is >= theta (STRICT: > theta); kNone when none is.  *before gets the
// sum before that copy.  theta must be finite.
template <bool STRICT>
HRF_HD uint32_t run_find(float a, float x, uint32_t m, float theta, float* before) {
  uint32_t done = 0u;
  while (m > 0u) {
    const int e = binade(a);
    const uint32_t A = to_A(a);
    const Inc c = classify(x, e);
    const uint32_t cc = cross_copy(A, c);
    // theta in ulps of this binade (exact in double)
    double tu = (double)theta;
    {
      int sh = 150 - e;  // multiply by 2^sh, in steps that stay exact
      while (sh > 60) { tu *= 1152921504606846976.0; sh -= 60; }
      while (sh < -60) { tu *= 8.673617379884035e-19; sh += 60; }
      tu *= (sh >= 0) ? (double)(1ull << sh) : 1.0 / (double)(1ull << -sh);
    }
    // smallest integer K with K >= tu (K > tu when STRICT)
    double kd = STRICT ? __builtin_floor(tu) + 1.0 : __builtin_ceil(tu);
    const uint32_t lim = cc > m ? m : cc - 1u;  // copies that stay in the binade
    if (lim > 0u) {
      const uint32_t p = A & 1u;
      const int64_t s = (int64_t)steady(c);
      const int64_t dl = delta(c, p);
      // first c0 >= 1 with A + c0 * s + dl >= K
      uint64_t c0;
      if (kd <= (double)((int64_t)A + s + dl)) {
        c0 = 1u;
      } else if (s == 0 || kd > 9.0e15) {
        c0 = kNone;
      } else {
        const int64_t need = (int64_t)kd - (int64_t)A - dl;
        c0 = (uint64_t)((need + s - 1) / s);
      }
      if (c0 <= lim) {
        if (before) *before = from_A(after_copies(A, c, (uint32_t)c0 - 1u), e);
        return done + (uint32_t)c0;
      }
    }
    if (cc > m) return kNone;
    const float prev = from_A(after_copies(A, c, cc - 1u), e);
    a = fadd(prev, x);
    if (STRICT ? (a > theta) : (a >= theta)) {
      if (before) *before = prev;
      return done + cc;
    }
    done += cc;
    m -= cc;
  }
  return kNone;
}

}  // namespace fold
}  // namespace hi_rocm
