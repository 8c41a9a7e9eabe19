// Workgroup form of the exact sequential f32 fold (exact_fold.h): runs of
// equal non-negative terms r = 0 .. R-1 (term x_r, count m_r >= 1), folded
// left to right from a start value, by NTH threads at once.
//
//  plan   Each thread takes a contiguous block of runs.  A prefix sum in
//         double predicts the fold value before every run, hence its binade
//         pe[r] (the predicted values only choose binades; they never enter
//         a result).  A run whose predicted binade differs from the next
//         run's is a boundary run.  Between boundary runs the binade is
//         constant, so the runs of such a segment compose into one parity
//         map (a segmented scan over the threads).
//  chain  One thread walks the segments in order from the exact start
//         value: a segment applies only if the value is in its predicted
//         binade and stays below the binade's top; a boundary run is added
//         in closed form (run_walk).  At most 254 segments.
//  emit   Every run's exact start value, from its segment's start and its
//         prefix map.
// A misprediction (a value next to a power of two) stops the chain at that
// segment; the fold resumes there with the exact value, after folding one
// run exactly, so every round makes progress.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "exact_fold.h"
#include "wave_ops.h"

namespace hi_rocm {
namespace fold {

// Lane moves of a map or a double by a DPP control (wave_ops.h): a lane
// with no source lane (or outside ROW_MASK) gets all-zero bits, which are
// the identity map, a zero count and +0.0.
template <int CTRL, int RM, bool BC>
__device__ __forceinline__ Map dpp_map(Map m) {
  return Map{dpp32<CTRL, RM, BC>(0u, m.t0), dpp32<CTRL, RM, BC>(0u, m.t1)};
}
template <int CTRL, int RM, bool BC>
__device__ __forceinline__ double dpp_f64(double v) {
  const uint64_t b = (uint64_t)__double_as_longlong(v);
  const uint64_t r = ((uint64_t)dpp32<CTRL, RM, BC>(0u, (uint32_t)(b >> 32)) << 32) | dpp32<CTRL, RM, BC>(0u, (uint32_t)b);
  return __longlong_as_double((long long)r);
}
// Inclusive scan in lane order (lane l: m_0, then m_1, ..., then m_l): four
// row shifts within the 16-lane rows, then the row broadcasts of lanes 15
// and 31; each step composes the lower lanes' part first.
__device__ __forceinline__ Map wave_map_scan(Map m) {
  m = compose(dpp_map<kDppShr1, 0xf, true>(m), m);
  m = compose(dpp_map<kDppShr1 + 1, 0xf, true>(m), m);
  m = compose(dpp_map<kDppShr1 + 3, 0xf, true>(m), m);
  m = compose(dpp_map<kDppShr1 + 7, 0xf, true>(m), m);
  m = compose(dpp_map<kDppBcast15, 0xa, false>(m), m);
  m = compose(dpp_map<kDppBcast31, 0xc, false>(m), m);
  return m;
}
// The value of the lane below (wave_shr:1; the identity at lane 0).
__device__ __forceinline__ Map wave_map_prev(Map m) { return dpp_map<0x138, 0xf, true>(m); }
// Inclusive prefix sum of doubles in lane order.
__device__ __forceinline__ double wave_scan_f64(double v) {
  v += dpp_f64<kDppShr1, 0xf, true>(v);
  v += dpp_f64<kDppShr1 + 1, 0xf, true>(v);
  v += dpp_f64<kDppShr1 + 3, 0xf, true>(v);
  v += dpp_f64<kDppShr1 + 7, 0xf, true>(v);
  v += dpp_f64<kDppBcast15, 0xa, false>(v);
  v += dpp_f64<kDppBcast31, 0xc, false>(v);
  return v;
}

constexpr int kWgSeg = 256;  // segments of one plan: a monotone prefix has <= 254 binades

template <int NTH>
struct WgLds {
  double dsum[NTH / 64];
  uint32_t wflag[NTH / 64];
  Map wmap[NTH / 64];
  uint32_t wcnt[NTH / 64];
  Map tcarry[NTH];          // map of the thread's segment before its first run
  uint32_t tk[NTH];         // segment ordinal at the thread's first run
  Map seg_map[kWgSeg];      // map of segment k (its runs before boundary run k)
  Map seg_alt[kWgSeg];      // the same terms in the binade below (fold_plan<.., true>)
  Map walt[NTH / 64];
  uint32_t seg_A[kWgSeg];   // A at segment k's start (chain)
  uint32_t seg_e[kWgSeg];   // binade of segment k
  uint32_t bnd_run[kWgSeg]; // run index of boundary run k
  float bnd_start[kWgSeg];  // fold value before boundary run k (chain)
  uint32_t nb;              // boundary runs of the plan
  uint32_t fail;            // first segment the chain could not apply (> nb: none)
  uint32_t resume;          // first run of that segment
  float acc;                // chain result
};

// A DPP control as a type (for the generic steps of a scan).
template <int C, int RM, bool BC>
struct DppStep {
  static constexpr int c = C, rm = RM;
  static constexpr bool bc = BC;
};

// Segmented combine: (f1, m1) then (f2, m2).
__device__ __forceinline__ void seg_combine(uint32_t f1, Map m1, uint32_t& f2, Map& m2) {
  if (!f2) m2 = compose(m1, m2);
  f2 |= f1;
}

// What m copies of x add to an f32 sum in binade e, as a double: the
// rounded increments (exact halves counted as half an ulp), or the exact
// amount when the run leaves the binade.
__device__ __forceinline__ double rounded_inc(float x, uint32_t m, int e) {
  const Map mp = run_map(classify(x, e), m);
  if (mp.t0 >= kTop) return (double)m * (double)x;
  const double ulp = __builtin_ldexp(1.0, e - 150);
  return 0.5 * ((double)mp.t0 + (double)mp.t1) * ulp;
}

template <int NTH>
__device__ __forceinline__ void block_of(int pos, int R, int& r0, int& r1) {
  const int n = R - pos;
  const int J = (n + NTH - 1) / NTH;
  r0 = pos + (int)threadIdx.x * J;
  if (r0 > R) r0 = R;
  r1 = r0 + J < R ? r0 + J : R;
}

// The map of a run in binade e, and (ALT) in the binade below.
template <bool ALT>
__device__ __forceinline__ void run_maps(float x, uint32_t m, int e, Map& mp, Map& ma) {
  mp = run_map(classify(x, e), m);
  if (ALT) ma = e > 1 ? run_map(classify(x, e - 1), m) : mp;
}

// Plan of runs [pos, R) from the predicted start value `base`.  pe has
// room for R + 1 entries.  With ALT, every segment also gets its map in the
// binade below its predicted one (seg_alt), for a start value that lags
// the prediction.  Ends with a barrier.
template <int NTH, typename TermF, typename MultF, bool ALT = false>
__device__ __forceinline__ void fold_plan(WgLds<NTH>& L, uint8_t* pe, int pos, int R, double base, TermF term, MultF mult) {
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  int r0, r1;
  block_of<NTH>(pos, R, r0, r1);
  // 1. predicted binades from a prefix sum in double
  double my = 0.0;
  for (int r = r0; r < r1; ++r) my += (double)mult(r) * (double)term(r);
  double inc = wave_scan_f64(my);
  if (lane == 63) L.dsum[wid] = inc;
  __syncthreads();
  double before = 0.0, all = 0.0;
  #pragma unroll
  for (int w = 0; w < NTH / 64; ++w) {
    if (w < wid) before += L.dsum[w];
    all += L.dsum[w];
  }
  double P = base + (before + (inc - my));
  for (int r = r0; r < r1; ++r) {
    pe[r] = (uint8_t)binade((float)P);
    P += (double)mult(r) * (double)term(r);
  }
  if (tid == NTH - 1) pe[R] = (uint8_t)binade((float)(base + all));
  __syncthreads();
  // 1b. refine with the increments the fold makes in those binades: terms
  //     below half an ulp add nothing to an f32 sum, so exact sums run ahead
  //     of it (a value just below a power of two can stay there while the
  //     exact sum passes it, which would mispredict every later boundary)
  my = 0.0;
  for (int r = r0; r < r1; ++r) my += rounded_inc(term(r), mult(r), pe[r]);
  inc = wave_scan_f64(my);
  __syncthreads();
  if (lane == 63) L.dsum[wid] = inc;
  __syncthreads();
  before = 0.0;
  all = 0.0;
  #pragma unroll
  for (int w = 0; w < NTH / 64; ++w) {
    if (w < wid) before += L.dsum[w];
    all += L.dsum[w];
  }
  P = base + (before + (inc - my));
  uint8_t eprev = 0;
  for (int r = r0; r < r1; ++r) {
    const double d = rounded_inc(term(r), mult(r), pe[r]);
    eprev = (uint8_t)binade((float)P);
    P += d;
    pe[r] = eprev;  // pe[r] is read above before it is rewritten
  }
  __syncthreads();
  if (tid == NTH - 1) pe[R] = (uint8_t)binade((float)(base + all));
  __syncthreads();
  // 2. per-thread summary: boundary runs, the map before the first one
  //    (head) and after the last one (tail)
  uint32_t nbt = 0u;
  Map head = map_identity(), tail = map_identity();
  Map head_a = map_identity(), tail_a = map_identity();
  for (int r = r0; r < r1; ++r) {
    const int e = pe[r];
    if (e != pe[r + 1]) {
      ++nbt;
      tail = map_identity();
      tail_a = map_identity();
    } else {
      Map mp, ma;
      run_maps<ALT>(term(r), mult(r), e, mp, ma);
      if (nbt) {
        tail = compose(tail, mp);
        if (ALT) tail_a = compose(tail_a, ma);
      } else {
        head = compose(head, mp);
        if (ALT) head_a = compose(head_a, ma);
      }
    }
  }
  // 3. segmented exclusive scan over threads: the map of the segment the
  //    thread starts in, up to its first run; and the boundary ordinal
  uint32_t f = nbt ? 1u : 0u;
  Map m = nbt ? tail : head;
  Map ma = nbt ? tail_a : head_a;
  uint32_t cnt = nbt;
  // (DPP steps: a lane with no lane below combines with zero flags, the
  // identity map and a zero count, which changes nothing)
  auto step = [&](auto ctl) {
    constexpr int C = decltype(ctl)::c, RM = decltype(ctl)::rm;
    constexpr bool BC = decltype(ctl)::bc;
    const uint32_t of = dpp32<C, RM, BC>(0u, f);
    const Map om = dpp_map<C, RM, BC>(m);
    const uint32_t oc = dpp32<C, RM, BC>(0u, cnt);
    if (ALT) {
      const Map oa = dpp_map<C, RM, BC>(ma);
      if (!f) ma = compose(oa, ma);
    }
    seg_combine(of, om, f, m);
    cnt += oc;
  };
  step(DppStep<kDppShr1, 0xf, true>{});
  step(DppStep<kDppShr1 + 1, 0xf, true>{});
  step(DppStep<kDppShr1 + 3, 0xf, true>{});
  step(DppStep<kDppShr1 + 7, 0xf, true>{});
  step(DppStep<kDppBcast15, 0xa, false>{});
  step(DppStep<kDppBcast31, 0xc, false>{});
  if (lane == 63) {
    L.wflag[wid] = f;
    L.wmap[wid] = m;
    if (ALT) L.walt[wid] = ma;
    L.wcnt[wid] = cnt;
  }
  // exclusive: the inclusive value of the lane below (zero at lane 0)
  uint32_t ef = dpp32<0x138, 0xf, true>(0u, f);
  Map em = wave_map_prev(m);
  Map ea = map_identity();
  if (ALT) ea = wave_map_prev(ma);
  uint32_t ec = dpp32<0x138, 0xf, true>(0u, cnt);
  __syncthreads();
  uint32_t cf = 0u, cc = 0u, tot = 0u;
  Map cm = map_identity(), ca = map_identity();
  #pragma unroll
  for (int w = 0; w < NTH / 64; ++w) {
    if (w < wid) {
      uint32_t ff = L.wflag[w];
      Map mm = L.wmap[w];
      if (ALT) ca = ff ? L.walt[w] : compose(ca, L.walt[w]);
      seg_combine(cf, cm, ff, mm);
      cf = ff;
      cm = mm;
      cc += L.wcnt[w];
    }
    tot += L.wcnt[w];
  }
  if (ALT && !ef) ea = compose(ca, ea);
  seg_combine(cf, cm, ef, em);  // previous waves, then the lanes below
  L.tcarry[tid] = em;
  L.tk[tid] = cc + ec;
  if (tid == 0) L.nb = tot;
  // 4. segment records, written by the thread holding each boundary run
  //    (and the thread holding the last run, for the last segment)
  {
    uint32_t k = cc + ec;
    Map cur = em, cura = ea;
    for (int r = r0; r < r1; ++r) {
      const int e = pe[r];
      if (e != pe[r + 1]) {
        L.seg_map[k] = cur;
        if (ALT) L.seg_alt[k] = cura;
        L.seg_e[k] = (uint32_t)e;
        L.bnd_run[k] = (uint32_t)r;
        ++k;
        cur = map_identity();
        cura = map_identity();
      } else {
        Map mp, mq;
        run_maps<ALT>(term(r), mult(r), e, mp, mq);
        cur = compose(cur, mp);
        if (ALT) cura = compose(cura, mq);
      }
    }
    if (r0 < r1 && r1 == R) {
      L.seg_map[k] = cur;
      if (ALT) L.seg_alt[k] = cura;
      L.seg_e[k] = pe[R];
    }
  }
  __syncthreads();
}

// The chain from the exact value `a` before run pos (thread 0).  Ends with
// a barrier; L.acc holds the value after the last applied part.
template <int NTH, typename TermF, typename MultF>
__device__ __forceinline__ void fold_chain(WgLds<NTH>& L, int pos, int R, float a, TermF term, MultF mult) {
  if (threadIdx.x == 0) {
    const uint32_t nb = L.nb;
    uint32_t fail = nb + 1u, resume = (uint32_t)R;
    for (uint32_t k = 0; k <= nb; ++k) {
      const int first = k == 0 ? pos : (int)L.bnd_run[k - 1] + 1;
      const int last = k < nb ? (int)L.bnd_run[k] - 1 : R - 1;
      if (first <= last) {
        const int e = (int)L.seg_e[k];
        const uint32_t A = to_A(a);
        const uint32_t t = apply(L.seg_map[k], A & 1u);
        if (binade(a) != e || (uint64_t)A + t >= kTop) {
          fail = k;
          resume = (uint32_t)first;
          break;
        }
        L.seg_A[k] = A;
        a = from_A(A + t, e);
      }
      if (k < nb) {
        const int b = (int)L.bnd_run[k];
        L.bnd_start[k] = a;
        a = run_walk(a, term(b), mult(b));
      }
    }
    L.fail = fail;
    L.resume = resume;
    L.acc = a;
  }
  __syncthreads();
}

// out(r, v): the exact fold value v before run r, for every run the chain
// applied.
template <int NTH, typename TermF, typename MultF, typename OutF>
__device__ __forceinline__ void fold_emit(WgLds<NTH>& L, const uint8_t* pe, int pos, int R, TermF term, MultF mult, OutF out) {
  int r0, r1;
  block_of<NTH>(pos, R, r0, r1);
  const uint32_t fail = L.fail;
  uint32_t k = L.tk[threadIdx.x];
  Map cur = L.tcarry[threadIdx.x];
  for (int r = r0; r < r1 && k < fail; ++r) {
    const int e = pe[r];
    if (e != pe[r + 1]) {
      out(r, L.bnd_start[k]);
      ++k;
      cur = map_identity();
    } else {
      const uint32_t A0 = L.seg_A[k];
      out(r, from_A(A0 + apply(cur, A0 & 1u), e));
      cur = compose(cur, run_map(classify(term(r), e), mult(r)));
    }
  }
}

// The fold of runs [0, R) from a0; out(r, v) receives the value before each
// run.  Returns the final value (uniform).  pe: LDS, R + 1 bytes.
template <int NTH, typename TermF, typename MultF, typename OutF>
__device__ __forceinline__ float fold_runs(WgLds<NTH>& L, uint8_t* pe, int R, float a0, TermF term, MultF mult, OutF out) {
  int pos = 0;
  float a = a0;
  while (pos < R) {
    fold_plan<NTH>(L, pe, pos, R, (double)a, term, mult);
    fold_chain<NTH>(L, pos, R, a, term, mult);
    fold_emit<NTH>(L, pe, pos, R, term, mult, out);
    const uint32_t fail = L.fail, nb = L.nb;
    const int resume = (int)L.resume;
    a = L.acc;
    __syncthreads();  // the next plan rewrites L and pe
    if (fail > nb) break;
    if (threadIdx.x == 0) out(resume, a);
    a = run_walk(a, term(resume), mult(resume));
    pos = resume + 1;
  }
  return a;
}

}  // namespace fold
}  // namespace hi_rocm
