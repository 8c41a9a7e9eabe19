// hi-rocm batched token sampler: device code shared by the kernel translation
// units (sampler_rows.hip, sampler_select.hip, sampler_fused.hip,
// sampler_chunked.hip, lm_head.hip, sampler_debug.hip).
//
// Logits [B, V] (f32 or bf16) stay in HBM and are read once, with 128-bit
// (f32) or 64-bit (bf16) loads.  launch_sample() picks one of four shapes:
//
//   row_kernel          B >= 192, V <= 2^18, no logprobs: one 1024-thread
//                       workgroup per row streams the row in 16384-logit
//                       tiles (two in flight), keeps per-wave candidate lists
//                       against a running bound, and finishes the row itself
//                       (one launch per step).  Rows the fast path cannot
//                       resolve take row_general, out of line.
//   select_finish       small grids (<= 512 workgroups): one workgroup per
//                       (row, chunk) of 4096 or 16384 logits selects the
//                       chunk's candidates; the last workgroup of a row
//                       (per-row counter) finishes it (one launch).
//   select + finish     larger grids: the same select kernel, then
//                       finish_grid_kernel on a 1-D grid whose first B
//                       workgroups finish the rows (spread over every XCD)
//                       and whose other workgroups run the wide pass of
//                       top-p rows.
//   scan + finish       more than 256 logprobs, or rows not aligned for
//                       vector loads: scan_generic_kernel, then
//                       finish_kernel, one workgroup per row.
//
// Per element: allowed-token mask, penalties from an LDS count table of the
// row's history, temperature.  Candidates are 64-bit keys (processed logit,
// index) so that one integer compare ranks them; selections are MSD radix
// descents over LDS histograms with DPP scans and ballots.
//
// Finishes: the lean finish (greedy; top-k <= 256) ranks by counting and
// runs the reference's sequential f32 folds on every wave from registers
// (wave_draw); top-k rows up to 1024 rank their candidates (register
// bitonic sort) and draw the same way; top-p rows without top-k take the
// wide pass: exact weights per chunk, the vocabulary-order normaliser as an
// exact parallel emulation of the f32 fold (exact_fold.h / fold_wg.h: per
// binade integer maps, one real add per binade crossing), the nucleus from
// a mass histogram as a superset of distinct weights, and the rank-order
// folds over those runs in closed form.  finish_row is the general
// fallback and reproduces the reference step by step.
//
// Every operation that decides a token mirrors the reference bit for bit
// (crates/hi-cuda/src/gpu.rs:753-900): IEEE f32 division and addition in
// the reference's order, no contraction (the library is built with
// -ffp-contract=off), and exact_expf() equal to host glibc expf.
// Selections use integer histograms and prefix scans in a fixed order, so
// results are deterministic run to run.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <float.h>
#include <stddef.h>

#include <type_traits>
#include <utility>

#include "hi_rocm.h"
#include "exact_expf.h"
#include "fold_wg.h"
#include "softcap.h"
#include "wave_ops.h"
#include "sampler_internal.h"

namespace hi_rocm {

constexpr int NT = kScanThreads;  // threads of the fused kernel
constexpr int kBuf = 1024;        // ranked entries held in LDS
constexpr int kGather = 4096;     // candidates of a row gathered into LDS
constexpr int kBufCap = 2048;     // running chunk candidates held in LDS
constexpr int kHashCap = 1024;    // distinct history tokens per chunk held in LDS
constexpr int kBins = 1024;       // weight histogram of the wide paths (w bits >> 20)

// --------------------------------------------------------------------------
// small helpers

__device__ __forceinline__ bool finitef_(float x) {
  return (__float_as_uint(x) & 0x7f800000u) != 0x7f800000u;
}

// Order-preserving unsigned key of a float (NaN never occurs here).
__device__ __forceinline__ uint32_t okey(float f) {
  const uint32_t u = __float_as_uint(f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ float okey_inv(uint32_t k) {
  const uint32_t u = (k & 0x80000000u) ? (k & 0x7fffffffu) : ~k;
  return __uint_as_float(u);
}

// Key of a processed logit: its order key, non-finite values as -inf
// (gpu.rs:767-777 maps them to -inf before ranking).
constexpr uint32_t kKeyNegInf = 0x007fffffu;  // okey(-inf)
__device__ __forceinline__ uint32_t lkey(float l) { return finitef_(l) ? okey(l) : kKeyNegInf; }

// Scaled logit s = l / t_eff of a key (gpu.rs:767-777); the key of -inf
// decodes to -inf and t_eff is positive, so no case needs a branch.
__device__ __forceinline__ float key_to_s(uint32_t key, float t_eff) {
  return okey_inv(key) / t_eff;
}

// Tie order of the finite-lane argmax (kernels.cu:7775-7801).  Thread t of
// 256 keeps the first maximum among indices t, t+256, ...; the tree then
// halves the stride from 128 to 1 and keeps the lower slot unless the upper
// one is strictly larger.  The slot compared last (bit 0 of t) weighs most,
// so among tied maxima the smallest 8-bit bit reversal of (idx mod 256)
// wins, then the smallest idx.  fin_order packs that order into one integer
// (smaller wins); fin_index inverts it.
__device__ __forceinline__ uint32_t fin_order(uint32_t idx) {
  return (__builtin_bitreverse32(idx) & 0xff000000u) | (idx >> 8);
}
__device__ __forceinline__ uint32_t fin_index(uint32_t ord) {
  return ((ord & 0x00ffffffu) << 8) | (__builtin_bitreverse32(ord) & 0xffu);
}

// Rust's f32::total_cmp as a signed key (gpu.rs:744).
__device__ __forceinline__ int32_t total_key(float f) {
  const int32_t i = (int32_t)__float_as_uint(f);
  return i ^ (int32_t)(((uint32_t)(i >> 31)) >> 1);
}

// Candidate key: scaled-logit key high, inverted index low, so a larger
// 64-bit value ranks first (value desc, index asc).
__device__ __forceinline__ uint64_t cand_key(uint32_t key, uint32_t idx) {
  return ((uint64_t)key << 32) | (uint64_t)(0xffffffffu - idx);
}
__device__ __forceinline__ uint32_t cand_idx(uint64_t c) { return 0xffffffffu - (uint32_t)c; }
__device__ __forceinline__ uint32_t cand_skey(uint64_t c) { return (uint32_t)(c >> 32); }

// Rank key of the reference order (weight desc by total_cmp, index asc);
// weights are >= +0, so their bits order like the floats.
__device__ __forceinline__ uint64_t rank_key(float w, uint32_t idx) {
  return ((uint64_t)__float_as_uint(w) << 32) | (uint64_t)(0xffffffffu - idx);
}
__device__ __forceinline__ float rank_w(uint64_t r) { return __uint_as_float((uint32_t)(r >> 32)); }

// Chunk-local composite (48 bits): key << 16 | (0xffff - local index).
__device__ __forceinline__ uint64_t local_comp(uint32_t key, uint32_t li) {
  return ((uint64_t)key << 16) | (uint64_t)(0xffffu - li);
}

__device__ __forceinline__ float bf16_to_f32(uint16_t h) { return __uint_as_float((uint32_t)h << 16); }

__device__ __forceinline__ float clamp_uniform(float u) {
  // gpu.rs:882-886
  return finitef_(u) ? (u < 0.f ? 0.f : (u > 0.99999994f ? 0.99999994f : u)) : 0.f;
}

__device__ __forceinline__ int next_pow2(int x) {
  int p = 1;
  while (p < x) p <<= 1;
  return p;
}

// ---- parameters ----------------------------------------------------------

// A value no kernel writes, read through the constant address space: at a
// workgroup-uniform address the compiler reads it with a scalar load, which
// does not wait behind the vector loads in flight.
template <typename T>
__device__ __forceinline__ T const_load(const T* p) {
  return *(const __attribute__((address_space(4))) T*)p;
}

__device__ __forceinline__ float row_uniform(const ParamsView& pv, int row) {
  return pv.uniforms ? const_load(pv.uniforms + row) : pv.uniform_value;
}

__device__ __forceinline__ RowCfg load_cfg(const ParamsView& pv, int row, int V, int n_lp, int need_lse) {
  RowCfg c;
  // The batch-wide values first; the per-row modes replace them.  (Every
  // field is defined before the mode branches: a three-way if/else-if here
  // has been compiled for gfx950 with top_k undefined on the uniform path.)
  c.T = pv.T; c.top_p = pv.top_p; c.top_k = pv.top_k;
  c.min_p = 0.f; c.rep = 1.f; c.freq = 0.f; c.pres = 0.f; c.eos = 0u; c.flags = 0u;
  const int mode = pv.mode;
  if (mode == kParamsSoA) {
    c.T = const_load(pv.temps + row); c.top_p = const_load(pv.top_ps + row); c.top_k = const_load(pv.top_ks + row);
  }
  if (mode == kParamsRows) {
    const hi_rocm_row_params* p = pv.rows + row;
    c.T = const_load(&p->temperature); c.top_p = const_load(&p->top_p); c.min_p = const_load(&p->min_p);
    c.rep = const_load(&p->repetition_penalty); c.freq = const_load(&p->frequency_penalty);
    c.pres = const_load(&p->presence_penalty); c.top_k = const_load(&p->top_k); c.eos = const_load(&p->eos_id);
    c.flags = const_load(&p->flags);
  }
  const bool greedy = !(finitef_(c.T) && c.T > 0.f);
  const bool minp_on = finitef_(c.min_p) && c.min_p > 0.f;
  // gpu.rs:731-738, extended with min_p.
  const bool ranked = !greedy && ((finitef_(c.top_p) && c.top_p < 1.f) || c.top_k > 0 || minp_on);
  c.cls = greedy ? kGreedy : (ranked ? (c.top_k > 0 ? kTopK : kTopP) : kTempOnly);
  c.k_eff = c.cls == kTopK ? min(c.top_k, V) : 0;
  c.t_eff = greedy ? 1.f : c.T;
  c.cutoff = finitef_(c.top_p) ? (c.top_p < 0.f ? 0.f : (c.top_p > 1.f ? 1.f : c.top_p)) : 1.f;
  c.min_p = minp_on ? fminf(c.min_p, 1.f) : 0.f;
  c.rep_on = finitef_(c.rep) && c.rep > 0.f && fabsf(c.rep - 1.f) > FLT_EPSILON;
  c.freq = finitef_(c.freq) ? c.freq : 0.f;
  c.pres = finitef_(c.pres) ? c.pres : 0.f;
  c.wide = c.cls == kTopK && c.k_eff > kLeanK;
  // top-k rows keep their top k as candidates in the streaming pass; beyond
  // what the ranked finish holds (kBuf) they keep their scaled logits
  const bool ranked_k = c.cls == kTopK && c.k_eff <= kBuf;
  c.k_sel = ranked_k ? max(c.k_eff, n_lp) : n_lp;
  // Logprobs need the normaliser to ~1e-7 relative: its largest terms are
  // summed in double from the candidates, so every chunk keeps a few.
  if (need_lse) c.k_sel = max(c.k_sel, kLseTop);
  if (c.k_sel > V) c.k_sel = V;
  c.store_s = c.cls == kTopP || c.cls == kTempOnly || (c.wide && !ranked_k);
  // Every caller's row is uniform over the workgroup: the float fields are
  // kept in scalar registers (as vector values they would hold vector
  // registers for the whole kernel, or be spilled to scratch memory)
  auto su = [](float v) { return __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(v))); };
  c.T = su(c.T); c.top_p = su(c.top_p); c.min_p = su(c.min_p); c.rep = su(c.rep);
  c.freq = su(c.freq); c.pres = su(c.pres); c.t_eff = su(c.t_eff); c.cutoff = su(c.cutoff);
  c.u = su(row_uniform(pv, row));  // loaded with the parameters, long before the draw
  return c;
}


// Stages 2 and 3 of the processed logit (the mask is applied by the caller):
// repetition penalty per occurrence (crates/hi-mlx/src/generate.rs:60-70),
// then frequency and presence penalties as separate f32 roundings.
__device__ __forceinline__ float apply_penalties(float l, uint32_t cnt, const RowCfg& c) {
  if (cnt == 0u) return l;
  if (c.rep_on) {
    const uint32_t reps = (c.flags & HI_ROCM_FLAG_REP_ONCE) ? 1u : cnt;
    for (uint32_t r = 0; r < reps; ++r) l = l < 0.f ? l * c.rep : l / c.rep;
  }
  const float fc = c.freq * (float)cnt;
  l = l - fc;
  l = l - c.pres;
  return l;
}

// apply_penalties for rows without a repetition penalty, with no branch.
__device__ __forceinline__ float apply_penalties_norep(float l, uint32_t cnt, const RowCfg& c) {
  const float p = (l - c.freq * (float)cnt) - c.pres;
  return cnt == 0u ? l : p;
}

// ---- wave-wide reductions and scans on DPP lane moves ---------------------
//
// A reduction combines each lane with its quad neighbours (quad_perm), then
// the mirrored lanes of its half row and row (row_half_mirror, row_mirror),
// so that every lane of a 16-lane row holds the row's result; row_bcast:15
// and row_bcast:31 then fold the rows into lane 63, which readlane hands to
// every lane.  The scan is the Hillis-Steele sequence row_shr:1,2,4,8
// followed by the same two row broadcasts.  Each step is one VALU
// instruction with no LDS round trip.

// Reduction of a 32-bit value under a commutative, associative op with
// identity `id`.
template <typename Op>
__device__ __forceinline__ uint32_t wave_reduce32(uint32_t v, uint32_t id, Op op) {
  v = op(v, dpp32<kDppXor1>(id, v));
  v = op(v, dpp32<kDppXor2>(id, v));
  v = op(v, dpp32<kDppHalfMirror>(id, v));
  v = op(v, dpp32<kDppMirror>(id, v));
  v = op(v, dpp32<kDppBcast15, 0xa>(id, v));
  v = op(v, dpp32<kDppBcast31, 0xc>(id, v));
  return (uint32_t)__builtin_amdgcn_readlane((int)v, 63);
}

// The same for 64-bit values (both halves move together).
template <typename Op>
__device__ __forceinline__ uint64_t wave_reduce64(uint64_t v, uint64_t id, Op op) {
  const uint32_t il = (uint32_t)id, ih = (uint32_t)(id >> 32);
  auto step = [&](auto mov) {
    const uint64_t t = ((uint64_t)mov(ih, (uint32_t)(v >> 32)) << 32) | mov(il, (uint32_t)v);
    v = op(v, t);
  };
  step([](uint32_t o, uint32_t x) { return dpp32<kDppXor1>(o, x); });
  step([](uint32_t o, uint32_t x) { return dpp32<kDppXor2>(o, x); });
  step([](uint32_t o, uint32_t x) { return dpp32<kDppHalfMirror>(o, x); });
  step([](uint32_t o, uint32_t x) { return dpp32<kDppMirror>(o, x); });
  step([](uint32_t o, uint32_t x) { return dpp32<kDppBcast15, 0xa>(o, x); });
  step([](uint32_t o, uint32_t x) { return dpp32<kDppBcast31, 0xc>(o, x); });
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)v, 63);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(v >> 32), 63);
  return ((uint64_t)hi << 32) | lo;
}

__device__ __forceinline__ float wave_max_f32(float v) {
  return __uint_as_float(wave_reduce32(__float_as_uint(v), 0xff800000u, [](uint32_t a, uint32_t b) {
    return __float_as_uint(fmaxf(__uint_as_float(a), __uint_as_float(b)));
  }));
}
// Sum in a fixed tree order (deterministic).
__device__ __forceinline__ float wave_sum_f32(float v) {
  return __uint_as_float(wave_reduce32(__float_as_uint(v), 0u, [](uint32_t a, uint32_t b) {
    return __float_as_uint(__uint_as_float(a) + __uint_as_float(b));
  }));
}
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
  return wave_reduce32(v, 0u, [](uint32_t a, uint32_t b) { return a > b ? a : b; });
}
__device__ __forceinline__ uint32_t wave_sum_u32(uint32_t v) {
  return wave_reduce32(v, 0u, [](uint32_t a, uint32_t b) { return a + b; });
}
__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) {
  return wave_reduce64(v, 0ull, [](uint64_t a, uint64_t b) { return a > b ? a : b; });
}
__device__ __forceinline__ uint64_t wave_min_u64(uint64_t v) {
  return wave_reduce64(v, ~0ull, [](uint64_t a, uint64_t b) { return a < b ? a : b; });
}
__device__ __forceinline__ double wave_sum_f64(double v) {
  return __longlong_as_double((long long)wave_reduce64((uint64_t)__double_as_longlong(v), 0ull, [](uint64_t a, uint64_t b) {
    return (uint64_t)__double_as_longlong(__longlong_as_double((long long)a) + __longlong_as_double((long long)b));
  }));
}

// Orders this wave's LDS accesses (a wave executes its LDS operations in
// order; this keeps the compiler from moving them across the point).
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Number of set bits of m below the calling lane.
__device__ __forceinline__ uint32_t lanes_below(uint64_t m) {
  return __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
}

__device__ __forceinline__ uint32_t wave_last_u32(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_readlane((int)v, 63);
}

// ---- block-level reductions (DPP within each wave, then LDS) --------------

template <int N>
__device__ __forceinline__ uint32_t block_sum_u32(uint32_t v, uint32_t* red) {
  v = wave_sum_u32(v);
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  __syncthreads();
  if (lane == 0) red[wid] = v;
  __syncthreads();
  uint32_t s = 0;
  for (int i = 0; i < N / 64; ++i) s += red[i];
  return s;
}

template <int N>
__device__ __forceinline__ float block_sum_f32(float v, float* red) {
  v = wave_sum_f32(v);
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  __syncthreads();
  if (lane == 0) red[wid] = v;
  __syncthreads();
  float s = 0.f;
  for (int i = 0; i < N / 64; ++i) s += red[i];
  return s;
}

template <int N>
__device__ __forceinline__ double block_sum_f64(double v, double* red) {
  v = wave_sum_f64(v);
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  __syncthreads();
  if (lane == 0) red[wid] = v;
  __syncthreads();
  double s = 0.0;
  for (int i = 0; i < N / 64; ++i) s += red[i];
  return s;
}

template <int N>
__device__ __forceinline__ uint32_t block_max_u32(uint32_t v, uint32_t* red) {
  v = wave_max_u32(v);
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  __syncthreads();
  if (lane == 0) red[wid] = v;
  __syncthreads();
  uint32_t s = 0;
  for (int i = 0; i < N / 64; ++i) s = max(s, red[i]);
  return s;
}

// The 64-bit value of lane (lane ^ j), j a power of two below 64: DPP moves
// within a 16-lane row for j <= 8 (quad_perm; row_shl/row_shr:4 and a
// select; row_ror:8), ds_swizzle's xor mode across the rows of a 32-lane
// half for j = 16, ds_bpermute across the halves for j = 32.  j is a
// constant once the caller's loops are unrolled, so the switch folds.
__device__ __forceinline__ uint32_t lane_xor32(uint32_t v, int j) {
  switch (j) {
    case 1: return dpp32<kDppXor1>(v, v);
    case 2: return dpp32<kDppXor2>(v, v);
    case 4: {
      const uint32_t up = dpp32<0x104>(v, v);  // row_shl:4: lane l gets lane l + 4
      const uint32_t dn = dpp32<0x114>(v, v);  // row_shr:4: lane l gets lane l - 4
      return (threadIdx.x & 4u) ? dn : up;
    }
    case 8: return dpp32<0x128>(v, v);         // row_ror:8: lane l gets lane (l + 8) mod 16 of its row
    case 16: return (uint32_t)__builtin_amdgcn_ds_swizzle((int)v, 0x401f);  // and 0x1f, xor 0x10
    default: return (uint32_t)__shfl_xor((int)v, 32, 64);
  }
}
__device__ __forceinline__ uint64_t lane_xor64(uint64_t v, int j) {
  return ((uint64_t)lane_xor32((uint32_t)(v >> 32), j) << 32) | lane_xor32((uint32_t)v, j);
}
__device__ __forceinline__ uint64_t readlane64(uint64_t v, int l) {
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)v, l);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(v >> 32), l);
  return ((uint64_t)hi << 32) | lo;
}

__device__ __forceinline__ uint64_t shfl_xor_u64(uint64_t v, int o) {
  const uint32_t hi = (uint32_t)__shfl_xor((int)(uint32_t)(v >> 32), o, 64);
  const uint32_t lo = (uint32_t)__shfl_xor((int)(uint32_t)v, o, 64);
  return ((uint64_t)hi << 32) | lo;
}

template <int N>
__device__ __forceinline__ uint64_t block_max_u64(uint64_t v, uint64_t* red) {
  v = wave_max_u64(v);
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  __syncthreads();
  if (lane == 0) red[wid] = v;
  __syncthreads();
  uint64_t s = red[0];
  for (int i = 1; i < N / 64; ++i) s = red[i] > s ? red[i] : s;
  return s;
}

template <int N>
__device__ __forceinline__ uint64_t block_min_u64(uint64_t v, uint64_t* red) {
  return ~block_max_u64<N>(~v, red);
}

// Exclusive prefix sum over the block in thread order; *total gets the sum.
template <int N>
__device__ __forceinline__ uint32_t block_excl_scan_u32(uint32_t v, uint32_t* red, uint32_t* total) {
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  const uint32_t inc = wave_incl_scan_u32(v);
  __syncthreads();
  if (lane == 63) red[wid] = inc;
  __syncthreads();
  uint32_t before = 0, tot = 0;
  for (int i = 0; i < N / 64; ++i) {
    if (i < wid) before += red[i];
    tot += red[i];
  }
  *total = tot;
  return before + inc - v;
}

// ---- chunk statistics ------------------------------------------------------

// Associative, order-independent merge of two statistics records.
__device__ __forceinline__ void stat_merge(ChunkStat& a, const ChunkStat& b) {
  a.max_l = fmaxf(a.max_l, b.max_l);
  if (b.am_ieee_i != 0xffffffffu &&
      (a.am_ieee_i == 0xffffffffu || b.am_ieee_v > a.am_ieee_v ||
       (b.am_ieee_v == a.am_ieee_v && b.am_ieee_i < a.am_ieee_i))) {
    a.am_ieee_v = b.am_ieee_v; a.am_ieee_i = b.am_ieee_i;
  }
  if (b.am_fin_i != 0xffffffffu) {
    bool take = a.am_fin_i == 0xffffffffu || b.am_fin_v > a.am_fin_v;
    if (!take && b.am_fin_v == a.am_fin_v) take = fin_order(b.am_fin_i) < fin_order(a.am_fin_i);
    if (take) { a.am_fin_v = b.am_fin_v; a.am_fin_i = b.am_fin_i; }
  }
  a.any_finite |= b.any_finite;
}

__device__ __forceinline__ void stat_init(ChunkStat& s) {
  s.max_l = -__builtin_inff();
  s.am_ieee_v = -__builtin_inff(); s.am_ieee_i = 0xffffffffu;
  s.am_fin_v = -__builtin_inff(); s.am_fin_i = 0xffffffffu;
  s.any_finite = 0u;
  s.lse_m = -__builtin_inff(); s.lse_sum = 0.f;
  s.n_cand = 0u; s.trunc = 0u; s.unkept_key = 0u; s.pad0 = 0u;
  s.min_kept = 0ull;
  s.pad1 = 0ull;
}

__device__ __forceinline__ ChunkStat stat_shfl_xor(const ChunkStat& s, int o) {
  ChunkStat r;
  stat_init(r);
  r.max_l = __shfl_xor(s.max_l, o, 64);
  r.am_ieee_v = __shfl_xor(s.am_ieee_v, o, 64); r.am_ieee_i = __shfl_xor(s.am_ieee_i, o, 64);
  r.am_fin_v = __shfl_xor(s.am_fin_v, o, 64); r.am_fin_i = __shfl_xor(s.am_fin_i, o, 64);
  r.any_finite = __shfl_xor(s.any_finite, o, 64);
  return r;
}

// Reduce a per-thread statistics record over the block (valid in all threads).
template <int N>
__device__ __forceinline__ ChunkStat block_stat(ChunkStat s, ChunkStat* red) {
  for (int o = 32; o > 0; o >>= 1) {
    const ChunkStat t = stat_shfl_xor(s, o);
    stat_merge(s, t);
  }
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  __syncthreads();
  if (lane == 0) red[wid] = s;
  __syncthreads();
  ChunkStat r = red[0];
  for (int i = 1; i < N / 64; ++i) stat_merge(r, red[i]);
  return r;
}

// ---- element access -------------------------------------------------------

__device__ __forceinline__ float load_raw(const void* base, int dtype, int64_t off) {
  if (dtype == HI_ROCM_DTYPE_BF16) return bf16_to_f32(((const uint16_t*)base)[off]);
  return ((const float*)base)[off];
}

__device__ __forceinline__ bool allowed(const SampleArgs& a, int row, uint32_t idx) {
  return !a.mask || ((a.mask[(int64_t)row * a.mask_words + (idx >> 5)] >> (idx & 31u)) & 1u);
}

// Processed logit of one token (mask + penalties), computed by the whole
// block: its history count is reduced over the row's history list.
template <int N>
__device__ __forceinline__ float processed_single(const SampleArgs& a, int row, const RowCfg& c, uint32_t idx,
                                  uint32_t* red) {
  uint32_t cnt = 0;
  if (a.hoff) {
    const uint32_t h0 = a.hoff[row], h1 = a.hoff[row + 1];
    for (uint32_t h = h0 + threadIdx.x; h < h1; h += N)
      if (a.hids[h] == idx) cnt += a.hcnt[h];
  }
  cnt = block_sum_u32<N>(cnt, red);
  float l = load_raw(a.logits, a.dtype, (int64_t)row * a.row_stride + idx);
  if (!allowed(a, row, idx)) l = -__builtin_inff();
  return apply_penalties(l, cnt, c);
}

// ---- radix selection ------------------------------------------------------

// Threshold T such that exactly k of the block's items (unique keys of
// `bits` bits, a multiple of 8) are >= T.  for_each(cb) calls cb(key) for
// every item the calling thread owns.  8-bit MSD descent with early exit;
// hist has 256 entries, sel 3.
template <typename ForEach>
__device__ __forceinline__ uint64_t radix_select_top(uint32_t* hist, uint32_t* sel, uint32_t k, int bits,
                                     ForEach for_each) {
  const int tid = threadIdx.x;
  uint64_t prefix = 0;
  uint32_t remaining = k;
  for (int shift = bits - 8; shift >= 0; shift -= 8) {
    for (int b = tid; b < 256; b += NT) hist[b] = 0u;
    __syncthreads();
    const int hs = shift + 8;
    const uint64_t hp = hs >= 64 ? 0ull : (prefix >> hs);
    for_each([&](uint64_t x) {
      if (hs >= 64 || (x >> hs) == hp) atomicAdd(&hist[(uint32_t)(x >> shift) & 255u], 1u);
    });
    __syncthreads();
    if (tid < 64) {
      // lane l owns bins 255-4l .. 252-4l (descending)
      uint32_t loc[4], lsum = 0;
      #pragma unroll
      for (int q = 0; q < 4; ++q) { loc[q] = hist[255 - 4 * tid - q]; lsum += loc[q]; }
      const uint32_t inc = wave_incl_scan_u32(lsum);
      const uint32_t above = inc - lsum;
      if (above < remaining && remaining <= above + lsum) {
        uint32_t acc = above;
        #pragma unroll
        for (int q = 0; q < 4; ++q) {
          if (remaining <= acc + loc[q] && acc < remaining) {
            sel[0] = 255u - 4u * tid - q; sel[1] = acc; sel[2] = loc[q];
          }
          acc += loc[q];
        }
      }
    }
    __syncthreads();
    prefix |= (uint64_t)sel[0] << shift;
    remaining -= sel[1];
    const bool done = sel[2] == remaining;
    __syncthreads();
    if (done) break;
  }
  return prefix;
}

// ==========================================================================
// LDS layouts
// ==========================================================================

struct ScanLds {
  uint64_t cbuf[kBufCap];     // running candidates (48-bit local composites)
  uint32_t U[kBuf];           // per-thread top-j keys of the first tile
  uint32_t hist[256];
  ChunkStat red[NT / 64];
  uint32_t redu[NT / 64];
  uint64_t red64[NT / 64];
  float redf[NT / 64];
  double redd[NT / 64];
  uint32_t sel[4];
  uint32_t bound, count, hovf;
  // when the batch has histories: bitmap[chunk / 32], hash keys[kHashCap],
  // hash counts[kHashCap] follow
};

// exact_expf's table read from an LDS copy: in the tail of a launch a load
// from global memory waits behind the other workgroups' streams, and after
// an acquire fence it misses the emptied L2.
struct Exp2TabLds {
  const uint64_t* p;
  __device__ uint64_t operator()(uint32_t i) const { return p[i]; }
};

struct FinLds {
  uint64_t cbig[kGather];     // gathered candidates (32 KiB) -- also a fold tile
  uint64_t buf[kBuf];         // selected candidates / rank keys
  uint32_t pay[kBuf];         // scaled-logit keys riding with buf
  float fa[kBuf];             // weights in rank order
  float fb[kBuf];             // w / total
  uint32_t hist[kBins];
  uint64_t mass[kBins];
  uint32_t aux[kBins];
  ChunkStat red[NT / 64];
  uint32_t redu[NT / 64];
  double redd[NT / 64];
  uint64_t red64[NT / 64];
  uint64_t red64b[NT / 64];
  uint32_t sel[4];
  uint32_t counter, n_ext, token, flag;
  float fval0, fval1;
  uint64_t below;   // largest candidate left out of the selection
  uint32_t wmin;    // bits of the smallest selected weight
  uint64_t thr;     // the selection threshold of a one-wave select
  int pick;         // wg_draw's result
  uint32_t nparts;  // finish_core_wave: waves that added their logprob share
  double lsum;      // finish_core_wave: log of the logprob normaliser
  uint64_t exptab[32];  // exact_expf's table (finish_lean and rank_candidates copy it)
};
constexpr int kTileFloats = kGather * 2;  // floats of the fold tile (cbig)


// ==========================================================================
// Finish phase (one workgroup per row)
// ==========================================================================

// Candidates of `row` (written by the chunks): chunk c wrote
// stats[c].n_cand of them at the start of its kFast slots.  f(x, pos) gets
// each candidate and its position in the chunk-major concatenation.
template <typename F>
__device__ __forceinline__ void for_each_candidate(const SampleArgs& a, int row, F f) {
  const int nch = a.n_chunks;
  const ChunkStat* stats = a.stats + (int64_t)row * nch;
  const uint64_t* cand = a.cand + (int64_t)row * nch * kFast;
  int off = 0;
  for (int c = 0; c < nch; ++c) {
    const int n = (int)stats[c].n_cand;
    for (int s = threadIdx.x; s < n; s += NT) f(cand[(int64_t)c * kFast + s], off + s);
    off += n;
  }
}

// One compare-exchange step of a descending bitonic sort over element
// indices i (this value) and i ^ j (the partner's value y / q), in stage k:
// the lower index of a pair keeps the larger key when (i & k) == 0.
// The exchange is a select under an all-ones / all-zero mask, with no
// branch (a conditional exchange compiles to divergent branches per step).
// Equal keys occur only for the zero padding, whose payloads are equal too.
__device__ __forceinline__ void bitonic_keep(uint64_t& x, uint32_t& p, uint64_t y, uint32_t q, int i, int j, int k) {
  const uint32_t keep_max = (((i & k) == 0) == ((i & j) == 0)) ? 1u : 0u;
  const uint32_t gt = y > x ? 1u : 0u;
  const uint64_t take = 0ull - (uint64_t)(1u ^ gt ^ keep_max);
  x = (y & take) | (x & ~take);
  p = (q & (uint32_t)take) | (p & ~(uint32_t)take);
}

// Descending sort of fs.buf[0..n) carrying fs.pay; n <= kBuf.
__device__ __forceinline__ void sort_ranked(FinLds& fs, int n) {
  const int tid = threadIdx.x;
  if (n <= NT) {
    // rank by counting (keys are unique), then scatter
    uint64_t x = 0;
    uint32_t p = 0, r = 0;
    if (tid < n) {
      x = fs.buf[tid];
      p = fs.pay[tid];
      for (int j = 0; j < n; ++j) r += fs.buf[j] > x;
    }
    __syncthreads();
    if (tid < n) { fs.buf[r] = x; fs.pay[r] = p; }
    __syncthreads();
    return;
  }
  // Bitonic network over kBuf elements (zero keys pad, and sort last), four
  // consecutive elements per thread in registers: distances 1 and 2 inside
  // the thread, 4 .. 128 across the lanes of a wave (shuffles), 256 and 512
  // across waves through LDS.
  static_assert(kBuf == 4 * NT, "four elements per thread");
  uint64_t x[4];
  uint32_t p[4];
  #pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int i = 4 * tid + r;
    x[r] = i < n ? fs.buf[i] : 0ull;
    p[r] = i < n ? fs.pay[i] : 0u;
  }
  __syncthreads();
  #pragma unroll
  for (int k = 2; k <= kBuf; k <<= 1) {
    #pragma unroll
    for (int j = k >> 1; j > 0; j >>= 1) {
      if (j >= 256) {
        #pragma unroll
        for (int r = 0; r < 4; ++r) { fs.buf[4 * tid + r] = x[r]; fs.pay[4 * tid + r] = p[r]; }
        __syncthreads();
        #pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int i = 4 * tid + r;
          bitonic_keep(x[r], p[r], fs.buf[i ^ j], fs.pay[i ^ j], i, j, k);
        }
        __syncthreads();
      } else if (j >= 4) {
        const int o = j >> 2;  // partner lane: lane ^ o (same wave: 4 * 64 = 256 elements)
        #pragma unroll
        for (int r = 0; r < 4; ++r) {
          const uint64_t y = lane_xor64(x[r], o);  // DPP within rows of 16 lanes
          const uint32_t q = lane_xor32(p[r], o);
          bitonic_keep(x[r], p[r], y, q, 4 * tid + r, j, k);
        }
      } else {
        // partners inside the thread: (0, j) and (1 or 2, 1 + j or 3)
        uint64_t y[4];
        uint32_t q[4];
        #pragma unroll
        for (int r = 0; r < 4; ++r) {
          y[r] = j == 1 ? x[r ^ 1] : x[r ^ 2];
          q[r] = j == 1 ? p[r ^ 1] : p[r ^ 2];
        }
        #pragma unroll
        for (int r = 0; r < 4; ++r) bitonic_keep(x[r], p[r], y[r], q[r], 4 * tid + r, j, k);
      }
    }
  }
  #pragma unroll
  for (int r = 0; r < 4; ++r) { fs.buf[4 * tid + r] = x[r]; fs.pay[4 * tid + r] = p[r]; }
  __syncthreads();
}

// Descending bitonic sort of the keys buf[0..n), n <= PER * NT, keys only
// (zero pads them and sorts last; equal keys are equal values).  PER
// consecutive elements per thread in registers: distances below PER inside
// the thread, up to 32 * PER across the lanes of a wave (DPP, swizzle and
// bpermute lane moves), 64 * PER and more through buf with barriers.  buf
// has room for PER * NT keys; all of them are written.
template <int PER>
__device__ __forceinline__ void block_sort_desc(uint64_t* buf, int n) {
  const int tid = threadIdx.x;
  uint64_t x[PER];
  #pragma unroll
  for (int r = 0; r < PER; ++r) {
    const int i = PER * tid + r;
    x[r] = i < n ? buf[i] : 0ull;
  }
  auto keep = [](uint64_t& v, uint64_t y, int i, int j, int k) {
    const bool keep_max = ((i & k) == 0) == ((i & j) == 0);
    const uint64_t hi = y > v ? y : v, lo = y > v ? v : y;
    v = keep_max ? hi : lo;
  };
  #pragma unroll
  for (int k = 2; k <= PER * NT; k <<= 1) {
    #pragma unroll
    for (int j = k >> 1; j > 0; j >>= 1) {
      if (j >= 64 * PER) {
        __syncthreads();
        #pragma unroll
        for (int r = 0; r < PER; ++r) buf[PER * tid + r] = x[r];
        __syncthreads();
        #pragma unroll
        for (int r = 0; r < PER; ++r) {
          const int i = PER * tid + r;
          keep(x[r], buf[i ^ j], i, j, k);
        }
      } else if (j >= PER) {
        #pragma unroll
        for (int r = 0; r < PER; ++r) keep(x[r], lane_xor64(x[r], j / PER), PER * tid + r, j, k);
      } else {
        uint64_t y[PER];
        #pragma unroll
        for (int r = 0; r < PER; ++r) y[r] = x[r ^ j];
        #pragma unroll
        for (int r = 0; r < PER; ++r) keep(x[r], y[r], PER * tid + r, j, k);
      }
    }
  }
  __syncthreads();
  #pragma unroll
  for (int r = 0; r < PER; ++r) buf[PER * tid + r] = x[r];
  __syncthreads();
}

// Calls f(key) with the candidate key (processed-logit key, index) of every
// logit of `row` this thread owns, recomputing the processed logits: tiles
// of 2048 logits with an LDS count table of the row's history (cnt has
// 2048 entries).  All threads call it.
template <typename F>
__device__ __forceinline__ void for_each_row_key(const SampleArgs& a, int row, const RowCfg& cfg, uint32_t* cnt,
                                                 F f) {
  constexpr int T = 2048;
  const int tid = threadIdx.x;
  uint32_t h0 = 0, h1 = 0;
  if (a.hoff) { h0 = a.hoff[row]; h1 = a.hoff[row + 1]; }
  const int64_t rbase = (int64_t)row * a.row_stride;
  for (int t0 = 0; t0 < a.V; t0 += T) {
    const int t1 = min(t0 + T, a.V);
    __syncthreads();
    for (int i = tid; i < T; i += NT) cnt[i] = 0u;
    __syncthreads();
    for (uint32_t h = h0 + tid; h < h1; h += NT) {
      const uint32_t id = a.hids[h];
      if (id >= (uint32_t)t0 && id < (uint32_t)t1) atomicAdd(&cnt[id - t0], a.hcnt[h]);
    }
    __syncthreads();
    for (int e = t0 + tid; e < t1; e += NT) {
      float l = load_raw(a.logits, a.dtype, rbase + e);
      if (!allowed(a, row, (uint32_t)e)) l = -__builtin_inff();
      l = apply_penalties(l, cnt[e - t0], cfg);
      f(cand_key(lkey(l), (uint32_t)e));
    }
  }
  __syncthreads();
}

// The exact top kk candidate keys of the whole row into fs.buf[0, kk),
// from the logits themselves (for a row whose chunks' candidates may miss
// part of its top kk).  Returns the kk-th key; *below gets the largest key
// left out.
__device__ __forceinline__ uint64_t row_select_exact(FinLds& fs, const SampleArgs& a, int row, const RowCfg& cfg,
                                                     int kk, uint64_t* below) {
  const int tid = threadIdx.x;
  uint32_t* cnt = reinterpret_cast<uint32_t*>(fs.mass);
  static_assert(sizeof(fs.mass) >= 2048 * sizeof(uint32_t), "count table fits");
  uint64_t thr = 0ull;
  if (kk < a.V)
    thr = radix_select_top(fs.hist, fs.sel, (uint32_t)kk, 64,
                           [&](auto cb) { for_each_row_key(a, row, cfg, cnt, cb); });
  if (tid == 0) fs.counter = 0u;
  __syncthreads();
  uint64_t umax = 0ull;
  for_each_row_key(a, row, cfg, cnt, [&](uint64_t x) {
    if (x >= thr) fs.buf[atomicAdd(&fs.counter, 1u)] = x;
    else if (x > umax) umax = x;
  });
  *below = block_max_u64<NT>(umax, fs.red64);
  return thr;
}

// Number of candidates the chunks of `row` wrote.
// The exact first `kk` entries of the reference rank order (weight desc,
// index asc) of `row`.  On return fs.buf[0..kk) holds rank keys in order and
// fs.pay[0..kk) the scaled-logit keys; returns kk.  M is the row max of s.
// *n_lds (when given) gets the number of the row's candidates when all of
// them are in fs.cbig[0, n) in chunk order, else -1.
__device__ __forceinline__ int rank_candidates(FinLds& fs, const SampleArgs& a, int row, const RowCfg& cfg,
                               int kk_req, float M, int* n_lds = nullptr) {
  const int tid = threadIdx.x;
  const int nch = a.n_chunks;
  const ChunkStat* stats = a.stats + (int64_t)row * nch;
  if (n_lds) *n_lds = -1;
  // the chunks' candidate offsets, fs.aux[0, nch] when they fit (the chunk
  // records are read once, all at a time)
  const bool offs = nch < kBins;
  uint32_t run = 0u;
  for (int cb = 0; cb < nch; cb += NT) {
    const int c = cb + tid;
    const uint32_t n = c < nch ? stats[c].n_cand : 0u;
    uint32_t tot;
    const uint32_t ex = block_excl_scan_u32<NT>(n, fs.redu, &tot);
    if (offs && c < nch) fs.aux[c] = run + ex;
    run += tot;
  }
  if (offs && tid == 0) fs.aux[nch] = run;
  __syncthreads();
  const int n_total = (int)run;
  int kk = min(kk_req, n_total);
  if (kk <= 0) return 0;
  auto s_of = [&](uint64_t x) { return key_to_s(cand_skey(x), cfg.t_eff); };
  // exact_expf's table from an LDS copy (after the finish's acquire fence a
  // load of the constant table misses the emptied L2); the barrier after
  // step 1 publishes it
  if (tid < 32) fs.exptab[tid] = exp2_tab32((uint32_t)tid);
  const Exp2TabLds et{fs.exptab};
  auto wexp = [&](float x) { return exact_expf_t(x, et); };
  // 1. candidates into LDS: all of them when they fit, else those at or above
  //    t0, the largest chunk cut (the kk-th composite is at least every
  //    truncated chunk's smallest kept composite)
  uint64_t t0 = 0;
  uint64_t below_max = 0;  // largest candidate left out of LDS
  int n_u;
  bool in_lds = true;
  if (n_total <= kGather && !offs) {
    for_each_candidate(a, row, [&](uint64_t x, int pos) { fs.cbig[pos] = x; });
    n_u = n_total;
    if (n_lds) *n_lds = n_total;
  } else if (n_total <= kGather) {
    // every candidate, all loads issued before the stores
    constexpr int kPer = kGather / NT;
    const uint64_t* cand = a.cand + (int64_t)row * nch * kFast;
    uint64_t v[kPer];
    int c = 0;
    #pragma unroll
    for (int r = 0; r < kPer; ++r) {
      const int i = tid + r * NT;
      v[r] = 0ull;
      if (i < n_total) {
        while ((int)fs.aux[c + 1] <= i) ++c;
        v[r] = cand[(int64_t)c * kFast + (i - (int)fs.aux[c])];
      }
    }
    #pragma unroll
    for (int r = 0; r < kPer; ++r) {
      const int i = tid + r * NT;
      if (i < n_total) fs.cbig[i] = v[r];
    }
    n_u = n_total;
    if (n_lds) *n_lds = n_total;
  } else {
    for (int c = tid; c < nch; c += NT)
      if (stats[c].trunc && stats[c].min_kept > t0) t0 = stats[c].min_kept;
    t0 = block_max_u64<NT>(t0, fs.red64);
    uint32_t nu = 0;
    for_each_candidate(a, row, [&](uint64_t x, int) {
      nu += x >= t0;
      if (x < t0 && x > below_max) below_max = x;
    });
    n_u = (int)block_sum_u32<NT>(nu, fs.redu);
    below_max = block_max_u64<NT>(below_max, fs.red64);
    in_lds = n_u <= kGather;
    if (in_lds) {
      if (tid == 0) fs.counter = 0u;
      __syncthreads();
      for_each_candidate(a, row, [&](uint64_t x, int) {
        if (x >= t0) fs.cbig[atomicAdd(&fs.counter, 1u)] = x;
      });
    }
  }
  __syncthreads();
  // 2. the kk largest
  uint64_t thr = 0;
  if (in_lds) {
    if (n_u > kk) {
      thr = radix_select_top(fs.hist, fs.sel, (uint32_t)kk, 64, [&](auto cb) {
        for (int i = tid; i < n_u; i += NT) cb(fs.cbig[i]);
      });
    }
    uint64_t umax = 0;  // largest unselected
    if (tid == 0) fs.counter = 0u;
    __syncthreads();
    for (int i = tid; i < n_u; i += NT) {
      const uint64_t x = fs.cbig[i];
      if (x >= thr) fs.buf[atomicAdd(&fs.counter, 1u)] = x;
      else if (x > umax) umax = x;
    }
    below_max = max(below_max, block_max_u64<NT>(umax, fs.red64));
  } else {
    // rare: more than kGather candidates above t0; select over global memory
    thr = radix_select_top(fs.hist, fs.sel, (uint32_t)kk, 64, [&](auto cb) {
      for_each_candidate(a, row, [&](uint64_t x, int) { if (x >= t0) cb(x); });
    });
    if (tid == 0) fs.counter = 0u;
    __syncthreads();
    uint64_t umax = 0;
    for_each_candidate(a, row, [&](uint64_t x, int) {
      if (x >= thr && x >= t0) {
        const uint32_t p = atomicAdd(&fs.counter, 1u);
        if (p < (uint32_t)kBuf) fs.buf[p] = x;
      } else if (x > umax) {
        umax = x;
      }
    });
    below_max = max(below_max, block_max_u64<NT>(umax, fs.red64));
  }
  thr = thr > t0 ? thr : t0;
  // the candidates hold the row's top kk only if the kk-th key is above
  // every key a truncated chunk left out; else select from the logits
  {
    uint32_t ub = 0u;
    for (int c = tid; c < nch; c += NT)
      if (stats[c].trunc) ub = max(ub, stats[c].unkept_key);
    ub = block_max_u32<NT>(ub, fs.redu);
    uint64_t mn = ~0ull;
    for (int i = tid; i < kk; i += NT) mn = fs.buf[i] < mn ? fs.buf[i] : mn;
    mn = block_min_u64<NT>(mn, fs.red64);
    const uint64_t kth = kk < n_total ? thr : mn;
    if (ub != 0u && cand_skey(kth) <= ub) {
      if (n_lds) *n_lds = -1;  // (row_select_exact uses fs.cbig)
      kk = min(kk_req, a.V);
      uint64_t bm;
      thr = row_select_exact(fs, a, row, cfg, kk, &bm);
      below_max = bm;
      t0 = 0ull;
      in_lds = false;
    }
  }
  // 3. weights; the smallest selected weight is w_b
  uint32_t wmin_bits = 0xffffffffu;
  for (int i = tid; i < kk; i += NT) {
    const uint64_t x = fs.buf[i];
    const float sx = s_of(x);
    const float w = wexp(sx - M);
    fs.buf[i] = rank_key(w, cand_idx(x));
    fs.pay[i] = okey(sx);
    wmin_bits = min(wmin_bits, __float_as_uint(w));
  }
  const float w_b = __uint_as_float(~block_max_u32<NT>(~wmin_bits, fs.redu));
  // 4. tie extension: elements outside the selection with weight w_b can
  //    still belong to the first kk of the rank order (lower index)
  if (tid == 0) fs.n_ext = 0u;
  __syncthreads();
  uint64_t* ext = a.ws_list + (int64_t)row * a.list_stride;
  uint32_t* ext_aux = reinterpret_cast<uint32_t*>(a.ws_w + (int64_t)row * a.V);
  const int64_t ext_cap = a.V;
  auto add_ext = [&](float w, uint32_t idx, float sx) {
    const uint32_t p = atomicAdd(&fs.n_ext, 1u);
    if (p < ext_cap) { ext[p] = rank_key(w, idx); ext_aux[p] = okey(sx); }
  };
  if (w_b > 0.f) {
    // (a) unselected candidates: weights are monotone in the key, so only if
    //     the largest of them ties
    if (below_max != 0 && wexp(s_of(below_max) - M) == w_b) {
      if (in_lds) {
        for (int i = tid; i < n_u; i += NT) {
          const uint64_t x = fs.cbig[i];
          if (x >= thr) continue;
          const float sx = s_of(x);
          const float w = wexp(sx - M);
          if (w == w_b) add_ext(w, cand_idx(x), sx);
        }
      }
      if (!in_lds || t0 != 0) {
        for_each_candidate(a, row, [&](uint64_t x, int) {
          if (x >= thr || (in_lds && x >= t0)) return;  // selected, or seen in LDS
          const float sx = s_of(x);
          const float w = wexp(sx - M);
          if (w == w_b) add_ext(w, cand_idx(x), sx);
        });
      }
    }
    // (b) elements a truncated chunk did not keep (rare: recompute the
    //     chunk); chunks are checked NT at a time
    for (int cb = 0; cb < nch; cb += NT) {
      if (tid == 0) fs.counter = 0u;
      __syncthreads();
      {
        const int c = cb + tid;
        if (c < nch) {
          const ChunkStat cs = stats[c];
          if (cs.trunc && wexp(key_to_s(cs.unkept_key, cfg.t_eff) - M) == w_b)
            fs.aux[atomicAdd(&fs.counter, 1u)] = (uint32_t)c;
        }
      }
      __syncthreads();
      const uint32_t n_flag = fs.counter;
      for (uint32_t f = 0; f < n_flag; ++f) {
        const int c = (int)fs.aux[f];
        const ChunkStat cs = stats[c];
        const int c0 = c * a.chunk, c1 = min(c0 + a.chunk, a.V);
        const int64_t rbase = (int64_t)row * a.row_stride;
        uint32_t h0 = 0, h1 = 0;
        if (a.hoff) { h0 = a.hoff[row]; h1 = a.hoff[row + 1]; }
        for (int e = c0 + tid; e < c1; e += NT) {
          float l = load_raw(a.logits, a.dtype, rbase + e);
          if (!allowed(a, row, (uint32_t)e)) l = -__builtin_inff();
          uint32_t cnt = 0;
          for (uint32_t h = h0; h < h1; ++h) if (a.hids[h] == (uint32_t)e) cnt += a.hcnt[h];
          l = apply_penalties(l, cnt, cfg);
          const uint32_t kl = lkey(l);
          const uint64_t ck = cand_key(kl, (uint32_t)e);
          if (ck >= cs.min_kept || ck >= thr) continue;  // a candidate, or selected
          const float sx = key_to_s(kl, cfg.t_eff);
          const float w = wexp(sx - M);
          if (w == w_b) add_ext(w, (uint32_t)e, sx);
        }
      }
      __syncthreads();
    }
  }
  __syncthreads();
  const uint32_t n_ext = min(fs.n_ext, (uint32_t)(ext_cap - kk));
  if (n_ext > 0) {
    // union of selection and extension, then its first kk by rank key
    const int n_all = kk + (int)n_ext;
    for (int i = tid; i < kk; i += NT) { ext[n_ext + i] = fs.buf[i]; ext_aux[n_ext + i] = fs.pay[i]; }
    __syncthreads();
    const uint64_t t2 = radix_select_top(fs.hist, fs.sel, (uint32_t)kk, 64, [&](auto cb) {
      for (int j = tid; j < n_all; j += NT) cb(ext[j]);
    });
    if (tid == 0) fs.counter = 0u;
    __syncthreads();
    for (int j = tid; j < n_all; j += NT) {
      const uint64_t x = ext[j];
      if (x >= t2) {
        const uint32_t p = atomicAdd(&fs.counter, 1u);
        if (p < (uint32_t)kBuf) { fs.buf[p] = x; fs.pay[p] = ext_aux[j]; }
      }
    }
    __syncthreads();
  }
  sort_ranked(fs, kk);
  return kk;
}

// Reference steps 7-10 over the first k entries of the rank order in fs.buf
// (top-k rows); defined with the wave folds below.
__device__ __forceinline__ uint32_t draw_topk(FinLds& fs, const RowCfg& cfg, int k);

// Serial f32 fold of a global float array in index order (Rust's Sum: a fold
// from -0.0), by thread 0, staged through LDS tiles.  Valid in all threads.
__device__ __forceinline__ float fold_global(FinLds& fs, const float* x, int n) {
  float* tile = reinterpret_cast<float*>(fs.cbig);
  float acc = -0.0f;  // meaningful in thread 0 only
  for (int t0 = 0; t0 < n; t0 += kTileFloats) {
    const int m = min(kTileFloats, n - t0);
    __syncthreads();
    for (int i = threadIdx.x; i < m; i += NT) tile[i] = x[t0 + i];
    __syncthreads();
    if (threadIdx.x == 0)
      for (int i = 0; i < m; ++i) acc += tile[i];
  }
  __syncthreads();
  if (threadIdx.x == 0) fs.fval0 = acc;
  __syncthreads();
  const float r = fs.fval0;
  __syncthreads();
  return r;
}

// Bitonic sort of a global array (descending) by one workgroup.
__device__ __forceinline__ void global_sort_desc(uint64_t* g, int n2) {
  for (int k = 2; k <= n2; k <<= 1) {
    for (int j = k >> 1; j > 0; j >>= 1) {
      for (int i = threadIdx.x; i < n2; i += NT) {
        const int ixj = i ^ j;
        if (ixj > i) {
          const uint64_t x = g[i], y = g[ixj];
          const bool desc = (i & k) == 0;
          if (desc ? (x < y) : (x > y)) { g[i] = y; g[ixj] = x; }
        }
      }
      __syncthreads();
    }
  }
}

// Rows without top-k (or with top_k > 1024): the distribution is re-read from
// the workspace (ws_s holds the scaled logits).  Returns the token or
// 0xffffffff for the argmax fallback.
__device__ __forceinline__ uint32_t draw_wide(FinLds& fs, const SampleArgs& a, int row, const RowCfg& cfg,
                              float M, float u) {
  const int tid = threadIdx.x;
  const int V = a.V;
  const float* srow = a.ws_s + (int64_t)row * V;
  float* wrow = a.ws_w + (int64_t)row * V;
  uint64_t* list = a.ws_list + (int64_t)row * a.list_stride;
  for (int b = tid; b < kBins; b += NT) { fs.hist[b] = 0u; fs.mass[b] = 0ull; }
  __syncthreads();
  for (int i = tid; i < V; i += NT) {
    float w = exact_expf(srow[i] - M);
    if (w < cfg.min_p) w = 0.f;
    wrow[i] = w;
    if (w > 0.f) {
      const uint32_t b = __float_as_uint(w) >> 20;
      atomicAdd(&fs.hist[b], 1u);
      atomicAdd((unsigned long long*)&fs.mass[b], (unsigned long long)((double)w * 1099511627776.0));
    }
  }
  __syncthreads();
  const bool wide_k = cfg.cls == kTopK;
  float total = 0.f;
  if (!wide_k) {
    total = fold_global(fs, wrow, V);  // gpu.rs:837: vocab-order sum
    if (total <= 0.f || !finitef_(total)) return 0xffffffffu;
  }
  if (tid == 0) {
    uint64_t all_mass = 0;
    for (int b = 0; b < kBins; ++b) all_mass += fs.mass[b];
    int bstar = 0;
    if (wide_k) {
      uint32_t c = 0;
      for (int b = kBins - 1; b >= 0; --b) { c += fs.hist[b]; if (c >= (uint32_t)cfg.k_eff) { bstar = b; break; } }
    } else if (cfg.cutoff < 1.f) {
      // superset holding the nucleus with margin (verified below)
      const double need = fmin(1.0, (double)cfg.cutoff + 0.02) * (double)all_mass;
      uint64_t c = 0;
      for (int b = kBins - 1; b >= 0; --b) { c += fs.mass[b]; if ((double)c >= need) { bstar = b; break; } }
    }
    fs.flag = (uint32_t)bstar;
  }
  __syncthreads();
  int bstar = (int)fs.flag;
  uint32_t tok = 0xffffffffu;
  for (int attempt = 0; attempt < 2; ++attempt) {
    __syncthreads();
    if (tid == 0) {
      uint32_t off = 0;
      for (int b = kBins - 1; b >= 0; --b) {
        fs.aux[b] = off;
        if (b >= bstar) off += fs.hist[b];
      }
      fs.counter = off;
    }
    __syncthreads();
    const int n_sup = (int)fs.counter;
    for (int i = tid; i < V; i += NT) {
      const float w = wrow[i];
      if (w > 0.f) {
        const int b = (int)(__float_as_uint(w) >> 20);
        if (b >= bstar) list[atomicAdd(&fs.aux[b], 1u)] = rank_key(w, (uint32_t)i);
      }
    }
    __syncthreads();
    const int n2 = next_pow2(max(n_sup, 1));
    for (int i = n_sup + tid; i < n2; i += NT) list[i] = 0ull;
    __syncthreads();
    global_sort_desc(list, n2);
    if (tid == 0) {
      int k = n_sup;
      if (wide_k) {
        k = min(cfg.k_eff, n_sup);  // zero-weight entries add nothing
        float t = -0.0f;
        for (int i = 0; i < k; ++i) t += rank_w(list[i]);
        total = t;
      }
      uint32_t r = 0xffffffffu;
      uint32_t flag = 1u;
      if (total > 0.f && finitef_(total)) {
        float cum_p = 0.f;
        int m_end = 0;
        bool reached = false;
        for (int i = 0; i < k; ++i) {
          m_end = i + 1;
          cum_p += rank_w(list[i]) / total;
          if (cfg.cutoff < 1.f && cum_p >= cfg.cutoff) { reached = true; break; }
        }
        if (!wide_k && !reached && bstar != 0) {
          flag = 0xffffffffu;  // superset too small: retry with every positive weight
        } else {
          float ct = -0.0f;
          for (int i = 0; i < m_end; ++i) ct += rank_w(list[i]);
          if (m_end > 0 && ct > 0.f && finitef_(ct)) {
            const float target = clamp_uniform(u) * ct;
            float cum = 0.f;
            int pick = m_end - 1;
            for (int i = 0; i < m_end; ++i) {
              cum += rank_w(list[i]);
              if (target < cum) { pick = i; break; }
            }
            r = cand_idx(list[pick]);
          }
        }
      }
      fs.token = r;
      fs.flag = flag;
    }
    __syncthreads();
    if (fs.flag != 0xffffffffu) { tok = fs.token; break; }
    bstar = 0;
  }
  return tok;
}

// Temperature-only rows: kernels.cu:7803-7867 with the exact weight function.
// 256 contiguous chunks, one per thread of the (256-thread) workgroup.
__device__ __forceinline__ uint32_t draw_temp_only(FinLds& fs, const SampleArgs& a, int row, float M, float u,
                                   uint32_t argmax_fin) {
  static_assert(NT == 256, "the reference's temperature-only path uses 256 chunks");
  const int tid = threadIdx.x;
  const int V = a.V;
  const float* srow = a.ws_s + (int64_t)row * V;
  const int chunk = (V + 255) / 256;
  float* csum = fs.fa;
  float* prefix = fs.fb;
  {
    const int start = tid * chunk, end = min(start + chunk, V);
    float s = 0.f;
    for (int i = start; i < end; ++i) s += exact_expf(srow[i] - M);
    csum[tid] = s;
  }
  __syncthreads();
  if (tid == 0) {
    float acc = 0.f;
    for (int j = 0; j < 256; ++j) { prefix[j] = acc; acc += csum[j]; }
    fs.fval0 = acc;
    fs.token = 0xffffffffu;
  }
  __syncthreads();
  const float total = fs.fval0;
  if (total <= 0.f || !finitef_(total)) return argmax_fin;
  const float uu = finitef_(u) ? fminf(fmaxf(u, 0.f), 0.99999994f) : 0.f;
  const float target = uu * total;
  {
    const int start = tid * chunk, end = min(start + chunk, V);
    const float lo = prefix[tid];
    const float hi = lo + csum[tid];
    if (start < end && target >= lo && (target < hi || tid == 255)) {
      float cum = lo;
      int chosen = -1;
      for (int i = start; i < end; ++i) {
        const float w = exact_expf(srow[i] - M);
        if (w <= 0.f) continue;
        chosen = i;
        cum += w;
        if (target < cum) break;
      }
      if (chosen >= 0) atomicMin(&fs.token, (uint32_t)chosen);
    }
  }
  __syncthreads();
  return fs.token != 0xffffffffu ? fs.token : argmax_fin;
}

// argmax_host (gpu.rs:739-751, total_cmp, lowest index) over the processed
// logits of the row.  Only needed when no scaled logit is finite (or l / T
// overflows), so the row is re-read here, 4096 logits at a time, with an LDS
// count table for the penalties.
__device__ __forceinline__ uint32_t row_argmax_total(FinLds& fs, const SampleArgs& a, int row,
                                                     const RowCfg& cfg) {
  const int tid = threadIdx.x;
  const int V = a.V;
  constexpr int T = 4096;
  static_assert(kGather * 2 >= T, "count table fits cbig");
  uint32_t* cnt = reinterpret_cast<uint32_t*>(fs.cbig);
  uint32_t h0 = 0, h1 = 0;
  if (a.hoff) { h0 = a.hoff[row]; h1 = a.hoff[row + 1]; }
  const int64_t rbase = (int64_t)row * a.row_stride;
  uint64_t best = 0ull;  // (total key biased) << 32 | (0xffffffff - index)
  for (int t0 = 0; t0 < V; t0 += T) {
    const int t1 = min(t0 + T, V);
    __syncthreads();
    for (int i = tid; i < T; i += NT) cnt[i] = 0u;
    __syncthreads();
    for (uint32_t h = h0 + tid; h < h1; h += NT) {
      const uint32_t id = a.hids[h];
      if (id >= (uint32_t)t0 && id < (uint32_t)t1) atomicAdd(&cnt[id - t0], a.hcnt[h]);
    }
    __syncthreads();
    for (int e = t0 + tid; e < t1; e += NT) {
      float l = load_raw(a.logits, a.dtype, rbase + e);
      if (!allowed(a, row, (uint32_t)e)) l = -__builtin_inff();
      l = apply_penalties(l, cnt[e - t0], cfg);
      const uint64_t v = ((uint64_t)((uint32_t)total_key(l) ^ 0x80000000u) << 32) |
                         (uint64_t)(0xffffffffu - (uint32_t)e);
      best = v > best ? v : best;
    }
  }
  best = block_max_u64<NT>(best, fs.red64);
  return 0xffffffffu - (uint32_t)best;
}

__device__ __forceinline__ void finish_logprobs(FinLds& fs, const SampleArgs& a, int row, const RowCfg& cfg, uint32_t token,
                                float M, bool eos, int ranked_k, double log_sum_known = __builtin_nan(""));

template <int DM>
__device__ __forceinline__ int wave_draw(const uint64_t* keys, int k, const RowCfg& cfg);

// This thread's share of the logprob normaliser relative to M, threads t0,
// t0 + nt, ... of the row's work: the candidates of every chunk in double
// (from fs.cbig[0, n_lds) when they are all there, n_lds >= 0, else from
// the workspace), the other logits from each chunk's mass.
__device__ __forceinline__ double logprob_part(FinLds& fs, const SampleArgs& a, int row, const RowCfg& cfg, float M,
                                              int n_lds, int t0, int nt) {
  double part = 0.0;
  auto add = [&](uint64_t x) {
    if (cand_skey(x) > kKeyNegInf) part += exp((double)key_to_s(cand_skey(x), cfg.t_eff) - (double)M);
  };
  const int nch = a.n_chunks;
  const ChunkStat* stats = a.stats + (int64_t)row * nch;
  if (n_lds >= 0) {
    for (int i = t0; i < n_lds; i += nt) add(fs.cbig[i]);
  } else {
    const uint64_t* cand = a.cand + (int64_t)row * nch * kFast;
    for (int c = 0; c < nch; ++c) {
      const int n = (int)stats[c].n_cand;
      for (int j = t0; j < n; j += nt) add(cand[(int64_t)c * kFast + j]);
    }
  }
  for (int c = t0; c < nch; c += nt) {
    const ChunkStat cs = stats[c];
    if (cs.lse_sum > 0.f) part += (double)cs.lse_sum * exp((double)cs.lse_m - (double)M);
  }
  return part;
}

__device__ __forceinline__ void finish_row(FinLds& fs, const SampleArgs& a, int row, const RowCfg& cfg) {
  const int tid = threadIdx.x;
  ChunkStat st;
  stat_init(st);
  for (int c = tid; c < a.n_chunks; c += NT) stat_merge(st, a.stats[(int64_t)row * a.n_chunks + c]);
  const ChunkStat rs = block_stat<NT>(st, fs.red);
  // row max of s = l / T: division is monotone, so it is max(l) / T
  const float M = finitef_(rs.max_l) ? rs.max_l / cfg.t_eff : -__builtin_inff();
  const uint32_t am_ieee = rs.am_ieee_i == 0xffffffffu ? 0u : rs.am_ieee_i;
  const uint32_t am_fin = rs.am_fin_i == 0xffffffffu ? 0u : rs.am_fin_i;
  const float u = cfg.u;

  const bool eos = a.mask && !rs.any_finite;
  const bool want_lp = a.n_lp > 0 || a.out_token_lp != nullptr;
  uint32_t token;
  int ranked_k = 0;  // entries of fs.buf in rank order
  double log_sum = __builtin_nan("");  // the logprob normaliser's log, once known
  if (eos) {
    token = cfg.eos;
  } else if (cfg.cls == kGreedy) {
    token = a.pv.greedy_rule == kGreedyFiniteLane ? am_fin : am_ieee;
  } else if (!finitef_(M)) {
    token = cfg.cls == kTempOnly ? am_fin : row_argmax_total(fs, a, row, cfg);
  } else if (cfg.cls == kTopK && !cfg.store_s) {
    int n_lds = -1;
    ranked_k = rank_candidates(fs, a, row, cfg, cfg.k_sel, M, &n_lds);
    // the draw on wave 0 (gpu.rs:831-899); meanwhile the other waves add up
    // the logprob normaliser
    int pick = -1;
    if (tid < 64) {
      pick = wave_draw<kBuf / 64>(fs.buf, min(cfg.k_eff, ranked_k), cfg);
      if (tid == 0) fs.pick = pick;
    } else if (want_lp) {
      double part = logprob_part(fs, a, row, cfg, M, n_lds, tid - 64, NT - 64);
      part = wave_sum_f64(part);
      if ((tid & 63) == 0) fs.redd[tid >> 6] = part;
    }
    __syncthreads();
    pick = fs.pick;
    if (want_lp) {
      double tot = 0.0;
      #pragma unroll
      for (int v = 1; v < NT / 64; ++v) tot += fs.redd[v];
      log_sum = log(tot);
    }
    token = pick < 0 ? 0xffffffffu : cand_idx(fs.buf[pick]);
    if (token == 0xffffffffu) token = row_argmax_total(fs, a, row, cfg);
  } else if (cfg.cls == kTempOnly) {
    token = draw_temp_only(fs, a, row, M, u, am_fin);
  } else {
    token = draw_wide(fs, a, row, cfg, M, u);
    if (token == 0xffffffffu) token = row_argmax_total(fs, a, row, cfg);
  }
  if (tid == 0) a.out_tokens[row] = token;
  if (!want_lp) return;
  __syncthreads();
  finish_logprobs(fs, a, row, cfg, token, M, eos, ranked_k, log_sum);
}

// Logprobs of the processed distribution (extension) once the row's token
// is known: the top n_lp in rank order and the token's own.  M is the row
// max of s; fs.buf / fs.pay hold the first ranked_k entries of the rank
// order (0: none yet).  The normaliser sums the candidates of every chunk
// in double and the other logits from each chunk's mass.
__device__ __forceinline__ void finish_logprobs(FinLds& fs, const SampleArgs& a, int row, const RowCfg& cfg, uint32_t token,
                                float M, bool eos, int ranked_k, double log_sum_known) {
  const int tid = threadIdx.x;
  const int V = a.V;
  const int N = a.n_lp;
  if (eos || !finitef_(M)) {
    for (int j = tid; j < N; j += NT) {
      a.out_lp[(int64_t)row * N + j] = -__builtin_inff();
      a.out_lp_ids[(int64_t)row * N + j] = 0xffffffffu;
    }
    if (tid == 0 && a.out_token_lp) a.out_token_lp[row] = eos ? 0.f : -__builtin_inff();
    return;
  }
  if (N > 0 && ranked_k < N) ranked_k = rank_candidates(fs, a, row, cfg, N, M);
  const double log_sum = log_sum_known == log_sum_known
                             ? log_sum_known
                             : log(block_sum_f64<NT>(logprob_part(fs, a, row, cfg, M, -1, tid, NT), fs.redd));
  for (int j = tid; j < N; j += NT) {
    float lp = -__builtin_inff();
    uint32_t id = 0xffffffffu;
    if (j < ranked_k) {
      id = cand_idx(fs.buf[j]);
      lp = (float)(((double)okey_inv(fs.pay[j]) - (double)M) - log_sum);
    }
    a.out_lp_ids[(int64_t)row * N + j] = id;
    a.out_lp[(int64_t)row * N + j] = lp;
  }
  if (a.out_token_lp) {
    if (tid == 0) fs.flag = 0u;
    __syncthreads();
    for (int j = tid; j < ranked_k; j += NT)
      if (cand_idx(fs.buf[j]) == token) { fs.flag = 1u; fs.fval1 = okey_inv(fs.pay[j]); }
    __syncthreads();
    float s;
    if (fs.flag) {
      s = fs.fval1;
    } else {
      const float l = processed_single<NT>(a, row, cfg, token < (uint32_t)V ? token : 0u, fs.redu);
      s = finitef_(l) ? l / cfg.t_eff : -__builtin_inff();
    }
    if (tid == 0)
      a.out_token_lp[row] = token < (uint32_t)V ? (float)(((double)s - (double)M) - log_sum) : -__builtin_inff();
  }
}

// ==========================================================================
// Lean finish (greedy rows; top-k rows with k_eff <= kLeanK)
// ==========================================================================
//
// The common case of the finish without its general machinery: every wave
// merges the chunk records on its own (no barrier), the candidates are
// gathered into LDS, a radix select that starts below their common high
// bits keeps the top k_sel, each thread ranks one of them by counting, and
// every wave runs the reference's sequential f32 folds from registers
// (readlane), so the draw is computed without a barrier either.  A row
// whose k_sel-th weight could tie with a logit outside the candidates, or
// whose fold hits the reference's argmax fallback, returns false and takes
// finish_row.

constexpr int kFinPer = kGather / NT;  // candidates each thread gathers

// Threshold T such that exactly k of item(0 .. n-1) (unique keys) are
// >= T, 1 <= k <= n: an 8-bit MSD radix select over the workgroup that
// starts below the common high bits of the keys' bounds lo <= key <= hi
// (lo > hi: the bounds are the keys' own minimum and maximum, found here).
// Two 256-bin histograms (hist[0, 512)) alternate, so a pass takes two
// barriers: counts, then the chosen bin.  All threads call it.  kmax > k
// asks for a threshold that keeps at least k and at most kmax keys (the
// passes stop at the first digit that allows it).
template <typename LoadF>
__device__ __forceinline__ uint64_t block_select_skip_f(LoadF item, int n, uint32_t k, uint32_t* hist, uint32_t* sel,
                                                        uint64_t* reda, uint64_t* redb, uint64_t lo = ~0ull,
                                                        uint64_t hi_b = 0ull, uint32_t kmax = 0u) {
  const uint32_t kcap = kmax > k ? kmax : k;
  const int tid = threadIdx.x;
  const int lane = tid & 63, wid = tid >> 6;
  uint64_t mn = lo, mx = hi_b;
  for (int b = tid; b < 256; b += NT) hist[b] = 0u;
  if (lo > hi_b) {
    mn = ~0ull;
    mx = 0ull;
    for (int i = tid; i < n; i += NT) {
      const uint64_t x = item(i);
      mn = x < mn ? x : mn;
      mx = x > mx ? x : mx;
    }
    mn = wave_min_u64(mn);
    mx = wave_max_u64(mx);
    if (lane == 0) { reda[wid] = mn; redb[wid] = mx; }
  }
  __syncthreads();  // also: hist[0, 256) is zero
  if (lo > hi_b) {
    mn = reda[0];
    mx = redb[0];
    #pragma unroll
    for (int w = 1; w < NT / 64; ++w) { mn = reda[w] < mn ? reda[w] : mn; mx = redb[w] > mx ? redb[w] : mx; }
  }
  if (mn == mx) return mx;
  int hi = 64 - __clzll(mn ^ mx);
  uint64_t prefix = hi >= 64 ? 0ull : (mx >> hi) << hi;
  uint32_t remaining = k;
  int cur = 0;
  #pragma unroll 1
  while (hi > 0) {
    const int db = hi >= 8 ? 8 : hi;
    const int lo_bit = hi - db;
    const uint64_t hp = hi >= 64 ? 0ull : (prefix >> hi);
    uint32_t* h = hist + cur * 256;
    uint32_t* o = hist + (cur ^ 1) * 256;  // the next pass's bins: last read before the previous barrier
    for (int b = tid; b < 256; b += NT) o[b] = 0u;
    for (int i = tid; i < n; i += NT) {
      const uint64_t x = item(i);
      if (hi >= 64 || (x >> hi) == hp) atomicAdd(&h[(uint32_t)(x >> lo_bit) & ((1u << db) - 1u)], 1u);
    }
    __syncthreads();
    if (tid < 64) {
      // lane l owns bins 255-4l .. 252-4l (descending)
      uint32_t loc[4], lsum = 0;
      #pragma unroll
      for (int q = 0; q < 4; ++q) { loc[q] = h[255 - 4 * tid - q]; lsum += loc[q]; }
      const uint32_t inc = wave_incl_scan_u32(lsum);
      const uint32_t above = inc - lsum;
      if (above < remaining && remaining <= above + lsum) {
        uint32_t acc = above;
        #pragma unroll
        for (int q = 0; q < 4; ++q) {
          if (remaining <= acc + loc[q] && acc < remaining) {
            sel[0] = 255u - 4u * tid - q; sel[1] = acc; sel[2] = loc[q];
          }
          acc += loc[q];
        }
      }
    }
    __syncthreads();
    // keys at or above the chosen bin's lower edge (with kcap == k the
    // exact stop: the bin holds exactly the keys still needed)
    const uint32_t kept = (k - remaining) + sel[1] + sel[2];
    prefix |= (uint64_t)sel[0] << lo_bit;
    remaining -= sel[1];
    hi = lo_bit;
    cur ^= 1;
    if (kept <= kcap) break;
  }
  return prefix;
}

// block_select_skip_f over items[0, n) (LDS or global memory).
__device__ __forceinline__ uint64_t block_select_skip(const uint64_t* items, int n, uint32_t k, uint32_t* hist,
                                                      uint32_t* sel, uint64_t* reda, uint64_t* redb,
                                                      uint64_t lo = ~0ull, uint64_t hi_b = 0ull) {
  return block_select_skip_f([&](int i) { return items[i]; }, n, k, hist, sel, reda, redb, lo, hi_b);
}

// block_select_skip for n <= 64 * PER items, by one wave: the keys in
// registers, a 256-bin histogram in `hist` that only this wave touches, and
// no barrier (LDS operations of one wave complete in order).  Same result.
//
// kmax > k asks for a threshold that keeps at least k and at most kmax
// keys (the radix passes stop at the first digit that allows it).
// wave_select_skip_r takes the keys from registers (entry m * 64 + lane in
// x[m], entries from n on ignored).
template <int PER>
__device__ __forceinline__ uint64_t wave_select_skip_r(const uint64_t (&x)[PER], int n, uint32_t k, uint32_t* hist,
                                                       uint64_t lo, uint64_t hi_b, uint32_t kmax = 0u) {
  const int lane = threadIdx.x & 63;
  const uint32_t kcap = kmax > k ? kmax : k;
  uint64_t mn = ~0ull, mx = 0ull;
  #pragma unroll
  for (int m = 0; m < PER; ++m) {
    if (m * 64 + lane < n) {
      mn = x[m] < mn ? x[m] : mn;
      mx = x[m] > mx ? x[m] : mx;
    }
  }
  if (lo > hi_b) {
    mn = wave_min_u64(mn);
    mx = wave_max_u64(mx);
  } else {
    mn = lo;
    mx = hi_b;
  }
  if (mn == mx) return mx;
  int hi = 64 - __clzll(mn ^ mx);
  uint64_t prefix = hi >= 64 ? 0ull : (mx >> hi) << hi;
  uint32_t remaining = k;
  #pragma unroll 1
  while (hi > 0) {
    const int db = hi >= 8 ? 8 : hi;
    const int lo_bit = hi - db;
    const uint64_t hp = hi >= 64 ? 0ull : (prefix >> hi);
    #pragma unroll
    for (int q = 0; q < 4; ++q) hist[lane * 4 + q] = 0u;
    #pragma unroll
    for (int m = 0; m < PER; ++m)
      if (m * 64 + lane < n && (hi >= 64 || (x[m] >> hi) == hp))
        atomicAdd(&hist[(uint32_t)(x[m] >> lo_bit) & ((1u << db) - 1u)], 1u);
    // lane l owns bins 255-4l .. 252-4l (descending)
    uint32_t loc[4], lsum = 0u;
    #pragma unroll
    for (int q = 0; q < 4; ++q) { loc[q] = hist[255 - 4 * lane - q]; lsum += loc[q]; }
    const uint32_t inc = wave_incl_scan_u32(lsum);
    const uint32_t above = inc - lsum;
    const bool mine = above < remaining && remaining <= above + lsum;
    uint32_t d = 0u, acc_b = 0u, cnt = 0u;
    if (mine) {
      uint32_t acc = above;
      #pragma unroll
      for (int q = 0; q < 4; ++q) {
        if (remaining <= acc + loc[q] && acc < remaining) { d = 255u - 4u * (uint32_t)lane - (uint32_t)q; acc_b = acc; cnt = loc[q]; }
        acc += loc[q];
      }
    }
    const int owner = __ffsll((unsigned long long)__ballot(mine)) - 1;
    d = (uint32_t)__builtin_amdgcn_readlane((int)d, owner);
    acc_b = (uint32_t)__builtin_amdgcn_readlane((int)acc_b, owner);
    cnt = (uint32_t)__builtin_amdgcn_readlane((int)cnt, owner);
    // keys at or above the boundary bin's lower edge (with kcap == k this
    // is the exact stop: the bin holds exactly the keys still needed)
    const uint32_t kept = (k - remaining) + acc_b + cnt;
    prefix |= (uint64_t)d << lo_bit;
    remaining -= acc_b;
    hi = lo_bit;
    if (kept <= kcap) break;
  }
  return prefix;
}
template <int PER, typename LoadF>
__device__ __forceinline__ uint64_t wave_select_skip_f(LoadF item, int n, uint32_t k, uint32_t* hist,
                                                       uint64_t lo, uint64_t hi_b, uint32_t kmax = 0u) {
  const int lane = threadIdx.x & 63;
  uint64_t x[PER];
  #pragma unroll
  for (int m = 0; m < PER; ++m) {
    const int i = m * 64 + lane;
    x[m] = i < n ? item(i) : 0ull;
  }
  return wave_select_skip_r<PER>(x, n, k, hist, lo, hi_b, kmax);
}
template <int PER>
__device__ __forceinline__ uint64_t wave_select_skip(const uint64_t* items, int n, uint32_t k, uint32_t* hist,
                                                     uint64_t lo, uint64_t hi_b) {
  return wave_select_skip_f<PER>([&](int i) { return items[i]; }, n, k, hist, lo, hi_b);
}

constexpr int kLeanChunks = 256;  // chunks per row the lean finish merges
constexpr int kSpecChunks = 40;   // rows of up to this many chunks load their candidates early

// Reference steps 7-10 (gpu.rs:831-899) over the rank order held in
// registers: entry m * 64 + lane of the rank keys sits in lane `lane` of
// kr[m], entries [0, k) are the kept ones (k <= 64 * DM).  Returns the
// drawn entry, or -1 for the reference's argmax_host fallback (no positive
// weight, or a total or candidate total that is not positive and finite).
// Wave-local: every wave that calls it returns the same, with no barrier.
template <int DM>
__device__ __forceinline__ int wave_draw_r(const uint64_t (&kr)[DM], int k, const RowCfg& cfg) {
  const uint32_t lane = threadIdx.x & 63u;
  float fa[DM], pa[DM];
  #pragma unroll
  for (int m = 0; m < DM; ++m) {
    const int i = m * 64 + (int)lane;
    const float w = i < k ? rank_w(kr[m]) : 0.f;
    fa[m] = w < cfg.min_p ? 0.f : w;  // min-p: excluded like w <= 0 (gpu.rs:847-849)
  }
  // the weights are in rank order, so the positive ones are a prefix
  // [0, last_pos] (min-p and underflow zeros sit at the end)
  int last_pos = -1;
  #pragma unroll
  for (int m = 0; m < DM; ++m) {
    const int i = m * 64 + (int)lane;
    const uint64_t pm = __ballot(i < k && fa[m] > 0.f);
    if (pm != 0ull) last_pos = m * 64 + 63 - __clzll((unsigned long long)pm);
  }
  if (last_pos < 0) return -1;  // no candidate: argmax_host fallback
  // P_i: the sequential sum of fa[0..i]: the total of gpu.rs:834-836 (the
  // kept weights in rank order; the zeros after last_pos add nothing) and,
  // at positive entries, the candidate total and CDF of gpu.rs:874-896
  const int kp = last_pos + 1;
  float P = -0.0f;
  #pragma unroll
  for (int m = 0; m < DM; ++m) {
    if (m * 64 < kp) {
      pa[m] = wave_fold_f32(fa[m], P, min(64, kp - m * 64));
      P = __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(pa[m]), min(63, kp - 1 - m * 64)));
    } else {
      pa[m] = P;
    }
  }
  const float total = P;
  if (!(total > 0.f) || !finitef_(total)) return -1;  // argmax_host fallback
  // the nucleus: cum_p over w / total of the positive entries (gpu.rs:843-856),
  // folded slot by slot as far as the slot where it reaches the cutoff (a
  // check per slot, not per step: each check is a round trip through the
  // scalar unit)
  int cut = -1;  // first positive entry where cum_p reaches the cutoff
  if (cfg.cutoff < 1.f) {
    float Q = 0.f;
    #pragma unroll
    for (int m = 0; m < DM; ++m) {
      if (cut < 0 && m * 64 < kp) {
        const int i = m * 64 + (int)lane;
        const bool pos = i < kp;
        const float fb = pos ? fa[m] / total : 0.f;
        const float q = wave_fold_f32(fb, Q, min(64, kp - m * 64));
        const uint64_t hm = __ballot(pos && q >= cfg.cutoff);
        if (hm != 0ull) cut = m * 64 + __ffsll((unsigned long long)hm) - 1;
        else Q = __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(q), min(63, kp - 1 - m * 64)));
      }
    }
  }
  const int m_end = cut >= 0 ? cut + 1 : last_pos + 1;
  const int me = m_end - 1;
  float ct = 0.f;
  #pragma unroll
  for (int m = 0; m < DM; ++m)
    if ((me >> 6) == m) ct = __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(pa[m]), me & 63));
  if (!(ct > 0.f) || !finitef_(ct)) return -1;
  // inverse CDF: the first candidate whose cumulative weight passes target
  const float target = clamp_uniform(cfg.u) * ct;
  int pick = -1;
  #pragma unroll
  for (int m = 0; m < DM; ++m) {
    const int i = m * 64 + (int)lane;
    const uint64_t hit = __ballot(i < m_end && fa[m] > 0.f && target < pa[m]);
    if (pick < 0 && hit != 0ull) pick = m * 64 + __ffsll((unsigned long long)hit) - 1;
  }
  return pick < 0 ? me : pick;
}

// wave_draw_r over the rank order keys[0, k) in LDS (k <= 64 * DM), by
// every wave from registers.
template <int DM>
__device__ __forceinline__ int wave_draw(const uint64_t* keys, int k, const RowCfg& cfg) {
  const uint32_t lane = threadIdx.x & 63u;
  uint64_t kr[DM];
  #pragma unroll
  for (int m = 0; m < DM; ++m) {
    const int i = m * 64 + (int)lane;
    kr[m] = i < k ? keys[i] : 0ull;
  }
  return wave_draw_r<DM>(kr, k, cfg);
}


// The rank (entries above it) of this lane's key among the wave's keys
// (zero keys count for nothing): over the lanes of km one at a time, or,
// for many, over all 64 lanes in an unrolled loop of independent compares.
__device__ __forceinline__ uint32_t wave_rank_desc(uint64_t x, uint64_t km) {
  uint32_t r = 0u;
  if (__popcll(km) <= 16) {
    for (uint64_t mm = km; mm != 0ull; mm &= mm - 1ull)
      r += readlane64(x, __builtin_ctzll(mm)) > x ? 1u : 0u;
    return r;
  }
  uint32_t r1 = 0u, r2 = 0u, r3 = 0u;
  #pragma unroll
  for (int j = 0; j < 64; j += 4) {
    r += readlane64(x, j) > x ? 1u : 0u;
    r1 += readlane64(x, j + 1) > x ? 1u : 0u;
    r2 += readlane64(x, j + 2) > x ? 1u : 0u;
    r3 += readlane64(x, j + 3) > x ? 1u : 0u;
  }
  return (r + r1) + (r2 + r3);
}

// Descending sort of the wave's 64 * S keys, entry m * 64 + lane in x[m]:
// a bitonic network whose compare-exchanges between slots stay in a lane's
// registers and whose exchanges between lanes are lane_xor64 moves.
template <int S>
__device__ __forceinline__ void wave_sort_desc(uint64_t (&x)[S]) {
  const uint32_t lane = threadIdx.x & 63u;
  constexpr int N = 64 * S;
  #pragma unroll
  for (int k = 2; k <= N; k <<= 1) {
    #pragma unroll
    for (int j = k >> 1; j > 0; j >>= 1) {
      if (j >= 64) {
        const int js = j >> 6;
        #pragma unroll
        for (int m = 0; m < S; ++m) {
          if (m & js) continue;
          // the lower entry of the pair keeps the larger key when (i & k) == 0
          // (a compile-time choice here)
          const uint64_t lo = x[m], hi = x[m ^ js];
          const uint64_t mx = hi > lo ? hi : lo, mn = hi > lo ? lo : hi;
          const bool desc = ((m * 64) & k) == 0;
          x[m] = desc ? mx : mn;
          x[m ^ js] = desc ? mn : mx;
        }
      } else {
        #pragma unroll
        for (int m = 0; m < S; ++m) {
          const uint32_t i = (uint32_t)m * 64u + lane;
          const uint64_t y = lane_xor64(x[m], j);
          // keep the partner's key when it is larger and this entry keeps
          // the maximum, or smaller and it keeps the minimum: an all-ones or
          // all-zero mask, so the exchange is a select with no branch
          const uint32_t keep_max = (((i & (uint32_t)k) == 0u) == ((i & (uint32_t)j) == 0u)) ? 1u : 0u;
          const uint32_t gt = y > x[m] ? 1u : 0u;
          const uint64_t take = 0ull - (uint64_t)(1u ^ gt ^ keep_max);
          x[m] = (y & take) | (x[m] & ~take);
        }
      }
    }
  }
}

// wave_draw by wave 0 alone, the pick handed to every thread: the folds are
// serial chains, and copies of them in the other waves would only take
// issue slots from wave 0 on the shared SIMDs.  Ends with a barrier.
template <int DM>
__device__ __forceinline__ int wg_draw(FinLds& fs, const uint64_t* keys, int k, const RowCfg& cfg) {
  if (threadIdx.x < 64u) {
    const int pick = wave_draw<DM>(keys, k, cfg);
    if (threadIdx.x == 0u) fs.pick = pick;
  }
  __syncthreads();
  return fs.pick;
}

// Reference steps 7-10 (gpu.rs:831-899) over the first k <= kBuf entries of
// the rank order in fs.buf (top-k rows).  Returns the token, or 0xffffffff
// for "fall back to argmax_host".
__device__ __forceinline__ uint32_t draw_topk(FinLds& fs, const RowCfg& cfg, int k) {
  const int pick = wg_draw<kBuf / 64>(fs, fs.buf, k, cfg);
  return pick < 0 ? 0xffffffffu : cand_idx(fs.buf[pick]);
}

// finish_core for at most 64 selected candidates (kk <= 64, n <= 64 PER) on
// wave 0 alone, from registers: the one-wave select, the selection, the
// weights and tie checks, the rank order by counting and the draw, with no
// workgroup barrier; meanwhile the other waves add up the candidates'
// logprob terms.  One barrier at the end publishes the result; the
// logprobs are then written by every thread.  Same result as the
// workgroup steps.  The select first bounds the kk-th key by the kk-th
// largest of the lanes' maxima and, when at most 128 keys reach that bound,
// sorts them in registers.  On entry fs.nparts is zero and fs.exptab holds
// exact_expf's table (finish_lean sets both).
constexpr int kWavePer = 20;  // candidates per lane of finish_core_wave (n <= 1280)

// The keys of x[0, S) (entry m * 64 + lane in x[m], entries from n on
// ignored) that reach thr, written to buf[0, min(count, 128)) in lane-major
// order (a lane's keys together); returns the count.  Every lane writes
// every slot (the ones left out, and kept ones past 128, to its own word
// buf[128 + lane]), so the writes take no branch; buf holds 192 keys.
template <int S>
__device__ __forceinline__ uint32_t wave_keep_into(const uint64_t (&x)[S], int n, uint64_t thr, uint64_t* buf) {
  const uint32_t lane = threadIdx.x & 63u;
  uint32_t c = 0u;
  #pragma unroll
  for (int m = 0; m < S; ++m) c += (m * 64 + (int)lane < n && x[m] >= thr) ? 1u : 0u;
  const uint32_t incl = wave_incl_scan_u32(c);
  uint32_t at = incl - c;
  const uint32_t spare = 128u + lane;
  #pragma unroll
  for (int m = 0; m < S; ++m) {
    const bool k = m * 64 + (int)lane < n && x[m] >= thr;
    buf[k && at < 128u ? at : spare] = x[m];
    at += k ? 1u : 0u;
  }
  return (uint32_t)__builtin_amdgcn_readlane((int)incl, 63);
}

// The largest of x[0, S) under thr (0: none).
template <int S>
__device__ __forceinline__ uint64_t wave_max_below(const uint64_t (&x)[S], int n, uint64_t thr) {
  const uint32_t lane = threadIdx.x & 63u;
  uint64_t b = 0ull;
  #pragma unroll
  for (int m = 0; m < S; ++m)
    if (m * 64 + (int)lane < n && x[m] < thr) b = x[m] > b ? x[m] : b;
  return wave_max_u64(b);
}

template <int PER>
__device__ __forceinline__ bool finish_core_wave(FinLds& fs, const SampleArgs& a, int row, const RowCfg& cfg, int n,
                                                 float M, uint32_t ub_key, double part, uint32_t above, uint64_t lo,
                                                 uint64_t hi) {
  const int tid = threadIdx.x;
  const uint32_t lane = (uint32_t)tid & 63u;
  const int wid = tid >> 6;
  const bool want_lp = a.n_lp > 0 || a.out_token_lp != nullptr;
  const int kk = min(cfg.k_sel, n);
  if (wid == 0) {
    uint32_t status = 0u;  // 1: the workgroup finish (finish_row) takes the row
    uint64_t xr[PER];
    #pragma unroll
    for (int m = 0; m < PER; ++m) {
      const int i = m * 64 + (int)lane;
      xr[m] = i < n ? fs.cbig[i] : 0ull;
    }
    // 4. the top kk by (processed logit desc, index asc) (keys are
    //    distinct), in lanes [0, kk) of y[0], sorted when `sorted`; below
    //    is the largest key left out.  A first bound: the kk-th largest of
    //    the lanes' maxima (more than kk lanes hold a key when n > kk, and
    //    their maxima are distinct), so at least kk keys reach it; when at
    //    most 128 do, they are sorted in registers
    uint64_t y[1] = {0ull};
    uint64_t below = 0ull;
    bool sorted = true;
    if (n <= kk) {
      y[0] = xr[0];
      wave_sort_desc<1>(y);
    } else {
      uint64_t lmx[1] = {0ull};
      #pragma unroll
      for (int m = 0; m < PER; ++m) lmx[0] = xr[m] > lmx[0] ? xr[m] : lmx[0];
      wave_sort_desc<1>(lmx);
      const uint64_t g = readlane64(lmx[0], kk - 1);
      const uint32_t n2 = wave_keep_into<PER>(xr, n, g, fs.buf);
      wave_lds_sync();
      if (n2 <= 64u) {
        y[0] = (int)lane < (int)n2 ? fs.buf[lane] : 0ull;
        wave_sort_desc<1>(y);
        below = (int)n2 > kk ? readlane64(y[0], kk) : wave_max_below<PER>(xr, n, g);
      } else if (n2 <= 128u) {
        uint64_t y2[2];
        #pragma unroll
        for (int m = 0; m < 2; ++m) y2[m] = m * 64 + (int)lane < (int)n2 ? fs.buf[m * 64 + lane] : 0ull;
        wave_sort_desc<2>(y2);
        y[0] = y2[0];
        below = kk < 64 ? readlane64(y2[0], kk) : readlane64(y2[1], 0);
      } else {
        wave_lds_sync();
        const uint64_t thr = wave_select_skip_r<PER>(xr, n, (uint32_t)kk, fs.hist, lo, hi);
        wave_keep_into<PER>(xr, n, thr, fs.buf);
        below = wave_max_below<PER>(xr, n, thr);
        wave_lds_sync();
        y[0] = (int)lane < kk ? fs.buf[lane] : 0ull;
        sorted = false;
      }
    }
    const uint64_t x = (int)lane < kk ? y[0] : 0ull;
    const uint64_t thr = sorted ? readlane64(x, kk - 1) : wave_min_u64((int)lane < kk ? x : ~0ull);  // the kk-th key
    if (n > kk && cand_skey(thr) <= above) status = 1u;
    // 5. weights and rank keys; the smallest selected weight w_b
    uint64_t rk = 0ull;
    uint32_t pk = 0u, wbits = 0xffffffffu;
    const Exp2TabLds tab{fs.exptab};
    if ((int)lane < kk) {
      const float sx = key_to_s(cand_skey(x), cfg.t_eff);
      const float w = exact_expf_t(sx - M, tab);
      rk = rank_key(w, cand_idx(x));
      pk = okey(sx);
      wbits = __float_as_uint(w);
    }
    const float w_b = __uint_as_float(wave_reduce32(wbits, 0xffffffffu, [](uint32_t p, uint32_t q) { return p < q ? p : q; }));
    // 6. could a logit outside the selection tie with w_b?
    const uint32_t xk = max(ub_key, below != 0ull ? cand_skey(below) : 0u);
    if (w_b > 0.f && xk > kKeyNegInf && exact_expf_t(key_to_s(xk, cfg.t_eff) - M, tab) == w_b) status = 1u;
    // 7. rank order: weights are monotone in the key, so in key order they
    //    are the rank order unless two neighbours weigh the same (then, and
    //    for an unsorted selection, by counting: rank keys are distinct,
    //    each entry moved to the lane of its rank)
    uint64_t yr[1] = {rk};
    uint32_t yp = pk;
    const uint32_t wprev = dpp32<0x138, 0xf, true>(0u, wbits);  // wave_shr:1: lane l - 1's weight
    if (!sorted || __ballot(lane >= 1u && (int)lane < kk && wbits == wprev) != 0ull) {
      const uint64_t km = __ballot((int)lane < kk);
      const uint32_t r = wave_rank_desc(rk, km);
      const int to = (int)lane < kk ? (int)(r * 4u) : 63 * 4;  // the other lanes write past kk or nowhere
      const uint32_t ylo = (uint32_t)__builtin_amdgcn_ds_permute(to, (int)(uint32_t)rk);
      const uint32_t yhi = (uint32_t)__builtin_amdgcn_ds_permute(to, (int)(uint32_t)(rk >> 32));
      yp = (uint32_t)__builtin_amdgcn_ds_permute(to, (int)pk);
      yr[0] = (int)lane < kk ? ((uint64_t)yhi << 32) | ylo : 0ull;
    }
    if ((int)lane < kk) {
      fs.buf[lane] = yr[0];
      fs.pay[lane] = yp;
    }
    // 8. the draw (gpu.rs:831-899)
    int pick = -1;
    if (status == 0u) {
      pick = wave_draw_r<1>(yr, min(cfg.k_eff, kk), cfg);
      if (pick < 0) status = 1u;  // argmax_host fallback
    }
    if (lane == 0u) {
      if (status == 0u) a.out_tokens[row] = cand_idx(readlane64(yr[0], pick));
      fs.flag = status;
      fs.pick = pick;
    }
  } else if (want_lp) {
    // the candidates' share of the logprob normaliser, in double, added to
    // the caller's share (wave 1's lanes); the last of these waves to end
    // takes the log of the sum
    for (int j = tid - 64; j < n; j += NT - 64) {
      const uint32_t kv = cand_skey(fs.cbig[j]);
      if (kv > kKeyNegInf) part += exp((double)key_to_s(kv, cfg.t_eff) - (double)M);
    }
    part = wave_sum_f64(part);
    if (lane == 0u) {
      fs.redd[wid] = part;
      const uint32_t done = __hip_atomic_fetch_add(&fs.nparts, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_WORKGROUP);
      if (done == (uint32_t)(NT / 64 - 2)) {
        double tot = 0.0;
        #pragma unroll
        for (int v = 1; v < NT / 64; ++v) tot += __hip_atomic_load(&fs.redd[v], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        fs.lsum = log(tot);
      }
    }
  }
  __syncthreads();
  if (fs.flag != 0u) return false;
  if (!want_lp) return true;
  // 9. logprobs of the processed distribution (extension)
  const double log_sum = fs.lsum;
  const int N = a.n_lp;
  for (int j = tid; j < N; j += NT) {
    float lp = -__builtin_inff();
    uint32_t id = 0xffffffffu;
    if (j < kk) {
      id = cand_idx(fs.buf[j]);
      lp = (float)(((double)okey_inv(fs.pay[j]) - (double)M) - log_sum);
    }
    a.out_lp_ids[(int64_t)row * N + j] = id;
    a.out_lp[(int64_t)row * N + j] = lp;
  }
  if (a.out_token_lp && tid == 0)
    a.out_token_lp[row] = (float)(((double)okey_inv(fs.pay[fs.pick]) - (double)M) - log_sum);
  return true;
}

// Steps 4-9 of the lean finish over the candidates fs.cbig[0, n) of `row`
// (candidate keys, any order; n >= 1).  M is the row max of s; ub_key bounds
// the processed-logit keys of the row's logits that are not candidates (0:
// none); part is this thread's share of the logprob normaliser over those
// logits (double, relative to M); when n exceeds the selection size, its
// last key must be above `above`; lo <= hi bound the candidates' keys when
// the caller knows them (lo > hi: unknown).  Returns false when the row needs the
// general finish; all threads return the same.
__device__ __forceinline__ bool finish_core(FinLds& fs, const SampleArgs& a, int row, const RowCfg& cfg, int n,
                                            float M, uint32_t ub_key, double part, uint32_t above = 0u,
                                            uint64_t lo = ~0ull, uint64_t hi = 0ull, bool one_wave_select = true) {
  if (one_wave_select && min(cfg.k_sel, n) <= 64 && n <= 64 * kWavePer)
    return finish_core_wave<kWavePer>(fs, a, row, cfg, n, M, ub_key, part, above, lo, hi);
  const int tid = threadIdx.x;
  const uint32_t lane = (uint32_t)tid & 63u;
  const bool want_lp = a.n_lp > 0 || a.out_token_lp != nullptr;
  if (want_lp) {
    // the candidates' share, in double (fixed order)
    for (int j = tid; j < n; j += NT) {
      const uint32_t kv = cand_skey(fs.cbig[j]);
      if (kv > kKeyNegInf) part += exp((double)key_to_s(kv, cfg.t_eff) - (double)M);
    }
  }

  // 4. the top kk by (processed logit desc, index asc)
  const int kk = min(cfg.k_sel, n);
  uint64_t thr = 0ull;
  if (tid == 0) { fs.counter = 0u; fs.below = 0ull; fs.wmin = 0xffffffffu; }
  if (one_wave_select && n > kk && n <= 1024) {
    // one wave selects; the barrier publishes the threshold
    if (tid < 64) {
      const uint64_t t = wave_select_skip<16>(fs.cbig, n, (uint32_t)kk, fs.hist, lo, hi);
      if (tid == 0) fs.thr = t;
    }
    __syncthreads();
    thr = fs.thr;
  } else if (n > kk) {
    thr = block_select_skip(fs.cbig, n, (uint32_t)kk, fs.hist, fs.sel, fs.red64, fs.red64b, lo, hi);
  } else {
    __syncthreads();  // the counters above are set
  }
  // the caller's candidates hold the row's top kk only if the kk-th key is
  // above `above` (the largest key the caller may have left out)
  if (n > kk && cand_skey(thr) <= above) return false;
  // the selection into fs.buf and the largest candidate left out, both
  // complete at one barrier (one LDS atomic per wave: same-address atomics
  // of every lane would be serialised)
  {
    uint32_t c = 0u;
    uint64_t below = 0ull;
    for (int j = tid; j < n; j += NT) {
      const uint64_t x = fs.cbig[j];
      c += x >= thr ? 1u : 0u;
      if (x < thr) below = x > below ? x : below;
    }
    const uint32_t incl = wave_incl_scan_u32(c);
    uint32_t base = 0u;
    if (lane == 63u) base = atomicAdd(&fs.counter, incl);
    uint32_t at = (uint32_t)__builtin_amdgcn_readlane((int)base, 63) + incl - c;
    for (int j = tid; j < n; j += NT) {
      const uint64_t x = fs.cbig[j];
      if (x >= thr) fs.buf[at++] = x;
    }
    below = wave_max_u64(below);
    if (lane == 0u && below != 0ull) atomicMax((unsigned long long*)&fs.below, (unsigned long long)below);
  }
  __syncthreads();
  const uint64_t below = fs.below;  // largest candidate left out (0: none)

  // 5. weights and rank keys; the smallest selected weight w_b
  uint64_t rk = 0ull;
  uint32_t pk = 0u;
  uint32_t wnot = 0u;  // ~(bits of w): w >= 0, so its bits order as the value
  if (tid < kk) {
    const uint64_t x = fs.buf[tid];
    const float sx = key_to_s(cand_skey(x), cfg.t_eff);
    const float w = exact_expf(sx - M);
    rk = rank_key(w, cand_idx(x));
    pk = okey(sx);
    wnot = ~__float_as_uint(w);
    fs.buf[tid] = rk;
    fs.hist[tid] = 0u;  // its rank, summed in step 7
  }
  if (tid < ((kk + 63) & ~63)) {
    wnot = wave_max_u32(wnot);
    if (lane == 0u) atomicMin(&fs.wmin, ~wnot);
  }
  __syncthreads();
  const float w_b = __uint_as_float(fs.wmin);
  // 6. could a logit outside the selection tie with w_b?  Weights are
  //    monotone in the key, so the largest excluded key decides (finish_row
  //    resolves those rows exactly).
  const uint32_t xk = max(ub_key, below != 0ull ? cand_skey(below) : 0u);
  if (w_b > 0.f && xk > kKeyNegInf && exact_expf(key_to_s(xk, cfg.t_eff) - M) == w_b) return false;

  // 7. rank order by counting: an entry's rank is the number of rank keys
  //    above its own.  `parts` threads share each entry's count (every
  //    thread works when kk <= NT / 2), reading two keys per LDS read; the
  //    parts add up in LDS.
  {
    const int parts = kk <= NT / 4 ? 4 : (kk <= NT / 2 ? 2 : 1);
    const int G = NT / parts;
    const int e = tid % G, part = tid / G;
    if (e < kk) {
      const uint64_t me = fs.buf[e];
      const int span = ((kk + parts - 1) / parts + 1) & ~1;  // even: 16-byte reads
      const int j0 = part * span, j1 = min(kk, j0 + span);
      uint32_t r = 0u;
      int j = j0;
      #pragma unroll 4
      for (; j + 2 <= j1; j += 2) {
        const ulonglong2 y = *reinterpret_cast<const ulonglong2*>(&fs.buf[j]);
        r += (y.x > me ? 1u : 0u) + (y.y > me ? 1u : 0u);
      }
      if (j < j1) r += fs.buf[j] > me ? 1u : 0u;
      if (parts == 1) {
        fs.cbig[r] = rk;
        fs.aux[r] = pk;
      } else if (r != 0u) {
        atomicAdd(&fs.hist[e], r);
      }
    }
    if (parts > 1) {
      __syncthreads();
      if (tid < kk) {
        const uint32_t r = fs.hist[tid];
        fs.cbig[r] = rk;
        fs.aux[r] = pk;
      }
    }
  }
  __syncthreads();

  // 8. the draw (gpu.rs:831-899)
  const int pick = wg_draw<kLeanK / 64>(fs, fs.cbig, min(cfg.k_eff, kk), cfg);
  if (pick < 0) return false;  // argmax_host fallback
  const uint32_t token = cand_idx(fs.cbig[pick]);
  if (tid == 0) a.out_tokens[row] = token;
  if (!want_lp) return true;

  // 9. logprobs of the processed distribution (extension)
  const double log_sum = log(block_sum_f64<NT>(part, fs.redd));
  const int N = a.n_lp;
  for (int j = tid; j < N; j += NT) {
    float lp = -__builtin_inff();
    uint32_t id = 0xffffffffu;
    if (j < kk) {
      id = cand_idx(fs.cbig[j]);
      lp = (float)(((double)okey_inv(fs.aux[j]) - (double)M) - log_sum);
    }
    a.out_lp_ids[(int64_t)row * N + j] = id;
    a.out_lp[(int64_t)row * N + j] = lp;
  }
  if (a.out_token_lp && tid == 0)
    a.out_token_lp[row] = (float)(((double)okey_inv(fs.aux[pick]) - (double)M) - log_sum);
  return true;
}

// Lean finish of the chunk pass: merges the chunk records and gathers their
// candidates, then finish_core.
__device__ __forceinline__ bool finish_lean(FinLds& fs, const SampleArgs& a, int row, const RowCfg& cfg) {
  const int tid = threadIdx.x;
  const uint32_t lane = (uint32_t)tid & 63u;
  const bool want_lp = a.n_lp > 0 || a.out_token_lp != nullptr;
  if (cfg.cls == kGreedy) {
    if (want_lp) return false;
  } else if (cfg.cls != kTopK || cfg.wide) {
    return false;
  }
  const int nch = a.n_chunks;
  if (nch > kLeanChunks) return false;
  const ChunkStat* stats = a.stats + (int64_t)row * nch;
  const uint64_t* cand = a.cand + (int64_t)row * nch * kFast;

  // 0. rows of few chunks: the first 64 candidate slots of every chunk are
  //    loaded before the records arrive (one round trip for both; wave w
  //    takes chunks w, w + 4, ...); the counts in the records then say which
  //    slots are candidates
  constexpr int kSpecPer = kSpecChunks / (NT / 64);
  const bool spec = nch <= kSpecChunks;
  const uint64_t et = tid < 32 ? exp2_tab32((uint32_t)tid) : 0ull;  // for fs.exptab
  uint64_t sp[kSpecPer];
  if (spec) {
    #pragma unroll
    for (int i = 0; i < kSpecPer; ++i) {
      const int c = (tid >> 6) + (NT / 64) * i;
      sp[i] = c < nch ? cand[(int64_t)c * kFast + lane] : 0ull;
    }
  }

  // 1. the chunk records, merged by every wave on its own; candidate counts
  //    and their chunk-major offsets; the largest key left out of them
  constexpr int CQ = kLeanChunks / 64;
  float mx = -__builtin_inff();
  uint32_t anyf = 0u, ub = 0u;
  float iv = -__builtin_inff(), fv = -__builtin_inff();
  uint32_t ii = 0xffffffffu, fi = 0xffffffffu;
  uint32_t cnt[CQ];
  double part = 0.0;  // the other logits' share of the logprob normaliser
  #pragma unroll
  for (int q = 0; q < CQ; ++q) {
    const int c = q * 64 + (int)lane;
    cnt[q] = 0u;
    if (c >= nch) continue;
    const ChunkStat& cs = stats[c];
    cnt[q] = cs.n_cand;
    mx = fmaxf(mx, cs.max_l);
    anyf |= cs.any_finite;
    if (cs.trunc) ub = max(ub, cs.unkept_key);
    if (cs.am_ieee_i != 0xffffffffu &&
        (ii == 0xffffffffu || cs.am_ieee_v > iv || (cs.am_ieee_v == iv && cs.am_ieee_i < ii))) {
      iv = cs.am_ieee_v; ii = cs.am_ieee_i;
    }
    if (cs.am_fin_i != 0xffffffffu) {
      bool take = fi == 0xffffffffu || cs.am_fin_v > fv;
      if (!take && cs.am_fin_v == fv) take = fin_order(cs.am_fin_i) < fin_order(fi);
      if (take) { fv = cs.am_fin_v; fi = cs.am_fin_i; }
    }
  }
  mx = wave_max_f32(mx);
  anyf = wave_reduce32(anyf, 0u, [](uint32_t x, uint32_t y) { return x | y; });
  ub = wave_max_u32(ub);
  // argmax merges as 64-bit keys: IEEE (value desc, index asc) and the
  // finite-lane rule (value desc, then fin_order asc)
  {
    // -0 and +0 compare equal under IEEE '>': both map to the +0 key
    const float iz = iv == 0.f ? 0.f : iv;
    const uint64_t ik = ii == 0xffffffffu ? 0ull
                        : ((uint64_t)okey(iz) << 32) | (uint64_t)(0xffffffffu - ii);
    const uint64_t best = wave_max_u64(ik);
    ii = best == 0ull ? 0xffffffffu : 0xffffffffu - (uint32_t)best;
  }
  {
    const float fz = fv == 0.f ? 0.f : fv;
    const uint64_t fk = fi == 0xffffffffu ? 0ull
                        : ((uint64_t)okey(fz) << 32) | (uint64_t)(0xffffffffu - fin_order(fi));
    const uint64_t best = wave_max_u64(fk);
    fi = best == 0ull ? 0xffffffffu : fin_index(0xffffffffu - (uint32_t)best);
  }
  const bool eos = a.mask && !anyf;
  if (cfg.cls == kGreedy) {
    if (tid == 0) {
      const uint32_t am = a.pv.greedy_rule == kGreedyFiniteLane ? fi : ii;
      a.out_tokens[row] = eos ? cfg.eos : (am == 0xffffffffu ? 0u : am);
    }
    return true;
  }
  const float M = finitef_(mx) ? mx / cfg.t_eff : -__builtin_inff();
  if (eos || !finitef_(M)) return false;
  if (want_lp && tid >= 64 && tid < 128) {  // wave 1 (finish_core_wave's first adder)
    #pragma unroll
    for (int q = 0; q < CQ; ++q) {
      const int c = q * 64 + (int)lane;
      if (c >= nch) continue;
      const ChunkStat& cs = stats[c];
      if (cs.lse_sum > 0.f) part += (double)cs.lse_sum * exp((double)cs.lse_m - (double)M);
    }
  }
  uint32_t offq[CQ];  // exclusive offset of chunk q * 64 + lane
  uint32_t n_total = 0u;
  #pragma unroll
  for (int q = 0; q < CQ; ++q) {
    const uint32_t incl = wave_incl_scan_u32(cnt[q]);
    offq[q] = n_total + incl - cnt[q];
    n_total += wave_last_u32(incl);
  }
  if (n_total > (uint32_t)kGather || n_total == 0u) return false;
  // chunks keep fewer than k_sel candidates when the row has many: with a
  // chunk truncated, fewer than k_sel candidates cannot hold the top k_sel
  if (ub != 0u && n_total < (uint32_t)cfg.k_sel) return false;
  if (tid < 64) {
    #pragma unroll
    for (int q = 0; q < CQ; ++q) if (q * 64 + (int)lane < nch) fs.aux[q * 64 + lane] = offq[q];
    if (lane == 0u) {
      fs.aux[nch] = n_total;
      fs.nparts = 0u;
    }
    if (lane < 32u) fs.exptab[lane] = et;
  }
  __syncthreads();

  // 2. the candidates into LDS (chunk-major): all loads first
  if (spec) {
    // (every wave holds every chunk's offset and count: lane c of offq[0]
    // and cnt[0], nch <= 64)
    static_assert(kSpecChunks <= 64, "the early chunks' offsets sit in one register");
    const int w0 = __builtin_amdgcn_readfirstlane(tid >> 6);
    #pragma unroll
    for (int i = 0; i < kSpecPer; ++i) {
      const int c = w0 + (NT / 64) * i;
      if (c < nch) {
        const uint32_t o = (uint32_t)__builtin_amdgcn_readlane((int)offq[0], c);
        const uint32_t nc = (uint32_t)__builtin_amdgcn_readlane((int)cnt[0], c);
        if (lane < nc) fs.cbig[o + lane] = sp[i];
        for (uint32_t j = 64u + lane; j < nc; j += 64u) fs.cbig[o + j] = cand[(int64_t)c * kFast + j];
      }
    }
    __syncthreads();
    return finish_core(fs, a, row, cfg, (int)n_total, M, ub, part, ub);
  }
  uint64_t cr[kFinPer];
  {
    int c = 0;
    #pragma unroll
    for (int r = 0; r < kFinPer; ++r) {
      const uint32_t j = (uint32_t)(tid + r * NT);
      cr[r] = 0ull;
      if (j < n_total) {
        while (fs.aux[c + 1] <= j) ++c;
        cr[r] = cand[(int64_t)c * kFast + (j - fs.aux[c])];
      }
    }
    #pragma unroll
    for (int r = 0; r < kFinPer; ++r) {
      const uint32_t j = (uint32_t)(tid + r * NT);
      if (j < n_total) fs.cbig[j] = cr[r];
    }
  }
  __syncthreads();
  // the k_sel-th candidate must be above every key a chunk left out
  return finish_core(fs, a, row, cfg, (int)n_total, M, ub, part, ub);
}


// --------------------------------------------------------------------------
// launch plumbing shared by the translation units

// Chunks of the streaming select pass: 64 logits per thread when the batch
// alone gives at least 4 workgroups per CU, 16 otherwise.
constexpr int kSelChunkLarge = NT * 64;
constexpr int kSelChunkSmall = NT * 16;
constexpr size_t kLdsPerCu = 160 * 1024;  // gfx950

// Raises a kernel's dynamic LDS limit to at least `bytes` on the current
// device (once per device and size; the attribute is per device).
hipError_t ensure_lds(const void* fn, size_t bytes);
hipError_t record(const LaunchEvents* le, int i, hipStream_t stream);

// The launchers of each kernel family (one translation unit each).
bool row_kernel_fits(const SampleArgs& a);
hipError_t launch_rows(const SampleArgs& a, hipStream_t stream);           // sampler_rows.hip
bool fused_fits(const SampleArgs& a);
hipError_t launch_fused(const SampleArgs& a, hipStream_t stream);          // sampler_fused.hip
hipError_t launch_select(const SampleArgs& a, hipStream_t stream);         // sampler_select.hip

}  // namespace hi_rocm
