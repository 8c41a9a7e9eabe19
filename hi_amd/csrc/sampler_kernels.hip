// hi-rocm batched token sampler: CDNA4 (gfx950) kernels.
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
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <float.h>
#include <stddef.h>

#include <map>
#include <mutex>
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
__device__ __forceinline__ void bitonic_keep(uint64_t& x, uint32_t& p, uint64_t y, uint32_t q, int i, int j, int k) {
  const bool keep_max = ((i & k) == 0) == ((i & j) == 0);
  if (keep_max ? (y > x) : (y < x)) {
    x = y;
    p = q;
  }
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
          const uint64_t y = shfl_xor_u64(x[r], o);
          const uint32_t q = (uint32_t)__shfl_xor((int)p[r], o, 64);
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
__device__ __forceinline__ int candidate_count(const SampleArgs& a, int row) {
  const ChunkStat* stats = a.stats + (int64_t)row * a.n_chunks;
  int n = 0;
  for (int c = 0; c < a.n_chunks; ++c) n += (int)stats[c].n_cand;
  return n;
}

// The exact first `kk` entries of the reference rank order (weight desc,
// index asc) of `row`.  On return fs.buf[0..kk) holds rank keys in order and
// fs.pay[0..kk) the scaled-logit keys; returns kk.  M is the row max of s.
__device__ __forceinline__ int rank_candidates(FinLds& fs, const SampleArgs& a, int row, const RowCfg& cfg,
                               int kk_req, float M) {
  const int tid = threadIdx.x;
  const int nch = a.n_chunks;
  const ChunkStat* stats = a.stats + (int64_t)row * nch;
  const int n_total = candidate_count(a, row);
  int kk = min(kk_req, n_total);
  if (kk <= 0) return 0;
  auto s_of = [&](uint64_t x) { return key_to_s(cand_skey(x), cfg.t_eff); };
  // 1. candidates into LDS: all of them when they fit, else those at or above
  //    t0, the largest chunk cut (the kk-th composite is at least every
  //    truncated chunk's smallest kept composite)
  uint64_t t0 = 0;
  uint64_t below_max = 0;  // largest candidate left out of LDS
  int n_u;
  bool in_lds = true;
  if (n_total <= kGather) {
    for_each_candidate(a, row, [&](uint64_t x, int pos) { fs.cbig[pos] = x; });
    n_u = n_total;
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
    const float w = exact_expf(sx - M);
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
    if (below_max != 0 && exact_expf(s_of(below_max) - M) == w_b) {
      if (in_lds) {
        for (int i = tid; i < n_u; i += NT) {
          const uint64_t x = fs.cbig[i];
          if (x >= thr) continue;
          const float sx = s_of(x);
          const float w = exact_expf(sx - M);
          if (w == w_b) add_ext(w, cand_idx(x), sx);
        }
      }
      if (!in_lds || t0 != 0) {
        for_each_candidate(a, row, [&](uint64_t x, int) {
          if (x >= thr || (in_lds && x >= t0)) return;  // selected, or seen in LDS
          const float sx = s_of(x);
          const float w = exact_expf(sx - M);
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
          if (cs.trunc && exact_expf(key_to_s(cs.unkept_key, cfg.t_eff) - M) == w_b)
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
          const float w = exact_expf(sx - M);
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
                                float M, bool eos, int ranked_k);

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
  uint32_t token;
  int ranked_k = 0;  // entries of fs.buf in rank order
  if (eos) {
    token = cfg.eos;
  } else if (cfg.cls == kGreedy) {
    token = a.pv.greedy_rule == kGreedyFiniteLane ? am_fin : am_ieee;
  } else if (!finitef_(M)) {
    token = cfg.cls == kTempOnly ? am_fin : row_argmax_total(fs, a, row, cfg);
  } else if (cfg.cls == kTopK && !cfg.store_s) {
    ranked_k = rank_candidates(fs, a, row, cfg, cfg.k_sel, M);
    token = draw_topk(fs, cfg, min(cfg.k_eff, ranked_k));
    if (token == 0xffffffffu) token = row_argmax_total(fs, a, row, cfg);
  } else if (cfg.cls == kTempOnly) {
    token = draw_temp_only(fs, a, row, M, u, am_fin);
  } else {
    token = draw_wide(fs, a, row, cfg, M, u);
    if (token == 0xffffffffu) token = row_argmax_total(fs, a, row, cfg);
  }
  if (tid == 0) a.out_tokens[row] = token;
  if (a.n_lp <= 0 && !a.out_token_lp) return;
  __syncthreads();
  finish_logprobs(fs, a, row, cfg, token, M, eos, ranked_k);
}

// Logprobs of the processed distribution (extension) once the row's token
// is known: the top n_lp in rank order and the token's own.  M is the row
// max of s; fs.buf / fs.pay hold the first ranked_k entries of the rank
// order (0: none yet).  The normaliser sums the candidates of every chunk
// in double and the other logits from each chunk's mass.
__device__ __forceinline__ void finish_logprobs(FinLds& fs, const SampleArgs& a, int row, const RowCfg& cfg, uint32_t token,
                                float M, bool eos, int ranked_k) {
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
  // log of the normaliser relative to M: the candidates of every chunk in
  // double, the other logits from each chunk's mass
  double part = 0.0;
  for_each_candidate(a, row, [&](uint64_t x, int) {
    if (cand_skey(x) > kKeyNegInf) part += exp((double)key_to_s(cand_skey(x), cfg.t_eff) - (double)M);
  });
  for (int c = tid; c < a.n_chunks; c += NT) {
    const ChunkStat cs = a.stats[(int64_t)row * a.n_chunks + c];
    if (cs.lse_sum > 0.f) part += (double)cs.lse_sum * exp((double)cs.lse_m - (double)M);
  }
  const double log_sum = log(block_sum_f64<NT>(part, fs.redd));
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
template <int PER, typename LoadF>
__device__ __forceinline__ uint64_t wave_select_skip_f(LoadF item, int n, uint32_t k, uint32_t* hist,
                                                       uint64_t lo, uint64_t hi_b, uint32_t kmax = 0u) {
  const int lane = threadIdx.x & 63;
  const uint32_t kcap = kmax > k ? kmax : k;
  uint64_t x[PER];
  uint64_t mn = ~0ull, mx = 0ull;
  #pragma unroll
  for (int m = 0; m < PER; ++m) {
    const int i = m * 64 + lane;
    x[m] = i < n ? item(i) : 0ull;
    if (i < n) {
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
template <int PER>
__device__ __forceinline__ uint64_t wave_select_skip(const uint64_t* items, int n, uint32_t k, uint32_t* hist,
                                                     uint64_t lo, uint64_t hi_b) {
  return wave_select_skip_f<PER>([&](int i) { return items[i]; }, n, k, hist, lo, hi_b);
}

constexpr int kLeanChunks = 256;  // chunks per row the lean finish merges
constexpr int kSpecChunks = 40;   // rows of up to this many chunks load their candidates early

// wave_fold_f32 that stops once a lane at or below the last final one has
// hit set and p >= cutoff; returns the first such lane (-1: none, all n
// lanes final).  Lanes past the returned one may hold partial sums.
__device__ __forceinline__ float wave_fold_f32_until(float v, float start, int n, bool hit, float cutoff,
                                                     int& first) {
  const int lane = (int)(threadIdx.x & 63u);
  const float u = lane == 0 ? start + v : v;
  float p = u;
  first = -1;
  #pragma unroll 1
  for (int s = 0;; s += 8) {
    // lanes [0, s] are final
    const uint64_t m = __ballot(hit && lane <= s && p >= cutoff);
    if (m != 0ull) {
      first = __ffsll((unsigned long long)m) - 1;
      break;
    }
    if (s >= n - 1) break;
    #pragma unroll
    for (int i = 0; i < 8; ++i) p = wave_fold_u(p) + u;
  }
  return p;
}

// Reference steps 7-10 (gpu.rs:831-899) over the rank order keys[0, k)
// (LDS, k <= 64 * DM), by every wave from registers: entry m * 64 + lane
// sits in lane `lane` of slot m.  Returns the drawn entry, or -1 for the
// reference's argmax_host fallback (no positive weight, or a total or
// candidate total that is not positive and finite).  All waves return the
// same, with no barrier.
template <int DM>
__device__ __forceinline__ int wave_draw(const uint64_t* keys, int k, const RowCfg& cfg) {
  const uint32_t lane = threadIdx.x & 63u;
  float fa[DM], pa[DM];
  #pragma unroll
  for (int m = 0; m < DM; ++m) {
    const int i = m * 64 + (int)lane;
    const float w = i < k ? rank_w(keys[i]) : 0.f;
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
  // folded only as far as the first one that reaches the cutoff
  int cut = -1;  // first positive entry where cum_p reaches the cutoff
  if (cfg.cutoff < 1.f) {
    float Q = 0.f;
    #pragma unroll
    for (int m = 0; m < DM; ++m) {
      if (cut < 0 && m * 64 < kp) {
        const int i = m * 64 + (int)lane;
        const bool pos = i < kp;
        const float fb = pos ? fa[m] / total : 0.f;
        int first;
        const float q = wave_fold_f32_until(fb, Q, min(64, kp - m * 64), pos, cfg.cutoff, first);
        if (first >= 0) cut = m * 64 + first;
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

// Reference steps 7-10 (gpu.rs:831-899) over the first k <= kBuf entries of
// the rank order in fs.buf (top-k rows).  Returns the token, or 0xffffffff
// for "fall back to argmax_host".
__device__ __forceinline__ uint32_t draw_topk(FinLds& fs, const RowCfg& cfg, int k) {
  const int pick = wave_draw<kBuf / 64>(fs.buf, k, cfg);
  return pick < 0 ? 0xffffffffu : cand_idx(fs.buf[pick]);
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

  // 8. the draw, by every wave from registers (gpu.rs:831-899)
  const int pick = wave_draw<kLeanK / 64>(fs.cbig, min(cfg.k_eff, kk), cfg);
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
  if (want_lp && tid < 64) {
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
    if (lane == 0u) fs.aux[nch] = n_total;
  }
  __syncthreads();

  // 2. the candidates into LDS (chunk-major): all loads first
  if (spec) {
    #pragma unroll
    for (int i = 0; i < kSpecPer; ++i) {
      const int c = (tid >> 6) + (NT / 64) * i;
      if (c < nch) {
        const uint32_t o = fs.aux[c], nc = fs.aux[c + 1] - o;
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

// ==========================================================================
// The scan kernel: one pass over the logits
// ==========================================================================

// Online sum of exp(s - m) with a running maximum m (for the log-sum-exp of
// the elements a chunk does not keep).
struct RestAcc {
  float m, sum;
  __device__ __forceinline__ void init() { m = -__builtin_inff(); sum = 0.f; }
  __device__ __forceinline__ void add(float s) {
    if (!finitef_(s)) return;
    if (sum == 0.f) { m = s; sum = 1.f; }
    else if (s > m) { sum = sum * __expf(m - s) + 1.f; m = s; }
    else sum += __expf(s - m);
  }
};

// Per-chunk running selection state (kept in registers, uniform over the
// workgroup): tau is a 48-bit local composite below which no element can be
// among the chunk's top k.
struct SelState {
  uint64_t tau;
  uint32_t unkept;  // largest key known not to be kept
  RestAcc rest;
  bool rest_on;
  float t_eff;
};

__device__ __forceinline__ void reject_key(SelState& ss, uint32_t key) {
  ss.unkept = max(ss.unkept, key);
  if (ss.rest_on) ss.rest.add(key_to_s(key, ss.t_eff));
}
__device__ __forceinline__ void reject(SelState& ss, uint64_t comp) {
  reject_key(ss, (uint32_t)(comp >> 16));
}

// Keep the k largest composites of the LDS buffer; raises tau and rejects
// the others.  All threads call it.
__device__ __forceinline__ void compact_buffer(ScanLds& sh, SelState& ss, uint32_t k) {
  const int tid = threadIdx.x;
  const uint32_t n = sh.count;
  if (n <= k) return;
  const uint64_t thr = radix_select_top(sh.hist, sh.sel, k, 48, [&](auto cb) {
    for (uint32_t i = tid; i < n; i += NT) cb(sh.cbuf[i]);
  });
  constexpr int PER = kBufCap / NT;
  uint64_t v[PER];
  uint32_t keep = 0;
  #pragma unroll
  for (int r = 0; r < PER; ++r) {
    const uint32_t i = r * NT + tid;
    v[r] = i < n ? sh.cbuf[i] : 0ull;
    if (i < n) {
      if (v[r] >= thr) ++keep;
      else reject(ss, v[r]);
    }
  }
  uint32_t total;
  uint32_t pos = block_excl_scan_u32<NT>(keep, sh.redu, &total);  // has barriers
  #pragma unroll
  for (int r = 0; r < PER; ++r) {
    const uint32_t i = r * NT + tid;
    if (i < n && v[r] >= thr) sh.cbuf[pos++] = v[r];
  }
  if (thr > ss.tau) ss.tau = thr;
  __syncthreads();
  if (tid == 0) sh.count = total;
  __syncthreads();
}

// Append NI items per thread to the running selection.  Item i has scaled-
// logit key key[i] (0 = no item) and local index li_of(i).  Items below tau
// are rejected, the rest go to the LDS buffer.  The caller guarantees that
// NI * NT <= kBufCap - k, so after one compaction (which leaves at most k
// entries) every batch fits.
template <int NI, typename LiOf>
__device__ __forceinline__ void append_batch(ScanLds& sh, SelState& ss, uint32_t k,
                                             const uint32_t (&key)[NI], LiOf li_of) {
  static_assert(NI * NT + kFast <= kBufCap, "a batch must fit after compaction");
  uint32_t mine = 0;
  #pragma unroll
  for (int i = 0; i < NI; ++i) mine += key[i] != 0u && local_comp(key[i], li_of(i)) >= ss.tau;
  uint32_t total;
  uint32_t off = block_excl_scan_u32<NT>(mine, sh.redu, &total);
  if (sh.count + total > (uint32_t)kBufCap) {
    compact_buffer(sh, ss, k);
    mine = 0;
    #pragma unroll
    for (int i = 0; i < NI; ++i) mine += key[i] != 0u && local_comp(key[i], li_of(i)) >= ss.tau;
    off = block_excl_scan_u32<NT>(mine, sh.redu, &total);
  }
  const uint32_t base = sh.count;
  #pragma unroll
  for (int i = 0; i < NI; ++i) {
    if (key[i] == 0u) continue;
    const uint64_t c = local_comp(key[i], li_of(i));
    if (c >= ss.tau) sh.cbuf[base + off++] = c;
    else reject(ss, c);
  }
  __syncthreads();
  if (threadIdx.x == 0) sh.count = base + total;
  __syncthreads();
}

template <int VEC>
__device__ __forceinline__ void load_tile(const SampleArgs& a, int64_t rbase, int tb, int c1,
                                          float (&raw)[VEC * 4]) {
  const int tid = threadIdx.x;
  if (a.dtype == HI_ROCM_DTYPE_BF16) {
    #pragma unroll
    for (int j = 0; j < VEC; ++j) {
      const int e0 = tb + (j * NT + tid) * 4;
      if (a.vec_ok && e0 + 3 < c1) {
        const uint2 v = *(const uint2*)((const uint16_t*)a.logits + rbase + e0);
        raw[4 * j + 0] = __uint_as_float(v.x << 16); raw[4 * j + 1] = __uint_as_float(v.x & 0xffff0000u);
        raw[4 * j + 2] = __uint_as_float(v.y << 16); raw[4 * j + 3] = __uint_as_float(v.y & 0xffff0000u);
      } else {
        #pragma unroll
        for (int q = 0; q < 4; ++q) raw[4 * j + q] = (e0 + q < c1) ? load_raw(a.logits, a.dtype, rbase + e0 + q) : 0.f;
      }
    }
  } else {
    #pragma unroll
    for (int j = 0; j < VEC; ++j) {
      const int e0 = tb + (j * NT + tid) * 4;
      if (a.vec_ok && e0 + 3 < c1) {
        const float4 v = *(const float4*)((const float*)a.logits + rbase + e0);
        raw[4 * j + 0] = v.x; raw[4 * j + 1] = v.y; raw[4 * j + 2] = v.z; raw[4 * j + 3] = v.w;
      } else {
        #pragma unroll
        for (int q = 0; q < 4; ++q) raw[4 * j + q] = (e0 + q < c1) ? load_raw(a.logits, a.dtype, rbase + e0 + q) : 0.f;
      }
    }
  }
}

// Which statistics a row needs from the scan (uniform per row).
struct StatNeeds {
  bool ieee;  // greedy rows: block_argmax_last
  bool fin;   // temperature-only rows and the finite-lane greedy rule
};

__device__ __forceinline__ StatNeeds stat_needs(const RowCfg& c, const ParamsView& pv) {
  StatNeeds n;
  n.ieee = c.cls == kGreedy && pv.greedy_rule == kGreedyIeee;
  n.fin = c.cls == kTempOnly || (c.cls == kGreedy && pv.greedy_rule == kGreedyFiniteLane);
  return n;
}

// Statistics update for one processed logit l at index e.  The maximum is
// tracked on the order key of l (non-finite l maps to the key of -inf),
// which also tells whether any finite value exists.
__device__ __forceinline__ void stat_add(ChunkStat& st, const StatNeeds& nd, uint32_t& maxkey,
                                         float l, uint32_t kl, uint32_t e) {
  maxkey = max(maxkey, kl);
  if (nd.ieee && l > st.am_ieee_v) { st.am_ieee_v = l; st.am_ieee_i = e; }
  if (nd.fin && finitef_(l) &&
      (st.am_fin_i == 0xffffffffu || l > st.am_fin_v ||
       (l == st.am_fin_v && fin_order(e) < fin_order(st.am_fin_i)))) {
    st.am_fin_v = l; st.am_fin_i = e;
  }
}


// History count of token `id` from the chunk's LDS hash (linear probing);
// `found` is false when the hash overflowed before the token was inserted.
__device__ __forceinline__ uint32_t hash_count(const uint32_t* hkey, const uint32_t* hcnt,
                                               uint32_t id, bool& found) {
  uint32_t slot = (id * 2654435761u) & (kHashCap - 1);
  for (int p = 0; p < kHashCap; ++p) {
    const uint32_t kk = hkey[slot];
    if (kk == id) { found = true; return hcnt[slot]; }
    if (kk == 0xffffffffu) break;
    slot = (slot + 1) & (kHashCap - 1);
  }
  found = false;
  return 0u;
}

// Block reduction of (min u64, max u32, f32 sum): the chunk's smallest kept
// candidate, largest dropped key and dropped log-sum-exp mass.
__device__ __forceinline__ void block_tail3(uint64_t& mn, uint32_t& mx, float& sum, ScanLds& sh) {
  uint64_t a = ~mn;
  for (int o = 32; o > 0; o >>= 1) {
    const uint64_t t = shfl_xor_u64(a, o);
    a = t > a ? t : a;
    mx = max(mx, (uint32_t)__shfl_xor(mx, o, 64));
    sum += __shfl_xor(sum, o, 64);
  }
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  __syncthreads();
  if (lane == 0) { sh.red64[wid] = a; sh.redu[wid] = mx; sh.redf[wid] = sum; }
  __syncthreads();
  a = sh.red64[0]; mx = sh.redu[0]; sum = sh.redf[0];
  for (int i = 1; i < NT / 64; ++i) {
    a = sh.red64[i] > a ? sh.red64[i] : a;
    mx = max(mx, sh.redu[i]);
    sum += sh.redf[i];
  }
  mn = ~a;
}

// ==========================================================================
// Wave-level helpers
// ==========================================================================

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

// The largest key prefix with the low 12 bits clear that at least `need`
// of the wave's group-maximum keys (four per lane) reach, or 0 when none
// does: it is the need-th largest key with its low 12 bits cleared.  For
// need <= 16 that key comes from `need` extractions of the wave maximum
// (each a DPP reduction, the lane holding it moving to its next key); a
// 20-step bit-by-bit search with a ballot count per step is the general
// form, and gives the same prefix.  `need` is uniform over the wave.
__device__ __forceinline__ uint32_t wave_prefix_reach(const uint32_t (&gk)[4], uint32_t need) {
  if (need <= 16u) {
    const uint32_t lane = threadIdx.x & 63u;
    uint32_t s0 = gk[0], s1 = gk[1], s2 = gk[2], s3 = gk[3];
    auto cx = [](uint32_t& p, uint32_t& q) {
      const uint32_t hi = max(p, q), lo = min(p, q);
      p = hi;
      q = lo;
    };
    cx(s0, s1); cx(s2, s3); cx(s0, s2); cx(s1, s3); cx(s1, s2);  // s0 >= s1 >= s2 >= s3
    uint32_t v = 0u;
    #pragma unroll 1
    for (uint32_t it = 0; it < need; ++it) {
      v = wave_max_u32(s0);
      const uint64_t who = __ballot(s0 == v);
      if (lane == (uint32_t)(__ffsll((unsigned long long)who) - 1)) {
        s0 = s1;
        s1 = s2;
        s2 = s3;
        s3 = 0u;
      }
    }
    return v & 0xfffff000u;
  }
  uint32_t prefix = 0u;
  #pragma unroll 1
  for (int bit = 31; bit >= 12; --bit) {
    const uint32_t probe = prefix | (1u << bit);
    uint32_t c = 0u;
    #pragma unroll
    for (int g = 0; g < 4; ++g) c += (uint32_t)__popcll(__ballot(gk[g] >= probe));
    if (c >= need) prefix = probe;
  }
  return prefix;
}

// Up to NS LDS arrays of candidate keys, read as one list.
template <int NS>
struct Segs {
  const uint64_t* p[NS];
  uint32_t n[NS];
  int ns;
};

// Threshold T such that exactly `need` of the listed entries (unique keys)
// are >= T, for 1 <= need <= the number of entries.  8-bit MSD descent with
// early exit over a 256-bin LDS histogram owned by the wave.
template <int NS>
__device__ __forceinline__ uint64_t wave_select(const Segs<NS>& sg, uint32_t need, uint32_t* hist) {
  const uint32_t lane = threadIdx.x & 63u;
  uint64_t prefix = 0;
  uint32_t remaining = need;
  #pragma unroll 1
  for (int shift = 56; shift >= 0; shift -= 8) {
    wave_lds_sync();
    *reinterpret_cast<uint4*>(hist + 4 * lane) = make_uint4(0u, 0u, 0u, 0u);
    wave_lds_sync();
    const int hs = shift + 8;
    const uint64_t hp = hs >= 64 ? 0ull : (prefix >> hs);
    #pragma unroll
    for (int sgi = 0; sgi < NS; ++sgi) {
      if (sgi >= sg.ns) break;
      const uint64_t* p = sg.p[sgi];
      const uint32_t n = sg.n[sgi];
      #pragma unroll 2
      for (uint32_t i = lane; i < n; i += 64u) {
        const uint64_t x = p[i];
        if (hs >= 64 || (x >> hs) == hp) atomicAdd(&hist[(uint32_t)(x >> shift) & 255u], 1u);
      }
    }
    wave_lds_sync();
    // lane l owns bins 255-4l, 254-4l, 253-4l, 252-4l (descending)
    const uint4 h = *reinterpret_cast<const uint4*>(hist + 252 - 4 * lane);
    const uint32_t cs[4] = {h.w, h.z, h.y, h.x};
    const uint32_t lsum = cs[0] + cs[1] + cs[2] + cs[3];
    const uint32_t inc = wave_incl_scan_u32(lsum);
    uint32_t acc = inc - lsum, d = 0, da = 0, dc = 0;
    #pragma unroll
    for (int q = 0; q < 4; ++q) {
      if (acc < remaining && remaining <= acc + cs[q]) { d = 255u - 4u * lane - (uint32_t)q; da = acc; dc = cs[q]; }
      acc += cs[q];
    }
    const uint64_t who = __ballot(inc - lsum < remaining && remaining <= inc);
    const int src = __ffsll((unsigned long long)who) - 1;
    d = (uint32_t)__builtin_amdgcn_readlane((int)d, src);
    da = (uint32_t)__builtin_amdgcn_readlane((int)da, src);
    dc = (uint32_t)__builtin_amdgcn_readlane((int)dc, src);
    prefix |= (uint64_t)d << shift;
    remaining -= da;
    if (dc == remaining) break;
  }
  return prefix;
}

// Range-checked loads of one row (byte offsets at or past the range read
// as zero; nothing faults).
typedef int i32x4_t __attribute__((ext_vector_type(4)));
typedef int i32x2_t __attribute__((ext_vector_type(2)));
constexpr int kBufferConfig = 0x00020000;  // raw buffer, 32-bit data (gfx9 family)

struct RowBuf {
  __amdgpu_buffer_rsrc_t logits, mask;
};

// Range [c0, c1) of `row` (c0 a multiple of 32).
template <int DT, bool MASK>
__device__ __forceinline__ RowBuf row_buf(const SampleArgs& a, int row, int c0, int c1) {
  RowBuf rb;
  const int esize = DT == HI_ROCM_DTYPE_BF16 ? 2 : 4;
  const char* base = (const char*)a.logits + ((int64_t)row * a.row_stride + c0) * esize;
  rb.logits = __builtin_amdgcn_make_buffer_rsrc((void*)base, (short)0, (c1 - c0) * esize, kBufferConfig);
  if (MASK)
    rb.mask = __builtin_amdgcn_make_buffer_rsrc((void*)(a.mask + (int64_t)row * a.mask_words + (c0 >> 5)),
                                                (short)0, ((c1 - c0 + 31) >> 5) * 4, kBufferConfig);
  return rb;
}

// The general per-chunk pass (top-p, min-p, temperature-only and wide rows,
// the finite-lane greedy rule, large logprob counts): block-level running
// selection, scaled logits stored for the finish.
template <int VEC, int TILES>
__device__ __forceinline__ void scan_generic(const SampleArgs& a, const RowCfg& cfg, ScanLds& sh,
                                             const float (&tile0)[VEC * 4],
                                             const uint32_t* bitmap, const uint32_t* hkey,
                                             const uint32_t* hcnt, bool pen, uint32_t h0, uint32_t h1,
                                             int row, int chunk, int c0, int c1) {
  constexpr int TILE = NT * VEC * 4;
  constexpr int E = VEC * 4;
  const int tid = threadIdx.x;
  const int V = a.V;
  const int len = c1 - c0;
  const int64_t rbase = (int64_t)row * a.row_stride;
  const uint32_t* mrow = a.mask ? a.mask + (int64_t)row * a.mask_words : nullptr;
  float* srow = cfg.store_s ? a.ws_s + (int64_t)row * V : nullptr;
  const uint32_t k = (uint32_t)cfg.k_sel;

  float cur[E];
  #pragma unroll
  for (int i = 0; i < E; ++i) cur[i] = tile0[i];
  if (tid == 0) sh.count = 0u;
  __syncthreads();

  SelState ss;
  ss.tau = 0ull;
  ss.unkept = 0u;
  ss.rest.init();
  ss.rest_on = a.need_lse != 0;
  ss.t_eff = cfg.t_eff;
  ChunkStat st;
  stat_init(st);
  const StatNeeds nd = stat_needs(cfg, a.pv);
  uint32_t maxkey = 0u;

  #pragma unroll 1
  for (int t = 0; t < TILES; ++t) {
    const int tb = c0 + t * TILE;
    if (tb >= c1) break;
    float nxt[E];
    if (t + 1 < TILES && tb + TILE < c1) load_tile<VEC>(a, rbase, tb + TILE, c1, nxt);
    uint32_t key[E];  // 0: no element (past the end)
    #pragma unroll
    for (int j = 0; j < VEC; ++j) {
      const int e0 = tb + (j * NT + tid) * 4;
      const uint32_t mword = (mrow && e0 < c1) ? mrow[e0 >> 5] : 0xffffffffu;
      uint32_t flags = 0u;
      if (pen && e0 < c1) flags = (bitmap[(e0 - c0) >> 5] >> ((e0 - c0) & 31)) & 15u;
      #pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int e = e0 + q;
        float l = cur[4 * j + q];
        if (!((mword >> (e & 31)) & 1u)) l = -__builtin_inff();
        if ((flags >> q) & 1u) {
          bool found;
          uint32_t cnt = hash_count(hkey, hcnt, (uint32_t)e, found);
          if (!found) {  // the hash overflowed: count from the global list (slow)
            cnt = 0u;
            for (uint32_t h = h0; h < h1; ++h) if (a.hids[h] == (uint32_t)e) cnt += a.hcnt[h];
          }
          l = apply_penalties(l, cnt, cfg);
        }
        const uint32_t kl = lkey(l);
        const bool in = e < c1;
        if (in) stat_add(st, nd, maxkey, l, kl, (uint32_t)e);
        key[4 * j + q] = in ? kl : 0u;
      }
      if (srow) {
        float sv[4];
        #pragma unroll
        for (int q = 0; q < 4; ++q) sv[q] = key[4 * j + q] ? key_to_s(key[4 * j + q], cfg.t_eff) : -__builtin_inff();
        if (e0 + 3 < c1 && (V & 3) == 0) {
          *(float4*)(srow + e0) = make_float4(sv[0], sv[1], sv[2], sv[3]);
        } else {
          for (int q = 0; q < 4; ++q) if (e0 + q < c1) srow[e0 + q] = sv[q];
        }
      }
    }
    if (k > 0) {
      if (t == 0 && len > (int)k) {
        // bound from the first tile: the k-th largest of the per-thread
        // top-j keys, rounded down to 16 bits (k or more real elements are
        // at or above it)
        const int jt = ((int)k + NT - 1) / NT;  // 1..4
        uint32_t t4[4] = {0u, 0u, 0u, 0u};
        #pragma unroll
        for (int i = 0; i < E; ++i) {
          uint32_t x = key[i];
          #pragma unroll
          for (int r = 0; r < 4; ++r) {
            const uint32_t hi = max(t4[r], x);
            x = min(t4[r], x);
            t4[r] = hi;
          }
        }
        for (int r = 0; r < jt; ++r) sh.U[r * NT + tid] = t4[r];
        __syncthreads();
        if (tid < 64) {
          const int nr = jt * NT / 64;
          uint32_t prefix = 0u;
          for (int bit = 31; bit >= 16; --bit) {
            const uint32_t probe = prefix | (1u << bit);
            uint32_t c = 0;
            for (int r = 0; r < nr; ++r) c += (uint32_t)__popcll(__ballot(sh.U[r * 64 + tid] >= probe));
            if (c >= k) prefix = probe;
          }
          if (tid == 0) sh.bound = prefix;
        }
        __syncthreads();
        ss.tau = (uint64_t)sh.bound << 16;
      }
      const uint32_t li0 = (uint32_t)(tb - c0);
      auto li_of = [&](int i) { return li0 + (uint32_t)(((i >> 2) * NT + tid) * 4 + (i & 3)); };
      // fast path: the whole tile's survivors fit the buffer (one scan).
      // Survivors are compared on the key alone (a superset of the
      // composite test; the extra entries are dropped at compaction).
      const uint32_t tk = (uint32_t)(ss.tau >> 16);
      uint32_t mine = 0;
      #pragma unroll
      for (int i = 0; i < E; ++i) mine += key[i] >= tk && key[i] != 0u;
      uint32_t total;
      uint32_t off = block_excl_scan_u32<NT>(mine, sh.redu, &total);
      if (sh.count + total <= (uint32_t)kBufCap) {
        const uint32_t base = sh.count;
        #pragma unroll
        for (int i = 0; i < E; ++i) {
          if (key[i] == 0u) continue;
          if (key[i] >= tk) sh.cbuf[base + off++] = local_comp(key[i], li_of(i));
          else reject_key(ss, key[i]);
        }
        __syncthreads();
        if (tid == 0) sh.count = base + total;
        __syncthreads();
      } else {
        // one float4 column (NT * 4 items) at a time, so each batch fits
        #pragma unroll
        for (int j = 0; j < VEC; ++j) {
          const uint32_t kj[4] = {key[4 * j], key[4 * j + 1], key[4 * j + 2], key[4 * j + 3]};
          const uint32_t lij = li0 + (uint32_t)((j * NT + tid) * 4);
          append_batch<4>(sh, ss, k, kj, [&](int q) { return lij + (uint32_t)q; });
        }
      }
    }
    #pragma unroll
    for (int i = 0; i < E; ++i) cur[i] = nxt[i];
  }

  st.max_l = maxkey > kKeyNegInf ? okey_inv(maxkey) : -__builtin_inff();
  st.any_finite = maxkey > kKeyNegInf ? 1u : 0u;
  ChunkStat bs = block_stat<NT>(st, sh.red);
  uint64_t* cand = a.cand + ((int64_t)row * a.n_chunks + chunk) * kFast;
  if (k > 0) {
    // the chunk's exact top-k: select in the buffer, emit in thread order
    compact_buffer(sh, ss, k);
    const uint32_t n = sh.count;
    constexpr int PER = kBufCap / NT;
    uint32_t mine = 0;
    #pragma unroll
    for (int r = 0; r < PER; ++r) mine += (uint32_t)(r * NT + tid) < n;
    uint32_t total;
    uint32_t pos = block_excl_scan_u32<NT>(mine, sh.redu, &total);
    uint64_t minkept = ~0ull;
    const float mc = finitef_(bs.max_l) ? bs.max_l / cfg.t_eff : -__builtin_inff();
    #pragma unroll
    for (int r = 0; r < PER; ++r) {
      const uint32_t i = r * NT + tid;
      if (i >= n) continue;
      const uint64_t v = sh.cbuf[i];
      const uint32_t li = 0xffffu - (uint32_t)(v & 0xffffu);
      const uint64_t ck = cand_key((uint32_t)(v >> 16), (uint32_t)c0 + li);
      if (pos < (uint32_t)kFast) cand[pos] = ck;
      ++pos;
      minkept = ck < minkept ? ck : minkept;
    }
    float part = (ss.rest_on && ss.rest.sum > 0.f && finitef_(mc)) ? ss.rest.sum * __expf(ss.rest.m - mc) : 0.f;
    uint32_t unkept = ss.unkept;
    block_tail3(minkept, unkept, part, sh);
    bs.n_cand = min(total, (uint32_t)kFast);
    bs.trunc = len > (int)k ? 1u : 0u;
    bs.min_kept = minkept;
    bs.unkept_key = unkept;
    bs.lse_m = mc;
    bs.lse_sum = part;
  }
  if (tid == 0) a.stats[(int64_t)row * a.n_chunks + chunk] = bs;
}

// History tokens of the chunk [c0, c1) for the general pass: an LDS bitmap
// of the tokens present and an (id -> summed count) hash with linear
// probing.  All threads call it.
template <int CH>
__device__ __forceinline__ void stage_history_hash(const SampleArgs& a, uint32_t h0, uint32_t h1, int c0,
                                                   int c1, uint32_t* bitmap, uint32_t* hkey, uint32_t* hcnt) {
  const int tid = threadIdx.x;
  for (int i = tid; i < CH / 32; i += NT) bitmap[i] = 0u;
  for (int i = tid; i < kHashCap; i += NT) { hkey[i] = 0xffffffffu; hcnt[i] = 0u; }
  __syncthreads();
  for (uint32_t hb = h0; hb < h1; hb += NT * 8) {
    uint32_t ids[8], cnts[8];
    #pragma unroll
    for (int r = 0; r < 8; ++r) {  // independent loads first
      const uint32_t h = hb + r * NT + tid;
      ids[r] = h < h1 ? a.hids[h] : 0xffffffffu;
      cnts[r] = h < h1 ? a.hcnt[h] : 0u;
    }
    #pragma unroll
    for (int r = 0; r < 8; ++r) {
      const uint32_t id = ids[r];
      if (id < (uint32_t)c0 || id >= (uint32_t)c1) continue;
      const uint32_t li = id - (uint32_t)c0;
      atomicOr(&bitmap[li >> 5], 1u << (li & 31u));
      // a token that finds no free slot is counted from the global list
      // when it is looked up (hash_count reports it as not found)
      uint32_t slot = (id * 2654435761u) & (kHashCap - 1);
      for (int probe = 0; probe < kHashCap; ++probe) {
        const uint32_t prev = atomicCAS(&hkey[slot], 0xffffffffu, id);
        if (prev == 0xffffffffu || prev == id) {
          atomicAdd(&hcnt[slot], cnts[r]);
          break;
        }
        slot = (slot + 1) & (kHashCap - 1);
      }
    }
  }
  __syncthreads();
}

// ==========================================================================
// Streaming select pass
// ==========================================================================
//
// One workgroup of NT threads per (chunk, row).  A chunk is NT * E logits;
// thread tid owns the EPL logits of each 16-byte load j at local index
// (j * NT + tid) * EPL, so every load instruction of a wave covers 1 KiB of
// consecutive HBM.  The row's history list and then every load of the chunk
// are issued before anything waits on them.  The row's class picks the path
// (uniform per workgroup):
//
// select_lean   greedy rows and top-k rows that keep no scaled logits.
//   phase A   per-lane maxima of 4 groups of E/4 logits (allowed-token mask
//             as -inf; history tokens keep their raw logit here);
//   bound     each wave binary-searches, with ballots and popcounts, the
//             largest key t_w such that at least ceil(m/4) + h_w of its
//             group maxima are >= t_w, h_w being the history tokens among
//             the wave's logits: at least ceil(m/4) of those maxima are then
//             distinct non-history logits, so the workgroup bound
//             t = min t_w has at least m logits >= t (m = chunk_keep: k
//             when the row has few chunks);
//   phase B   one compare per logit builds a per-lane survivor bitmask; a
//             short per-lane loop re-reads the few survivors (L2 hits),
//             skipping history tokens, whose penalised values were computed
//             out of band;
//   select    wave 0 runs an 8-bit radix select that starts below the
//             survivors' common key prefix and keeps the chunk's exact top
//             k_sel by (processed logit desc, index asc).
//
// select_wide   rows that keep their scaled logits (top-p / min-p only,
//             temperature-only, top-k above kLeanK): history tokens are
//             marked absent in the stream, the scaled logits are stored, and
//             candidates (for logprobs) come from wave-private survivor lists.
//
// Chunks with +inf, no finite logit, a zero maximum on an argmax row, a
// failed bound or too many survivors take select_exact(), which reads the
// chunk again and recomputes everything element by element with integer
// keys.  Every path writes the same record and candidates.

// Candidates a lean chunk guarantees: at least its top k_sel, or fewer when
// the row is split into many chunks.  A chunk holds on average
// mu = k_sel / n_chunks of the row's top k_sel; it keeps at least
// ceil(mu + 4 sqrt(mu) + 4) (at least kLseTop on logprob rows, whose
// normaliser sums the largest terms from the candidates).  A chunk holding
// more of the row's top k_sel than it kept is caught by the finish (the
// k_sel-th key is not above the largest key left out), and the row takes
// the exact finish.
__device__ __forceinline__ uint32_t chunk_keep(uint32_t k_sel, int n_chunks, bool lse) {
  const float mu = (float)k_sel / (float)n_chunks;
  uint32_t m = (uint32_t)ceilf(mu + 4.f * sqrtf(mu) + 4.f);
  if (lse) m = max(m, (uint32_t)kLseTop);
  return min(m, k_sel);
}

constexpr int kSurvCap = 640;              // survivors per wave
constexpr uint32_t kSelHistCap = 1024;     // distinct history tokens per chunk held in LDS
constexpr int kSelHistPer = 8;             // history entries each thread loads up front
constexpr int kSelOb = (int)kSelHistCap / NT;  // out-of-band history items per thread
constexpr int kLaneSurv = 6;               // streamed survivors a lane takes per round (lean path)
constexpr int kWideCopies = 8;             // copies of the mass histogram (lane % 8 picks one)

struct SelLds {
  uint64_t surv[NT / 64][kSurvCap];
  uint32_t hist[256];
  float whist[kWideBins * kWideCopies];  // top-p rows: the chunk's mass histogram (WideStat),
                                         // kWideCopies interleaved copies
  uint32_t sel[4];
  uint32_t hw[NT / 64];       // history tokens among each wave's logits
  uint32_t wcnt[NT / 64];
  uint32_t wkept[NT / 64];
  uint32_t wflag[NT / 64];
  uint32_t wkey[NT / 64];
  float wmax[NT / 64];
  uint64_t red64[NT / 64];
  uint64_t red64b[NT / 64];
  uint64_t red64c[NT / 64];
  uint32_t redu[NT / 64];
  uint32_t redu2[NT / 64];
  float redf[NT / 64];
  double redd[NT / 64];
  ChunkStat red[NT / 64];
};
constexpr size_t kSelHead = (sizeof(SelLds) + 15) & ~(size_t)15;

// History tokens of the chunk: bit li of `bitmap` marks token c0 + li,
// prefix[w] counts the marked tokens of the words below w, and the token of
// rank r (r < kSelHistCap) has id ids[r] and summed count cnts[r].
struct SelHist {
  const uint32_t* bitmap;
  const uint32_t* prefix;
  const uint32_t* cnts;
  const uint32_t* ids;
  uint32_t distinct;
  uint32_t h0, h1;
  bool on;
  bool ovf;  // more marked tokens than kSelHistCap
};

__host__ __device__ constexpr size_t sel_hist_bytes(int len) {
  return (size_t)2 * ((len + 31) / 32) * 4 + (size_t)2 * kSelHistCap * 4 + 64;
}

// Builds the SelHist of [c0, c0 + len) in `mem` from the history entries
// each thread loaded (hid/hcs: entry h0 + r * NT + tid); entries past those
// are read here.  hw[w] counts the entries that fall on wave w's logits
// (logit li belongs to wave ((li / epl) % NT) / 64).  All threads call it.
__device__ __forceinline__ SelHist stage_history_sel(const SampleArgs& a, int c0, int len, int epl, uint32_t* mem,
                                                     uint32_t* hw, const uint32_t (&hid)[kSelHistPer],
                                                     const uint32_t (&hcs)[kSelHistPer], uint32_t h0,
                                                     uint32_t h1) {
  const int tid = threadIdx.x;
  const int W = (len + 31) >> 5;
  uint32_t* bitmap = mem;
  uint32_t* prefix = mem + W;
  uint32_t* cnts = prefix + W;
  uint32_t* ids = cnts + kSelHistCap;
  uint32_t* red = ids + kSelHistCap;
  SelHist hv;
  hv.bitmap = bitmap; hv.prefix = prefix; hv.cnts = cnts; hv.ids = ids;
  hv.distinct = 0u; hv.h0 = h0; hv.h1 = h1;
  hv.on = h1 > h0;
  hv.ovf = false;
  if (tid < NT / 64) hw[tid] = 0u;
  if (!hv.on) {
    __syncthreads();
    return hv;
  }
  constexpr uint32_t kFirst = (uint32_t)(kSelHistPer * NT);
  for (int i = tid; i < W; i += NT) bitmap[i] = 0u;
  __syncthreads();
  auto mark = [&](uint32_t id) {
    const uint32_t li = id - (uint32_t)c0;
    if (id >= (uint32_t)c0 && li < (uint32_t)len) {
      atomicOr(&bitmap[li >> 5], 1u << (li & 31u));
      atomicAdd(&hw[((li / (uint32_t)epl) % (uint32_t)NT) >> 6], 1u);
    }
  };
  #pragma unroll
  for (int r = 0; r < kSelHistPer; ++r) mark(hid[r]);
  for (uint32_t h = h0 + kFirst + tid; h < h1; h += NT) mark(a.hids[h]);
  __syncthreads();
  const int PW = (W + NT - 1) / NT;
  uint32_t loc = 0;
  for (int i = 0; i < PW; ++i) {
    const int w = tid * PW + i;
    if (w < W) loc += (uint32_t)__popc(bitmap[w]);
  }
  uint32_t total;
  uint32_t run = block_excl_scan_u32<NT>(loc, red, &total);
  for (int i = 0; i < PW; ++i) {
    const int w = tid * PW + i;
    if (w < W) { prefix[w] = run; run += (uint32_t)__popc(bitmap[w]); }
  }
  const uint32_t nz = min(total, kSelHistCap);
  for (uint32_t i = tid; i < nz; i += NT) cnts[i] = 0u;
  __syncthreads();
  auto add = [&](uint32_t id, uint32_t c) {
    const uint32_t li = id - (uint32_t)c0;
    if (id >= (uint32_t)c0 && li < (uint32_t)len) {
      const uint32_t w = li >> 5;
      const uint32_t rank = prefix[w] + (uint32_t)__popc(bitmap[w] & ((1u << (li & 31u)) - 1u));
      if (rank < kSelHistCap) {
        atomicAdd(&cnts[rank], c);
        ids[rank] = id;  // every occurrence writes the same id
      }
    }
  };
  #pragma unroll
  for (int r = 0; r < kSelHistPer; ++r) add(hid[r], hcs[r]);
  for (uint32_t h = h0 + kFirst + tid; h < h1; h += NT) add(a.hids[h], a.hcnt[h]);
  __syncthreads();
  hv.distinct = total;
  hv.ovf = total > kSelHistCap;
  return hv;
}

__device__ __forceinline__ bool hist_marked(const SelHist& hv, uint32_t li) {
  return hv.on && ((hv.bitmap[li >> 5] >> (li & 31u)) & 1u);
}

// Summed history count of token e (local index li) for the exact path.
__device__ __forceinline__ uint32_t sel_hist_count(const SampleArgs& a, const SelHist& hv, int c0, uint32_t li,
                                                   bool& marked) {
  const uint32_t w = li >> 5;
  marked = hist_marked(hv, li);
  if (!marked) return 0u;
  const uint32_t rank = hv.prefix[w] + (uint32_t)__popc(hv.bitmap[w] & ((1u << (li & 31u)) - 1u));
  if (rank < kSelHistCap) return hv.cnts[rank];
  const uint32_t e = (uint32_t)c0 + li;
  uint32_t c = 0u;
  for (uint32_t h = hv.h0; h < hv.h1; ++h) if (a.hids[h] == e) c += a.hcnt[h];
  return c;
}

// Threshold T such that exactly `need` of the listed entries (unique keys)
// are >= T, 1 <= need <= entries.  Like wave_select, but the first digit
// starts just below the entries' common high bits, and the last digit may be
// narrower than 8 bits.  Called by one whole wave.
template <int NS>
__device__ __forceinline__ uint64_t wave_select_skip(const Segs<NS>& sg, uint32_t need, uint32_t* hist) {
  const uint32_t lane = threadIdx.x & 63u;
  uint64_t mn = ~0ull, mx = 0ull;
  #pragma unroll
  for (int s = 0; s < NS; ++s) {
    if (s >= sg.ns) break;
    for (uint32_t i = lane; i < sg.n[s]; i += 64u) {
      const uint64_t x = sg.p[s][i];
      mn = x < mn ? x : mn;
      mx = x > mx ? x : mx;
    }
  }
  mn = wave_min_u64(mn);
  mx = wave_max_u64(mx);
  if (mn == mx) return mx;
  int hi = 64 - __clzll(mn ^ mx);  // bits [0, hi) still undecided
  uint64_t prefix = hi >= 64 ? 0ull : (mx >> hi) << hi;
  uint32_t remaining = need;
  #pragma unroll 1
  while (hi > 0) {
    const int db = hi >= 8 ? 8 : hi;
    const int lo = hi - db;
    const uint64_t hp = hi >= 64 ? 0ull : (prefix >> hi);
    wave_lds_sync();
    *reinterpret_cast<uint4*>(hist + 4 * lane) = make_uint4(0u, 0u, 0u, 0u);
    wave_lds_sync();
    #pragma unroll
    for (int s = 0; s < NS; ++s) {
      if (s >= sg.ns) break;
      for (uint32_t i = lane; i < sg.n[s]; i += 64u) {
        const uint64_t x = sg.p[s][i];
        if (hi >= 64 || (x >> hi) == hp) atomicAdd(&hist[(uint32_t)(x >> lo) & ((1u << db) - 1u)], 1u);
      }
    }
    wave_lds_sync();
    // lane l owns bins 255-4l .. 252-4l (descending)
    const uint4 h = *reinterpret_cast<const uint4*>(hist + 252 - 4 * lane);
    const uint32_t cs[4] = {h.w, h.z, h.y, h.x};
    const uint32_t lsum = cs[0] + cs[1] + cs[2] + cs[3];
    const uint32_t inc = wave_incl_scan_u32(lsum);
    uint32_t acc = inc - lsum, d = 0, da = 0, dc = 0;
    #pragma unroll
    for (int q = 0; q < 4; ++q) {
      if (acc < remaining && remaining <= acc + cs[q]) { d = 255u - 4u * lane - (uint32_t)q; da = acc; dc = cs[q]; }
      acc += cs[q];
    }
    const uint64_t who = __ballot(inc - lsum < remaining && remaining <= inc);
    const int src = __ffsll((unsigned long long)who) - 1;
    d = (uint32_t)__builtin_amdgcn_readlane((int)d, src);
    da = (uint32_t)__builtin_amdgcn_readlane((int)da, src);
    dc = (uint32_t)__builtin_amdgcn_readlane((int)dc, src);
    prefix |= (uint64_t)d << lo;
    remaining -= da;
    hi = lo;
    if (dc == remaining) break;
  }
  return prefix;
}

// What a row needs from the pass (uniform per row).
struct SelNeeds {
  bool ieee, fin;   // argmax rules (greedy rows, temperature-only rows)
  bool sel;         // candidates (k_sel > 0)
  bool surv;        // a survivor list at all (sel or an argmax)
  bool lse;         // normaliser rest for logprobs
  bool whist;       // top-p rows: the chunk's mass histogram for the wide pass
};

__device__ __forceinline__ SelNeeds sel_needs(const SampleArgs& a, const RowCfg& cfg) {
  SelNeeds n;
  n.ieee = cfg.cls == kGreedy && a.pv.greedy_rule == kGreedyIeee;
  n.fin = cfg.cls == kTempOnly || (cfg.cls == kGreedy && a.pv.greedy_rule == kGreedyFiniteLane);
  n.sel = cfg.k_sel > 0;
  n.surv = n.sel || n.ieee || n.fin;
  n.lse = a.need_lse != 0;
  n.whist = cfg.cls == kTopP;
  return n;
}

// Adds one processed logit v (NaN: absent) to a top-p row's chunk mass
// histogram: w' = exp((v - m) / T) = 2^r, bin floor(-r), clamped.  Lane l
// adds to copy l % kWideCopies: the lanes of a wave that hit one bin (a
// row's logits fill a few bins) then conflict kWideCopies times less.  The
// masses are approximate (the wide pass keeps a margin), so the order of
// the additions does not matter.
__device__ __forceinline__ void wide_hist_add(float* whist, float v, float m, float a2) {
  if (!finitef_(v)) return;
  const float r = (v - m) * a2;
  const int j = -r < (float)(kWideBins - 1) ? (int)(-r) : kWideBins - 1;
  atomicAdd(&whist[j * kWideCopies + (int)(threadIdx.x & (kWideCopies - 1))], __builtin_amdgcn_exp2f(r));
}
__device__ __forceinline__ void wide_hist_clear(float* whist) {
  for (int i = threadIdx.x; i < kWideBins * kWideCopies; i += NT) whist[i] = 0.f;
}
// Bin b (b < kWideBins) summed over the copies.
__device__ __forceinline__ float wide_hist_bin(const float* whist, int b) {
  float s = 0.f;
  #pragma unroll
  for (int c = 0; c < kWideCopies; ++c) s += whist[b * kWideCopies + c];
  return s;
}

// Exact pass over the chunk from global memory, element by element.  Used
// for the rare chunks the fast paths do not take.  All threads call it.
__device__ __forceinline__ void select_exact(SelLds& L, const SampleArgs& a, const RowCfg& cfg, const SelHist& hv,
                                             const SelNeeds& nd, int row, int c0, int len, int64_t slot) {
  const int tid = threadIdx.x;
  const int64_t rbase = (int64_t)row * a.row_stride;
  auto proc = [&](int li) -> float {
    const uint32_t e = (uint32_t)(c0 + li);
    float l = load_raw(a.logits, a.dtype, rbase + e);
    if (!allowed(a, row, e)) l = -__builtin_inff();
    bool marked;
    const uint32_t cnt = sel_hist_count(a, hv, c0, (uint32_t)li, marked);
    return marked ? apply_penalties(l, cnt, cfg) : l;
  };
  // statistics (per thread in increasing index order, then merged)
  ChunkStat st;
  stat_init(st);
  uint32_t maxkey = 0u;
  for (int li = tid; li < len; li += NT) {
    const float l = proc(li);
    const uint32_t e = (uint32_t)(c0 + li);
    maxkey = max(maxkey, lkey(l));
    if (nd.ieee && l > st.am_ieee_v) { st.am_ieee_v = l; st.am_ieee_i = e; }
    if (nd.fin && finitef_(l) &&
        (st.am_fin_i == 0xffffffffu || l > st.am_fin_v ||
         (l == st.am_fin_v && fin_order(e) < fin_order(st.am_fin_i)))) {
      st.am_fin_v = l; st.am_fin_i = e;
    }
  }
  st.max_l = maxkey > kKeyNegInf ? okey_inv(maxkey) : -__builtin_inff();
  st.any_finite = maxkey > kKeyNegInf ? 1u : 0u;
  ChunkStat bs = block_stat<NT>(st, L.red);
  const float lmax = bs.max_l;
  const float a2 = 1.4426950408889634f / cfg.t_eff;
  if (nd.sel) {
    const uint32_t k = (uint32_t)cfg.k_sel;
    uint64_t thr = 0ull;
    if ((uint32_t)len > k)
      thr = radix_select_top(L.hist, L.sel, k, 64, [&](auto cb) {
        for (int li = tid; li < len; li += NT) cb(cand_key(lkey(proc(li)), (uint32_t)(c0 + li)));
      });
    uint32_t mine = 0u;
    for (int li = tid; li < len; li += NT) mine += cand_key(lkey(proc(li)), (uint32_t)(c0 + li)) >= thr;
    uint32_t total;
    uint32_t pos = block_excl_scan_u32<NT>(mine, L.redu, &total);
    uint64_t* cand = a.cand + slot * kFast;
    uint64_t minkept = ~0ull;
    uint32_t unkept = 0u;
    float rest = 0.f;
    const float lm = finitef_(lmax) ? lmax / cfg.t_eff : -__builtin_inff();
    for (int li = tid; li < len; li += NT) {
      const float l = proc(li);
      const uint32_t kl = lkey(l);
      const uint64_t ck = cand_key(kl, (uint32_t)(c0 + li));
      const bool live = nd.lse && finitef_(lmax) && kl > kKeyNegInf;
      if (ck >= thr) {
        cand[pos++] = ck;
        minkept = ck < minkept ? ck : minkept;
      } else {
        unkept = max(unkept, kl);
        if (live) rest += exp2f((l - lmax) * a2);
      }
    }
    minkept = ~block_max_u64<NT>(~minkept, L.red64);
    unkept = block_max_u32<NT>(unkept, L.redu);
    rest = block_sum_f32<NT>(rest, L.redf);
    bs.n_cand = total;
    bs.trunc = (uint32_t)len > k ? 1u : 0u;
    bs.min_kept = minkept;
    bs.unkept_key = unkept;
    bs.lse_m = lm;
    bs.lse_sum = nd.lse ? rest : 0.f;
  }
  if (nd.whist) wide_hist_clear(L.whist);
  __syncthreads();
  if (cfg.store_s) {
    float* srow = a.ws_s + (int64_t)row * a.V + c0;
    for (int li = tid; li < len; li += NT) {
      const float l = proc(li);
      srow[li] = key_to_s(lkey(l), cfg.t_eff);
      if (nd.whist) wide_hist_add(L.whist, l, lmax, a2);
    }
  }
  if (tid == 0) a.stats[slot] = bs;
  if (nd.whist) {
    __syncthreads();
    WideStat* ws = a.wstat + slot;
    if (tid < kWideBins) ws->hist[tid] = wide_hist_bin(L.whist, tid);
    if (tid == 0) {
      ws->ms = finitef_(lmax) ? lmax / cfg.t_eff : lmax;
      ws->valid = 1u;
    }
  }
}

// Raw logits of load j as floats.
template <int DT, int EPL>
__device__ __forceinline__ void unpack16(const i32x4_t& r, float (&v)[EPL]) {
  if constexpr (DT == HI_ROCM_DTYPE_BF16) {
    #pragma unroll
    for (int w = 0; w < 4; ++w) {
      v[2 * w] = __uint_as_float((uint32_t)r[w] << 16);
      v[2 * w + 1] = __uint_as_float((uint32_t)r[w] & 0xffff0000u);
    }
  } else {
    #pragma unroll
    for (int q = 0; q < 4; ++q) v[q] = __int_as_float(r[q]);
  }
}

// One raw logit of the chunk (local index li), range-checked.
template <int DT>
__device__ __forceinline__ float load_one(const RowBuf& rb, uint32_t li) {
  if constexpr (DT == HI_ROCM_DTYPE_BF16)
    return __uint_as_float((uint32_t)(uint16_t)__builtin_amdgcn_raw_buffer_load_b16(rb.logits, li * 2, 0, 0) << 16);
  else
    return __int_as_float(__builtin_amdgcn_raw_buffer_load_b32(rb.logits, li * 4, 0, 0));
}

// Inputs every path of the select pass shares.
template <int NL>
struct SelIn {
  i32x4_t raw[NL];            // the chunk's logits, load j
  uint32_t mw[NL];            // mask word of load j
  float ob[kSelOb];           // processed logits of the chunk's history tokens
  uint32_t obi[kSelOb];       // their indices
  uint32_t n_ob;              // history tokens held out of band
};

// Lean rows (see the section comment).  Returns false when the chunk needs
// the exact path; all threads call it and get the same answer.
template <int DT, int NL, bool MASK>
__device__ __forceinline__ bool select_lean(SelLds& L, const SampleArgs& a, const RowCfg& cfg, const SelNeeds& nd,
                                            const RowBuf& rb, const float (&x)[NL * (DT == HI_ROCM_DTYPE_BF16 ? 8 : 4)],
                                            const SelIn<NL>& in, const SelHist& hv, int c0, int len, int64_t slot) {
  constexpr int EPL = DT == HI_ROCM_DTYPE_BF16 ? 8 : 4;
  constexpr int E = NL * EPL;
  constexpr int GS = E / 4;
  constexpr int NBW = (E + 31) / 32;  // bitmask words per lane
  static_assert(NBW <= 2, "survivor bitmask words");
  const int tid = threadIdx.x;
  const uint32_t lane = (uint32_t)tid & 63u;
  const int wid = tid >> 6;

  // phase A: group maxima (history tokens keep their raw logit here)
  float G[4];
  #pragma unroll
  for (int g = 0; g < 4; ++g) G[g] = -__builtin_inff();
  #pragma unroll
  for (int i = 0; i < E; ++i) G[i / GS] = fmaxf(G[i / GS], x[i]);

  // bound.  In a chunk shorter than one load per thread (the row's last)
  // only the first `act` waves hold logits: they share the count, and the
  // others set no bound.
  const uint32_t keep = chunk_keep((uint32_t)cfg.k_sel, a.n_chunks, nd.lse);
  const uint32_t k1 = nd.sel ? keep : 1u;
  const uint32_t act = (uint32_t)min(NT / 64, (len + 64 * EPL - 1) / (64 * EPL));
  const bool idle = (uint32_t)wid >= act;
  const uint32_t need = (k1 + act - 1) / act + (hv.on ? L.hw[wid] : 0u);
  uint32_t gk[4];
  bool inf = false;
  #pragma unroll
  for (int g = 0; g < 4; ++g) { gk[g] = okey(G[g]); inf |= G[g] == __builtin_inff(); }
  const uint32_t prefix = wave_prefix_reach(gk, need);
  const bool bad = !idle && (__ballot(inf) != 0ull || need > 4u * 64u || prefix <= kKeyNegInf);
  if (lane == 0u) { L.wkey[wid] = idle ? 0xffffffffu : prefix; L.wflag[wid] = bad ? 1u : 0u; }
  __syncthreads();
  uint32_t tk = L.wkey[0];
  uint32_t rare = L.wflag[0];
  #pragma unroll
  for (int w = 1; w < NT / 64; ++w) { tk = min(tk, L.wkey[w]); rare |= L.wflag[w]; }
  if (rare) return false;
  const float t = okey_inv(tk);
  const float a2 = 1.4426950408889634f / cfg.t_eff;

  // phase B: survivor bitmasks (element i of word w at bit nb - 1 - (i - 32 w))
  uint32_t bm[NBW];
  #pragma unroll
  for (int w = 0; w < NBW; ++w) bm[w] = 0u;
  #pragma unroll
  for (int i = 0; i < E; ++i) bm[i >> 5] = (bm[i >> 5] << 1) + (x[i] >= t ? 1u : 0u);
  float rest = 0.f;
  if (nd.lse) {
    // the normaliser rest relative to t (history tokens count out of band)
    #pragma unroll
    for (int j = 0; j < NL; ++j) {
      const int li0 = (j * NT + tid) * EPL;
      const uint32_t hb = (hv.on && li0 < len) ? hv.bitmap[li0 >> 5] >> (li0 & 31) : 0u;
      #pragma unroll
      for (int q = 0; q < EPL; ++q) {
        const float v = x[j * EPL + q];
        rest += (v < t && !((hb >> q) & 1u)) ? __builtin_amdgcn_exp2f((v - t) * a2) : 0.f;
      }
    }
  }
  // survivors of this lane: streamed ones (re-read, history tokens
  // skipped) and out-of-band history tokens
  uint32_t nbits = 0u;
  #pragma unroll
  for (int w = 0; w < NBW; ++w) nbits += (uint32_t)__popc(bm[w]);
  uint32_t nob = 0u;
  #pragma unroll
  for (int i = 0; i < kSelOb; ++i) {
    const float o = in.ob[i];
    nob += o >= t ? 1u : 0u;
    if (nd.lse) rest += o < t ? __builtin_amdgcn_exp2f((o - t) * a2) : 0.f;
  }
  // the wave's list: out-of-band survivors, then the streamed ones in rounds
  // of up to kLaneSurv per lane (a list past kSurvCap takes the exact path)
  uint64_t* surv = L.surv[wid];
  uint32_t mkey = 0u;
  uint32_t wtot;
  {
    const uint32_t incl = wave_incl_scan_u32(nob);
    uint32_t pos = incl - nob;
    wtot = wave_last_u32(incl);
    #pragma unroll
    for (int i = 0; i < kSelOb; ++i) {
      if (in.ob[i] >= t) {
        const uint32_t kv = okey(in.ob[i]);
        surv[pos++] = cand_key(kv, in.obi[i]);
        mkey = max(mkey, kv);
      }
    }
  }
  (void)nbits;
  #pragma unroll 1
  while (__ballot(bm[0] != 0u || bm[NBW - 1] != 0u) != 0ull && wtot <= (uint32_t)kSurvCap) {
    float sv[kLaneSurv];
    uint32_t si[kLaneSurv];
    uint32_t sok = 0u;  // bit s: slot s holds a survivor
    #pragma unroll
    for (int s = 0; s < kLaneSurv; ++s) {
      int w = 0;
      #pragma unroll
      for (int ww = NBW - 1; ww >= 0; --ww) if (bm[ww] != 0u) w = ww;
      const uint32_t word = w == 0 ? bm[0] : bm[NBW - 1];
      const int nb = (w + 1) * 32 <= E ? 32 : E - w * 32;
      const bool has = word != 0u;
      const int b = has ? 31 - __clz(word) : 0;
      const int i = w * 32 + (nb - 1 - b);
      if (has) {
        if (w == 0) bm[0] &= ~(1u << b);
        else bm[NBW - 1] &= ~(1u << b);
      }
      const int j = i / EPL, q = i % EPL;
      const uint32_t li = (uint32_t)((j * NT + tid) * EPL + q);
      const bool take = has && !hist_marked(hv, li);
      si[s] = li;
      sv[s] = take ? load_one<DT>(rb, li) : 0.f;
      sok |= take ? (1u << s) : 0u;
    }
    const uint32_t mine = (uint32_t)__popc(sok);
    const uint32_t incl = wave_incl_scan_u32(mine);
    const uint32_t rtot = wave_last_u32(incl);
    if (wtot + rtot <= (uint32_t)kSurvCap) {
      uint32_t pos = wtot + incl - mine;
      #pragma unroll
      for (int s = 0; s < kLaneSurv; ++s) {
        if ((sok >> s) & 1u) {
          const uint32_t kv = okey(sv[s]);
          surv[pos++] = cand_key(kv, (uint32_t)c0 + si[s]);
          mkey = max(mkey, kv);
        }
      }
    }
    wtot += rtot;
  }
  // the wave's smallest and largest entries, and the finite-lane argmax key
  // (index mod 256, index) among its largest values
  (void)mkey;
  wave_lds_sync();
  const uint32_t wn = min(wtot, (uint32_t)kSurvCap);
  uint64_t wmin = ~0ull, wmax = 0ull;
  for (uint32_t i = lane; i < wn; i += 64u) {
    const uint64_t e = surv[i];
    wmin = e < wmin ? e : wmin;
    wmax = e > wmax ? e : wmax;
  }
  wmin = wave_min_u64(wmin);
  wmax = wave_max_u64(wmax);
  uint64_t wfin = ~0ull;
  if (nd.fin) {
    for (uint32_t i = lane; i < wn; i += 64u) {
      const uint64_t e = surv[i];
      if (cand_skey(e) == cand_skey(wmax)) {
        const uint32_t idx = cand_idx(e);
        const uint64_t fk = ((uint64_t)fin_order(idx) << 32) | idx;
        wfin = fk < wfin ? fk : wfin;
      }
    }
    wfin = wave_min_u64(wfin);
  }
  if (nd.lse) rest = wave_sum_f32(rest);
  if (lane == 0u) {
    L.wcnt[wid] = wtot;
    L.red64[wid] = wmin;
    L.red64b[wid] = wmax;
    L.red64c[wid] = wfin;
    L.redf[wid] = rest;
  }
  __syncthreads();
  uint32_t n = 0u, off = 0u;
  uint64_t best = 0ull;
  #pragma unroll
  for (int w = 0; w < NT / 64; ++w) {
    if (L.wcnt[w] > (uint32_t)kSurvCap) return false;
    if (w < wid) off += L.wcnt[w];
    n += L.wcnt[w];
    best = L.red64b[w] > best ? L.red64b[w] : best;
  }
  if (nd.sel && n > (uint32_t)kFast) return false;
  const uint32_t mk = cand_skey(best);
  const float m = okey_inv(mk);
  if ((nd.ieee || nd.fin) && m == 0.f) return false;  // -0 / +0 ties: IEEE compare rules

  // every survivor is a candidate: each wave writes its list at its offset
  if (nd.sel) {
    uint64_t* cand = a.cand + slot * kFast + off;
    for (uint32_t i = lane; i < wtot; i += 64u) cand[i] = surv[i];
  }
  if (wid != 0) return true;
  if (lane == 0u) {
    ChunkStat bs;
    stat_init(bs);
    bs.max_l = m;
    bs.any_finite = 1u;
    uint64_t mn = ~0ull, fb = ~0ull;
    float rs = 0.f;
    #pragma unroll
    for (int w = 0; w < NT / 64; ++w) {
      mn = L.red64[w] < mn ? L.red64[w] : mn;
      if (cand_skey(L.red64b[w]) == mk) fb = L.red64c[w] < fb ? L.red64c[w] : fb;
      rs += L.redf[w];
    }
    if (nd.sel) {
      bs.n_cand = n;
      bs.trunc = n < (uint32_t)len ? 1u : 0u;
      bs.min_kept = mn;
      // the logits that are not candidates have keys below tk
      bs.unkept_key = n < (uint32_t)len ? tk - 1u : 0u;
      bs.lse_m = m / cfg.t_eff;
      bs.lse_sum = nd.lse ? rs * __builtin_amdgcn_exp2f((t - m) * a2) : 0.f;
    }
    if (nd.ieee) { bs.am_ieee_v = m; bs.am_ieee_i = cand_idx(best); }
    if (nd.fin) { bs.am_fin_v = m; bs.am_fin_i = (uint32_t)fb; }
    a.stats[slot] = bs;
  }
  return true;
}

// Rows that keep their scaled logits (see the section comment).  Returns
// false when the chunk needs the exact path; all threads call it.
template <int DT, int NL, bool MASK>
__device__ __forceinline__ bool select_wide(SelLds& L, const SampleArgs& a, const RowCfg& cfg, const SelNeeds& nd,
                                            float (&x)[NL * (DT == HI_ROCM_DTYPE_BF16 ? 8 : 4)], const SelIn<NL>& in,
                                            const SelHist& hv, int row, int c0, int len, int64_t slot) {
  constexpr int EPL = DT == HI_ROCM_DTYPE_BF16 ? 8 : 4;
  constexpr int E = NL * EPL;
  constexpr int GS = E / 4;
  constexpr uint32_t EMASK = (1u << EPL) - 1u;
  const int tid = threadIdx.x;
  const uint32_t lane = (uint32_t)tid & 63u;
  const int wid = tid >> 6;

  // phase A: history tokens absent (NaN), maxima
  float G[4];
  #pragma unroll
  for (int g = 0; g < 4; ++g) G[g] = -__builtin_inff();
  #pragma unroll
  for (int j = 0; j < NL; ++j) {
    const int li0 = (j * NT + tid) * EPL;
    if (hv.on) {
      const uint32_t hb = li0 < len ? (hv.bitmap[li0 >> 5] >> (li0 & 31)) & EMASK : 0u;
      #pragma unroll
      for (int q = 0; q < EPL; ++q) x[j * EPL + q] = ((hb >> q) & 1u) ? __builtin_nanf("") : x[j * EPL + q];
    }
    #pragma unroll
    for (int q = 0; q < EPL; ++q) {
      const int i = j * EPL + q;
      G[i / GS] = fmaxf(G[i / GS], x[i]);
    }
  }
  float lm = fmaxf(fmaxf(G[0], G[1]), fmaxf(G[2], G[3]));
  #pragma unroll
  for (int i = 0; i < kSelOb; ++i) lm = fmaxf(lm, in.ob[i]);

  // wave bound (candidates for logprobs) and workgroup statistics
  const float wm = wave_max_f32(lm);
  uint32_t flag = (hv.ovf || wm == __builtin_inff()) ? 1u : 0u;
  uint32_t tkey = 0xffffffffu;
  if (nd.sel) {
    const uint32_t k1w = ((uint32_t)cfg.k_sel + (NT / 64) - 1) / (NT / 64);
    const int J = k1w <= 16u ? 1 : (k1w <= 32u ? 2 : 4);
    uint32_t gk[4];
    if (J == 1) {
      gk[0] = okey(fmaxf(fmaxf(G[0], G[1]), fmaxf(G[2], G[3])));
      gk[1] = gk[2] = gk[3] = 0u;
    } else if (J == 2) {
      gk[0] = okey(fmaxf(G[0], G[1]));
      gk[1] = okey(fmaxf(G[2], G[3]));
      gk[2] = gk[3] = 0u;
    } else {
      #pragma unroll
      for (int g = 0; g < 4; ++g) gk[g] = okey(G[g]);
    }
    const uint32_t prefix = wave_prefix_reach(gk, k1w);
    tkey = prefix;
    if (prefix <= kKeyNegInf) flag = 1u;
  }
  if (lane == 0u) { L.wmax[wid] = wm; L.wkey[wid] = tkey; L.wflag[wid] = flag; }
  if (nd.whist) wide_hist_clear(L.whist);
  __syncthreads();
  float m = L.wmax[0];
  uint32_t tk = L.wkey[0];
  uint32_t rare = L.wflag[0];
  #pragma unroll
  for (int w = 1; w < NT / 64; ++w) { m = fmaxf(m, L.wmax[w]); tk = min(tk, L.wkey[w]); rare |= L.wflag[w]; }
  // a chunk with no finite logit is fine for a row that only needs its
  // scaled logits and mass (a top-p row's masked-out or short chunk)
  const bool empty_ok = m == -__builtin_inff() && !nd.sel && !nd.ieee && !nd.fin && !nd.lse;
  if ((!finitef_(m) && !empty_ok) || ((nd.ieee || nd.fin) && m == 0.f)) rare = 1u;
  if (rare) return false;
  // candidates need t = the bound; an argmax alone needs the ties of m
  const float t = nd.sel ? okey_inv(tk) : m;
  const float a2 = 1.4426950408889634f / cfg.t_eff;

  // phase B
  uint32_t cnt = 0u;
  float rest = 0.f;
  uint64_t* surv = L.surv[wid];
  #pragma unroll
  for (int j = 0; j < NL; ++j) {
    const int li0 = (j * NT + tid) * EPL;
    #pragma unroll
    for (int q = 0; q < EPL; ++q) {
      const float v = x[j * EPL + q];
      if (nd.surv) {
        const bool s = v >= t;
        const uint64_t bmk = __ballot(s);
        if (bmk != 0ull) {
          const uint32_t p = cnt + lanes_below(bmk);
          if (s && p < (uint32_t)kSurvCap) surv[p] = cand_key(okey(v), (uint32_t)(c0 + li0 + q));
          cnt += (uint32_t)__popcll(bmk);
        }
      }
      if (nd.lse) rest += v < t ? __builtin_amdgcn_exp2f((v - m) * a2) : 0.f;
      if (nd.whist) wide_hist_add(L.whist, v, m, a2);
    }
    if (cfg.store_s) {
      float svl[EPL];
      #pragma unroll
      for (int q = 0; q < EPL; ++q) {
        const float v = x[j * EPL + q];
        svl[q] = finitef_(v) ? v / cfg.t_eff : -__builtin_inff();
      }
      float* dst = a.ws_s + (int64_t)row * a.V + c0 + li0;
      const uint32_t hb = (hv.on && li0 < len) ? (hv.bitmap[li0 >> 5] >> (li0 & 31)) & EMASK : 0u;
      if (li0 + EPL <= len && hb == 0u && ((a.V & 3) == 0)) {
        #pragma unroll
        for (int q = 0; q < EPL; q += 4) *(float4*)(dst + q) = make_float4(svl[q], svl[q + 1], svl[q + 2], svl[q + 3]);
      } else {
        #pragma unroll
        for (int q = 0; q < EPL; ++q) if (li0 + q < len && !((hb >> q) & 1u)) dst[q] = svl[q];
      }
    }
  }
  #pragma unroll
  for (int i = 0; i < kSelOb; ++i) {
    const float v = in.ob[i];
    if (nd.surv) {
      const bool s = v >= t;
      const uint64_t bmk = __ballot(s);
      if (bmk != 0ull) {
        const uint32_t p = cnt + lanes_below(bmk);
        if (s && p < (uint32_t)kSurvCap) surv[p] = cand_key(okey(v), in.obi[i]);
        cnt += (uint32_t)__popcll(bmk);
      }
    }
    if (nd.lse) rest += v < t ? __builtin_amdgcn_exp2f((v - m) * a2) : 0.f;
    if (nd.whist) wide_hist_add(L.whist, v, m, a2);
    if (cfg.store_s && (uint32_t)(i * NT + tid) < in.n_ob)
      a.ws_s[(int64_t)row * a.V + in.obi[i]] = finitef_(v) ? v / cfg.t_eff : -__builtin_inff();
  }
  if (nd.lse) rest = wave_sum_f32(rest);
  if (lane == 0u) { L.wcnt[wid] = cnt; L.redf[wid] = rest; }
  __syncthreads();
  uint32_t n = 0u;
  #pragma unroll
  for (int w = 0; w < NT / 64; ++w) { n += L.wcnt[w]; rare |= L.wcnt[w] > (uint32_t)kSurvCap ? 1u : 0u; }
  if (rare) return false;
  if (wid != 0) return true;

  // wave 0: the chunk's top k_sel of the survivors, argmaxes, record
  Segs<NT / 64> sg;
  float rs = 0.f;
  #pragma unroll
  for (int w = 0; w < NT / 64; ++w) { sg.p[w] = L.surv[w]; sg.n[w] = L.wcnt[w]; rs += L.redf[w]; }
  sg.ns = NT / 64;
  const uint32_t k = (uint32_t)cfg.k_sel;
  uint64_t thr = 0ull;
  if (nd.sel && n > k) thr = wave_select_skip(sg, k, L.hist);
  const uint32_t mkey = okey(m);
  uint64_t* cand = a.cand + slot * kFast;
  uint32_t wpos = 0u, unkept = 0u;
  uint64_t minkept = ~0ull, best = 0ull, finb = ~0ull;
  float urest = 0.f;
  #pragma unroll
  for (int w = 0; w < NT / 64; ++w) {
    const uint32_t nw = sg.n[w];
    for (uint32_t b0 = 0; b0 < nw; b0 += 64u) {
      const uint32_t i = b0 + lane;
      const bool valid = i < nw;
      const uint64_t e = valid ? sg.p[w][i] : 0ull;
      const bool keep = valid && nd.sel && e >= thr;
      const uint64_t km = __ballot(keep);
      if (keep) {
        cand[wpos + lanes_below(km)] = e;
        minkept = e < minkept ? e : minkept;
      }
      wpos += (uint32_t)__popcll(km);
      if (valid) {
        best = e > best ? e : best;
        if (cand_skey(e) == mkey) {
          const uint32_t idx = cand_idx(e);
          const uint64_t fk = ((uint64_t)fin_order(idx) << 32) | idx;
          finb = fk < finb ? fk : finb;
        }
        if (nd.sel && !keep) {
          unkept = max(unkept, cand_skey(e));
          if (nd.lse) urest += __builtin_amdgcn_exp2f((okey_inv(cand_skey(e)) - m) * a2);
        }
      }
    }
  }
  minkept = wave_min_u64(minkept);
  best = wave_max_u64(best);
  finb = wave_min_u64(finb);
  unkept = wave_max_u32(unkept);
  if (nd.lse) urest = wave_sum_f32(urest);
  if (lane == 0u) {
    ChunkStat bs;
    stat_init(bs);
    bs.max_l = m;
    bs.any_finite = finitef_(m) ? 1u : 0u;
    if (nd.sel) {
      bs.n_cand = wpos;
      bs.trunc = (uint32_t)len > k ? 1u : 0u;
      bs.min_kept = minkept;
      bs.unkept_key = max(unkept, n < (uint32_t)len ? tk - 1u : 0u);
      bs.lse_m = m / cfg.t_eff;
      bs.lse_sum = nd.lse ? rs + urest : 0.f;
    }
    if (nd.ieee) { bs.am_ieee_v = m; bs.am_ieee_i = cand_idx(best); }
    if (nd.fin) { bs.am_fin_v = m; bs.am_fin_i = (uint32_t)finb; }
    a.stats[slot] = bs;
  }
  if (nd.whist) {
    WideStat* ws = a.wstat + slot;
    if (lane < (uint32_t)kWideBins) ws->hist[lane] = wide_hist_bin(L.whist, (int)lane);
    if (lane == 0u) {
      ws->ms = m / cfg.t_eff;
      ws->valid = 1u;
    }
  }
  return true;
}

// One (chunk, row) of the streaming select pass, by one workgroup.  DT:
// logit dtype; NL: 16-byte loads per thread; MASK: an allowed-token bitmask
// is given.  lds_raw holds SelLds and the history table.
template <int DT, int NL, bool MASK>
__device__ __forceinline__ void select_chunk(const SampleArgs& a, int row, int chunk, unsigned char* lds_raw) {
  SelLds& L = *reinterpret_cast<SelLds*>(lds_raw);
  constexpr int EPL = DT == HI_ROCM_DTYPE_BF16 ? 8 : 4;  // logits per 16-byte load
  constexpr int ESZ = DT == HI_ROCM_DTYPE_BF16 ? 2 : 4;
  constexpr int E = NL * EPL;                             // logits per thread
  constexpr int CH = NT * E;
  static_assert(E % 4 == 0 && CH % 32 == 0, "chunk shape");
  const int tid = threadIdx.x;
  const int c0 = chunk * CH;
  const int len = min(CH, a.V - c0);
  const int64_t slot = (int64_t)row * a.n_chunks + chunk;

  // 1. the row's history list, then the chunk's logits and mask words
  uint32_t h0 = 0u, h1 = 0u;
  uint32_t hid[kSelHistPer], hcs[kSelHistPer];
  if (a.hoff) { h0 = a.hoff[row]; h1 = a.hoff[row + 1]; }
  #pragma unroll
  for (int r = 0; r < kSelHistPer; ++r) {
    const uint32_t h = h0 + (uint32_t)(r * NT + tid);
    hid[r] = h < h1 ? a.hids[h] : 0xffffffffu;
    hcs[r] = h < h1 ? a.hcnt[h] : 0u;
  }
  const RowBuf rb = row_buf<DT, MASK>(a, row, c0, c0 + len);
  SelIn<NL> in;
  #pragma unroll
  for (int j = 0; j < NL; ++j) {
    const int li0 = (j * NT + tid) * EPL;
    in.raw[j] = __builtin_amdgcn_raw_buffer_load_b128(rb.logits, li0 * ESZ, 0, 0);
    if (MASK) in.mw[j] = (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(rb.mask, (li0 >> 5) * 4, 0, 0);
  }
  const RowCfg cfg = load_cfg(a.pv, row, a.V, a.n_lp, a.need_lse);
  const SelNeeds nd = sel_needs(a, cfg);

  // 2. history table, then the out-of-band history logits
  const SelHist hv = stage_history_sel(a, c0, len, EPL, reinterpret_cast<uint32_t*>(lds_raw + kSelHead), L.hw, hid,
                                       hcs, h0, h1);
  in.n_ob = hv.on ? min(hv.distinct, kSelHistCap) : 0u;
  uint32_t obm[kSelOb];
  #pragma unroll
  for (int i = 0; i < kSelOb; ++i) {
    const uint32_t r = (uint32_t)(i * NT + tid);
    in.obi[i] = r < in.n_ob ? hv.ids[r] : (uint32_t)c0;
    const uint32_t li = in.obi[i] - (uint32_t)c0;
    in.ob[i] = load_one<DT>(rb, li);
    obm[i] = MASK ? (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(rb.mask, (li >> 5) * 4, 0, 0) >> (li & 31u) : 1u;
  }
  #pragma unroll
  for (int i = 0; i < kSelOb; ++i) {
    const uint32_t r = (uint32_t)(i * NT + tid);
    if (r < in.n_ob) {
      const float l = (obm[i] & 1u) ? in.ob[i] : -__builtin_inff();
      in.ob[i] = apply_penalties(l, hv.cnts[r], cfg);
    } else {
      in.ob[i] = __builtin_nanf("");
    }
  }

  // 3. the chunk's logits as floats: mask as -inf, past the range absent
  float x[E];
  #pragma unroll
  for (int j = 0; j < NL; ++j) {
    const int li0 = (j * NT + tid) * EPL;
    float v[EPL];
    unpack16<DT, EPL>(in.raw[j], v);
    if (MASK) {
      const uint32_t bits = in.mw[j] >> (li0 & 31);
      #pragma unroll
      for (int q = 0; q < EPL; ++q) v[q] = ((bits >> q) & 1u) ? v[q] : -__builtin_inff();
    }
    if (len != CH) {
      #pragma unroll
      for (int q = 0; q < EPL; ++q) v[q] = li0 + q < len ? v[q] : __builtin_nanf("");
    }
    #pragma unroll
    for (int q = 0; q < EPL; ++q) x[j * EPL + q] = v[q];
  }

  // 4. the row's path
  bool done;
  if (cfg.store_s) {
    done = select_wide<DT, NL, MASK>(L, a, cfg, nd, x, in, hv, row, c0, len, slot);
  } else if (hv.ovf) {
    done = false;
  } else {
    done = select_lean<DT, NL, MASK>(L, a, cfg, nd, rb, x, in, hv, c0, len, slot);
  }
  if (done) return;
  __syncthreads();
  select_exact(L, a, cfg, hv, nd, row, c0, len, slot);
}

// The streaming select pass: workgroup (chunk, row).
__device__ __forceinline__ void wide_row_prepare(SelLds& L, const SampleArgs& a, int row, const RowCfg& cfg);

template <int DT, int NL, bool MASK>
__global__ void __launch_bounds__(NT) select_kernel(SampleArgs a) {
  extern __shared__ __align__(16) unsigned char lds_raw[];
  const int row = blockIdx.y;
  select_chunk<DT, NL, MASK>(a, row, blockIdx.x, lds_raw);
  const RowCfg cfg = load_cfg(a.pv, row, a.V, a.n_lp, a.need_lse);
  if (cfg.cls != kTopP) return;
  // top-p rows: the last workgroup of the row merges the chunks' maxima and
  // mass histograms for the wide pass (as select_finish_kernel's counter)
  SelLds& L = *reinterpret_cast<SelLds*>(lds_raw);
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  uint32_t* counter = a.done + row;
  if (threadIdx.x == 0) {
    __threadfence();
    L.wflag[0] = atomicAdd(counter, 1u) == (uint32_t)(a.n_chunks - 1) ? 1u : 0u;
    if (L.wflag[0]) {
      __threadfence();
      *counter = 0u;
    }
  }
  __syncthreads();
  if (L.wflag[0] == 0u) return;
  wide_row_prepare(L, a, row, cfg);
}

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

// ==========================================================================
// Wide pass: top-p rows without a top-k bound (gpu.rs:820-899 with
// top_k unset), chunk-parallel
// ==========================================================================
//
// The reference walks such a row's whole rank order with three sequential
// f32 folds: the normaliser over every weight in vocabulary order
// (gpu.rs:837), then cum_p += w / total in rank order up to the cutoff
// (:843-856), then the candidate total and the inverse CDF (:874-899).  Here
// the select pass leaves the scaled logits s in ws_s and a mass histogram
// per chunk (WideStat); then one workgroup per (chunk, row):
//   1. merges the row's chunk maxima (M) and histograms: a conservative
//      weight bound w_lo such that the weights >= w_lo hold at least
//      cutoff + kWideMargin of the mass (every weight of the nucleus is
//      >= w_lo unless the f32 folds differ from exact sums by more than the
//      margin, which the finish detects), and the predicted sum before the
//      chunk;
//   2. computes its weights w = expf(s - M) exactly (min-p zeros them),
//      plans its part of the vocabulary-order fold (fold_plan: segments of
//      one predicted binade and boundary terms) and writes the plan;
//   3. counts its weights >= w_lo by distinct value in an LDS hash: the
//      rank order only needs each distinct weight's multiplicity (equal
//      weights rank by index, and the folds do not see indices);
//   4. bumps the row's counter; the last workgroup finishes the row:
//      chains the chunk plans into the exact normaliser (refolding a chunk
//      whose prediction missed), merges the chunks' runs, sorts them
//      (weight descending), folds cum_p, the candidate total and the CDF
//      over the runs with the closed forms for equal terms, and finds the
//      drawn index among the equal weights of the drawn run.
// Rows whose chunks took the select pass's exact path, whose tables
// overflow, or whose nucleus is not inside the superset take finish_row.

constexpr float kWideMargin = 0.005f;  // extra probability mass of the superset
constexpr int kWideChunkHash = 2048;   // distinct superset weights per chunk
constexpr int kWideFinHash = 2048;     // distinct superset weights per row
constexpr int kWideRunCap = kWideFinHash;
constexpr int kWideBatch = 64;         // chunk plans the chain holds in LDS at a time
constexpr int kWideGBins = 64;         // threshold bins (binades of w below M)

// LDS of a (chunk, row) workgroup; the chunk's weights and fold binades
// follow at wide_w_off / wide_pe_off.
struct WideChunkLds {
  fold::WgLds<NT> fl;
  uint32_t hkey[kWideChunkHash];
  uint32_t hcnt[kWideChunkHash];
  uint32_t hmin[kWideChunkHash];
  uint32_t nrun, ovf, last, fu;
  float fend;
};
constexpr size_t kWideChunkHead = (sizeof(WideChunkLds) + 15) & ~(size_t)15;
// Weights sit in LDS with one pad word per 16, so that threads reading
// their own 16 consecutive terms hit distinct banks.
__host__ __device__ inline int wide_pad(int i) { return i + (i >> 4); }
__host__ __device__ inline size_t wide_w_bytes(int chunk) { return (size_t)wide_pad(chunk) * 4 + 16; }
__host__ __device__ inline size_t wide_w_off(int) { return kWideChunkHead; }
__host__ __device__ inline size_t wide_pe_off(int chunk) { return kWideChunkHead + wide_w_bytes(chunk); }
__host__ __device__ inline size_t wide_chunk_lds(int chunk) { return wide_pe_off(chunk) + (size_t)chunk + 16; }

// LDS of the row finish.  Its phases reuse one union: the chain (chunk
// plans, and the refold arrays past them), the merge (hash table and sort
// keys), the draw (runs in rank order and the fold values before them).
struct WideFinLds {
  fold::WgLds<NT> fl;
  union {
    struct {
      ChunkFold batch[kWideBatch];
    } ch;
    struct {
      uint32_t hkey[kWideFinHash];
      uint32_t hcnt[kWideFinHash];
      uint32_t hmin[kWideFinHash];
      uint64_t sortk[kWideRunCap];
    } mg;
    struct {
      float rx[kWideRunCap];   // weight of run r (rank order)
      uint32_t rm[kWideRunCap];  // its multiplicity
      uint32_t ri[kWideRunCap];  // its smallest index
      float st[kWideRunCap];   // cum_p before run r
      float st2[kWideRunCap];  // candidate weight sum before run r
    } fo;
    uint32_t cntc[kWideRunCap];  // the drawn weight's multiplicity per chunk
  } u;
  uint8_t pe[kWideRunCap + 4];
  uint32_t noff[NT + 1];
  uint32_t cnt, fail_c, rsel, csel, tok, fu;
  float acc, acc2;
};
// The refold arrays (weights, then fold binades) start after the chain's
// plans, inside or past the union.
__host__ __device__ inline size_t wide_fin_w_off() {
  return (offsetof(WideFinLds, u) + sizeof(ChunkFold) * kWideBatch + 15) & ~(size_t)15;
}
__host__ __device__ inline size_t wide_fin_lds(int chunk) {
  const size_t r = wide_fin_w_off() + wide_w_bytes(chunk);
  return r > sizeof(WideFinLds) ? r : sizeof(WideFinLds);
}

__device__ __forceinline__ uint32_t wide_hash(uint32_t key, int log2n) {
  return (key * 0x9E3779B1u) >> (32 - log2n);
}

// Inserts `count` copies of weight bits `key` with smallest index `idx`
// into an LDS table of 2^log2n slots (key 0 = empty; weights here are > 0).
// Returns false when the table is full.
__device__ __forceinline__ bool wide_insert(uint32_t* hkey, uint32_t* hcnt, uint32_t* hmin, int log2n,
                                            uint32_t key, uint32_t count, uint32_t idx) {
  const uint32_t mask = (1u << log2n) - 1u;
  uint32_t h = wide_hash(key, log2n);
  for (uint32_t probe = 0; probe <= mask; ++probe, h = (h + 1u) & mask) {
    const uint32_t old = atomicCAS(&hkey[h], 0u, key);
    if (old == 0u || old == key) {
      atomicAdd(&hcnt[h], count);
      atomicMin(&hmin[h], idx);
      return true;
    }
  }
  return false;
}

// Step 1, once per top-p row, by the select pass's last workgroup of the
// row: M, the superset bound w_lo and the predicted fold value before each
// chunk (WideRow, WideStat::pred).  The masses use approximate exp; they
// only size the superset and predict binades.
__device__ __forceinline__ void wide_row_prepare(SelLds& L, const SampleArgs& a, int row, const RowCfg& cfg) {
  const int tid = threadIdx.x;
  const int nch = a.n_chunks;
  const ChunkStat* stats = a.stats + (int64_t)row * nch;
  WideStat* wst = a.wstat + (int64_t)row * nch;
  uint32_t mk = 0u, bad = 0u;
  for (int c = tid; c < nch; c += NT) {
    mk = max(mk, okey(stats[c].max_l));
    bad |= wst[c].valid ^ 1u;
  }
  unsigned long long* gmass = reinterpret_cast<unsigned long long*>(L.surv[0]);  // kWideGBins entries
  if (tid < kWideGBins) gmass[tid] = 0ull;
  mk = block_max_u32<NT>(mk, L.redu);
  bad = block_max_u32<NT>(bad, L.redu);
  const float ml = okey_inv(mk);
  const float M = finitef_(ml) ? ml / cfg.t_eff : -__builtin_inff();
  WideRow* wr = a.wrow + row;
  if (!finitef_(M) || bad) {
    if (tid == 0) { wr->valid = 0u; wr->M = M; wr->w_lo = 0.f; }
    return;
  }
  // chunk masses relative to M, in fixed point (2^-32): per binade of their
  // lower end (for w_lo) and per chunk (for the predictions); one (chunk,
  // bin) pair per thread step, so the whole workgroup works on every chunk
  unsigned long long* cmass = reinterpret_cast<unsigned long long*>(L.surv[1]);  // up to kSurvCap chunks at a time
  double S = 0.0;  // thread 0: the running prediction
  for (int cb = 0; cb < nch; cb += kSurvCap) {
    const int nb = min(kSurvCap, nch - cb);
    for (int i = tid; i < nb; i += NT) cmass[i] = 0ull;
    __syncthreads();
    for (int it = tid; it < nb * kWideBins; it += NT) {
      const int i = it / kWideBins, j = it % kWideBins;
      const WideStat& ws = wst[cb + i];
      const float lb = (M - ws.ms) * 1.4426950408889634f;  // log2 of M's weight over the chunk max's
      const float m = ws.hist[j] * __builtin_amdgcn_exp2f(-lb);
      if (!(m > 0.f)) continue;
      const unsigned long long fx = (unsigned long long)((double)m * 4294967296.0);
      int g = j == kWideBins - 1 ? kWideGBins - 1 : (int)floorf((float)(j + 1) + lb);
      g = g < kWideGBins ? g : kWideGBins - 1;
      atomicAdd(&gmass[g], fx);
      atomicAdd(&cmass[i], fx);
    }
    __syncthreads();
    if (tid == 0) {
      for (int i = 0; i < nb; ++i) {
        wst[cb + i].pred = S;
        S += (double)cmass[i] * (1.0 / 4294967296.0);
      }
    }
    __syncthreads();
  }
  if (tid == 0) {
    unsigned long long tot = 0ull;
    for (int g = 0; g < kWideGBins; ++g) tot += gmass[g];
    const double frac = (double)cfg.cutoff + (double)kWideMargin;
    float w_lo = 0.f;
    if (cfg.cutoff < 1.f && frac < 1.0) {
      const unsigned long long target = (unsigned long long)(frac * (double)tot);
      unsigned long long cum = 0ull;
      for (int g = 0; g < kWideGBins - 1; ++g) {
        cum += gmass[g];
        if (cum >= target) { w_lo = __builtin_ldexpf(1.f, -(g + 1)); break; }
      }
    }
    wr->w_lo = fmaxf(w_lo, cfg.min_p);
    wr->M = M;
    wr->valid = 1u;
  }
}

// w[wide_pad(i)] = the weight of scaled logit s[i] (exact expf; min-p
// zeros it), i < len: all of a thread's loads of a block are issued before
// any is used.
__device__ __forceinline__ void wide_weights(const float* s, int len, float M, float min_p, float* w) {
  constexpr int kB = 8;
  for (int base = 0; base < len; base += kB * NT) {
    float v[kB];
    #pragma unroll
    for (int k = 0; k < kB; ++k) {
      const int i = base + k * NT + (int)threadIdx.x;
      v[k] = i < len ? s[i] : -__builtin_inff();
    }
    #pragma unroll
    for (int k = 0; k < kB; ++k) {
      const int i = base + k * NT + (int)threadIdx.x;
      const float x = exact_expf(v[k] - M);
      if (i < len) w[wide_pad(i)] = x < min_p ? 0.f : x;  // min-p: excluded like a zero weight
    }
  }
}

// Map of one term in binade e (exact_fold.h): n ulps, plus one above half
// an ulp, plus one on an exact half when that makes the sum even.
__device__ __forceinline__ fold::Map term_map(float x, int e) {
  const fold::Inc c = fold::classify(x, e);
  const uint32_t base = c.n + (c.cls == 2u ? 1u : 0u);
  const uint32_t odd = c.n & 1u;
  fold::Map m;
  m.t0 = base + ((c.cls == 1u && odd) ? 1u : 0u);
  m.t1 = base + ((c.cls == 1u && !odd) ? 1u : 0u);
  return m;
}

// Exclusive scan of maps over the workgroup in thread order; *tot gets the
// composition of all.  Two barriers.
__device__ __forceinline__ fold::Map block_map_scan(fold::Map m, fold::Map* wm, fold::Map* tot) {
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  fold::Map inc = m;
  #pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    fold::Map o;
    o.t0 = (uint32_t)__shfl_up((int)inc.t0, (unsigned)d, 64);
    o.t1 = (uint32_t)__shfl_up((int)inc.t1, (unsigned)d, 64);
    if (lane >= d) inc = fold::compose(o, inc);
  }
  fold::Map ex;
  ex.t0 = (uint32_t)__shfl_up((int)inc.t0, 1u, 64);
  ex.t1 = (uint32_t)__shfl_up((int)inc.t1, 1u, 64);
  if (lane == 0) ex = fold::map_identity();
  __syncthreads();
  if (lane == 63) wm[wid] = inc;
  __syncthreads();
  fold::Map before = fold::map_identity(), all = fold::map_identity();
  #pragma unroll
  for (int w = 0; w < NT / 64; ++w) {
    if (w < wid) before = fold::compose(before, wm[w]);
    all = fold::compose(all, wm[w]);
  }
  *tot = all;
  return fold::compose(before, ex);
}

// The exact sequential f32 fold of w[wide_pad(0 .. len)) (LDS) from a0, by
// the workgroup.  Thread t holds a block of consecutive terms; in the
// current binade every block is one map, so a scan gives each block's
// exact start until the first block whose terms leave the binade.  That
// thread adds its terms (and, while crossings come close together, the
// next blocks' terms) as real f32 additions, and the scan resumes after
// them in the new binade.  Returns the sum (uniform).
__device__ __forceinline__ float exact_chunk_fold(const float* w, int len, float a0, fold::Map* wm, float* shf,
                                                  uint32_t* red) {
  constexpr int kSeqBlocks = 4;  // blocks one thread adds after a crossing
  const int tid = threadIdx.x;
  const int J = (len + NT - 1) / NT;
  const int r0 = min(tid * J, len), r1 = min(r0 + J, len);
  float a = a0;
  int pos = 0;
  while (pos < NT) {
    const int e = fold::binade(a);
    const uint32_t A = fold::to_A(a);
    fold::Map m = fold::map_identity();
    if (tid >= pos)
      for (int r = r0; r < r1; ++r) m = fold::compose(m, term_map(w[wide_pad(r)], e));
    fold::Map tot;
    const fold::Map ex = block_map_scan(m, wm, &tot);
    const uint32_t p = A & 1u;
    if ((uint64_t)A + fold::apply(tot, p) < fold::kTop) {
      a = fold::from_A(A + fold::apply(tot, p), e);
      break;
    }
    const uint64_t At = (uint64_t)A + fold::apply(ex, p);
    const bool cross = tid >= pos && (At >= fold::kTop || At + fold::apply(m, (uint32_t)At & 1u) >= fold::kTop);
    uint32_t first = ~block_max_u32<NT>(cross ? ~(uint32_t)tid : 0u, red);
    if (first == 0xffffffffu) first = (uint32_t)pos;  // (not reached: the total leaves the binade)
    if (tid == (int)first) {
      // At < kTop: the blocks before this one stayed in the binade
      float x = fold::from_A((uint32_t)At, e);
      const int stop = min(len, (tid + kSeqBlocks) * J);
      for (int r = r0; r < stop; ++r) x = fold::fadd(x, w[wide_pad(r)]);
      shf[0] = x;
    }
    __syncthreads();
    a = shf[0];
    pos = (int)first + kSeqBlocks;
    __syncthreads();
  }
  return a;
}

// Steps 2-3 for one (chunk, row), with the row's M, w_lo and the chunk's
// predicted start S.
__device__ __forceinline__ void wide_chunk_work(WideChunkLds& L, unsigned char* lds_raw, const SampleArgs& a, int row, int chunk,
                                const RowCfg& cfg, float M, float w_lo, double S) {
  const int tid = threadIdx.x;
  const int c0 = chunk * a.chunk;
  const int len = min(a.chunk, a.V - c0);
  float* w = reinterpret_cast<float*>(lds_raw + wide_w_off(a.chunk));
  const float* srow = a.ws_s + (int64_t)row * a.V + c0;
  wide_weights(srow, len, M, cfg.min_p, w);
  for (int h = tid; h < kWideChunkHash; h += NT) { L.hkey[h] = 0u; L.hcnt[h] = 0u; L.hmin[h] = 0xffffffffu; }
  if (tid == 0) { L.nrun = 0u; L.ovf = 0u; }
  __syncthreads();
  // the weights for the finish's exact refolds
  {
    float* wg = a.ws_w + (int64_t)row * a.V + c0;
    for (int i = tid; i < len; i += NT) wg[i] = w[wide_pad(i)];
  }
  // the chunk's part of the vocabulary-order fold: chunk 0 starts from the
  // known -0.0 and folds exactly; the others give their maps in the
  // binades around the predicted start
  ChunkFold* cf = a.wfold + (int64_t)row * a.n_chunks + chunk;
  if (chunk == 0) {
    const float end = exact_chunk_fold(w, len, -0.0f, L.fl.wmap, &L.fend, L.fl.wcnt);
    if (tid == 0) { cf->has_end = 1u; cf->end = end; cf->e0 = 1u; }
  } else {
    const int ep = fold::binade((float)S);
    const int e0 = ep > 1 ? ep - 1 : 1;
    const int J = (len + NT - 1) / NT;
    const int r0 = min(tid * J, len), r1 = min(r0 + J, len);
    fold::Map m0 = fold::map_identity(), m1 = m0, m2 = m0;
    for (int r = r0; r < r1; ++r) {
      const float x = w[wide_pad(r)];
      m0 = fold::compose(m0, term_map(x, e0));
      m1 = fold::compose(m1, term_map(x, e0 + 1));
      m2 = fold::compose(m2, term_map(x, e0 + 2));
    }
    // each thread's block maps, for the finish's crossing search
    fold::Map* bm = a.wbmap + ((int64_t)row * a.n_chunks + chunk) * 3 * NT;
    bm[tid] = m0;
    bm[NT + tid] = m1;
    bm[2 * NT + tid] = m2;
    fold::Map t0, t1, t2;
    block_map_scan(m0, L.fl.wmap, &t0);
    block_map_scan(m1, L.fl.wmap, &t1);
    block_map_scan(m2, L.fl.wmap, &t2);
    if (tid == 0) {
      cf->has_end = 0u;
      cf->e0 = (uint32_t)e0;
      cf->map[0] = t0;
      cf->map[1] = t1;
      cf->map[2] = t2;
    }
  }
  // the superset's distinct weights
  constexpr int kLog2 = 11;
  static_assert((1 << kLog2) == kWideChunkHash, "hash size");
  bool full = false;
  for (int i = tid; i < len; i += NT) {
    const float x = w[wide_pad(i)];
    if (x > 0.f && x >= w_lo)
      full |= !wide_insert(L.hkey, L.hcnt, L.hmin, kLog2, __float_as_uint(x), 1u, (uint32_t)i);
  }
  if (full) L.ovf = 1u;
  __syncthreads();
  uint64_t* out = a.ws_list + (int64_t)row * a.list_stride + (int64_t)chunk * a.chunk;
  for (int h = tid; h < kWideChunkHash; h += NT) {
    const uint32_t k = L.hkey[h];
    if (k != 0u) {
      const uint32_t p = atomicAdd(&L.nrun, 1u);
      out[p] = ((uint64_t)k << 32) | ((uint64_t)L.hcnt[h] << 16) | (uint64_t)L.hmin[h];
    }
  }
  __syncthreads();
  if (tid == 0) cf->nruns = L.ovf ? kFoldNone : L.nrun;
}

// The exact fold value after chunk c's weights, from `acc` before them:
// reads the chunk's weights back (the chain's path when a chunk's sum
// leaves its binades).  All threads call it.
__device__ __forceinline__ float wide_refold(WideFinLds& F, unsigned char* lds_raw, const SampleArgs& a, int row,
                                             int c, float acc) {
  const int c0 = c * a.chunk;
  const int len = min(a.chunk, a.V - c0);
  float* w = reinterpret_cast<float*>(lds_raw + wide_fin_w_off());
  const float* wg = a.ws_w + (int64_t)row * a.V + c0;
  constexpr int kB = 8;
  for (int base = 0; base < len; base += kB * NT) {
    float v[kB];
    #pragma unroll
    for (int k = 0; k < kB; ++k) {
      const int i = base + k * NT + (int)threadIdx.x;
      v[k] = i < len ? wg[i] : 0.f;
    }
    #pragma unroll
    for (int k = 0; k < kB; ++k) {
      const int i = base + k * NT + (int)threadIdx.x;
      if (i < len) w[wide_pad(i)] = v[k];
    }
  }
  __syncthreads();
  return exact_chunk_fold(w, len, acc, F.fl.wmap, &F.acc2, F.fl.wcnt);
}

// The exact fold value after chunk c's weights from the exact value `acc`
// before them, when the chunk's sum leaves the binade it starts in: wave 0
// finds the crossing block from the chunk's stored block maps (a scan of the
// maps over the blocks; block b holds the chunk's terms [b * J, b * J + J),
// J = ceil(len / NT)), adds that block's terms one by one as real f32
// additions, and repeats in the new binade.  Returns kNone's float bits
// (NaN) when a binade falls outside the three stored ones; the caller then
// refolds the chunk.  Wave 0 only; the result is in lane 0 and every lane.
__device__ __forceinline__ float wide_cross_wave(const SampleArgs& a, int row, int c, float acc, bool& ok) {
  constexpr int PB = NT / 64;  // blocks per lane
  const int lane = threadIdx.x & 63;
  const ChunkFold cf = a.wfold[(int64_t)row * a.n_chunks + c];
  const fold::Map* bm = a.wbmap + ((int64_t)row * a.n_chunks + c) * 3 * NT;
  const int c0 = c * a.chunk;
  const int len = min(a.chunk, a.V - c0);
  const int J = (len + NT - 1) / NT;
  const float* wg = a.ws_w + (int64_t)row * a.V + c0;
  float x = acc;
  int bstart = 0;
  ok = true;
  while (bstart < NT) {
    const int ey = fold::binade(x);
    const int k = ey - (int)cf.e0;
    if (k < 0 || k >= 3) { ok = false; return x; }
    // this lane's blocks 4 * lane .. (those before bstart count as identity)
    fold::Map bl[PB];
    fold::Map mine = fold::map_identity();
    #pragma unroll
    for (int q = 0; q < PB; ++q) {
      const int b = PB * lane + q;
      bl[q] = b >= bstart ? bm[k * NT + b] : fold::map_identity();
      mine = fold::compose(mine, bl[q]);
    }
    fold::Map inc = mine;
    #pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      fold::Map o;
      o.t0 = (uint32_t)__shfl_up((int)inc.t0, (unsigned)d, 64);
      o.t1 = (uint32_t)__shfl_up((int)inc.t1, (unsigned)d, 64);
      if (lane >= d) inc = fold::compose(o, inc);
    }
    fold::Map ex;
    ex.t0 = (uint32_t)__shfl_up((int)inc.t0, 1u, 64);
    ex.t1 = (uint32_t)__shfl_up((int)inc.t1, 1u, 64);
    if (lane == 0) ex = fold::map_identity();
    const uint32_t A = fold::to_A(x), p = A & 1u;
    const uint64_t cross = __ballot((uint64_t)A + fold::apply(inc, p) >= fold::kTop);
    if (cross == 0ull) {
      const fold::Map all = {(uint32_t)__builtin_amdgcn_readlane((int)inc.t0, 63),
                             (uint32_t)__builtin_amdgcn_readlane((int)inc.t1, 63)};
      return fold::from_A(A + fold::apply(all, p), ey);
    }
    const int fl = __ffsll((unsigned long long)cross) - 1;
    // in lane fl: the block where the sum leaves the binade, and the value before it
    uint32_t Ab = A + fold::apply(ex, p);  // A before this lane's blocks (< kTop: earlier lanes stayed)
    int blk = PB * lane + PB - 1;
    bool found = false;
    #pragma unroll
    for (int q = 0; q < PB; ++q) {
      const uint32_t t = fold::apply(bl[q], Ab & 1u);
      if (!found && (uint64_t)Ab + t >= fold::kTop) { blk = PB * lane + q; found = true; }
      if (!found) Ab += t;
    }
    blk = __builtin_amdgcn_readlane(blk, fl);
    Ab = (uint32_t)__builtin_amdgcn_readlane((int)Ab, fl);
    // the crossing block's terms as real additions (lane 0; the rest wait)
    float y = fold::from_A(Ab, ey);
    if (lane == 0) {
      const int r0 = min(blk * J, len), r1 = min(r0 + J, len);
      for (int r = r0; r < r1; ++r) y = fold::fadd(y, wg[r]);
    }
    x = __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(y), 0));
    bstart = blk + 1;
  }
  return x;
}

// Calls f(c, e) for every superset run entry e of chunk c of `row`, in
// parallel: chunks in blocks of NT, their run counts scanned into offsets.
template <typename F>
__device__ __forceinline__ void wide_for_each_run(WideFinLds& W, const SampleArgs& a, int row, F f) {
  const int tid = threadIdx.x;
  const int nch = a.n_chunks;
  const ChunkFold* folds = a.wfold + (int64_t)row * nch;
  for (int cb = 0; cb < nch; cb += NT) {
    const int c = cb + tid;
    const uint32_t n = c < nch ? folds[c].nruns : 0u;
    uint32_t tot;
    const uint32_t off = block_excl_scan_u32<NT>(n, W.fl.wcnt, &tot);
    W.noff[tid] = off;
    if (tid == 0) W.noff[NT] = tot;
    __syncthreads();
    for (uint32_t p = (uint32_t)tid; p < tot; p += NT) {
      int lo = 0, hi = NT - 1;  // the last block whose offset is <= p
      while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (W.noff[mid] <= p) lo = mid; else hi = mid - 1;
      }
      const uint64_t* src = a.ws_list + (int64_t)row * a.list_stride + (int64_t)(cb + lo) * a.chunk;
      f(cb + lo, src[p - W.noff[lo]]);
    }
    __syncthreads();
  }
}

// Step 4: the row finish by the last workgroup.  Returns the token, or
// 0xffffffff when the row must take finish_row (nothing written); `path`
// gets the WidePath code.
__device__ __forceinline__ uint32_t wide_finish(unsigned char* lds_raw, const SampleArgs& a, int row, const RowCfg& cfg, float M,
                                float w_lo, uint32_t& path) {
  WideFinLds& F = *reinterpret_cast<WideFinLds*>(lds_raw);
  const int tid = threadIdx.x;
  const int nch = a.n_chunks;
  const ChunkFold* folds = a.wfold + (int64_t)row * nch;

  // a. the normaliser: the chunk plans chained in vocabulary order
  //    (Rust's Sum folds from -0.0)
  float acc = -0.0f;
  bool ovf = false;
  for (int cb = 0; cb < nch; cb += kWideBatch) {
    const int nb = min(kWideBatch, nch - cb);
    {
      const uint32_t* src = reinterpret_cast<const uint32_t*>(folds + cb);
      uint32_t* dst = reinterpret_cast<uint32_t*>(F.u.ch.batch);
      const int words = nb * (int)(sizeof(ChunkFold) / 4);
      for (int i = tid; i < words; i += NT) dst[i] = src[i];
    }
    __syncthreads();
    for (int i = tid; i < nb; i += NT)
      if (F.u.ch.batch[i].nruns == kFoldNone) ovf = true;
    int c = cb;
    while (c < cb + nb) {
      if (tid == 0) {
        float x = acc;
        uint32_t fail = 0xffffffffu;
        for (int cc = c; cc < cb + nb; ++cc) {
          const ChunkFold& cf = F.u.ch.batch[cc - cb];
          if (cf.has_end) { x = cf.end; continue; }  // chunk 0, from -0.0
          const int ey = fold::binade(x);
          const int k = ey - (int)cf.e0;
          bool ok = k >= 0 && k < 3;
          float y = x;
          if (ok) {
            const uint32_t A = fold::to_A(x);
            const uint32_t t = fold::apply(cf.map[k], A & 1u);
            ok = (uint64_t)A + t < fold::kTop;
            y = fold::from_A(A + t, ey);
          }
          if (!ok) { fail = (uint32_t)cc; break; }
          x = y;
        }
        F.acc = x;
        F.fail_c = fail;
      }
      __syncthreads();
      acc = F.acc;
      const uint32_t fail = F.fail_c;
      __syncthreads();
      if (fail == 0xffffffffu) break;
      // the chunk whose sum leaves its binade: the crossing from the block
      // maps (wave 0), else an exact refold of its weights
      if (tid < 64) {
        bool okw = true;
        const float y = wide_cross_wave(a, row, (int)fail, acc, okw);
        if (tid == 0) { F.acc = y; F.fail_c = okw ? 1u : 0u; }
      }
      __syncthreads();
      const bool crossed = F.fail_c != 0u;
      const float ycross = F.acc;
      __syncthreads();
      acc = crossed ? ycross : wide_refold(F, lds_raw, a, row, (int)fail, acc);
      c = (int)fail + 1;
    }
    __syncthreads();
  }
  ovf = __syncthreads_or(ovf);
  const float total = acc;
  path = kWideTotal;
  if (!(total > 0.f) || !finitef_(total)) return 0xffffffffu;  // argmax_host fallback (finish_row)
  path = kWideChunkFull;
  if (ovf) return 0xffffffffu;
  path = kWideMergeFull;

  // c. merge the chunks' runs by weight
  constexpr int kLog2 = 11;
  static_assert((1 << kLog2) == kWideFinHash, "hash size");
  for (int h = tid; h < kWideFinHash; h += NT) {
    F.u.mg.hkey[h] = 0u;
    F.u.mg.hcnt[h] = 0u;
    F.u.mg.hmin[h] = 0xffffffffu;
  }
  if (tid == 0) F.cnt = 0u;
  __syncthreads();
  bool full = false;
  wide_for_each_run(F, a, row, [&](int c, uint64_t e) {
    full |= !wide_insert(F.u.mg.hkey, F.u.mg.hcnt, F.u.mg.hmin, kLog2, (uint32_t)(e >> 32),
                         (uint32_t)(e >> 16) & 0xffffu, (uint32_t)(c * a.chunk) + ((uint32_t)e & 0xffffu));
  });
  if (__syncthreads_or(full)) return 0xffffffffu;
  path = kWideDrawFail;
  // d. distinct weights, descending
  for (int h = tid; h < kWideFinHash; h += NT) {
    const uint32_t k = F.u.mg.hkey[h];
    if (k != 0u) F.u.mg.sortk[atomicAdd(&F.cnt, 1u)] = ((uint64_t)k << 32) | (uint64_t)h;
  }
  __syncthreads();
  const int R = (int)F.cnt;
  if (R == 0) return 0xffffffffu;
  {
    const int n2 = next_pow2(R);
    for (int i = R + tid; i < n2; i += NT) F.u.mg.sortk[i] = 0ull;
    __syncthreads();
    for (int k = 2; k <= n2; k <<= 1) {
      for (int j = k >> 1; j > 0; j >>= 1) {
        for (int i = tid; i < n2; i += NT) {
          const int ixj = i ^ j;
          if (ixj > i) {
            const uint64_t x = F.u.mg.sortk[i], y = F.u.mg.sortk[ixj];
            const bool desc = (i & k) == 0;
            if (desc ? (x < y) : (x > y)) { F.u.mg.sortk[i] = y; F.u.mg.sortk[ixj] = x; }
          }
        }
        __syncthreads();
      }
    }
  }
  {
    // runs in rank order: read everything first, the arrays overlap
    constexpr int kPer = kWideRunCap / NT;
    float rx[kPer];
    uint32_t rm[kPer], ri[kPer];
    #pragma unroll
    for (int q = 0; q < kPer; ++q) {
      const int r = q * NT + tid;
      if (r < R) {
        const uint64_t k = F.u.mg.sortk[r];
        const uint32_t h = (uint32_t)k;
        rx[q] = __uint_as_float((uint32_t)(k >> 32));
        rm[q] = F.u.mg.hcnt[h];
        ri[q] = F.u.mg.hmin[h];
      }
    }
    __syncthreads();
    #pragma unroll
    for (int q = 0; q < kPer; ++q) {
      const int r = q * NT + tid;
      if (r < R) { F.u.fo.rx[r] = rx[q]; F.u.fo.rm[r] = rm[q]; F.u.fo.ri[r] = ri[q]; }
    }
    __syncthreads();
  }

  // e. cum_p += w / total in rank order (from 0.0), up to the cutoff
  auto q_of = [&](int r) { return F.u.fo.rx[r] / total; };
  auto m_of = [&](int r) { return F.u.fo.rm[r]; };
  const float cum_end = fold::fold_runs<NT>(F.fl, F.pe, R, 0.0f, q_of, m_of,
                                            [&](int r, float v) { F.u.fo.st[r] = v; });
  __syncthreads();
  int rstar = R - 1;
  uint32_t cstar = F.u.fo.rm[R - 1];
  if (cfg.cutoff < 1.f) {
    uint32_t first = 0xffffffffu;
    for (int r = tid; r < R; r += NT) {
      const float end = r + 1 < R ? F.u.fo.st[r + 1] : cum_end;
      if (end >= cfg.cutoff) first = min(first, (uint32_t)r);
    }
    first = ~block_max_u32<NT>(~first, F.fl.wcnt);
    if (first == 0xffffffffu) {
      // the cutoff is not reached inside the superset: that is the whole
      // nucleus only when the superset holds every positive weight
      if (w_lo > cfg.min_p) {
        path = kWideNoCutoff;
        return 0xffffffffu;
      }
    } else {
      rstar = (int)first;
      cstar = fold::run_find<false>(F.u.fo.st[rstar], q_of(rstar), F.u.fo.rm[rstar], cfg.cutoff, nullptr);
      if (cstar == fold::kNone) return 0xffffffffu;
    }
  }
  // f. the candidate total: the weights of the ranks before m_end (from -0.0)
  auto m2_of = [&](int r) { return r == rstar ? cstar : F.u.fo.rm[r]; };
  const float ct = fold::fold_runs<NT>(F.fl, F.pe, rstar + 1, -0.0f, [&](int r) { return F.u.fo.rx[r]; }, m2_of,
                                       [&](int r, float v) { F.u.fo.st2[r] = v; });
  __syncthreads();
  if (!(ct > 0.f) || !finitef_(ct)) return 0xffffffffu;
  // g. the inverse CDF: the first rank whose running weight passes target
  const float target = clamp_uniform(cfg.u) * ct;
  uint32_t pr = 0xffffffffu;
  for (int r = tid; r <= rstar; r += NT) {
    const float end = r < rstar ? F.u.fo.st2[r + 1] : ct;
    if (target < end) pr = min(pr, (uint32_t)r);
  }
  pr = ~block_max_u32<NT>(~pr, F.fl.wcnt);
  int rp = rstar;
  uint32_t cp = cstar;  // gpu.rs:899: the last candidate
  if (pr != 0xffffffffu) {
    const uint32_t c = fold::run_find<true>(F.u.fo.st2[pr], F.u.fo.rx[pr], m2_of((int)pr), target, nullptr);
    if (c != fold::kNone) { rp = (int)pr; cp = c; }
  }
  // h. the drawn index: the cp-th smallest index among the weights equal
  //    to the run's (equal weights rank by index)
  const uint32_t first_idx = F.u.fo.ri[rp];
  path = kWideDone;
  if (cp == 1u) return first_idx;
  const uint32_t key = __float_as_uint(F.u.fo.rx[rp]);
  __syncthreads();
  for (int c = tid; c < kWideRunCap; c += NT) F.u.cntc[c] = 0u;
  __syncthreads();
  if (nch > kWideRunCap) {
    path = kWideDrawFail;
    return 0xffffffffu;
  }
  wide_for_each_run(F, a, row, [&](int c, uint64_t e) {
    if ((uint32_t)(e >> 32) == key) F.u.cntc[c] = (uint32_t)(e >> 16) & 0xffffu;
  });
  if (tid == 0) {
    uint32_t seen = 0u;
    F.csel = 0xffffffffu;
    for (int c = 0; c < nch; ++c) {
      const uint32_t k = F.u.cntc[c];
      if (k != 0u && seen + k >= cp) { F.csel = (uint32_t)c; F.rsel = cp - seen; break; }
      seen += k;
    }
    F.tok = 0xffffffffu;
    F.cnt = 0u;
  }
  __syncthreads();
  const uint32_t csel = F.csel, want = F.rsel;
  if (csel == 0xffffffffu) {
    path = kWideDrawFail;
    return 0xffffffffu;
  }
  // the want-th weight equal to key in chunk csel, in index order
  const int c0 = (int)csel * a.chunk;
  const int len = min(a.chunk, a.V - c0);
  const float* srow = a.ws_s + (int64_t)row * a.V + c0;
  const uint32_t wid = (uint32_t)tid >> 6;
  for (int base = 0; base < len; base += NT) {
    const int i = base + tid;
    bool eq = false;
    if (i < len) {
      float x = exact_expf(srow[i] - M);
      x = x < cfg.min_p ? 0.f : x;
      eq = __float_as_uint(x) == key;
    }
    const uint64_t bm = __ballot(eq);
    if ((tid & 63) == 0) F.fl.wcnt[wid] = (uint32_t)__popcll(bm);
    __syncthreads();
    uint32_t before = F.cnt;
    for (uint32_t v = 0; v < wid; ++v) before += F.fl.wcnt[v];
    if (eq && before + lanes_below(bm) + 1u == want) F.tok = (uint32_t)(c0 + i);
    __syncthreads();
    if (tid == 0) {
      uint32_t s = 0u;
      for (int v = 0; v < NT / 64; ++v) s += F.fl.wcnt[v];
      F.cnt += s;
    }
    __syncthreads();
    if (F.tok != 0xffffffffu) break;
  }
  if (F.tok == 0xffffffffu) path = kWideDrawFail;
  return F.tok;
}

// The second kernel of the chunked path: one workgroup per (row, chunk),
// on a 1-D grid whose first B workgroups are chunk 0 of rows 0 .. B-1 and
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
  const WideRow wr = a.wrow[row];
  const bool valid = wr.valid != 0u;
  const float M = wr.M, w_lo = wr.w_lo;
  if (valid) wide_chunk_work(L, lds_raw, a, row, chunk, cfg, M, w_lo, a.wstat[(int64_t)row * a.n_chunks + chunk].pred);
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
    if (pen) l = apply_penalties(l, cnt[e - c0], cfg);
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

// ==========================================================================
// LM-head projection + bias + final softcap fused into the first pass
// ==========================================================================
//
// gpu.rs:20999-21009 output_logits_f32_device: logits = hidden . W^T, plus
// the optional bias, then the final softcap (gpu.rs:23232-23249); the
// sampler then reads the logits back.  Here each workgroup owns a tile of
// kLmTile vocabulary columns for every row: 2 waves, each 64 columns, run
// bf16 MFMAs (16x16x32, f32 accumulation) over the hidden dimension, add the
// bias, apply the softcap (softcap.h), and keep the tile's processed logits
// in LDS.  The fused kernel then records, per (row, tile), what the finish
// needs -- the maximum, both argmaxes and the largest candidate key -- and
// leaves the tile's logits in the workspace only for top-k rows, whose
// finish reads back the few tiles that can hold the row's top k (greedy
// rows write no logits at all).  The twin kernel runs the same code and
// writes every logit instead: the fused path's logits are bit-identical to
// the twin's by construction (same tiles, same MFMA order, same epilogue).
//
// MFMA 16x16x32 bf16 operand layout (lane l = 16 * g + r): A row r, K
// elements 8g .. 8g + 7; B column r, the same K elements; D rows 4g .. 4g + 3
// of column r.
typedef __bf16 lm_bf16x8 __attribute__((ext_vector_type(8)));
typedef float lm_f32x4 __attribute__((ext_vector_type(4)));

struct LmTileRec {
  uint32_t max_lk;       // largest processed-logit key (lkey) of the tile
  uint32_t am_ieee_i;    // IEEE '>' argmax (0xffffffff: no value above -inf)
  float am_ieee_v;
  uint32_t tot_key;      // largest total_cmp key (biased to unsigned)
  uint32_t tot_i;        // its lowest index
  uint32_t pad;
  uint64_t top;          // largest candidate key of the tile
};
static_assert(sizeof(LmTileRec) == 32, "LmTileRec layout");

// Loads of one K block for a lane: 16 bytes at element `off` of each operand
// row (rows past the batch or the vocabulary read row 0 and are dropped in
// the epilogue, so every load is unconditional).
__device__ __forceinline__ lm_bf16x8 lm_ld(const __bf16* p) { return *reinterpret_cast<const lm_bf16x8*>(p); }

// The logits of vocabulary columns [tile0, tile0 + kLmTile) for rows
// [0, B), B <= 32 RG, processed (bias, softcap), into tile[m * kLmTile +
// column].  Wave w owns 64 columns as four 16-column MFMA tiles, times two
// 16-row tiles for each of the RG groups of 32 rows (every weight block
// loaded is used by all rows).
// K runs in blocks of 64: lane (g, r) loads 32 contiguous bytes of its
// weight row at element 16g and gives the first half to one MFMA and the
// second to the next, so each row's 128-byte line is used whole by one load
// pair (both operands share that K order, which is all the product needs).
// Two register slots hold weight blocks: a slot multiplies, then refills
// with the block two ahead.  The hidden rows' block (32 rows x 64 elements,
// 4 KB) is loaded once per workgroup -- 32 bytes a thread, three blocks
// ahead -- and staged through a two-slot LDS ring that both waves read, so
// the hidden state is fetched once per tile instead of once per wave (the
// product then runs about 5% faster).  With the kernels held to 3 waves per
// SIMD, every workgroup of a 151936-column head is resident at once.  The
// workgroup starts at K block (tile mod the block count) and wraps around,
// so the reads in flight spread over the rows' whole length instead of all
// sitting at one offset (about 10% more HBM throughput than a common
// start).  A trailing 32-element block (H % 64 == 32) takes the plain
// layout, element 8g, last.  The order is fixed per tile, so every kernel
// built on this function produces the same bits (and a row's logits do not
// depend on RG or on the other rows).
template <int RG>
__device__ __forceinline__ void lm_gemm_tile(const LmArgs& a, int tile0, float* tile) {
  static_assert(kLmThreads == 128, "hidden block staging: 128 threads x 32 bytes per row group");
  __shared__ __align__(16) __bf16 a_lds[2][RG * 32 * 64];
  const int tid = threadIdx.x;
  const int lane = tid & 63, wid = tid >> 6;
  const int r = lane & 15, g = lane >> 4;
  const int H = a.H, nb = a.H >> 6;
  const int v0 = tile0 + wid * 64;
  lm_f32x4 acc[RG][2][4];
  #pragma unroll
  for (int q = 0; q < RG; ++q)
    #pragma unroll
    for (int mt = 0; mt < 2; ++mt)
      #pragma unroll
      for (int nt = 0; nt < 4; ++nt) acc[q][mt][nt] = lm_f32x4{0.f, 0.f, 0.f, 0.f};
  const __bf16* wrow[4];
  #pragma unroll
  for (int nt = 0; nt < 4; ++nt) {
    const int v = v0 + nt * 16 + r;
    wrow[nt] = a.weight + (int64_t)(v < a.V ? v : 0) * H;
  }
  // this thread's share of a hidden block: rows 32 q + tid / 4, elements
  // 16 (tid % 4) .. + 15 of the block, which is MFMA lane (tid % 4, row % 16)'s
  // operand
  const __bf16* arow[RG];
  #pragma unroll
  for (int q = 0; q < RG; ++q) {
    const int am = 32 * q + (tid >> 2);
    arow[q] = a.hidden + (int64_t)(am < a.B ? am : 0) * H + 16 * (tid & 3);
  }
  const int rot = nb > 0 ? (int)((uint32_t)(tile0 / kLmTile) % (uint32_t)nb) : 0;
  auto blk = [&](int i) { const int b = i + rot; return (b >= nb ? b - nb : b) * 64; };
  lm_bf16x8 bb[2][4][2], ar[3][RG][2];
  auto load_w = [&](lm_bf16x8 (&br)[4][2], int i) {
    const int off = blk(i) + 16 * g;
    #pragma unroll
    for (int nt = 0; nt < 4; ++nt) { br[nt][0] = lm_ld(wrow[nt] + off); br[nt][1] = lm_ld(wrow[nt] + off + 8); }
  };
  auto load_h = [&](lm_bf16x8 (&x)[RG][2], int i) {
    const int off = blk(i);
    #pragma unroll
    for (int q = 0; q < RG; ++q) {
      x[q][0] = lm_ld(arow[q] + off);
      x[q][1] = lm_ld(arow[q] + off + 8);
    }
  };
  auto stage_h = [&](const lm_bf16x8 (&x)[RG][2], int slot) {
    #pragma unroll
    for (int q = 0; q < RG; ++q) {
      lm_bf16x8* d = reinterpret_cast<lm_bf16x8*>(&a_lds[slot][(q * kLmThreads + tid) * 16]);
      d[0] = x[q][0];
      d[1] = x[q][1];
    }
  };
  if (nb > 0) { load_w(bb[0], 0); load_h(ar[0], 0); }
  if (nb > 1) { load_w(bb[1], 1); load_h(ar[1], 1); }
  if (nb > 2) load_h(ar[2], 2);
  if (nb > 0) stage_h(ar[0], 0);
  // block j: weights in register slot j % 2, hidden in LDS slot j % 2 and
  // register slot j % 3; six blocks per trip keep every index static
  #pragma unroll 1
  for (int j0 = 0; j0 < nb; j0 += 6) {
    #pragma unroll
    for (int u = 0; u < 6; ++u) {
      const int j = j0 + u;
      if (j < nb) {
        __syncthreads();  // LDS slot j % 2 written, slot (j + 1) % 2 read by both waves
        if (j + 1 < nb) stage_h(ar[(u + 1) % 3], (u + 1) % 2);
        #pragma unroll
        for (int q = 0; q < RG; ++q) {
          lm_bf16x8 af[2][2];
          #pragma unroll
          for (int mt = 0; mt < 2; ++mt) {
            const lm_bf16x8* src =
                reinterpret_cast<const lm_bf16x8*>(&a_lds[u % 2][(q * kLmThreads + (mt * 16 + r) * 4 + g) * 16]);
            af[mt][0] = src[0];
            af[mt][1] = src[1];
          }
          #pragma unroll
          for (int h = 0; h < 2; ++h)
            #pragma unroll
            for (int mt = 0; mt < 2; ++mt)
              #pragma unroll
              for (int nt = 0; nt < 4; ++nt)
                acc[q][mt][nt] =
                    __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[mt][h], bb[u % 2][nt][h], acc[q][mt][nt], 0, 0, 0);
        }
        if (j + 2 < nb) load_w(bb[u % 2], j + 2);
        if (j + 3 < nb) load_h(ar[u % 3], j + 3);
      }
    }
  }
  if ((nb << 6) < H) {
    const int off = (nb << 6) + 8 * g;
    lm_bf16x8 bt[4];
    #pragma unroll
    for (int nt = 0; nt < 4; ++nt) bt[nt] = lm_ld(wrow[nt] + off);
    #pragma unroll
    for (int q = 0; q < RG; ++q) {
      lm_bf16x8 at[2];
      #pragma unroll
      for (int mt = 0; mt < 2; ++mt) {
        const int m = 32 * q + mt * 16 + r;
        at[mt] = lm_ld(a.hidden + (int64_t)(m < a.B ? m : 0) * H + off);
      }
      #pragma unroll
      for (int mt = 0; mt < 2; ++mt)
        #pragma unroll
        for (int nt = 0; nt < 4; ++nt)
          acc[q][mt][nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(at[mt], bt[nt], acc[q][mt][nt], 0, 0, 0);
    }
  }
  // epilogue: bias, softcap; tile[m * kLmTile + column]
  #pragma unroll
  for (int q = 0; q < RG; ++q)
    #pragma unroll
    for (int mt = 0; mt < 2; ++mt)
      #pragma unroll
      for (int nt = 0; nt < 4; ++nt)
        #pragma unroll
        for (int jj = 0; jj < 4; ++jj) {
          const int m = 32 * q + mt * 16 + 4 * g + jj;
          const int v = v0 + nt * 16 + r;
          if (m >= a.B || v >= a.V) continue;
          float x = acc[q][mt][nt][jj];
          if (a.bias) x = x + a.bias[v];
          if (a.cap > 0.f) x = softcap_f32(x, a.cap);
          tile[m * kLmTile + (v - tile0)] = x;
        }
}

// Registers: one row group fits 3 waves per SIMD (every workgroup of a
// 151936-column head resident at once), two row groups 2.
template <int RG>
constexpr int lm_waves_per_eu() { return RG == 1 ? 3 : 2; }

// The twin: the same tiles, written to logits [B][V].
template <int RG>
__global__ void __launch_bounds__(kLmThreads) __attribute__((amdgpu_waves_per_eu(lm_waves_per_eu<RG>(), 8)))
    lm_logits_kernel(LmArgs a) {
  extern __shared__ __align__(16) unsigned char lds_raw[];
  float* tile = reinterpret_cast<float*>(lds_raw);
  const int tile0 = blockIdx.x * kLmTile;
  lm_gemm_tile<RG>(a, tile0, tile);
  __syncthreads();
  const int len = min(kLmTile, a.V - tile0);
  for (int i = threadIdx.x; i < a.B * kLmTile; i += kLmThreads) {
    const int m = i / kLmTile, c = i % kLmTile;
    if (c < len) a.out_logits[(int64_t)m * a.V + tile0 + c] = tile[i];
  }
}

// Whether the fused finish takes a row: greedy, or top-k up to kLmMaxK
// (with temperature, top-p, min-p), no penalties (the fused entry point
// takes no history).
__device__ __forceinline__ bool lm_row_ok(const RowCfg& c) {
  return c.cls == kGreedy || (c.cls == kTopK && c.k_eff <= kLmMaxK);
}

// IEEE '>' argmax key of a value above -inf: -0 counts as +0 (the two are
// equal under '>', so the lowest index among them wins).
__device__ __forceinline__ uint64_t ieee_key(float l, uint32_t e) { return cand_key(okey(l == 0.f ? 0.f : l), e); }

// The fused pass: per (row, tile) records.  Wave w takes the rows w,
// w + kLmThreads / 64, ... of the tile.  A top-k row also leaves the tile's
// logits in the workspace, where the finish reads the few tiles that can
// hold the row's top k (greedy rows leave nothing but the records).
template <int RG>
__global__ void __launch_bounds__(kLmThreads) __attribute__((amdgpu_waves_per_eu(lm_waves_per_eu<RG>(), 8)))
    lm_select_kernel(LmArgs a) {
  extern __shared__ __align__(16) unsigned char lds_raw[];
  float* tile = reinterpret_cast<float*>(lds_raw);
  const int t = blockIdx.x, tile0 = t * kLmTile;
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  // lane m holds row m's k (0: greedy or not taken), loaded before the
  // product so that its latency hides there
  uint32_t my_k = 0u;
  if (lane < a.B) {
    const RowCfg cfg = load_cfg(a.pv, lane, a.V, 0, 0);
    my_k = (cfg.cls == kTopK && cfg.k_eff <= kLmMaxK) ? (uint32_t)cfg.k_eff : 0u;
  }
  lm_gemm_tile<RG>(a, tile0, tile);
  __syncthreads();
  const int len = min(kLmTile, a.V - tile0);
  constexpr int PER = kLmTile / 64;
  for (int m = wid; m < a.B; m += kLmThreads / 64) {
    const uint32_t k = (uint32_t)__builtin_amdgcn_readlane((int)my_k, m);
    const float* row = tile + m * kLmTile;
    // the largest candidate key; values that are not finite or are -0 take
    // the exact record path below
    uint64_t top = 0ull;
    bool special = false;
    #pragma unroll
    for (int q = 0; q < PER; ++q) {
      const int i = q * 64 + lane;
      if (i < len) {
        const float l = row[i];
        const uint64_t x = cand_key(lkey(l), (uint32_t)(tile0 + i));
        top = x > top ? x : top;
        special |= !finitef_(l) || __float_as_uint(l) == 0x80000000u;
      }
    }
    top = wave_max_u64(top);
    LmTileRec rec;
    if (!__any(special)) {
      // every value finite and no -0: lkey, the IEEE key and total_cmp order
      // the tile alike, so the maximum key gives all three argmaxes
      const uint32_t i0 = cand_idx(top);
      const float l0 = okey_inv(cand_skey(top));
      rec.max_lk = cand_skey(top);
      rec.am_ieee_i = i0;
      rec.am_ieee_v = l0;
      rec.tot_key = (uint32_t)total_key(l0) ^ 0x80000000u;
      rec.tot_i = i0;
    } else {
      uint32_t mk = 0u, tk = 0u, ti = 0xffffffffu;
      uint64_t am = 0ull;
      for (int i = lane; i < len; i += 64) {
        const float l = row[i];
        const uint32_t e = (uint32_t)(tile0 + i);
        mk = max(mk, lkey(l));
        if (l > -__builtin_inff()) {  // IEEE '>' from -inf: NaN and -inf never win
          const uint64_t kk = ieee_key(l, e);
          am = kk > am ? kk : am;
        }
        const uint32_t tot = (uint32_t)total_key(l) ^ 0x80000000u;
        if (tot > tk || (tot == tk && e < ti)) { tk = tot; ti = e; }
      }
      mk = wave_max_u32(mk);
      am = wave_max_u64(am);
      const uint64_t tot64 = ((uint64_t)tk << 32) | (uint64_t)(0xffffffffu - ti);
      const uint64_t best = wave_max_u64(lane < len ? tot64 : 0ull);
      rec.max_lk = mk;
      rec.am_ieee_i = am ? cand_idx(am) : 0xffffffffu;
      rec.am_ieee_v = am ? okey_inv(cand_skey(am)) : -__builtin_inff();
      rec.tot_key = (uint32_t)(best >> 32);
      rec.tot_i = 0xffffffffu - (uint32_t)best;
    }
    rec.pad = 0u;
    rec.top = top;
    if (lane == 0) a.lm_recs[(int64_t)m * a.n_chunks + t] = rec;
  }
  // the tile logits of top-k rows, row after row as the twin writes them
  // (a wave covers half a row, so the row's k is uniform over the wave)
  for (int i = threadIdx.x; i < a.B * kLmTile; i += kLmThreads) {
    const int m = i / kLmTile, c = i % kLmTile;
    const uint32_t k = (uint32_t)__builtin_amdgcn_readlane((int)my_k, m);
    if (k > 0u && c < len) a.lm_logits[(int64_t)m * a.V + tile0 + c] = tile[i];
  }
}

// The fused finish: one workgroup per row (gpu.rs:753-900 on the row's
// candidates, as the lean finish does).  out_tokens[row] = 0xffffffff for a
// row the fused path does not take (its class), 0xfffffffe for a tie it
// cannot resolve without the logits: the caller samples such a row from the
// twin's logits.
__global__ void __launch_bounds__(NT) lm_finish_kernel(LmArgs a) {
  extern __shared__ __align__(16) unsigned char lds_raw[];
  FinLds& fs = *reinterpret_cast<FinLds*>(lds_raw);
  const int row = blockIdx.x, tid = threadIdx.x;
  const RowCfg cfg = load_cfg(a.pv, row, a.V, 0, 0);
  if (!lm_row_ok(cfg)) {
    if (tid == 0) a.out_tokens[row] = 0xffffffffu;
    return;
  }
  // merge the tile records
  uint32_t mk = 0u, tk = 0u, ti = 0xffffffffu, ai = 0xffffffffu;
  float av = -__builtin_inff();
  for (int c = tid; c < a.n_chunks; c += NT) {
    const LmTileRec r = a.lm_recs[(int64_t)row * a.n_chunks + c];
    fs.cbig[c] = r.top;
    mk = max(mk, r.max_lk);
    if (r.tot_key > tk || (r.tot_key == tk && r.tot_i < ti)) { tk = r.tot_key; ti = r.tot_i; }
    if (r.am_ieee_i != 0xffffffffu && (ai == 0xffffffffu || r.am_ieee_v > av || (r.am_ieee_v == av && r.am_ieee_i < ai))) {
      av = r.am_ieee_v; ai = r.am_ieee_i;
    }
  }
  {
    // the three maxima in one exchange: the logit key, total_cmp's argmax
    // and the IEEE argmax ((value key, -index) over the tiles that have one)
    uint64_t m3[3] = {(uint64_t)mk, ((uint64_t)tk << 32) | (uint64_t)(0xffffffffu - ti),
                      ai == 0xffffffffu ? 0ull : ieee_key(av, ai)};
    #pragma unroll
    for (int q = 0; q < 3; ++q) m3[q] = wave_max_u64(m3[q]);
    const int lane = tid & 63, wid = tid >> 6;
    if (lane == 0) { fs.red64[wid] = m3[0]; fs.red64b[wid] = m3[1]; fs.mass[wid] = m3[2]; }
    __syncthreads();
    #pragma unroll
    for (int w = 0; w < NT / 64; ++w) {
      m3[0] = fs.red64[w] > m3[0] ? fs.red64[w] : m3[0];
      m3[1] = fs.red64b[w] > m3[1] ? fs.red64b[w] : m3[1];
      m3[2] = fs.mass[w] > m3[2] ? fs.mass[w] : m3[2];
    }
    __syncthreads();
    mk = (uint32_t)m3[0];
    tk = (uint32_t)(m3[1] >> 32);
    ti = 0xffffffffu - (uint32_t)m3[1];
    ai = m3[2] ? cand_idx(m3[2]) : 0xffffffffu;
  }
  const uint32_t host_argmax = ti;  // argmax_host (gpu.rs:739-751)
  if (cfg.cls == kGreedy) {
    if (tid == 0) a.out_tokens[row] = ai == 0xffffffffu ? 0u : ai;
    return;
  }
  const float M = mk > kKeyNegInf ? okey_inv(mk) / cfg.t_eff : -__builtin_inff();
  if (!finitef_(M)) {
    if (tid == 0) a.out_tokens[row] = host_argmax;
    return;
  }
  // A threshold L with between k and kLmMaxK tile tops at or above it
  // bounds the row's k-th key from below (those tops are k distinct keys),
  // and only the tiles whose top is >= L -- at most kLmMaxK of them, or
  // every tile when there are fewer than k -- can hold the row's top k.
  // Their keys >= L are gathered into LDS; when more than kGather are, the
  // select runs over the listed tiles in global memory instead.
  static_assert(kLmMaxTiles <= kGather, "tile tops fit the gather buffer");
  const int k = cfg.k_eff;
  const int nt = a.n_chunks;
  const uint64_t L = nt > kLmMaxK ? block_select_skip_f([&](int i) { return fs.cbig[i]; }, nt, (uint32_t)k, fs.hist,
                                                        fs.sel, fs.red64, fs.red64b, ~0ull, 0ull, (uint32_t)kLmMaxK)
                                  : 0ull;
  if (tid == 0) fs.counter = 0u;
  __syncthreads();
  uint64_t out_max = 0ull;  // the largest key of the tiles not scanned
  uint32_t* list = fs.aux;  // tiles to scan (at most kLmMaxK)
  for (int c = tid; c < nt; c += NT) {
    const uint64_t t = fs.cbig[c];
    if (t >= L) list[atomicAdd(&fs.counter, 1u)] = (uint32_t)c;
    else out_max = t > out_max ? t : out_max;
  }
  __syncthreads();
  const int n_list = (int)fs.counter;
  __syncthreads();
  if (tid == 0) fs.counter = 0u;
  __syncthreads();
  const float* lg = a.lm_logits + (int64_t)row * a.V;
  const int n_items = n_list * kLmTile;
  // item i: column i % kLmTile of listed tile i / kLmTile (0 past the
  // vocabulary: below every key)
  auto item = [&](int i) -> uint64_t {
    const uint32_t v = list[i / kLmTile] * kLmTile + (uint32_t)(i % kLmTile);
    return v < (uint32_t)a.V ? cand_key(lkey(lg[v]), v) : 0ull;
  };
  constexpr int kScanPer = kLmMaxK * kLmTile / NT;
  static_assert(kScanPer * NT == kLmMaxK * kLmTile, "scan split");
  uint64_t below = 0ull;
  bool over = false;
  {
    float xs[kScanPer];
    #pragma unroll
    for (int q = 0; q < kScanPer; ++q) {
      const int i = tid + q * NT;
      const int li = i / kLmTile;
      const uint32_t v = list[li < n_list ? li : 0] * kLmTile + (uint32_t)(i % kLmTile);
      xs[q] = lg[v < (uint32_t)a.V ? v : 0u];  // unconditional: the address is valid
    }
    #pragma unroll
    for (int q = 0; q < kScanPer; ++q) {
      const int i = tid + q * NT;
      const int li = i / kLmTile;
      const uint32_t v = list[li < n_list ? li : 0] * kLmTile + (uint32_t)(i % kLmTile);
      if (li < n_list && v < (uint32_t)a.V) {
        const uint64_t x = cand_key(lkey(xs[q]), v);
        if (x >= L) {
          const uint32_t o = atomicAdd(&fs.counter, 1u);
          if (o < (uint32_t)kGather) fs.cbig[o] = x;
          else over = true;
        } else {
          below = x > below ? x : below;
        }
      }
    }
  }
  over = __syncthreads_or(over);
  const int n = over ? n_items : (int)fs.counter;
  uint64_t thr = 0ull;
  if (over) thr = block_select_skip_f(item, n_items, (uint32_t)k, fs.hist, fs.sel, fs.red64, fs.red64b);
  else if (n > k) thr = block_select_skip(fs.cbig, n, (uint32_t)k, fs.hist, fs.sel, fs.red64, fs.red64b);
  // the selection (order does not matter: it is ranked below) and the
  // largest candidate left out
  if (tid == 0) fs.counter = 0u;
  __syncthreads();
  for (int j = tid; j < n; j += NT) {
    const uint64_t x = over ? item(j) : fs.cbig[j];
    if (x >= thr) fs.buf[atomicAdd(&fs.counter, 1u)] = x;
    else below = x > below ? x : below;
  }
  below = below > out_max ? below : out_max;
  below = block_max_u64<NT>(below, fs.red64);
  __syncthreads();
  // weights; the smallest selected weight w_b and key S.  The selection
  // ranks by (key desc, index asc), the reference by (weight desc, index
  // asc): they agree unless keys with weight w_b sit on both sides of the
  // cut with different keys.  When the largest key left out (in a tile or
  // among the candidates) has weight w_b, the row is resolved only if that
  // key is S, no selected key of weight w_b differs from S, and the key
  // just below S weighs less than w_b (so no key left out below S can
  // weigh w_b); else the tie is unresolved.
  if (tid == 0) { fs.wmin = 0xffffffffu; fs.token = 0xffffffffu; }
  __syncthreads();
  for (int j = tid; j < k; j += NT) {
    const uint64_t x = fs.buf[j];
    const float w = exact_expf(key_to_s(cand_skey(x), cfg.t_eff) - M);
    fs.pay[j] = cand_skey(x);
    fs.buf[j] = rank_key(w, cand_idx(x));
    atomicMin(&fs.wmin, __float_as_uint(w));
    atomicMin(&fs.token, cand_skey(x));
  }
  __syncthreads();
  const float w_b = __uint_as_float(fs.wmin);
  const uint32_t S = fs.token;
  const uint32_t xk = below ? cand_skey(below) : 0u;
  if (w_b > 0.f && xk > kKeyNegInf && exact_expf(key_to_s(xk, cfg.t_eff) - M) == w_b) {
    if (tid == 0) fs.flag = 0u;
    __syncthreads();
    for (int j = tid; j < k; j += NT)
      if (fs.pay[j] != S && exact_expf(key_to_s(fs.pay[j], cfg.t_eff) - M) == w_b) fs.flag = 1u;
    __syncthreads();
    const bool lone = xk == S && fs.flag == 0u && !(exact_expf(key_to_s(S - 1u, cfg.t_eff) - M) == w_b);
    if (!lone) {
      if (tid == 0) a.out_tokens[row] = 0xfffffffeu;
      return;
    }
  }
  sort_ranked(fs, k);
  const int pick = wave_draw<kLmMaxK / 64>(fs.buf, k, cfg);
  if (tid == 0) a.out_tokens[row] = pick < 0 ? host_argmax : cand_idx(fs.buf[pick]);
}

size_t lm_recs_bytes(int B, int n_tiles) { return ((size_t)B * n_tiles * sizeof(LmTileRec) + 255) & ~(size_t)255; }
size_t lm_workspace_bytes(int B, int V) {
  const int tiles = (V + kLmTile - 1) / kLmTile;
  return lm_recs_bytes(B, tiles) + (size_t)B * V * sizeof(float);
}

size_t lm_tile_lds(int B) { return (size_t)(B <= 32 ? 32 : kLmRows) * kLmTile * sizeof(float); }
size_t lm_finish_lds() { return (sizeof(FinLds) + 15) & ~(size_t)15; }

// --------------------------------------------------------------------------
// launch wrappers (called from the host API)

// Chunks of the streaming select pass: 64 logits per thread when the batch
// alone gives at least 4 workgroups per CU, 16 otherwise.
constexpr int kSelChunkLarge = NT * 64;
constexpr int kSelChunkSmall = NT * 16;

// ==========================================================================
// Row kernel: one workgroup streams a whole row and finishes it in place
// ==========================================================================
//
// For large batches (kRowMinBatch rows or more, f32 logits, no logprobs) one
// workgroup of kRowThreads per row replaces the select pass and the finish
// kernel.  Sixteen waves share a CU (four per SIMD), so one wave's LDS
// round trips and branches overlap the others' work and loads.
//  - The row streams through a register pipeline kRowDepth tiles deep per
//    wave (tile = kRowTile logits, 16-byte loads).  Per logit the common
//    case is one max over its raw bits.
//  - Each wave keeps the top kw of its own logits (by candidate key) in an
//    LDS list, kw = ceil(k/16) + ceil(sqrt(k)) + 4: a logit whose key passes
//    the wave's threshold is appended, and when the list passes kRowHW
//    entries the wave keeps its kw largest and raises the threshold to the
//    last one's key.  A later logit with that key has a larger index and
//    ranks below all kept ones, so the test is strict.  The first tile
//    starts from a bound of the wave's group maxima instead of -inf.
//  - The first tiles are issued before the row's parameters are read.
//  - History tokens stream like the others (their raw logits).  The history
//    is ranked in LDS after the first tile (a word of marks per 32 logits
//    and the number of marked logits before it), and its logits are loaded
//    while the stream runs.  Each thread applies the penalties to its own
//    history entries as soon as its part of the stream ends (the waves
//    finish up to ~2.5 us apart, in age order per SIMD, so most of that work
//    hides behind the youngest waves' last tiles) and stores the processed
//    keys by rank; list entries that are history tokens are dropped.
//  - Every logit left out has a key at or below the largest wave threshold
//    Tm, so the union of the lists and the processed history logits above
//    Tm holds the row's top k whenever its k-th key is above Tm (finish_core
//    checks that).  A wave holding more than kw of the row's top k breaks it
//    and sends the row to the general path; with kw at mean + 4 sd of that
//    count it does not happen for rows whose top tokens are spread over the
//    vocabulary.
// Once every wave has written its list, the others end and the first four
// waves (one per SIMD) gather the candidates and run finish_core.  Rows the
// fast path does not cover (other row classes, more than kRowHistCap
// distinct history tokens, a list overflow, no finite logit, +inf logits, a
// tie finish_core will not resolve) run the chunk select and the finish of
// the two-kernel path inside the same workgroup, on its first four waves.

constexpr int kRowThreads = 1024;
constexpr int kRowWaves = kRowThreads / 64;
constexpr int kRowTV = 4;                             // 16-byte loads per thread per tile
constexpr int kRowEl = kRowTV * 4;                    // logits per thread per tile
constexpr int kRowTile = kRowThreads * kRowEl;        // 16384 logits
constexpr int kRowDepth = 2;                          // tiles in flight per wave
constexpr int kRowHW = 64;                            // list length that triggers a selection
constexpr int kRowCap = 128;                          // list capacity (past it: general path)
constexpr int kRowHistCap = 2048;                     // distinct history tokens per row
constexpr int kRowHistPer = kRowHistCap / kRowThreads;  // history entries per thread in registers
constexpr int kRowMaxV = 1 << 18;
constexpr int kRowMinBatch = 192;
constexpr int kRowKwMax = kLeanK / 16 + 16 + 4;       // kw at k = kLeanK (sqrt(256) = 16)
static_assert(kRowKwMax < kRowHW, "a full list holds more than kw entries");

struct RowLds {
  uint64_t wbuf[kRowWaves][kRowCap];   // per-wave candidate lists
  uint32_t ob_raw[kRowHistCap];        // key of the processed logit (mask, penalties) of the
                                       // history token of rank r
  uint32_t ob_cnt[kRowHistCap];        // its summed count
  uint32_t ob_id[kRowHistCap];         // its id
  float xscr[kRowWaves][64 * kRowEl];  // a wave's tile when a branch needs single logits; also
                                       // the wave's selection histogram
  // the fields below stay valid while the finish reuses the space above
  uint32_t wthr[kRowWaves];
  uint32_t wbad[kRowWaves];
  uint32_t wcnt[kRowWaves];
  uint32_t redu[kRowWaves];
  uint64_t red64[kRowWaves];
};
constexpr size_t kRowHead = (sizeof(RowLds) + 15) & ~(size_t)15;
static_assert(sizeof(FinLds) <= offsetof(RowLds, wthr), "finish LDS must fit the stream's lists");
static_assert(offsetof(RowLds, ob_raw) % 16 == 0 && offsetof(RowLds, ob_cnt) % 16 == 0 &&
                  offsetof(RowLds, ob_id) % 16 == 0,
              "the history arrays are read 16 bytes at a time");

// Keeps the `need` largest entries of the wave's list (unique keys,
// need <= n) at its front; returns the key of the last one kept.
__device__ __forceinline__ uint32_t row_wave_keep(uint64_t* wl, uint32_t& n, uint32_t need, uint32_t* hist) {
  const uint32_t lane = threadIdx.x & 63u;
  wave_lds_sync();
  Segs<1> sg;
  sg.p[0] = wl;
  sg.n[0] = n;
  sg.ns = 1;
  const uint64_t thr = wave_select_skip<1>(sg, need, hist);
  uint32_t nn = 0u;
  for (uint32_t b = 0; b < n; b += 64u) {
    const uint32_t i = b + lane;
    const uint64_t x = i < n ? wl[i] : 0ull;
    const bool keep = i < n && x >= thr;
    const uint64_t m = __ballot(keep);
    wave_lds_sync();  // the block is read before any lane writes
    if (keep) wl[nn + lanes_below(m)] = x;
    nn += (uint32_t)__popcll(m);
  }
  wave_lds_sync();
  n = nn;
  return cand_skey(thr);
}

// A wave's tile in LDS (float4 j of lane l at j * 256 + 4 l): branches that
// need single logits read them back by element (per-lane indices into a
// register array would move the tile to scratch memory).
__device__ __forceinline__ void row_spill(float* xs, const float (&x)[kRowEl]) {
  const uint32_t lane = threadIdx.x & 63u;
  #pragma unroll
  for (int j = 0; j < kRowTV; ++j)
    *reinterpret_cast<float4*>(xs + j * 256 + 4 * lane) = make_float4(x[4 * j], x[4 * j + 1], x[4 * j + 2], x[4 * j + 3]);
  wave_lds_sync();
}
__device__ __forceinline__ float row_elem(const float* xs, uint32_t e) {
  return xs[(e >> 2) * 256u + 4u * (threadIdx.x & 63u) + (e & 3u)];
}

// Cache policy of the stream's loads: non-temporal (the nt bit of gfx950's
// buffer loads), so that the logits, each read once, do not push the code
// and the small per-row data out of the L2 cache.
constexpr int kStreamLoad = 2;

constexpr uint32_t kKeyNegZero = 0x7fffffffu;  // okey(-0.0f)
constexpr uint32_t kKeyPosInf = 0xff800000u;   // okey(+inf)

// The row's loads in flight: kRowDepth slots of kRowTV 16-byte loads per
// thread (and their mask words) with the buffer resources they use, and the
// row's history entries.
template <bool MASK>
struct RowPipe {
  __amdgpu_buffer_rsrc_t rs, ms;
  i32x4_t buf[kRowDepth][kRowTV];
  uint32_t mw[kRowDepth][kRowTV];
  uint32_t h0, h1;                   // the row's history entries [h0, h1)
  uint32_t hid[kRowHistPer], hcs[kRowHistPer];
};

// Issues the row's first kRowDepth tiles (range-checked: loads past the row
// read zero), then its history entries.  They need only the kernel
// arguments, so they go out before the row's parameters arrive.
template <bool MASK>
__device__ __forceinline__ void row_issue(const SampleArgs& a, int row, RowPipe<MASK>& pp) {
  const int tid = threadIdx.x;
  const int V = a.V;
  const float* lrow = reinterpret_cast<const float*>((const char*)a.logits + (int64_t)row * a.row_stride * 4);
  pp.rs = __builtin_amdgcn_make_buffer_rsrc((void*)lrow, (short)0, V * 4, kBufferConfig);
  if (MASK) {
    const uint32_t* mrow = a.mask + (int64_t)row * a.mask_words;
    pp.ms = __builtin_amdgcn_make_buffer_rsrc((void*)mrow, (short)0, ((V + 31) >> 5) * 4, kBufferConfig);
  }
  #pragma unroll
  for (int d = 0; d < kRowDepth; ++d) {
    #pragma unroll
    for (int j = 0; j < kRowTV; ++j) {
      const int e0 = d * kRowTile + (j * kRowThreads + tid) * 4;
      pp.buf[d][j] = __builtin_amdgcn_raw_buffer_load_b128(pp.rs, e0 * 4, 0, kStreamLoad);
      if (MASK) pp.mw[d][j] = (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(pp.ms, (e0 >> 5) * 4, 0, 0);
    }
  }
  // unconditional range-checked loads (entries past the row read zero): a
  // load under a condition would leave the compiler unsure how many loads
  // are in flight in the stream loop, and it would then wait for all
  pp.h0 = a.hoff ? const_load(a.hoff + row) : 0u;
  pp.h1 = a.hoff ? const_load(a.hoff + row + 1) : 0u;
  // (a scalar: a range in a vector register would make each load a loop)
  const int nh = __builtin_amdgcn_readfirstlane(pp.h1 > pp.h0 ? (int)(pp.h1 - pp.h0) : 0);
  const __amdgpu_buffer_rsrc_t ri =
      __builtin_amdgcn_make_buffer_rsrc((void*)(a.hids + pp.h0), (short)0, nh * 4, kBufferConfig);
  const __amdgpu_buffer_rsrc_t rc =
      __builtin_amdgcn_make_buffer_rsrc((void*)(a.hcnt + pp.h0), (short)0, nh * 4, kBufferConfig);
  #pragma unroll
  for (int r = 0; r < kRowHistPer; ++r) {
    const int h = r * kRowThreads + tid;
    pp.hid[r] = (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(ri, h * 4, 0, 0);
    pp.hcs[r] = (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(rc, h * 4, 0, 0);
    if (h >= nh) pp.hid[r] = 0xffffffffu;
  }
}

// The fast path of one row, with its first tiles in flight (row_issue);
// false sends the row to the general path (all threads return the same).
template <bool MASK>
__device__ __forceinline__ bool row_stream(RowLds& L, const SampleArgs& a, int row, const RowCfg& cfg,
                                           unsigned char* lds_raw, RowPipe<MASK>& pp) {
  const int tid = threadIdx.x;
  const uint32_t lane = (uint32_t)tid & 63u;
  const int wid = tid >> 6;
  const int V = a.V;
  const int Wm = (V + 31) >> 5;
  const int ntiles = (V + kRowTile - 1) / kRowTile;
  // word w of the row's history: {bits of logits 32w..32w+31, marked logits before 32w}
  uint2* hw = reinterpret_cast<uint2*>(lds_raw + kRowHead);
  const float* lrow = reinterpret_cast<const float*>((const char*)a.logits + (int64_t)row * a.row_stride * 4);
  const uint32_t* mrow = MASK ? a.mask + (int64_t)row * a.mask_words : nullptr;

  // 1. the loads in flight
  const uint32_t h0 = pp.h0, h1 = pp.h1;
  const bool hist = h1 > h0;
  auto& hid = pp.hid;
  auto& hcs = pp.hcs;
  const __amdgpu_buffer_rsrc_t rs = pp.rs;
  const __amdgpu_buffer_rsrc_t ms = pp.ms;
  auto& buf = pp.buf;
  auto& mw = pp.mw;

  // 2. the stream state
  const uint32_t kk = (uint32_t)cfg.k_sel;  // 1..kLeanK
  const uint32_t kw = min(kk, (kk + 15u) / 16u + (uint32_t)ceilf(sqrtf((float)kk)) + 4u);
  uint64_t* wl = L.wbuf[wid];
  float* xs = L.xscr[wid];
  uint32_t* wh = reinterpret_cast<uint32_t*>(xs);  // the selection histogram (xs is idle then)
  uint32_t wn = 0u;              // entries in this wave's list
  uint32_t T = kKeyNegInf;       // the wave's threshold key (strict)
  float tf = -__builtin_inff();  // the float of T
  int32_t ti = INT32_MIN;        // the bits of tf when T is a positive key, else INT32_MIN
  auto set_t = [&](uint32_t key) {
    T = key;
    tf = okey_inv(key);
    ti = key > 0x80000000u ? (int32_t)__float_as_uint(tf) : INT32_MIN;
  };
  bool bad = false;              // the list overflowed

  // One tile: tile t from slot D, which is then refilled with tile
  // t + kRowDepth.  Every slot is processed and refilled on every pass, also
  // past the row's last tile (those logits read as -inf and their loads move
  // no memory): with no conditional load in the loop the compiler keeps the
  // other slot's loads in flight while it waits for one slot.
  auto step = [&](auto slot, int t, bool first) {
    constexpr int D = decltype(slot)::value;
    const int base = t * kRowTile;
    float x[kRowEl];
    #pragma unroll
    for (int j = 0; j < kRowTV; ++j) {
      const int e0 = base + (j * kRowThreads + tid) * 4;
      const uint32_t mbits = MASK ? mw[D][j] >> (e0 & 31) : 0xfu;
      #pragma unroll
      for (int q = 0; q < 4; ++q) {
        float v = __int_as_float(buf[D][j][q]);
        if (MASK && !((mbits >> q) & 1u)) v = -__builtin_inff();
        x[j * 4 + q] = v;
      }
    }
    if (base + kRowTile > V) {
      #pragma unroll
      for (int j = 0; j < kRowTV; ++j) {
        const int e0 = base + (j * kRowThreads + tid) * 4;
        #pragma unroll
        for (int q = 0; q < 4; ++q) if (e0 + q >= V) x[j * 4 + q] = -__builtin_inff();
      }
    }
    if (first) {
      // first tile: a bound with at least kw of the wave's logits at or
      // above it, from its group maxima (4 logits of a lane each): the
      // largest prefix of 20 key bits that kw group maxima reach
      constexpr int NG = kRowEl / 4;
      uint32_t gk[NG];
      #pragma unroll
      for (int g = 0; g < NG; ++g)
        gk[g] = lkey(fmaxf(fmaxf(x[4 * g], x[4 * g + 1]), fmaxf(x[4 * g + 2], x[4 * g + 3])));
      static_assert(NG == 4, "four group maxima per lane");
      const uint32_t prefix = wave_prefix_reach(gk, kw);
      if (prefix > kKeyNegInf + 1u) set_t(prefix - 1u);
    }
    // any logit above the threshold?  Against a positive threshold the raw
    // bits compare as signed integers (negative logits fall below; a NaN
    // passes here and fails the exact test); against any other ti is
    // INT_MIN and every tile takes the exact test
    int32_t mi = (int32_t)__float_as_uint(x[0]);
    #pragma unroll
    for (int e = 1; e < kRowEl; ++e) mi = max(mi, (int32_t)__float_as_uint(x[e]));
    if (__ballot(mi > ti) != 0ull) {
      // survivors: key above T, i.e. x > tf (NaN never passes; +inf passes
      // and sends the row to the general path at the end); the signed-zero
      // threshold compares keys
      uint32_t sb = 0u;
      if (T == kKeyNegZero) {
        #pragma unroll
        for (int e = 0; e < kRowEl; ++e) sb |= lkey(x[e]) > T ? (1u << e) : 0u;
      } else {
        #pragma unroll
        for (int e = 0; e < kRowEl; ++e) sb |= x[e] > tf ? (1u << e) : 0u;
      }
      if (__ballot(sb != 0u) != 0ull) {
        row_spill(xs, x);
        // appended one per lane per round (the list stops at its capacity)
        for (;;) {
          const uint64_t m = __ballot(sb != 0u);
          if (m == 0ull) break;
          const uint32_t add = (uint32_t)__popcll(m);
          if (wn + add > (uint32_t)kRowCap) {
            bad = true;
            break;
          }
          if (sb != 0u) {
            const uint32_t e = (uint32_t)__builtin_ctz(sb);
            sb &= sb - 1u;
            const uint32_t idx = (uint32_t)(base + ((int)(e >> 2) * kRowThreads + tid) * 4) + (e & 3u);
            wl[wn + lanes_below(m)] = cand_key(okey(row_elem(xs, e)), idx);
          }
          wn += add;
        }
        if (wn > (uint32_t)kRowHW) set_t(row_wave_keep(wl, wn, kw, wh));
        wave_lds_sync();  // xs is read before the next spill
      }
    }
    #pragma unroll
    for (int j = 0; j < kRowTV; ++j) {
      const int e0 = (t + kRowDepth) * kRowTile + (j * kRowThreads + tid) * 4;
      buf[D][j] = __builtin_amdgcn_raw_buffer_load_b128(rs, e0 * 4, 0, kStreamLoad);
      if (MASK) mw[D][j] = (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(ms, (e0 >> 5) * 4, 0, 0);
    }
  };
  using Slot0 = std::integral_constant<int, 0>;
  using Slot1 = std::integral_constant<int, 1>;
  static_assert(kRowDepth == 2, "the stream alternates two slots");

  // 3. the first two tiles
  step(Slot0{}, 0, true);
  step(Slot1{}, 1, false);

  // 4. the history ranked, while tiles 2 and 3 are in flight (its entries
  //    were issued before them, so they have arrived): marks and rank
  //    prefix, then the summed count and id of each distinct token by rank,
  //    whose logit is loaded during the stream
  constexpr uint32_t kFirst = (uint32_t)(kRowHistPer * kRowThreads);
  uint32_t distinct = 0u;
  if (hist) {
    for (int i = tid; i < Wm; i += kRowThreads) hw[i] = make_uint2(0u, 0u);
    for (int r = tid; r < kRowHistCap; r += kRowThreads) L.ob_cnt[r] = 0u;
    __syncthreads();
    auto mark = [&](uint32_t id) {
      if (id < (uint32_t)V) atomicOr(&hw[id >> 5].x, 1u << (id & 31u));
    };
    #pragma unroll
    for (int r = 0; r < kRowHistPer; ++r) mark(hid[r]);
    for (uint32_t h = h0 + kFirst + (uint32_t)tid; h < h1; h += kRowThreads) mark(a.hids[h]);
    __syncthreads();
    // prefix: wave v owns the contiguous words [v * PB, (v + 1) * PB), read
    // 64 consecutive words at a time (no LDS bank conflicts)
    const int PB = (((Wm + kRowWaves - 1) / kRowWaves) + 63) & ~63;
    const int w0 = wid * PB;
    uint32_t wsum = 0u;
    for (int b = 0; b < PB; b += 64) {
      const int w = w0 + b + (int)lane;
      wsum += w < Wm ? (uint32_t)__popc(hw[w].x) : 0u;
    }
    wsum = wave_sum_u32(wsum);
    if (lane == 0u) L.redu[wid] = wsum;
    __syncthreads();
    uint32_t run = 0u;
    #pragma unroll
    for (int v = 0; v < kRowWaves; ++v) {
      const uint32_t c = L.redu[v];
      run += v < wid ? c : 0u;
      distinct += c;
    }
    if (distinct > (uint32_t)kRowHistCap) return false;
    for (int b = 0; b < PB; b += 64) {
      const int w = w0 + b + (int)lane;
      const uint32_t c = w < Wm ? (uint32_t)__popc(hw[w].x) : 0u;
      const uint32_t incl = wave_incl_scan_u32(c);
      if (w < Wm) hw[w].y = run + incl - c;
      run += wave_last_u32(incl);
    }
    __syncthreads();
    auto add = [&](uint32_t id, uint32_t c) {
      if (id < (uint32_t)V) {
        const uint2 h = hw[id >> 5];
        const uint32_t rank = h.y + (uint32_t)__popc(h.x & ((1u << (id & 31u)) - 1u));
        atomicAdd(&L.ob_cnt[rank], c);
        L.ob_id[rank] = id;  // every occurrence writes the same id
      }
    };
    #pragma unroll
    for (int r = 0; r < kRowHistPer; ++r) add(hid[r], hcs[r]);
    for (uint32_t h = h0 + kFirst + (uint32_t)tid; h < h1; h += kRowThreads) add(a.hids[h], a.hcnt[h]);
    __syncthreads();  // the summed counts are complete before any wave's stream ends
  }
  // the history tokens' logits, in flight during the stream: unconditional
  // range-checked loads (an id past the row reads zero and is not stored)
  uint32_t hraw[kRowHistPer], hmw[kRowHistPer];
  #pragma unroll
  for (int r = 0; r < kRowHistPer; ++r) {
    hraw[r] = (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(rs, (int)(hid[r] * 4u), 0, 0);
    if (MASK) hmw[r] = (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(ms, (int)((hid[r] >> 5) * 4u), 0, 0);
  }

  // 5. the rest of the row, tiles 2, 3, ... (the last pass may run past it)
  const int npass = (ntiles + 1) / 2;
  for (int p = 1; p < npass; ++p) {
    step(Slot0{}, 2 * p, false);
    step(Slot1{}, 2 * p + 1, false);
  }
  if (lane == 0u) {
    L.wthr[wid] = T;
    L.wbad[wid] = bad ? 1u : 0u;
    L.wcnt[wid] = wn;
  }
  if (hist) {
    auto put = [&](uint32_t id, uint32_t raw) {
      const uint2 h = hw[id >> 5];
      const uint32_t rank = h.y + (uint32_t)__popc(h.x & ((1u << (id & 31u)) - 1u));
      const float l = __uint_as_float(raw);
      const uint32_t c = L.ob_cnt[rank];
      L.ob_raw[rank] = lkey(cfg.rep_on ? apply_penalties(l, c, cfg) : apply_penalties_norep(l, c, cfg));
    };
    constexpr uint32_t kNegInfBits = 0xff800000u;
    #pragma unroll
    for (int r = 0; r < kRowHistPer; ++r) {
      if (hid[r] < (uint32_t)V) put(hid[r], MASK && !((hmw[r] >> (hid[r] & 31u)) & 1u) ? kNegInfBits : hraw[r]);
    }
    for (uint32_t h = h0 + kFirst + (uint32_t)tid; h < h1; h += kRowThreads) {
      const uint32_t id = a.hids[h];
      if (id < (uint32_t)V) {
        const bool off = MASK && !((mrow[id >> 5] >> (id & 31u)) & 1u);
        put(id, off ? kNegInfBits : __float_as_uint(lrow[id]));
      }
    }
  }
  __syncthreads();  // lists, thresholds and the history complete

  // 6. the rest runs on the first NT threads, one wave per SIMD; the other
  //    waves end here (ended waves no longer count at barriers)
  if (wid >= NT / 64) return true;
  uint32_t Tm = L.wthr[0];
  uint32_t anybad = L.wbad[0];
  #pragma unroll
  for (int w = 1; w < kRowWaves; ++w) { Tm = max(Tm, L.wthr[w]); anybad |= L.wbad[w]; }
  if (anybad) return false;

  // the candidates: list entries that are not history tokens and processed
  // history logits, at or above Tm.  Wave f reads the lists f, f + 4, ...
  // (lane l their entries l and l + 64: a list holds at most kRowCap)
  constexpr int kFinWaves = NT / 64;
  constexpr int kLists = kRowWaves / kFinWaves * (kRowCap / 64);
  constexpr int kHq = kRowHistCap / NT;
  static_assert(kRowCap == 128, "two list entries per lane");
  uint64_t sc[kLists];
  uint64_t hc[kHq];
  uint32_t mine = 0u;
  uint64_t top = 0ull;
  {
    // every LDS read is issued before any result is used
    uint32_t nv[kLists], mk[kLists];
    #pragma unroll
    for (int m = 0; m < kLists; ++m) {
      const int v = wid + kFinWaves * (m >> 1);
      const uint32_t i = lane + 64u * (m & 1);
      nv[m] = L.wcnt[v] > i ? 1u : 0u;
      sc[m] = L.wbuf[v][i];
    }
    if (hist) {
      #pragma unroll
      for (int m = 0; m < kLists; ++m) mk[m] = hw[min(cand_idx(sc[m]), (uint32_t)V - 1u) >> 5].x;
    }
    #pragma unroll
    for (int m = 0; m < kLists; ++m) {
      bool keep = nv[m] != 0u && cand_skey(sc[m]) >= Tm;
      if (hist) keep = keep && !((mk[m] >> (cand_idx(sc[m]) & 31u)) & 1u);
      sc[m] = keep ? sc[m] : 0ull;
      mine += keep ? 1u : 0u;
      top = sc[m] > top ? sc[m] : top;
    }
  }
  #pragma unroll
  for (int q = 0; q < kHq; ++q) hc[q] = 0ull;
  const uint32_t r0 = (uint32_t)tid * (uint32_t)kHq;  // this thread's ranks: r0 .. r0 + kHq - 1
  if (r0 < distinct) {
    static_assert(kHq % 4 == 0, "ranks are read four at a time");
    uint32_t kys[kHq], ids[kHq];
    #pragma unroll
    for (int q = 0; q < kHq; q += 4) {
      const uint4 x = *reinterpret_cast<const uint4*>(&L.ob_raw[r0 + q]);
      const uint4 i = *reinterpret_cast<const uint4*>(&L.ob_id[r0 + q]);
      kys[q] = x.x; kys[q + 1] = x.y; kys[q + 2] = x.z; kys[q + 3] = x.w;
      ids[q] = i.x; ids[q + 1] = i.y; ids[q + 2] = i.z; ids[q + 3] = i.w;
    }
    #pragma unroll
    for (int q = 0; q < kHq; ++q) {
      const uint32_t k = kys[q];
      const bool keep = r0 + q < distinct && k > kKeyNegInf && k >= Tm;
      hc[q] = keep ? cand_key(k, ids[q]) : 0ull;
      mine += keep ? 1u : 0u;
      top = hc[q] > top ? hc[q] : top;
    }
  }
  // one barrier for the candidates' positions and the row's top key
  uint32_t pos, n = 0u;
  {
    const uint32_t incl = wave_incl_scan_u32(mine);
    const uint64_t wtop = wave_max_u64(top);
    if (lane == 63u) { L.redu[wid] = incl; L.red64[wid] = wtop; }
    __syncthreads();  // also: every LDS input above has been read
    uint32_t before = 0u;
    top = 0ull;
    #pragma unroll
    for (int v = 0; v < kFinWaves; ++v) {
      const uint32_t c = L.redu[v];
      before += v < wid ? c : 0u;
      n += c;
      top = L.red64[v] > top ? L.red64[v] : top;
    }
    pos = before + incl - mine;
  }
  // +inf logits rank as -inf (gpu.rs:767-777): the general path resolves
  // them; fewer candidates than kk hold the row's top kk only if nothing
  // finite was left out
  if (n == 0u || n > (uint32_t)kGather || cand_skey(top) >= kKeyPosInf) return false;
  if (n < kk && Tm > kKeyNegInf) return false;
  FinLds& fs = *reinterpret_cast<FinLds*>(lds_raw);
  #pragma unroll
  for (int m = 0; m < kLists; ++m) if (sc[m] != 0ull) fs.cbig[pos++] = sc[m];
  #pragma unroll
  for (int q = 0; q < kHq; ++q) if (hc[q] != 0ull) fs.cbig[pos++] = hc[q];
  __syncthreads();
  const float M = key_to_s(cand_skey(top), cfg.t_eff);
  // key bounds for the selection: every candidate's key is at least Tm
  // (the 16-wave row kernel keeps the workgroup select: the one-wave select's
  // registers cost its stream more than the select saves)
  return finish_core(fs, a, row, cfg, (int)n, M, Tm > kKeyNegInf ? Tm : 0u, 0.0, Tm, (uint64_t)Tm << 32, top, false);
}

// The general path of a row (see the section comment), on the first NT
// threads: the chunk select and the finish of the two-kernel path.  It is
// not inlined, so that its register demand (it spills) stays out of the
// fast path's code.  `ap` points at the row kernel's own SampleArgs
// argument in the kernel argument segment: a pointer to a local copy would
// make every workgroup store that copy to scratch memory on entry.
typedef const __attribute__((address_space(4))) SampleArgs KernargSampleArgs;

template <bool MASK>
__device__ __noinline__ void row_general(KernargSampleArgs* ap, int row) {
  extern __shared__ __align__(16) unsigned char lds_raw[];
  SampleArgs a;
  {
    static_assert(sizeof(SampleArgs) % 8 == 0, "copied 8 bytes at a time");
    typedef const __attribute__((address_space(4))) uint64_t KernargWord;
    KernargWord* w = (KernargWord*)ap;
    uint64_t* d = reinterpret_cast<uint64_t*>(&a);
    #pragma unroll
    for (int i = 0; i < (int)(sizeof(SampleArgs) / 8); ++i) d[i] = w[i];
  }
  // 8192-logit chunks (the launch's records are not used here): half the
  // registers of 16384-logit ones, which halves the path's spills (its
  // scratch is allocated for every wave of the launch, and costs the
  // launch time even when no row comes here)
  a.chunk = kRowGeneralChunk;
  a.n_chunks = (a.V + kRowGeneralChunk - 1) / kRowGeneralChunk;
  const RowCfg cfg = load_cfg(a.pv, row, a.V, a.n_lp, a.need_lse);
  for (int c = 0; c < a.n_chunks; ++c) {
    select_chunk<HI_ROCM_DTYPE_F32, kRowGeneralChunk / NT / 4, MASK>(a, row, c, lds_raw);
    __syncthreads();
  }
  FinLds& fs = *reinterpret_cast<FinLds*>(lds_raw);
  if (finish_lean(fs, a, row, cfg)) return;
  __syncthreads();
  finish_row(fs, a, row, cfg);
}

// The row kernel's arguments as its argument segment lays them out: each at
// the next offset aligned for its type, as in this struct.
struct RowKernelArgs {
  const void* logits;
  int64_t row_stride;
  int V;
  SampleArgs a;
};

// One workgroup per row (see the section comment).  The first tiles' loads
// need only the logits, the row stride and V: they lead the kernel's
// arguments, which gfx950 preloads into scalar registers at wave launch
// (the library is built with -amdgpu-kernarg-preload-count), so the loads
// do not wait for an argument fetch.
template <bool MASK>
__global__ void __launch_bounds__(kRowThreads) row_kernel(const void* logits, int64_t row_stride, int V,
                                                          SampleArgs a) {
  extern __shared__ __align__(16) unsigned char lds_raw[];
  RowLds& L = *reinterpret_cast<RowLds*>(lds_raw);
  const int row = blockIdx.x;
  a.logits = logits;  // the same values, from the preloaded arguments
  a.row_stride = row_stride;
  a.V = V;
  RowPipe<MASK> pp;
  row_issue<MASK>(a, row, pp);  // unused by rows that take the general path
  const RowCfg cfg = load_cfg(a.pv, row, a.V, a.n_lp, a.need_lse);
  if (cfg.cls == kTopK && !cfg.wide) {
    if (row_stream<MASK>(L, a, row, cfg, lds_raw, pp)) return;
    __syncthreads();
  }
  if (threadIdx.x >= NT) return;
  typedef const __attribute__((address_space(4))) char KernargByte;
  row_general<MASK>(
      (KernargSampleArgs*)((KernargByte*)__builtin_amdgcn_kernarg_segment_ptr() + offsetof(RowKernelArgs, a)), row);
}

size_t row_lds_bytes(int V) {
  const size_t fast = kRowHead + sizeof(uint2) * ((V + 31) / 32);
  const size_t general = kSelHead + sel_hist_bytes(kSelChunkLarge);
  size_t b = fast > general ? fast : general;
  return b > sizeof(FinLds) ? b : sizeof(FinLds);
}

constexpr size_t kLdsPerCu = 160 * 1024;  // gfx950

bool row_kernel_fits(const SampleArgs& a) {
  return a.dtype == HI_ROCM_DTYPE_F32 && a.B >= kRowMinBatch && a.n_lp == 0 && a.out_token_lp == nullptr &&
         a.vec_ok && a.chunk == kSelChunkLarge && a.V <= kRowMaxV && row_lds_bytes(a.V) <= kLdsPerCu;
}

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

template <int DT, int NL, bool MASK>
hipError_t launch_select_t(const SampleArgs& a, hipStream_t stream) {
  constexpr int E = NL * (DT == HI_ROCM_DTYPE_BF16 ? 8 : 4);
  const size_t lds = kSelHead + (a.hoff ? sel_hist_bytes(NT * E) : 0);
  hipLaunchKernelGGL((select_kernel<DT, NL, MASK>), dim3(a.n_chunks, a.B), dim3(NT), lds, stream, a);
  return hipGetLastError();
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

template <int DT, bool MASK>
hipError_t launch_select_d(const SampleArgs& a, hipStream_t stream) {
  constexpr int EPL = DT == HI_ROCM_DTYPE_BF16 ? 8 : 4;
  if (a.chunk == kSelChunkLarge) return launch_select_t<DT, kSelChunkLarge / NT / EPL, MASK>(a, stream);
  return launch_select_t<DT, kSelChunkSmall / NT / EPL, MASK>(a, stream);
}

template <bool MASK>
hipError_t launch_rows(const SampleArgs& a, hipStream_t stream) {
  const size_t lds = row_lds_bytes(a.V);
  hipError_t e = ensure_lds((const void*)row_kernel<MASK>, lds);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(row_kernel<MASK>, dim3(a.B), dim3(kRowThreads), lds, stream, a.logits, a.row_stride, a.V, a);
  return hipGetLastError();
}

hipError_t launch_sample(const SampleArgs& a, hipStream_t stream, const LaunchEvents* le) {
  if (!select_mode(a.n_lp, a.vec_ok) || (a.chunk != kSelChunkLarge && a.chunk != kSelChunkSmall))
    return launch_chunked(a, stream, le);
  hipError_t e = record(le, 0, stream);
  if (e != hipSuccess) return e;
  if (row_kernel_fits(a)) {
    e = a.mask ? launch_rows<true>(a, stream) : launch_rows<false>(a, stream);
    if (e == hipSuccess) e = record(le, 1, stream);
    return e == hipSuccess ? record(le, 2, stream) : e;
  }
  if (fused_fits(a)) {
    if (a.dtype == HI_ROCM_DTYPE_BF16)
      e = a.mask ? launch_fused_d<HI_ROCM_DTYPE_BF16, true>(a, stream) : launch_fused_d<HI_ROCM_DTYPE_BF16, false>(a, stream);
    else
      e = a.mask ? launch_fused_d<HI_ROCM_DTYPE_F32, true>(a, stream) : launch_fused_d<HI_ROCM_DTYPE_F32, false>(a, stream);
    if (e == hipSuccess) e = record(le, 1, stream);
    return e == hipSuccess ? record(le, 2, stream) : e;
  }
  if (a.dtype == HI_ROCM_DTYPE_BF16)
    e = a.mask ? launch_select_d<HI_ROCM_DTYPE_BF16, true>(a, stream) : launch_select_d<HI_ROCM_DTYPE_BF16, false>(a, stream);
  else
    e = a.mask ? launch_select_d<HI_ROCM_DTYPE_F32, true>(a, stream) : launch_select_d<HI_ROCM_DTYPE_F32, false>(a, stream);
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

template <int RG>
hipError_t launch_lm_logits_rg(const LmArgs& a, hipStream_t stream) {
  const size_t lds = lm_tile_lds(a.B);
  hipError_t e = ensure_lds((const void*)lm_logits_kernel<RG>, lds);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(lm_logits_kernel<RG>, dim3((unsigned)a.n_chunks), dim3(kLmThreads), lds, stream, a);
  return hipGetLastError();
}

hipError_t launch_lm_logits(const LmArgs& a, hipStream_t stream) {
  return a.B <= 32 ? launch_lm_logits_rg<1>(a, stream) : launch_lm_logits_rg<2>(a, stream);
}

hipError_t launch_lm_sample(const LmArgs& a, hipStream_t stream) {
  const size_t l1 = lm_tile_lds(a.B);
  const void* sel = a.B <= 32 ? (const void*)lm_select_kernel<1> : (const void*)lm_select_kernel<2>;
  hipError_t e = ensure_lds(sel, l1);
  if (e != hipSuccess) return e;
  if (a.B <= 32)
    hipLaunchKernelGGL(lm_select_kernel<1>, dim3((unsigned)a.n_chunks), dim3(kLmThreads), l1, stream, a);
  else
    hipLaunchKernelGGL(lm_select_kernel<2>, dim3((unsigned)a.n_chunks), dim3(kLmThreads), l1, stream, a);
  e = hipGetLastError();
  if (e != hipSuccess) return e;
  const size_t l2 = lm_finish_lds();
  e = ensure_lds((const void*)lm_finish_kernel, l2);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(lm_finish_kernel, dim3((unsigned)a.B), dim3(NT), l2, stream, a);
  return hipGetLastError();
}

}  // namespace hi_rocm
