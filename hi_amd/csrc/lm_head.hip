// hi-rocm: the LM-head projection + bias + softcap, alone (the twin) or fused
// into the sampler's first pass, and their launchers.
#include "sampler_wide.h"

namespace hi_rocm {

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
// leaves the tile's logits in the workspace for every row that is not
// greedy: a top-k row's finish reads back the few tiles that can hold the
// row's top k, and the rows it cannot resolve (other classes, a cut between
// distinct logits of equal weight) take the general per-row path over the
// whole row (greedy rows write no logits at all).  The twin kernel runs the same code and
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
// (with temperature, top-p, min-p), and plain: no mask, no logprobs, and no
// penalty that changes a logit (the records hold the logits as the
// projection gives them).
__device__ __forceinline__ bool lm_plain(const LmArgs& a, int row, const RowCfg& c) {
  if (a.gen.mask != nullptr || a.gen.n_lp > 0 || a.gen.out_token_lp != nullptr) return false;
  const bool hist = a.gen.hoff != nullptr && a.gen.hoff[row + 1] > a.gen.hoff[row];
  return !(hist && (c.rep_on || c.freq != 0.f || c.pres != 0.f));
}
__device__ __forceinline__ bool lm_row_ok(const LmArgs& a, int row, const RowCfg& c) {
  return (c.cls == kGreedy || (c.cls == kTopK && c.k_eff <= kLmMaxK)) && lm_plain(a, row, c);
}

// IEEE '>' argmax key of a value above -inf: -0 counts as +0 (the two are
// equal under '>', so the lowest index among them wins).
__device__ __forceinline__ uint64_t ieee_key(float l, uint32_t e) { return cand_key(okey(l == 0.f ? 0.f : l), e); }

// The fused pass: per (row, tile) records.  Wave w takes the rows w,
// w + kLmThreads / 64, ... of the tile.  Every row but a greedy one also
// leaves the tile's logits in the workspace (greedy rows leave nothing but
// the records).
template <int RG>
__global__ void __launch_bounds__(kLmThreads) __attribute__((amdgpu_waves_per_eu(lm_waves_per_eu<RG>(), 8)))
    lm_select_kernel(LmArgs a) {
  extern __shared__ __align__(16) unsigned char lds_raw[];
  float* tile = reinterpret_cast<float*>(lds_raw);
  const int t = blockIdx.x, tile0 = t * kLmTile;
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  // lane m: whether row m keeps its tile logits (every row but a plain
  // greedy one), loaded before the product so that its latency hides there
  uint32_t keep = 0u;
  if (lane < a.B) {
    const RowCfg cfg = load_cfg(a.pv, lane, a.V, 0, 0);
    keep = (cfg.cls == kGreedy && lm_plain(a, lane, cfg)) ? 0u : 1u;
  }
  lm_gemm_tile<RG>(a, tile0, tile);
  __syncthreads();
  const int len = min(kLmTile, a.V - tile0);
  constexpr int PER = kLmTile / 64;
  for (int m = wid; m < a.B; m += kLmThreads / 64) {
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
  // the tile logits of the rows that keep them, row after row as the twin
  // writes them (a wave covers half a row, so the flag is uniform over it)
  for (int i = threadIdx.x; i < a.B * kLmTile; i += kLmThreads) {
    const int m = i / kLmTile, c = i % kLmTile;
    const uint32_t k = (uint32_t)__builtin_amdgcn_readlane((int)keep, m);
    if (k != 0u && c < len) a.lm_logits[(int64_t)m * lm_stride(a.V) + tile0 + c] = tile[i];
  }
}

typedef const __attribute__((address_space(4))) SampleArgs KernargSampleArgs;
typedef const __attribute__((address_space(4))) char KernargByte;

// The general per-row path (general_row_path) over the row's logits in the
// workspace, for the rows the fused finish does not resolve.  Not inlined,
// so that its register demand stays out of the fused finish; `ap` points at
// the kernel's own LmArgs::gen in the argument segment (a pointer to a local
// copy would make every workgroup store that copy to scratch on entry).
__device__ __noinline__ void lm_general(KernargSampleArgs* ap, int row) {
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
  if (a.mask) general_row_path<true>(a, row, lds_raw);
  else general_row_path<false>(a, row, lds_raw);
}

__device__ __forceinline__ KernargSampleArgs* lm_gen_args() {
  return (KernargSampleArgs*)((KernargByte*)__builtin_amdgcn_kernarg_segment_ptr() + offsetof(LmArgs, gen));
}

// The fused finish: one workgroup per row (gpu.rs:753-900 on the row's
// candidates, as the lean finish does).  Rows of other classes, rows with a
// mask, logprobs or penalties, and top-k rows whose cut falls between
// distinct logits of equal weight, take the general per-row path over the
// row's logits in the workspace: every row gets its token.
__global__ void __launch_bounds__(NT) lm_finish_kernel(LmArgs a) {
  extern __shared__ __align__(16) unsigned char lds_raw[];
  FinLds& fs = *reinterpret_cast<FinLds*>(lds_raw);
  const int row = blockIdx.x, tid = threadIdx.x;
  const RowCfg cfg = load_cfg(a.pv, row, a.V, 0, 0);
  if (!lm_row_ok(a, row, cfg)) {
    lm_general(lm_gen_args(), row);
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
  const float* lg = a.lm_logits + (int64_t)row * lm_stride(a.V);
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
      __syncthreads();
      lm_general(lm_gen_args(), row);
      return;
    }
  }
  sort_ranked(fs, k);
  const int pick = wg_draw<kLmMaxK / 64>(fs, fs.buf, k, cfg);
  if (tid == 0) a.out_tokens[row] = pick < 0 ? host_argmax : cand_idx(fs.buf[pick]);
}

size_t lm_recs_bytes(int B, int n_tiles) { return ((size_t)B * n_tiles * sizeof(LmTileRec) + 255) & ~(size_t)255; }
size_t lm_logits_bytes(int B, int V) { return ((size_t)B * lm_stride(V) * sizeof(float) + 255) & ~(size_t)255; }
size_t lm_workspace_bytes(int B, int V) {
  const int tiles = (V + kLmTile - 1) / kLmTile;
  return lm_recs_bytes(B, tiles) + lm_logits_bytes(B, V) + general_layout(B, V).total;
}

size_t lm_tile_lds(int B) { return (size_t)(B <= 32 ? 32 : kLmRows) * kLmTile * sizeof(float); }
size_t lm_finish_lds(bool hist) {
  const size_t gen = kSelHead + (hist ? sel_hist_bytes(kRowGeneralChunk) : 0);  // general_row_path
  const size_t b = sizeof(FinLds) > gen ? sizeof(FinLds) : gen;
  return (b + 15) & ~(size_t)15;
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
  const size_t l2 = lm_finish_lds(a.gen.hoff != nullptr);
  e = ensure_lds((const void*)lm_finish_kernel, l2);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(lm_finish_kernel, dim3((unsigned)a.B), dim3(NT), l2, stream, a);
  return hipGetLastError();
}

}  // namespace hi_rocm
