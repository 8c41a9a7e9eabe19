// hi-rocm: the row kernel (one workgroup streams a whole row and finishes
// it in place) for large batches, and its launcher.
#include "sampler_wide.h"

namespace hi_rocm {

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
constexpr int kRowSCap = 512;                         // min-p support entries held in LDS
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
  // min-p rows: the logits each wave keeps at the end of its stream (list
  // entries and processed history logits at or above its bound), their
  // count, the largest processed-logit key seen so far
  uint64_t sbuf[kRowSCap];
  uint64_t exptab[32];                 // exact_expf's table (wave 0 copies it at its stream's end)
  // [kSCnt] entries in sbuf, [kSMax] the largest key seen so far, [kSThr] the
  // largest list threshold, [kSBad] a list overflowed: one 16-byte read
  alignas(16) uint32_t sst[4];
  uint32_t sdone;                      // wave 0's min-p finish: kMinpOk, or why it missed
};
enum : int { kSCnt = 0, kSMax = 1, kSThr = 2, kSBad = 3 };
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

// ---- min-p rows -----------------------------------------------------------
//
// With min_p > 0 only the logits whose weight w = expf(s - M) reaches min_p
// are ever drawn or summed: the reference gives every other one weight 0
// (gpu.rs:847-849 skips w <= 0; min-p extends that to w < min_p), and the
// rank order puts them after the others.  Weights are monotone in the
// processed logit, so that support S is every logit above one key.  At the
// end of its stream each wave keeps, of its list and of its threads'
// processed history logits, those whose key reaches a bound below which no
// weight can reach min_p whatever the final row max (the bound comes from
// the largest key seen so far, a lower bound of the row max M), and appends
// them to L.sbuf.  After the barrier one wave (four for more than 64
// entries) computes the exact weights against M, keeps S, sorts it by
// (w desc, index asc) in registers, and runs the reference's folds: the kept top-k of the rank order is the first
// min(|S|, k) entries of S.  That needs the lists to have dropped nothing
// that ranks among them: either their thresholds' weights are below min_p
// (nothing of S was dropped), or the k-th weight of S is above them.

// Processed-logit key at and above which a weight can reach min_p when the
// row max is at least the logit of key mk: l_lo = l_m + t ln(min_p) - d, with
// a margin d far above the rounding of s = l / t, s - M and expf (a weight
// w >= min_p needs s - M >= ln(min_p) - 2^-22 or so).  Uniform per wave.
__device__ __forceinline__ uint32_t minp_key_bound(uint32_t mk, float t, float ln_mp) {
  if (mk <= kKeyNegInf) return kKeyNegInf;
  const float lm = okey_inv(mk);
  if (!finitef_(lm)) return 0xffffffffu;  // +inf: the general path takes the row
  const float span = t * ln_mp;                      // <= 0
  const float d = t * 0x1p-10f + (fabsf(lm) - span) * 0x1p-18f;
  const float lo = (lm + span) - d;
  return lkey(lo);
}

// With the support known only above the lists' largest threshold (weights
// there up to wT >= min_p), the kept top k is still exact when the support
// holds k entries and the k-th weight of the sorted support is above wT:
// every logit left out then ranks below all of them.
template <int S>
__device__ __forceinline__ bool minp_topk_known(const uint64_t (&x)[S], int c, int k, bool complete, float wT) {
  if (complete) return true;
  if (c < k) return false;
  uint64_t v = 0ull;
  #pragma unroll
  for (int m = 0; m < S; ++m)
    if (((k - 1) >> 6) == m) v = readlane64(x[m], (k - 1) & 63);
  return rank_w(v) > wT;
}

// Why the min-p finish left a row to the general finish (0: it did not).
enum MinpMiss : uint32_t { kMinpOk = 0, kMinpArray = 1, kMinpTopK = 2, kMinpDraw = 3 };

// The min-p finish of a support of at most 64 entries on one wave (see
// above).  Tm is the largest list threshold of the row.  A miss (MinpMiss)
// sends the row to the candidate lists' finish.
__device__ __forceinline__ uint32_t row_minp_finish(const RowLds& L, const RowCfg& cfg, uint32_t& token) {
  const uint32_t lane = threadIdx.x & 63u;
  const uint4 st = *reinterpret_cast<const uint4*>(L.sst);
  const uint32_t ns = st.x, mk = st.y, Tm = st.z;
  if (st.w != 0u || ns == 0u || ns > (uint32_t)kRowSCap || mk <= kKeyNegInf || mk >= kKeyPosInf) return kMinpArray;
  const Exp2TabLds tab{L.exptab};
  const float M = key_to_s(mk, cfg.t_eff);
  if (ns > 64u) return kMinpArray;  // (row_minp_finish4)
  {
    // one slot: the support stays where it is
    const uint64_t x = lane < ns ? L.sbuf[lane] : 0ull;
    uint64_t rk = 0ull;
    if (x != 0ull) {
      const float w = exact_expf_t(key_to_s(cand_skey(x), cfg.t_eff) - M, tab);
      if (w >= cfg.min_p) rk = rank_key(w, cand_idx(x));
    }
    // every logit left out of the lists has a key at or below Tm, so a
    // weight of at most wT: with wT below min_p none of them is in the support
    const float wT = Tm > kKeyNegInf ? exact_expf_t(key_to_s(Tm, cfg.t_eff) - M, tab) : 0.f;
    const bool complete = wT < cfg.min_p;
    const uint64_t km = __ballot(rk != 0ull);
    const uint32_t c = (uint32_t)__popcll(km);
    // rank by counting (distinct keys: the ranks of the kept lanes are a
    // permutation of [0, c)), then each entry moves to the lane of its rank
    const uint32_t r = wave_rank_desc(rk, km);
    const int to = rk != 0ull ? (int)(r * 4u) : 63 * 4;  // the other lanes write past c (c < 64) or
                                                        // nowhere (c == 64: every lane is kept)
    const uint32_t lo = (uint32_t)__builtin_amdgcn_ds_permute(to, (int)(uint32_t)rk);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_ds_permute(to, (int)(uint32_t)(rk >> 32));
    uint64_t y[1] = {lane < c ? ((uint64_t)hi << 32) | lo : 0ull};
    if (!minp_topk_known<1>(y, (int)c, cfg.k_eff, complete, wT)) return kMinpTopK;
    const int pick = wave_draw_r<1>(y, min((int)c, cfg.k_eff), cfg);
    if (pick < 0) return kMinpDraw;
    token = cand_idx(readlane64(y[0], pick));
    return kMinpOk;
  }
}

// The min-p finish of a support of 65 .. kRowSCap entries on the first four
// waves (one per SIMD): wave v weighs entries [v * 64S, (v + 1) * 64S) of
// L.sbuf and sorts them in registers into list v of lst (zero keys, outside
// the support, last); after a barrier each kept entry's rank is its index in
// its list plus, for every other list, the number of its keys above it (a
// binary search), and the entries ranked below k_eff land at their rank in
// out; after another barrier wave 0 draws from out.  cnt: 4 words.  Called
// by the four waves alike; the result is wave 0's (the others return kMinpOk
// and token 0).
template <int S>
__device__ __forceinline__ uint32_t row_minp_finish4(const RowLds& L, const RowCfg& cfg, uint32_t ns, uint32_t mk,
                                                     uint32_t Tm, uint64_t* lst, uint64_t* out, uint32_t* cnt,
                                                     uint32_t& token) {
  constexpr int LN = 64 * S;  // entries per list
  const uint32_t lane = threadIdx.x & 63u;
  const int v = (int)(threadIdx.x >> 6);
  const Exp2TabLds tab{L.exptab};
  const float M = key_to_s(mk, cfg.t_eff);
  const uint32_t ke = (uint32_t)cfg.k_eff;
  uint64_t rk[S];
  #pragma unroll
  for (int m = 0; m < S; ++m) {
    const uint32_t i = (uint32_t)(v * LN + m * 64) + lane;
    rk[m] = 0ull;
    if (i < ns) {
      const uint64_t x = L.sbuf[i];
      const float w = exact_expf_t(key_to_s(cand_skey(x), cfg.t_eff) - M, tab);
      if (w >= cfg.min_p) rk[m] = rank_key(w, cand_idx(x));
    }
  }
  wave_sort_desc<S>(rk);
  uint32_t cv = 0u;
  #pragma unroll
  for (int m = 0; m < S; ++m) {
    lst[v * LN + m * 64 + (int)lane] = rk[m];
    cv += (uint32_t)__popcll(__ballot(rk[m] != 0ull));
  }
  if (lane == 0u) cnt[v] = cv;
  __syncthreads();
  const uint4 cn = *reinterpret_cast<const uint4*>(cnt);
  const uint32_t c = cn.x + cn.y + cn.z + cn.w;
  // the ranks of this wave's entries among the first k_eff (keys are
  // distinct: ranks of the support are a permutation of [0, c))
  #pragma unroll
  for (int m = 0; m < S; ++m) {
    const uint32_t j = (uint32_t)(m * 64) + lane;
    if (j < cv && j < ke) {
      const uint64_t x = rk[m];
      // the keys above x in each other list, by a binary search whose
      // probes are read unconditionally (one LDS wait per step for the
      // three lists; zero keys past a list's support never pass)
      uint32_t pos[3] = {0u, 0u, 0u};
      int base[3];
      #pragma unroll
      for (int t = 0; t < 3; ++t) base[t] = ((v + 1 + t) & 3) * LN;
      #pragma unroll
      for (int st = LN; st >= 1; st >>= 1) {
        uint64_t pr[3];
        #pragma unroll
        for (int t = 0; t < 3; ++t) pr[t] = lst[base[t] + (int)min(pos[t] + (uint32_t)st, (uint32_t)LN) - 1];
        #pragma unroll
        for (int t = 0; t < 3; ++t) pos[t] = (pos[t] + (uint32_t)st <= (uint32_t)LN && pr[t] > x) ? pos[t] + (uint32_t)st : pos[t];
      }
      const uint32_t r = j + pos[0] + pos[1] + pos[2];
      if (r < ke) out[r] = x;
    }
  }
  const float wT = Tm > kKeyNegInf ? exact_expf_t(key_to_s(Tm, cfg.t_eff) - M, tab) : 0.f;
  const bool complete = wT < cfg.min_p;
  __syncthreads();
  token = 0u;
  if (v != 0) return kMinpOk;
  const uint32_t c2 = min(c, ke);
  auto draw = [&](auto slots) -> uint32_t {
    constexpr int D = decltype(slots)::value;
    uint64_t y[D];
    #pragma unroll
    for (int m = 0; m < D; ++m) {
      const uint32_t i = (uint32_t)(m * 64) + lane;
      y[m] = i < c2 ? out[i] : 0ull;
    }
    if (!minp_topk_known<D>(y, (int)c, cfg.k_eff, complete, wT)) return kMinpTopK;
    const int pick = wave_draw_r<D>(y, (int)c2, cfg);
    if (pick < 0) return kMinpDraw;
    uint64_t t = 0ull;
    #pragma unroll
    for (int m = 0; m < D; ++m)
      if ((pick >> 6) == m) t = readlane64(y[m], pick & 63);
    token = cand_idx(t);
    return kMinpOk;
  };
  static_assert(kLeanK <= 256, "four slots hold the kept top k");
  if (c2 <= 64u) return draw(std::integral_constant<int, 1>{});
  if (c2 <= 128u) return draw(std::integral_constant<int, 2>{});
  return draw(std::integral_constant<int, 4>{});
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
  constexpr uint32_t kFirst = (uint32_t)(kRowHistPer * kRowThreads);
  // min-p rows take the min-p finish when their history entries sit in
  // registers (at most kFirst)
  bool sp = cfg.min_p > 0.f && (!hist || h1 - h0 <= kFirst);
  uint32_t minp_miss = 0u;  // why the min-p finish missed (diag bits 8-15)
  const float ln_mp = sp ? logf(cfg.min_p) : 0.f;
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

  // 3. the first two tiles (the min-p state is set before any wave's stream
  //    can end: the history ranking below has barriers, else one here)
  if (sp && tid == 0) {
    L.sst[kSCnt] = 0u;
    L.sst[kSMax] = kKeyNegInf;
    L.sst[kSThr] = 0u;
    L.sst[kSBad] = 0u;
  }
  if (sp && !hist) __syncthreads();
  step(Slot0{}, 0, true);
  step(Slot1{}, 1, false);

  // 4. the history ranked, while tiles 2 and 3 are in flight (its entries
  //    were issued before them, so they have arrived): marks and rank
  //    prefix, then the summed count and id of each distinct token by rank,
  //    whose logit is loaded during the stream
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
    // min-p rows append each history token once: with no id repeated in
    // the list, the entries holding an id below V are as many as the
    // distinct tokens (else the row takes the candidate lists' finish)
    uint32_t nv = 0u;
    #pragma unroll
    for (int r = 0; r < kRowHistPer; ++r) nv += hid[r] < (uint32_t)V ? 1u : 0u;
    nv = wave_sum_u32(nv);
    if (lane == 0u) {
      L.redu[wid] = wsum;
      L.red64[wid] = nv;
    }
    __syncthreads();
    uint32_t run = 0u, valid = 0u;
    #pragma unroll
    for (int v = 0; v < kRowWaves; ++v) {
      const uint32_t c = L.redu[v];
      run += v < wid ? c : 0u;
      distinct += c;
      valid += (uint32_t)L.red64[v];
    }
    if (distinct > (uint32_t)kRowHistCap) return false;
    sp = sp && valid == distinct;
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
  if (sp) {
    // a lower bound of the row max for the waves' end-of-stream bounds: the
    // largest key of this wave's list after its first two tiles that is not
    // a history token
    uint32_t mx = 0u;
    #pragma unroll
    for (int m = 0; m < 2; ++m) {
      const uint32_t i = lane + 64u * (uint32_t)m;
      const uint64_t x = i < wn ? wl[i] : 0ull;
      const uint32_t id = min(cand_idx(x), (uint32_t)V - 1u);
      const bool off = hist && ((hw[id >> 5].x >> (id & 31u)) & 1u);
      if (x != 0ull && !off) mx = max(mx, cand_skey(x));
    }
    mx = wave_max_u32(mx);
    if (lane == 0u && mx != 0u) atomicMax(&L.sst[kSMax], mx);
  }
  // the history tokens' logits, in flight during the stream: unconditional
  // range-checked loads (an id past the row reads zero and is not stored)
  uint32_t hraw[kRowHistPer], hmw[kRowHistPer];
  #pragma unroll
  for (int r = 0; r < kRowHistPer; ++r) {
    hraw[r] = (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(rs, (int)(hid[r] * 4u), 0, 0);
    if (MASK) hmw[r] = (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(ms, (int)((hid[r] >> 5) * 4u), 0, 0);
  }

  // the penalties of this thread's history entries held in registers
  // (their logits and mask words arrive behind tiles 2 and 3, so applying
  // them after the first pass below waits for nothing the stream needs)
  uint32_t hk[kRowHistPer];  // processed keys of this thread's history entries
  #pragma unroll
  for (int r = 0; r < kRowHistPer; ++r) hk[r] = kKeyNegInf;
  auto put = [&](uint32_t id, uint32_t raw) {
    const uint2 h = hw[id >> 5];
    const uint32_t rank = h.y + (uint32_t)__popc(h.x & ((1u << (id & 31u)) - 1u));
    const float l = __uint_as_float(raw);
    const uint32_t c = L.ob_cnt[rank];
    const uint32_t k = lkey(cfg.rep_on ? apply_penalties(l, c, cfg) : apply_penalties_norep(l, c, cfg));
    L.ob_raw[rank] = k;
    return k;
  };
  constexpr uint32_t kNegInfBits = 0xff800000u;
  auto put_registers = [&]() {
    if (!hist) return;
    #pragma unroll
    for (int r = 0; r < kRowHistPer; ++r) {
      if (hid[r] < (uint32_t)V)
        hk[r] = put(hid[r], MASK && !((hmw[r] >> (hid[r] & 31u)) & 1u) ? kNegInfBits : hraw[r]);
    }
  };

  // 5. the rest of the row, tiles 2, 3, ... (the last pass may run past
  //    it); the first pass is peeled so that the history entries' wait
  //    names exactly the loads before them
  const int npass = (ntiles + 1) / 2;
  if (npass > 1) {
    step(Slot0{}, 2, false);
    step(Slot1{}, 3, false);
    put_registers();
  }
  for (int p = 2; p < npass; ++p) {
    step(Slot0{}, 2 * p, false);
    step(Slot1{}, 2 * p + 1, false);
  }
  if (npass <= 1) put_registers();
  if (lane == 0u) {
    L.wthr[wid] = T;
    L.wbad[wid] = bad ? 1u : 0u;
    L.wcnt[wid] = wn;
  }
  if (hist) {
    for (uint32_t h = h0 + kFirst + (uint32_t)tid; h < h1; h += kRowThreads) {
      const uint32_t id = a.hids[h];
      if (id < (uint32_t)V) {
        const bool off = MASK && !((mrow[id >> 5] >> (id & 31u)) & 1u);
        put(id, off ? kNegInfBits : __float_as_uint(lrow[id]));
      }
    }
  }
  if (sp) {
    // min-p rows: this wave's list entries that are not history tokens and
    // its threads' processed history logits (first occurrences) whose key
    // reaches the bound of the largest key seen so far go to L.sbuf
    if (wid == 0 && lane < 32u) L.exptab[lane] = exp2_tab32(lane);
    if (lane == 0u) {
      atomicMax(&L.sst[kSThr], T);
      if (bad) atomicOr(&L.sst[kSBad], 1u);
    }
    uint64_t e[2 + kRowHistPer];
    const uint32_t mprev = L.sst[kSMax];  // a lower bound of the row max
    #pragma unroll
    for (int m = 0; m < 2; ++m) {
      const uint32_t i = lane + 64u * (uint32_t)m;
      e[m] = i < wn ? wl[i] : 0ull;
    }
    if (hist) {
      uint32_t mk[2];
      #pragma unroll
      for (int m = 0; m < 2; ++m) mk[m] = hw[min(cand_idx(e[m]), (uint32_t)V - 1u) >> 5].x;
      #pragma unroll
      for (int m = 0; m < 2; ++m)
        if ((mk[m] >> (cand_idx(e[m]) & 31u)) & 1u) e[m] = 0ull;
    }
    #pragma unroll
    for (int r = 0; r < kRowHistPer; ++r)
      e[2 + r] = hk[r] > kKeyNegInf ? cand_key(hk[r], hid[r]) : 0ull;
    uint32_t mx = 0u;
    #pragma unroll
    for (int m = 0; m < 2 + kRowHistPer; ++m) mx = max(mx, cand_skey(e[m]));
    mx = wave_max_u32(mx);
    if (lane == 0u && mx > mprev) atomicMax(&L.sst[kSMax], mx);
    const uint32_t mcur = (uint32_t)__builtin_amdgcn_readfirstlane((int)max(mprev, mx));
    const uint32_t kb = max(minp_key_bound(mcur, cfg.t_eff, ln_mp), kKeyNegInf + 1u);
    uint64_t bm[2 + kRowHistPer];
    uint32_t nk = 0u;
    #pragma unroll
    for (int m = 0; m < 2 + kRowHistPer; ++m) {
      bm[m] = __ballot(e[m] != 0ull && cand_skey(e[m]) >= kb);
      nk += (uint32_t)__popcll(bm[m]);
    }
    if (nk != 0u) {
      uint32_t at = 0u;
      if (lane == 0u) at = atomicAdd(&L.sst[kSCnt], nk);
      at = (uint32_t)__builtin_amdgcn_readfirstlane((int)at);
      #pragma unroll
      for (int m = 0; m < 2 + kRowHistPer; ++m) {
        const uint32_t pos = at + lanes_below(bm[m]);
        if (((bm[m] >> lane) & 1ull) && pos < (uint32_t)kRowSCap) L.sbuf[pos] = e[m];
        at += (uint32_t)__popcll(bm[m]);
      }
    }
  }
  __syncthreads();  // lists, thresholds and the history complete

  // 6. the rest runs on the first NT threads, one wave per SIMD; the other
  //    waves end here (ended waves no longer count at barriers)
  if (wid >= NT / 64) return true;
  if (sp) {
    // the min-p finish (wave 0, or the four waves for a support of more
    // than 64 entries) publishes whether it resolved the row: the four
    // waves then take the same path (the general finish below needs all of
    // them)
    const uint4 st = *reinterpret_cast<const uint4*>(L.sst);
    if (st.w == 0u && st.x > 64u && st.x <= (uint32_t)kRowSCap && st.y > kKeyNegInf && st.y < kKeyPosInf) {
      // a support of more than one wave's slot: the four waves weigh and
      // sort it (scratch: the tile buffers of waves 0-2)
      uint32_t tok = 0u;
      uint64_t* lst = reinterpret_cast<uint64_t*>(L.xscr[0]);
      uint64_t* out = reinterpret_cast<uint64_t*>(L.xscr[1]);
      uint32_t* cnt = reinterpret_cast<uint32_t*>(L.xscr[2]);
      const uint32_t miss = st.x <= 256u ? row_minp_finish4<1>(L, cfg, st.x, st.y, st.z, lst, out, cnt, tok)
                                         : row_minp_finish4<2>(L, cfg, st.x, st.y, st.z, lst, out, cnt, tok);
      if (tid == 0) {
        L.sdone = miss;
        if (miss == kMinpOk) {
          a.out_tokens[row] = tok;
          a.diag[row] = kRowPathMinp;
        }
      }
    } else if (wid == 0) {
      uint32_t tok = 0u;
      const uint32_t miss = row_minp_finish(L, cfg, tok);
      if (lane == 0u) {
        L.sdone = miss;
        if (miss == kMinpOk) {
          a.out_tokens[row] = tok;
          a.diag[row] = kRowPathMinp;
        }
      }
    }
    __syncthreads();
    minp_miss = L.sdone;
    if (minp_miss == kMinpOk) return true;
  }
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
  const bool ok = finish_core(fs, a, row, cfg, (int)n, M, Tm > kKeyNegInf ? Tm : 0u, 0.0, Tm, (uint64_t)Tm << 32, top, false);
  if (ok && tid == 0) a.diag[row] = kRowPathLists | (minp_miss << 8);
  return ok;
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
  general_row_path<MASK>(a, row, lds_raw);
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


bool row_kernel_fits(const SampleArgs& a) {
  return a.dtype == HI_ROCM_DTYPE_F32 && a.B >= kRowMinBatch && a.n_lp == 0 && a.out_token_lp == nullptr &&
         a.vec_ok && a.chunk == kSelChunkLarge && a.V <= kRowMaxV && row_lds_bytes(a.V) <= kLdsPerCu;
}

template <bool MASK>
hipError_t launch_rows_t(const SampleArgs& a, hipStream_t stream) {
  const size_t lds = row_lds_bytes(a.V);
  hipError_t e = ensure_lds((const void*)row_kernel<MASK>, lds);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(row_kernel<MASK>, dim3(a.B), dim3(kRowThreads), lds, stream, a.logits, a.row_stride, a.V, a);
  return hipGetLastError();
}

hipError_t launch_rows(const SampleArgs& a, hipStream_t stream) {
  return a.mask ? launch_rows_t<true>(a, stream) : launch_rows_t<false>(a, stream);
}

}  // namespace hi_rocm
