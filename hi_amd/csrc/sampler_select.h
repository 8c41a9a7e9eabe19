// The streaming select pass and the general scan: device code shared by the
// select kernels (sampler_select.hip), the chunked path's kernels
// (sampler_chunked.hip) and the row kernel's general path (sampler_rows.hip).
#pragma once
#include "sampler_common.h"

namespace hi_rocm {

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
  uint32_t whist[kWideBins * kWideCopies];  // top-p rows: the chunk's mass histogram (WideStat),
                                            // copy c of bin j at j * kWideCopies + c
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
// histogram: w' = exp((v - m) / T) = 2^r, bin j = floor(-r), clamped.
// The bins hold integers, w' * 2^(j + 16) (in [2^15, 2^16] inside a bin;
// the clamped last bin drops what lies below 2^-47), because LDS float
// atomics are slow on this part: with ds_add_f32 C2's select pass took
// 41-44 us (with 8 or 64 copies of the bins alike), with ds_add_u32 20 us,
// the same as with no histogram.  Thread t adds to copy t % kWideCopies.
// A copy takes the terms of NT / kWideCopies threads, at most 64 + kSelOb a
// thread, each at most 2^16: below 2^28.  The masses are approximate (the
// wide pass keeps a margin), so the order of the additions does not
// matter.
__device__ __forceinline__ void wide_hist_add(uint32_t* whist, float v, float m, float a2) {
  if (!finitef_(v)) return;
  const float r = (v - m) * a2;
  const int j = -r < (float)(kWideBins - 1) ? (int)(-r) : kWideBins - 1;
  const uint32_t fx = (uint32_t)__builtin_amdgcn_exp2f(r + (float)(j + 16));
  atomicAdd(&whist[j * kWideCopies + (int)(threadIdx.x & (kWideCopies - 1))], fx);
}
__device__ __forceinline__ void wide_hist_clear(uint32_t* whist) {
  for (int i = threadIdx.x; i < kWideBins * kWideCopies; i += NT) whist[i] = 0u;
}
// The bins' masses (relative to the chunk maximum) summed over their
// copies into out[0 .. kWideBins), by all NT threads: thread t adds copies
// 8 (t & 7) .. + 7 of bin t / 8 (two 16-byte reads), then the eight
// threads of a bin add up (DPP).
__device__ __forceinline__ void wide_hist_store(const uint32_t* whist, float* out) {
  static_assert(kWideBins * 8 == NT && kWideCopies % 8 == 0, "eight threads a bin");
  constexpr int kPer = kWideCopies / 8;
  const int t = threadIdx.x;
  const uint32_t* p = whist + (t >> 3) * kWideCopies + (t & 7) * kPer;
  uint32_t u = 0u;
  #pragma unroll
  for (int c = 0; c < kPer; ++c) u += p[c];
  float s = (float)u * __builtin_ldexpf(1.f, -(t >> 3) - 16);
  #pragma unroll
  for (int o = 1; o < 8; o <<= 1) s += __uint_as_float(lane_xor32(__float_as_uint(s), o));
  if ((t & 7) == 0) out[t >> 3] = s;
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
    wide_hist_store(L.whist, ws->hist);
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
  // (every wave's atomics are in: the barrier above)
  if (nd.whist) wide_hist_store(L.whist, a.wstat[slot].hist);
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


}  // namespace hi_rocm
