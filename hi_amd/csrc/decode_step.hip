// hi-rocm decode-step upkeep on the device: the per-request token history
// that the penalties read, and the per-request uniforms of the draw.
//
// The reference keeps both on the host: each request's generated tokens in
// a Vec (crates/hi-cuda/src/lib.rs:4342, pushed at :5550 and friends; the
// penalties count occurrences over prompt + generated tokens,
// crates/hi-mlx/src/generate.rs:52-73), and one uniform per request per step
// from the request's StdRng (lib.rs:6415-6429, seeded at :4865 with
// StdRng::seed_from_u64).  Here both live in device memory and are updated
// by kernels on the decode stream, so a captured decode step needs no host
// round trip.
//
// History: request slot r owns `capacity` entries (ids, counts) at r *
// capacity in insertion order, and lens[r] of them are in use.  An append
// kernel adds (slot, token) pairs; a pack kernel writes the compact CSR
// (offsets [B+1], ids, counts) that hi_rocm_sample reads.
//
// Uniforms: StdRng in rand 0.8.7 (Cargo.lock:5495) is ChaCha12 (rand_chacha
// 0.3.1) with a 64-bit block counter and stream 0; seed_from_u64 expands the
// seed with PCG32 (rand_core 0.6.4).  Draw k of a request is keystream word k (block k / 16,
// word k % 16), and gen_range(0.0f32..1.0f32) maps a word w to
// f32((w >> 9) | 0x3f800000) - 1.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "hi_rocm.h"
#include "sampler_internal.h"

namespace hi_rocm {
namespace {

constexpr int kAppendWaves = 4;  // request slots per workgroup (one wave each)

__device__ __forceinline__ uint32_t load_agent(const uint32_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void store_agent(uint32_t* p, uint32_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// One wave per request slot: the slot's pairs in call order.  The search
// for a token is wave-parallel (64 entries per step); lane 0 writes.
// Entries are read at agent scope and every write is followed by an agent
// fence, so the wave's later searches see its own earlier appends.
__global__ void __launch_bounds__(64 * kAppendWaves)
    history_append_kernel(uint32_t* slot_ids, uint32_t* slot_counts, uint32_t* lens, int batch, int cap,
                          const int32_t* rows, const uint32_t* tokens, int n, uint32_t* overflow) {
  const int lane = threadIdx.x & 63;
  const int slot = (int)blockIdx.x * kAppendWaves + (int)(threadIdx.x >> 6);
  if (slot >= batch) return;
  uint32_t* ids = slot_ids + (int64_t)slot * cap;
  uint32_t* cnt = slot_counts + (int64_t)slot * cap;
  uint32_t len = min(lens[slot], (uint32_t)cap);
  uint32_t lost = 0u;
  // without `rows`, pair j is slot j's
  const int j0 = rows ? 0 : slot, j1 = rows ? n : min(slot + 1, n);
  for (int j = j0; j < j1; ++j) {
    if (rows && rows[j] != slot) continue;
    const uint32_t t = tokens[j];
    if (t == HI_ROCM_HISTORY_RESET) {
      len = 0u;
      continue;
    }
    int found = -1;
    for (uint32_t b = 0; b < len; b += 64u) {
      const uint32_t i = b + (uint32_t)lane;
      const uint64_t m = __ballot(i < len && load_agent(ids + i) == t);
      if (m != 0ull) {
        found = (int)b + __ffsll((unsigned long long)m) - 1;
        break;
      }
    }
    if (found >= 0) {
      if (lane == 0) store_agent(cnt + found, load_agent(cnt + found) + 1u);
    } else if (len < (uint32_t)cap) {
      if (lane == 0) {
        store_agent(ids + len, t);
        store_agent(cnt + len, 1u);
      }
      ++len;
    } else {
      ++lost;
    }
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "agent");
  }
  if (lane == 0) {
    lens[slot] = len;
    if (lost != 0u && overflow) atomicAdd(overflow, lost);
  }
}

// Exclusive scan of lens into offsets[0 .. batch] (one workgroup).
constexpr int kScanT = 1024;
__global__ void __launch_bounds__(kScanT)
    history_offsets_kernel(const uint32_t* lens, int batch, int cap, uint32_t* offsets) {
  __shared__ uint32_t wsum[kScanT / 64];
  __shared__ uint32_t carry;
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  if (tid == 0) carry = 0u;
  __syncthreads();
  for (int base = 0; base < batch; base += kScanT) {
    const int r = base + tid;
    const uint32_t v = r < batch ? min(lens[r], (uint32_t)cap) : 0u;
    uint32_t inc = v;
    #pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      const uint32_t o = (uint32_t)__shfl_up((int)inc, (unsigned)d, 64);
      if (lane >= d) inc += o;
    }
    if (lane == 63) wsum[wid] = inc;
    __syncthreads();
    uint32_t before = carry;
    for (int w = 0; w < wid; ++w) before += wsum[w];
    if (r < batch) offsets[r] = before + inc - v;
    __syncthreads();
    if (tid == kScanT - 1) carry = before + inc;
    __syncthreads();
  }
  if (tid == 0) offsets[batch] = carry;
}

// Copy each slot's entries to its CSR range (one workgroup per slot).
__global__ void __launch_bounds__(256)
    history_pack_kernel(const uint32_t* slot_ids, const uint32_t* slot_counts, const uint32_t* lens, int cap,
                        const uint32_t* offsets, uint32_t* out_ids, uint32_t* out_counts) {
  const int slot = blockIdx.x;
  const uint32_t len = min(lens[slot], (uint32_t)cap), o = offsets[slot];
  const uint32_t* ids = slot_ids + (int64_t)slot * cap;
  const uint32_t* cnt = slot_counts + (int64_t)slot * cap;
  for (uint32_t i = threadIdx.x; i < len; i += 256u) {
    out_ids[o + i] = ids[i];
    out_counts[o + i] = cnt[i];
  }
}

// ---- ChaCha (RFC 8439 block function; rand_chacha's ChaCha12 uses 12
//      rounds, words 12-13 a 64-bit block counter, words 14-15 the stream) ----

__host__ __device__ __forceinline__ uint32_t rotl32(uint32_t x, int n) { return (x << n) | (x >> (32 - n)); }

__host__ __device__ __forceinline__ void chacha_qr(uint32_t* s, int a, int b, int c, int d) {
  s[a] += s[b]; s[d] = rotl32(s[d] ^ s[a], 16);
  s[c] += s[d]; s[b] = rotl32(s[b] ^ s[c], 12);
  s[a] += s[b]; s[d] = rotl32(s[d] ^ s[a], 8);
  s[c] += s[d]; s[b] = rotl32(s[b] ^ s[c], 7);
}

// One block: the state (constants, key, w12 .. w15) after `rounds` rounds,
// plus the input state.
__host__ __device__ __forceinline__ void chacha_block(const uint32_t* key, uint32_t w12, uint32_t w13, uint32_t w14,
                                                     uint32_t w15, int rounds, uint32_t* out) {
  uint32_t in[16] = {0x61707865u, 0x3320646eu, 0x79622d32u, 0x6b206574u, key[0], key[1], key[2], key[3],
                     key[4],      key[5],      key[6],      key[7],      w12,    w13,    w14,    w15};
  uint32_t s[16];
  for (int i = 0; i < 16; ++i) s[i] = in[i];
  for (int r = 0; r < rounds; r += 2) {
    chacha_qr(s, 0, 4, 8, 12);
    chacha_qr(s, 1, 5, 9, 13);
    chacha_qr(s, 2, 6, 10, 14);
    chacha_qr(s, 3, 7, 11, 15);
    chacha_qr(s, 0, 5, 10, 15);
    chacha_qr(s, 1, 6, 11, 12);
    chacha_qr(s, 2, 7, 8, 13);
    chacha_qr(s, 3, 4, 9, 14);
  }
  for (int i = 0; i < 16; ++i) out[i] = s[i] + in[i];
}

// One thread per request: the next gen_range(0.0f32..1.0f32) of its StdRng,
// or 0 for a request without one (lib.rs:6415-6429: greedy requests).
__global__ void __launch_bounds__(256)
    rng_uniforms_kernel(const uint32_t* keys, uint64_t* words_used, const uint8_t* sampled, float* out, int batch) {
  const int b = (int)(blockIdx.x * blockDim.x + threadIdx.x);
  if (b >= batch) return;
  if (sampled && sampled[b] == 0) {
    out[b] = 0.0f;
    return;
  }
  const uint64_t k = words_used[b];
  const uint64_t blk = k >> 4;
  uint32_t key[8], w[16];
  for (int i = 0; i < 8; ++i) key[i] = keys[(int64_t)b * 8 + i];
  chacha_block(key, (uint32_t)blk, (uint32_t)(blk >> 32), 0u, 0u, 12, w);
  uint32_t x = w[0];
  for (int i = 1; i < 16; ++i)
    if ((uint32_t)(k & 15u) == (uint32_t)i) x = w[i];
  out[b] = __uint_as_float((x >> 9) | 0x3f800000u) - 1.0f;
  words_used[b] = k + 1u;
}

// The next step's graph inputs from this step's samples
// (upload_batch_graph_inputs, gpu.rs:10200-10245, on the device): rows
// below n_active decode their sampled token at the next position; pad rows
// decode token 0 at position 0.
__global__ void __launch_bounds__(256)
    step_advance_kernel(const uint32_t* sampled, uint32_t* tokens, uint32_t* positions, int n_active, int bucket) {
  const int r = (int)(blockIdx.x * blockDim.x + threadIdx.x);
  if (r >= bucket) return;
  const bool live = r < n_active;
  tokens[r] = live ? sampled[r] : 0u;
  positions[r] = live ? positions[r] + 1u : 0u;
}

}  // namespace
}  // namespace hi_rocm

extern "C" {

int hi_rocm_history_append(uint32_t* slot_ids, uint32_t* slot_counts, uint32_t* lens, int batch, int capacity,
                           const int32_t* rows, const uint32_t* tokens, int n, uint32_t* overflow, void* stream) {
  if (slot_ids == nullptr || slot_counts == nullptr || lens == nullptr || tokens == nullptr || batch <= 0 ||
      capacity <= 0 || n < 0 || stream == nullptr || (rows == nullptr && n > batch))
    return hi_rocm::api_fail(HI_ROCM_ERR_ARGS, "hi_rocm_history_append: invalid arguments");
  if (n == 0) return HI_ROCM_OK;
  const int blocks = (batch + hi_rocm::kAppendWaves - 1) / hi_rocm::kAppendWaves;
  hipLaunchKernelGGL(hi_rocm::history_append_kernel, dim3(blocks), dim3(64 * hi_rocm::kAppendWaves), 0,
                     (hipStream_t)stream, slot_ids, slot_counts, lens, batch, capacity, rows, tokens, n, overflow);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? HI_ROCM_OK : hi_rocm::api_hip_fail(e, "history append launch");
}

int hi_rocm_history_pack(const uint32_t* slot_ids, const uint32_t* slot_counts, const uint32_t* lens, int batch,
                         int capacity, uint32_t* out_offsets, uint32_t* out_ids, uint32_t* out_counts, void* stream) {
  if (slot_ids == nullptr || slot_counts == nullptr || lens == nullptr || out_offsets == nullptr ||
      out_ids == nullptr || out_counts == nullptr || batch <= 0 || capacity <= 0 || stream == nullptr)
    return hi_rocm::api_fail(HI_ROCM_ERR_ARGS, "hi_rocm_history_pack: invalid arguments");
  if ((int64_t)batch * capacity > (int64_t)UINT32_MAX)
    return hi_rocm::api_fail(HI_ROCM_ERR_UNSUPPORTED, "hi_rocm_history_pack: batch x capacity above 2^32");
  hipLaunchKernelGGL(hi_rocm::history_offsets_kernel, dim3(1), dim3(hi_rocm::kScanT), 0, (hipStream_t)stream, lens,
                     batch, capacity, out_offsets);
  hipLaunchKernelGGL(hi_rocm::history_pack_kernel, dim3(batch), dim3(256), 0, (hipStream_t)stream, slot_ids,
                     slot_counts, lens, capacity, out_offsets, out_ids, out_counts);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? HI_ROCM_OK : hi_rocm::api_hip_fail(e, "history pack launch");
}

int hi_rocm_rng_key_from_seed(uint64_t seed, uint32_t* key) {
  if (key == nullptr) return hi_rocm::api_fail(HI_ROCM_ERR_ARGS, "hi_rocm_rng_key_from_seed: null key");
  // rand_core 0.6 SeedableRng::seed_from_u64: PCG32 (advance, then XSH-RR
  // of the new state), one little-endian u32 per key word
  const uint64_t kMul = 6364136223846793005ull, kInc = 11634580027462260723ull;
  uint64_t state = seed;
  for (int i = 0; i < 8; ++i) {
    state = state * kMul + kInc;
    const uint32_t xorshifted = (uint32_t)(((state >> 18) ^ state) >> 27);
    const uint32_t rot = (uint32_t)(state >> 59);
    key[i] = (xorshifted >> rot) | (xorshifted << ((32u - rot) & 31u));
  }
  return HI_ROCM_OK;
}

int hi_rocm_rng_uniforms(const uint32_t* keys, uint64_t* words_used, const uint8_t* sampled, float* out_uniforms,
                         int batch, void* stream) {
  if (keys == nullptr || words_used == nullptr || out_uniforms == nullptr || batch <= 0 || stream == nullptr)
    return hi_rocm::api_fail(HI_ROCM_ERR_ARGS, "hi_rocm_rng_uniforms: invalid arguments");
  hipLaunchKernelGGL(hi_rocm::rng_uniforms_kernel, dim3((batch + 255) / 256), dim3(256), 0, (hipStream_t)stream, keys,
                     words_used, sampled, out_uniforms, batch);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? HI_ROCM_OK : hi_rocm::api_hip_fail(e, "rng uniforms launch");
}

int hi_rocm_decode_step_advance(const uint32_t* sampled, uint32_t* tokens, uint32_t* positions, int n_active,
                                int bucket, void* stream) {
  if (sampled == nullptr || tokens == nullptr || positions == nullptr || bucket <= 0 || n_active < 0 ||
      n_active > bucket || stream == nullptr)
    return hi_rocm::api_fail(HI_ROCM_ERR_ARGS, "hi_rocm_decode_step_advance: invalid arguments");
  hipLaunchKernelGGL(hi_rocm::step_advance_kernel, dim3((bucket + 255) / 256), dim3(256), 0, (hipStream_t)stream,
                     sampled, tokens, positions, n_active, bucket);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? HI_ROCM_OK : hi_rocm::api_hip_fail(e, "decode step advance launch");
}

int hi_rocm_debug_chacha_block(const uint32_t* key, const uint32_t* words12_15, int rounds, uint32_t* out) {
  if (key == nullptr || words12_15 == nullptr || out == nullptr || rounds <= 0 || (rounds & 1))
    return hi_rocm::api_fail(HI_ROCM_ERR_ARGS, "hi_rocm_debug_chacha_block: invalid arguments");
  hi_rocm::chacha_block(key, words12_15[0], words12_15[1], words12_15[2], words12_15[3], rounds, out);
  return HI_ROCM_OK;
}

}  // extern "C"
