/*
 * hi-rocm host layer bridges (C ABI over the C++ mirror of the reference's
 * Rust sampler API, hi_amd/csrc/sampler_host.hip).
 *
 * The reference's per-step sampler API is Rust (crates/hi-cuda/src/gpu.rs:
 * 15542-15967); these functions take the same arguments as those Rust
 * functions, with host arrays in place of slices and Option<u32> top_k as an
 * int64 (< 0 = None).  Logits are device memory; parameters and outputs are
 * host memory; each call synchronises `stream` like the Rust functions'
 * blocking copy_to_host.  Return 0 on success, 1 on error with the Rust
 * function's error message copied to `err`.
 */
#ifndef HI_ROCM_HOST_H
#define HI_ROCM_HOST_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* gpu.rs:15810 select_batched_last_token_per_row: n_rows row configs
 * (kinds[r]: 0 = Greedy, 1 = Sampled) and n_samples uniforms; out_tokens
 * receives batch_count tokens. */
int hi_rocm_host_select_batched_last_token_per_row(
    const float* logits, size_t rows, size_t cols, size_t batch_count, size_t seq_len,
    size_t n_rows, const int32_t* kinds, const float* temperatures, const float* top_ps,
    const int64_t* top_ks, const float* samples, size_t n_samples, uint32_t* out_tokens,
    char* err, size_t err_len, void* stream);

/* gpu.rs:15685 sample_batched_last_token. */
int hi_rocm_host_sample_batched_last_token(const float* logits, size_t rows, size_t cols,
                                           size_t batch_count, size_t seq_len, float temperature,
                                           float top_p, int64_t top_k, const float* samples,
                                           size_t n_samples, uint32_t* out_tokens, char* err,
                                           size_t err_len, void* stream);

/* gpu.rs:15658 argmax_batched_last_token. */
int hi_rocm_host_argmax_batched_last_token(const float* logits, size_t rows, size_t cols,
                                           size_t batch_count, size_t seq_len,
                                           uint32_t* out_tokens, char* err, size_t err_len,
                                           void* stream);

/* gpu.rs:15606 sample_last_row_with_sample. */
int hi_rocm_host_sample_last_row_with_sample(const float* logits, size_t rows, size_t cols,
                                             float temperature, float top_p, int64_t top_k,
                                             float sample, uint32_t* out_token, char* err,
                                             size_t err_len, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* HI_ROCM_HOST_H */
