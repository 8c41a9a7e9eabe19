/*
 * hi-rocm: MI355X (gfx950) batched token sampler, C ABI.
 *
 * Drop-in for the sampler launchers of the reference's hi-cuda crate
 * (crates/hi-cuda/src/kernels.cu:14737-14880, bound in Rust at
 * crates/hi-cuda/src/kernels.rs:1507-1563), plus one extended entry point that
 * adds the stages the serving path needs (penalties, allowed-token mask,
 * min-p, logprobs, bf16 logits).
 *
 * Conventions shared by every entry point:
 *   - every pointer argument is caller-owned device memory (HBM) unless the
 *     comment says otherwise; logits are never copied to the host;
 *   - work is enqueued on `stream` (a hipStream_t) and is asynchronous;
 *   - return 0 = launched, 1 = rejected arguments (nothing enqueued),
 *     2 = unsupported shape or option, 3 = HIP launch/runtime error;
 *     hi_rocm_last_error() gives a message for the calling thread;
 *   - no entry point throws or aborts across the ABI;
 *   - every row is resolved on the device: unlike the reference there is no
 *     0xFFFFFFFF overflow sentinel and no host re-sampling.
 */
#ifndef HI_ROCM_H
#define HI_ROCM_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define HI_ROCM_OK 0
#define HI_ROCM_ERR_ARGS 1
#define HI_ROCM_ERR_UNSUPPORTED 2
#define HI_ROCM_ERR_HIP 3

#define HI_ROCM_DTYPE_F32 0
#define HI_ROCM_DTYPE_BF16 1

/* Repetition penalty once per distinct history token instead of once per
 * occurrence. */
#define HI_ROCM_FLAG_REP_ONCE 1u

/* Largest n_logprobs accepted by hi_rocm_sample. */
#define HI_ROCM_MAX_LOGPROBS 1024

/*
 * Per-row sampling parameters (40 bytes, device array of `batch` entries).
 * Meaning of the reference fields follows CudaRowSampling
 * (crates/hi-cuda/src/gpu.rs:55-65) and its device form
 * (gpu.rs:15861-15884): temperature <= 0 or non-finite is greedy; top_k <= 0
 * is "unset"; top_p >= 1 or non-finite disables the nucleus cut.
 * The other fields are extensions the reference's CUDA path lacks:
 *   min_p               keep tokens with p >= min_p * p_max (<= 0: off)
 *   repetition_penalty  l < 0 ? l * p : l / p per history occurrence
 *                       (crates/hi-mlx/src/generate.rs:60-70); off when
 *                       |p - 1| <= FLT_EPSILON, p <= 0 or non-finite
 *   frequency_penalty   l -= f * count   (count > 0)
 *   presence_penalty    l -= presence    (count > 0)
 *   eos_id              output of a row whose mask allows no finite logit
 *   flags               HI_ROCM_FLAG_*
 */
typedef struct hi_rocm_row_params {
  float temperature;
  float top_p;
  float min_p;
  float repetition_penalty;
  float frequency_penalty;
  float presence_penalty;
  int32_t top_k;
  uint32_t eos_id;
  uint32_t flags;
  uint32_t reserved;
} hi_rocm_row_params;

/* ---- drop-in mirrors of the reference launchers (same arguments, same
 *      argument checks; `stream` must be non-null like the reference) ---- */

/* kernels.cu:14737 hi_cuda_launch_argmax: argmax of `len` f32 logits,
 * IEEE '>' with ties to the lowest index (kernels.cu:7153-7186). */
int hi_rocm_launch_argmax(const void* logits, void* output_token, int len, void* stream);

/* kernels.cu:14753 hi_cuda_launch_argmax_last_row: argmax of row rows-1. */
int hi_rocm_launch_argmax_last_row(const void* logits, void* output_token, int rows, int cols,
                                   void* stream);

/* kernels.cu:14771 hi_cuda_launch_argmax_batched_last_token: argmax of row
 * b*seq_len + seq_len-1 for every b. */
int hi_rocm_launch_argmax_batched_last_token(const void* logits, void* output_tokens,
                                             int batch_count, int seq_len, int cols,
                                             void* stream);

/* kernels.cu:14794 hi_cuda_launch_sample_last_row (+ the host ranking of
 * gpu.rs:15561-15656): one token from row rows-1 with the given config and
 * uniform `sample`.  Ranked configs follow gpu.rs:753-900 exactly. */
int hi_rocm_launch_sample_last_row(const void* logits, void* output_token, int rows, int cols,
                                   float temperature, float top_p, int top_k, float sample,
                                   void* stream);

/* kernels.cu:14819 hi_cuda_launch_sample_batched_last_token (+ gpu.rs:15685-
 * 15767): one config for all rows, samples[b] the uniform of row b.
 * `gpu_ranked` is accepted for ABI compatibility and ignored: ranked rows
 * are always resolved on the device, bit-exact with the host sampler. */
int hi_rocm_launch_sample_batched_last_token(const void* logits, void* output_tokens,
                                             const void* samples, int batch_count, int seq_len,
                                             int cols, float temperature, float top_p, int top_k,
                                             int gpu_ranked, void* stream);

/* kernels.cu:14850 hi_cuda_launch_select_batched_last_token_per_row (+ the
 * host pass of gpu.rs:15810-15967): per-row temperatures (f32[B]), top_ps
 * (f32[B]), top_ks (i32[B], 0 = unset) and samples (f32[B]). */
int hi_rocm_launch_select_batched_last_token_per_row(const void* logits, void* output_tokens,
                                                     const void* samples,
                                                     const void* temperatures,
                                                     const void* top_ps, const void* top_ks,
                                                     int batch_count, int seq_len, int cols,
                                                     int gpu_ranked, void* stream);

/* kernels.cu:8482 hi_cuda_launch_moe_topk_router (kernel kernels.cu:536-684):
 * scores f32[rows][experts], output_ids u32[rows][top_k], output_weights
 * f32[rows][top_k], selection_bias f32[experts] or null (sigmoid gating
 * ranks on score + bias, weights stay bias-free).  Same checks (status 1)
 * and semantics; one wave per row; experts <= 2048 (status 2 above).  The
 * exponential is glibc's expf, as everywhere in this library, where the
 * reference calls CUDA's expf. */
int hi_rocm_launch_moe_topk_router(const void* scores, void* output_ids, void* output_weights,
                                   const void* selection_bias, int rows, int experts, int top_k,
                                   int norm_topk, int gating_sigmoid, float weights_scale, void* stream);

/* LM-head projection + bias + final softcap fused into the sampler's first
 * pass (gpu.rs:20999-21009 output_logits_f32_device: project, add the bias,
 * apply_final_logit_softcap gpu.rs:23232-23249; then the sampler).
 *   hidden  bf16[batch][hidden_dim], weight bf16[vocab][hidden_dim] (both
 *           16-byte aligned), bias f32[vocab] or null, softcap > 0 applies
 *           cap * tanh(x / cap) (tanh defined in hi_amd/csrc/softcap.h; the
 *           reference uses CUDA's tanhf), batch <= 64, hidden_dim % 32 == 0,
 *           vocab <= 524288 (status 2 otherwise).
 * hi_rocm_lm_head_logits writes the logits f32[batch][vocab] (the unfused
 * twin).  hi_rocm_sample_lm_head samples from the same logits (bit for bit)
 * and returns a token for every row: per-row params as hi_rocm_sample (any
 * class; penalties, mask and logprobs through hi_rocm_sample_lm_head_ext)
 * and one uniform per row.  Greedy
 * rows and top-k <= 64 rows (with temperature / top-p / min-p) finish from
 * per-tile records and the few tiles that can hold the top k; rows of other
 * classes, and the rare top-k row whose cut falls between distinct logits of
 * equal weight, take the general per-row path over the row's logits in the
 * workspace.  Workspace (device, hi_rocm_lm_head_workspace_bytes): per-tile
 * records, the logits of every row that is not greedy, and the general
 * path's per-row buffers. */
int hi_rocm_lm_head_workspace_bytes(int batch, int vocab, size_t* out_bytes);
int hi_rocm_lm_head_logits(const void* hidden, const void* weight, const float* bias, float softcap, int batch,
                           int hidden_dim, int vocab, float* out_logits, void* stream);
int hi_rocm_sample_lm_head(const void* hidden, const void* weight, const float* bias, float softcap, int batch,
                           int hidden_dim, int vocab, const hi_rocm_row_params* params, const float* uniforms,
                           uint32_t* out_tokens, void* workspace, size_t workspace_bytes, void* stream);
/* hi_rocm_sample_lm_head with hi_rocm_sample's history (penalties), mask and
 * logprob arguments (same meaning; n_logprobs <= 256).  Rows with a mask,
 * logprobs or a penalty that changes a logit take the general per-row path;
 * the others as hi_rocm_sample_lm_head.  Same workspace. */
int hi_rocm_sample_lm_head_ext(const void* hidden, const void* weight, const float* bias, float softcap, int batch,
                               int hidden_dim, int vocab, const hi_rocm_row_params* params, const float* uniforms,
                               const uint32_t* hist_offsets, const uint32_t* hist_ids, const uint32_t* hist_counts,
                               const uint32_t* mask_words, uint32_t* out_tokens, float* out_logprobs,
                               uint32_t* out_logprob_ids, float* out_token_logprobs, int n_logprobs, void* workspace,
                               size_t workspace_bytes, void* stream);

/* Greedy speculative-decoding verification (gpu.rs:10725-10762
 * speculative_greedy_next_tokens_paged_with_page_table, batched): logits
 * f32[batch][max_draft + 1][vocab] (row i of a request predicts the token
 * after its i-th verify input), draft_tokens u32[batch][max_draft],
 * draft_len i32[batch] (null: every request drafted max_draft tokens).
 * Writes out_greedy u32[batch][max_draft + 1] (each row's argmax by the
 * host rule of gpu.rs:6406-6435: first maximum by '>', a NaN at index 0
 * keeps index 0), and per request the accepted prefix: out_tokens
 * u32[batch][max_draft + 1] receives greedy[0 ..= accepted] and out_count
 * i32[batch] its length.  Device arrays; no allocation. */
int hi_rocm_spec_verify_greedy(const void* logits, int batch, int max_draft, int vocab, const void* draft_tokens,
                               const void* draft_len, void* out_greedy, void* out_tokens, void* out_count,
                               void* stream);

/* ---- decode-step upkeep on the device (the reference keeps these on the
 *      host: generated tokens in a Vec, crates/hi-cuda/src/lib.rs:4342, and
 *      one StdRng draw per request per step, lib.rs:6415-6429) ---- */

/* Per-request token history for the penalties (occurrence counts over the
 * prompt and the generated tokens, crates/hi-mlx/src/generate.rs:52-73).
 * Request slot r owns `capacity` entries of slot_ids / slot_counts (device
 * u32[batch][capacity]) in first-occurrence order; lens[r] (device u32[batch])
 * of them are in use.  Appends the pairs (rows[j], tokens[j]), j < n, in order
 * (rows null: pair j is slot j, n <= batch); rows[j] outside [0, batch) are
 * skipped; HI_ROCM_HISTORY_RESET as a token empties the slot (a new request).
 * A new id that finds its slot full is dropped and counted in *overflow
 * (device u32, may be null).  No allocation: graph-capturable. */
#define HI_ROCM_HISTORY_RESET 0xffffffffu
int hi_rocm_history_append(uint32_t* slot_ids, uint32_t* slot_counts, uint32_t* lens, int batch, int capacity,
                           const int32_t* rows, const uint32_t* tokens, int n, uint32_t* overflow, void* stream);

/* The compact CSR that hi_rocm_sample reads (hist_offsets u32[batch + 1],
 * hist_ids / hist_counts u32[batch * capacity] at most), from the slots. */
int hi_rocm_history_pack(const uint32_t* slot_ids, const uint32_t* slot_counts, const uint32_t* lens, int batch,
                         int capacity, uint32_t* out_offsets, uint32_t* out_ids, uint32_t* out_counts, void* stream);

/* Host: the ChaCha12 key of rand 0.8's StdRng::seed_from_u64(seed)
 * (rand_core 0.6's PCG32 expansion; key: u32[8]).  lib.rs:4865 seeds each
 * sampled request this way. */
int hi_rocm_rng_key_from_seed(uint64_t seed, uint32_t* key);

/* One uniform per request (lib.rs:6415-6429 continuous_sampling_values):
 * request b with sampled[b] != 0 (sampled null: every request) draws
 * gen_range(0.0f32..1.0f32) from its StdRng -- keystream word
 * words_used[b] of ChaCha12 under keys[b] (u32[batch][8]) -- and advances
 * words_used[b] (device u64[batch]); the others get 0.  Device arrays;
 * graph-capturable. */
int hi_rocm_rng_uniforms(const uint32_t* keys, uint64_t* words_used, const uint8_t* sampled, float* out_uniforms,
                         int batch, void* stream);

/* The next decode step's token and position inputs from this step's
 * samples, on the device (upload_batch_graph_inputs, gpu.rs:10200-10245,
 * copies them from the host every step): for r < n_active, tokens[r] =
 * sampled[r] and positions[r] += 1; pad rows n_active <= r < bucket get
 * token 0 at position 0.  Device u32 arrays of `bucket` entries (sampled
 * may be hi_rocm_sample's out_tokens); graph-capturable, no allocation. */
int hi_rocm_decode_step_advance(const uint32_t* sampled, uint32_t* tokens, uint32_t* positions, int n_active,
                                int bucket, void* stream);

/* Host: one ChaCha block (RFC 8439 block function) of `rounds` rounds with
 * state words 12-15 given; for the known-answer tests. */
int hi_rocm_debug_chacha_block(const uint32_t* key, const uint32_t* words12_15, int rounds, uint32_t* out);

/* hi_rocm_launch_select_batched_last_token_per_row without any allocation.
 * No counterpart in the reference: it is for callers that cannot allocate
 * (code under stream capture, serving loops that forbid hipMalloc).  Same
 * arguments, checks and results as the mirror above; its workspace is a
 * static device array of HI_ROCM_NOALLOC_SCRATCH_BYTES per GPU (held by
 * every GPU the library runs on until the process ends).  A batch whose
 * workspace (hi_rocm_sampler_workspace_bytes) exceeds it runs in groups of
 * as many rows as fit (15 at vocabulary 151,936), one launch sequence a
 * group; a vocabulary of which one row does not fit is rejected with
 * HI_ROCM_ERR_UNSUPPORTED.
 * Every call on a GPU shares that GPU's array: calls that overlap on one
 * GPU (several streams or threads) race and must be serialised. */
#define HI_ROCM_NOALLOC_SCRATCH_BYTES ((size_t)64 << 20)
int hi_rocm_launch_select_batched_last_token_per_row_noalloc(const void* logits, void* output_tokens,
                                                             const void* samples,
                                                             const void* temperatures,
                                                             const void* top_ps, const void* top_ks,
                                                             int batch_count, int seq_len, int cols,
                                                             int gpu_ranked, void* stream);

/* The mirrors above take no workspace, like the reference.  They use a
 * workspace per (device, stream) that the library grows on demand
 * (hipMalloc; growing waits for that stream), so calls on different
 * streams, from any threads, never share one.  Growing is refused while the
 * stream is being captured (status 2, nothing enqueued).  Call this once per
 * stream, before any stream capture, with the largest shape to be sampled
 * on it so that no allocation happens afterwards.  No reference counterpart (the
 * reference pre-warms its buffer pool instead,
 * crates/hi-cuda/src/runtime.rs:240-262). */
int hi_rocm_sampler_reserve(int max_batch, int vocab, int n_logprobs, void* stream);

/* Frees the calling device's workspace of `stream` (after waiting for the
 * stream's work): for a stream that will make no more sampler calls, or
 * whose buffer should shrink.  A later call on the stream allocates again.
 * Status 2 while the stream is being captured.  No reference counterpart
 * (the reference's buffer pool is thread-local and freed with its thread,
 * crates/hi-cuda/src/runtime.rs:218-231). */
int hi_rocm_sampler_release(void* stream);

/* ---- extended pipeline (the decode-step API: per-row parameters, history,
 *      mask, logprobs and bf16 in one call; no single reference
 *      counterpart) ---- */

/* Workspace bytes hi_rocm_sample needs for up to max_batch rows of `vocab`. */
int hi_rocm_sampler_workspace_bytes(int max_batch, int vocab, int n_logprobs,
                                    size_t* out_bytes);

/*
 * Sample one token per row.
 *   logits       [batch][row_stride] elements of `dtype` (f32 or bf16)
 *   params       hi_rocm_row_params[batch]
 *   uniforms     f32[batch], one U[0,1) draw per row (clamped like gpu.rs:882-886)
 *   hist_offsets u32[batch+1] CSR offsets into hist_ids/hist_counts, or NULL
 *   hist_ids     u32 token ids (ids >= vocab are ignored)
 *   hist_counts  u32 occurrence counts (repeated ids add up)
 *   mask_words   u32[batch][ceil(vocab/32)] allowed-token bitmask (bit i%32 of
 *                word i/32, 1 = allowed), or NULL for no mask
 *   out_tokens   u32[batch]
 *   out_logprobs, out_logprob_ids  f32/u32[batch][n_logprobs] (NULL if 0):
 *                the first n_logprobs tokens in rank order (weight desc,
 *                index asc) with log-softmax of the processed distribution
 *   out_token_logprobs f32[batch] log-prob of the sampled token, or NULL
 *   workspace    >= hi_rocm_sampler_workspace_bytes(batch, vocab, n_logprobs);
 *                zero-filled before its first use (it holds per-row counters
 *                that every call leaves at zero); one stream at a time per
 *                workspace
 * No allocation and no host synchronisation: safe to capture in a hipGraph.
 */
int hi_rocm_sample(const void* logits, int dtype, int batch, int vocab, int64_t row_stride,
                   const hi_rocm_row_params* params, const float* uniforms,
                   const uint32_t* hist_offsets, const uint32_t* hist_ids,
                   const uint32_t* hist_counts, const uint32_t* mask_words,
                   uint32_t* out_tokens, float* out_logprobs, uint32_t* out_logprob_ids,
                   float* out_token_logprobs, int n_logprobs, void* workspace,
                   size_t workspace_bytes, void* stream);

/*
 * Debug export for the 1e-5 numerics check: the processed logits
 * (mask + penalties, before temperature) and the full-vocabulary
 * probabilities softmax(l / T) (T = 1 for greedy rows), f32[batch][vocab]
 * each.  Same inputs as hi_rocm_sample.  No reference counterpart.
 */
int hi_rocm_debug_distribution(const void* logits, int dtype, int batch, int vocab,
                               int64_t row_stride, const hi_rocm_row_params* params,
                               const uint32_t* hist_offsets, const uint32_t* hist_ids,
                               const uint32_t* hist_counts, const uint32_t* mask_words,
                               float* out_processed, float* out_probs, void* stream);

/* kernels.cu:2696 hi_cuda_launch_dsv4_indexer_select (Rust wrapper
 * kernels.rs:3455 launch_dsv4_indexer_select): the exact top-k block
 * selection of the DSV4 sparse-attention indexer.  scores: f32[n_blocks];
 * keeps take = min(top_k, n_blocks) blocks ranked by total_cmp descending,
 * the lower index first on equal scores (dsv4_cpu.rs:3258-3270);
 * sel_out: int32[take], the kept indices in ascending order; marks:
 * uint8[n_blocks], 1 for a kept block and 0 otherwise.  Status 1 for null
 * pointers, n_blocks <= 0, top_k <= 0 or a null stream, as the reference. */
int hi_rocm_launch_dsv4_indexer_select(const void* scores, int n_blocks, int top_k, void* marks,
                                       void* sel_out, void* stream);

/* Debug export: the workgroup form of the sequential f32 fold that every
 * sum of the sampler's draw uses (the reference's folds at gpu.rs:834-838,
 * :851, :878, :889-896), on its own.  runs (1 .. 65536) runs of equal terms:
 * terms[r] (f32 >= 0) repeated counts[r] >= 1 times, folded left to right
 * from start; out_start[r] = the value before run r, *out_final = the value
 * after the last run (device arrays).  No reference counterpart. */
int hi_rocm_debug_fold(const float* terms, const uint32_t* counts, int runs, float start,
                       float* out_start, float* out_final, void* stream);

/* Debug export: how the last hi_rocm_sample call on this workspace
 * finished each row (u32[batch] to host memory; blocking).  Top-p rows
 * without a top-k bound on the chunked path: 1 = the chunk-parallel wide
 * pass, 2-7 = a named fallback to the general finish.  Rows of the row
 * kernel (batches of 192+ rows without logprobs): 8 = the min-p support
 * finish, 9 = the candidate lists' finish (bits 8-15: why a min-p row missed
 * the min-p finish: 1 its support array, 2 its top k not known, 3 the
 * draw), 10 = the general path.  0 = none of these.  The batch and vocab must be the call's; any stream, the null
 * one included.  No reference counterpart. */
int hi_rocm_debug_wide_paths(const void* workspace, size_t workspace_bytes, int batch, int vocab,
                             uint32_t* out_paths, void* stream);

/* Debug export: for the last call on `workspace`, the wide pass's two f32
 * sums of each top-p row it finished (rows whose hi_rocm_debug_wide_paths
 * code is 1): the normaliser (the vocabulary-order sum of the weights) and
 * the candidate total, as float[batch][2] to host memory (blocking).
 * Entries of other rows are left from earlier calls.  The batch and vocab
 * must be the call's; any stream.  No reference counterpart: the sums are
 * gpu.rs:837's `total` and :874's `candidate_total`, which the parity tests
 * compare with the oracle's bit for bit. */
int hi_rocm_debug_wide_totals(const void* workspace, size_t workspace_bytes, int batch, int vocab,
                              float* out_totals, void* stream);

/* Debug export: y[i] = the device weight function exp(x[i]) for n floats
 * (device arrays).  Bit-identical to host glibc expf.  No reference
 * counterpart; the reference's closest check is crates/hi-cuda/src/
 * dsv4_gpu.rs:7332 for its own device expf. */
int hi_rocm_debug_expf(const float* x, float* y, int64_t n, void* stream);

/* Measurement hooks (no counterpart in the reference; for benchmarks).
 * hi_rocm_profile_begin opens a profile on the calling thread: each of its
 * next max_calls sampler calls records three hipEvents on its own stream,
 * before its first kernel, between the pass over the logits and the finish,
 * and after the finish.  hi_rocm_profile_end waits for them, returns the
 * summed durations of the two parts (ms) and the number of calls recorded,
 * and closes the profile.  Not for use under stream capture. */
int hi_rocm_profile_begin(int max_calls);
int hi_rocm_profile_end(double* pass_ms, double* finish_ms, int* calls);

/* Thread-local message for the last non-zero status. */
const char* hi_rocm_last_error(void);

/* Library version string. */
const char* hi_rocm_version(void);

#ifdef __cplusplus
}
#endif

#endif /* HI_ROCM_H */
