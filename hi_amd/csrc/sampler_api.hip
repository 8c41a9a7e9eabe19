// hi-rocm C ABI: argument checks, workspace carving and kernel launches.
//
// The mirrors of the reference launchers (crates/hi-cuda/src/kernels.cu:
// 14737-14880) keep their argument checks (status 1 for null pointers,
// non-positive sizes, negative top_k, null stream).  The reference then
// resolves ranked rows on the host (gpu.rs:15685-15967); here every row is
// finished on the device by the same kernels as hi_rocm_sample.
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <string.h>

#include <algorithm>
#include <map>
#include <mutex>
#include <string>
#include <utility>
#include <vector>

#include "hi_rocm.h"
#include "sampler_internal.h"

namespace {

thread_local std::string g_last_error;

int fail(int code, const std::string& msg) {
  g_last_error = msg;
  return code;
}

int hip_fail(hipError_t e, const char* where) {
  g_last_error = std::string(where) + ": " + hipGetErrorString(e);
  return HI_ROCM_ERR_HIP;
}

}  // namespace

namespace hi_rocm {
// The calling thread's message for hi_rocm_last_error, from other sources.
int api_fail(int code, const char* msg) { return fail(code, msg); }
int api_hip_fail(hipError_t e, const char* where) { return hip_fail(e, where); }
}  // namespace hi_rocm

namespace {

// The per-row chunk counters of a workspace start at zero (the kernels
// leave them so): a fill kernel, not a memset node, so that a call that
// sets them can be captured in a graph.
__global__ void zero_words_kernel(uint32_t* p, int n) {
  const int i = (int)(blockIdx.x * blockDim.x + threadIdx.x);
  if (i < n) p[i] = 0u;
}

hipError_t zero_counters(void* ws, int n, hipStream_t stream) {
  hipLaunchKernelGGL(zero_words_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream,
                     (uint32_t*)ws, n);
  return hipGetLastError();
}

// Library-owned workspace for the workspace-free reference mirrors: one
// buffer per (device, stream), grown on demand, never shrunk, like the
// reference's thread-local buffer pool (crates/hi-cuda/src/runtime.rs:
// 218-231); hi_rocm_sampler_release frees a stream's buffer.  Calls on one
// stream are ordered by the stream, so a buffer is never used by two
// kernels at once; calls on different streams (from any thread) use
// different buffers.  Growing waits for the buffer's own stream only, and
// is refused while the stream is being captured (like the reference's pool,
// runtime.rs:238-257, which does not allocate during capture): the caller
// reserves before capturing.
struct DeviceWorkspace {
  void* ptr = nullptr;
  size_t bytes = 0;
};
// Buffers of a (device, stream): the sampler's, and the DSV4 indexer's
// (a few KB per 4096 scores; its histogram kept at zero between calls).
enum WsKind { kWsSampler = 0, kWsIndexer = 1 };
std::mutex g_ws_mutex;
std::map<std::tuple<int, uintptr_t, int>, DeviceWorkspace> g_ws;

// The stream's buffer of `kind`, at least `bytes`, with its first
// zero_words words zero after a growth.  When it would grow during capture:
// an error, or with `optional` success and *out = nullptr (the caller takes
// a path without it).
int stream_buffer(int kind, size_t bytes, int zero_words, bool optional, hipStream_t stream, void** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
  std::lock_guard<std::mutex> lock(g_ws_mutex);
  DeviceWorkspace& ws = g_ws[std::make_tuple(dev, (uintptr_t)stream, kind)];
  if (ws.bytes < bytes) {
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    e = hipStreamIsCapturing(stream, &cs);
    if (e != hipSuccess) return hip_fail(e, "hipStreamIsCapturing");
    if (cs != hipStreamCaptureStatusNone && optional) {
      *out = nullptr;
      return HI_ROCM_OK;
    }
    if (cs != hipStreamCaptureStatusNone)
      return fail(HI_ROCM_ERR_UNSUPPORTED,
                  "hi-rocm: the stream's sampler workspace would grow to " + std::to_string(bytes) +
                      " bytes during stream capture (an allocation); call hi_rocm_sampler_reserve with the "
                      "largest shape before capturing");
    if (ws.ptr) {
      e = hipStreamSynchronize(stream);
      if (e != hipSuccess) return hip_fail(e, "hipStreamSynchronize");
      e = hipFree(ws.ptr);
      if (e != hipSuccess) return hip_fail(e, "hipFree");
      ws.ptr = nullptr;
      ws.bytes = 0;
    }
    e = hipMalloc(&ws.ptr, bytes);
    if (e != hipSuccess) return hip_fail(e, "hipMalloc(sampler workspace)");
    e = zero_counters(ws.ptr, zero_words, stream);
    if (e != hipSuccess) return hip_fail(e, "sampler workspace counter reset");
    ws.bytes = bytes;
  }
  *out = ws.ptr;
  return HI_ROCM_OK;
}

int internal_workspace(size_t bytes, hipStream_t stream, void** out) {
  return stream_buffer(kWsSampler, bytes, hi_rocm::kDoneRows, false, stream, out);
}

// Frees the calling device's workspace of `stream` after the stream's work.
int release_workspace(hipStream_t stream) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
  std::lock_guard<std::mutex> lock(g_ws_mutex);
  auto it0 = g_ws.find(std::make_tuple(dev, (uintptr_t)stream, (int)kWsSampler));
  auto it1 = g_ws.find(std::make_tuple(dev, (uintptr_t)stream, (int)kWsIndexer));
  if (it0 == g_ws.end() && it1 == g_ws.end()) return HI_ROCM_OK;
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  e = hipStreamIsCapturing(stream, &cs);
  if (e != hipSuccess) return hip_fail(e, "hipStreamIsCapturing");
  if (cs != hipStreamCaptureStatusNone)
    return fail(HI_ROCM_ERR_UNSUPPORTED, "hi_rocm_sampler_release: the stream is being captured");
  e = hipStreamSynchronize(stream);
  if (e != hipSuccess) return hip_fail(e, "hipStreamSynchronize");
  for (auto it : {it0, it1}) {
    if (it == g_ws.end()) continue;
    if (it->second.ptr) {
      e = hipFree(it->second.ptr);
      if (e != hipSuccess) return hip_fail(e, "hipFree");
    }
    g_ws.erase(it);
  }
  return HI_ROCM_OK;
}

void carve(hi_rocm::SampleArgs& a, void* ws, const hi_rocm::WorkspaceLayout& L) {
  char* base = (char*)ws;
  a.stats = (hi_rocm::ChunkStat*)(base + L.stats);
  a.cand = (uint64_t*)(base + L.cand);
  a.ws_s = (float*)(base + L.ws_s);
  a.ws_w = (float*)(base + L.ws_w);
  a.ws_list = (uint64_t*)(base + L.ws_list);
  a.list_stride = L.list_stride;
  a.done = (uint32_t*)(base + L.done);
  a.wstat = (hi_rocm::WideStat*)(base + L.wstat);
  a.wfold = (hi_rocm::ChunkFold*)(base + L.wfold);
  a.wbmap = (hi_rocm::fold::Map*)(base + L.wbmap);
  a.diag = (uint32_t*)(base + L.diag);
  a.wtot = (float*)(base + L.wtot);
  a.chunk = hi_rocm::choose_chunk(a.B, a.V, a.n_lp, a.vec_ok, a.hoff != nullptr);
  a.n_chunks = (a.V + a.chunk - 1) / a.chunk;
}

// Rows that start on 16 bytes take the streaming pass's 16-byte loads.
int vec_aligned(const void* p, int dtype, int64_t row_stride) {
  const int64_t esize = dtype == HI_ROCM_DTYPE_BF16 ? 2 : 4;
  return ((uintptr_t)p % 16 == 0) && ((row_stride * esize) % 16 == 0);
}

hi_rocm::SampleArgs base_args(const void* logits, int dtype, int B, int V, int64_t row_stride) {
  hi_rocm::SampleArgs a;
  memset(&a, 0, sizeof(a));
  a.logits = logits;
  a.dtype = dtype;
  a.B = B;
  a.V = V;
  a.row_stride = row_stride;
  a.vec_ok = vec_aligned(logits, dtype, row_stride);
  a.mask_words = (V + 31) / 32;
  return a;
}

// Run the two sampling kernels with the library workspace.
// Measurement hook state of the calling thread: one set of events per
// sampler call while a profile is open (hi_rocm_profile_begin / _end).
struct ProfileState {
  std::vector<hi_rocm::LaunchEvents> events;
  size_t used = 0;
  bool open = false;
};
thread_local ProfileState g_prof;

const hi_rocm::LaunchEvents* next_events() {
  if (!g_prof.open || g_prof.used >= g_prof.events.size()) return nullptr;
  return &g_prof.events[g_prof.used++];
}

void destroy_events() {
  for (auto& le : g_prof.events)
    for (hipEvent_t ev : le.ev) (void)hipEventDestroy(ev);
  g_prof.events.clear();
  g_prof.used = 0;
  g_prof.open = false;
}

int run_with_internal_ws(hi_rocm::SampleArgs& a, hipStream_t stream) {
  if (a.B > hi_rocm::kDoneRows) return fail(HI_ROCM_ERR_UNSUPPORTED, "batch above 65536 rows");
  const hi_rocm::WorkspaceLayout L = hi_rocm::workspace_layout(a.B, a.V);
  void* ws = nullptr;
  int rc = internal_workspace(L.total, stream, &ws);
  if (rc != HI_ROCM_OK) return rc;
  carve(a, ws, L);
  hipError_t e = hi_rocm::launch_sample(a, stream, next_events());
  if (e != hipSuccess) return hip_fail(e, "sampler launch");
  return HI_ROCM_OK;
}

bool vocab_ok(int V) { return V > 0 && V <= hi_rocm::kMaxVocab; }

}  // namespace

extern "C" {

const char* hi_rocm_last_error(void) { return g_last_error.c_str(); }

const char* hi_rocm_version(void) { return "hi-rocm 0.1.0 (gfx950)"; }

int hi_rocm_launch_argmax(const void* logits, void* output_token, int len, void* stream) {
  if (logits == nullptr || output_token == nullptr || len <= 0 || stream == nullptr)
    return fail(HI_ROCM_ERR_ARGS, "hi_rocm_launch_argmax: invalid arguments");
  hipError_t e = hi_rocm::launch_argmax((const float*)logits, (uint32_t*)output_token, 1, len, 0,
                                        len, (hipStream_t)stream);
  return e == hipSuccess ? HI_ROCM_OK : hip_fail(e, "argmax launch");
}

int hi_rocm_launch_argmax_last_row(const void* logits, void* output_token, int rows, int cols,
                                   void* stream) {
  if (logits == nullptr || output_token == nullptr || rows <= 0 || cols <= 0 || stream == nullptr)
    return fail(HI_ROCM_ERR_ARGS, "hi_rocm_launch_argmax_last_row: invalid arguments");
  hipError_t e = hi_rocm::launch_argmax((const float*)logits, (uint32_t*)output_token, 1, cols,
                                        (int64_t)(rows - 1) * cols, cols, (hipStream_t)stream);
  return e == hipSuccess ? HI_ROCM_OK : hip_fail(e, "argmax launch");
}

int hi_rocm_launch_argmax_batched_last_token(const void* logits, void* output_tokens,
                                             int batch_count, int seq_len, int cols,
                                             void* stream) {
  if (logits == nullptr || output_tokens == nullptr || batch_count <= 0 || seq_len <= 0 ||
      cols <= 0 || stream == nullptr)
    return fail(HI_ROCM_ERR_ARGS, "hi_rocm_launch_argmax_batched_last_token: invalid arguments");
  hipError_t e = hi_rocm::launch_argmax((const float*)logits, (uint32_t*)output_tokens,
                                        batch_count, (int64_t)seq_len * cols,
                                        (int64_t)(seq_len - 1) * cols, cols, (hipStream_t)stream);
  return e == hipSuccess ? HI_ROCM_OK : hip_fail(e, "argmax launch");
}

int hi_rocm_launch_sample_last_row(const void* logits, void* output_token, int rows, int cols,
                                   float temperature, float top_p, int top_k, float sample,
                                   void* stream) {
  if (logits == nullptr || output_token == nullptr || rows <= 0 || cols <= 0 || top_k < 0 ||
      stream == nullptr)
    return fail(HI_ROCM_ERR_ARGS, "hi_rocm_launch_sample_last_row: invalid arguments");
  if (!vocab_ok(cols)) return fail(HI_ROCM_ERR_UNSUPPORTED, "vocabulary too large");
  const float* row = (const float*)logits + (int64_t)(rows - 1) * cols;
  hi_rocm::SampleArgs a = base_args(row, HI_ROCM_DTYPE_F32, 1, cols, cols);
  a.pv.mode = hi_rocm::kParamsUniform;
  a.pv.T = temperature;
  a.pv.top_p = top_p;
  a.pv.top_k = top_k;
  a.pv.uniforms = nullptr;
  a.pv.uniform_value = sample;
  a.pv.greedy_rule = hi_rocm::kGreedyIeee;  // kernels.cu:7990-7993
  a.out_tokens = (uint32_t*)output_token;
  return run_with_internal_ws(a, (hipStream_t)stream);
}

int hi_rocm_launch_sample_batched_last_token(const void* logits, void* output_tokens,
                                             const void* samples, int batch_count, int seq_len,
                                             int cols, float temperature, float top_p, int top_k,
                                             int gpu_ranked, void* stream) {
  (void)gpu_ranked;
  if (logits == nullptr || output_tokens == nullptr || samples == nullptr || batch_count <= 0 ||
      seq_len <= 0 || cols <= 0 || top_k < 0 || stream == nullptr)
    return fail(HI_ROCM_ERR_ARGS, "hi_rocm_launch_sample_batched_last_token: invalid arguments");
  if (!vocab_ok(cols)) return fail(HI_ROCM_ERR_UNSUPPORTED, "vocabulary too large");
  const float* first = (const float*)logits + (int64_t)(seq_len - 1) * cols;
  hi_rocm::SampleArgs a = base_args(first, HI_ROCM_DTYPE_F32, batch_count, cols,
                                    (int64_t)seq_len * cols);
  a.pv.mode = hi_rocm::kParamsUniform;
  a.pv.T = temperature;
  a.pv.top_p = top_p;
  a.pv.top_k = top_k;
  a.pv.uniforms = (const float*)samples;
  a.pv.greedy_rule = hi_rocm::kGreedyFiniteLane;  // kernels.cu:7803-7808
  a.out_tokens = (uint32_t*)output_tokens;
  return run_with_internal_ws(a, (hipStream_t)stream);
}

}  // extern "C"

namespace {

// Argument checks and kernel arguments of the per-row mirror
// (kernels.cu:14850-14880); `what` names the entry point in messages.
int per_row_args(const void* logits, void* output_tokens, const void* samples, const void* temperatures,
                 const void* top_ps, const void* top_ks, int batch_count, int seq_len, int cols, void* stream,
                 const char* what, hi_rocm::SampleArgs& a) {
  if (logits == nullptr || output_tokens == nullptr || samples == nullptr ||
      temperatures == nullptr || top_ps == nullptr || top_ks == nullptr || batch_count <= 0 ||
      seq_len <= 0 || cols <= 0 || stream == nullptr)
    return fail(HI_ROCM_ERR_ARGS, std::string(what) + ": invalid arguments");
  if (!vocab_ok(cols)) return fail(HI_ROCM_ERR_UNSUPPORTED, "vocabulary too large");
  const float* first = (const float*)logits + (int64_t)(seq_len - 1) * cols;
  a = base_args(first, HI_ROCM_DTYPE_F32, batch_count, cols, (int64_t)seq_len * cols);
  a.pv.mode = hi_rocm::kParamsSoA;
  a.pv.temps = (const float*)temperatures;
  a.pv.top_ps = (const float*)top_ps;
  a.pv.top_ks = (const int*)top_ks;
  a.pv.uniforms = (const float*)samples;
  a.pv.greedy_rule = hi_rocm::kGreedyIeee;  // kernels.cu:8058-8061
  a.out_tokens = (uint32_t*)output_tokens;
  return HI_ROCM_OK;
}

}  // namespace

extern "C" {

int hi_rocm_launch_select_batched_last_token_per_row(const void* logits, void* output_tokens,
                                                     const void* samples,
                                                     const void* temperatures,
                                                     const void* top_ps, const void* top_ks,
                                                     int batch_count, int seq_len, int cols,
                                                     int gpu_ranked, void* stream) {
  (void)gpu_ranked;
  hi_rocm::SampleArgs a;
  const int rc = per_row_args(logits, output_tokens, samples, temperatures, top_ps, top_ks, batch_count,
                              seq_len, cols, stream, "hi_rocm_launch_select_batched_last_token_per_row", a);
  if (rc != HI_ROCM_OK) return rc;
  return run_with_internal_ws(a, (hipStream_t)stream);
}

int hi_rocm_sampler_reserve(int max_batch, int vocab, int n_logprobs, void* stream) {
  if (max_batch <= 0 || vocab <= 0 || n_logprobs < 0 || n_logprobs > HI_ROCM_MAX_LOGPROBS ||
      stream == nullptr)
    return fail(HI_ROCM_ERR_ARGS, "hi_rocm_sampler_reserve: invalid arguments");
  if (!vocab_ok(vocab)) return fail(HI_ROCM_ERR_UNSUPPORTED, "vocabulary too large");
  if (max_batch > hi_rocm::kDoneRows) return fail(HI_ROCM_ERR_UNSUPPORTED, "batch above 65536 rows");
  void* ws = nullptr;
  return internal_workspace(hi_rocm::workspace_layout(max_batch, vocab).total, (hipStream_t)stream, &ws);
}

int hi_rocm_sampler_release(void* stream) {
  if (stream == nullptr) return fail(HI_ROCM_ERR_ARGS, "hi_rocm_sampler_release: null stream");
  return release_workspace((hipStream_t)stream);
}

int hi_rocm_sampler_workspace_bytes(int max_batch, int vocab, int n_logprobs, size_t* out_bytes) {
  if (max_batch <= 0 || vocab <= 0 || n_logprobs < 0 || out_bytes == nullptr)
    return fail(HI_ROCM_ERR_ARGS, "hi_rocm_sampler_workspace_bytes: invalid arguments");
  if (n_logprobs > HI_ROCM_MAX_LOGPROBS)
    return fail(HI_ROCM_ERR_UNSUPPORTED, "n_logprobs above HI_ROCM_MAX_LOGPROBS");
  if (!vocab_ok(vocab)) return fail(HI_ROCM_ERR_UNSUPPORTED, "vocabulary too large");
  *out_bytes = hi_rocm::workspace_layout(max_batch, vocab).total;
  return HI_ROCM_OK;
}

static int check_sample_args(const void* logits, int dtype, int batch, int vocab,
                             int64_t row_stride, const void* params,
                             const uint32_t* hist_offsets, const uint32_t* hist_ids,
                             const uint32_t* hist_counts, const void* out_tokens) {
  if (logits == nullptr || params == nullptr || out_tokens == nullptr || batch <= 0 ||
      vocab <= 0 || row_stride < vocab)
    return fail(HI_ROCM_ERR_ARGS, "hi_rocm: invalid logits/params/outputs/sizes");
  if (batch > hi_rocm::kDoneRows) return fail(HI_ROCM_ERR_UNSUPPORTED, "batch above 65536 rows");
  if (dtype != HI_ROCM_DTYPE_F32 && dtype != HI_ROCM_DTYPE_BF16)
    return fail(HI_ROCM_ERR_ARGS, "hi_rocm: unknown dtype");
  if ((hist_offsets == nullptr) != (hist_ids == nullptr) ||
      (hist_offsets == nullptr) != (hist_counts == nullptr))
    return fail(HI_ROCM_ERR_ARGS, "hi_rocm: history needs offsets, ids and counts together");
  if (!vocab_ok(vocab)) return fail(HI_ROCM_ERR_UNSUPPORTED, "vocabulary too large");
  return HI_ROCM_OK;
}

int hi_rocm_sample(const void* logits, int dtype, int batch, int vocab, int64_t row_stride,
                   const hi_rocm_row_params* params, const float* uniforms,
                   const uint32_t* hist_offsets, const uint32_t* hist_ids,
                   const uint32_t* hist_counts, const uint32_t* mask_words,
                   uint32_t* out_tokens, float* out_logprobs, uint32_t* out_logprob_ids,
                   float* out_token_logprobs, int n_logprobs, void* workspace,
                   size_t workspace_bytes, void* stream) {
  int rc = check_sample_args(logits, dtype, batch, vocab, row_stride, params, hist_offsets,
                             hist_ids, hist_counts, out_tokens);
  if (rc != HI_ROCM_OK) return rc;
  if (uniforms == nullptr) return fail(HI_ROCM_ERR_ARGS, "hi_rocm_sample: null uniforms");
  if (n_logprobs < 0) return fail(HI_ROCM_ERR_ARGS, "hi_rocm_sample: negative n_logprobs");
  if (n_logprobs > HI_ROCM_MAX_LOGPROBS)
    return fail(HI_ROCM_ERR_UNSUPPORTED, "n_logprobs above HI_ROCM_MAX_LOGPROBS");
  if (n_logprobs > 0 && (out_logprobs == nullptr || out_logprob_ids == nullptr))
    return fail(HI_ROCM_ERR_ARGS, "hi_rocm_sample: logprob outputs missing");
  const hi_rocm::WorkspaceLayout L = hi_rocm::workspace_layout(batch, vocab);
  if (workspace == nullptr || workspace_bytes < L.total)
    return fail(HI_ROCM_ERR_ARGS, "hi_rocm_sample: workspace too small");
  hi_rocm::SampleArgs a = base_args(logits, dtype, batch, vocab, row_stride);
  a.pv.mode = hi_rocm::kParamsRows;
  a.pv.rows = params;
  a.pv.uniforms = uniforms;
  a.pv.greedy_rule = hi_rocm::kGreedyIeee;
  a.hoff = hist_offsets;
  a.hids = hist_ids;
  a.hcnt = hist_counts;
  a.mask = mask_words;
  a.n_lp = n_logprobs;
  a.need_lse = (n_logprobs > 0 || out_token_logprobs != nullptr) ? 1 : 0;
  a.out_tokens = out_tokens;
  a.out_lp = out_logprobs;
  a.out_lp_ids = out_logprob_ids;
  a.out_token_lp = out_token_logprobs;
  carve(a, workspace, L);
  hipError_t e = hi_rocm::launch_sample(a, (hipStream_t)stream, next_events());
  if (e != hipSuccess) return hip_fail(e, "sampler launch");
  return HI_ROCM_OK;
}

int hi_rocm_profile_begin(int max_calls) {
  if (max_calls <= 0) return fail(HI_ROCM_ERR_ARGS, "hi_rocm_profile_begin: max_calls <= 0");
  destroy_events();
  g_prof.events.resize((size_t)max_calls);
  for (auto& le : g_prof.events) {
    for (hipEvent_t& ev : le.ev) {
      hipError_t e = hipEventCreate(&ev);
      if (e != hipSuccess) {
        ev = nullptr;
        destroy_events();
        return hip_fail(e, "hipEventCreate");
      }
    }
  }
  g_prof.open = true;
  return HI_ROCM_OK;
}

int hi_rocm_profile_end(double* pass_ms, double* finish_ms, int* calls) {
  if (pass_ms == nullptr || finish_ms == nullptr || calls == nullptr)
    return fail(HI_ROCM_ERR_ARGS, "hi_rocm_profile_end: null output");
  if (!g_prof.open) return fail(HI_ROCM_ERR_ARGS, "hi_rocm_profile_end: no open profile");
  double p = 0.0, f = 0.0;
  for (size_t i = 0; i < g_prof.used; ++i) {
    const hi_rocm::LaunchEvents& le = g_prof.events[i];
    hipError_t e = hipEventSynchronize(le.ev[2]);
    float a = 0.f, b = 0.f;
    if (e == hipSuccess) e = hipEventElapsedTime(&a, le.ev[0], le.ev[1]);
    if (e == hipSuccess) e = hipEventElapsedTime(&b, le.ev[1], le.ev[2]);
    if (e != hipSuccess) {
      destroy_events();
      return hip_fail(e, "profile events");
    }
    p += a;
    f += b;
  }
  *pass_ms = p;
  *finish_ms = f;
  *calls = (int)g_prof.used;
  destroy_events();
  return HI_ROCM_OK;
}

int hi_rocm_debug_distribution(const void* logits, int dtype, int batch, int vocab,
                               int64_t row_stride, const hi_rocm_row_params* params,
                               const uint32_t* hist_offsets, const uint32_t* hist_ids,
                               const uint32_t* hist_counts, const uint32_t* mask_words,
                               float* out_processed, float* out_probs, void* stream) {
  int rc = check_sample_args(logits, dtype, batch, vocab, row_stride, params, hist_offsets,
                             hist_ids, hist_counts, out_processed);
  if (rc != HI_ROCM_OK) return rc;
  if (out_probs == nullptr) return fail(HI_ROCM_ERR_ARGS, "hi_rocm_debug_distribution: null output");
  hi_rocm::SampleArgs a = base_args(logits, dtype, batch, vocab, row_stride);
  a.pv.mode = hi_rocm::kParamsRows;
  a.pv.rows = params;
  a.hoff = hist_offsets;
  a.hids = hist_ids;
  a.hcnt = hist_counts;
  a.mask = mask_words;
  const hi_rocm::WorkspaceLayout L = hi_rocm::workspace_layout(batch, vocab);
  void* ws = nullptr;
  rc = internal_workspace(L.total, (hipStream_t)stream, &ws);
  if (rc != HI_ROCM_OK) return rc;
  carve(a, ws, L);
  hipError_t e = hi_rocm::launch_debug_distribution(a, out_processed, out_probs, (hipStream_t)stream);
  return e == hipSuccess ? HI_ROCM_OK : hip_fail(e, "debug distribution launch");
}

int hi_rocm_debug_fold(const float* terms, const uint32_t* counts, int runs, float start,
                      float* out_start, float* out_final, void* stream) {
  if (terms == nullptr || counts == nullptr || out_start == nullptr || out_final == nullptr || runs <= 0 ||
      runs > hi_rocm::kDebugFoldMaxRuns || stream == nullptr)
    return fail(HI_ROCM_ERR_ARGS, "hi_rocm_debug_fold: invalid arguments");
  hipError_t e = hi_rocm::launch_debug_fold(terms, counts, runs, start, out_start, out_final, (hipStream_t)stream);
  return e == hipSuccess ? HI_ROCM_OK : hip_fail(e, "debug fold launch");
}

int hi_rocm_debug_wide_paths(const void* workspace, size_t workspace_bytes, int batch, int vocab,
                             uint32_t* out_paths, void* stream) {
  if (workspace == nullptr || out_paths == nullptr || batch <= 0 || vocab <= 0 || batch > hi_rocm::kDoneRows ||
      !vocab_ok(vocab))
    return fail(HI_ROCM_ERR_ARGS, "hi_rocm_debug_wide_paths: invalid arguments");
  const hi_rocm::WorkspaceLayout L = hi_rocm::workspace_layout(batch, vocab);
  if (workspace_bytes < L.total) return fail(HI_ROCM_ERR_ARGS, "hi_rocm_debug_wide_paths: workspace too small");
  hipError_t e = hipMemcpyAsync(out_paths, (const char*)workspace + L.diag, (size_t)batch * 4,
                                hipMemcpyDeviceToHost, (hipStream_t)stream);
  if (e == hipSuccess) e = hipStreamSynchronize((hipStream_t)stream);
  return e == hipSuccess ? HI_ROCM_OK : hip_fail(e, "debug wide paths copy");
}

int hi_rocm_debug_wide_totals(const void* workspace, size_t workspace_bytes, int batch, int vocab,
                              float* out_totals, void* stream) {
  if (workspace == nullptr || out_totals == nullptr || batch <= 0 || vocab <= 0 || batch > hi_rocm::kDoneRows ||
      !vocab_ok(vocab))
    return fail(HI_ROCM_ERR_ARGS, "hi_rocm_debug_wide_totals: invalid arguments");
  const hi_rocm::WorkspaceLayout L = hi_rocm::workspace_layout(batch, vocab);
  if (workspace_bytes < L.total) return fail(HI_ROCM_ERR_ARGS, "hi_rocm_debug_wide_totals: workspace too small");
  hipError_t e = hipMemcpyAsync(out_totals, (const char*)workspace + L.wtot, (size_t)batch * 2 * sizeof(float),
                                hipMemcpyDeviceToHost, (hipStream_t)stream);
  if (e == hipSuccess) e = hipStreamSynchronize((hipStream_t)stream);
  return e == hipSuccess ? HI_ROCM_OK : hip_fail(e, "debug wide totals copy");
}

int hi_rocm_debug_expf(const float* x, float* y, int64_t n, void* stream) {
  if (x == nullptr || y == nullptr || n <= 0)
    return fail(HI_ROCM_ERR_ARGS, "hi_rocm_debug_expf: invalid arguments");
  hipError_t e = hi_rocm::launch_debug_expf(x, y, n, (hipStream_t)stream);
  return e == hipSuccess ? HI_ROCM_OK : hip_fail(e, "debug expf launch");
}

int hi_rocm_launch_dsv4_indexer_select(const void* scores, int n_blocks, int top_k, void* marks,
                                       void* sel_out, void* stream) {
  if (scores == nullptr || marks == nullptr || sel_out == nullptr || n_blocks <= 0 || top_k <= 0 ||
      stream == nullptr)
    return fail(HI_ROCM_ERR_ARGS, "hi_rocm_launch_dsv4_indexer_select: invalid arguments");
  // the kernels' span and loop arithmetic is in int: keep it clear of overflow
  if (n_blocks > INT32_MAX - (1 << 20))
    return fail(HI_ROCM_ERR_UNSUPPORTED, "hi_rocm_launch_dsv4_indexer_select: n_blocks above 2^31 - 2^20");
  // above kMultiMinN scores: a workgroup per 4096 of them, with a small
  // per-stream buffer (one workgroup when that buffer would have to be
  // allocated during stream capture)
  const size_t wsb = hi_rocm::index_select_ws_bytes(n_blocks);
  void* ws = nullptr;
  if (wsb > 0) {
    const int rc = stream_buffer(kWsIndexer, wsb, (int)(hi_rocm::kIndexHistBytes / 4), true, (hipStream_t)stream, &ws);
    if (rc != HI_ROCM_OK) return rc;
  }
  hipError_t e = ws ? hi_rocm::launch_index_select_multi((const float*)scores, n_blocks, top_k, (uint8_t*)marks,
                                                         (int32_t*)sel_out, ws, (hipStream_t)stream)
                    : hi_rocm::launch_index_select((const float*)scores, n_blocks, top_k, (uint8_t*)marks,
                                                   (int32_t*)sel_out, (hipStream_t)stream);
  return e == hipSuccess ? HI_ROCM_OK : hip_fail(e, "indexer select launch");
}

}  // extern "C"

// ---- LM-head projection + bias + softcap fused into the first pass -------

namespace {

int lm_args(const void* hidden, const void* weight, const float* bias, float softcap, int batch, int hidden_dim,
            int vocab, const char* what, hi_rocm::LmArgs& a) {
  if (hidden == nullptr || weight == nullptr || batch <= 0 || hidden_dim <= 0 || vocab <= 0)
    return fail(HI_ROCM_ERR_ARGS, std::string(what) + ": invalid arguments");
  if (batch > hi_rocm::kLmRows || hidden_dim % 32 != 0 || (uintptr_t)hidden % 16 != 0 || (uintptr_t)weight % 16 != 0)
    return fail(HI_ROCM_ERR_UNSUPPORTED,
                std::string(what) + ": needs batch <= 64, hidden_dim a multiple of 32, 16-byte aligned bf16 arrays");
  const int tiles = (vocab + hi_rocm::kLmTile - 1) / hi_rocm::kLmTile;
  if (tiles > hi_rocm::kLmMaxTiles)
    return fail(HI_ROCM_ERR_UNSUPPORTED, std::string(what) + ": vocabulary above 524,288");
  memset(&a, 0, sizeof(a));
  a.hidden = (const __bf16*)hidden;
  a.weight = (const __bf16*)weight;
  a.bias = bias;
  a.cap = softcap;
  a.B = batch;
  a.H = hidden_dim;
  a.V = vocab;
  a.n_chunks = tiles;
  return HI_ROCM_OK;
}

}  // namespace

extern "C" {

int hi_rocm_lm_head_workspace_bytes(int batch, int vocab, size_t* out_bytes) {
  if (batch <= 0 || vocab <= 0 || out_bytes == nullptr)
    return fail(HI_ROCM_ERR_ARGS, "hi_rocm_lm_head_workspace_bytes: invalid arguments");
  // the shapes hi_rocm_sample_lm_head accepts (lm_args)
  if (batch > hi_rocm::kLmRows)
    return fail(HI_ROCM_ERR_UNSUPPORTED, "hi_rocm_lm_head_workspace_bytes: batch above 64");
  if ((vocab + hi_rocm::kLmTile - 1) / hi_rocm::kLmTile > hi_rocm::kLmMaxTiles)
    return fail(HI_ROCM_ERR_UNSUPPORTED, "hi_rocm_lm_head_workspace_bytes: vocabulary above 524,288");
  *out_bytes = hi_rocm::lm_workspace_bytes(batch, vocab);
  return HI_ROCM_OK;
}

int hi_rocm_lm_head_logits(const void* hidden, const void* weight, const float* bias, float softcap, int batch,
                           int hidden_dim, int vocab, float* out_logits, void* stream) {
  hi_rocm::LmArgs a;
  int rc = lm_args(hidden, weight, bias, softcap, batch, hidden_dim, vocab, "hi_rocm_lm_head_logits", a);
  if (rc != HI_ROCM_OK) return rc;
  if (out_logits == nullptr || stream == nullptr)
    return fail(HI_ROCM_ERR_ARGS, "hi_rocm_lm_head_logits: invalid arguments");
  a.out_logits = out_logits;
  const hipError_t e = hi_rocm::launch_lm_logits(a, (hipStream_t)stream);
  return e == hipSuccess ? HI_ROCM_OK : hip_fail(e, "lm head launch");
}

int hi_rocm_sample_lm_head_ext(const void* hidden, const void* weight, const float* bias, float softcap, int batch,
                               int hidden_dim, int vocab, const hi_rocm_row_params* params, const float* uniforms,
                               const uint32_t* hist_offsets, const uint32_t* hist_ids, const uint32_t* hist_counts,
                               const uint32_t* mask_words, uint32_t* out_tokens, float* out_logprobs,
                               uint32_t* out_logprob_ids, float* out_token_logprobs, int n_logprobs, void* workspace,
                               size_t workspace_bytes, void* stream) {
  static const char* kWhat = "hi_rocm_sample_lm_head";
  hi_rocm::LmArgs a;
  int rc = lm_args(hidden, weight, bias, softcap, batch, hidden_dim, vocab, kWhat, a);
  if (rc != HI_ROCM_OK) return rc;
  if (params == nullptr || uniforms == nullptr || out_tokens == nullptr || stream == nullptr)
    return fail(HI_ROCM_ERR_ARGS, std::string(kWhat) + ": invalid arguments");
  if (hist_offsets != nullptr && (hist_ids == nullptr || hist_counts == nullptr))
    return fail(HI_ROCM_ERR_ARGS, std::string(kWhat) + ": history ids or counts missing");
  if (n_logprobs < 0 || (n_logprobs > 0 && (out_logprobs == nullptr || out_logprob_ids == nullptr)))
    return fail(HI_ROCM_ERR_ARGS, std::string(kWhat) + ": logprob outputs missing");
  if (n_logprobs > hi_rocm::kLeanK)
    return fail(HI_ROCM_ERR_UNSUPPORTED, std::string(kWhat) + ": n_logprobs above 256");
  const size_t need = hi_rocm::lm_workspace_bytes(batch, vocab);
  if (workspace == nullptr || workspace_bytes < need)
    return fail(HI_ROCM_ERR_ARGS, std::string(kWhat) + ": workspace too small");
  a.pv.mode = hi_rocm::kParamsRows;
  a.pv.rows = params;
  a.pv.uniforms = uniforms;
  a.pv.greedy_rule = hi_rocm::kGreedyIeee;
  const size_t recs = hi_rocm::lm_recs_bytes(batch, a.n_chunks);
  a.lm_recs = (hi_rocm::LmTileRec*)workspace;
  a.lm_logits = (float*)((char*)workspace + recs);
  a.out_tokens = out_tokens;
  // the general per-row path over the workspace's logits, for the rows the
  // fused finish leaves; its penalties, mask and logprobs are the call's
  a.gen = base_args(a.lm_logits, HI_ROCM_DTYPE_F32, batch, vocab, hi_rocm::lm_stride(vocab));
  a.gen.pv = a.pv;
  a.gen.hoff = hist_offsets;
  a.gen.hids = hist_ids;
  a.gen.hcnt = hist_counts;
  a.gen.mask = mask_words;
  a.gen.n_lp = n_logprobs;
  a.gen.need_lse = (n_logprobs > 0 || out_token_logprobs != nullptr) ? 1 : 0;
  a.gen.out_tokens = out_tokens;
  a.gen.out_lp = out_logprobs;
  a.gen.out_lp_ids = out_logprob_ids;
  a.gen.out_token_lp = out_token_logprobs;
  carve(a.gen, (char*)workspace + recs + hi_rocm::lm_logits_bytes(batch, vocab),
        hi_rocm::general_layout(batch, vocab));
  const hipError_t e = hi_rocm::launch_lm_sample(a, (hipStream_t)stream);
  return e == hipSuccess ? HI_ROCM_OK : hip_fail(e, "lm head sample launch");
}

int hi_rocm_sample_lm_head(const void* hidden, const void* weight, const float* bias, float softcap, int batch,
                           int hidden_dim, int vocab, const hi_rocm_row_params* params, const float* uniforms,
                           uint32_t* out_tokens, void* workspace, size_t workspace_bytes, void* stream) {
  return hi_rocm_sample_lm_head_ext(hidden, weight, bias, softcap, batch, hidden_dim, vocab, params, uniforms,
                                    nullptr, nullptr, nullptr, nullptr, out_tokens, nullptr, nullptr, nullptr, 0,
                                    workspace, workspace_bytes, stream);
}

}  // extern "C"

// ---- the per-row mirror without allocation ------------------------------
//
// For callers that cannot call hipMalloc (code under stream capture, tight
// serving loops): the workspace is a file-scope device array of fixed size,
// one copy per GPU, held by every GPU the library runs on until the process
// ends.  Every call on a GPU uses that GPU's copy, so calls that overlap on
// one GPU (two streams, two threads) race; callers serialise them.
namespace {

constexpr size_t kNoAllocScratchBytes = HI_ROCM_NOALLOC_SCRATCH_BYTES;  // per GPU

static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

std::mutex g_scratch_mutex;
std::map<int, void*> g_scratch_ptr;  // device -> address of its `scratch`

// The device address of the current device's `scratch`, looked up once per
// device (the array's name in host code is not that address).
int scratch_address(void** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  auto it = g_scratch_ptr.find(dev);
  if (it == g_scratch_ptr.end()) {
    void* ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return hip_fail(e, "hipGetSymbolAddress(scratch)");
    if (ptr == nullptr) return fail(HI_ROCM_ERR_HIP, "hipGetSymbolAddress(scratch): null address");
    it = g_scratch_ptr.emplace(dev, ptr).first;
  }
  *out = it->second;
  return HI_ROCM_OK;
}

}  // namespace

extern "C" {

int hi_rocm_launch_select_batched_last_token_per_row_noalloc(
    const void* logits, void* output_tokens, const void* samples, const void* temperatures, const void* top_ps,
    const void* top_ks, int batch_count, int seq_len, int cols, int gpu_ranked, void* stream) {
  (void)gpu_ranked;
  static const char* kWhat = "hi_rocm_launch_select_batched_last_token_per_row_noalloc";
  hi_rocm::SampleArgs a;
  int rc = per_row_args(logits, output_tokens, samples, temperatures, top_ps, top_ks, batch_count, seq_len,
                        cols, stream, kWhat, a);
  if (rc != HI_ROCM_OK) return rc;
  if (batch_count > hi_rocm::kDoneRows) return fail(HI_ROCM_ERR_UNSUPPORTED, "batch above 65536 rows");
  // Rows are independent, so a batch whose workspace exceeds the array runs
  // in groups of as many rows as fit (15 at vocabulary 151,936), one after
  // another on the stream, each group reusing the array; only a vocabulary
  // of which one row does not fit is rejected.
  const size_t one = hi_rocm::workspace_layout(1, cols).total;
  if (one > kNoAllocScratchBytes)
    return fail(HI_ROCM_ERR_UNSUPPORTED,
                std::string(kWhat) + ": one row of vocab " + std::to_string(cols) + " needs " +
                    std::to_string(one) + " bytes of workspace, above the " +
                    std::to_string(kNoAllocScratchBytes) + "-byte static scratch");
  int lo = 1, hi = batch_count;  // the largest group that fits
  while (lo < hi) {
    const int mid = lo + (hi - lo + 1) / 2;
    if (hi_rocm::workspace_layout(mid, cols).total <= kNoAllocScratchBytes) lo = mid;
    else hi = mid - 1;
  }
  const int group = lo;
  void* ptr = nullptr;
  rc = scratch_address(&ptr);
  if (rc != HI_ROCM_OK) return rc;
  for (int r0 = 0; r0 < batch_count; r0 += group) {
    const int n = std::min(group, batch_count - r0);
    hi_rocm::SampleArgs g;
    rc = per_row_args((const float*)logits + (int64_t)r0 * seq_len * cols, (uint32_t*)output_tokens + r0,
                      (const float*)samples + r0, (const float*)temperatures + r0, (const float*)top_ps + r0,
                      (const int*)top_ks + r0, n, seq_len, cols, stream, kWhat, g);
    if (rc != HI_ROCM_OK) return rc;
    carve(g, ptr, hi_rocm::workspace_layout(n, cols));
    // the per-row counters start at zero (the array keeps whatever the
    // last call or group left)
    hipError_t e = zero_counters(g.done, n, (hipStream_t)stream);
    if (e != hipSuccess) return hip_fail(e, "scratch counter reset");
    e = hi_rocm::launch_sample(g, (hipStream_t)stream, next_events());
    if (e != hipSuccess) return hip_fail(e, "sampler launch");
  }
  return HI_ROCM_OK;
}

}  // extern "C"
