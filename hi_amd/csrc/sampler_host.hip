// Host-side mirror of the reference's per-decode-step sampler API
// (crates/hi-cuda/src/gpu.rs:15542-15967), written in C++ over the hi-rocm C
// ABI because no Rust toolchain is available to build the original crate.
// Same routing, same argument checks and the same error messages as the
// Rust functions; what differs is that ranked rows never leave the device
// (the reference copies each ranked row to the host and re-samples it there).
//
// The extern "C" bridges at the bottom let tests drive this layer with host
// parameter arrays, the way the Rust callers pass slices.
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <string.h>

#include <map>
#include <optional>
#include <stdexcept>
#include <string>
#include <vector>

#include "hi_rocm.h"

namespace hi_rocm {

// gpu.rs:55-65 CudaRowSampling.
struct RowSampling {
  bool greedy;
  float temperature;
  float top_p;
  std::optional<uint32_t> top_k;
};

// The logits tensor the reference passes (GpuF32Tensor: rows x cols f32 in
// device memory, gpu.rs:25964-25968).
struct DeviceLogits {
  const float* data;
  size_t rows;
  size_t cols;
};

class SamplerError : public std::runtime_error {
 public:
  using std::runtime_error::runtime_error;
};

namespace {

void hip_check(hipError_t e, const char* what) {
  if (e != hipSuccess) throw SamplerError(std::string(what) + ": " + hipGetErrorString(e));
}

void status_check(int rc, const char* what) {
  if (rc != HI_ROCM_OK) throw SamplerError(std::string(what) + ": " + hi_rocm_last_error());
}

// Device staging for the per-call arrays (tokens, samples, row parameters):
// one buffer per (thread, device), grown on demand and kept, in the manner
// of the reference's thread-local buffer pool (runtime.rs:218-231).  Every
// Sampler call ends by synchronising its stream, so a thread's buffer is
// idle between calls and growing it needs no further wait.  The buffers
// are not freed at thread exit (the HIP runtime may be gone by then).
struct DeviceBuffer {
  void* ptr;
};

struct Staging {
  void* ptr = nullptr;
  size_t bytes = 0;
};
thread_local std::map<int, Staging> t_staging;

constexpr size_t kSlot = 256;  // slot alignment

size_t slot_bytes(size_t bytes) { return (bytes + kSlot - 1) & ~(kSlot - 1); }

// `count` slots of `bytes` each in this thread's staging buffer.
std::vector<DeviceBuffer> staging(size_t count, size_t bytes, const char* what) {
  int dev = 0;
  hip_check(hipGetDevice(&dev), what);
  Staging& st = t_staging[dev];
  const size_t per = slot_bytes(bytes > 0 ? bytes : 1), need = per * count;
  if (st.bytes < need) {
    if (st.ptr) hip_check(hipFree(st.ptr), what);
    st.ptr = nullptr;
    st.bytes = 0;
    hip_check(hipMalloc(&st.ptr, need), what);
    st.bytes = need;
  }
  std::vector<DeviceBuffer> v;
  for (size_t i = 0; i < count; ++i) v.push_back({(char*)st.ptr + i * per});
  return v;
}

template <typename T>
void upload(const DeviceBuffer& b, const std::vector<T>& v, hipStream_t s, const char* what) {
  hip_check(hipMemcpyAsync(b.ptr, v.data(), v.size() * sizeof(T), hipMemcpyHostToDevice, s), what);
}

std::vector<uint32_t> download(const DeviceBuffer& b, size_t n, hipStream_t s) {
  std::vector<uint32_t> out(n);
  hip_check(hipMemcpyAsync(out.data(), b.ptr, n * sizeof(uint32_t), hipMemcpyDeviceToHost, s),
            "copying tokens to host");
  hip_check(hipStreamSynchronize(s), "synchronizing sampler stream");
  return out;
}

}  // namespace

class Sampler {
 public:
  explicit Sampler(hipStream_t stream) : stream_(stream) {}

  // gpu.rs:15542-15559
  uint32_t argmax_last_row(const DeviceLogits& logits) {
    const DeviceBuffer token = staging(1, sizeof(uint32_t), "allocating CUDA argmax token")[0];
    status_check(hi_rocm_launch_argmax_last_row(logits.data, token.ptr, (int)logits.rows,
                                                (int)logits.cols, stream_),
                 "argmax launch");
    auto v = download(token, 1, stream_);
    return v[0];
  }

  // gpu.rs:15606-15656 (the ranked branch runs on the device here)
  uint32_t sample_last_row_with_sample(const DeviceLogits& logits, float temperature, float top_p,
                                       std::optional<uint32_t> top_k, float sample) {
    if (logits.rows == 0 || logits.cols == 0)
      throw SamplerError("CUDA sampled token selection requires non-empty logits, got " +
                         std::to_string(logits.rows) + "x" + std::to_string(logits.cols));
    const DeviceBuffer token = staging(1, sizeof(uint32_t), "allocating CUDA sampled token")[0];
    status_check(hi_rocm_launch_sample_last_row(logits.data, token.ptr, (int)logits.rows,
                                                (int)logits.cols, temperature, top_p,
                                                top_k_i32(top_k), sample, stream_),
                 "sample launch");
    auto v = download(token, 1, stream_);
    return v[0];
  }

  // gpu.rs:15658-15683
  std::vector<uint32_t> argmax_batched_last_token(const DeviceLogits& logits, size_t batch_count,
                                                  size_t seq_len) {
    if (logits.rows != batch_count * seq_len)
      throw SamplerError("CUDA batched argmax logits rows " + std::to_string(logits.rows) +
                         " do not match batch " + std::to_string(batch_count) + " x seq " +
                         std::to_string(seq_len));
    const DeviceBuffer tokens =
        staging(1, batch_count * sizeof(uint32_t), "allocating CUDA batched argmax tokens")[0];
    status_check(hi_rocm_launch_argmax_batched_last_token(logits.data, tokens.ptr,
                                                          (int)batch_count, (int)seq_len,
                                                          (int)logits.cols, stream_),
                 "argmax launch");
    return download(tokens, batch_count, stream_);
  }

  // gpu.rs:15685-15767
  std::vector<uint32_t> sample_batched_last_token(const DeviceLogits& logits, size_t batch_count,
                                                  size_t seq_len, float temperature, float top_p,
                                                  std::optional<uint32_t> top_k,
                                                  const std::vector<float>& samples) {
    if (logits.rows != batch_count * seq_len)
      throw SamplerError("CUDA batched sampler logits rows " + std::to_string(logits.rows) +
                         " do not match batch " + std::to_string(batch_count) + " x seq " +
                         std::to_string(seq_len));
    if (samples.size() != batch_count)
      throw SamplerError("CUDA batched sampler got " + std::to_string(samples.size()) +
                         " random samples for " + std::to_string(batch_count) + " requests");
    if (batch_count == 0 || seq_len == 0 || logits.cols == 0)
      throw SamplerError(
          "CUDA batched sampled token selection requires non-empty logits, got batch=" +
          std::to_string(batch_count) + ", seq_len=" + std::to_string(seq_len) +
          ", cols=" + std::to_string(logits.cols));
    const auto bufs = staging(2, batch_count * sizeof(uint32_t), "allocating CUDA batched sampled tokens");
    const DeviceBuffer tokens = bufs[0], sample_buffer = bufs[1];
    upload(sample_buffer, samples, stream_, "copying CUDA batched sampler samples");
    status_check(hi_rocm_launch_sample_batched_last_token(
                     logits.data, tokens.ptr, sample_buffer.ptr, (int)batch_count, (int)seq_len,
                     (int)logits.cols, temperature, top_p, top_k_i32(top_k), 1, stream_),
                 "sample launch");
    return download(tokens, batch_count, stream_);
  }

  // gpu.rs:15810-15967
  std::vector<uint32_t> select_batched_last_token_per_row(const DeviceLogits& logits,
                                                          size_t batch_count, size_t seq_len,
                                                          const std::vector<RowSampling>& rows,
                                                          const std::vector<float>& samples) {
    if (rows.size() != batch_count || samples.size() != batch_count)
      throw SamplerError("CUDA per-row token selection got " + std::to_string(rows.size()) +
                         " sampling row(s) and " + std::to_string(samples.size()) +
                         " sample(s) for batch " + std::to_string(batch_count));
    if (batch_count == 0 || seq_len == 0 || logits.cols == 0)
      throw SamplerError("CUDA per-row token selection requires non-empty logits, got batch=" +
                         std::to_string(batch_count) + ", seq_len=" + std::to_string(seq_len) +
                         ", cols=" + std::to_string(logits.cols));
    if (logits.rows != batch_count * seq_len)
      throw SamplerError("CUDA per-row token selection logits rows " +
                         std::to_string(logits.rows) + " do not match batch " +
                         std::to_string(batch_count) + " x seq " + std::to_string(seq_len));
    bool all_greedy = true;
    for (const auto& r : rows) all_greedy = all_greedy && r.greedy;
    if (all_greedy) return argmax_batched_last_token(logits, batch_count, seq_len);
    bool uniform = !rows[0].greedy;
    for (const auto& r : rows)
      uniform = uniform && !r.greedy && same_bits(r.temperature, rows[0].temperature) &&
                same_bits(r.top_p, rows[0].top_p) && r.top_k == rows[0].top_k;
    if (uniform)
      return sample_batched_last_token(logits, batch_count, seq_len, rows[0].temperature,
                                       rows[0].top_p, rows[0].top_k, samples);
    std::vector<float> temperatures, top_ps;
    std::vector<int32_t> top_ks;
    for (const auto& r : rows) {
      if (r.greedy) {
        temperatures.push_back(0.0f);
        top_ps.push_back(1.0f);
        top_ks.push_back(0);
      } else {
        temperatures.push_back(r.temperature);
        top_ps.push_back(r.top_p);
        if (r.top_k && *r.top_k > (uint32_t)INT32_MAX)
          throw SamplerError("CUDA per-row top_k exceeds i32 range");
        top_ks.push_back(r.top_k ? (int32_t)*r.top_k : 0);
      }
    }
    const auto bufs = staging(5, batch_count * 4, "allocating CUDA per-row selected tokens");
    const DeviceBuffer tokens = bufs[0], sample_buffer = bufs[1], temperature_buffer = bufs[2],
                       top_p_buffer = bufs[3], top_k_buffer = bufs[4];
    upload(sample_buffer, samples, stream_, "copying CUDA per-row samples");
    upload(temperature_buffer, temperatures, stream_, "copying CUDA per-row temperatures");
    upload(top_p_buffer, top_ps, stream_, "copying CUDA per-row top_p values");
    upload(top_k_buffer, top_ks, stream_, "copying CUDA per-row top_k values");
    status_check(hi_rocm_launch_select_batched_last_token_per_row(
                     logits.data, tokens.ptr, sample_buffer.ptr, temperature_buffer.ptr,
                     top_p_buffer.ptr, top_k_buffer.ptr, (int)batch_count, (int)seq_len,
                     (int)logits.cols, 1, stream_),
                 "per-row launch");
    return download(tokens, batch_count, stream_);
  }

 private:
  static int top_k_i32(std::optional<uint32_t> k) {
    if (!k) return 0;
    if (*k > (uint32_t)INT32_MAX) throw SamplerError("top_k exceeds i32 range");
    return (int)*k;
  }
  // CudaRowSampling derives PartialEq over f32 fields (gpu.rs:58); NaN never
  // compares equal, which same_bits() reproduces for the uniform-batch check.
  static bool same_bits(float a, float b) { return a == b; }
  hipStream_t stream_;
};

}  // namespace hi_rocm

namespace {

int bridge_error(const std::exception& e, char* err, size_t err_len) {
  if (err && err_len > 0) {
    strncpy(err, e.what(), err_len - 1);
    err[err_len - 1] = '\0';
  }
  return 1;
}

std::optional<uint32_t> opt_k(int64_t k) {
  if (k < 0) return std::nullopt;
  return (uint32_t)k;
}

}  // namespace

// ---- bridges for tests (host parameter arrays, device logits) -----------
extern "C" {

// kinds[r]: 0 = CudaRowSampling::Greedy, 1 = Sampled; top_ks[r] < 0 = None.
// n_rows sampling rows and n_samples uniforms are passed as given (the
// function itself reports a mismatch with batch_count); out_tokens holds
// batch_count entries.
int hi_rocm_host_select_batched_last_token_per_row(
    const float* logits, size_t rows, size_t cols, size_t batch_count, size_t seq_len,
    size_t n_rows, const int32_t* kinds, const float* temperatures, const float* top_ps,
    const int64_t* top_ks, const float* samples, size_t n_samples, uint32_t* out_tokens,
    char* err, size_t err_len, void* stream) {
  try {
    std::vector<hi_rocm::RowSampling> rs;
    for (size_t r = 0; r < n_rows; ++r)
      rs.push_back({kinds[r] == 0, temperatures[r], top_ps[r], opt_k(top_ks[r])});
    std::vector<float> sm(samples, samples + n_samples);
    hi_rocm::Sampler s((hipStream_t)stream);
    auto t = s.select_batched_last_token_per_row({logits, rows, cols}, batch_count, seq_len, rs, sm);
    memcpy(out_tokens, t.data(), t.size() * sizeof(uint32_t));
    return 0;
  } catch (const std::exception& e) {
    return bridge_error(e, err, err_len);
  }
}

int hi_rocm_host_sample_batched_last_token(const float* logits, size_t rows, size_t cols,
                                           size_t batch_count, size_t seq_len, float temperature,
                                           float top_p, int64_t top_k, const float* samples,
                                           size_t n_samples, uint32_t* out_tokens, char* err,
                                           size_t err_len, void* stream) {
  try {
    std::vector<float> sm(samples, samples + n_samples);
    hi_rocm::Sampler s((hipStream_t)stream);
    auto t = s.sample_batched_last_token({logits, rows, cols}, batch_count, seq_len, temperature,
                                         top_p, opt_k(top_k), sm);
    memcpy(out_tokens, t.data(), t.size() * sizeof(uint32_t));
    return 0;
  } catch (const std::exception& e) {
    return bridge_error(e, err, err_len);
  }
}

int hi_rocm_host_argmax_batched_last_token(const float* logits, size_t rows, size_t cols,
                                           size_t batch_count, size_t seq_len,
                                           uint32_t* out_tokens, char* err, size_t err_len,
                                           void* stream) {
  try {
    hi_rocm::Sampler s((hipStream_t)stream);
    auto t = s.argmax_batched_last_token({logits, rows, cols}, batch_count, seq_len);
    memcpy(out_tokens, t.data(), t.size() * sizeof(uint32_t));
    return 0;
  } catch (const std::exception& e) {
    return bridge_error(e, err, err_len);
  }
}

int hi_rocm_host_sample_last_row_with_sample(const float* logits, size_t rows, size_t cols,
                                             float temperature, float top_p, int64_t top_k,
                                             float sample, uint32_t* out_token, char* err,
                                             size_t err_len, void* stream) {
  try {
    hi_rocm::Sampler s((hipStream_t)stream);
    *out_token = s.sample_last_row_with_sample({logits, rows, cols}, temperature, top_p,
                                               opt_k(top_k), sample);
    return 0;
  } catch (const std::exception& e) {
    return bridge_error(e, err, err_len);
  }
}

}  // extern "C"
