// Shared between the kernels (sampler_kernels.hip) and the host API
// (sampler_api.hip).  Not part of the public ABI.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "hi_rocm.h"
#include "exact_fold.h"

namespace hi_rocm {

constexpr int kScanThreads = 256;                  // workgroup (4 wave64s)
constexpr int kVecLarge = 4;                       // float4 loads per thread per tile
constexpr int kTilesLarge = 4;                     // tiles per chunk
constexpr int kChunk = kScanThreads * kVecLarge * 4 * kTilesLarge;  // 16384 logits per chunk
constexpr int kVecSmall = 2;
constexpr int kChunkSmall = kScanThreads * kVecSmall * 4;  // 2048 (one tile), small batches
constexpr int kFast = 1024;                        // candidates kept per chunk (max)
constexpr int kLeanK = 256;                        // largest top-k of the streaming selection
constexpr int kMaxVocab = 1 << 23;                 // 8,388,608
constexpr int kLseTop = 16;                        // per-chunk candidates kept for logprobs
constexpr int kRowGeneralChunk = kScanThreads * 32;  // logits per chunk of the row kernel's general path

enum RowClass : int { kGreedy = 0, kTopK = 1, kTopP = 2, kTempOnly = 3 };
enum ParamsMode : int { kParamsRows = 0, kParamsSoA = 1, kParamsUniform = 2 };
// Greedy rows: block_argmax_last (kernels.cu:7153-7186), or the finite-only
// argmax of sample_last_token_row (kernels.cu:7775-7801), which is what the
// reference's uniform-config batched kernel returns for temperature <= 0.
enum GreedyRule : int { kGreedyIeee = 0, kGreedyFiniteLane = 1 };

// Where the per-row parameters come from: the extended API's struct array,
// the reference per-row launcher's three arrays, or one config for all rows.
struct ParamsView {
  const hi_rocm_row_params* rows;
  const float* temps;
  const float* top_ps;
  const int* top_ks;
  float T, top_p;
  int top_k;
  int mode;
  const float* uniforms;  // device f32[B], or null: uniform_value for every row
  float uniform_value;
  int greedy_rule;        // GreedyRule
};

// Decoded row configuration.
struct RowCfg {
  float T, top_p, min_p, rep, freq, pres;
  int top_k;
  uint32_t eos, flags;
  int cls;        // RowClass
  int k_eff;      // min(top_k, V) for top-k rows
  float t_eff;    // temperature used for s = l / t_eff (1 for greedy rows)
  float cutoff;   // clamped top_p (gpu.rs:789-793)
  bool rep_on;
  bool wide;      // top-k row with k_eff > kLeanK
  int k_sel;      // candidates each chunk keeps
  bool store_s;   // scaled logits go to the workspace
  float u;        // the row's uniform for the draw
};

// Per (row, chunk) statistics written by the scan, merged by the finish.
struct ChunkStat {
  float max_l;                    // max finite processed logit l (-inf: none);
                                  // the debug kernels keep the max of s here
  float am_ieee_v;                // argmax, IEEE '>' (kernels.cu:7153-7186)
  uint32_t am_ieee_i;
  float am_fin_v;                 // finite argmax, lane rule (kernels.cu:7775-7801)
  uint32_t am_fin_i;
  uint32_t any_finite;
  float lse_m;                    // scaled-logit reference of the masses below
  float lse_sum;                  // sum of exp(s - lse_m) over the logits not written as candidates
  uint32_t n_cand;                // candidates written
  uint32_t trunc;                 // the chunk has logits that are not candidates
  uint32_t unkept_key;            // bound on the keys of those logits
  uint32_t pad0;
  uint64_t min_kept;              // smallest candidate key
  uint64_t pad1;
};
static_assert(sizeof(ChunkStat) == 64, "ChunkStat layout");

// Per (row, chunk) mass histogram of a top-p row, written by the select
// pass: bin j holds the sum of w' = exp(s - ms) (approximate exp) over the
// chunk's logits with w' in (2^-(j+1), 2^-j], the last bin also everything
// below.  It only sizes the nucleus superset; no result depends on it.
constexpr int kWideBins = 32;
struct WideStat {
  float ms;                  // the chunk's max scaled logit (the bins' reference)
  uint32_t valid;            // 1: written by this call's select pass
  float hist[kWideBins];
};

static_assert(sizeof(WideStat) == 136, "WideStat layout");

// Per (row, chunk) result of the wide pass for a top-p row: the maps of
// the chunk's weights in the vocabulary-order fold for a start value in
// binade e0, e0 + 1 or e0 + 2 (exact while the sum stays in that binade),
// and the number of distinct-weight runs of the nucleus superset it wrote.
constexpr int kCrossTerms = 48;  // terms of a crossing window
constexpr int kCrossWins = 2;    // crossing windows a chunk records
struct ChunkFold {
  uint32_t e0;
  uint32_t nruns;            // superset runs written; kFoldNone: the chunk's table overflowed
  uint32_t has_end;          // chunk 0: `end` is the exact fold of its weights from -0.0
  float end;
  fold::Map map[3];          // the chunk's terms in binades e0, e0 + 1, e0 + 2
  // the predicted crossings: nw windows (0: none predicted) around the
  // terms where the fold leaves a binade; segment s (before window 0,
  // between the windows, after the last) is folded in binade be[s] by its
  // map seg[s]; window w holds wn[w] terms, added one by one
  uint32_t nw;
  uint32_t be[kCrossWins + 1];
  uint32_t wn[kCrossWins];
  fold::Map seg[kCrossWins + 1];
  float term[kCrossWins][kCrossTerms];
  uint32_t flags;            // bit k: map[k] holds the chunk's map; bit 3: the block maps are stored
  uint32_t pad;
};
static_assert(sizeof(ChunkFold) == 480, "ChunkFold layout");
constexpr uint32_t kFoldNone = 0xffffffffu;

struct SampleArgs {
  const void* logits;  // row 0 of the batch
  int dtype;
  int B, V;
  int64_t row_stride;  // elements between rows
  int vec_ok;          // 128-bit (f32) / 64-bit (bf16) loads are aligned
  ParamsView pv;
  const uint32_t* hoff;
  const uint32_t* hids;
  const uint32_t* hcnt;
  const uint32_t* mask;
  int mask_words;      // ceil(V / 32)
  int n_lp;
  int need_lse;
  int chunk;           // logits per chunk (kChunk or kChunkSmall)
  int n_chunks;
  uint32_t* out_tokens;
  float* out_lp;
  uint32_t* out_lp_ids;
  float* out_token_lp;
  // workspace
  ChunkStat* stats;    // [B][n_chunks]
  uint64_t* cand;      // [B][n_chunks][kFast]
  float* ws_s;         // [B][V]
  float* ws_w;         // [B][V]
  uint64_t* ws_list;   // [B][list_stride]; the wide pass's superset runs
  int64_t list_stride;
  uint32_t* done;      // [kDoneRows] chunks of the row finished (zero between launches)
  WideStat* wstat;     // [B][n_chunks]
  ChunkFold* wfold;    // [B][n_chunks]
  fold::Map* wbmap;    // [B][n_chunks][3][kScanThreads]: per-thread block maps of each ChunkFold binade
  uint32_t* diag;      // [B] how the wide pass finished each top-p row (WidePath)
  float* wtot;         // [B][2] the wide pass's normaliser and candidate total (debug export)
};

// diag values for top-p rows of the chunked path (0: not a top-p row of
// that path, or an older call).
enum WidePath : uint32_t {
  kWideDone = 1,          // finished by the wide pass
  kWideNoStats = 2,       // a chunk's statistics were not written by this call's pass, or no finite logit
  kWideChunkFull = 3,     // a chunk's table of distinct weights overflowed
  kWideTotal = 4,         // the normaliser is not positive and finite (argmax fallback)
  kWideMergeFull = 5,     // the row's table of distinct weights overflowed
  kWideNoCutoff = 6,      // the cutoff lies outside the superset
  kWideDrawFail = 7,      // the candidate total or the drawn index could not be resolved
  // rows of the row kernel
  kRowPathMinp = 8,       // the min-p support finish
  kRowPathLists = 9,      // the candidate lists' finish (finish_core)
  kRowPathGeneral = 10,   // the general path (chunk select and finish)
};

// Batches whose (chunk, row) grid has at most this many workgroups run the
// select and the finish as one kernel; that bounds their rows too.
constexpr int kFusedMaxWorkgroups = 512;
constexpr int kFusedMaxRows = kFusedMaxWorkgroups;
// Per-row counters of the kernels whose last workgroup of a row finishes it
// (both leave them at zero); this also bounds the rows of one call.
constexpr int kDoneRows = 65536;

struct WorkspaceLayout {
  size_t stats, cand, ws_s, ws_w, ws_list, done, wstat, wfold, wbmap, diag, wtot, total;
  int64_t slots;       // (row, chunk) records reserved
  int64_t list_stride;
};

int choose_chunk(int B, int V, int n_lp, int vec_ok, bool hist);

inline int64_t next_pow2_i64(int64_t x) {
  int64_t p = 1;
  while (p < x) p <<= 1;
  return p;
}

// The layout with `slots` (row, chunk) records for up to max_batch rows.
inline WorkspaceLayout workspace_layout_slots(int max_batch, int V, int64_t slots) {
  auto align = [](size_t x) { return (x + 255) & ~(size_t)255; };
  WorkspaceLayout L;
  L.slots = slots;
  L.list_stride = next_pow2_i64(V);
  size_t off = 0;
  // the fused path's per-row counters first, at the same place in every
  // layout (calls of any shape may share a workspace)
  L.done = off; off = align(off + (size_t)kDoneRows * sizeof(uint32_t));
  L.stats = off; off = align(off + (size_t)L.slots * sizeof(ChunkStat));
  L.wstat = off; off = align(off + (size_t)L.slots * sizeof(WideStat));
  L.wfold = off; off = align(off + (size_t)L.slots * sizeof(ChunkFold));
  L.wbmap = off; off = align(off + (size_t)L.slots * 3 * kScanThreads * sizeof(fold::Map));
  L.diag = off; off = align(off + (size_t)max_batch * sizeof(uint32_t));
  L.wtot = off; off = align(off + (size_t)max_batch * 2 * sizeof(float));
  L.cand = off; off = align(off + (size_t)L.slots * kFast * sizeof(uint64_t));
  L.ws_s = off; off = align(off + (size_t)max_batch * V * sizeof(float));
  L.ws_w = off; off = align(off + (size_t)max_batch * V * sizeof(float));
  L.ws_list = off; off = align(off + (size_t)max_batch * L.list_stride * sizeof(uint64_t));
  L.total = off;
  return L;
}

// Workspace for any call with up to max_batch rows of V logits.
inline WorkspaceLayout workspace_layout(int max_batch, int V) {
  int64_t slots = 0;
  for (int b = 1; b <= max_batch; ++b) {
    // records of either pass (streaming select or general scan) at b rows
    for (int n_lp : {0, kLeanK + 1}) {
      const int ch = choose_chunk(b, V, n_lp, 1, true);
      const int64_t s = (int64_t)b * ((V + ch - 1) / ch);
      if (s > slots) slots = s;
    }
    // the row kernel's general path (8192-logit chunks)
    const int64_t sg = (int64_t)b * ((V + kRowGeneralChunk - 1) / kRowGeneralChunk);
    if (sg > slots) slots = sg;
  }
  return workspace_layout_slots(max_batch, V, slots);
}

// Workspace of general_row_path alone for up to max_batch rows.
inline WorkspaceLayout general_layout(int max_batch, int V) {
  return workspace_layout_slots(max_batch, V, (int64_t)max_batch * ((V + kRowGeneralChunk - 1) / kRowGeneralChunk));
}

// Measurement hook: when given, the launcher records ev[0] before its first
// kernel, ev[1] after the pass over the logits and ev[2] after the finish,
// all on the launch stream (ev[1] == ev[2] for a one-kernel step).
struct LaunchEvents {
  hipEvent_t ev[3];
};

hipError_t launch_sample(const SampleArgs& a, hipStream_t stream, const LaunchEvents* le = nullptr);
hipError_t launch_argmax(const float* logits, uint32_t* out, int B, int64_t row_stride,
                         int64_t row_offset, int cols, hipStream_t stream);
hipError_t launch_debug_expf(const float* x, float* y, int64_t n, hipStream_t stream);
constexpr int kDebugFoldMaxRuns = 65536;
size_t debug_fold_lds(int R);
hipError_t launch_debug_fold(const float* x, const uint32_t* m, int R, float a0, float* out_start,
                             float* out_final, hipStream_t stream);
hipError_t launch_debug_distribution(const SampleArgs& a, float* out_proc, float* out_probs,
                                     hipStream_t stream);

// Status helpers of the C ABI (sampler_api.hip): set the calling thread's
// hi_rocm_last_error message and return the status code.
int api_fail(int code, const char* msg);
int api_hip_fail(hipError_t e, const char* where);

// The LM-head projection + bias + softcap fused into the sampler's first
// pass (sampler_kernels.hip).
constexpr int kLmTile = 128;     // vocabulary columns per workgroup (chunk)
constexpr int kLmThreads = 128;  // 2 waves of 64 columns
constexpr int kLmRows = 64;      // rows per call (two groups of 32)
constexpr int kLmMaxK = 64;      // largest top-k of the fused finish
constexpr int kLmMaxTiles = 4096;  // tiles per row the fused finish holds (V <= 524,288)
struct LmTileRec;
struct LmArgs {
  const __bf16* hidden;   // [B][H]
  const __bf16* weight;   // [V][H]
  const float* bias;      // [V] or null
  float cap;              // softcap (<= 0: none)
  int B, H, V;
  int n_chunks;           // tiles: ceil(V / kLmTile)
  float* out_logits;      // the twin: [B][V]
  ParamsView pv;
  LmTileRec* lm_recs;     // [B][n_chunks]
  float* lm_logits;       // [B][lm_stride(V)]: the tiles of every row but greedy ones
  uint32_t* out_tokens;   // [B]
  SampleArgs gen;         // general_row_path over lm_logits, for the rows the fused finish leaves
};
// Rows of lm_logits start on 16 bytes (the general path's 16-byte loads).
__host__ __device__ inline int64_t lm_stride(int V) { return ((int64_t)V + 3) & ~(int64_t)3; }
hipError_t launch_lm_logits(const LmArgs& a, hipStream_t stream);
hipError_t launch_lm_sample(const LmArgs& a, hipStream_t stream);
size_t lm_workspace_bytes(int B, int V);
size_t lm_recs_bytes(int B, int n_tiles);
size_t lm_logits_bytes(int B, int V);

// Exact top-k block selection of the DSV4 indexer (index_select.hip): one
// workgroup (no workspace), or for kMultiMinN < n <= 4096 * 1024 a
// workgroup per 4096 scores in three kernels, with a workspace of
// index_select_ws_bytes(n) whose first kIndexHistBytes are zero between
// calls.
constexpr int kMultiMinN = 8192;
constexpr size_t kIndexHistBytes = 4096 * sizeof(uint32_t);
hipError_t launch_index_select(const float* scores, int n, int top_k, uint8_t* marks, int32_t* sel,
                               hipStream_t stream);
size_t index_select_ws_bytes(int n);
hipError_t launch_index_select_multi(const float* scores, int n, int top_k, uint8_t* marks, int32_t* sel,
                                     void* ws, hipStream_t stream);

}  // namespace hi_rocm
