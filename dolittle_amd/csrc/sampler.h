// Device categorical selection over BF16 logits rows (the sampling law of
// src/inference/sampling/categorical.cpp:146-201 and the device selector of
// src/kernels/cuda/sampling.cu:106-376), shared by the standalone sampler
// (dl_sampler_*) and the token loop.
//
// Law.  Finite candidates only (NaN or +inf rejects the row with status 1,
// no finite value gives status 2).  Greedy takes the largest value, lowest
// id.  Categorical orders candidates by descending value (signed zeros equal)
// then ascending id, keeps the first top_k, weighs each by
// w = exp((z - z0) / T) in binary64, folds the weights serially in that order
// (F_k), keeps the smallest prefix c with F_c / F_n >= top_p, draws
// u = (x >> 11) * 2^-53 and returns the first i <= c whose serial fold of
// w / F_c exceeds u (else candidate c).
//
// Algorithm.  A BF16 row has at most 65536 distinct values, and equal values
// have equal weights, so a counting sort over the 16-bit order key replaces
// the reference's four radix passes: k_sample_count builds the per-value
// histogram (plus argmax partials and the NaN/finite flags), k_sample_select
// turns it into FP64 prefix estimates with one exp per distinct value and
// decides cutoff and draw with guarded comparisons: every estimate is within
// a proven relative bound g of the host's serial fold, so a decision that
// holds with margin g is the host's decision.  When u or top_p falls inside
// the band, one lane replays the serial fold exactly (weights from the same
// deterministic exp as the CPU restatement).  The token is then the j-th
// smallest id holding the selected value.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

#include "dl_control.h"

namespace dl::sampling {

constexpr int kBins = 65536;
constexpr int kCountBlocks = 64;
constexpr int kCountThreads = 256;
constexpr int kSelectThreads = 1024;
constexpr int kBinsPerThread = kBins / kSelectThreads;
constexpr int kMtWords = 312;

struct Settings {
  uint32_t mode;  // 0 greedy, 1 categorical
  uint32_t top_k; // 0 disables
  double temperature;
  double top_p;
};

struct Result {
  uint32_t token, status;
};

// Per-row selection state: the MT19937-64 stream (sampler.h:52) and the
// DeviceCategorical terminal latch (sampling.cu commit_selection).
struct RowState {
  uint64_t words[kMtWords];
  uint32_t index;
  uint32_t terminal;
  double draw;
  Result result;
  Result previous;
  uint64_t exact_replays;  // selections decided by the serial replay
};

// Device workspace of `rows` selection rows.
struct Workspace {
  uint32_t* hist;          // [rows][kBins], all zero between selections
  double* weights;         // [rows][kBins]
  uint64_t* partial_keys;  // [rows][kCountBlocks]
  uint32_t* partial_flags; // [rows][kCountBlocks]
  RowState* state;         // [rows]
  uint8_t* stop_mask;      // [vocabulary] (standalone sampler)
};

std::size_t workspace_bytes(int rows, uint64_t vocabulary);
Workspace carve_workspace(void* base, int rows, uint64_t vocabulary);

// Token-loop destination of each row's selection.
struct LoopOutput {
  Control* ctl;            // null: standalone sampler
  uint32_t* selected;      // [rows]
  uint32_t* out_tokens;    // [rows][out_capacity]
  uint32_t out_capacity;
  const uint8_t* stop_mask;
};

struct RowsArgs {
  const uint16_t* logits;  // row r at logits + r * row_stride
  uint64_t row_stride;
  uint32_t n;
  int rows;
  Settings settings;
  Workspace ws;
  const double* draw;      // device draw (standalone live stream) or null
  double draw_value;       // explicit draw when `draw` and `loop_rng` are unset
  int loop_rng;            // draw from each row's stream inside the selection
  int exact;               // always decide by the serial replay (diagnostic)
  LoopOutput loop;
  Result* result_out;      // standalone: the caller's {token, status} instead of the row state's
};

struct Seeds {
  uint64_t seed[kMaxBatch];
};

void launch_count(hipStream_t stream, const RowsArgs& args);
void launch_select(hipStream_t stream, const RowsArgs& args);
void launch_seed(hipStream_t stream, RowState* state, int rows, const Seeds& seeds);
void launch_clear(hipStream_t stream, const Workspace& ws, int rows);

}  // namespace dl::sampling
