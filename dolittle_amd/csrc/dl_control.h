// Device-owned state of the token loop, shared by the step kernels and the
// device sampler.  It plays the role of the reference's decode.cu State and
// Control blocks (src/kernels/cuda/decode.cu:94-137): position, budget, stop
// and cancel latches live in device memory and are updated by kernels only,
// so the host never reads back per token.
#pragma once

#include <cstdint>

namespace dl {

constexpr int kMaxBatch = 8;

struct Control {
  uint64_t position;        // absolute position consumed by the current step
  uint32_t active;          // loop running
  uint32_t prompt_length;   // positions [0, prompt_length) come from `tokens`
  uint32_t generated;       // selection steps made so far (lockstep over sequences)
  uint32_t max_new;         // selection budget
  uint32_t stop_pending;    // last selection made; the next step only consumes
  uint32_t finished_mask;   // sequences that emitted a stop id
  uint32_t all_mask;        // (1 << batch) - 1
  uint32_t status;          // 0 ok, 1 NaN/+inf logit, 2 no finite logit, 4 bad token,
                            // 8 invalid injection, 16 invalid residual intervention
  uint32_t reason;          // 0 limit, 1 eos, 2 cancelled, 3 failure
  uint32_t mode;            // 0 greedy, 1 categorical
  uint32_t override_active;
  uint32_t override_mask;
  uint64_t override_position;
  int32_t capture_layer;
  int32_t steer_layer;
  uint32_t steer_mask;
  uint32_t select_row;      // 1 when the current step selects (set by k_step_begin)
  uint32_t row_generated[kMaxBatch];  // tokens emitted per sequence
};

// True when sequence `b` draws a token in the current step: the step selects
// and the sequence has not emitted a stop id yet.
__host__ __device__ inline bool row_selects(const Control* c, int b) {
  return c->active && c->select_row && !((c->finished_mask >> b) & 1u);
}

}  // namespace dl
