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
  // Event journal state (k_step_begin / k_step_end): events published per
  // sequence, sequences whose terminal event is out, and the snapshots the
  // step's end needs of its beginning.
  uint32_t events[kMaxBatch];
  uint32_t terminal_mask;   // sequences whose terminal event is published
  uint32_t select_mask;     // sequences selecting in this step (taken at its beginning)
  uint32_t finished_before; // finished_mask at the beginning of this step
  uint32_t cancel_pending;  // a cancellation seen with a selection pending consumption
  uint32_t steps;           // steps executed while the loop was active
};

// DeviceSequence event (src/inference/decoding/device.h:86-102): 32 bytes,
// kind in the low byte of the first word.  Kinds and reasons keep the
// reference's numbering.
enum EventKind : uint32_t { kConsumed = 0, kSelected = 1, kTerminal = 2, kInjection = 3 };
enum Reason : uint32_t { kLimit = 0, kEos = 1, kCancelled = 2, kFailure = 3 };
struct Event {
  uint32_t kind;
  uint32_t status;
  uint64_t position;
  uint64_t count;
  uint32_t token;
  float norm;
};
static_assert(sizeof(Event) == 32, "event layout");

// Host-mapped publication words, one 64-byte line each: the number of
// events of a sequence, published with a system-scope release after the
// events themselves; and the loop's liveness and executed step count, which
// the host reads to pace a bounded step window.
struct Publication {
  uint32_t completed;
  uint32_t pad[15];
};
struct Mirror {
  uint32_t active;
  uint32_t steps;
  uint32_t pad[14];
};
// Device addresses of a plan's journal (pinned, host-mapped memory).
struct Journal {
  Publication* publication;  // [kMaxBatch]
  Mirror* mirror;
  Event* events;             // [kMaxBatch][capacity]
  uint32_t capacity;         // events per sequence
};

// True when sequence `b` draws a token in the current step: the step selects
// and the sequence has not emitted a stop id yet.
__host__ __device__ inline bool row_selects(const Control* c, int b) {
  return c->active && c->select_row && !((c->finished_mask >> b) & 1u);
}

}  // namespace dl
