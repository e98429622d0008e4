// DeviceSequence for HIP: the reference's autonomous prepared sequence
// (src/inference/decoding/device.h:84-137, CUDA form in
// src/kernels/cuda/decode.cu) without conditional graph nodes.
//
// The caller records the same stages as for CUDA (begin, begin_stage,
// end_stage, begin_selection, capture, replace, complete); everything it
// submits to the queue in between is captured from the queue's stream into
// one HIP graph per segment:
//
//   pre        begin() .. begin_stage(prefill): state reset, the caller's
//              set-up work (intervention reset, injection), decide(prefill)
//   prefill    one full prompt chunk, then finish_prompt (decides repeat)
//   link 1     decide(tail)        tail       the remainder chunk
//   link 2     decide(first)       first      head + first selection
//   link 3     decide(decode)      decode A   forward of the selected token,
//                                             finish_consumption (decides B)
//              decode B            head + selection, continue (decides A)
//   final      finish_sequence (the terminal event)
//
// Each decision is taken on the device from device words (position, budget,
// error latches, the sampler's result and terminal words, the cancel word),
// exactly where the CUDA graph's conditional nodes read them, and published
// to pinned host-mapped memory with a system-scope release.  start() hands
// the segments to a driver thread that launches a segment, waits for the
// decision the device publishes at its end and launches the segment the
// decision names.  So every body runs exactly as often as its conditional
// node would run, nothing runs speculatively (no body has to be made a
// no-op), and the host never decides: it only relays the device's decision.
// The cost is one device-to-host round trip and one graph launch per
// decision (two per generated token).  Events are the reference's 32-byte
// records in host-mapped memory, published with the same release / acquire
// pair; collect() and request_stop() may run on other threads.
#include <algorithm>
#include <atomic>
#include <chrono>
#include <cstring>
#include <limits>
#include <memory>
#include <string>
#include <thread>
#include <vector>

#include "dl_device.h"
#include "dl_internal.h"

namespace dl::seq {

constexpr int kPrefill = 0, kTail = 1, kFirst = 2, kDecode = 3;
constexpr uint32_t kConsumed = 0, kSelected = 1, kTerminal = 2, kInjection = 3;
constexpr uint32_t kLimit = 0, kEos = 1, kCancelled = 2, kFailure = 3;

struct State {
  uint64_t position, generated;
  uint32_t events, error, decisions, reserved;
};

// Pinned, host-mapped: publication words on their own 64-byte lines, then
// the event journal.
struct Publication {
  alignas(64) uint32_t completed;  // events published
  alignas(64) uint32_t cancel;     // host -> device stop request
  alignas(64) uint32_t decisions;  // decisions published
  uint32_t decision;               // the latest decision (1 run, 0 skip)
};
constexpr uint64_t kEventsOffset = 256;
static_assert(sizeof(Publication) <= kEventsOffset, "publication block");

struct Event {
  uint8_t kind;
  uint8_t reserved[3];
  uint32_t status;
  uint64_t position, count;
  uint32_t token;
  float norm;
};
static_assert(sizeof(Event) == 32 && sizeof(Event) == sizeof(dl_sequence_event), "the reference's 32-byte event");

struct Control {
  State* state;
  Publication* publication;  // device view of the mapped block
  Event* events;
  uint64_t capacity;         // events
  const uint32_t *selection, *terminal, *prompt_ids, *injection_status;
  const float* injection_norm;
  const uint32_t *intervention_status, *intervention_count;
  uint32_t* token_input;
  uint64_t prompt, generated, chunk;
  int forward_only;
};

__device__ bool cancelled(const Control& c) {
  return __hip_atomic_load(&c.publication->cancel, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_SYSTEM) != 0u;
}

__device__ void publish(const Control& c, uint32_t kind, uint32_t status, uint64_t position, uint64_t count,
                        uint32_t token, float norm) {
  State& s = *c.state;
  if (s.events >= c.capacity) return;  // capacity is P + 2G + 2, never exceeded
  Event e{};
  e.kind = static_cast<uint8_t>(kind);
  e.status = status;
  e.position = position;
  e.count = count;
  e.token = token;
  e.norm = norm;
  c.events[s.events] = e;
  s.events += 1;
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "");
  __hip_atomic_store(&c.publication->completed, s.events, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}

// Publishes the decision the host driver waits for.
__device__ void decide(const Control& c, bool run) {
  State& s = *c.state;
  c.publication->decision = run ? 1u : 0u;
  s.decisions += 1;
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "");
  __hip_atomic_store(&c.publication->decisions, s.decisions, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}

__global__ void k_init(Control c) { *c.state = State{}; }

// Whether `stage` runs (decode.cu decide_stage): the injection status is
// published and latched before the prompt, an intervention failure is
// latched before every stage, and a stage runs only without a latched error.
__global__ void k_decide(Control c, int stage) {
  State& s = *c.state;
  if (stage == kPrefill && c.injection_status) {
    s.error = *c.injection_status;
    publish(c, kInjection, s.error, 0, 0, 0, *c.injection_norm);
  }
  if (c.intervention_status) s.error |= *c.intervention_status;
  bool run = false;
  if (s.error == 0u) {
    const uint64_t remainder = c.prompt % c.chunk;
    if (stage == kPrefill) {
      run = !cancelled(c) && s.position + c.chunk <= c.prompt;
    } else if (stage == kTail) {
      run = !cancelled(c) && remainder != 0 && s.position == c.prompt - remainder;
    } else if (stage == kFirst) {
      run = !cancelled(c) && s.position == c.prompt && (c.generated != 0 || c.forward_only);
    } else {
      run = s.generated != 0;  // a selection is always consumed, even after a stop
    }
  }
  decide(c, run);
}

// Token ids of the body's rows: the prompt at the device position, or the
// last selection for a decode body.
__global__ void k_load_tokens(Control c, uint64_t rows, int from_selection) {
  for (uint64_t i = threadIdx.x; i < rows; i += blockDim.x)
    c.token_input[i] = from_selection ? c.selection[0] : c.prompt_ids[c.state->position + i];
}

// A prompt chunk is consumed; a full-chunk body decides whether it repeats.
__global__ void k_finish_prompt(Control c, uint64_t rows, int repeat) {
  State& s = *c.state;
  publish(c, kConsumed, 0, s.position, rows, 0, 0.0f);
  s.position += rows;
  if (c.intervention_status) s.error |= *c.intervention_status;
  if (repeat) decide(c, s.error == 0u && !cancelled(c) && s.position + c.chunk <= c.prompt);
}

// The sampler's {token, status}: a failure latches, a token is published.
__global__ void k_finish_selection(Control c) {
  State& s = *c.state;
  s.error = c.selection[1];
  if (s.error == 0u) {
    s.generated += 1;
    publish(c, kSelected, 0, s.position, 1, c.selection[0], 0.0f);
  }
}

// The selected token is consumed; the selection tail runs while the budget,
// the stop latch, the error latch and the cancel word allow.
__global__ void k_finish_consumption(Control c) {
  State& s = *c.state;
  publish(c, kConsumed, 0, s.position, 1, 0, 0.0f);
  s.position += 1;
  if (c.intervention_status) s.error |= *c.intervention_status;
  const bool stopped = c.terminal != nullptr && *c.terminal != 0u;
  decide(c, s.error == 0u && !stopped && s.generated < c.generated && !cancelled(c));
}

// After a selection the decode body repeats unless it failed.
__global__ void k_continue(Control c) { decide(c, c.state->error == 0u); }

// The terminal event (decode.cu finish_sequence): an intervention must have
// been applied exactly once once the prompt is consumed.
__global__ void k_finish(Control c) {
  State& s = *c.state;
  if (c.intervention_status) {
    s.error |= *c.intervention_status;
    if (s.position >= c.prompt && *c.intervention_count != 1u) s.error = 1u;
  }
  uint32_t reason;
  if (s.error != 0u) {
    reason = kFailure;
  } else if (s.generated != 0 && c.terminal != nullptr && *c.terminal != 0u) {
    reason = kEos;
  } else if (s.position == c.prompt + s.generated && s.generated == c.generated) {
    reason = kLimit;
  } else {
    reason = kCancelled;
  }
  publish(c, kTerminal, reason, s.position, s.generated, s.error, 0.0f);
  decide(c, false);  // the driver's end-of-sequence marker
}

// Rows of a body copied to the capture arena at the device position.
__global__ void k_capture(Control c, const uint8_t* source, uint8_t* destination, uint64_t row_bytes,
                          uint64_t rows) {
  const uint64_t bytes = rows * row_bytes;
  uint8_t* target = destination + c.state->position * row_bytes;
  const uint64_t first = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const uint64_t stride = static_cast<uint64_t>(gridDim.x) * blockDim.x;
  if (((reinterpret_cast<uintptr_t>(source) | reinterpret_cast<uintptr_t>(target) | bytes) & 3u) == 0) {
    const uint32_t* from = reinterpret_cast<const uint32_t*>(source);
    uint32_t* to = reinterpret_cast<uint32_t*>(target);
    for (uint64_t i = first; i < bytes / 4; i += stride) to[i] = from[i];
  } else {
    for (uint64_t i = first; i < bytes; i += stride) target[i] = source[i];
  }
}

// The row of prompt position `marker` is replaced when this body holds it.
__global__ void k_replace(Control c, const uint8_t* row, uint8_t* embeddings, uint64_t row_bytes, uint64_t marker,
                          uint64_t rows) {
  const uint64_t position = c.state->position;
  if (marker < position || marker - position >= rows) return;
  uint8_t* target = embeddings + (marker - position) * row_bytes;
  for (uint64_t i = threadIdx.x; i < row_bytes; i += blockDim.x) target[i] = row[i];
}

enum Segment { kPre, kPrefillBody, kLink1, kTailBody, kLink2, kFirstBody, kLink3, kDecodeA, kDecodeB, kFinal, kSegments };

uint64_t event_capacity(uint64_t prompt, uint64_t generated, uint64_t chunk) {
  const uint64_t max = std::numeric_limits<uint64_t>::max();
  require(prompt > 0 && chunk > 0 && prompt <= max - 2 && generated <= (max - prompt - 2) / 2 &&
              chunk <= prompt + generated,
          "sequence capacity", DL_LENGTH_ERROR);
  const uint64_t n = prompt + 2 * generated + 2;
  require(n <= std::numeric_limits<uint32_t>::max(), "event count", DL_LENGTH_ERROR);
  return n;
}

}  // namespace dl::seq

using namespace dl::seq;

struct dl_sequence {
  dl_queue* queue = nullptr;
  Control control{};
  State* state = nullptr;
  void* host = nullptr;  // pinned, mapped: Publication + events
  uint64_t host_bytes = 0;
  Publication* publication = nullptr;
  hipGraphExec_t segments[kSegments] = {};
  int current = -1;  // segment being captured
  int next_stage = 0, stage = -1;
  bool begun = false, in_stage = false, selection = false, completed = false, launched = false;
  std::thread driver;
  std::atomic<bool> driver_done{false};
  std::atomic<int> driver_status{DL_OK};
  std::string driver_error;

  void begin_capture(int segment) {
    dl::check_hip(hipStreamBeginCapture(queue->stream, hipStreamCaptureModeThreadLocal), "sequence capture");
    current = segment;
  }
  void end_capture() {
    hipGraph_t graph = nullptr;
    const hipError_t e = hipStreamEndCapture(queue->stream, &graph);
    const int segment = current;
    current = -1;
    dl::check_hip(e, "sequence capture end");
    hipGraphExec_t exec = nullptr;
    const hipError_t i = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
    (void)hipGraphDestroy(graph);
    dl::check_hip(i, "sequence graph instantiation");
    segments[segment] = exec;
  }
  void stop() { __atomic_store_n(&publication->cancel, 1u, __ATOMIC_RELEASE); }
  uint32_t completed_events() const { return __atomic_load_n(&publication->completed, __ATOMIC_ACQUIRE); }
  void run_driver();
};

// Launches segments in the order the device's decisions name (see the top
// of this file).  A failed launch or stream, or a stream that goes idle
// without the awaited decision, ends the driver with an error that drain()
// and collect() report.
void dl_sequence::run_driver() {
  uint32_t awaited = 0;
  auto fail = [&](int status, const std::string& message) {
    driver_error = message;
    driver_status.store(status, std::memory_order_release);
  };
  auto launch = [&](int segment) {
    const hipError_t e = hipGraphLaunch(segments[segment], queue->stream);
    if (e != hipSuccess) {
      fail(DL_RUNTIME_ERROR, std::string("sequence segment launch failed: ") + hipGetErrorString(e));
      return false;
    }
    return true;
  };
  // Waits for decision number ++awaited; returns 1 run, 0 skip, -1 failure.
  auto wait = [&]() -> int {
    ++awaited;
    uint64_t spins = 0;
    for (;;) {
      if (__atomic_load_n(&publication->decisions, __ATOMIC_ACQUIRE) >= awaited)
        return __atomic_load_n(&publication->decision, __ATOMIC_ACQUIRE) != 0u ? 1 : 0;
      if (++spins % 4096 == 0) {
        const hipError_t q = hipStreamQuery(queue->stream);
        if (q == hipSuccess) {
          if (__atomic_load_n(&publication->decisions, __ATOMIC_ACQUIRE) >= awaited) continue;
          fail(DL_RUNTIME_ERROR, "sequence stream went idle without a decision");
          return -1;
        }
        if (q != hipErrorNotReady) {
          fail(DL_RUNTIME_ERROR, std::string("sequence stream failed: ") + hipGetErrorString(q));
          return -1;
        }
        std::this_thread::sleep_for(std::chrono::microseconds(20));
      } else {
        std::this_thread::yield();
      }
    }
  };
  queue->device->activate();
  int run = 0;
  do {
    if (!launch(kPre) || (run = wait()) < 0) break;
    while (run == 1) {
      if (!launch(kPrefillBody) || (run = wait()) < 0) break;
    }
    if (run < 0) break;
    if (!launch(kLink1) || (run = wait()) < 0) break;
    if (run == 1 && !launch(kTailBody)) break;
    if (!launch(kLink2) || (run = wait()) < 0) break;
    if (run == 1 && !launch(kFirstBody)) break;
    if (!launch(kLink3) || (run = wait()) < 0) break;
    while (run == 1) {
      if (!launch(kDecodeA) || (run = wait()) < 0) break;
      if (run == 0) break;
      if (!launch(kDecodeB) || (run = wait()) < 0) break;
    }
    if (run < 0) break;
    if (!launch(kFinal)) break;
    (void)wait();
  } while (false);
  const hipError_t e = hipStreamSynchronize(queue->stream);
  if (e != hipSuccess && driver_status.load(std::memory_order_acquire) == DL_OK)
    fail(DL_RUNTIME_ERROR, std::string("sequence stream failed: ") + hipGetErrorString(e));
  driver_done.store(true, std::memory_order_release);
}

namespace {
using dl::guard;
using dl::require;

void join_driver(dl_sequence* s) {
  if (s->driver.joinable()) s->driver.join();
}

void check_driver(dl_sequence* s) {
  const int status = s->driver_status.load(std::memory_order_acquire);
  if (status != DL_OK) dl::fail(status, s->driver_error);
}
}  // namespace

extern "C" {

int dl_sequence_device_bytes(uint64_t* bytes) {
  return guard([&] {
    require(bytes != nullptr, "null argument");
    *bytes = sizeof(State);
  });
}

int dl_sequence_host_bytes(uint64_t prompt, uint64_t generated, uint64_t chunk, uint64_t* bytes) {
  return guard([&] {
    require(bytes != nullptr, "null argument");
    const uint64_t n = event_capacity(prompt, generated, chunk);
    require(n <= (std::numeric_limits<uint64_t>::max() - kEventsOffset) / sizeof(Event), "sequence journal bytes",
            DL_LENGTH_ERROR);
    *bytes = kEventsOffset + n * sizeof(Event);
  });
}

int dl_sequence_create(dl_queue* queue, uint64_t prompt, uint64_t generated, uint64_t chunk, int forward_only,
                       dl_sequence** out) {
  return guard([&] {
    require(queue && out, "null argument");
    dl::enter(queue);
    uint64_t host_bytes = 0;
    if (const int st = dl_sequence_host_bytes(prompt, generated, chunk, &host_bytes); st != DL_OK)
      dl::fail(st, dl_last_error());
    auto s = std::make_unique<dl_sequence>();
    s->queue = queue;
    dl::check_hip(hipMalloc(reinterpret_cast<void**>(&s->state), sizeof(State)), "sequence state");
    const hipError_t e = hipHostMalloc(&s->host, host_bytes, hipHostMallocMapped | hipHostMallocCoherent);
    if (e != hipSuccess) {
      (void)hipFree(s->state);
      dl::fail(DL_LENGTH_ERROR, "sequence journal allocation failed");
    }
    std::memset(s->host, 0, host_bytes);
    s->host_bytes = host_bytes;
    s->publication = static_cast<Publication*>(s->host);
    void* mapped = nullptr;
    dl::check_hip(hipHostGetDevicePointer(&mapped, s->host, 0), "sequence journal mapping");
    Control& c = s->control;
    c.state = s->state;
    c.publication = static_cast<Publication*>(mapped);
    c.events = reinterpret_cast<Event*>(static_cast<uint8_t*>(mapped) + kEventsOffset);
    c.capacity = event_capacity(prompt, generated, chunk);
    c.prompt = prompt;
    c.generated = generated;
    c.chunk = chunk;
    c.forward_only = forward_only ? 1 : 0;
    *out = s.release();
  });
}

int dl_sequence_destroy(dl_sequence* s) {
  return guard([&] {
    if (!s) return;
    s->queue->device->activate();
    s->stop();
    if (s->current >= 0) {
      hipGraph_t ignored = nullptr;
      (void)hipStreamEndCapture(s->queue->stream, &ignored);
      if (ignored) (void)hipGraphDestroy(ignored);
    }
    join_driver(s);
    (void)hipStreamSynchronize(s->queue->stream);
    for (auto& g : s->segments)
      if (g) (void)hipGraphExecDestroy(g);
    (void)hipFree(s->state);
    (void)hipHostFree(s->host);
    delete s;
  });
}

int dl_sequence_position_address(dl_sequence* s, void** out) {
  return guard([&] {
    require(s && out, "null argument");
    *out = &s->state->position;
  });
}

int dl_sequence_begin(dl_sequence* s, const uint32_t* selection, const uint32_t* terminal, uint32_t* token_input,
                      uint64_t token_input_bytes, const uint32_t* prompt, uint64_t prompt_bytes,
                      const uint32_t* injection_status, const float* injection_norm,
                      const uint32_t* intervention_status, const uint32_t* intervention_count) {
  return guard([&] {
    require(s != nullptr, "null sequence");
    Control& c = s->control;
    require(!s->begun, "invalid sequence begin: already begun");
    require(c.forward_only ? (selection == nullptr && terminal == nullptr && c.generated == 0)
                           : (selection != nullptr && terminal != nullptr),
            "invalid sequence begin: selection words");
    require(token_input && token_input_bytes >= c.chunk * sizeof(uint32_t), "invalid sequence begin: token input");
    require(prompt && prompt_bytes == c.prompt * sizeof(uint32_t), "invalid sequence begin: prompt");
    require((injection_status == nullptr) == (injection_norm == nullptr), "invalid injection controls");
    require((intervention_status == nullptr) == (intervention_count == nullptr), "intervention control bounds");
    dl::enter(s->queue);
    c.selection = selection;
    c.terminal = terminal;
    c.token_input = token_input;
    c.prompt_ids = prompt;
    c.injection_status = injection_status;
    c.injection_norm = injection_norm;
    c.intervention_status = intervention_status;
    c.intervention_count = intervention_count;
    s->begin_capture(kPre);
    hipLaunchKernelGGL(k_init, dim3(1), dim3(1), 0, s->queue->stream, c);
    dl::check_launch(s->queue, "sequence begin");
    s->begun = true;
  });
}

int dl_sequence_begin_stage(dl_sequence* s, int stage) {
  return guard([&] {
    require(s != nullptr, "null sequence");
    require(s->begun && !s->in_stage && stage == s->next_stage && s->current >= 0, "invalid sequence stage order");
    dl::enter(s->queue);
    const Control& c = s->control;
    hipLaunchKernelGGL(k_decide, dim3(1), dim3(1), 0, s->queue->stream, c, stage);
    dl::check_launch(s->queue, "sequence stage decision");
    s->end_capture();
    static const int body[4] = {kPrefillBody, kTailBody, kFirstBody, kDecodeA};
    s->begin_capture(body[stage]);
    if (stage != kFirst) {
      const uint64_t rows = stage == kPrefill ? c.chunk : (stage == kTail ? c.prompt % c.chunk : 1);
      hipLaunchKernelGGL(k_load_tokens, dim3(1), dim3(256), 0, s->queue->stream, c, rows, stage == kDecode ? 1 : 0);
      dl::check_launch(s->queue, "sequence token load");
    }
    s->stage = stage;
    s->in_stage = true;
  });
}

int dl_sequence_begin_selection(dl_sequence* s) {
  return guard([&] {
    require(s != nullptr, "null sequence");
    require(s->in_stage && s->stage == kDecode && !s->selection, "invalid decode selection branch");
    dl::enter(s->queue);
    hipLaunchKernelGGL(k_finish_consumption, dim3(1), dim3(1), 0, s->queue->stream, s->control);
    dl::check_launch(s->queue, "sequence consumption");
    s->end_capture();
    s->begin_capture(kDecodeB);
    s->selection = true;
  });
}

int dl_sequence_end_stage(dl_sequence* s) {
  return guard([&] {
    require(s != nullptr, "null sequence");
    require(s->in_stage, "no sequence stage");
    require(s->stage != kDecode || s->selection, "missing selection tail");
    dl::enter(s->queue);
    const Control& c = s->control;
    hipStream_t stream = s->queue->stream;
    if (s->stage == kPrefill || s->stage == kTail) {
      const uint64_t rows = s->stage == kPrefill ? c.chunk : c.prompt % c.chunk;
      hipLaunchKernelGGL(k_finish_prompt, dim3(1), dim3(1), 0, stream, c, rows, s->stage == kPrefill ? 1 : 0);
    } else {
      if (!c.forward_only) hipLaunchKernelGGL(k_finish_selection, dim3(1), dim3(1), 0, stream, c);
      if (s->stage == kDecode) hipLaunchKernelGGL(k_continue, dim3(1), dim3(1), 0, stream, c);
    }
    dl::check_launch(s->queue, "sequence stage end");
    s->end_capture();
    static const int link[4] = {kLink1, kLink2, kLink3, kFinal};
    s->begin_capture(link[s->stage]);
    s->in_stage = false;
    s->next_stage += 1;
  });
}

int dl_sequence_capture(dl_sequence* s, const void* source, uint64_t source_bytes, void* destination,
                        uint64_t destination_bytes, uint64_t row_bytes, uint64_t rows) {
  return guard([&] {
    require(s != nullptr, "null sequence");
    require(s->in_stage && s->stage != kFirst && !s->selection, "capture requires a consumption body");
    const Control& c = s->control;
    const uint64_t capacity = c.prompt + c.generated;
    require(source && destination && row_bytes && rows && rows <= c.chunk &&
                row_bytes <= std::numeric_limits<uint64_t>::max() / capacity && source_bytes == rows * row_bytes &&
                destination_bytes == capacity * row_bytes,
            "invalid sequence capture bounds");
    dl::enter(s->queue);
    const unsigned blocks =
        static_cast<unsigned>(std::min<uint64_t>(65535, 1 + (source_bytes - 1) / (256 * sizeof(uint32_t))));
    hipLaunchKernelGGL(k_capture, dim3(blocks), dim3(256), 0, s->queue->stream, c,
                       static_cast<const uint8_t*>(source), static_cast<uint8_t*>(destination), row_bytes, rows);
    dl::check_launch(s->queue, "sequence capture copy");
  });
}

int dl_sequence_replace(dl_sequence* s, const void* row, uint64_t row_bytes, void* embeddings,
                        uint64_t embeddings_bytes, uint64_t marker, uint64_t rows) {
  return guard([&] {
    require(s != nullptr, "null sequence");
    const Control& c = s->control;
    require(s->in_stage && row && embeddings && marker < c.prompt && rows && row_bytes &&
                row_bytes <= embeddings_bytes / rows,
            "embedding override bounds");
    dl::enter(s->queue);
    hipLaunchKernelGGL(k_replace, dim3(1), dim3(256), 0, s->queue->stream, c, static_cast<const uint8_t*>(row),
                       static_cast<uint8_t*>(embeddings), row_bytes, marker, rows);
    dl::check_launch(s->queue, "sequence embedding override");
  });
}

int dl_sequence_complete(dl_sequence* s) {
  return guard([&] {
    require(s != nullptr, "null sequence");
    require(s->next_stage == 4 && !s->in_stage && !s->completed && s->current == kFinal, "incomplete sequence");
    dl::enter(s->queue);
    hipLaunchKernelGGL(k_finish, dim3(1), dim3(1), 0, s->queue->stream, s->control);
    dl::check_launch(s->queue, "sequence finish");
    s->end_capture();
    s->completed = true;
  });
}

int dl_sequence_resources(dl_sequence* s, uint64_t* device_bytes, uint64_t* host_bytes) {
  return guard([&] {
    require(s && device_bytes && host_bytes, "null argument");
    require(s->completed, "sequence not prepared");
    *device_bytes = sizeof(State);
    *host_bytes = s->host_bytes + sizeof(dl_sequence);
  });
}

int dl_sequence_start(dl_sequence* s) {
  return guard([&] {
    require(s != nullptr, "null sequence");
    require(s->completed && !s->launched, "sequence start");
    dl::enter(s->queue);
    s->launched = true;
    s->driver = std::thread([s] { s->run_driver(); });
  });
}

int dl_sequence_request_stop(dl_sequence* s) {
  return guard([&] {
    require(s != nullptr, "null sequence");
    s->stop();
  });
}

int dl_sequence_drain(dl_sequence* s) {
  return guard([&] {
    require(s != nullptr, "null sequence");
    join_driver(s);
    check_driver(s);
    if (const int st = dl_queue_drain(s->queue); st != DL_OK) dl::fail(st, dl_last_error());
  });
}

int dl_sequence_collect(dl_sequence* s, uint64_t index, int wait, dl_sequence_event* event, int* ready) {
  return guard([&] {
    require(s && event && ready, "null argument");
    require(s->launched, "event outside sequence: not started");
    require(index < s->control.capacity, "event outside sequence", DL_LENGTH_ERROR);
    *ready = 0;
    for (;;) {
      if (s->completed_events() > index) break;
      if (s->driver_done.load(std::memory_order_acquire)) {
        if (s->completed_events() > index) break;
        check_driver(s);
        dl::fail(DL_RUNTIME_ERROR, "sequence ended without event");
      }
      if (!wait) return;
      std::this_thread::sleep_for(std::chrono::microseconds(50));
    }
    std::memcpy(event, static_cast<const uint8_t*>(s->host) + kEventsOffset + index * sizeof(Event), sizeof(Event));
    *ready = 1;
  });
}

int dl_sequence_event_count(dl_sequence* s, uint64_t* count) {
  return guard([&] {
    require(s && count, "null argument");
    *count = s->completed_events();
  });
}

}  // extern "C"
