// Internal definitions shared by the libdlhip.so translation units.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <stdexcept>
#include <string>
#include <vector>

#include "../../include/dolittle_hip.h"

namespace dl {

// A failure carrying the C-ABI status it maps to.
struct Error : std::runtime_error {
  int status;
  Error(int s, const std::string& message) : std::runtime_error(message), status(s) {}
};

[[noreturn]] inline void fail(int status, const std::string& message) { throw Error(status, message); }

inline void require(bool condition, const char* message, int status = DL_INVALID_ARGUMENT) {
  if (!condition) fail(status, message);
}

void check_hip(hipError_t error, const char* what);
void set_last_error(const std::string& message);

// Runs `body`, converting exceptions into a status and the thread's last
// error message (the reference rethrows the same classes in its adapter).
template <class F>
int guard(F&& body) {
  try {
    body();
    return DL_OK;
  } catch (const Error& e) {
    set_last_error(e.what());
    return e.status;
  } catch (const std::bad_alloc&) {
    set_last_error("host allocation failed");
    return DL_LENGTH_ERROR;
  } catch (const std::exception& e) {
    set_last_error(e.what());
    return DL_RUNTIME_ERROR;
  } catch (...) {
    set_last_error("unknown failure");
    return DL_RUNTIME_ERROR;
  }
}

}  // namespace dl

struct dl_device {
  int ordinal = 0;
  hipDeviceProp_t properties{};
  bool poisoned = false;
  void activate() const;
};

struct dl_buffer {
  dl_device* device = nullptr;
  void* pointer = nullptr;
  uint64_t bytes = 0;
  bool staging = false;
};

struct dl_queue {
  dl_device* device = nullptr;
  hipStream_t stream = nullptr;
  uint64_t next_point = 1;
  struct Point {
    uint64_t id;
    hipEvent_t event;
  };
  std::vector<Point> points;
};

struct dl_event {
  dl_device* device = nullptr;
  hipEvent_t event = nullptr;
};

namespace dl {
// Checks that the queue's device is usable and makes it current.
void enter(dl_queue* queue);
// Reports an immediate launch failure (asynchronous ones surface at wait).
void check_launch(dl_queue* queue, const char* what);
__host__ __device__ inline uint64_t ceil_div(uint64_t a, uint64_t b) { return a / b + (a % b != 0); }
}  // namespace dl
