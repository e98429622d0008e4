// HIP runtime bridge: devices, buffers, ordered queues, completion points.
//
// Replaces the reference's CUDA runtime bridge (src/gpu/cuda/device.cpp,
// interface src/gpu/device.h:73-184).  One non-blocking HIP stream per queue
// at the default priority; completion points are HIP events recorded on the
// stream; staging buffers are pinned host memory from hipHostMalloc.
#include <cstring>
#include <string>

#include "dl_internal.h"

namespace dl {
namespace {
thread_local std::string last_error;
}

void set_last_error(const std::string& message) { last_error = message; }

void check_hip(hipError_t error, const char* what) {
  if (error != hipSuccess) {
    fail(DL_RUNTIME_ERROR, std::string(what) + ": " + hipGetErrorString(error));
  }
}

void enter(dl_queue* queue) {
  require(queue != nullptr && queue->device != nullptr, "null queue");
  if (queue->device->poisoned) fail(DL_POISONED, "device is poisoned by an earlier failure");
  queue->device->activate();
}

void check_launch(dl_queue* queue, const char* what) {
  const hipError_t error = hipGetLastError();
  if (error != hipSuccess) {
    queue->device->poisoned = true;
    fail(DL_RUNTIME_ERROR, std::string(what) + " launch failed: " + hipGetErrorString(error));
  }
}
}  // namespace dl

void dl_device::activate() const { dl::check_hip(hipSetDevice(ordinal), "hipSetDevice"); }

using dl::guard;
using dl::require;

extern "C" {

const char* dl_last_error(void) { return dl::last_error.c_str(); }

int dl_device_open(int ordinal, dl_device** out) {
  return guard([&] {
    require(out != nullptr, "null output");
    int count = 0;
    dl::check_hip(hipGetDeviceCount(&count), "hipGetDeviceCount");
    require(ordinal >= 0 && ordinal < count, "device ordinal out of range");
    auto* device = new dl_device();
    device->ordinal = ordinal;
    const hipError_t e = hipGetDeviceProperties(&device->properties, ordinal);
    if (e != hipSuccess) {
      delete device;
      dl::check_hip(e, "hipGetDeviceProperties");
    }
    *out = device;
  });
}

int dl_device_close(dl_device* device) {
  return guard([&] {
    if (!device) return;
    device->activate();
    (void)hipDeviceSynchronize();
    delete device;
  });
}

int dl_device_info_get(dl_device* device, dl_device_info* out) {
  return guard([&] {
    require(device && out, "null argument");
    std::memset(out, 0, sizeof *out);
    std::strncpy(out->name, device->properties.name, sizeof out->name - 1);
    std::strncpy(out->arch, device->properties.gcnArchName, sizeof out->arch - 1);
    out->compute_units = static_cast<uint32_t>(device->properties.multiProcessorCount);
    out->total_bytes = device->properties.totalGlobalMem;
  });
}

int dl_memory_snapshot(dl_device* device, uint64_t* free_bytes, uint64_t* total_bytes) {
  return guard([&] {
    require(device && free_bytes && total_bytes, "null argument");
    device->activate();
    size_t f = 0, t = 0;
    dl::check_hip(hipMemGetInfo(&f, &t), "hipMemGetInfo");
    *free_bytes = f;
    *total_bytes = t;
  });
}

int dl_buffer_alloc(dl_device* device, uint64_t bytes, uint64_t alignment, dl_buffer** out) {
  return guard([&] {
    require(device && out, "null argument");
    require(bytes > 0, "zero-byte allocation");
    require(alignment == 0 || (alignment & (alignment - 1)) == 0, "alignment must be a power of two");
    require(alignment <= 256, "alignment above 256 bytes is not supported", DL_LENGTH_ERROR);
    device->activate();
    void* p = nullptr;
    const hipError_t e = hipMalloc(&p, bytes);
    if (e != hipSuccess) {
      (void)hipGetLastError();
      dl::fail(DL_LENGTH_ERROR, std::string("device allocation failed: ") + hipGetErrorString(e));
    }
    *out = new dl_buffer{device, p, bytes, false};
  });
}

int dl_staging_alloc(dl_device* device, uint64_t bytes, dl_buffer** out) {
  return guard([&] {
    require(device && out, "null argument");
    require(bytes > 0, "zero-byte allocation");
    device->activate();
    void* p = nullptr;
    const hipError_t e = hipHostMalloc(&p, bytes, hipHostMallocDefault);
    if (e != hipSuccess) {
      (void)hipGetLastError();
      dl::fail(DL_LENGTH_ERROR, std::string("staging allocation failed: ") + hipGetErrorString(e));
    }
    *out = new dl_buffer{device, p, bytes, true};
  });
}

int dl_buffer_free(dl_buffer* buffer) {
  return guard([&] {
    if (!buffer) return;
    buffer->device->activate();
    if (buffer->staging) {
      (void)hipHostFree(buffer->pointer);
    } else {
      (void)hipFree(buffer->pointer);
    }
    delete buffer;
  });
}

int dl_buffer_address(dl_buffer* buffer, void** out) {
  return guard([&] {
    require(buffer && out, "null argument");
    *out = buffer->pointer;
  });
}

int dl_buffer_size(dl_buffer* buffer, uint64_t* out) {
  return guard([&] {
    require(buffer && out, "null argument");
    *out = buffer->bytes;
  });
}

int dl_queue_create(dl_device* device, dl_queue** out) {
  return guard([&] {
    require(device && out, "null argument");
    device->activate();
    auto* q = new dl_queue();
    q->device = device;
    const hipError_t e = hipStreamCreateWithFlags(&q->stream, hipStreamNonBlocking);
    if (e != hipSuccess) {
      delete q;
      dl::check_hip(e, "hipStreamCreateWithFlags");
    }
    *out = q;
  });
}

int dl_queue_destroy(dl_queue* queue) {
  return guard([&] {
    if (!queue) return;
    queue->device->activate();
    (void)hipStreamSynchronize(queue->stream);
    for (auto& p : queue->points) (void)hipEventDestroy(p.event);
    (void)hipStreamDestroy(queue->stream);
    delete queue;
  });
}

namespace {
void check_region(const dl_buffer* b, uint64_t offset, uint64_t bytes, bool staging) {
  require(b != nullptr, "null buffer");
  require(b->staging == staging, staging ? "expected a staging buffer" : "expected a device buffer");
  require(offset <= b->bytes && bytes <= b->bytes - offset, "region outside buffer", DL_LENGTH_ERROR);
}
}  // namespace

int dl_queue_upload(dl_queue* queue, dl_buffer* dst, uint64_t dst_offset, dl_buffer* src,
                    uint64_t src_offset, uint64_t bytes) {
  return guard([&] {
    dl::enter(queue);
    check_region(dst, dst_offset, bytes, false);
    check_region(src, src_offset, bytes, true);
    if (!bytes) return;
    dl::check_hip(hipMemcpyAsync(static_cast<char*>(dst->pointer) + dst_offset,
                                 static_cast<char*>(src->pointer) + src_offset, bytes,
                                 hipMemcpyHostToDevice, queue->stream),
                  "upload");
  });
}

int dl_queue_download(dl_queue* queue, dl_buffer* dst, uint64_t dst_offset, dl_buffer* src,
                      uint64_t src_offset, uint64_t bytes) {
  return guard([&] {
    dl::enter(queue);
    check_region(dst, dst_offset, bytes, true);
    check_region(src, src_offset, bytes, false);
    if (!bytes) return;
    dl::check_hip(hipMemcpyAsync(static_cast<char*>(dst->pointer) + dst_offset,
                                 static_cast<char*>(src->pointer) + src_offset, bytes,
                                 hipMemcpyDeviceToHost, queue->stream),
                  "download");
  });
}

int dl_queue_copy(dl_queue* queue, dl_buffer* dst, uint64_t dst_offset, dl_buffer* src,
                  uint64_t src_offset, uint64_t bytes) {
  return guard([&] {
    dl::enter(queue);
    check_region(dst, dst_offset, bytes, false);
    check_region(src, src_offset, bytes, false);
    if (!bytes) return;
    dl::check_hip(hipMemcpyAsync(static_cast<char*>(dst->pointer) + dst_offset,
                                 static_cast<char*>(src->pointer) + src_offset, bytes,
                                 hipMemcpyDeviceToDevice, queue->stream),
                  "copy");
  });
}

int dl_queue_write(dl_queue* queue, dl_buffer* dst, uint64_t dst_offset, const void* host,
                   uint64_t bytes) {
  return guard([&] {
    dl::enter(queue);
    check_region(dst, dst_offset, bytes, false);
    require(host != nullptr || bytes == 0, "null host pointer");
    if (!bytes) return;
    dl::check_hip(hipMemcpyAsync(static_cast<char*>(dst->pointer) + dst_offset, host, bytes,
                                 hipMemcpyHostToDevice, queue->stream),
                  "write");
    dl::check_hip(hipStreamSynchronize(queue->stream), "write wait");
  });
}

int dl_queue_read(dl_queue* queue, void* host, dl_buffer* src, uint64_t src_offset, uint64_t bytes) {
  return guard([&] {
    dl::enter(queue);
    check_region(src, src_offset, bytes, false);
    require(host != nullptr || bytes == 0, "null host pointer");
    if (!bytes) return;
    dl::check_hip(hipMemcpyAsync(host, static_cast<char*>(src->pointer) + src_offset, bytes,
                                 hipMemcpyDeviceToHost, queue->stream),
                  "read");
    dl::check_hip(hipStreamSynchronize(queue->stream), "read wait");
  });
}

int dl_queue_transfer(dl_queue* queue, void* dst, const void* src, uint64_t bytes) {
  return guard([&] {
    dl::enter(queue);
    require((dst != nullptr && src != nullptr) || bytes == 0, "null transfer address");
    if (!bytes) return;
    dl::check_hip(hipMemcpyAsync(dst, src, bytes, hipMemcpyDefault, queue->stream), "transfer");
  });
}

int dl_queue_mark(dl_queue* queue, uint64_t* point) {
  return guard([&] {
    dl::enter(queue);
    require(point != nullptr, "null point");
    hipEvent_t event;
    dl::check_hip(hipEventCreateWithFlags(&event, hipEventDisableTiming), "hipEventCreate");
    const hipError_t e = hipEventRecord(event, queue->stream);
    if (e != hipSuccess) {
      (void)hipEventDestroy(event);
      dl::check_hip(e, "hipEventRecord");
    }
    queue->points.push_back({queue->next_point, event});
    *point = queue->next_point++;
  });
}

int dl_queue_wait(dl_queue* queue, uint64_t point) {
  return guard([&] {
    dl::enter(queue);
    require(point < queue->next_point, "completion point was never marked");
    // Every point up to `point` is reached once that point's event is.
    size_t keep = 0;
    hipError_t status = hipSuccess;
    for (auto& p : queue->points) {
      if (p.id == point) status = hipEventSynchronize(p.event);
    }
    for (auto& p : queue->points) {
      if (p.id <= point) {
        (void)hipEventDestroy(p.event);
      } else {
        queue->points[keep++] = p;
      }
    }
    queue->points.resize(keep);
    if (status != hipSuccess) {
      queue->device->poisoned = true;
      dl::check_hip(status, "queue wait");
    }
  });
}

int dl_queue_drain(dl_queue* queue) {
  return guard([&] {
    dl::enter(queue);
    const hipError_t status = hipStreamSynchronize(queue->stream);
    for (auto& p : queue->points) (void)hipEventDestroy(p.event);
    queue->points.clear();
    if (status != hipSuccess) {
      queue->device->poisoned = true;
      dl::check_hip(status, "queue drain");
    }
  });
}

int dl_event_create(dl_device* device, dl_event** out) {
  return guard([&] {
    require(device && out, "null argument");
    device->activate();
    auto* e = new dl_event();
    e->device = device;
    const hipError_t status = hipEventCreate(&e->event);
    if (status != hipSuccess) {
      delete e;
      dl::check_hip(status, "hipEventCreate");
    }
    *out = e;
  });
}

int dl_event_destroy(dl_event* event) {
  return guard([&] {
    if (!event) return;
    (void)hipEventDestroy(event->event);
    delete event;
  });
}

int dl_event_record(dl_event* event, dl_queue* queue) {
  return guard([&] {
    require(event != nullptr, "null event");
    dl::enter(queue);
    dl::check_hip(hipEventRecord(event->event, queue->stream), "hipEventRecord");
  });
}

int dl_event_elapsed_ms(dl_event* start, dl_event* stop, float* ms) {
  return guard([&] {
    require(start && stop && ms, "null argument");
    dl::check_hip(hipEventSynchronize(stop->event), "hipEventSynchronize");
    dl::check_hip(hipEventElapsedTime(ms, start->event, stop->event), "hipEventElapsedTime");
  });
}

}  // extern "C"
