// HIP backend of Dolittle's device interfaces over libdlhip.so: the file a
// maintainer adds to the reference tree (as src/gpu/hip/backend.cpp) to run
// its gpu::Device / gpu::Queue users, DeviceCategorical users and
// DeviceSequence::collect's consumers on the C ABI of include/dolittle_hip.h.
//
// Interfaces implemented, member by member:
//   src/gpu/device.h:73-184            DeviceBuffer, HostBuffer, Queue, Device
//   src/inference/sampling/device.h:54-85  DeviceCategorical
//   src/inference/decoding/device.h:84-137 DeviceSequence::Event (collect)
// Build:
//   g++ -std=c++20 -fPIC -shared -I<reference>/src -Iinclude integration/hip_backend.cpp
//       -Ldolittle_amd -ldlhip -Wl,--no-undefined -o libdolittle_hip_backend.so

#include <chrono>
#include <cstring>
#include <limits>
#include <stdexcept>
#include <stop_token>
#include <string>
#include <thread>
#include <utility>

#include "dolittle_hip.h"
#include "gpu/device.h"
#include "inference/decoding/device.h"
#include "inference/sampling/device.h"

namespace dolittle::gpu::hip {

// The exception classes the reference's callers catch (src/gpu/device.h:23-25).
inline void check(int status) {
  switch (status) {
    case DL_OK:
      return;
    case DL_INVALID_ARGUMENT:
      throw std::invalid_argument(dl_last_error());
    case DL_LENGTH_ERROR:
      throw std::length_error(dl_last_error());
    default:
      throw std::runtime_error(dl_last_error());
  }
}

std::unique_ptr<Device> open_device(int ordinal);

}  // namespace dolittle::gpu::hip

namespace dolittle::gpu {

// A buffer either owns a dl_buffer or borrows device memory that another
// object owns (the sampler's result words): `handle` is null when borrowed.
struct DeviceBuffer::Impl {
  dl_buffer* handle = nullptr;
  void* address = nullptr;
  std::size_t bytes = 0;
};
struct HostBuffer::Impl {
  dl_buffer* handle = nullptr;
  std::byte* host = nullptr;
  std::size_t bytes = 0;
};
struct Queue::Impl {
  dl_queue* handle = nullptr;
  std::uint64_t identity = 0;
};

namespace detail {
struct BackendAccess {
  static DeviceBuffer own(dl_buffer* handle, std::size_t bytes) {
    void* address = nullptr;
    const int status = dl_buffer_address(handle, &address);
    if (status != DL_OK) {
      dl_buffer_free(handle);
      hip::check(status);
    }
    return DeviceBuffer(std::unique_ptr<DeviceBuffer::Impl>(new DeviceBuffer::Impl{handle, address, bytes}));
  }
  static DeviceBuffer borrow(void* address, std::size_t bytes) {
    return DeviceBuffer(std::unique_ptr<DeviceBuffer::Impl>(new DeviceBuffer::Impl{nullptr, address, bytes}));
  }
  static HostBuffer staging(dl_buffer* handle, std::size_t bytes) {
    void* host = nullptr;
    const int status = dl_buffer_address(handle, &host);
    if (status != DL_OK) {
      dl_buffer_free(handle);
      hip::check(status);
    }
    return HostBuffer(
        std::unique_ptr<HostBuffer::Impl>(new HostBuffer::Impl{handle, static_cast<std::byte*>(host), bytes}));
  }
  static Queue queue(dl_queue* handle) {
    static std::uint64_t next_identity = 1;
    return Queue(std::unique_ptr<Queue::Impl>(new Queue::Impl{handle, next_identity++}));
  }
  static dl_queue* handle(Queue& q) {
    if (!q.impl_) throw std::invalid_argument("moved-from queue");
    return q.impl_->handle;
  }

  // Checked [offset, offset + bytes) of a live owner (device.h: "Regions
  // borrow an unmoved owner and checked ... bytes").
  template <class Owner>
  static const typename Owner::Impl& checked(const Owner* owner, std::size_t offset, std::size_t bytes) {
    if (owner == nullptr || !owner->impl_) throw std::invalid_argument("region without a live owner");
    const auto& impl = *owner->impl_;
    if (offset > impl.bytes || bytes > impl.bytes - offset) throw std::invalid_argument("region out of range");
    return impl;
  }
  static const void* address(ConstDeviceRegion r) {
    return static_cast<const std::byte*>(checked(r.owner, r.offset, r.bytes).address) + r.offset;
  }
  static void* address(DeviceRegion r) {
    return static_cast<std::byte*>(checked(r.owner, r.offset, r.bytes).address) + r.offset;
  }
  // Transfers name an owning dl_buffer; borrowed memory is addressed directly.
  static dl_buffer* owned(const DeviceBuffer* owner, std::size_t offset, std::size_t bytes) {
    const auto& impl = checked(owner, offset, bytes);
    if (impl.handle == nullptr) throw std::invalid_argument("transfer on borrowed device memory");
    return impl.handle;
  }
  static dl_buffer* owned(const HostBuffer* owner, std::size_t offset, std::size_t bytes) {
    return checked(owner, offset, bytes).handle;
  }
};
}  // namespace detail

using detail::BackendAccess;

DeviceBuffer::DeviceBuffer(std::unique_ptr<Impl> impl) : impl_(std::move(impl)) {}
DeviceBuffer::~DeviceBuffer() {
  if (impl_ && impl_->handle) dl_buffer_free(impl_->handle);
}
DeviceBuffer::DeviceBuffer(DeviceBuffer&& other) noexcept = default;
DeviceBuffer& DeviceBuffer::operator=(DeviceBuffer&& other) noexcept {
  if (this != &other) {
    if (impl_ && impl_->handle) dl_buffer_free(impl_->handle);
    impl_ = std::move(other.impl_);
  }
  return *this;
}
std::size_t DeviceBuffer::size_bytes() const noexcept { return impl_ ? impl_->bytes : 0; }

HostBuffer::HostBuffer(std::unique_ptr<Impl> impl) : impl_(std::move(impl)) {}
HostBuffer::~HostBuffer() {
  if (impl_) dl_buffer_free(impl_->handle);
}
HostBuffer::HostBuffer(HostBuffer&& other) noexcept = default;
HostBuffer& HostBuffer::operator=(HostBuffer&& other) noexcept {
  if (this != &other) {
    if (impl_) dl_buffer_free(impl_->handle);
    impl_ = std::move(other.impl_);
  }
  return *this;
}
std::span<std::byte> HostBuffer::bytes() noexcept {
  return impl_ ? std::span<std::byte>(impl_->host, impl_->bytes) : std::span<std::byte>();
}
std::span<const std::byte> HostBuffer::bytes() const noexcept {
  return impl_ ? std::span<const std::byte>(impl_->host, impl_->bytes) : std::span<const std::byte>();
}

Queue::Queue(std::unique_ptr<Impl> impl) : impl_(std::move(impl)) {}
Queue::~Queue() {
  if (impl_) dl_queue_destroy(impl_->handle);  // drains first
}
Queue::Queue(Queue&& other) noexcept = default;
Queue& Queue::operator=(Queue&& other) noexcept {
  if (this != &other) {
    if (impl_) dl_queue_destroy(impl_->handle);
    impl_ = std::move(other.impl_);
  }
  return *this;
}

static void same_size(std::size_t a, std::size_t b) {
  if (a != b) throw std::invalid_argument("transfer regions differ in size");
}

void Queue::upload(DeviceRegion destination, ConstHostRegion source) {
  same_size(destination.bytes, source.bytes);
  hip::check(dl_queue_upload(BackendAccess::handle(*this),
                             BackendAccess::owned(destination.owner, destination.offset, destination.bytes),
                             destination.offset, BackendAccess::owned(source.owner, source.offset, source.bytes),
                             source.offset, source.bytes));
}
void Queue::download(HostRegion destination, ConstDeviceRegion source) {
  same_size(destination.bytes, source.bytes);
  hip::check(dl_queue_download(BackendAccess::handle(*this),
                               BackendAccess::owned(destination.owner, destination.offset, destination.bytes),
                               destination.offset, BackendAccess::owned(source.owner, source.offset, source.bytes),
                               source.offset, source.bytes));
}
void Queue::copy(DeviceRegion destination, ConstDeviceRegion source) {
  same_size(destination.bytes, source.bytes);
  hip::check(dl_queue_copy(BackendAccess::handle(*this),
                           BackendAccess::owned(destination.owner, destination.offset, destination.bytes),
                           destination.offset, BackendAccess::owned(source.owner, source.offset, source.bytes),
                           source.offset, source.bytes));
}
// Completion points are an unbounded counter here: nothing to reserve.
void Queue::reserve_completion_points(std::size_t) {}
CompletionPoint Queue::mark() {
  std::uint64_t point = 0;
  hip::check(dl_queue_mark(BackendAccess::handle(*this), &point));
  return {impl_->identity, point};
}
void Queue::wait(CompletionPoint point) {
  if (!impl_ || point.queue_identity != impl_->identity) throw std::invalid_argument("point of another queue");
  hip::check(dl_queue_wait(impl_->handle, point.sequence));
}
void Queue::drain() { hip::check(dl_queue_drain(BackendAccess::handle(*this))); }

Device::Device() = default;
Device::~Device() = default;

namespace hip {

class HipDevice final : public Device {
 public:
  explicit HipDevice(int ordinal) {
    check(dl_device_open(ordinal, &device_));
    dl_device_info raw{};
    const int status = dl_device_info_get(device_, &raw);
    if (status != DL_OK) {
      dl_device_close(device_);
      check(status);
    }
    info_.backend = "hip";
    info_.name = raw.name;
    info_.architecture = raw.arch;
    info_.driver_version = "";
    info_.total_memory_bytes = raw.total_bytes;
  }
  ~HipDevice() override { dl_device_close(device_); }
  const DeviceInfo& info() const noexcept override { return info_; }
  DeviceBuffer allocate(AllocationRequest request) override {
    dl_buffer* b = nullptr;
    check(dl_buffer_alloc(device_, request.bytes, request.alignment, &b));
    return BackendAccess::own(b, request.bytes);
  }
  HostBuffer allocate_staging(AllocationRequest request) override {
    dl_buffer* b = nullptr;
    check(dl_staging_alloc(device_, request.bytes, &b));
    return BackendAccess::staging(b, request.bytes);
  }
  Queue create_queue() override {
    dl_queue* q = nullptr;
    check(dl_queue_create(device_, &q));
    return BackendAccess::queue(q);
  }
  dl_device* handle() const noexcept { return device_; }

 private:
  dl_device* device_ = nullptr;
  DeviceInfo info_;
};

std::unique_ptr<Device> open_device(int ordinal) { return std::make_unique<HipDevice>(ordinal); }

dl_device* handle(Device& device) {
  auto* hip = dynamic_cast<HipDevice*>(&device);
  if (hip == nullptr) throw std::invalid_argument("device of another backend");
  return hip->handle();
}

}  // namespace hip
}  // namespace dolittle::gpu

namespace dolittle::inference::sampling {

using gpu::detail::BackendAccess;

// The sampler's arena is the library's; the result, terminal and token words
// are exposed as borrowed device regions for graph readers and copies.
struct DeviceCategorical::Impl {
  Impl(dl_sampler* s, std::size_t n, void* result_word, void* terminal_word, void* token_word)
      : sampler(s),
        vocabulary(n),
        result(BackendAccess::borrow(result_word, 2 * sizeof(std::uint32_t))),
        terminal(BackendAccess::borrow(terminal_word, sizeof(std::uint32_t))),
        token(BackendAccess::borrow(token_word, sizeof(std::uint32_t))) {}
  ~Impl() { dl_sampler_destroy(sampler); }
  Impl(const Impl&) = delete;
  Impl& operator=(const Impl&) = delete;
  dl_sampler* sampler;
  std::size_t vocabulary;
  gpu::DeviceBuffer result, terminal, token;
};

static dl_sampling native(Settings s) {
  dl_sampling out{};
  out.mode = s.mode == SelectionMode::greedy ? 0u : 1u;
  if (s.top_k > std::numeric_limits<std::uint32_t>::max()) throw std::invalid_argument("top_k out of range");
  out.top_k = static_cast<std::uint32_t>(s.top_k);
  out.temperature = s.temperature;
  out.top_p = s.top_p;
  return out;
}

DeviceCategorical::DeviceCategorical(gpu::Device& device, gpu::Queue& queue, std::size_t vocabulary,
                                     tensors::ElementType type, std::size_t budget) {
  if (type != tensors::ElementType::bfloat16) throw std::invalid_argument("the HIP sampler reads BF16 rows");
  dl_sampler* sampler = nullptr;
  gpu::hip::check(dl_sampler_create(gpu::hip::handle(device), BackendAccess::handle(queue), vocabulary, DL_BF16,
                                    budget, &sampler));
  void *result = nullptr, *terminal = nullptr, *token = nullptr;
  int status = dl_sampler_result_address(sampler, &result);
  if (status == DL_OK) status = dl_sampler_terminal_address(sampler, &terminal);
  if (status == DL_OK) status = dl_sampler_current_token_address(sampler, &token);
  if (status != DL_OK) {
    dl_sampler_destroy(sampler);
    gpu::hip::check(status);
  }
  impl_ = std::make_unique<Impl>(sampler, vocabulary, result, terminal, token);
}
DeviceCategorical::~DeviceCategorical() = default;

std::size_t DeviceCategorical::required_bytes(std::size_t vocabulary) {
  std::uint64_t bytes = 0;
  gpu::hip::check(dl_sampler_required_bytes(vocabulary, &bytes));
  return bytes;
}

gpu::ConstDeviceRegion DeviceCategorical::submit(gpu::ConstDeviceRegion row, DeviceDraw draw) {
  const dl_sampling s = native(draw.settings);
  gpu::hip::check(dl_sampler_submit(impl_->sampler, BackendAccess::address(row), row.bytes, &s, draw.bits));
  return result_storage();
}
void DeviceCategorical::start(Settings settings, std::uint64_t seed, std::span<const std::uint32_t> stop_ids) {
  const dl_sampling s = native(settings);
  if (stop_ids.size() > std::numeric_limits<std::uint32_t>::max()) throw std::length_error("too many stop ids");
  gpu::hip::check(dl_sampler_start(impl_->sampler, &s, seed, stop_ids.data(),
                                   static_cast<std::uint32_t>(stop_ids.size())));
}
gpu::ConstDeviceRegion DeviceCategorical::submit_next(gpu::ConstDeviceRegion row) {
  gpu::hip::check(dl_sampler_submit_next(impl_->sampler, BackendAccess::address(row), row.bytes));
  return result_storage();
}
gpu::ConstDeviceRegion DeviceCategorical::current_token() const {
  return {&impl_->token, 0, impl_->token.size_bytes()};
}
gpu::ConstDeviceRegion DeviceCategorical::result_storage() const {
  return {&impl_->result, 0, impl_->result.size_bytes()};
}
gpu::ConstDeviceRegion DeviceCategorical::terminal_state() const {
  return {&impl_->terminal, 0, impl_->terminal.size_bytes()};
}

}  // namespace dolittle::inference::sampling

namespace dolittle::inference::hip {

// DeviceSequence::collect (decoding/device.h:136; decode.cu:579-610) over a
// plan's journal: polls event `index` of `sequence` without blocking the
// device, forwarding a stop request of the caller's token to the loop.
DeviceSequence::Event collect(dl_plan* plan, std::uint32_t sequence, std::size_t index,
                              const std::stop_token& stop) {
  dl_sequence_event e{};
  bool forwarded = false;
  for (;;) {
    if (!forwarded && stop.stop_requested()) {
      gpu::hip::check(dl_plan_request_stop(plan));
      forwarded = true;
    }
    int ready = 0;
    gpu::hip::check(dl_plan_collect_event(plan, sequence, index, 0, &e, &ready));
    if (ready) break;
    std::this_thread::sleep_for(std::chrono::microseconds(50));
  }
  DeviceSequence::Event out;
  out.kind = static_cast<DeviceSequence::Kind>(e.kind);
  out.status = e.status;
  out.position = e.position;
  out.count = e.count;
  out.token = e.token;
  out.norm = e.norm;
  return out;
}

static_assert(sizeof(dl_sequence_event) == sequence_event_bytes, "the reference's 32-byte event");
static_assert(static_cast<int>(DeviceSequence::Kind::consumed) == 0 &&
                  static_cast<int>(DeviceSequence::Kind::selected) == 1 &&
                  static_cast<int>(DeviceSequence::Kind::terminal) == 2 &&
                  static_cast<int>(DeviceSequence::Kind::injection) == 3,
              "event kinds as the journal writes them");
static_assert(static_cast<int>(DeviceSequence::Reason::limit) == 0 &&
                  static_cast<int>(DeviceSequence::Reason::eos) == 1 &&
                  static_cast<int>(DeviceSequence::Reason::cancelled) == 2 &&
                  static_cast<int>(DeviceSequence::Reason::failure) == 3,
              "terminal reasons as the journal writes them");

}  // namespace dolittle::inference::hip
