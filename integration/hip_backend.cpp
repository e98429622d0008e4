// HIP backend of Dolittle's device interfaces over libdlhip.so: the file a
// maintainer adds to the reference tree (as src/gpu/hip/backend.cpp, in
// place of src/gpu/cuda/*.cpp and src/kernels/cuda/*) to run the reference's
// executor, generation loop, sampler, sequence and NLA users on the C ABI of
// include/dolittle_hip.h.
//
// Interfaces implemented, member by member:
//   src/gpu/device.h:73-184                 DeviceBuffer, HostBuffer, Queue, Device
//   src/kernels/operations.h:204-271        prepare, PreparedOperation
//   src/inference/sampling/device.h:54-85   DeviceCategorical
//   src/inference/decoding/device.h:84-137  DeviceSequence
//   src/inference/injection/device.h:26-47  DeviceInjection
//   src/inference/steering/device.h:30-68   DeviceDirection, DeviceIntervention
// plus dolittle::gpu::hip::open_device (the counterpart of
// src/gpu/cuda/device.h:29) and dolittle::inference::hip::collect, the
// journal reader of the Qwen3 plan (dl_plan).
// Build:
//   g++ -std=c++20 -fPIC -shared -I<reference>/src -Iinclude integration/hip_backend.cpp
//       -Ldolittle_amd -ldlhip -Wl,--no-undefined -o libdolittle_hip_backend.so
// (validate_operation, element_bytes and required_bytes come from the
// reference's own kernels/operations.cpp and tensors/tensor.cpp when the
// adapter is linked into the reference's library).

#include <algorithm>
#include <array>
#include <chrono>
#include <cmath>
#include <cstring>
#include <limits>
#include <stdexcept>
#include <stop_token>
#include <string>
#include <thread>
#include <type_traits>
#include <utility>
#include <variant>
#include <vector>

#include "dolittle_hip.h"
#include "gpu/device.h"
#include "inference/cache/contiguous.h"
#include "inference/decoding/device.h"
#include "inference/injection/device.h"
#include "inference/sampling/device.h"
#include "inference/steering/device.h"
#include "kernels/operations.h"
#include "tensors/tensor.h"

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
  static const void* address(ConstHostRegion r) { return checked(r.owner, r.offset, r.bytes).host + r.offset; }
  static void* address(HostRegion r) { return checked(r.owner, r.offset, r.bytes).host + r.offset; }
  // Device address of a whole buffer (owned or borrowed), checked live.
  static std::byte* base(const DeviceBuffer& buffer) {
    if (!buffer.impl_) throw std::invalid_argument("moved-from device buffer");
    return static_cast<std::byte*>(buffer.impl_->address);
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

// Every transfer goes by address (dl_queue_transfer), so borrowed regions
// such as DeviceCategorical's result words download like owned ones.
void Queue::upload(DeviceRegion destination, ConstHostRegion source) {
  same_size(destination.bytes, source.bytes);
  hip::check(dl_queue_transfer(BackendAccess::handle(*this), BackendAccess::address(destination),
                               BackendAccess::address(source), source.bytes));
}
void Queue::download(HostRegion destination, ConstDeviceRegion source) {
  same_size(destination.bytes, source.bytes);
  hip::check(dl_queue_transfer(BackendAccess::handle(*this), BackendAccess::address(destination),
                               BackendAccess::address(source), source.bytes));
}
void Queue::copy(DeviceRegion destination, ConstDeviceRegion source) {
  same_size(destination.bytes, source.bytes);
  hip::check(dl_queue_transfer(BackendAccess::handle(*this), BackendAccess::address(destination),
                               BackendAccess::address(source), source.bytes));
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

// The sampler's arena is the library's; the {token, status} result words and
// the terminal word are exposed as borrowed device regions for graph readers
// and copies (the current token is the result's first word).
struct DeviceCategorical::Impl {
  Impl(dl_sampler* s, std::size_t n, void* result_word, void* terminal_word)
      : sampler(s),
        vocabulary(n),
        result(BackendAccess::borrow(result_word, 2 * sizeof(std::uint32_t))),
        terminal(BackendAccess::borrow(terminal_word, sizeof(std::uint32_t))) {}
  ~Impl() { dl_sampler_destroy(sampler); }
  Impl(const Impl&) = delete;
  Impl& operator=(const Impl&) = delete;
  dl_sampler* sampler;
  std::size_t vocabulary;
  gpu::DeviceBuffer result, terminal;
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
  void *result = nullptr, *terminal = nullptr;
  int status = dl_sampler_result_address(sampler, &result);
  if (status == DL_OK) status = dl_sampler_terminal_address(sampler, &terminal);
  if (status != DL_OK) {
    dl_sampler_destroy(sampler);
    gpu::hip::check(status);
  }
  impl_ = std::make_unique<Impl>(sampler, vocabulary, result, terminal);
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
// Only after a selection (sampling.cu current_token: logic_error before).
gpu::ConstDeviceRegion DeviceCategorical::current_token() const {
  void* token = nullptr;
  const int status = dl_sampler_current_token_address(impl_->sampler, &token);
  if (status == DL_INVALID_ARGUMENT) throw std::logic_error(dl_last_error());
  gpu::hip::check(status);
  return {&impl_->result, 0, sizeof(std::uint32_t)};
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

// ----------------------------------------------------- operation catalog
namespace dolittle::kernels {

using gpu::detail::BackendAccess;

namespace {
void require(bool value, const char* message) {
  if (!value) throw std::invalid_argument(message);
}
std::size_t product(std::size_t a, std::size_t b) {
  if (b && a > std::numeric_limits<std::size_t>::max() / b) throw std::length_error("prepared size overflows");
  return a * b;
}
int native_type(tensors::ElementType t) { return t == tensors::ElementType::bfloat16 ? DL_BF16 : DL_F32; }

// A bound operand: owner, device address and byte extent.
struct Bound {
  const gpu::DeviceBuffer* owner = nullptr;
  std::byte* address = nullptr;
  std::size_t offset = 0, bytes = 0;
};
}  // namespace

// The descriptor copied at preparation with its flattened dimensions:
//   Embedding {rows, width, vocabulary}, Projection {rows, in, out},
//   RmsNorm {rows, width}, Rotary {positions, heads, width},
//   CausalAttention {positions, query heads, kv heads, width},
//   Add / SiluMultiply {elements}, GatherRows {row bytes}.
// Nothing the device reads belongs to it (the operations take their
// operands as launch arguments), so destruction needs no drain.
struct PreparedOperation::Impl {
  gpu::Device* device;
  Operation operation;
  tensors::ElementType type;
  std::vector<OperandRequirement> requirements;
  std::vector<std::size_t> extents;
  std::array<std::size_t, 4> dims{};
  RowPolicy rows;
};

PreparedOperation::PreparedOperation(std::unique_ptr<Impl> impl) : impl_(std::move(impl)) {}
PreparedOperation::~PreparedOperation() = default;
PreparedOperation::PreparedOperation(PreparedOperation&&) noexcept = default;
PreparedOperation& PreparedOperation::operator=(PreparedOperation&&) noexcept = default;

// Only attention keeps a device constant: its FP32 1/sqrt(width)
// (src/kernels/cuda/operations.cpp:151-155).
WorkspaceRequirement PreparedOperation::workspace() const noexcept {
  return std::holds_alternative<CausalAttention>(impl_->operation) ? WorkspaceRequirement{sizeof(float), alignof(float)}
                                                                   : WorkspaceRequirement{0, 1};
}

void PreparedOperation::initialize(gpu::Queue& queue, gpu::DeviceRegion region) const {
  const auto need = workspace();
  require(region.bytes == need.bytes, "constant region size mismatch");
  if (!region.bytes) return;
  require(region.owner && region.offset % need.alignment == 0, "invalid constant region");
  auto* scale = static_cast<float*>(BackendAccess::address(region));
  gpu::hip::check(dl_attention_scale(BackendAccess::handle(queue), scale, impl_->dims[3]));
}

std::span<const OperandRequirement> PreparedOperation::operands() const noexcept { return impl_->requirements; }

std::string_view PreparedOperation::implementation_name() const noexcept {
  return "hip-gfx950-exact-fp32-accumulation";
}

PreparedOperation prepare(gpu::Device& device, const Operation& operation, std::span<const tensors::Layout> layouts,
                          tensors::ComputationMode mode, RowPolicy rows) {
  const auto uses = validate_operation(operation, layouts, mode);
  (void)gpu::hip::handle(device);  // a HIP device, or invalid_argument
  auto impl = std::make_unique<PreparedOperation::Impl>();
  impl->device = &device;
  impl->operation = operation;
  impl->type = mode.activation_storage;
  impl->rows = rows;
  for (const auto& use : uses) {
    const auto& layout = layouts[use.tensor.value];
    impl->requirements.push_back({use.tensor, use.access, tensors::element_bytes(layout.element_type)});
    impl->extents.push_back(tensors::required_bytes(layout));
  }
  auto& d = impl->dims;
  const auto layout = [&](TensorId id) -> const tensors::Layout& { return layouts[id.value]; };
  const auto elements = [&](TensorId id) {
    return tensors::required_bytes(layout(id)) / tensors::element_bytes(layout(id).element_type);
  };
  std::visit(
      [&](const auto& op) {
        using T = std::decay_t<decltype(op)>;
        if constexpr (std::is_same_v<T, Embedding>) {
          d = {layout(op.tokens).shape.at(0), layout(op.weight).shape.at(1), layout(op.weight).shape.at(0), 0};
        } else if constexpr (std::is_same_v<T, Projection>) {
          d = {layout(op.input).shape.at(0), layout(op.weight).shape.at(1), layout(op.weight).shape.at(0), 0};
        } else if constexpr (std::is_same_v<T, RmsNorm>) {
          d[1] = layout(op.input).shape.back();
          d[0] = elements(op.input) / d[1];
        } else if constexpr (std::is_same_v<T, Rotary>) {
          const auto& shape = layout(op.input).shape;
          d = {shape.at(0), shape.at(1), shape.at(2), 0};
          require(std::isfinite(static_cast<float>(op.theta)) && static_cast<float>(op.theta) > 0,
                  "RoPE theta must fit a positive FP32 value");
        } else if constexpr (std::is_same_v<T, CausalAttention>) {
          const auto& shape = layout(op.query).shape;
          d = {shape.at(0), shape.at(1), layout(op.key).shape.at(1), shape.at(2)};
        } else if constexpr (std::is_same_v<T, Add>) {
          d[0] = elements(op.left);
        } else if constexpr (std::is_same_v<T, SiluMultiply>) {
          d[0] = elements(op.gate);
        } else if constexpr (std::is_same_v<T, GatherRows>) {
          d[0] = tensors::required_bytes(layout(op.input)) / layout(op.input).shape.at(0);
        }
      },
      operation);
  if (rows.last_row) {
    const auto* gather = std::get_if<GatherRows>(&operation);
    require(rows.max_rows && gather && gather->rows == std::vector<std::size_t>{rows.max_rows - 1},
            "last-row policy requires a final-row gather");
  } else if (rows.max_rows) {
    require(!std::holds_alternative<GatherRows>(operation), "dynamic gather requires last-row policy");
    // Every operand but a weight leads with the admitted row count.
    for (const auto& use : uses) {
      const bool weight = std::visit(
          [&](const auto& op) {
            using T = std::decay_t<decltype(op)>;
            if constexpr (std::is_same_v<T, Embedding> || std::is_same_v<T, Projection> ||
                          std::is_same_v<T, RmsNorm>)
              return use.tensor.value == op.weight.value;
            else
              return false;
          },
          operation);
      require(weight || layouts[use.tensor.value].shape.at(0) == rows.max_rows,
              "dynamic operation leading dimension mismatch");
    }
  }
  return PreparedOperation(std::move(impl));
}

void PreparedOperation::submit(gpu::Queue& queue, std::span<const BufferBinding> bindings,
                               gpu::DeviceRegion workspace_region, const ExecutionExtent* extent,
                               const inference::cache::ContiguousLayerView* cache) const {
  const auto& p = *impl_;
  dl_queue* q = BackendAccess::handle(queue);
  const bool dynamic = p.rows.max_rows != 0;
  require(dynamic == (extent != nullptr), "runtime extent/preparation mismatch");
  if (extent) {
    require(extent->active_rows && extent->active_rows <= p.rows.max_rows, "active rows outside prepared capacity");
    require(extent->first_position <= std::numeric_limits<std::size_t>::max() - extent->active_rows,
            "runtime positions overflow");
  }
  const bool attention = std::holds_alternative<CausalAttention>(p.operation);
  require(!cache || (dynamic && attention), "cache binding requires dynamic attention");
  require(!dynamic || !attention || cache, "dynamic attention requires an initialized cache prefix");
  require(bindings.size() == p.requirements.size(), "binding count differs from operation");
  require(workspace_region.bytes == workspace().bytes, "operation constant size mismatch");
  const float* scale = nullptr;
  if (workspace_region.bytes) {
    require(workspace_region.owner && workspace_region.offset % alignof(float) == 0,
            "invalid operation constant region");
    scale = static_cast<const float*>(BackendAccess::address(workspace_region));
  }
  const std::uint64_t* device_position = nullptr;
  if (extent && extent->device_position) {
    const auto region = *extent->device_position;
    require(extent->device_capacity && extent->active_rows <= extent->device_capacity && region.owner &&
                region.bytes == sizeof(std::size_t) && region.offset % alignof(std::size_t) == 0,
            "invalid device position binding");
    device_position = static_cast<const std::uint64_t*>(BackendAccess::address(region));
  }

  // One binding per distinct operand, exact extents, mutable outputs,
  // natural alignment; a positioned output spans the device capacity.
  std::vector<Bound> bound(p.requirements.size());
  std::vector<bool> positioned(p.requirements.size(), false);
  for (std::size_t i = 0; i < p.requirements.size(); ++i) {
    const auto& need = p.requirements[i];
    const BufferBinding* match = nullptr;
    for (const auto& candidate : bindings) {
      if (candidate.tensor.value == need.tensor.value) {
        require(match == nullptr, "duplicate tensor binding");
        match = &candidate;
      }
    }
    require(match != nullptr, "missing tensor binding");
    const auto* owner = std::visit([](auto* b) -> const gpu::DeviceBuffer* { return b; }, match->storage);
    require(owner != nullptr, "null tensor storage");
    if (need.access == OperandAccess::write)
      require(std::holds_alternative<gpu::DeviceBuffer*>(match->storage), "write operand has immutable storage");
    if (match->offset > std::numeric_limits<std::size_t>::max() - match->bytes)
      throw std::length_error("binding extent overflows");
    require(match->bytes == p.extents[i] && match->offset <= owner->size_bytes() &&
                match->bytes <= owner->size_bytes() - match->offset,
            "tensor binding extent mismatch");
    std::size_t bytes = match->bytes;
    if (match->positioned_output) {
      require(device_position && need.access == OperandAccess::write &&
                  (std::holds_alternative<Projection>(p.operation) || std::holds_alternative<Rotary>(p.operation)),
              "positioned binding requires a cache producer");
      bytes = product(match->bytes / p.rows.max_rows, extent->device_capacity);
      require(bytes <= owner->size_bytes() - match->offset, "positioned output capacity exceeds allocation");
      positioned[i] = true;
    }
    std::byte* address = BackendAccess::base(*owner) + match->offset;
    require(reinterpret_cast<std::uintptr_t>(address) % need.alignment == 0, "tensor binding alignment mismatch");
    bound[i] = {owner, address, match->offset, bytes};
  }
  for (std::size_t i = 0; i < bound.size(); ++i)
    for (std::size_t j = i + 1; j < bound.size(); ++j)
      if (bound[i].owner == bound[j].owner && (p.requirements[i].access == OperandAccess::write ||
                                               p.requirements[j].access == OperandAccess::write))
        require(bound[i].offset >= bound[j].offset + bound[j].bytes ||
                    bound[j].offset >= bound[i].offset + bound[i].bytes,
                "write operand overlaps another operand");
  const auto operand = [&](TensorId id) -> std::size_t {
    for (std::size_t i = 0; i < p.requirements.size(); ++i)
      if (p.requirements[i].tensor.value == id.value) return i;
    throw std::logic_error("prepared operand is absent");
  };
  const auto at = [&](TensorId id) { return bound[operand(id)].address; };

  auto d = p.dims;
  if (dynamic && !p.rows.last_row) d[0] = (d[0] / p.rows.max_rows) * extent->active_rows;
  const void* keys = nullptr;
  const void* values = nullptr;
  if (cache) {
    require((!device_position || extent->device_capacity == cache->capacity) &&
                extent->first_position <= cache->capacity &&
                extent->active_rows <= cache->capacity - extent->first_position && cache->shape.kv_heads == d[2] &&
                cache->shape.head_width == d[3],
            "cached attention shape mismatch");
    const auto bytes = product(product(product(cache->capacity, d[2]), d[3]), tensors::element_bytes(p.type));
    const auto view = [&](gpu::ConstDeviceRegion region) -> const void* {
      require(region.owner && region.bytes == bytes, "cache region extent mismatch");
      const void* address = BackendAccess::address(region);
      require(reinterpret_cast<std::uintptr_t>(address) % tensors::element_bytes(p.type) == 0,
              "cache alignment mismatch");
      for (std::size_t i = 0; i < bound.size(); ++i)
        if (p.requirements[i].access == OperandAccess::write && bound[i].owner == region.owner)
          require(bound[i].offset >= region.offset + bytes || region.offset >= bound[i].offset + bound[i].bytes,
                  "attention output overlaps cache");
      return address;
    };
    keys = view(cache->keys);
    values = view(cache->values);
  }
  const int type = native_type(p.type);
  const std::size_t first = extent ? extent->first_position : 0;
  std::visit(
      [&](const auto& op) {
        using T = std::decay_t<decltype(op)>;
        int status = DL_OK;
        if constexpr (std::is_same_v<T, Embedding>) {
          status = dl_embedding(q, type, reinterpret_cast<const std::uint32_t*>(at(op.tokens)), at(op.weight),
                                at(op.output), d[0], d[1], d[2]);
        } else if constexpr (std::is_same_v<T, Projection>) {
          status = dl_projection(q, type, at(op.input), at(op.weight), at(op.output), d[0], d[1], d[2],
                                 positioned[operand(op.output)] ? device_position : nullptr);
        } else if constexpr (std::is_same_v<T, RmsNorm>) {
          status = dl_rms_norm(q, type, at(op.input), at(op.weight), at(op.output), d[0], d[1], op.epsilon);
        } else if constexpr (std::is_same_v<T, Rotary>) {
          status = dl_rotary(q, type, at(op.input), at(op.output), d[0], d[1], d[2],
                             extent ? first : op.first_position, op.theta, device_position,
                             positioned[operand(op.output)] ? 1 : 0);
        } else if constexpr (std::is_same_v<T, CausalAttention>) {
          status = dl_attention(q, type, at(op.query), cache ? keys : at(op.key), cache ? values : at(op.value),
                                at(op.output), d[0], d[1], d[2], d[3], first, device_position,
                                cache ? cache->capacity : 0, scale);
        } else if constexpr (std::is_same_v<T, Add>) {
          status = dl_add(q, type, at(op.left), at(op.right), at(op.output), d[0]);
        } else if constexpr (std::is_same_v<T, SiluMultiply>) {
          status = dl_silu_multiply(q, type, at(op.gate), at(op.up), at(op.output), d[0]);
        } else if constexpr (std::is_same_v<T, GatherRows>) {
          std::byte* source = at(op.input);
          std::byte* destination = at(op.output);
          if (p.rows.last_row) {
            status = dl_queue_transfer(q, destination, source + (extent->active_rows - 1) * d[0], d[0]);
          } else {
            // One ordered copy per maximal run of consecutive rows.
            for (std::size_t r = 0; r < op.rows.size() && status == DL_OK;) {
              std::size_t end = r + 1;
              while (end < op.rows.size() && op.rows[end] == op.rows[end - 1] + 1) ++end;
              status = dl_queue_transfer(q, destination + r * d[0], source + op.rows[r] * d[0], (end - r) * d[0]);
              r = end;
            }
          }
        }
        gpu::hip::check(status);
      },
      p.operation);
}

}  // namespace dolittle::kernels

// ------------------------------------------------------- DeviceSequence
namespace dolittle::inference {

using gpu::detail::BackendAccess;

namespace {
// Stage-order and state misuse is logic_error in the reference
// (decode.cu:444-559); region bounds are invalid_argument.
void check_order(bool ok, const char* message) {
  if (!ok) throw std::logic_error(message);
}
std::uint64_t event_capacity(const DeviceSequence::Shape& s) { return s.prompt + 2 * s.generated + 2; }
}  // namespace

struct DeviceSequence::Impl {
  gpu::Queue& queue;
  Shape shape;
  dl_sequence* sequence = nullptr;
  gpu::DeviceBuffer position;  // borrowed: the sequence's device position word
  int next_stage = 0;
  Stage stage{};
  bool begun = false, in_stage = false, selection = false, completed = false, started = false;
  Impl(gpu::Queue& q, Shape s, dl_sequence* seq, void* position_word)
      : queue(q), shape(s), sequence(seq), position(BackendAccess::borrow(position_word, sizeof(std::size_t))) {}
  ~Impl() { dl_sequence_destroy(sequence); }  // stops, joins, drains; never throws
  Impl(const Impl&) = delete;
  Impl& operator=(const Impl&) = delete;
};

std::size_t DeviceSequence::device_bytes() {
  std::uint64_t bytes = 0;
  gpu::hip::check(dl_sequence_device_bytes(&bytes));
  return bytes;
}

std::size_t DeviceSequence::host_bytes(Shape s) {
  std::uint64_t bytes = 0;
  gpu::hip::check(dl_sequence_host_bytes(s.prompt, s.generated, s.chunk, &bytes));
  return bytes;
}

DeviceSequence::DeviceSequence(gpu::Device& device, gpu::Queue& queue, Shape shape) {
  (void)gpu::hip::handle(device);
  dl_sequence* sequence = nullptr;
  gpu::hip::check(dl_sequence_create(BackendAccess::handle(queue), shape.prompt, shape.generated, shape.chunk,
                                     shape.forward_only ? 1 : 0, &sequence));
  void* position = nullptr;
  const int status = dl_sequence_position_address(sequence, &position);
  if (status != DL_OK) {
    dl_sequence_destroy(sequence);
    gpu::hip::check(status);
  }
  impl_ = std::make_unique<Impl>(queue, shape, sequence, position);
}

DeviceSequence::~DeviceSequence() = default;

gpu::ConstDeviceRegion DeviceSequence::position() const { return {&impl_->position, 0, sizeof(std::size_t)}; }

void DeviceSequence::begin(gpu::ConstDeviceRegion selection, gpu::ConstDeviceRegion terminal,
                           gpu::DeviceRegion token_input, gpu::ConstDeviceRegion prompt,
                           gpu::ConstDeviceRegion injection_status, gpu::ConstDeviceRegion injection_norm,
                           gpu::ConstDeviceRegion intervention_status, gpu::ConstDeviceRegion intervention_count) {
  auto& p = *impl_;
  const auto& s = p.shape;
  const bool words = s.forward_only ? (!s.generated && !selection.owner && !terminal.owner)
                                    : (selection.bytes == 2 * sizeof(std::uint32_t) &&
                                       terminal.bytes == sizeof(std::uint32_t));
  check_order(!p.begun && words && token_input.bytes >= s.chunk * sizeof(std::uint32_t) &&
                  prompt.bytes == s.prompt * sizeof(std::uint32_t) && selection.offset % 4 == 0 &&
                  terminal.offset % 4 == 0 && token_input.offset % 4 == 0 && prompt.offset % 4 == 0,
              "invalid sequence begin");
  const std::uint32_t *iv_status = nullptr, *iv_count = nullptr, *inj_status = nullptr;
  const float* inj_norm = nullptr;
  if (intervention_status.owner || intervention_count.owner) {
    if (intervention_status.bytes != sizeof(std::uint32_t) || intervention_count.bytes != sizeof(std::uint32_t) ||
        intervention_status.offset % 4 || intervention_count.offset % 4)
      throw std::invalid_argument("intervention control bounds");
    iv_status = static_cast<const std::uint32_t*>(BackendAccess::address(intervention_status));
    iv_count = static_cast<const std::uint32_t*>(BackendAccess::address(intervention_count));
  }
  if (injection_status.owner) {
    if (injection_status.bytes != sizeof(std::uint32_t) || injection_norm.bytes != sizeof(float) ||
        injection_status.offset % 4 || injection_norm.offset % 4)
      throw std::invalid_argument("invalid injection controls");
    inj_status = static_cast<const std::uint32_t*>(BackendAccess::address(injection_status));
    inj_norm = static_cast<const float*>(BackendAccess::address(injection_norm));
  }
  gpu::hip::check(dl_sequence_begin(
      p.sequence, s.forward_only ? nullptr : static_cast<const std::uint32_t*>(BackendAccess::address(selection)),
      s.forward_only ? nullptr : static_cast<const std::uint32_t*>(BackendAccess::address(terminal)),
      static_cast<std::uint32_t*>(BackendAccess::address(token_input)), token_input.bytes,
      static_cast<const std::uint32_t*>(BackendAccess::address(prompt)), prompt.bytes, inj_status, inj_norm,
      iv_status, iv_count));
  p.begun = true;
}

void DeviceSequence::begin_stage(Stage stage) {
  auto& p = *impl_;
  check_order(p.begun && !p.in_stage && static_cast<int>(stage) == p.next_stage, "invalid sequence stage order");
  gpu::hip::check(dl_sequence_begin_stage(p.sequence, static_cast<int>(stage)));
  p.stage = stage;
  p.in_stage = true;
}

void DeviceSequence::begin_selection() {
  auto& p = *impl_;
  check_order(p.in_stage && p.stage == Stage::decode && !p.selection, "invalid decode selection branch");
  gpu::hip::check(dl_sequence_begin_selection(p.sequence));
  p.selection = true;
}

void DeviceSequence::end_stage() {
  auto& p = *impl_;
  check_order(p.in_stage, "no sequence stage");
  check_order(p.stage != Stage::decode || p.selection, "missing selection tail");
  gpu::hip::check(dl_sequence_end_stage(p.sequence));
  p.in_stage = false;
  ++p.next_stage;
}

void DeviceSequence::capture(gpu::ConstDeviceRegion source, gpu::DeviceRegion destination, std::size_t row_bytes,
                             std::size_t rows) {
  auto& p = *impl_;
  check_order(p.stage != Stage::first_selection && !p.selection, "capture requires a consumption body");
  const auto capacity = p.shape.prompt + p.shape.generated;
  if (!p.in_stage || !row_bytes || !rows || rows > p.shape.chunk ||
      row_bytes > std::numeric_limits<std::size_t>::max() / capacity || source.bytes != rows * row_bytes ||
      destination.bytes != capacity * row_bytes)
    throw std::invalid_argument("invalid sequence capture bounds");
  gpu::hip::check(dl_sequence_capture(p.sequence, BackendAccess::address(source), source.bytes,
                                      BackendAccess::address(destination), destination.bytes, row_bytes, rows));
}

void DeviceSequence::replace(gpu::ConstDeviceRegion row, gpu::DeviceRegion embeddings, std::size_t marker,
                             std::size_t rows) {
  auto& p = *impl_;
  if (!p.in_stage || marker >= p.shape.prompt || !rows || !row.bytes || row.bytes > embeddings.bytes / rows)
    throw std::invalid_argument("embedding override bounds");
  gpu::hip::check(dl_sequence_replace(p.sequence, BackendAccess::address(row), row.bytes,
                                      BackendAccess::address(embeddings), embeddings.bytes, marker, rows));
}

void DeviceSequence::complete() {
  auto& p = *impl_;
  check_order(p.next_stage == 4 && !p.in_stage && !p.completed, "incomplete sequence");
  gpu::hip::check(dl_sequence_complete(p.sequence));
  p.completed = true;
}

PreparedSequenceResources DeviceSequence::prepared_resources() const {
  check_order(impl_->completed, "sequence not prepared");
  std::uint64_t device = 0, host = 0;
  gpu::hip::check(dl_sequence_resources(impl_->sequence, &device, &host));
  return {{device, host + sizeof(Impl), 0}, 0};
}

void DeviceSequence::start() {
  auto& p = *impl_;
  check_order(p.completed && !p.started, "sequence start");
  gpu::hip::check(dl_sequence_start(p.sequence));
  p.started = true;
}

void DeviceSequence::request_stop() noexcept { (void)dl_sequence_request_stop(impl_->sequence); }

void DeviceSequence::drain() { gpu::hip::check(dl_sequence_drain(impl_->sequence)); }

DeviceSequence::Event DeviceSequence::collect(std::size_t index, const std::stop_token& stop) {
  auto& p = *impl_;
  check_order(p.started && index < event_capacity(p.shape), "event outside sequence");
  dl_sequence_event e{};
  bool forwarded = false;
  for (;;) {
    if (!forwarded && stop.stop_requested()) {
      request_stop();
      forwarded = true;
    }
    int ready = 0;
    gpu::hip::check(dl_sequence_collect(p.sequence, index, 0, &e, &ready));
    if (ready) break;
    std::this_thread::sleep_for(std::chrono::microseconds(100));
  }
  Event out;
  out.kind = static_cast<Kind>(e.kind);
  out.status = e.status;
  out.position = e.position;
  out.count = e.count;
  out.token = e.token;
  out.norm = e.norm;
  return out;
}

// --------------------------------------------------------- NLA objects
namespace {
// Storage of the injection (dl_injection_submit): [norm FP32][status
// uint32][output row], the layout of injection.cu's output_offset = 8.
constexpr std::size_t kInjectionRow = 8;
// DeviceDirection storage (dl_direction_submit): [status][pad][FP32 vector].
constexpr std::size_t kDirectionVector = 8;

gpu::DeviceBuffer allocate(gpu::Device& device, std::size_t bytes) { return device.allocate({bytes, 4}); }

// A naturally aligned region of at least `bytes`, or invalid_argument.
const void* region_address(gpu::ConstDeviceRegion r, std::size_t bytes, std::size_t alignment) {
  if (!r.owner || r.bytes < bytes || r.offset % alignment) throw std::invalid_argument("invalid NLA region");
  return BackendAccess::address(gpu::ConstDeviceRegion{r.owner, r.offset, bytes});
}
}  // namespace

struct DeviceInjection::Impl {
  gpu::Queue& queue;
  gpu::ConstDeviceRegion source;
  tensors::ElementType input, output;
  std::size_t width;
  float scale;
  gpu::DeviceBuffer storage;
};

std::size_t DeviceInjection::required_bytes(std::size_t width, tensors::ElementType type) {
  if (type != tensors::ElementType::float32 && type != tensors::ElementType::bfloat16)
    throw std::invalid_argument("unsupported injection type");
  std::uint64_t bytes = 0;
  gpu::hip::check(dl_injection_bytes(width, type == tensors::ElementType::bfloat16 ? DL_BF16 : DL_F32, &bytes));
  return bytes;
}

DeviceInjection::DeviceInjection(gpu::Device& device, gpu::Queue& queue, gpu::ConstDeviceRegion source,
                                 tensors::ElementType source_type, tensors::ElementType output_type,
                                 std::size_t width, float scale) {
  const auto expected = required_bytes(width, source_type) - kInjectionRow;
  if (!source.owner || source.offset % tensors::element_bytes(source_type) || source.bytes != expected ||
      !std::isfinite(scale) || scale <= 0)
    throw std::invalid_argument("invalid injection source");
  (void)BackendAccess::address(source);
  (void)BackendAccess::handle(queue);
  impl_ = std::unique_ptr<Impl>(new Impl{queue, source, source_type, output_type, width, scale,
                                         allocate(device, required_bytes(width, output_type))});
}

DeviceInjection::~DeviceInjection() = default;

void DeviceInjection::submit() {
  auto& p = *impl_;
  gpu::hip::check(dl_injection_submit(BackendAccess::handle(p.queue), BackendAccess::address(p.source),
                                      p.input == tensors::ElementType::bfloat16 ? DL_BF16 : DL_F32,
                                      p.output == tensors::ElementType::bfloat16 ? DL_BF16 : DL_F32, p.width,
                                      p.scale, BackendAccess::base(p.storage)));
}

gpu::ConstDeviceRegion DeviceInjection::output() const {
  return {&impl_->storage, kInjectionRow, impl_->storage.size_bytes() - kInjectionRow};
}
gpu::ConstDeviceRegion DeviceInjection::norm() const { return {&impl_->storage, 0, sizeof(float)}; }
gpu::ConstDeviceRegion DeviceInjection::status() const {
  return {&impl_->storage, sizeof(float), sizeof(std::uint32_t)};
}

struct DeviceDirection::Impl {
  gpu::Queue& queue;
  DeviceCapture original, edited;
  tensors::ElementType type;
  std::size_t width;
  std::shared_ptr<gpu::DeviceBuffer> storage;
  gpu::HostBuffer readback;
  bool submitted = false, finished = false;
  ~Impl() { (void)dl_queue_drain(BackendAccess::handle(queue)); }
};

std::size_t DeviceDirection::required_bytes(std::size_t width) {
  std::uint64_t bytes = 0;
  gpu::hip::check(dl_direction_bytes(width, &bytes));
  return bytes;
}

DeviceDirection::DeviceDirection(gpu::Device& device, gpu::Queue& queue, DeviceCapture original,
                                 DeviceCapture edited, tensors::ElementType type, std::size_t width) {
  (void)required_bytes(width);
  if (type != tensors::ElementType::bfloat16 && type != tensors::ElementType::float32)
    throw std::invalid_argument("steering storage type");
  const auto element = tensors::element_bytes(type);
  (void)region_address(original.region(), width * element, element);
  (void)region_address(edited.region(), width * element, element);
  auto storage = std::make_shared<gpu::DeviceBuffer>(allocate(device, required_bytes(width)));
  auto readback = device.allocate_staging({sizeof(std::uint32_t), alignof(std::uint32_t)});
  impl_ = std::unique_ptr<Impl>(new Impl{queue, std::move(original), std::move(edited), type, width,
                                         std::move(storage), std::move(readback)});
}

DeviceDirection::~DeviceDirection() = default;

void DeviceDirection::submit() {
  auto& p = *impl_;
  check_order(!p.submitted, "direction already submitted");
  const auto element = tensors::element_bytes(p.type);
  gpu::hip::check(dl_direction_submit(BackendAccess::handle(p.queue),
                                      region_address(p.original.region(), p.width * element, element),
                                      region_address(p.edited.region(), p.width * element, element),
                                      p.type == tensors::ElementType::bfloat16 ? DL_BF16 : DL_F32, p.width,
                                      BackendAccess::base(*p.storage)));
  p.submitted = true;
}

DeviceCapture DeviceDirection::finish() {
  auto& p = *impl_;
  check_order(p.submitted && !p.finished, "direction completion state");
  p.queue.download({&p.readback, 0, sizeof(std::uint32_t)}, {p.storage.get(), 0, sizeof(std::uint32_t)});
  p.queue.drain();
  std::uint32_t status = 0;
  std::memcpy(&status, p.readback.bytes().data(), sizeof status);
  if (status) throw std::invalid_argument("reconstructions have zero or nonfinite difference");
  p.finished = true;
  return {p.storage, kDirectionVector, p.width * sizeof(float)};
}

struct DeviceIntervention::Impl {
  gpu::Queue& queue;
  ResidualIntervention input;
  tensors::ElementType type;
  gpu::DeviceBuffer state;
  ~Impl() { (void)dl_queue_drain(BackendAccess::handle(queue)); }
};

DeviceIntervention::DeviceIntervention(gpu::Device& device, gpu::Queue& queue, ResidualIntervention input,
                                       tensors::ElementType type) {
  (void)DeviceDirection::required_bytes(input.width);
  (void)region_address(input.direction.region(), input.width * sizeof(float), alignof(float));
  if (!std::isfinite(input.strength) || input.strength < 0 ||
      (type != tensors::ElementType::bfloat16 && type != tensors::ElementType::float32))
    throw std::invalid_argument("invalid residual intervention");
  impl_ = std::unique_ptr<Impl>(new Impl{queue, std::move(input), type, allocate(device, required_bytes)});
}

DeviceIntervention::~DeviceIntervention() = default;

gpu::ConstDeviceRegion DeviceIntervention::status() const { return {&impl_->state, 0, sizeof(std::uint32_t)}; }
gpu::ConstDeviceRegion DeviceIntervention::count() const {
  return {&impl_->state, sizeof(std::uint32_t), sizeof(std::uint32_t)};
}

void DeviceIntervention::initialize() {
  gpu::hip::check(dl_intervention_initialize(BackendAccess::handle(impl_->queue),
                                             reinterpret_cast<std::uint32_t*>(BackendAccess::base(impl_->state))));
}

void DeviceIntervention::submit(gpu::DeviceRegion residual, gpu::ConstDeviceRegion position, std::size_t rows) {
  auto& p = *impl_;
  const auto element = tensors::element_bytes(p.type);
  if (!rows || rows > std::numeric_limits<std::size_t>::max() / p.input.width / element)
    throw std::length_error("intervention extent");
  if (!residual.owner || residual.bytes < rows * p.input.width * element || residual.offset % element)
    throw std::invalid_argument("invalid NLA region");
  gpu::hip::check(dl_intervention_submit(
      BackendAccess::handle(p.queue),
      BackendAccess::address(gpu::DeviceRegion{residual.owner, residual.offset, rows * p.input.width * element}),
      p.type == tensors::ElementType::bfloat16 ? DL_BF16 : DL_F32, rows, p.input.width,
      static_cast<const float*>(region_address(p.input.direction.region(), p.input.width * sizeof(float), 4)),
      static_cast<const std::uint64_t*>(region_address(position, sizeof(std::size_t), alignof(std::size_t))),
      p.input.position.value, p.input.strength, reinterpret_cast<std::uint32_t*>(BackendAccess::base(p.state))));
}

}  // namespace dolittle::inference
