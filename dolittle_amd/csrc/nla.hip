// Standalone device objects of the NLA protocol: DeviceInjection
// (src/inference/injection/device.h:29-47), DeviceDirection and
// DeviceIntervention (src/inference/steering/device.h:30-68).  Storage
// layouts are the reference's: injection [norm f32][status u32][output row],
// direction [status u32][u32][f32 row], intervention state [status][count].
#include <cmath>
#include <limits>

#include "dl_internal.h"
#include "nla.h"

namespace dl::nla {
namespace {

constexpr uint64_t kInjectionOutput = sizeof(float) + sizeof(uint32_t);
constexpr uint64_t kDirectionVector = 2 * sizeof(uint32_t);

uint64_t dtype_bytes(int dtype) { return dtype == DL_BF16 ? 2 : 4; }

// injection.cu:49-98: norm = sqrt(sum h^2) (eight strided lanes), then
// out[i] = narrow((h[i] / norm) * scale).  A nonfinite source value, a zero
// or nonfinite norm, or a nonfinite result (before or after narrowing)
// latches status; an invalid source writes no output.
template <class In, class Out>
__global__ __launch_bounds__(kThreads) void k_inject(const In* source, Out* output, float* norm, uint32_t* status,
                                                      uint64_t width, float scale) {
  __shared__ float sums[kLanes + 2];
  __shared__ uint32_t invalid;
  if (threadIdx.x == 0) invalid = 0;
  __syncthreads();
  const float sum = square_sum(width, [&](uint64_t i) {
    const float v = load_elem(source, i);
    if (!finite(v)) atomicOr(&invalid, 1u);
    return v;
  }, sums);
  if (threadIdx.x == 0) {
    const float n = __builtin_sqrtf(sum);
    *norm = n;
    sums[kLanes + 1] = n;
    if (!finite(n) || n == 0.0f) invalid = 1;
  }
  __syncthreads();
  const float n = sums[kLanes + 1];
  const bool valid = invalid == 0;  // before any output latch below
  __syncthreads();
  if (valid) {
    for (uint64_t i = threadIdx.x; i < width; i += blockDim.x) {
      const float value = __fmul_rn(__fdiv_rn(load_elem(source, i), n), scale);
      store_elem(output, i, value);
      if (!finite(value) || !finite(storage_round<Out>(value))) atomicOr(&invalid, 1u);
    }
  }
  __syncthreads();
  if (threadIdx.x == 0) *status = invalid;
}

// steering.cu:69-100: u = (edited - original) / ||edited - original||, FP32,
// every subtraction rounded separately; a zero or nonfinite norm latches
// status and writes no direction.
template <class In>
__global__ __launch_bounds__(kThreads) void k_direction(const In* original, const In* edited, float* direction,
                                                         uint32_t* status, uint64_t width) {
  __shared__ float sums[kLanes + 2];
  const float sum = square_sum(width, [&](uint64_t i) {
    return __fsub_rn(load_elem(edited, i), load_elem(original, i));
  }, sums);
  if (threadIdx.x == 0) {
    const float n = __builtin_sqrtf(sum);
    sums[kLanes + 1] = n;
    *status = (!finite(n) || n == 0.0f) ? 1u : 0u;
  }
  __syncthreads();
  const float n = sums[kLanes + 1];
  if (!finite(n) || n == 0.0f) return;
  for (uint64_t i = threadIdx.x; i < width; i += blockDim.x)
    direction[i] = __fdiv_rn(__fsub_rn(load_elem(edited, i), load_elem(original, i)), n);
}

__global__ void k_intervention_reset(uint32_t* state) {
  state[0] = 0;
  state[1] = 0;
}

// steering.cu:107-159: the residual chunk holds rows of absolute positions
// [*position, *position + rows); only the chunk holding `selected` updates
// that row.
template <class T>
__global__ __launch_bounds__(kThreads) void k_intervene(T* residual, const float* direction, const uint64_t* position,
                                                         uint32_t* state, uint64_t width, uint64_t selected,
                                                         uint64_t rows, float strength) {
  __shared__ float sums[kLanes + 2];
  __shared__ uint32_t invalid;
  const uint64_t first = *position;
  if (selected < first || selected - first >= rows) return;
  intervene_row(residual + (selected - first) * width, direction, state, width, strength, sums, &invalid);
}

}  // namespace
}  // namespace dl::nla

using dl::guard;
using dl::require;

extern "C" {

int dl_injection_bytes(uint64_t width, int output_dtype, uint64_t* bytes) {
  return guard([&] {
    require(bytes != nullptr, "null argument");
    require(output_dtype == DL_BF16 || output_dtype == DL_F32, "unsupported injection type");
    const uint64_t e = dl::nla::dtype_bytes(output_dtype);
    require(width > 0 && width <= (std::numeric_limits<uint64_t>::max() - dl::nla::kInjectionOutput) / e,
            "injection capacity", DL_LENGTH_ERROR);
    *bytes = dl::nla::kInjectionOutput + width * e;
  });
}

int dl_injection_submit(dl_queue* queue, const void* source, int source_dtype, int output_dtype, uint64_t width,
                        float scale, void* storage) {
  return guard([&] {
    dl::enter(queue);
    require(source && storage, "null operand");
    require((source_dtype == DL_BF16 || source_dtype == DL_F32) && (output_dtype == DL_BF16 || output_dtype == DL_F32),
            "unsupported injection type");
    require(width > 0, "empty injection", DL_LENGTH_ERROR);
    require(std::isfinite(scale) && scale > 0.0f, "invalid injection source");
    require(reinterpret_cast<uintptr_t>(storage) % 4 == 0 &&
                reinterpret_cast<uintptr_t>(source) % dl::nla::dtype_bytes(source_dtype) == 0,
            "misaligned injection region");
    auto* base = static_cast<uint8_t*>(storage);
    float* norm = reinterpret_cast<float*>(base);
    uint32_t* status = reinterpret_cast<uint32_t*>(base + sizeof(float));
    void* out = base + dl::nla::kInjectionOutput;
    auto launch = [&](auto in_tag, auto out_tag) {
      using In = decltype(in_tag);
      using Out = decltype(out_tag);
      dl::nla::k_inject<In, Out><<<1, dl::nla::kThreads, 0, queue->stream>>>(
          static_cast<const In*>(source), static_cast<Out*>(out), norm, status, width, scale);
    };
    if (source_dtype == DL_BF16) {
      if (output_dtype == DL_BF16) launch(uint16_t{}, uint16_t{});
      else launch(uint16_t{}, float{});
    } else {
      if (output_dtype == DL_BF16) launch(float{}, uint16_t{});
      else launch(float{}, float{});
    }
    dl::check_launch(queue, "injection");
  });
}

int dl_direction_bytes(uint64_t width, uint64_t* bytes) {
  return guard([&] {
    require(bytes != nullptr, "null argument");
    require(width > 0 && width <= (std::numeric_limits<uint64_t>::max() - dl::nla::kDirectionVector) / 4,
            "steering width", DL_LENGTH_ERROR);
    *bytes = dl::nla::kDirectionVector + width * 4;
  });
}

int dl_direction_submit(dl_queue* queue, const void* original, const void* edited, int dtype, uint64_t width,
                        void* storage) {
  return guard([&] {
    dl::enter(queue);
    require(original && edited && storage, "null operand");
    require(dtype == DL_BF16 || dtype == DL_F32, "steering storage type");
    require(width > 0, "steering width", DL_LENGTH_ERROR);
    require(reinterpret_cast<uintptr_t>(storage) % 4 == 0, "misaligned direction storage");
    auto* base = static_cast<uint8_t*>(storage);
    uint32_t* status = reinterpret_cast<uint32_t*>(base);
    float* direction = reinterpret_cast<float*>(base + dl::nla::kDirectionVector);
    if (dtype == DL_BF16)
      dl::nla::k_direction<uint16_t><<<1, dl::nla::kThreads, 0, queue->stream>>>(
          static_cast<const uint16_t*>(original), static_cast<const uint16_t*>(edited), direction, status, width);
    else
      dl::nla::k_direction<float><<<1, dl::nla::kThreads, 0, queue->stream>>>(
          static_cast<const float*>(original), static_cast<const float*>(edited), direction, status, width);
    dl::check_launch(queue, "direction");
  });
}

int dl_intervention_initialize(dl_queue* queue, uint32_t* state) {
  return guard([&] {
    dl::enter(queue);
    require(state != nullptr, "null operand");
    dl::nla::k_intervention_reset<<<1, 1, 0, queue->stream>>>(state);
    dl::check_launch(queue, "intervention reset");
  });
}

int dl_intervention_submit(dl_queue* queue, void* residual, int dtype, uint64_t rows, uint64_t width,
                           const float* direction, const uint64_t* position, uint64_t selected, float strength,
                           uint32_t* state) {
  return guard([&] {
    dl::enter(queue);
    require(residual && direction && position && state, "null operand");
    require(dtype == DL_BF16 || dtype == DL_F32, "invalid residual intervention");
    require(std::isfinite(strength) && strength >= 0.0f, "invalid residual intervention");
    require(rows > 0 && width > 0 && rows <= std::numeric_limits<uint64_t>::max() / width / 4,
            "intervention extent", DL_LENGTH_ERROR);
    if (dtype == DL_BF16)
      dl::nla::k_intervene<uint16_t><<<1, dl::nla::kThreads, 0, queue->stream>>>(
          static_cast<uint16_t*>(residual), direction, position, state, width, selected, rows, strength);
    else
      dl::nla::k_intervene<float><<<1, dl::nla::kThreads, 0, queue->stream>>>(
          static_cast<float*>(residual), direction, position, state, width, selected, rows, strength);
    dl::check_launch(queue, "intervention");
  });
}

}  // extern "C"
