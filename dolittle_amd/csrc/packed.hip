// Standalone packed projection: the resident-layout fast path of
// launch_projection (src/kernels/cuda/projection.cu:277-361) as its own
// operation, used by callers that pack a weight once and project many times.
#include <algorithm>

#include "dl_device.h"
#include "dl_internal.h"
#include "gemv.h"

namespace dl {
namespace {

constexpr int kWaves = 4;

int partials(uint64_t in_w, uint64_t out_w) { return (in_w <= 4096 && out_w > 1024) ? 16 : 32; }

void check_packable(uint64_t out_w, uint64_t in_w) {
  const int P = partials(in_w, out_w);
  require(out_w > 0 && in_w > 0, "empty projection");
  require(out_w % (64 / P) == 0, "output width must be a multiple of 64/P", DL_LENGTH_ERROR);
  require(in_w % (8 * P) == 0, "input width must be a multiple of 8P", DL_LENGTH_ERROR);
  require(in_w <= 16384, "input width above 16384 is not supported", DL_LENGTH_ERROR);
}

__global__ void k_pack(const uint16_t* __restrict__ w, uint16_t* __restrict__ packed, uint64_t out_w,
                       uint64_t in_w, int P) {
  const uint64_t n = out_w * in_w;
  const uint64_t step = static_cast<uint64_t>(gridDim.x) * blockDim.x;
  for (uint64_t p = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x; p < n; p += step) {
    uint64_t r, k;
    packed_coords(p, P, in_w, &r, &k);
    packed[p] = w[r * in_w + k];
  }
}

// One input row per launch; every wavefront owns whole 64/P-row tiles.
template <int P>
__global__ __launch_bounds__(kWaves * 64) void k_packed_gemv(const uint16_t* __restrict__ x,
                                                             const u32x4* __restrict__ w,
                                                             uint16_t* __restrict__ y, int in_w,
                                                             uint64_t out_w, const uint64_t* out_pos) {
  extern __shared__ float xs[];
  for (int i = threadIdx.x; i < in_w; i += blockDim.x) stage_put<P>(xs, in_w, 0, i, dl_bf16_to_f32(x[i]));
  __syncthreads();
  const uint64_t base = out_pos ? *out_pos * out_w : 0;
  const int wave = threadIdx.x / 64, lane = threadIdx.x % 64;
  constexpr int RW = 64 / P;
  const uint64_t tiles = out_w / RW;
  const uint64_t chunks = static_cast<uint64_t>(in_w / (8 * P)) * 64;
  for (uint64_t tile = static_cast<uint64_t>(blockIdx.x) * kWaves + wave; tile < tiles;
       tile += static_cast<uint64_t>(gridDim.x) * kWaves) {
    float acc[1];
    chain_tile<P, 1>(w + tile * chunks, xs, in_w, lane, acc);
    if (lane % P == 0) y[base + tile * RW + lane / P] = dl_f32_to_bf16(acc[0]);
  }
}

}  // namespace
}  // namespace dl

using dl::guard;
using dl::require;

extern "C" {

int dl_projection_packed_bytes(uint64_t output_width, uint64_t input_width, uint64_t* bytes) {
  return guard([&] {
    require(bytes != nullptr, "null output");
    dl::check_packable(output_width, input_width);
    *bytes = output_width * input_width * 2;
  });
}

int dl_projection_pack(dl_queue* queue, const void* weight, void* packed, uint64_t output_width,
                       uint64_t input_width) {
  return guard([&] {
    dl::enter(queue);
    require(weight && packed, "null operand");
    dl::check_packable(output_width, input_width);
    const int P = dl::partials(input_width, output_width);
    const uint64_t n = output_width * input_width;
    const unsigned grid = static_cast<unsigned>(std::min<uint64_t>(dl::ceil_div(n, 256), 65535));
    dl::k_pack<<<grid, 256, 0, queue->stream>>>(static_cast<const uint16_t*>(weight),
                                                static_cast<uint16_t*>(packed), output_width, input_width, P);
    dl::check_launch(queue, "projection pack");
  });
}

int dl_projection_packed(dl_queue* queue, const void* input, const void* packed, void* output, uint64_t rows,
                         uint64_t input_width, uint64_t output_width, const uint64_t* output_position) {
  return guard([&] {
    dl::enter(queue);
    require(input && packed && output, "null operand");
    require(rows > 0, "empty projection");
    dl::check_packable(output_width, input_width);
    const int P = dl::partials(input_width, output_width);
    const uint64_t tiles = output_width / (64 / P);
    const unsigned grid =
        static_cast<unsigned>(std::min<uint64_t>(dl::ceil_div(tiles, dl::kWaves), 2048));
    const size_t lds = static_cast<size_t>(dl::staged_floats(P, static_cast<int>(input_width))) * sizeof(float);
    for (uint64_t r = 0; r < rows; ++r) {
      const uint16_t* x = static_cast<const uint16_t*>(input) + r * input_width;
      uint16_t* y = static_cast<uint16_t*>(output) + r * output_width;
      const auto* w = static_cast<const dl::u32x4*>(packed);
      if (P == 16) {
        if (lds > 64 * 1024)
          dl::check_hip(hipFuncSetAttribute(reinterpret_cast<const void*>(dl::k_packed_gemv<16>),
                                            hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds)),
                        "hipFuncSetAttribute");
        dl::k_packed_gemv<16><<<grid, dl::kWaves * 64, lds, queue->stream>>>(
            x, w, y, static_cast<int>(input_width), output_width, output_position);
      } else {
        if (lds > 64 * 1024)
          dl::check_hip(hipFuncSetAttribute(reinterpret_cast<const void*>(dl::k_packed_gemv<32>),
                                            hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds)),
                        "hipFuncSetAttribute");
        dl::k_packed_gemv<32><<<grid, dl::kWaves * 64, lds, queue->stream>>>(
            x, w, y, static_cast<int>(input_width), output_width, output_position);
      }
    }
    dl::check_launch(queue, "packed projection");
  });
}

}  // extern "C"
