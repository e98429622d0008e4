// The reference's eight-operation catalog on gfx950, operand layouts as the
// reference stores them (row-major W[O,I], Q[B,Hq,d], K/V[C,Hkv,d]).
//
// Each kernel restates one launch of src/kernels/cuda/launch.h:79-109 with
// the same reduction ownership, merge order and storage-rounding points, so
// results are bit-identical with the reference contract
// (docs/architecture/transformer-execution.md:115-170).  The wave64 mapping
// differs from the reference's warp32 mapping, but every reduction below is
// written so that the value produced is the reference tree's value:
//  - shuffle-down within a width-P segment returns the lane's own value when
//    the source lane leaves the segment, exactly like the CUDA intrinsic; the
//    lane that keeps the result therefore sees the identical pairing.
//  - exp, sin, cos, pow come from dl_math.h (deterministic, shared with the
//    CPU oracle); sqrt and division are IEEE correctly rounded.
#include <algorithm>
#include <cstdint>

#include "dl_device.h"
#include "dl_internal.h"

namespace dl {
namespace {

constexpr int kThreads = 256;

inline unsigned grid_for(uint64_t tasks, uint64_t per_block, uint64_t cap = 1u << 30) {
  const uint64_t blocks = ceil_div(tasks, per_block);
  return static_cast<unsigned>(std::min<uint64_t>(std::max<uint64_t>(blocks, 1), cap));
}

// ----------------------------------------------------------------- projection
// projection.cu:277-318 (decode) and 218-275 (prefill): P lanes own one
// output; lane t is the FMA chain over features t, t+P, ...; a ragged input
// width emulates the tiled kernel's zero padding to 16 features
// (projection.cu:295-304); merge offsets P/2..1; round once.
template <class T, int P, int RT>
__global__ __launch_bounds__(kThreads) void projection_rowmajor(const T* __restrict__ x,
                                                                const T* __restrict__ w,
                                                                T* __restrict__ y, uint64_t rows,
                                                                uint64_t in_w, uint64_t out_w,
                                                                const uint64_t* out_pos) {
  constexpr int kOutputsPerBlock = kThreads / P;
  const int lane = threadIdx.x % P;
  const uint64_t o = static_cast<uint64_t>(blockIdx.x) * kOutputsPerBlock + threadIdx.x / P;
  const uint64_t r0 = static_cast<uint64_t>(blockIdx.y) * RT;
  const uint64_t base = out_pos ? *out_pos * out_w : 0;
  float acc[RT];
#pragma unroll
  for (int r = 0; r < RT; ++r) acc[r] = 0.0f;
  if (o < out_w) {
    const T* wr = w + o * in_w;
    for (uint64_t f = lane; f < in_w; f += P) {
      const float wv = load_elem(wr, f);
#pragma unroll
      for (int r = 0; r < RT; ++r)
        if (r0 + r < rows) acc[r] = fma_rn(load_elem(x + (r0 + r) * in_w, f), wv, acc[r]);
    }
    const uint64_t padded = ceil_div(in_w, 16) * 16;
    if (padded != in_w && static_cast<uint64_t>(lane) >= in_w % P &&
        static_cast<uint64_t>(lane) < (padded - 1) % P + 1) {
#pragma unroll
      for (int r = 0; r < RT; ++r) acc[r] = fma_rn(0.0f, 0.0f, acc[r]);
    }
  }
#pragma unroll
  for (int r = 0; r < RT; ++r) {
    float v = acc[r];
#pragma unroll
    for (int off = P / 2; off; off >>= 1) v = v + __shfl_down(v, off, P);
    if (lane == 0 && o < out_w && r0 + r < rows) store_elem(y, base + (r0 + r) * out_w + o, v);
  }
}

template <class T>
void launch_projection_rowmajor(hipStream_t s, const void* x, const void* w, void* y, uint64_t rows,
                                uint64_t in_w, uint64_t out_w, const uint64_t* out_pos) {
  constexpr int RT = 8;
  const bool narrow = in_w <= 4096 && out_w > 1024;
  const uint64_t row_blocks = ceil_div(rows, RT);
  require(row_blocks <= 65535, "projection rows exceed the launch limit", DL_LENGTH_ERROR);
  if (narrow) {
    dim3 grid(grid_for(out_w, kThreads / 16), static_cast<unsigned>(row_blocks));
    projection_rowmajor<T, 16, RT><<<grid, kThreads, 0, s>>>(
        static_cast<const T*>(x), static_cast<const T*>(w), static_cast<T*>(y), rows, in_w, out_w, out_pos);
  } else {
    dim3 grid(grid_for(out_w, kThreads / 32), static_cast<unsigned>(row_blocks));
    projection_rowmajor<T, 32, RT><<<grid, kThreads, 0, s>>>(
        static_cast<const T*>(x), static_cast<const T*>(w), static_cast<T*>(y), rows, in_w, out_w, out_pos);
  }
}

// ------------------------------------------------------------------ rms norm
// normalization.cu:82-186.  Thread i < 128 is lane t = i/4, component c = i%4:
// width > 128 sums squares of features 4t+c+128k; width <= 128 holds feature
// t+32c.  Components combine left to right, lanes reduce with shuffle-down
// offsets 1..16, inverse = 1/sqrt(total * FP32(1/width) + eps),
// y = round(round(x * inverse) * w).
template <class T>
__global__ __launch_bounds__(kThreads) void rms_norm_rows(const T* __restrict__ x,
                                                          const T* __restrict__ w,
                                                          T* __restrict__ y, uint64_t rows,
                                                          uint64_t width, float eps) {
  __shared__ float lanes[32];
  __shared__ float inverse_shared;
  for (uint64_t row = blockIdx.x; row < rows; row += gridDim.x) {
    const T* xr = x + row * width;
    if (threadIdx.x < 128) {
      const unsigned t = threadIdx.x / 4, c = threadIdx.x % 4;
      float comp = 0.0f;
      if (width <= 128) {
        const uint64_t col = t + 32u * c;
        if (col < width) {
          const float v = load_elem(xr, col);
          comp = v * v;
        }
      } else {
        for (uint64_t col = 4u * t + c; col < width; col += 128) {
          const float v = load_elem(xr, col);
          comp = comp + v * v;
        }
      }
      const float second = __shfl_down(comp, 1, 4);
      const float third = __shfl_down(comp, 2, 4);
      const float fourth = __shfl_down(comp, 3, 4);
      if (c == 0) lanes[t] = ((comp + second) + third) + fourth;
    }
    __syncthreads();
    if (threadIdx.x < 32) {
      float s = lanes[threadIdx.x];
#pragma unroll
      for (int off = 1; off < 32; off *= 2) s = s + __shfl_down(s, off, 32);
      if (threadIdx.x == 0) inverse_shared = inverse_sqrt(s * (1.0f / static_cast<float>(width)) + eps);
    }
    __syncthreads();
    const float inverse = inverse_shared;
    for (uint64_t col = threadIdx.x; col < width; col += blockDim.x) {
      const float normalized = storage_round<T>(load_elem(xr, col) * inverse);
      store_elem(y, row * width + col, normalized * load_elem(w, col));
    }
    __syncthreads();
  }
}

// -------------------------------------------------------------------- rotary
// rotary.cu:84-126.
template <class T>
__global__ __launch_bounds__(kThreads) void rotary_pairs(const T* __restrict__ x, T* __restrict__ y,
                                                         uint64_t pairs, uint64_t heads,
                                                         uint64_t width, uint64_t host_first,
                                                         double theta, const uint64_t* dev_pos,
                                                         int positioned) {
  const uint64_t first = position_or(dev_pos, host_first);
  T* out = y + (positioned ? first * heads * width : 0);
  const uint64_t half = width / 2;
  const uint64_t stride = static_cast<uint64_t>(gridDim.x) * blockDim.x;
  for (uint64_t idx = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x; idx < pairs;
       idx += stride) {
    const uint64_t feature = idx % half, row = idx / half;
    const uint64_t position = first + row / heads;
    const float exponent = static_cast<float>(2 * feature) / static_cast<float>(width);
    const float inverse_frequency = static_cast<float>(1.0 / dl_pow_pos(theta, static_cast<double>(exponent)));
    const float angle = static_cast<float>(position) * inverse_frequency;
    double s, c;
    dl_sincos(static_cast<double>(angle), &s, &c);
    const float cosine = storage_round<T>(static_cast<float>(c));
    const float sine = storage_round<T>(static_cast<float>(s));
    const float a = load_elem(x, row * width + feature);
    const float b = load_elem(x, row * width + feature + half);
    const float ac = storage_round<T>(a * cosine), bs = storage_round<T>(b * sine);
    const float bc = storage_round<T>(b * cosine), as = storage_round<T>(a * sine);
    store_elem(out, row * width + feature, ac - bs);
    store_elem(out, row * width + feature + half, bc + as);
  }
}

// ----------------------------------------------------------------- attention
// attention.cu:231-383 (retained scores) and 436-439 (scale).
__global__ void attention_scale_kernel(float* out, uint64_t width) {
  *out = static_cast<float>(1.0 / __builtin_sqrt(static_cast<double>(width)));
}

template <class T>
__global__ __launch_bounds__(kThreads) void attention_retained(
    const T* __restrict__ q, const T* __restrict__ k, const T* __restrict__ v, T* __restrict__ out,
    uint64_t tasks, uint64_t q_heads, uint64_t kv_heads, uint64_t width, uint64_t host_first,
    const float* scale_ptr, const uint64_t* dev_pos) {
  extern __shared__ float shared[];
  float* qs = shared;
  float* scores = qs + width;
  __shared__ float reduction[kThreads];
  __shared__ float denominator_shared;
  const unsigned tid = threadIdx.x;
  const unsigned lane = tid % 8, group = tid / 8;
  const uint64_t span = width / 8 + (width % 8 != 0);
  const float scale = *scale_ptr;
  for (uint64_t task = blockIdx.x; task < tasks; task += gridDim.x) {
    const uint64_t first = position_or(dev_pos, host_first);
    const uint64_t count = first + task / q_heads + 1;
    const uint64_t kvh = (task % q_heads) / (q_heads / kv_heads);
    for (uint64_t f = tid; f < width; f += blockDim.x) qs[f] = load_elem(q, task * width + f);
    __syncthreads();
    for (uint64_t base = 0; base < count; base += kThreads / 8) {
      const uint64_t j = base + group;
      float partial = 0.0f;
      if (j < count) {
        const uint64_t kv_offset = (j * kv_heads + kvh) * width;
        const uint64_t begin = lane * span;
        const uint64_t end = begin < width ? (begin + span < width ? begin + span : width) : width;
        for (uint64_t f = begin; f < end; ++f) partial = fma_rn(qs[f], load_elem(k, kv_offset + f), partial);
      }
#pragma unroll
      for (int off = 4; off; off >>= 1) partial = partial + __shfl_down(partial, off, 8);
      if (lane == 0 && j < count) scores[j] = partial * scale;
    }
    __syncthreads();
    float maximum = scores[0];
    for (uint64_t j = tid; j < count; j += blockDim.x) maximum = fmaxf(maximum, scores[j]);
    reduction[tid] = maximum;
    __syncthreads();
    for (unsigned off = kThreads / 2; off; off >>= 1) {
      if (tid < off) reduction[tid] = fmaxf(reduction[tid], reduction[tid + off]);
      __syncthreads();
    }
    maximum = reduction[0];
    __syncthreads();
    if (tid < 32) {
      float partial = 0.0f;
      for (uint64_t j = tid; j < count; j += 32) {
        const float e = dl_expf(scores[j] - maximum);
        scores[j] = e;
        partial = partial + e;
      }
#pragma unroll
      for (int off = 16; off; off >>= 1) partial = partial + __shfl_down(partial, off, 32);
      if (tid == 0) denominator_shared = partial;
    }
    __syncthreads();
    const float denominator = denominator_shared;
    for (uint64_t j = tid; j < count; j += blockDim.x) scores[j] = scores[j] / denominator;
    __syncthreads();
    const uint64_t split = (count - 1) / 2 + 1;
    if (width <= kThreads / 2) {
      const unsigned feature = tid % (kThreads / 2), half = tid / (kThreads / 2);
      const uint64_t begin = half == 0 ? 0 : split, end = half == 0 ? split : count;
      float sum = 0.0f;
      if (feature < width) {
        for (uint64_t j = begin; j < end; ++j)
          sum = fma_rn(scores[j], load_elem(v, (j * kv_heads + kvh) * width + feature), sum);
      }
      reduction[tid] = sum;
      __syncthreads();
      if (tid < width) store_elem(out, task * width + tid, reduction[tid] + reduction[tid + kThreads / 2]);
    } else {
      for (uint64_t feature = tid; feature < width; feature += blockDim.x) {
        float a = 0.0f, b = 0.0f;
        for (uint64_t j = 0; j < split; ++j)
          a = fma_rn(scores[j], load_elem(v, (j * kv_heads + kvh) * width + feature), a);
        for (uint64_t j = split; j < count; ++j)
          b = fma_rn(scores[j], load_elem(v, (j * kv_heads + kvh) * width + feature), b);
        store_elem(out, task * width + feature, a + b);
      }
    }
    __syncthreads();
  }
}

// -------------------------------------------------------- embedding, add, silu
// embedding.cu:60-80; a token outside the table writes zeros instead of
// reading out of bounds.
template <class Bits>
__global__ __launch_bounds__(kThreads) void embedding_rows(const uint32_t* __restrict__ tokens,
                                                           const Bits* __restrict__ table,
                                                           Bits* __restrict__ out, uint64_t rows,
                                                           uint64_t width, uint64_t vocabulary) {
  for (uint64_t row = blockIdx.x; row < rows; row += gridDim.x) {
    const uint32_t token = tokens[row];
    for (uint64_t f = threadIdx.x; f < width; f += blockDim.x)
      out[row * width + f] = token < vocabulary ? table[static_cast<uint64_t>(token) * width + f] : Bits(0);
  }
}

// elementwise.cu:2-18, 62-87.
template <class T, bool Silu>
__global__ __launch_bounds__(kThreads) void elementwise(const T* __restrict__ left,
                                                        const T* __restrict__ right,
                                                        T* __restrict__ out, uint64_t count) {
  const uint64_t stride = static_cast<uint64_t>(gridDim.x) * blockDim.x;
  for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < count; i += stride) {
    const float a = load_elem(left, i), b = load_elem(right, i);
    float result;
    if constexpr (Silu) {
      const float e = dl_expf(a >= 0.0f ? -a : a);
      const float sigmoid = a >= 0.0f ? 1.0f / (1.0f + e) : e / (1.0f + e);
      result = storage_round<T>(a * sigmoid) * b;
    } else {
      result = a + b;
    }
    store_elem(out, i, result);
  }
}

bool valid_dtype(int dtype) { return dtype == DL_BF16 || dtype == DL_F32; }

}  // namespace
}  // namespace dl

using dl::guard;
using dl::require;

extern "C" {

int dl_projection(dl_queue* queue, int dtype, const void* input, const void* weight, void* output,
                  uint64_t rows, uint64_t input_width, uint64_t output_width,
                  const uint64_t* output_position) {
  return guard([&] {
    dl::enter(queue);
    require(dl::valid_dtype(dtype), "unsupported storage type");
    require(input && weight && output, "null operand");
    require(rows > 0 && input_width > 0 && output_width > 0, "empty projection");
    if (dtype == DL_BF16)
      dl::launch_projection_rowmajor<uint16_t>(queue->stream, input, weight, output, rows, input_width,
                                               output_width, output_position);
    else
      dl::launch_projection_rowmajor<float>(queue->stream, input, weight, output, rows, input_width,
                                            output_width, output_position);
    dl::check_launch(queue, "projection");
  });
}

int dl_rms_norm(dl_queue* queue, int dtype, const void* input, const void* weight, void* output,
                uint64_t rows, uint64_t width, float epsilon) {
  return guard([&] {
    dl::enter(queue);
    require(dl::valid_dtype(dtype), "unsupported storage type");
    require(input && weight && output, "null operand");
    require(rows > 0 && width > 0, "empty normalization");
    require(epsilon > 0.0f, "epsilon must be positive");
    const unsigned grid = dl::grid_for(rows, 1, 65535);
    if (dtype == DL_BF16)
      dl::rms_norm_rows<uint16_t><<<grid, dl::kThreads, 0, queue->stream>>>(
          static_cast<const uint16_t*>(input), static_cast<const uint16_t*>(weight),
          static_cast<uint16_t*>(output), rows, width, epsilon);
    else
      dl::rms_norm_rows<float><<<grid, dl::kThreads, 0, queue->stream>>>(
          static_cast<const float*>(input), static_cast<const float*>(weight), static_cast<float*>(output),
          rows, width, epsilon);
    dl::check_launch(queue, "rms_norm");
  });
}

int dl_rotary(dl_queue* queue, int dtype, const void* input, void* output, uint64_t positions,
              uint64_t heads, uint64_t width, uint64_t first_position, double theta,
              const uint64_t* device_position, int positioned_output) {
  return guard([&] {
    dl::enter(queue);
    require(dl::valid_dtype(dtype), "unsupported storage type");
    require(input && output, "null operand");
    require(positions > 0 && heads > 0 && width > 0 && width % 2 == 0, "invalid rotary shape");
    require(theta > 0.0 && theta < 1e300, "theta must be positive and finite");
    const uint64_t pairs = positions * heads * (width / 2);
    const unsigned grid = dl::grid_for(pairs, dl::kThreads, 65535);
    if (dtype == DL_BF16)
      dl::rotary_pairs<uint16_t><<<grid, dl::kThreads, 0, queue->stream>>>(
          static_cast<const uint16_t*>(input), static_cast<uint16_t*>(output), pairs, heads, width,
          first_position, theta, device_position, positioned_output);
    else
      dl::rotary_pairs<float><<<grid, dl::kThreads, 0, queue->stream>>>(
          static_cast<const float*>(input), static_cast<float*>(output), pairs, heads, width,
          first_position, theta, device_position, positioned_output);
    dl::check_launch(queue, "rotary");
  });
}

int dl_attention_scale(dl_queue* queue, float* output, uint64_t width) {
  return guard([&] {
    dl::enter(queue);
    require(output != nullptr && width > 0, "invalid attention scale arguments");
    dl::attention_scale_kernel<<<1, 1, 0, queue->stream>>>(output, width);
    dl::check_launch(queue, "attention_scale");
  });
}

int dl_attention(dl_queue* queue, int dtype, const void* query, const void* key, const void* value,
                 void* output, uint64_t positions, uint64_t query_heads, uint64_t kv_heads,
                 uint64_t width, uint64_t first_position, const uint64_t* device_position,
                 uint64_t capacity, const float* scale) {
  return guard([&] {
    dl::enter(queue);
    require(dl::valid_dtype(dtype), "unsupported storage type");
    require(query && key && value && output && scale, "null operand");
    require(positions > 0 && query_heads > 0 && kv_heads > 0 && width > 0, "empty attention");
    require(query_heads % kv_heads == 0, "query heads must be a multiple of KV heads");
    const uint64_t keys = device_position ? capacity : first_position + positions;
    require(keys > 0, "no visible keys");
    const uint64_t shared_bytes = (width + keys) * sizeof(float);
    require(shared_bytes <= 160 * 1024 - 2 * 1024, "attention exceeds on-chip score storage",
            DL_LENGTH_ERROR);
    const uint64_t tasks = positions * query_heads;
    const unsigned grid = dl::grid_for(tasks, 1, 65535);
    if (dtype == DL_BF16)
      dl::attention_retained<uint16_t><<<grid, dl::kThreads, shared_bytes, queue->stream>>>(
          static_cast<const uint16_t*>(query), static_cast<const uint16_t*>(key),
          static_cast<const uint16_t*>(value), static_cast<uint16_t*>(output), tasks, query_heads,
          kv_heads, width, first_position, scale, device_position);
    else
      dl::attention_retained<float><<<grid, dl::kThreads, shared_bytes, queue->stream>>>(
          static_cast<const float*>(query), static_cast<const float*>(key),
          static_cast<const float*>(value), static_cast<float*>(output), tasks, query_heads, kv_heads,
          width, first_position, scale, device_position);
    dl::check_launch(queue, "attention");
  });
}

int dl_embedding(dl_queue* queue, int dtype, const uint32_t* tokens, const void* weight,
                 void* output, uint64_t rows, uint64_t width, uint64_t vocabulary) {
  return guard([&] {
    dl::enter(queue);
    require(dl::valid_dtype(dtype), "unsupported storage type");
    require(tokens && weight && output, "null operand");
    require(rows > 0 && width > 0 && vocabulary > 0, "empty embedding");
    const unsigned grid = dl::grid_for(rows, 1, 65535);
    if (dtype == DL_BF16)
      dl::embedding_rows<uint16_t><<<grid, dl::kThreads, 0, queue->stream>>>(
          tokens, static_cast<const uint16_t*>(weight), static_cast<uint16_t*>(output), rows, width,
          vocabulary);
    else
      dl::embedding_rows<uint32_t><<<grid, dl::kThreads, 0, queue->stream>>>(
          tokens, static_cast<const uint32_t*>(weight), static_cast<uint32_t*>(output), rows, width,
          vocabulary);
    dl::check_launch(queue, "embedding");
  });
}

static int elementwise_entry(dl_queue* queue, int dtype, const void* left, const void* right,
                             void* output, uint64_t count, bool silu) {
  return guard([&] {
    dl::enter(queue);
    require(dl::valid_dtype(dtype), "unsupported storage type");
    require(left && right && output, "null operand");
    require(count > 0, "empty elementwise operation");
    const unsigned grid = dl::grid_for(count, dl::kThreads, 65535);
    hipStream_t s = queue->stream;
    if (dtype == DL_BF16) {
      auto l = static_cast<const uint16_t*>(left), r = static_cast<const uint16_t*>(right);
      auto o = static_cast<uint16_t*>(output);
      if (silu)
        dl::elementwise<uint16_t, true><<<grid, dl::kThreads, 0, s>>>(l, r, o, count);
      else
        dl::elementwise<uint16_t, false><<<grid, dl::kThreads, 0, s>>>(l, r, o, count);
    } else {
      auto l = static_cast<const float*>(left), r = static_cast<const float*>(right);
      auto o = static_cast<float*>(output);
      if (silu)
        dl::elementwise<float, true><<<grid, dl::kThreads, 0, s>>>(l, r, o, count);
      else
        dl::elementwise<float, false><<<grid, dl::kThreads, 0, s>>>(l, r, o, count);
    }
    dl::check_launch(queue, silu ? "silu_multiply" : "add");
  });
}

int dl_add(dl_queue* queue, int dtype, const void* left, const void* right, void* output,
           uint64_t count) {
  return elementwise_entry(queue, dtype, left, right, output, count, false);
}

int dl_silu_multiply(dl_queue* queue, int dtype, const void* gate, const void* up, void* output,
                     uint64_t count) {
  return elementwise_entry(queue, dtype, gate, up, output, count, true);
}

int dl_gather_rows(dl_queue* queue, const void* input, void* output, uint64_t row_bytes,
                   const uint64_t* rows, uint64_t count) {
  return guard([&] {
    dl::enter(queue);
    require(input && output && (rows || count == 0), "null operand");
    require(row_bytes > 0, "empty rows");
    for (uint64_t i = 0; i < count; ++i) {
      dl::check_hip(hipMemcpyAsync(static_cast<char*>(output) + i * row_bytes,
                                   static_cast<const char*>(input) + rows[i] * row_bytes, row_bytes,
                                   hipMemcpyDeviceToDevice, queue->stream),
                    "gather rows");
    }
  });
}

}  // extern "C"
