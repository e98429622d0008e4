// Vector operations of the NLA injection and steering protocol on gfx950:
// the injection normalization (src/kernels/cuda/injection.cu:49-98, law H2
// of docs/architecture/execution-boundary.md:489-498), the steering direction
// (src/kernels/cuda/steering.cu:69-100) and the one-row residual intervention
// (steering.cu:107-159).  Each runs as one workgroup: eight lanes of the first
// wavefront hold the eight strided FP32 square sums, thread 0 combines them,
// and the whole workgroup applies the row update.
#pragma once

#include "dl_device.h"

namespace dl::nla {

constexpr unsigned kLanes = 8;      // strided partial sums of the reference reduction
constexpr unsigned kThreads = 256;  // one workgroup per vector operation

// sum_i value(i)^2 in the reference order: lane k < 8 accumulates
// i = k, k + 8, k + 16, ... ascending, with separately rounded multiply and
// add; thread 0 then adds lanes 0..7 left to right.  Every thread of the
// workgroup calls; all receive the sum (kept in sums[kLanes]).
template <class F>
__device__ __forceinline__ float square_sum(uint64_t width, F&& value, float* sums) {
  if (threadIdx.x < kLanes) {
    float sum = 0.0f;
    for (uint64_t i = threadIdx.x; i < width; i += kLanes) {
      const float v = value(i);
      sum = __fadd_rn(sum, __fmul_rn(v, v));
    }
    sums[threadIdx.x] = sum;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    float sum = 0.0f;
    for (unsigned k = 0; k < kLanes; ++k) sum = __fadd_rn(sum, sums[k]);
    sums[kLanes] = sum;
  }
  __syncthreads();
  return sums[kLanes];
}

__device__ __forceinline__ bool finite(float v) { return __builtin_isfinite(v); }

// The intervention's row update (steering.cu:107-159) on one row of width
// `width`: state[0] is the status latch, state[1] the application count.  A
// row already intervened on (count nonzero) or a prior failure makes this
// application invalid (the row is left unchanged, the count still grows).
// beta = strength * sqrt(sum h^2); h[i] = narrow(h[i] + beta * u[i]) with
// separate rounding; a nonfinite beta or stored value latches status.
// `sums` holds kLanes + 2 floats and `invalid` one word of LDS.
template <class T>
__device__ __forceinline__ void intervene_row(T* row, const float* direction, uint32_t* state, uint64_t width,
                                              float strength, float* sums, uint32_t* invalid) {
  if (threadIdx.x == 0) {
    *invalid = (state[0] != 0 || state[1] != 0) ? 1u : 0u;
    state[1] = state[1] + 1;
  }
  __syncthreads();
  const float sum = square_sum(width, [&](uint64_t i) { return load_elem(row, i); }, sums);
  if (threadIdx.x == 0) {
    const float beta = __fmul_rn(strength, __builtin_sqrtf(sum));
    sums[kLanes + 1] = beta;
    if (!finite(beta)) *invalid = 1u;
  }
  __syncthreads();
  const float beta = sums[kLanes + 1];
  const bool valid = *invalid == 0;
  __syncthreads();
  if (valid) {
    for (uint64_t i = threadIdx.x; i < width; i += blockDim.x) {
      const float value = __fadd_rn(load_elem(row, i), __fmul_rn(beta, direction[i]));
      store_elem(row, i, value);
      if (!finite(value) || !finite(storage_round<T>(value))) atomicOr(invalid, 1u);
    }
  }
  __syncthreads();
  if (threadIdx.x == 0) state[0] = *invalid;
}

}  // namespace dl::nla
