// Packed exact-chain GEMV core for gfx950.
//
// The reference projection (src/kernels/cuda/projection.cu:1-67) fixes, for
// every output, P strided partial sums (partial t is the FMA chain over
// features t, t+P, t+2P, ... in ascending order) merged upper-into-lower at
// offsets P/2..1.  Bit equality with that contract only constrains which
// lane owns which chain, not where the weights live, and the reference
// leaves the resident weight layout to the backend
// (docs/architecture/transformer-execution.md:47-48).
//
// Packed layout.  With RW = 64/P output rows per wavefront tile and
// S = I/(8P) steps, element W[r][k] (t = k mod P, m = k div P) lives at
//
//     ((g*S + s)*64 + lane)*8 + e,  g = r/RW, lane = (r mod RW)*P + t,
//                                   s = m/8,  e = m mod 8.
//
// Lane (row r, partial t) therefore reads its own chain 8 consecutive
// elements at a time with one 16-byte load, and each wavefront load covers
// one contiguous 1 KiB: full-width coalesced HBM streaming with the
// reference's exact accumulation order.  The input vector is staged once per
// workgroup in LDS transposed the same way (xs[t][m] = x[P*m + t], rows padded
// by 4 floats so the P distinct addresses of a wavefront hit distinct banks).
#pragma once

#include "dl_device.h"

namespace dl {

constexpr int kXsPad = 4;

// Floats of LDS that one staged input row occupies for P partials.
__host__ __device__ constexpr int staged_floats(int P, int I) { return P * (I / P + kXsPad); }

// Packed element offset of W[r][k].
__host__ __device__ inline uint64_t packed_index(uint64_t r, uint64_t k, int P, uint64_t I) {
  const uint64_t RW = 64 / P, S = I / (8 * P);
  const uint64_t g = r / RW, rl = r % RW, t = k % P, m = k / P;
  return ((g * S + m / 8) * 64 + rl * P + t) * 8 + (m % 8);
}

// Inverse of packed_index: row and column of packed element p.
__host__ __device__ inline void packed_coords(uint64_t p, int P, uint64_t I, uint64_t* r, uint64_t* k) {
  const uint64_t RW = 64 / P, S = I / (8 * P);
  const uint64_t e = p % 8, lane = (p / 8) % 64, gs = p / 512;
  const uint64_t s = gs % S, g = gs / S;
  *r = g * RW + lane / P;
  *k = static_cast<uint64_t>(P) * (8 * s + e) + lane % P;
}

// Writes value v of input element i into the staged layout of row b.
template <int P>
__device__ __forceinline__ void stage_put(float* xs, int I, int b, int i, float v) {
  const int stride = I / P + kXsPad;
  xs[b * P * stride + (i % P) * stride + i / P] = v;
}

// One wavefront computes RW output rows for B input rows.  `tile` points at
// the tile's first 16-byte chunk; on return lane (row, 0) of each P-lane
// segment holds the merged FP32 sum of that row for every b.
template <int P, int B>
__device__ __forceinline__ void chain_tile(const u32x4* __restrict__ tile, const float* __restrict__ xs,
                                           int I, int lane, float (&acc)[B]) {
  const int L = I / P, S = L / 8, stride = L + kXsPad, bstride = P * stride;
  const float* xt = xs + (lane % P) * stride;
  const u32x4* src = tile + lane;
#pragma unroll
  for (int b = 0; b < B; ++b) acc[b] = 0.0f;
#pragma unroll 8
  for (int s = 0; s < S; ++s) {
    const u32x4 w = load_stream(src + s * 64);
    const float w0 = dl_bf16_lo(w.x), w1 = dl_bf16_hi(w.x), w2 = dl_bf16_lo(w.y), w3 = dl_bf16_hi(w.y);
    const float w4 = dl_bf16_lo(w.z), w5 = dl_bf16_hi(w.z), w6 = dl_bf16_lo(w.w), w7 = dl_bf16_hi(w.w);
#pragma unroll
    for (int b = 0; b < B; ++b) {
      const float4 xa = *reinterpret_cast<const float4*>(xt + b * bstride + 8 * s);
      const float4 xb = *reinterpret_cast<const float4*>(xt + b * bstride + 8 * s + 4);
      float a = acc[b];
      a = fma_rn(xa.x, w0, a);
      a = fma_rn(xa.y, w1, a);
      a = fma_rn(xa.z, w2, a);
      a = fma_rn(xa.w, w3, a);
      a = fma_rn(xb.x, w4, a);
      a = fma_rn(xb.y, w5, a);
      a = fma_rn(xb.z, w6, a);
      a = fma_rn(xb.w, w7, a);
      acc[b] = a;
    }
  }
#pragma unroll
  for (int b = 0; b < B; ++b) {
#pragma unroll
    for (int off = P / 2; off; off >>= 1) acc[b] = acc[b] + __shfl_down(acc[b], off, P);
  }
}

// Inverse RMS of one BF16 row of width D > 128 with the reference tree
// (normalization.cu:134-186): thread i < 128 owns component sum i of
// features i + 128k, groups of four combine left to right, 32 lane totals
// reduce with shuffle-down offsets 1..16.  Every thread of the block calls;
// `scratch` holds at least 33 floats of LDS.  Returns the inverse to all.
__device__ __forceinline__ float block_rms_inverse(const uint16_t* __restrict__ x, int D, float eps,
                                                   float* scratch) {
  const int tid = threadIdx.x;
  if (tid < 128) {
    float comp = 0.0f;
    for (int col = tid; col < D; col += 128) {
      const float v = dl_bf16_to_f32(x[col]);
      comp = comp + v * v;
    }
    const float second = __shfl_down(comp, 1, 4);
    const float third = __shfl_down(comp, 2, 4);
    const float fourth = __shfl_down(comp, 3, 4);
    if ((tid & 3) == 0) scratch[tid >> 2] = ((comp + second) + third) + fourth;
  }
  __syncthreads();
  if (tid < 32) {
    float s = scratch[tid];
#pragma unroll
    for (int off = 1; off < 32; off *= 2) s = s + __shfl_down(s, off, 32);
    if (tid == 0) scratch[32] = inverse_sqrt(s * (1.0f / static_cast<float>(D)) + eps);
  }
  __syncthreads();
  const float inverse = scratch[32];
  __syncthreads();
  return inverse;
}

}  // namespace dl
