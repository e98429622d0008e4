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

// Stages BF16 rows [b0, b0 + R) of x (width I) into the P-partial layout.
// Each thread moves 16-byte chunks; all of a thread's loads are issued
// before any is consumed.  Requires I % 8 == 0 and I <= 8 * 8 * blockDim.x.
// `row_stride` (default I) is the distance between source rows, so a block
// of columns of wider rows can be staged.
//
// `active`, when given, is the token loop's grid-uniform liveness word: it
// is loaded first, and once the row's and the caller's loads are issued a
// stopped loop returns false before any conversion or LDS store (a stopped
// step then costs its launch and a few loads).  The word is only waited for
// after the vector loads are in flight, so a live step waits no longer.
template <int P, class Issue>
__device__ __forceinline__ bool stage_rows(const uint16_t* __restrict__ x, int I, int rows, float* xs,
                                           Issue&& issue, int row_stride = 0, const uint32_t* active = nullptr,
                                           int valid = 1 << 30) {
  constexpr int kMaxChunks = 8;
  const int chunks = I / 8;
  const uint64_t stride = row_stride ? row_stride : I;
  const uint32_t live = active ? *active : 1u;
  for (int b = 0; b < rows; ++b) {
    // Rows from `valid` on do not exist: their slots repeat the last row.
    const u32x4* src = reinterpret_cast<const u32x4*>(x + static_cast<uint64_t>(b < valid ? b : valid - 1) * stride);
    u32x4 v[kMaxChunks];
#pragma unroll
    for (int j = 0; j < kMaxChunks; ++j) {
      const int c = threadIdx.x + j * blockDim.x;
      v[j] = src[c < chunks ? c : 0];
    }
    if (b == 0) {
      // The caller's first weight batch follows this row's loads (loads
      // retire in order) and overlaps the staging below.
      __builtin_amdgcn_sched_barrier(0);
      issue();
      __builtin_amdgcn_sched_barrier(0);
      if (!live) return false;
    }
#pragma unroll
    for (int j = 0; j < kMaxChunks; ++j) {
      const int c = threadIdx.x + j * blockDim.x;
      if (c < chunks) {
        const int i = c * 8;
        stage_put<P>(xs, I, b, i + 0, dl_bf16_lo(v[j].x));
        stage_put<P>(xs, I, b, i + 1, dl_bf16_hi(v[j].x));
        stage_put<P>(xs, I, b, i + 2, dl_bf16_lo(v[j].y));
        stage_put<P>(xs, I, b, i + 3, dl_bf16_hi(v[j].y));
        stage_put<P>(xs, I, b, i + 4, dl_bf16_lo(v[j].z));
        stage_put<P>(xs, I, b, i + 5, dl_bf16_hi(v[j].z));
        stage_put<P>(xs, I, b, i + 6, dl_bf16_lo(v[j].w));
        stage_put<P>(xs, I, b, i + 7, dl_bf16_hi(v[j].w));
      }
    }
  }
  return true;
}

// Stages the columns [0, I) of B BF16 rows (source rows `row_stride` apart)
// into the P-partial layout with a compile-time shape: each of the T
// threads moves I / (8 T) 16-byte chunks per row, all B rows' loads issued
// before any is converted.  `issue` runs after the loads (loads retire in
// order).  Requires I % (8 T) == 0.  Only the first `rows` rows exist: the
// others' slots are staged from the last of them and never stored from.
template <int P, int B, int I, int T, class Issue>
__device__ __forceinline__ void stage_block(const uint16_t* __restrict__ x, uint64_t row_stride, float* xs,
                                            Issue&& issue, int rows = B) {
  constexpr int J = I / (8 * T);
  static_assert(J >= 1 && I % (8 * T) == 0, "block width must be a multiple of 8 per thread");
  u32x4 v[B][J];
#pragma unroll
  for (int b = 0; b < B; ++b) {
#pragma unroll
    for (int j = 0; j < J; ++j)
      v[b][j] = reinterpret_cast<const u32x4*>(x + (b < rows ? b : rows - 1) * row_stride)[threadIdx.x + j * T];
  }
  __builtin_amdgcn_sched_barrier(0);
  issue();
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int b = 0; b < B; ++b) {
#pragma unroll
    for (int j = 0; j < J; ++j) {
      const int i = (threadIdx.x + j * T) * 8;
      stage_put<P>(xs, I, b, i + 0, dl_bf16_lo(v[b][j].x));
      stage_put<P>(xs, I, b, i + 1, dl_bf16_hi(v[b][j].x));
      stage_put<P>(xs, I, b, i + 2, dl_bf16_lo(v[b][j].y));
      stage_put<P>(xs, I, b, i + 3, dl_bf16_hi(v[b][j].y));
      stage_put<P>(xs, I, b, i + 4, dl_bf16_lo(v[b][j].z));
      stage_put<P>(xs, I, b, i + 5, dl_bf16_hi(v[b][j].z));
      stage_put<P>(xs, I, b, i + 6, dl_bf16_lo(v[b][j].w));
      stage_put<P>(xs, I, b, i + 7, dl_bf16_hi(v[b][j].w));
    }
  }
}

// One wavefront computes RW output rows for B input rows.  `tile` points at
// the tile's first 16-byte chunk; on return lane (row, 0) of each P-lane
// segment holds the merged FP32 sum of that row for every b.
//
// Loads are issued in batches of kBatch independent 16-byte chunks held in
// distinct registers before any of them is consumed, so each wavefront keeps
// kBatch KiB in flight instead of serialising on one load-use chain.
constexpr int kBatch = 8;

// LDS per compute unit on gfx950.
constexpr uint64_t kLdsPerCu = 160 * 1024;

// One step of every lane's chain: 8 consecutive chain elements of weights w
// against the staged inputs at step s, for each of the B rows.
template <int B>
__device__ __forceinline__ void chain_step(const u32x4 w, const float* __restrict__ xt, int bstride, int s,
                                           float (&acc)[B]) {
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

// First kBatch 16-byte chunks of a tile, issued ahead of a prologue.
struct FirstBatch {
  u32x4 w[kBatch];
  bool valid;
};

__device__ __forceinline__ void issue_first(const u32x4* __restrict__ tile, int lane, FirstBatch& f) {
  const u32x4* src = tile + lane;
#pragma unroll
  for (int j = 0; j < kBatch; ++j) f.w[j] = load_stream(src + j * 64);
  f.valid = true;
}

// The batches of a tile are double-buffered (batch k + 1 is issued before
// batch k is consumed), so a wavefront keeps two batches in flight, and the
// last one overlaps the first batch of the wavefront's next tile (if there is
// one), handed back through `first`.  Needs an even batch count.
template <int P, int B>
__device__ __forceinline__ void chain_tile_pipelined(const u32x4* __restrict__ src, const float* __restrict__ xt,
                                                     int bstride, int batches, float (&acc)[B], FirstBatch* first,
                                                     const u32x4* __restrict__ next_src) {
  u32x4 wa[kBatch], wb[kBatch];
  auto load = [&](u32x4* w, const u32x4* from) {
#pragma unroll
    for (int j = 0; j < kBatch; ++j) w[j] = load_stream(from + j * 64);
  };
  // Whether a next tile follows is the same for the whole wavefront (only
  // the lane offset differs).
  const bool has_next = __builtin_amdgcn_readfirstlane(next_src != nullptr ? 1 : 0) != 0;
  if (first && first->valid) {
#pragma unroll
    for (int j = 0; j < kBatch; ++j) wa[j] = first->w[j];
  } else {
    load(wa, src);
  }
  for (int k = 0; k < batches; k += 2) {
    load(wb, src + (k + 1) * kBatch * 64);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int j = 0; j < kBatch; ++j) chain_step<B>(wa[j], xt, bstride, k * kBatch + j, acc);
    __builtin_amdgcn_sched_barrier(0);
    // Past the tile's last batch: the next tile's first batch, or (no next
    // tile) at one row nothing; at several rows the batch just loaded again,
    // which L2 still holds: a select, not a branch, so both register sets
    // stay in place (a branch there spills).
    if constexpr (B == 1) {
      if (k + 2 < batches || has_next) load(wa, k + 2 < batches ? src + (k + 2) * kBatch * 64 : next_src);
    } else {
      load(wa, k + 2 < batches ? src + (k + 2) * kBatch * 64
                               : (has_next ? next_src : src + (k + 1) * kBatch * 64));
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int j = 0; j < kBatch; ++j) chain_step<B>(wb[j], xt, bstride, (k + 1) * kBatch + j, acc);
    __builtin_amdgcn_sched_barrier(0);
  }
  if (first) {
#pragma unroll
    for (int j = 0; j < kBatch; ++j) first->w[j] = wa[j];
  }
}

// The chain steps of one tile over I staged inputs, accumulating into acc
// (not reset).  `next` (optional) is where the wavefront's chain continues
// (its next tile, or this tile's next block of inputs): with B >= 2 its
// first batch is loaded during this call's last batch and left in `first`.
// kDeep selects the double-buffered batches (the default for B >= 2; a
// single-row caller that leaves few wavefronts per SIMD asks for it too, to
// keep two batches in flight per wavefront).
template <int P, int B, bool kDeep = (B >= 2)>
__device__ __forceinline__ void chain_body(const u32x4* __restrict__ tile, const float* __restrict__ xs, int I,
                                           int lane, float (&acc)[B], FirstBatch* first = nullptr,
                                           const u32x4* __restrict__ next = nullptr) {
  const int L = I / P, S = L / 8, stride = L + kXsPad, bstride = P * stride;
  const float* xt = xs + (lane % P) * stride;
  const u32x4* src = tile + lane;
  if constexpr (kDeep) {
    const int batches = S / kBatch;
    if (S % kBatch == 0 && batches % 2 == 0) {
      chain_tile_pipelined<P, B>(src, xt, bstride, batches, acc, first, next ? next + lane : nullptr);
      if (first) first->valid = next != nullptr;
      return;
    }
  }
  int s0 = 0;
  if (first && first->valid && S >= kBatch) {
    // The tile's first batch was issued before the kernel's prologue.
#pragma unroll
    for (int j = 0; j < kBatch; ++j) chain_step<B>(first->w[j], xt, bstride, j, acc);
    first->valid = false;
    s0 = kBatch;
  }
  for (; s0 + kBatch <= S; s0 += kBatch) {
    u32x4 w[kBatch];
#pragma unroll
    for (int j = 0; j < kBatch; ++j) w[j] = load_stream(src + (s0 + j) * 64);
#pragma unroll
    for (int j = 0; j < kBatch; ++j) chain_step<B>(w[j], xt, bstride, s0 + j, acc);
  }
  for (; s0 < S; ++s0) chain_step<B>(load_stream(src + s0 * 64), xt, bstride, s0, acc);
}

// Merges the P partials of each row (offsets P/2 .. 1) into lane (row, 0);
// offsets below 16 move within a 16-lane row (DPP).
template <int P, int B>
__device__ __forceinline__ void chain_merge(float (&acc)[B]) {
  static_assert(P == 16 || P == 32, "16 or 32 partials per row");
#pragma unroll
  for (int b = 0; b < B; ++b) {
    if constexpr (P == 32) acc[b] = acc[b] + __shfl_down(acc[b], 16, P);
    acc[b] = acc[b] + row_down<8>(acc[b]);
    acc[b] = acc[b] + row_down<4>(acc[b]);
    acc[b] = acc[b] + row_down<2>(acc[b]);
    acc[b] = acc[b] + row_down<1>(acc[b]);
  }
}

template <int P, int B, bool kDeep = (B >= 2)>
__device__ __forceinline__ void chain_tile(const u32x4* __restrict__ tile, const float* __restrict__ xs,
                                           int I, int lane, float (&acc)[B], FirstBatch* first = nullptr,
                                           const u32x4* __restrict__ next = nullptr) {
#pragma unroll
  for (int b = 0; b < B; ++b) acc[b] = 0.0f;
  chain_body<P, B, kDeep>(tile, xs, I, lane, acc, first, next);
  chain_merge<P, B>(acc);
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
    const float second = row_down<1>(comp);
    const float third = row_down<2>(comp);
    const float fourth = row_down<3>(comp);
    if ((tid & 3) == 0) scratch[tid >> 2] = ((comp + second) + third) + fourth;
  }
  __syncthreads();
  if (tid < 32) {
    const float s = tree_sum32(scratch[tid]);
    if (tid == 0) scratch[32] = inverse_sqrt(s * (1.0f / static_cast<float>(D)) + eps);
  }
  __syncthreads();
  const float inverse = scratch[32];
  __syncthreads();
  return inverse;
}

// Stages round(round(h_b * inverse_b) * gain) for the rows [b0, b0 + R G)
// that exist (below B) of width D = 128 * kNormK into the staged LDS layouts
// for P = 16 (when S16) and P = 32 (when S32), computing inverse_b with the
// reference tree (normalization.cu:134-186) in the same pass.  Thread group
// g (threads 128 g .. 128 g + 127) owns rows b0 + R g .. b0 + R g + R - 1:
// thread t of the group keeps features t + 128k of its rows in registers, sums
// their squares in ascending k (component t), combines groups of four left
// to right, and the group's first wavefront reduces the 32 lane totals of
// each row with shuffle-down offsets 1..16.  The width and the layouts are
// compile-time so that loads, sums and LDS stores are straight-line code
// with every load in flight at once.  `scratch` holds 80 G floats of LDS.
constexpr int kNormK = 32;
constexpr int kNormWidth = 128 * kNormK;

template <int R, bool S16, bool S32, int G, class Issue>
__device__ __forceinline__ bool norm_stage_pass(const uint16_t* __restrict__ h, const uint16_t* __restrict__ gain,
                                                float eps, float* xs16, float* xs32, float* scratch, int b0, int B,
                                                Issue&& issue, const uint32_t* active) {
  constexpr int D = kNormWidth;
  const uint32_t live = active ? *active : 1u;
  const int tid = threadIdx.x, t = tid % 128, g = tid / 128;
  static_assert(R == 1 || R == 2, "a thread group owns one or two rows");
  const int r0 = b0 + R * g;
  const bool has0 = g < G && r0 < B, has1 = R == 2 && g < G && r0 + 1 < B;
  const int r1 = has1 ? r0 + 1 : r0;  // a missing second row repeats the first (never staged)
  float hv[R][kNormK];
  float gv[kNormK];
  if (has0) {
#pragma unroll
    for (int k = 0; k < kNormK; ++k) {
      gv[k] = dl_bf16_to_f32(gain[t + 128 * k]);
      hv[0][k] = dl_bf16_to_f32(h[r0 * D + t + 128 * k]);
      if constexpr (R == 2) hv[R - 1][k] = dl_bf16_to_f32(h[r1 * D + t + 128 * k]);
    }
  }
  // Loads retire in order: the caller's own traffic (the first weight batch)
  // goes after the row loads, and its latency overlaps the math below.
  __builtin_amdgcn_sched_barrier(0);
  issue();
  __builtin_amdgcn_sched_barrier(0);
  if (!live) return false;
  if (has0) {
#pragma unroll
    for (int b = 0; b < R; ++b) {
      float comp = 0.0f;
#pragma unroll
      for (int k = 0; k < kNormK; ++k) comp = comp + hv[b][k] * hv[b][k];
      const float second = row_down<1>(comp);
      const float third = row_down<2>(comp);
      const float fourth = row_down<3>(comp);
      if ((t & 3) == 0) scratch[(R * g + b) * 40 + (t >> 2)] = ((comp + second) + third) + fourth;
    }
  }
  __syncthreads();
  if (has0 && t < 32 * R) {
    const int slot = R * g + t / 32;
    const float s = tree_sum32(scratch[slot * 40 + (t & 31)]);
    if ((t & 31) == 0) scratch[slot * 40 + 32] = inverse_sqrt(s * (1.0f / static_cast<float>(D)) + eps);
  }
  __syncthreads();
  if (has0) {
#pragma unroll
    for (int b = 0; b < R; ++b) {
      if (b == 1 && !has1) break;
      const float inverse = scratch[(R * g + b) * 40 + 32];
#pragma unroll
      for (int k = 0; k < kNormK; ++k) {
        const float n = dl_round_bf16(dl_round_bf16(hv[b][k] * inverse) * gv[k]);
        const int col = t + 128 * k;
        if constexpr (S16) stage_put<16>(xs16, D, r0 + b, col, n);
        if constexpr (S32) stage_put<32>(xs32, D, r0 + b, col, n);
      }
    }
  }
  return true;
}

// norm_stage_pass over B rows, R G at a time (R = 1 row per group while the
// G groups cover the B rows in one pass, else 2) (scratch is reused between
// passes behind a barrier); G = threads / 128 of the calling workgroup.
// Rows have width kNormWidth.  Returns false, before any math, when the
// loop word `active` (read in the first pass, as in stage_rows) is zero.
// Only the first `rows` (at most B) rows exist and are read and staged; the
// staged slots of the others are left as they are.
template <int B, bool S16, bool S32, int G, class Issue>
__device__ __forceinline__ bool norm_stage(const uint16_t* __restrict__ h, const uint16_t* __restrict__ gain,
                                           float eps, float* xs16, float* xs32, float* scratch, Issue&& issue,
                                           const uint32_t* active = nullptr, int rows = B) {
  constexpr int R = B <= G ? 1 : 2;
  auto none = [] {};
#pragma unroll
  for (int b0 = 0; b0 < B; b0 += R * G) {
    if (b0) {
      __syncthreads();
      norm_stage_pass<R, S16, S32, G>(h, gain, eps, xs16, xs32, scratch, b0, rows, none, nullptr);
    } else if (!norm_stage_pass<R, S16, S32, G>(h, gain, eps, xs16, xs32, scratch, b0, rows, issue, active)) {
      return false;
    }
  }
  return true;
}

}  // namespace dl
