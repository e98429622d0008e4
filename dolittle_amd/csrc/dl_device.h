// Device-side helpers shared by the gfx950 kernels.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "dl_common.h"
#include "dl_math.h"

namespace dl {

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));

// Storage-typed element access: uint16_t holds BF16 bits, float is FP32.
__device__ __forceinline__ float load_elem(const uint16_t* p, size_t i) { return dl_bf16_to_f32(p[i]); }
__device__ __forceinline__ float load_elem(const float* p, size_t i) { return p[i]; }
__device__ __forceinline__ void store_elem(uint16_t* p, size_t i, float v) { p[i] = dl_f32_to_bf16(v); }
__device__ __forceinline__ void store_elem(float* p, size_t i, float v) { p[i] = v; }

// One explicit storage-rounding point for storage type T.
template <class T>
__device__ __forceinline__ float storage_round(float v);
template <>
__device__ __forceinline__ float storage_round<uint16_t>(float v) {
  return dl_round_bf16(v);
}
template <>
__device__ __forceinline__ float storage_round<float>(float v) {
  return v;
}

__device__ __forceinline__ float fma_rn(float a, float b, float c) { return __builtin_fmaf(a, b, c); }

// The value of lane + kOff (1 <= kOff <= 15), moved within a 16-lane row by
// DPP (row_shl) instead of the LDS crossbar; lanes whose source lies past
// their row receive 0.  A reduction whose needed lanes only read lanes of
// their own row gets the same values as __shfl_down.
template <int kOff>
__device__ __forceinline__ float row_down(float v) {
  static_assert(kOff >= 1 && kOff <= 15, "DPP row shifts within 16 lanes");
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x100 + kOff, 0xf, 0xf, true));
}

// row_down for an order-free reduction: a lane whose source lies past its
// row keeps its own value (DPP with the lane disabled instead of reading 0).
template <int kOff>
__device__ __forceinline__ float row_down_keep(float v) {
  static_assert(kOff >= 1 && kOff <= 15, "DPP row shifts within 16 lanes");
  return __int_as_float(
      __builtin_amdgcn_update_dpp(__float_as_int(v), __float_as_int(v), 0x100 + kOff, 0xf, 0xf, false));
}

// The maximum over the 64 lanes of a wavefront, returned to every lane.
// fmaxf is exact, so any tree gives the same value (a NaN input is ignored
// by every tree alike): DPP steps within each 16-lane row, then the four row
// maxima read from lanes 0, 16, 32 and 48.
__device__ __forceinline__ float wave_max(float v) {
  v = fmaxf(v, row_down_keep<1>(v));
  v = fmaxf(v, row_down_keep<2>(v));
  v = fmaxf(v, row_down_keep<4>(v));
  v = fmaxf(v, row_down_keep<8>(v));
  const int b = __float_as_int(v);
  const float r0 = __int_as_float(__builtin_amdgcn_readlane(b, 0));
  const float r1 = __int_as_float(__builtin_amdgcn_readlane(b, 16));
  const float r2 = __int_as_float(__builtin_amdgcn_readlane(b, 32));
  const float r3 = __int_as_float(__builtin_amdgcn_readlane(b, 48));
  return fmaxf(fmaxf(r0, r1), fmaxf(r2, r3));
}

// The adjacent-first tree over 32 lanes (offsets 1, 2, 4, 8, 16 as
// __shfl_down(s, off, 32)); lane 0 of each 32-lane half holds the total.
// Offsets below 16 stay in the row of the lanes that feed lane 0.
__device__ __forceinline__ float tree_sum32(float s) {
  s = s + row_down<1>(s);
  s = s + row_down<2>(s);
  s = s + row_down<4>(s);
  s = s + row_down<8>(s);
  return s + __shfl_down(s, 16, 32);
}

// Streaming 16-byte load that bypasses cache retention (weights are read once).
__device__ __forceinline__ u32x4 load_stream(const u32x4* p) { return __builtin_nontemporal_load(p); }

// 1/sqrt(x) from two correctly rounded IEEE operations (the reference's
// native rsqrtf is unpinned; this build fixes the value on host and device).
__device__ __forceinline__ float inverse_sqrt(float x) { return 1.0f / __builtin_sqrtf(x); }

// Reads the device-owned position when one is bound, else the host value.
__device__ __forceinline__ uint64_t position_or(const uint64_t* device_position, uint64_t host) {
  return device_position ? *device_position : host;
}

}  // namespace dl
