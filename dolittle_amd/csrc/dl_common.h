/*
 * Storage conversion shared by the host runtime and the gfx950 kernels.
 *
 * BF16 is a stored-bit format (src/tensors/representations/bf16.cpp:43-55):
 * widening shifts the 16 stored bits into the high half of a binary32;
 * narrowing rounds to nearest, ties to even, and canonicalises every NaN to
 * 0x7fc0.  `dl_round_bf16` narrows and widens again, which is how every
 * explicit storage-rounding point of the reference contract is expressed
 * (src/kernels/cuda/common.cuh:68-92 `storage_round`).
 *
 * The header is plain C/C++ so that the same definitions compile for the
 * host (gcc/clang) and for the device (hipcc).  Floating-point code that
 * includes it must be compiled with -ffp-contract=off: every fused
 * multiply-add in this project is written explicitly.
 */
#ifndef DL_COMMON_H
#define DL_COMMON_H

#include <stdint.h>
#include <string.h>

#if defined(__HIPCC__)
#define DL_HD __host__ __device__ __forceinline__
#else
#define DL_HD static inline
#endif

DL_HD float dl_bits_to_f32(uint32_t u) {
#if defined(__HIP_DEVICE_COMPILE__)
  return __uint_as_float(u);
#else
  float f;
  memcpy(&f, &u, sizeof f);
  return f;
#endif
}

DL_HD uint32_t dl_f32_to_bits(float f) {
#if defined(__HIP_DEVICE_COMPILE__)
  return __float_as_uint(f);
#else
  uint32_t u;
  memcpy(&u, &f, sizeof u);
  return u;
#endif
}

DL_HD double dl_bits_to_f64(uint64_t u) {
#if defined(__HIP_DEVICE_COMPILE__)
  return __longlong_as_double((long long)u);
#else
  double d;
  memcpy(&d, &u, sizeof d);
  return d;
#endif
}

DL_HD uint64_t dl_f64_to_bits(double d) {
#if defined(__HIP_DEVICE_COMPILE__)
  return (uint64_t)__double_as_longlong(d);
#else
  uint64_t u;
  memcpy(&u, &d, sizeof u);
  return u;
#endif
}

/* Exact widening of stored BF16 bits. */
DL_HD float dl_bf16_to_f32(uint16_t b) { return dl_bits_to_f32((uint32_t)b << 16); }

/* Round-to-nearest-even narrowing; NaN inputs map to the canonical 0x7fc0. */
DL_HD uint16_t dl_f32_to_bf16(float v) {
  const uint32_t bits = dl_f32_to_bits(v);
  if ((bits & 0x7fffffffu) > 0x7f800000u) return (uint16_t)0x7fc0u;
  const uint32_t rounded = bits + 0x7fffu + ((bits >> 16) & 1u);
  return (uint16_t)(rounded >> 16);
}

/* One explicit storage-rounding point: narrow to BF16 and widen again. */
DL_HD float dl_round_bf16(float v) { return dl_bf16_to_f32(dl_f32_to_bf16(v)); }

/* Low / high BF16 element of a little-endian 32-bit word, widened. */
DL_HD float dl_bf16_lo(uint32_t word) { return dl_bits_to_f32(word << 16); }
DL_HD float dl_bf16_hi(uint32_t word) { return dl_bits_to_f32(word & 0xffff0000u); }

#endif /* DL_COMMON_H */
