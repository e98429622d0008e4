/*
 * Seeded synthetic inputs for the benchmark configurations.
 *
 * The benchmark configurations use seeded random BF16 weights ~N(0, 0.02),
 * KV caches ~N(0, 1) and uniform random token ids.  Each value is a pure
 * function of (seed, stream, index), so a tensor can be generated in place
 * on the GPU and any element can be regenerated on the CPU for checking:
 *
 *   h(seed, stream, i) = mix(mix(seed ^ mix(stream)) + i)   (SplitMix64 mix)
 *   normal pair j (elements 2j, 2j+1) from Box-Muller on
 *     u1 = (h(.., 2j) >> 11 + 1) * 2^-53  in (0, 1]
 *     u2 = (h(.., 2j+1) >> 11) * 2^-53    in [0, 1)
 *     z_{2j} = sqrt(-2 ln u1) cos(2 pi u2), z_{2j+1} = sqrt(-2 ln u1) sin(2 pi u2)
 *   stored value = BF16(FP32(scale * z))
 *
 * ln, sin and cos are the deterministic implementations of dl_math.h, and
 * sqrt is the correctly rounded IEEE square root on both host and device,
 * so the host and device generators agree bit for bit.
 */
#ifndef DL_SYNTH_H
#define DL_SYNTH_H

#include "dl_math.h"

#if defined(__HIPCC__)
#define DL_SQRT(x) __builtin_sqrt(x)
#else
#define DL_SQRT(x) sqrt(x)
#endif

/* SplitMix64 output function (Steele, Lea and Flood 2014). */
DL_HD uint64_t dl_mix64(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
  z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
  return z ^ (z >> 31);
}

DL_HD uint64_t dl_hash3(uint64_t seed, uint64_t stream, uint64_t index) {
  return dl_mix64(dl_mix64(seed ^ dl_mix64(stream + 0x9e3779b97f4a7c15ull)) + index);
}

/* Standard normal sample for element `index` of stream `stream`. */
DL_HD double dl_normal(uint64_t seed, uint64_t stream, uint64_t index) {
  const uint64_t pair = index >> 1;
  const uint64_t a = dl_hash3(seed, stream, 2 * pair);
  const uint64_t b = dl_hash3(seed, stream, 2 * pair + 1);
  const double u1 = (double)((a >> 11) + 1) * 0x1p-53;
  const double u2 = (double)(b >> 11) * 0x1p-53;
  const double radius = DL_SQRT(-2.0 * dl_log(u1));
  double s, c;
  dl_sincos(DL_TWO_PI * u2, &s, &c);
  return radius * ((index & 1) ? s : c);
}

DL_HD uint16_t dl_normal_bf16(uint64_t seed, uint64_t stream, uint64_t index, float scale) {
  return dl_f32_to_bf16((float)((double)scale * dl_normal(seed, stream, index)));
}

/* Uniform id in [0, n) by multiply-shift of 32 random bits. */
DL_HD uint32_t dl_uniform_id(uint64_t seed, uint64_t stream, uint64_t index, uint32_t n) {
  const uint64_t h = dl_hash3(seed, stream, index);
  return (uint32_t)(((h >> 32) * (uint64_t)n) >> 32);
}

#endif /* DL_SYNTH_H */
