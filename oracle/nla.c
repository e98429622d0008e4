/*
 * TEST INFRASTRUCTURE ONLY.  CPU restatement of the NLA vector operations
 * (part of the contract mirror, prefix `orc_`):
 *   orc_inject     src/kernels/cuda/injection.cu:49-98 (law H2,
 *                  docs/architecture/execution-boundary.md:489-498)
 *   orc_direction  src/kernels/cuda/steering.cu:69-100
 *   orc_intervene  src/kernels/cuda/steering.cu:107-159
 * Compiled with -ffp-contract=off: every multiply, add, subtract, divide and
 * sqrt below is one correctly rounded binary32 operation, as the reference's
 * __fmul_rn/__fadd_rn/__fsub_rn/__fdiv_rn/__fsqrt_rn.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

#include "oracle.h"

#define NLA_LANES 8

static float widen(const void* p, int bf16, size_t i) {
  return bf16 ? or_f32_from_bf16(((const uint16_t*)p)[i]) : ((const float*)p)[i];
}

/* Narrowing to the storage type; returns the stored value widened again. */
static float narrow_store(void* p, int bf16, size_t i, float v) {
  if (bf16) {
    const uint16_t b = or_bf16_from_f32(v);
    ((uint16_t*)p)[i] = b;
    return or_f32_from_bf16(b);
  }
  ((float*)p)[i] = v;
  return v;
}

/* Lane k sums value(i)^2 over i = k, k + 8, ... ascending (separate multiply
 * and add); lanes 0..7 are then added left to right (injection.cu:62-80,
 * steering.cu:72-91, steering.cu:121-137). */
static float strided_square_sum(const void* a, const void* b, int bf16, size_t width, int difference,
                                int* nonfinite) {
  float lane[NLA_LANES];
  for (size_t k = 0; k < NLA_LANES; ++k) {
    float sum = 0.0f;
    for (size_t i = k; i < width; i += NLA_LANES) {
      const float v = difference ? widen(b, bf16, i) - widen(a, bf16, i) : widen(a, bf16, i);
      if (nonfinite && !isfinite(v)) *nonfinite = 1;
      const float sq = v * v;
      sum = sum + sq;
    }
    lane[k] = sum;
  }
  float total = 0.0f;
  for (size_t k = 0; k < NLA_LANES; ++k) total = total + lane[k];
  return total;
}

uint32_t orc_inject(const void* source, int source_bf16, void* output, int output_bf16, size_t width, float scale,
                    float* norm) {
  int invalid = 0;
  const float sum = strided_square_sum(source, NULL, source_bf16, width, 0, &invalid);
  const float n = sqrtf(sum);
  *norm = n;
  if (!isfinite(n) || n == 0.0f) invalid = 1;
  if (invalid) return 1;
  for (size_t i = 0; i < width; ++i) {
    const float q = widen(source, source_bf16, i) / n;
    const float value = q * scale;
    const float stored = narrow_store(output, output_bf16, i, value);
    if (!isfinite(value) || !isfinite(stored)) invalid = 1;
  }
  return (uint32_t)invalid;
}

uint32_t orc_direction(const void* original, const void* edited, int bf16, size_t width, float* direction) {
  const float sum = strided_square_sum(original, edited, bf16, width, 1, NULL);
  const float n = sqrtf(sum);
  if (!isfinite(n) || n == 0.0f) return 1;
  for (size_t i = 0; i < width; ++i) {
    const float d = widen(edited, bf16, i) - widen(original, bf16, i);
    direction[i] = d / n;
  }
  return 0;
}

int orc_intervene(void* residual, int bf16, size_t rows, size_t width, const float* direction, size_t first,
                  size_t selected, float strength, uint32_t* state) {
  if (selected < first || selected - first >= rows) return 0;
  int invalid = state[0] != 0 || state[1] != 0;
  state[1] += 1;
  const size_t r = selected - first;
  const size_t elem = bf16 ? 2 : 4;
  uint8_t* row = (uint8_t*)residual + r * width * elem;
  const float sum = strided_square_sum(row, NULL, bf16, width, 0, NULL);
  const float root = sqrtf(sum);
  const float beta = strength * root;
  if (!isfinite(beta)) invalid = 1;
  if (!invalid) {
    for (size_t i = 0; i < width; ++i) {
      const float product = beta * direction[i];
      const float value = widen(row, bf16, i) + product;
      const float stored = narrow_store(row, bf16, i, value);
      if (!isfinite(value) || !isfinite(stored)) invalid = 1;
    }
  }
  state[0] = (uint32_t)invalid;
  return 1;
}
