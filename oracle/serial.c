/*
 * TEST INFRASTRUCTURE ONLY: independent serial FP32 operator equations.
 *
 * Restates tests/gpu/operator_reference.cpp:167-314: plain left-to-right FP32
 * sums, glibc transcendentals, and only the storage rounding points the
 * reference equations apply.  This does NOT follow the CUDA reduction trees;
 * it is the independent check the contract mirror must agree with within the
 * per-operator tolerances of docs/architecture/numerical-portability.md:47-52.
 */
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "oracle.h"

static float rnd(float v) { return or_f32_from_bf16(or_bf16_from_f32(v)); }
static float wid(uint16_t b) { return or_f32_from_bf16(b); }

/* operator_reference.cpp:218-241 */
void ors_projection(const uint16_t* x, const uint16_t* w, uint16_t* y, size_t rows, size_t in_w,
                    size_t out_w) {
  for (size_t r = 0; r < rows; ++r)
    for (size_t o = 0; o < out_w; ++o) {
      float sum = 0;
      for (size_t i = 0; i < in_w; ++i) sum += wid(x[r * in_w + i]) * wid(w[o * in_w + i]);
      y[r * out_w + o] = or_bf16_from_f32(sum);
    }
}

/* operator_reference.cpp:167-192 */
void ors_rms_norm(const uint16_t* x, const uint16_t* w, uint16_t* y, size_t rows, size_t width,
                  float eps) {
  for (size_t r = 0; r < rows; ++r) {
    float sum = 0;
    for (size_t i = 0; i < width; ++i) {
      const float v = wid(x[r * width + i]);
      sum += v * v;
    }
    const float inverse = 1 / sqrtf(sum / (float)width + eps);
    for (size_t i = 0; i < width; ++i)
      y[r * width + i] = or_bf16_from_f32(rnd(wid(x[r * width + i]) * inverse) * wid(w[i]));
  }
}

/* operator_reference.cpp:242-272 */
void ors_rotary(const uint16_t* x, uint16_t* y, size_t positions, size_t heads, size_t width,
                size_t first_position, double theta) {
  for (size_t row = 0; row < positions; ++row)
    for (size_t i = 0; i < width / 2; ++i) {
      const float frequency = (float)pow(theta, -2.0 * (double)i / (double)width);
      const float angle = (float)(first_position + row) * frequency;
      const float c = rnd(cosf(angle));
      const float s = rnd(sinf(angle));
      for (size_t h = 0; h < heads; ++h) {
        const size_t a = (row * heads + h) * width + i, b = a + width / 2;
        const float xa = wid(x[a]), xb = wid(x[b]);
        y[a] = or_bf16_from_f32(rnd(xa * c) - rnd(xb * s));
        y[b] = or_bf16_from_f32(rnd(xb * c) + rnd(xa * s));
      }
    }
}

/* operator_reference.cpp:273-313 (causal prefix of each query row) */
void ors_attention(const uint16_t* q, const uint16_t* k, const uint16_t* v, uint16_t* y,
                   size_t positions, size_t q_heads, size_t kv_heads, size_t width,
                   size_t first_position, size_t pos_stride, size_t head_stride) {
  const float scale = (float)(1.0 / sqrt((double)width));
  const size_t group = q_heads / kv_heads;
  const size_t keys = first_position + positions;
  float* prob = (float*)malloc(keys * sizeof(float));
  for (size_t row = 0; row < positions; ++row)
    for (size_t h = 0; h < q_heads; ++h) {
      const size_t kv = h / group, count = first_position + row + 1;
      float maximum = -INFINITY;
      for (size_t j = 0; j < count; ++j) {
        float dot = 0;
        for (size_t i = 0; i < width; ++i)
          dot += wid(q[(row * q_heads + h) * width + i]) * wid(k[j * pos_stride + kv * head_stride + i]);
        prob[j] = dot * scale;
        if (prob[j] > maximum) maximum = prob[j];
      }
      float denominator = 0;
      for (size_t j = 0; j < count; ++j) {
        prob[j] = expf(prob[j] - maximum);
        denominator += prob[j];
      }
      for (size_t j = 0; j < count; ++j) prob[j] /= denominator;
      for (size_t i = 0; i < width; ++i) {
        float sum = 0;
        for (size_t j = 0; j < count; ++j) sum += prob[j] * wid(v[j * pos_stride + kv * head_stride + i]);
        y[(row * q_heads + h) * width + i] = or_bf16_from_f32(sum);
      }
    }
  free(prob);
}

/* operator_reference.cpp:193-217 */
void ors_silu_multiply(const uint16_t* gate, const uint16_t* up, uint16_t* y, size_t n) {
  for (size_t i = 0; i < n; ++i) {
    const float g = wid(gate[i]);
    y[i] = or_bf16_from_f32(rnd(g / (1 + expf(-g))) * wid(up[i]));
  }
}
