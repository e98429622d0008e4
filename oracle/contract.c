/*
 * TEST INFRASTRUCTURE ONLY: CPU contract mirror of the reference operators.
 *
 * Each function restates one reference CUDA operator with its exact
 * reduction order and BF16 rounding points (the "numerical contract" of
 * docs/architecture/transformer-execution.md:115-170).  The GPU kernels of
 * this build are required to reproduce these bits exactly.  Only the
 * transcendental kernels are shared with the product (dl_math.h): the
 * reference leaves them to the platform library, and the shared versions are
 * pinned against glibc by tests/test_oracle_kat.py (the math cases).
 *
 * Compile with -ffp-contract=off: every FMA below is an explicit fmaf().
 */
#include <math.h>
#include <omp.h>
#include <stdlib.h>
#include <string.h>

#include "../dolittle_amd/csrc/dl_math.h"
#include "oracle.h"

/* bf16.cpp:43-55: widen by shifting; narrow with RNE, NaN -> 0x7fc0. */
uint16_t or_bf16_from_f32(float v) {
  uint32_t bits;
  memcpy(&bits, &v, 4);
  if ((bits & 0x7fffffffu) > 0x7f800000u) return 0x7fc0u;
  return (uint16_t)((bits + 0x7fffu + ((bits >> 16) & 1u)) >> 16);
}

float or_f32_from_bf16(uint16_t b) {
  const uint32_t bits = (uint32_t)b << 16;
  float f;
  memcpy(&f, &bits, 4);
  return f;
}

static float rnd(float v) { return or_f32_from_bf16(or_bf16_from_f32(v)); }

void or_set_threads(int threads) {
  if (threads > 0) omp_set_num_threads(threads);
}

/* ------------------------------------------------------------------------
 * Projection (projection.cu:1-67, 277-361).
 * P = 16 when in_w <= 4096 and out_w > 1024, otherwise 32.  Partial t is an
 * FMA chain over features t, t+P, ... in ascending order from 0.  When in_w
 * is not a multiple of 16 the reference's tiled kernel zero-pads to a multiple
 * of 16 and the decode kernel emulates those padding FMAs
 * (projection.cu:295-304); the mirror applies the same fma(0, 0, acc).
 * Partials merge upper into lower at offsets P/2..1; the sum rounds once.
 * ---------------------------------------------------------------------- */
#define DEFINE_CHAIN(P)                                                              \
  static float chain_##P(const float* x, const float* w, size_t in_w) {              \
    float acc[P];                                                                    \
    for (int t = 0; t < P; ++t) acc[t] = 0.0f;                                       \
    const size_t full = in_w / P * P;                                                \
    for (size_t base = 0; base < full; base += P)                                    \
      for (int t = 0; t < P; ++t) acc[t] = fmaf(x[base + t], w[base + t], acc[t]);   \
    for (size_t t = 0; t < in_w - full; ++t) acc[t] = fmaf(x[full + t], w[full + t], acc[t]); \
    const size_t padded = (in_w + 15) / 16 * 16;                                     \
    if (padded != in_w) {                                                            \
      for (size_t t = in_w % P; t < (padded - 1) % P + 1; ++t) acc[t] = fmaf(0.0f, 0.0f, acc[t]); \
    }                                                                                \
    for (int off = P / 2; off; off >>= 1)                                            \
      for (int t = 0; t < off; ++t) acc[t] = acc[t] + acc[t + off];                  \
    return acc[0];                                                                   \
  }                                                                                  \
  /* Four output rows' chains side by side: each acc[i][t] is the same       */      \
  /* chain as chain_P on row i (same operands, same order); the rows are     */      \
  /* interleaved only so that independent FMAs overlap on the CPU.           */      \
  static void chain4_##P(const float* x, const float* w, size_t in_w, float* out) {  \
    float acc[4][P];                                                                 \
    for (int i = 0; i < 4; ++i)                                                      \
      for (int t = 0; t < P; ++t) acc[i][t] = 0.0f;                                  \
    const size_t full = in_w / P * P;                                                \
    for (size_t base = 0; base < full; base += P)                                    \
      for (int i = 0; i < 4; ++i)                                                    \
        for (int t = 0; t < P; ++t)                                                  \
          acc[i][t] = fmaf(x[base + t], w[i * in_w + base + t], acc[i][t]);          \
    for (int i = 0; i < 4; ++i) {                                                    \
      for (size_t t = 0; t < in_w - full; ++t)                                       \
        acc[i][t] = fmaf(x[full + t], w[i * in_w + full + t], acc[i][t]);            \
      const size_t padded = (in_w + 15) / 16 * 16;                                   \
      if (padded != in_w) {                                                          \
        for (size_t t = in_w % P; t < (padded - 1) % P + 1; ++t) acc[i][t] = fmaf(0.0f, 0.0f, acc[i][t]); \
      }                                                                              \
      for (int off = P / 2; off; off >>= 1)                                          \
        for (int t = 0; t < off; ++t) acc[i][t] = acc[i][t] + acc[i][t + off];       \
      out[i] = acc[i][0];                                                            \
    }                                                                                \
  }
DEFINE_CHAIN(16)
DEFINE_CHAIN(32)

static int projection_partials(size_t in_w, size_t out_w) {
  return (in_w <= 4096 && out_w > 1024) ? 16 : 32;
}

void orc_projection(const uint16_t* x, const uint16_t* w, uint16_t* y, size_t rows, size_t in_w,
                    size_t out_w) {
  const int P = projection_partials(in_w, out_w);
  float* xf = (float*)malloc(rows * in_w * sizeof(float));
  for (size_t i = 0; i < rows * in_w; ++i) xf[i] = or_f32_from_bf16(x[i]);
  const long groups = (long)((out_w + 3) / 4);
#pragma omp parallel
  {
    float* wf = (float*)malloc(4 * in_w * sizeof(float));
#pragma omp for schedule(static)
    for (long gi = 0; gi < groups; ++gi) {
      const size_t o0 = (size_t)gi * 4;
      const size_t n = out_w - o0 < 4 ? out_w - o0 : 4;
      for (size_t i = 0; i < n; ++i) {
        const uint16_t* wr = w + (o0 + i) * in_w;
        for (size_t k = 0; k < in_w; ++k) wf[i * in_w + k] = or_f32_from_bf16(wr[k]);
      }
      for (size_t r = 0; r < rows; ++r) {
        const float* xr = xf + r * in_w;
        if (n == 4) {
          float s[4];
          if (P == 16)
            chain4_16(xr, wf, in_w, s);
          else
            chain4_32(xr, wf, in_w, s);
          for (size_t i = 0; i < 4; ++i) y[r * out_w + o0 + i] = or_bf16_from_f32(s[i]);
        } else {
          for (size_t i = 0; i < n; ++i) {
            const float s = P == 16 ? chain_16(xr, wf + i * in_w, in_w) : chain_32(xr, wf + i * in_w, in_w);
            y[r * out_w + o0 + i] = or_bf16_from_f32(s);
          }
        }
      }
    }
    free(wf);
  }
  free(xf);
}

/* ------------------------------------------------------------------------
 * RMSNorm (normalization.cu:1-35, 82-186).  32 lanes x 4 components; for
 * width > 128 lane t, component c sums squares of features 4t+c+128k, for
 * width <= 128 it holds feature t+32c.  Squares and adds round separately.
 * Components combine left to right; lanes reduce with shuffle-down offsets
 * 1,2,4,8,16.  mean = total * FP32(1/width); inverse = 1/sqrt(mean + eps);
 * y = round(round(x * inverse) * w).
 * ---------------------------------------------------------------------- */
static float rms_inverse(const uint16_t* x, size_t width, float eps) {
  float comp[32][4];
  memset(comp, 0, sizeof comp);
  if (width <= 128) {
    for (int t = 0; t < 32; ++t)
      for (int c = 0; c < 4; ++c) {
        const size_t col = (size_t)t + 32u * (size_t)c;
        if (col < width) {
          const float v = or_f32_from_bf16(x[col]);
          comp[t][c] = v * v;
        }
      }
  } else {
    for (int t = 0; t < 32; ++t)
      for (size_t base = 4u * (size_t)t; base < width; base += 128)
        for (int c = 0; c < 4; ++c)
          if (base + (size_t)c < width) {
            const float v = or_f32_from_bf16(x[base + (size_t)c]);
            comp[t][c] = comp[t][c] + v * v;
          }
  }
  float lane[32];
  for (int t = 0; t < 32; ++t) lane[t] = ((comp[t][0] + comp[t][1]) + comp[t][2]) + comp[t][3];
  for (int off = 1; off < 32; off *= 2) {
    float next[32];
    for (int t = 0; t < 32; ++t) next[t] = lane[t] + (t + off < 32 ? lane[t + off] : lane[t]);
    memcpy(lane, next, sizeof lane);
  }
  const float mean = lane[0] * (1.0f / (float)width);
  return 1.0f / sqrtf(mean + eps);
}

float orc_rms_inverse(const uint16_t* x, size_t width, float eps) { return rms_inverse(x, width, eps); }

void orc_rms_norm(const uint16_t* x, const uint16_t* w, uint16_t* y, size_t rows, size_t width,
                  float eps) {
  for (size_t r = 0; r < rows; ++r) {
    const uint16_t* xr = x + r * width;
    const float inverse = rms_inverse(xr, width, eps);
    for (size_t i = 0; i < width; ++i) {
      const float normalized = rnd(or_f32_from_bf16(xr[i]) * inverse);
      y[r * width + i] = or_bf16_from_f32(normalized * or_f32_from_bf16(w[i]));
    }
  }
}

/* ------------------------------------------------------------------------
 * Rotary (rotary.cu:10-21, 84-126).  exponent = FP32(2i)/FP32(d);
 * f = FP32(1/pow(theta, exponent)) in binary64; angle = FP32(t) * f;
 * c = round(cos angle), s = round(sin angle); four rounded products, then
 * y_i = round(ac - bs), y_{i+d/2} = round(bc + as).
 * ---------------------------------------------------------------------- */
void orc_rope_angles(size_t position, size_t width, double theta, float* cosv, float* sinv) {
  for (size_t i = 0; i < width / 2; ++i) {
    const float exponent = (float)(2 * i) / (float)width;
    const float inverse_frequency = (float)(1.0 / dl_pow_pos(theta, (double)exponent));
    const float angle = (float)position * inverse_frequency;
    double s, c;
    dl_sincos((double)angle, &s, &c);
    cosv[i] = rnd((float)c);
    sinv[i] = rnd((float)s);
  }
}

void orc_rotary(const uint16_t* x, uint16_t* y, size_t positions, size_t heads, size_t width,
                size_t first_position, double theta) {
  const size_t half = width / 2;
  float* cosv = (float*)malloc(half * sizeof(float));
  float* sinv = (float*)malloc(half * sizeof(float));
  for (size_t p = 0; p < positions; ++p) {
    orc_rope_angles(first_position + p, width, theta, cosv, sinv);
    for (size_t h = 0; h < heads; ++h) {
      const size_t row = (p * heads + h) * width;
      for (size_t i = 0; i < half; ++i) {
        const float a = or_f32_from_bf16(x[row + i]);
        const float b = or_f32_from_bf16(x[row + i + half]);
        const float ac = rnd(a * cosv[i]), bs = rnd(b * sinv[i]);
        const float bc = rnd(b * cosv[i]), as = rnd(a * sinv[i]);
        y[row + i] = or_bf16_from_f32(ac - bs);
        y[row + i + half] = or_bf16_from_f32(bc + as);
      }
    }
  }
  free(cosv);
  free(sinv);
}

/* ------------------------------------------------------------------------
 * Causal GQA attention (attention.cu:231-383, 436-439).
 * score_j = (8 contiguous ceil(d/8)-feature FMA ranges merged at offsets
 * 4,2,1) * FP32(1/sqrt(d)); m = max; e_j = exp(s_j - m); 32 partials own
 * j mod 32 (ascending adds) merged at offsets 16..1; p_j = e_j / l; each
 * output feature is round(A + B) with A, B ascending FMA chains over the
 * first ceil(n/2) keys and the rest.
 * ---------------------------------------------------------------------- */
float orc_attention_scale(size_t width) { return (float)(1.0 / sqrt((double)width)); }

void orc_attention(const uint16_t* q, const uint16_t* k, const uint16_t* v, uint16_t* y,
                   size_t positions, size_t q_heads, size_t kv_heads, size_t width,
                   size_t first_position, size_t pos_stride, size_t head_stride) {
  const float scale = orc_attention_scale(width);
  const size_t span = width / 8 + (width % 8 != 0);
  const size_t group = q_heads / kv_heads;
  const long tasks = (long)(positions * q_heads);
#pragma omp parallel for schedule(dynamic, 1)
  for (long task = 0; task < tasks; ++task) {
    const size_t p = (size_t)task / q_heads, h = (size_t)task % q_heads;
    const size_t count = first_position + p + 1;
    const size_t g = h / group;
    float* qf = (float*)malloc(width * sizeof(float));
    float* scores = (float*)malloc(count * sizeof(float));
    const uint16_t* qr = q + (p * q_heads + h) * width;
    for (size_t f = 0; f < width; ++f) qf[f] = or_f32_from_bf16(qr[f]);
    for (size_t j = 0; j < count; ++j) {
      const uint16_t* kr = k + j * pos_stride + g * head_stride;
      float part[8];
      for (size_t l = 0; l < 8; ++l) {
        const size_t begin = l * span;
        const size_t end = begin < width ? (begin + span < width ? begin + span : width) : width;
        float acc = 0.0f;
        for (size_t f = begin; f < end; ++f) acc = fmaf(qf[f], or_f32_from_bf16(kr[f]), acc);
        part[l] = acc;
      }
      for (int off = 4; off; off >>= 1)
        for (int l = 0; l < off; ++l) part[l] = part[l] + part[l + off];
      scores[j] = part[0] * scale;
    }
    float maximum = scores[0];
    for (size_t j = 0; j < count; ++j) maximum = fmaxf(maximum, scores[j]);
    float denom[32];
    for (int t = 0; t < 32; ++t) denom[t] = 0.0f;
    for (size_t j = 0; j < count; ++j) {
      const float e = dl_expf(scores[j] - maximum);
      scores[j] = e;
      denom[j % 32] = denom[j % 32] + e;
    }
    for (int off = 16; off; off >>= 1)
      for (int t = 0; t < off; ++t) denom[t] = denom[t] + denom[t + off];
    const float l = denom[0];
    for (size_t j = 0; j < count; ++j) scores[j] = scores[j] / l;
    const size_t split = (count - 1) / 2 + 1;
    uint16_t* yr = y + (p * q_heads + h) * width;
    /* Feature f's two chains: first over keys [0, split), second over
     * [split, count), each in ascending key order.  The key loop is outside
     * the feature loop only so that the width chains advance side by side. */
    float* first = (float*)calloc(width, sizeof(float));
    float* second = (float*)calloc(width, sizeof(float));
    for (size_t j = 0; j < count; ++j) {
      const uint16_t* vr = v + j * pos_stride + g * head_stride;
      float* acc = j < split ? first : second;
      const float pj = scores[j];
      for (size_t f = 0; f < width; ++f) acc[f] = fmaf(pj, or_f32_from_bf16(vr[f]), acc[f]);
    }
    for (size_t f = 0; f < width; ++f) yr[f] = or_bf16_from_f32(first[f] + second[f]);
    free(first);
    free(second);
    free(qf);
    free(scores);
  }
}

/* ------------------------------------------------------------------------
 * Elementwise (elementwise.cu:2-18, 62-87) and embedding (embedding.cu:60-80).
 * sigmoid(a) = 1/(1+e^-a) for a >= 0, e^a/(1+e^a) otherwise;
 * y = round(round(a * sigmoid(a)) * b).
 * ---------------------------------------------------------------------- */
void orc_add(const uint16_t* a, const uint16_t* b, uint16_t* y, size_t n) {
  for (size_t i = 0; i < n; ++i) y[i] = or_bf16_from_f32(or_f32_from_bf16(a[i]) + or_f32_from_bf16(b[i]));
}

/* All-position steering of one row (the config-4 variant of
 * src/kernels/cuda/steering.cu:69-159 with a fixed FP32 vector): after the
 * block's second residual addition, h <- BF16(FP32(h) + v). */
void orc_steer(uint16_t* h, const float* v, size_t n) {
  for (size_t i = 0; i < n; ++i) h[i] = or_bf16_from_f32(or_f32_from_bf16(h[i]) + v[i]);
}

void orc_silu_multiply(const uint16_t* gate, const uint16_t* up, uint16_t* y, size_t n) {
  for (size_t i = 0; i < n; ++i) {
    const float a = or_f32_from_bf16(gate[i]);
    const float b = or_f32_from_bf16(up[i]);
    const float e = dl_expf(a >= 0.0f ? -a : a);
    const float sigmoid = a >= 0.0f ? 1.0f / (1.0f + e) : e / (1.0f + e);
    const float activated = rnd(a * sigmoid);
    y[i] = or_bf16_from_f32(activated * b);
  }
}

void orc_embedding(const uint32_t* tokens, const uint16_t* table, uint16_t* y, size_t rows,
                   size_t width) {
  for (size_t r = 0; r < rows; ++r) memcpy(y + r * width, table + (size_t)tokens[r] * width, width * 2);
}

/* ------------------------------------------------------------------------
 * Qwen3 block and head in recipe order (src/models/qwen3/model.cpp:343-409):
 * norm -> Q/K/V -> per-head norm + RoPE on Q and K -> cache append ->
 * attention -> O + residual -> norm -> gate/up -> SiLU*up -> down + residual.
 * ---------------------------------------------------------------------- */
void orc_qwen3_block_forward(const orc_qwen3_dims* dims, const orc_qwen3_block* b, uint16_t* h,
                             size_t rows, size_t first_position, uint16_t* k_cache,
                             uint16_t* v_cache) {
  const size_t D = dims->hidden, Hq = dims->q_heads, Hkv = dims->kv_heads, d = dims->head_dim;
  const size_t F = dims->ffn, QW = Hq * d, KW = Hkv * d;
  uint16_t* xn = (uint16_t*)malloc(rows * D * 2);
  uint16_t* qraw = (uint16_t*)malloc(rows * QW * 2);
  uint16_t* kraw = (uint16_t*)malloc(rows * KW * 2);
  uint16_t* qn = (uint16_t*)malloc(rows * QW * 2);
  uint16_t* kn = (uint16_t*)malloc(rows * KW * 2);
  uint16_t* qr = (uint16_t*)malloc(rows * QW * 2);
  uint16_t* att = (uint16_t*)malloc(rows * QW * 2);
  uint16_t* o = (uint16_t*)malloc(rows * D * 2);
  uint16_t* g = (uint16_t*)malloc(rows * F * 2);
  uint16_t* u = (uint16_t*)malloc(rows * F * 2);
  uint16_t* a = (uint16_t*)malloc(rows * F * 2);

  orc_rms_norm(h, b->input_norm, xn, rows, D, dims->eps);
  orc_projection(xn, b->wq, qraw, rows, D, QW);
  orc_projection(xn, b->wk, kraw, rows, D, KW);
  orc_projection(xn, b->wv, v_cache + first_position * KW, rows, D, KW);
  orc_rms_norm(qraw, b->q_norm, qn, rows * Hq, d, dims->eps);
  orc_rotary(qn, qr, rows, Hq, d, first_position, dims->theta);
  orc_rms_norm(kraw, b->k_norm, kn, rows * Hkv, d, dims->eps);
  orc_rotary(kn, k_cache + first_position * KW, rows, Hkv, d, first_position, dims->theta);
  orc_attention(qr, k_cache, v_cache, att, rows, Hq, Hkv, d, first_position, KW, d);
  orc_projection(att, b->wo, o, rows, QW, D);
  orc_add(h, o, h, rows * D);
  orc_rms_norm(h, b->post_norm, xn, rows, D, dims->eps);
  orc_projection(xn, b->wg, g, rows, D, F);
  orc_projection(xn, b->wu, u, rows, D, F);
  orc_silu_multiply(g, u, a, rows * F);
  orc_projection(a, b->wd, o, rows, F, D);
  orc_add(h, o, h, rows * D);

  free(xn); free(qraw); free(kraw); free(qn); free(kn); free(qr);
  free(att); free(o); free(g); free(u); free(a);
}

void orc_qwen3_logits(const orc_qwen3_dims* dims, const uint16_t* final_norm,
                      const uint16_t* lm_head, const uint16_t* h_row, uint16_t* logits) {
  uint16_t* xn = (uint16_t*)malloc(dims->hidden * 2);
  orc_rms_norm(h_row, final_norm, xn, 1, dims->hidden, dims->eps);
  orc_projection(xn, lm_head, logits, 1, dims->hidden, dims->vocab);
  free(xn);
}

/* categorical.cpp:168-173: greedy is the maximum finite value, lowest id on
 * ties; NaN and +inf are rejected; an all -inf row has no candidate. */
int orc_greedy_bf16(const uint16_t* logits, size_t n, uint32_t* id) {
  float best = 0.0f;
  long best_id = -1;
  for (size_t i = 0; i < n; ++i) {
    const float v = or_f32_from_bf16(logits[i]);
    if (isnan(v) || (isinf(v) && v > 0)) return 1;
    if (!isfinite(v)) continue;
    if (best_id < 0 || v > best) {
      best = v;
      best_id = (long)i;
    }
  }
  if (best_id < 0) return 2;
  *id = (uint32_t)best_id;
  return 0;
}

#include "../dolittle_amd/csrc/dl_synth.h"

void or_fill_normal_bf16(uint16_t* out, size_t n, uint64_t seed, uint64_t stream, float scale,
                         size_t first_index) {
#pragma omp parallel for schedule(static)
  for (long i = 0; i < (long)n; ++i) out[i] = dl_normal_bf16(seed, stream, first_index + (size_t)i, scale);
}

/* Array wrappers of the shared deterministic math, for pinning it against
 * an independent libm in the tests. */
void or_math_exp(const double* x, double* y, size_t n) {
  for (size_t i = 0; i < n; ++i) y[i] = dl_exp(x[i]);
}
void or_math_expf(const float* x, float* y, size_t n) {
  for (size_t i = 0; i < n; ++i) y[i] = dl_expf(x[i]);
}
void or_math_log(const double* x, double* y, size_t n) {
  for (size_t i = 0; i < n; ++i) y[i] = dl_log(x[i]);
}
void or_math_sincos(const double* x, double* s, double* c, size_t n) {
  for (size_t i = 0; i < n; ++i) dl_sincos(x[i], &s[i], &c[i]);
}
void or_math_pow(const double* b, const double* e, double* y, size_t n) {
  for (size_t i = 0; i < n; ++i) y[i] = dl_pow_pos(b[i], e[i]);
}
