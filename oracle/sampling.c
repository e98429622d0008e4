/*
 * TEST INFRASTRUCTURE ONLY: the host sampling law and MT19937-64.
 *
 * ors_categorical_select restates src/inference/sampling/categorical.cpp:
 * 146-201: finite candidates only (NaN or +inf rejects the row), greedy is
 * the largest value with the lowest id, categorical sorts by descending value
 * (signed zeros equal) and ascending id, keeps the first top_k, weighs each
 * candidate by exp((z - z0) / T) in binary64, sums the weights serially in
 * that order, keeps the smallest prefix whose running sum / total reaches
 * top_p, draws u = (x >> 11) * 2^-53 and returns the first candidate whose
 * serial sum of weight/retained exceeds u (the last kept one otherwise).
 *
 * or_mt64_* is the standard MT19937-64 engine (std::mt19937_64, the
 * RandomStream of src/inference/sampling/sampler.h:52).
 */
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "../dolittle_amd/csrc/dl_math.h"
#include "oracle.h"

void or_mt64_seed(or_mt64* s, uint64_t seed) {
  s->words[0] = seed;
  for (uint32_t i = 1; i < 312; ++i) {
    const uint64_t prev = s->words[i - 1];
    s->words[i] = 6364136223846793005ull * (prev ^ (prev >> 62)) + i;
  }
  s->index = 312;
}

uint64_t or_mt64_next(or_mt64* s) {
  if (s->index >= 312) {
    for (uint32_t i = 0; i < 312; ++i) {
      const uint64_t x = (s->words[i] & 0xffffffff80000000ull) | (s->words[(i + 1) % 312] & 0x7fffffffull);
      uint64_t xa = x >> 1;
      if (x & 1u) xa ^= 0xb5026f5aa96619e9ull;
      s->words[i] = s->words[(i + 156) % 312] ^ xa;
    }
    s->index = 0;
  }
  uint64_t y = s->words[s->index++];
  y ^= (y >> 29) & 0x5555555555555555ull;
  y ^= (y << 17) & 0x71d67fffeda60000ull;
  y ^= (y << 37) & 0xfff7eee000000000ull;
  y ^= y >> 43;
  return y;
}

typedef struct candidate {
  uint32_t id;
  float value;
  double weight;
} candidate;

/* Descending value, signed zeros equal, then ascending id. */
static int order(const void* pa, const void* pb) {
  const candidate* a = (const candidate*)pa;
  const candidate* b = (const candidate*)pb;
  if (a->value != b->value) return a->value > b->value ? -1 : 1;
  return a->id < b->id ? -1 : (a->id > b->id);
}

static int valid_settings(int mode, double temperature, double top_p, size_t top_k) {
  if (mode != 0 && mode != 1) return 0;
  if (!isfinite(temperature) || temperature <= 0) return 0;
  if (!isfinite(top_p) || top_p <= 0 || top_p > 1) return 0;
  if (mode == 0 && (temperature != 1 || top_k != 0 || top_p != 1)) return 0;
  return 1;
}

/* Weight exp: glibc's exp (the reference host, std::exp) or, for checking
 * the device's serial replay, the build's deterministic dl_exp. */
static double weight_exp(double x, int build_exp) { return build_exp ? dl_exp(x) : exp(x); }

/* Serial trace of the categorical law: sorted kept ids, the fold F_k of
 * the first k weights, the cutoff count and the cumulative draw sums G_i. */
typedef struct trace {
  uint32_t* ids;
  double* fold;
  double* cumulative;
  size_t size;
  size_t count;
} trace;

static int select_impl_exp(const float* logits, size_t n, int mode, double temperature, size_t top_k,
                           double top_p, or_mt64* rng, uint64_t bits, int build_exp, trace* out,
                           uint32_t* id) {
  if (!valid_settings(mode, temperature, top_p, top_k) || top_k > n) return 3;
  for (size_t i = 0; i < n; ++i)
    if (isnan(logits[i]) || (isinf(logits[i]) && logits[i] > 0)) return 1;
  candidate* c = (candidate*)malloc((n ? n : 1) * sizeof(candidate));
  size_t size = 0;
  for (size_t i = 0; i < n; ++i)
    if (isfinite(logits[i])) {
      c[size].id = (uint32_t)i;
      c[size].value = logits[i];
      c[size].weight = 0;
      ++size;
    }
  if (size == 0) {
    free(c);
    return 2;
  }
  if (mode == 0) {
    size_t best = 0;
    for (size_t i = 1; i < size; ++i)
      if (c[i].value > c[best].value) best = i;
    *id = c[best].id;
    free(c);
    return 0;
  }
  qsort(c, size, sizeof(candidate), order);
  if (top_k && size > top_k) size = top_k;
  const double maximum = (double)c[0].value;
  double total = 0;
  for (size_t i = 0; i < size; ++i) {
    c[i].weight = weight_exp(((double)c[i].value - maximum) / temperature, build_exp);
    total += c[i].weight;
    if (out) out->fold[i] = total;
  }
  double retained = 0;
  size_t count = 0;
  for (;;) {
    retained += c[count++].weight;
    if (!(count < size && retained / total < top_p)) break;
  }
  if (out) {
    out->size = size;
    out->count = count;
    double g = 0;
    for (size_t i = 0; i < size; ++i) out->ids[i] = c[i].id;
    for (size_t i = 0; i < count; ++i) {
      g += c[i].weight / retained;
      out->cumulative[i] = g;
    }
  }
  const uint64_t x = rng ? or_mt64_next(rng) : bits;
  const double u = (double)(x >> 11) * 0x1p-53;
  double cumulative = 0;
  uint32_t chosen = c[count - 1].id;
  for (size_t i = 0; i < count; ++i) {
    cumulative += c[i].weight / retained;
    if (u < cumulative) {
      chosen = c[i].id;
      break;
    }
  }
  *id = chosen;
  free(c);
  return 0;
}

int ors_categorical_select(const float* logits, size_t n, int mode, double temperature,
                           size_t top_k, double top_p, or_mt64* rng, uint32_t* id) {
  return select_impl_exp(logits, n, mode, temperature, top_k, top_p, rng, 0, 0, NULL, id);
}

int ors_categorical_select_bits(const float* logits, size_t n, int mode, double temperature,
                                size_t top_k, double top_p, uint64_t draw_bits, uint32_t* id) {
  return select_impl_exp(logits, n, mode, temperature, top_k, top_p, NULL, draw_bits, 0, NULL, id);
}

int ors_categorical_select_bits_exp(const float* logits, size_t n, int mode, double temperature,
                                    size_t top_k, double top_p, uint64_t draw_bits, int build_exp,
                                    uint32_t* id) {
  return select_impl_exp(logits, n, mode, temperature, top_k, top_p, NULL, draw_bits, build_exp, NULL,
                         id);
}

int ors_categorical_trace(const float* logits, size_t n, double temperature, size_t top_k,
                          double top_p, int build_exp, uint32_t* ids, double* fold,
                          double* cumulative, size_t* size, size_t* count) {
  trace t = {ids, fold, cumulative, 0, 0};
  uint32_t id = 0;
  const int status =
      select_impl_exp(logits, n, 1, temperature, top_k, top_p, NULL, 0, build_exp, &t, &id);
  *size = t.size;
  *count = t.count;
  return status;
}
