/*
 * CPU oracle for the Qwen3-8B token loop: TEST INFRASTRUCTURE ONLY.
 *
 * Nothing in the product (dolittle_amd/) links, loads or calls this code.
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use
 * it, always as the checker or as the timed CPU baseline, never as the thing
 * being measured or shipped.
 *
 * Three independent restatements live here:
 *
 *  1. The contract mirror (contract.c and nla.c, prefix `orc_`): the
 *     reference CUDA operators restated on the CPU with their exact
 *     reduction trees and BF16 rounding points, so the GPU path can be
 *     compared bit for bit.
 *     Transcendentals come from dolittle_amd/csrc/dl_math.h because the
 *     reference leaves them to each backend's native library (unpinned); the
 *     shared implementation is itself pinned against glibc by the tests.
 *  2. The serial FP32 reference (serial.c, prefix `ors_`): the independent
 *     per-operator equations of tests/gpu/operator_reference.cpp:167-314,
 *     with glibc transcendentals and plain left-to-right FP32 sums.  It pins
 *     the contract mirror within the reference's per-operator tolerances
 *     (docs/architecture/numerical-portability.md:47-52).
 *  3. The host sampler law (sampling.c, prefix `ors_`/`or_mt`): the
 *     categorical law of src/inference/sampling/categorical.cpp:146-201 and
 *     the standard MT19937-64 engine (src/inference/sampling/sampler.h:52).
 *
 * All BF16 tensors are passed as uint16_t bit patterns, row-major, exactly
 * as the reference lays them out (W[O,I], Q[B,Hq,d], K/V[C,Hkv,d]).
 */
#ifndef DL_ORACLE_H
#define DL_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- BF16 (src/tensors/representations/bf16.cpp:43-55) ---- */
uint16_t or_bf16_from_f32(float v);
float or_f32_from_bf16(uint16_t b);

/* ---- contract mirror: single operators ---- */
/* projection.cu:1-67,277-361; transformer-execution.md:122-137 */
void orc_projection(const uint16_t* x, const uint16_t* w, uint16_t* y, size_t rows, size_t in_w,
                    size_t out_w);
/* normalization.cu:1-35,82-186 */
void orc_rms_norm(const uint16_t* x, const uint16_t* w, uint16_t* y, size_t rows, size_t width,
                  float eps);
/* The inverse RMS of one row (the reduction above, exposed for tests). */
float orc_rms_inverse(const uint16_t* x, size_t width, float eps);
/* rotary.cu:10-21,84-126 (x and y are [positions, heads, width]) */
void orc_rotary(const uint16_t* x, uint16_t* y, size_t positions, size_t heads, size_t width,
                size_t first_position, double theta);
/* attention.cu:231-383,436-439.  K and V rows: element (j, g, f) at
 * k[j*pos_stride + g*head_stride + f]; the reference layout [C,Hkv,d] has
 * pos_stride = Hkv*d and head_stride = d. */
void orc_attention(const uint16_t* q, const uint16_t* k, const uint16_t* v, uint16_t* y,
                   size_t positions, size_t q_heads, size_t kv_heads, size_t width,
                   size_t first_position, size_t pos_stride, size_t head_stride);
float orc_attention_scale(size_t width);
/* elementwise.cu:2-18,62-87 */
void orc_add(const uint16_t* a, const uint16_t* b, uint16_t* y, size_t n);
/* h <- BF16(FP32(h) + v): all-position residual steering (steering.cu:69-159,
 * the fixed-vector variant). */
void orc_steer(uint16_t* h, const float* v, size_t n);
void orc_silu_multiply(const uint16_t* gate, const uint16_t* up, uint16_t* y, size_t n);
/* embedding.cu:60-80 */
void orc_embedding(const uint32_t* tokens, const uint16_t* table, uint16_t* y, size_t rows,
                   size_t width);

/* ---- contract mirror: Qwen3 composition (src/models/qwen3/model.cpp:343-409) ---- */
typedef struct orc_qwen3_dims {
  uint32_t hidden, q_heads, kv_heads, head_dim, ffn, vocab;
  float eps;
  double theta;
} orc_qwen3_dims;

typedef struct orc_qwen3_block {
  const uint16_t *input_norm, *wq, *wk, *wv, *q_norm, *k_norm, *wo, *post_norm, *wg, *wu, *wd;
} orc_qwen3_block;

/* Runs one block for `rows` consecutive positions first_position.. on the
 * residual rows h[rows, hidden] in place.  The block's K (post-RoPE) and V
 * rows are written into the per-layer caches k_cache/v_cache laid out as
 * [capacity, kv_heads, head_dim] before attention reads them. */
void orc_qwen3_block_forward(const orc_qwen3_dims* dims, const orc_qwen3_block* block,
                             uint16_t* h, size_t rows, size_t first_position, uint16_t* k_cache,
                             uint16_t* v_cache);

/* Final RMSNorm of one residual row followed by the LM head projection. */
void orc_qwen3_logits(const orc_qwen3_dims* dims, const uint16_t* final_norm,
                      const uint16_t* lm_head, const uint16_t* h_row, uint16_t* logits);

/* ---- NLA vectors (nla.c): injection.cu:49-98, steering.cu:69-159 ----
 * Element arrays are BF16 bits (bf16 != 0) or FP32.  orc_inject returns the
 * status word (writes no output when the source or norm is invalid);
 * orc_direction returns the status and writes the FP32 direction only when
 * it is 0; orc_intervene returns 1 when `selected` lies in the chunk (then
 * state[0] is the status latch and state[1] the application count). */
uint32_t orc_inject(const void* source, int source_bf16, void* output, int output_bf16, size_t width, float scale,
                    float* norm);
uint32_t orc_direction(const void* original, const void* edited, int bf16, size_t width, float* direction);
int orc_intervene(void* residual, int bf16, size_t rows, size_t width, const float* direction, size_t first,
                  size_t selected, float strength, uint32_t* state);

/* Greedy choice over BF16 logits: maximum value, lowest id on ties
 * (categorical.cpp:168-173).  Returns 0 on success, 1 on NaN/+inf, 2 when no
 * finite candidate exists. */
int orc_greedy_bf16(const uint16_t* logits, size_t n, uint32_t* id);

/* ---- independent serial FP32 reference (operator_reference.cpp:167-314) ---- */
void ors_projection(const uint16_t* x, const uint16_t* w, uint16_t* y, size_t rows, size_t in_w,
                    size_t out_w);
void ors_rms_norm(const uint16_t* x, const uint16_t* w, uint16_t* y, size_t rows, size_t width,
                  float eps);
void ors_rotary(const uint16_t* x, uint16_t* y, size_t positions, size_t heads, size_t width,
                size_t first_position, double theta);
void ors_attention(const uint16_t* q, const uint16_t* k, const uint16_t* v, uint16_t* y,
                   size_t positions, size_t q_heads, size_t kv_heads, size_t width,
                   size_t first_position, size_t pos_stride, size_t head_stride);
void ors_silu_multiply(const uint16_t* gate, const uint16_t* up, uint16_t* y, size_t n);

/* ---- sampler law (categorical.cpp:146-201) and MT19937-64 ---- */
typedef struct or_mt64 {
  uint64_t words[312];
  uint32_t index;
} or_mt64;
void or_mt64_seed(or_mt64* state, uint64_t seed);
uint64_t or_mt64_next(or_mt64* state);

/* mode 0 = greedy, 1 = categorical.  Returns 0 and writes *id on success;
 * 1 for a NaN/+inf logit; 2 when every logit is -inf; 3 for invalid
 * settings.  Categorical selection consumes exactly one draw. */
int ors_categorical_select(const float* logits, size_t n, int mode, double temperature,
                           size_t top_k, double top_p, or_mt64* rng, uint32_t* id);
/* Same law given the 64-bit draw directly (no engine state). */
int ors_categorical_select_bits(const float* logits, size_t n, int mode, double temperature,
                                size_t top_k, double top_p, uint64_t draw_bits, uint32_t* id);

/* Same law with the weight exp chosen: build_exp 0 = glibc exp (the
 * reference host), 1 = the build's dl_exp (the device's serial replay). */
int ors_categorical_select_bits_exp(const float* logits, size_t n, int mode, double temperature,
                                    size_t top_k, double top_p, uint64_t draw_bits, int build_exp,
                                    uint32_t* id);
/* The categorical law's serial quantities for building boundary cases:
 * kept ids in sorted order (size), fold[k-1] = F_k, the cutoff count and
 * cumulative[i-1] = G_i for i <= count.  Arrays hold n entries. */
int ors_categorical_trace(const float* logits, size_t n, double temperature, size_t top_k,
                          double top_p, int build_exp, uint32_t* ids, double* fold,
                          double* cumulative, size_t* size, size_t* count);

/* ---- synthetic inputs (dolittle_amd/csrc/dl_synth.h), regenerated on the CPU ---- */
void or_fill_normal_bf16(uint16_t* out, size_t n, uint64_t seed, uint64_t stream, float scale,
                         size_t first_index);

/* Number of worker threads used by the heavy loops (0 = all online CPUs). */
void or_set_threads(int threads);

/* Shared deterministic math over arrays (for tests). */
void or_math_exp(const double* x, double* y, size_t n);
void or_math_expf(const float* x, float* y, size_t n);
void or_math_log(const double* x, double* y, size_t n);
void or_math_sincos(const double* x, double* s, double* c, size_t n);
void or_math_pow(const double* b, const double* e, double* y, size_t n);

/* RoPE cos/sin (BF16-rounded, widened) for one absolute position. */
void orc_rope_angles(size_t position, size_t width, double theta, float* cosv, float* sinv);

#ifdef __cplusplus
}
#endif

#endif /* DL_ORACLE_H */
