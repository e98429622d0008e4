// Qwen3 resident model, cached forward plan and device-owned token loop.
//
// Recipe (src/models/qwen3/model.cpp:343-409), per block:
//   x = RMSNorm(h); q,k,v = x Wq, x Wk, x Wv; q,k = RoPE(RMSNorm_head(q,k));
//   cache append; a = attention; h = h + a Wo; x = RMSNorm(h);
//   h = h + (SiLU(x Wg) * (x Wu)) Wd
// then final RMSNorm of the last row and the LM head.
//
// Kernel fusion (each fused kernel keeps every storage-rounding point of the
// unfused operations, so results equal the reference operator sequence):
//   k_step_begin   embedding lookup (or embedding override) into h
//   k_qkv          RMSNorm prologue + packed Q|K|V GEMV; V stored straight into
//                  the V cache (the reference's positioned output)
//   k_attn_qk      per-head QK RMSNorm + RoPE prologue, K cache append, scores
//   k_attn_softmax max, exp, 32-partial denominator, p = e / l
//   k_attn_pv      the two ascending PV key ranges
//   k_residual     packed O or down GEMV + residual add (+ steering, capture)
//   k_gateup       RMSNorm prologue + packed gate|up GEMV + SiLU*up
//   k_lm_head      final RMSNorm prologue + packed LM head + argmax partials
//   k_step_end     greedy selection, token stream, position and stop latches
// One decode step is captured once into a hipGraph and replayed; every kernel
// reads the device-owned position and exits at once when the loop is
// inactive, replacing the reference's conditional CUDA graph nodes
// (src/kernels/cuda/decode.cu:103-194, 339-353), which HIP lacks.
#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <memory>
#include <thread>
#include <type_traits>
#include <utility>
#include <vector>

#include "archive.h"
#include "dl_control.h"
#include "dl_device.h"
#include "dl_internal.h"
#include "dl_synth.h"
#include "gemv.h"
#include "heads.h"
#include "nla.h"
#include "prefill.h"
#include "sampler.h"

namespace dl {


namespace {

constexpr int kWaves = 4;
constexpr int kBlock = kWaves * 64;
// Wavefronts per workgroup of the GEMV kernels for `rows` staged rows.  From
// four rows the staged inputs fill most of the LDS, so one workgroup is
// resident per CU; eight wavefronts (two per SIMD) keep twice the weight
// loads in flight.
constexpr int gemv_waves(int rows) { return rows >= 4 ? 8 : kWaves; }
constexpr int kHeadDim = 128;

__device__ __forceinline__ uint16_t bf16_bits(float v) { return dl_f32_to_bf16(v); }
__device__ __forceinline__ float rbf(float v) { return dl_round_bf16(v); }

// SiluMultiply on BF16-rounded operands (elementwise.cu:62-87).
__device__ __forceinline__ float silu_times(float a, float b) {
  const float e = dl_expf(a >= 0.0f ? -a : a);
  const float sigmoid = a >= 0.0f ? 1.0f / (1.0f + e) : e / (1.0f + e);
  return rbf(a * sigmoid) * b;
}

// Step selects a token when the prompt is consumed and the budget is open.
__device__ __forceinline__ bool selecting(const Control* c) { return c->select_row != 0; }

// ------------------------------------------------------------ weight layout
// Which packed matrix an element of a logical parameter belongs to.
struct PackedView {
  uint16_t* base;   // packed storage of the (possibly combined) matrix
  int P;            // partials of the logical projection
  uint64_t cols;    // input width
  int combined;     // 0 plain, 1 gate rows, 2 up rows of the interleaved gate|up matrix
};

__host__ __device__ inline uint64_t view_index(const PackedView& v, uint64_t r, uint64_t k) {
  uint64_t R = r;
  if (v.combined == 1) R = 4 * (r / 2) + (r % 2);
  if (v.combined == 2) R = 4 * (r / 2) + 2 + (r % 2);
  return packed_index(R, k, v.P, v.cols);
}

// Seeded N(0, std) fill of a logical [rows, cols] matrix into its view.
__global__ void k_fill_view(PackedView v, uint64_t rows, uint64_t seed, uint64_t stream, float scale) {
  const uint64_t n = rows * v.cols;
  const uint64_t step = static_cast<uint64_t>(gridDim.x) * blockDim.x;
  for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += step) {
    const uint64_t r = i / v.cols, k = i % v.cols;
    v.base[view_index(v, r, k)] = dl_normal_bf16(seed, stream, i, scale);
  }
}

__global__ void k_fill_const(uint16_t* p, uint64_t n, uint16_t value) {
  const uint64_t step = static_cast<uint64_t>(gridDim.x) * blockDim.x;
  for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += step) p[i] = value;
}

// Row-major <-> packed transfers of one logical matrix.
__global__ void k_pack_view(PackedView v, uint64_t rows, const uint16_t* src, int unpack, uint16_t* dst) {
  const uint64_t n = rows * v.cols;
  const uint64_t step = static_cast<uint64_t>(gridDim.x) * blockDim.x;
  for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += step) {
    const uint64_t r = i / v.cols, k = i % v.cols;
    if (unpack)
      dst[i] = v.base[view_index(v, r, k)];
    else
      v.base[view_index(v, r, k)] = src[i];
  }
}

// RoPE cos/sin table rope[pos][i] = (round(cos a), round(sin a)) with
// a = FP32(pos) * FP32(1/pow(theta, FP32(2i)/FP32(d))) (rotary.cu:84-126).
__global__ void k_rope_table(float* rope, uint64_t positions, int width, double theta) {
  const int half = width / 2;
  const uint64_t n = positions * half;
  const uint64_t step = static_cast<uint64_t>(gridDim.x) * blockDim.x;
  for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += step) {
    const uint64_t pos = i / half;
    const int pair = static_cast<int>(i % half);
    const float exponent = static_cast<float>(2 * pair) / static_cast<float>(width);
    const float inverse_frequency = static_cast<float>(1.0 / dl_pow_pos(theta, static_cast<double>(exponent)));
    const float angle = static_cast<float>(pos) * inverse_frequency;
    double s, c;
    dl_sincos(static_cast<double>(angle), &s, &c);
    rope[2 * i] = rbf(static_cast<float>(c));
    rope[2 * i + 1] = rbf(static_cast<float>(s));
  }
}

// ----------------------------------------------------------- control kernels
// ----------------------------------------------------------- event journal
// DeviceSequence publication (decode.cu publish, :94-101): events are
// written into host-mapped memory with vector stores, then one system-scope
// release fence orders them before the per-sequence counters, which the
// host reads with acquire loads.  One thread writes all of a step's events.
__device__ void journal_write(const Journal& j, Control* c, int b, uint32_t kind, uint32_t status,
                              uint64_t position, uint64_t count, uint32_t token, float norm) {
  const uint32_t n = c->events[b];
  if (!j.events || n >= j.capacity) return;  // capacity covers prompt + 2 * generated + 4 events
  u32x4* dst = reinterpret_cast<u32x4*>(j.events + static_cast<uint64_t>(b) * j.capacity + n);
  const u32x4 lo = {kind, status, static_cast<uint32_t>(position), static_cast<uint32_t>(position >> 32)};
  const u32x4 hi = {static_cast<uint32_t>(count), static_cast<uint32_t>(count >> 32), token, __float_as_uint(norm)};
  dst[0] = lo;
  dst[1] = hi;
  c->events[b] = n + 1;
}

// Publishes the event counts of sequences [0, batch) and the loop's
// liveness and step count.
__device__ void journal_publish(const Journal& j, const Control* c, int batch) {
  if (!j.events) return;
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "");
  for (int b = 0; b < batch; ++b)
    __hip_atomic_store(&j.publication[b].completed, c->events[b], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
  __hip_atomic_store(&j.mirror->steps, c->steps, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
  __hip_atomic_store(&j.mirror->active, c->active, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}

// Terminal events of the sequences not yet terminal when the loop ends at
// `position` (decode.cu finish_sequence): failure on a latched status, eos
// for a sequence that selected a stop id, limit when the whole budget was
// produced and consumed, cancelled otherwise.
__device__ void journal_finish(const Journal& j, Control* c, int batch, uint64_t position) {
  for (int b = 0; b < batch; ++b) {
    if ((c->terminal_mask >> b) & 1u) continue;
    const uint32_t generated = c->row_generated[b];
    const uint32_t reason =
        c->status ? kFailure
                  : (generated && ((c->finished_mask >> b) & 1u))
                        ? kEos
                        : (position == static_cast<uint64_t>(c->prompt_length) + generated && generated == c->max_new)
                              ? kLimit
                              : kCancelled;
    journal_write(j, c, b, kTerminal, reason, position, generated, c->status, 0.0f);
    c->terminal_mask |= 1u << b;
  }
}

struct InitArgs {
  Control* ctl;
  uint64_t position;
  uint32_t prompt_length, max_new, batch, mode;
  int32_t capture_layer, steer_layer;
  uint32_t steer_mask, override_active, override_mask;
  uint64_t override_position;
  Journal journal;
  const uint32_t* injection_status;  // installed injection's status word, or null
  const float* injection_norm;       // its norm word
};

__global__ void k_init_control(InitArgs a) {
  Control c{};
  c.position = a.position;
  c.active = 1;
  c.prompt_length = a.prompt_length;
  c.generated = 0;
  c.max_new = a.max_new;
  c.stop_pending = a.max_new == 0 ? 1u : 0u;
  c.finished_mask = 0;
  c.all_mask = a.batch >= 32 ? 0xffffffffu : ((1u << a.batch) - 1u);
  c.status = 0;
  c.reason = 0;
  c.mode = a.mode;
  c.override_active = a.override_active;
  c.override_mask = a.override_mask;
  c.override_position = a.override_position;
  c.capture_layer = a.capture_layer;
  c.steer_layer = a.steer_layer;
  c.steer_mask = a.steer_mask;
  c.select_row = 0;
  // The journal opens with the injection's status (decode.cu decide_stage,
  // prefill) and, after a prompt pass, the positions it consumed.
  for (uint32_t b = 0; b < a.batch; ++b) {
    if (a.injection_status)
      journal_write(a.journal, &c, b, kInjection, *a.injection_status, 0, 0, 0, *a.injection_norm);
    if (a.position > 0) journal_write(a.journal, &c, b, kConsumed, 0, 0, a.position, 0, 0.0f);
  }
  *a.ctl = c;
  journal_publish(a.journal, &c, static_cast<int>(a.batch));
}

struct BeginArgs {
  Control* ctl;
  const uint32_t* tokens;       // absolute-position token history [cap]
  const uint32_t* selected;     // [B] last selection
  uint16_t* h;                  // [B][D]
  const uint16_t* lm_packed;    // tied: packed LM head (P = 16)
  const uint16_t* embedding;    // untied: row-major [V][D]
  const uint16_t* override_row; // [D]
  const uint32_t* cancel;       // host-mapped cancel word
  const uint32_t* injection_status;    // installed injection's status word, or null
  const uint32_t* intervention_state;  // [status, count] of the plan's intervention, or null
  int D;
  uint32_t V;
  int tied;
  Journal journal;
  int batch;
};

// Embedding (embedding.cu:60-80), the embedding override, and the step's
// decisions (decode.cu decide_stage / finish_consumption).  Grid: one block
// per sequence.  An invalid injection (its status gates the prompt) or a
// latched intervention failure ends the loop with reason failure before the
// step consumes anything.  Cancellation is read once per step, here: while
// the step would consume a prompt position nothing is pending and the loop
// ends before it; when it would consume a selected token, that token is
// still consumed ("a selection promises consumption") and no new one is
// selected, so the loop ends after this step.
__global__ __launch_bounds__(kBlock) void k_step_begin(BeginArgs a) {
  Control* c = a.ctl;
  if (!c->active) return;
  const uint64_t pos = c->position;
  const int b = blockIdx.x;
  if (b == 0 && threadIdx.x == 0) {
    uint32_t failed = 0;
    if (a.injection_status && *a.injection_status) failed |= 8u;
    if (a.intervention_state && a.intervention_state[0]) failed |= 16u;
    const bool cancelled = __hip_atomic_load(a.cancel, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM) != 0;
    if (failed || (cancelled && pos < c->prompt_length)) {
      c->status |= failed;
      c->select_row = 0;
      c->active = 0;
      c->reason = failed ? 3u : 2u;
      journal_finish(a.journal, c, a.batch, pos);
      journal_publish(a.journal, c, a.batch);
    } else {
      if (cancelled) {
        c->cancel_pending = 1;
        c->stop_pending = 1;
      }
      c->select_row = (pos + 1 >= c->prompt_length && !c->stop_pending) ? 1u : 0u;
      c->finished_before = c->finished_mask;
      c->select_mask = c->select_row ? (c->all_mask & ~c->finished_mask) : 0u;
    }
  }
  const uint32_t token = pos < c->prompt_length ? a.tokens[pos] : a.selected[b];
  uint16_t* out = a.h + static_cast<uint64_t>(b) * a.D;
  const bool override_row = c->override_active && pos == c->override_position && ((c->override_mask >> b) & 1u);
  if (override_row) {
    for (int k = threadIdx.x; k < a.D; k += blockDim.x) out[k] = a.override_row[k];
  } else if (token >= a.V) {
    for (int k = threadIdx.x; k < a.D; k += blockDim.x) out[k] = 0;
    if (threadIdx.x == 0) atomicOr(&c->status, 4u);
  } else if (a.tied) {
    for (int k = threadIdx.x; k < a.D; k += blockDim.x) out[k] = a.lm_packed[packed_index(token, k, 16, a.D)];
  } else {
    const uint16_t* row = a.embedding + static_cast<uint64_t>(token) * a.D;
    for (int k = threadIdx.x; k < a.D; k += blockDim.x) out[k] = row[k];
  }
}

// ------------------------------------------------------------- QKV GEMV
struct QkvArgs {
  const Control* ctl;
  const uint16_t* h;
  const uint16_t* norm;
  const u32x4* w;            // packed Q (P=16) | K (P=32) | V (P=32)
  uint16_t* q_out;           // [B][QW]
  uint16_t* k_out;           // [B][KW]
  uint16_t* v_cache;         // V^T of this layer, sequence 0: [KW][cap]
  uint64_t cache_seq_stride; // elements
  int D, QW, KW, cap;
  float eps;
  // Rows of the launch that exist (a launch of a larger row template for
  // fewer rows reads and writes only these; see live_rows).
  int rows = 1 << 30;
};

// Rows that exist in a launch of the B-row kernels given the launch's `rows`
// field.  Only the 4- and 8-row kernels run for fewer rows (the host takes
// one or two rows with kernels of that size), so for B <= 2 this is B and
// the row guards compile away.
template <int B>
__device__ __forceinline__ int live_rows(int rows) {
  if constexpr (B <= 2) {
    return B;
  } else {
    return rows < B ? rows : B;
  }
}

// Part: kQkvAll projects Q, K and V; at eight rows both staged layouts do
// not fit in LDS together, so kQkvQ (Q rows, P = 16 layout) and kQkvKV (K
// and V rows, P = 32 layout) run in separate workgroups (k_qkv_roles).
enum QkvPart : int { kQkvAll = 0, kQkvQ = 1, kQkvKV = 2 };
// Input width of the batch-1 GEMV paths that hold a wavefront's whole weight
// tile in registers (Qwen3-8B's hidden width).
constexpr int kWholeTileInputs = 4096;
constexpr int qkv_waves(int rows, int part) { return part == kQkvAll ? kWaves : gemv_waves(rows); }

// Split > 1 divides each tile's B rows into Split work items of B / Split
// rows (the same tile's weights, read by Split wavefronts): with one tile
// per wavefront the chain length per wavefront, not the CU count, bounds
// these launches at eight rows.
// `block` of `blocks` is the workgroup's place among the launch's
// workgroups of this part (k_qkv_roles runs the Q and K/V parts of eight
// rows in one launch).
template <int B, int Part, int Split>
__device__ __forceinline__ void qkv_rows(const QkvArgs& a, int block, int blocks) {
  constexpr int W = qkv_waves(B, Part);
  constexpr int BR = B / Split;
  static_assert(B % Split == 0, "rows split evenly");
  extern __shared__ float lds[];
  float* xs16 = lds;
  float* xs32 = Part == kQkvKV ? lds : xs16 + B * staged_floats(16, a.D);
  __shared__ float scratch[W * 40];
  const int wave = threadIdx.x / 64, lane = threadIdx.x % 64;
  const int q_tiles = a.QW / 4, k_tiles = a.KW / 2, total = q_tiles + 2 * k_tiles;
  const int S16 = a.D / 128, S32 = a.D / 256;
  const uint64_t q_chunks = static_cast<uint64_t>(S16) * 64;
  const uint64_t k_chunks = static_cast<uint64_t>(S32) * 64;
  (void)S16;
  auto tile_src = [&](int tile) -> const u32x4* {
    if (tile < q_tiles) return a.w + tile * q_chunks;
    int kt = tile - q_tiles;
    const bool is_v = kt >= k_tiles;
    if (is_v) kt -= k_tiles;
    return a.w + q_tiles * q_chunks + (is_v ? k_tiles : 0) * k_chunks + kt * k_chunks;
  };
  const int tile_begin = Part == kQkvKV ? q_tiles : 0, tile_end = Part == kQkvQ ? q_tiles : total;
  const int items = (tile_end - tile_begin) * Split;
  const int first = block * W + wave;
  if constexpr (B == 1 && Part == kQkvAll && Split == 1) {
    if (blocks * W >= items && a.D == kWholeTileInputs) {
      // One tile per wavefront, held in registers (32 chunks per lane for a
      // Q tile, 16 for K or V): the first 16 chunks are issued before the
      // prologue, the rest right after it, and the chains run from
      // registers; the same chain steps as chain_tile.
      const bool has = first < items;
      const int tile = tile_begin + first;
      const bool is_q = tile < q_tiles;
      constexpr int SQ = kWholeTileInputs / 128, SK = kWholeTileInputs / 256;
      u32x4 w[SQ];
      if (!norm_stage<1, true, true, W / 2>(
              a.h, a.norm, a.eps, xs16, xs32, scratch,
              [&] {
                if (has) {
                  const u32x4* src = tile_src(tile) + lane;
#pragma unroll
                  for (int s = 0; s < SK; ++s) w[s] = load_stream(src + s * 64);
                }
              },
              &a.ctl->active))
        return;
      if (has && is_q) {
        const u32x4* src = tile_src(tile) + lane;
#pragma unroll
        for (int s = SK; s < SQ; ++s) w[s] = load_stream(src + s * 64);
      }
      __syncthreads();
      if (!has) return;
      float acc[1] = {0.0f};
      if (is_q) {
        constexpr int P = 16, stride = kWholeTileInputs / P + kXsPad;
        const float* xt = xs16 + (lane % P) * stride;
#pragma unroll
        for (int s = 0; s < SQ; ++s) chain_step<1>(w[s], xt, P * stride, s, acc);
        chain_merge<P, 1>(acc);
        if (lane % P == 0) a.q_out[tile * 4 + lane / P] = bf16_bits(acc[0]);
      } else {
        constexpr int P = 32, stride = kWholeTileInputs / P + kXsPad;
        const float* xt = xs32 + (lane % P) * stride;
#pragma unroll
        for (int s = 0; s < SK; ++s) chain_step<1>(w[s], xt, P * stride, s, acc);
        chain_merge<P, 1>(acc);
        if (lane % P == 0) {
          int kt = tile - q_tiles;
          const bool is_v = kt >= k_tiles;
          if (is_v) kt -= k_tiles;
          const int row = kt * 2 + lane / P;
          if (is_v)
            a.v_cache[static_cast<uint64_t>(row) * a.cap + a.ctl->position] = bf16_bits(acc[0]);
          else
            a.k_out[row] = bf16_bits(acc[0]);
        }
      }
      return;
    }
  }
  FirstBatch fb{};
  // The prologue returns, after issuing its loads, when the loop is stopped
  // (grid-uniform flag).
  const int rows = live_rows<B>(a.rows);
  if (!norm_stage<B, Part != kQkvKV, Part != kQkvQ, W / 2>(
          a.h, a.norm, a.eps, xs16, xs32, scratch,
          [&] {
            if (first < items) issue_first(tile_src(tile_begin + first / Split), lane, fb);
          },
          &a.ctl->active, rows))
    return;
  __syncthreads();
  const uint64_t pos = a.ctl->position;
  for (int item = first; item < items; item += blocks * W) {
    const int tile = tile_begin + item / Split, b0 = (item % Split) * BR;
    const bool is_q = tile < q_tiles;
    int kt = tile - q_tiles;
    const bool is_v = !is_q && kt >= k_tiles;
    if (is_v) kt -= k_tiles;
    const u32x4* src = tile_src(tile);
    const int next = item + blocks * W;
    const u32x4* next_src = next < items ? tile_src(tile_begin + next / Split) : nullptr;
    float acc[BR];
    if (Part == kQkvQ || (Part == kQkvAll && is_q)) {
      chain_tile<16, BR>(src, xs16 + b0 * staged_floats(16, a.D), a.D, lane, acc, &fb, next_src);
      if (lane % 16 == 0) {
        const int row = tile * 4 + lane / 16;
#pragma unroll
        for (int b = 0; b < BR; ++b)
          if (b0 + b < rows) a.q_out[(b0 + b) * a.QW + row] = bf16_bits(acc[b]);
      }
    } else {
      chain_tile<32, BR>(src, xs32 + b0 * staged_floats(32, a.D), a.D, lane, acc, &fb, next_src);
      if (lane % 32 == 0) {
        const int row = kt * 2 + lane / 32;
#pragma unroll
        for (int b = 0; b < BR; ++b) {
          if (b0 + b >= rows) break;
          if (is_v)
            a.v_cache[(b0 + b) * a.cache_seq_stride + static_cast<uint64_t>(row) * a.cap + pos] = bf16_bits(acc[b]);
          else
            a.k_out[(b0 + b) * a.KW + row] = bf16_bits(acc[b]);
        }
      }
    }
  }
}

// Two wavefronts per SIMD at least: the batch-1 whole-tile path holds 128
// weight VGPRs, and a grid of one tile per wavefront must be resident at once.
template <int B, int Part = kQkvAll, int Split = 1>
__global__ __launch_bounds__(qkv_waves(B, Part) * 64) __attribute__((amdgpu_waves_per_eu(2))) void k_qkv(QkvArgs a) {
  qkv_rows<B, Part, Split>(a, blockIdx.x, gridDim.x);
}

// The Q part (workgroups [0, q_blocks)) and the K/V part (the rest) of B
// rows in one launch: a compute unit whose Q workgroup is done takes a K/V
// workgroup without waiting for the whole Q grid.  Each workgroup stages only
// its part's layout, so both fit the LDS that one of them takes.
template <int B, int Split>
__global__ __launch_bounds__(qkv_waves(B, kQkvQ) * 64) __attribute__((amdgpu_waves_per_eu(2))) void k_qkv_roles(
    QkvArgs a, int q_blocks) {
  static_assert(qkv_waves(B, kQkvQ) == qkv_waves(B, kQkvKV), "both parts use the same workgroup shape");
  if (static_cast<int>(blockIdx.x) < q_blocks)
    qkv_rows<B, kQkvQ, Split>(a, blockIdx.x, q_blocks);
  else
    qkv_rows<B, kQkvKV, Split>(a, blockIdx.x - q_blocks, gridDim.x - q_blocks);
}

// Orders one wavefront's LDS writes before its own later LDS reads (and the
// reads before the next writes) when lanes exchange values through LDS.
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// ------------------------------------------------------------- attention
struct AttnArgs {
  const Control* ctl;
  const uint16_t* q_raw;     // [B][Hq*128]
  const uint16_t* k_raw;     // [B][Hkv*128]
  const uint16_t* q_norm;    // [128]
  const uint16_t* k_norm;    // [128]
  const float* rope;         // [cap][64][2]
  uint16_t* k_cache;         // this layer, sequence 0: [Hkv][cap][128]
  const uint16_t* v_cache;   // this layer, sequence 0: [Hkv*128][cap] (V^T)
  uint64_t cache_seq_stride; // elements
  float* scores;             // [B][Hq][cap]
  float* probs;              // [B][Hq][cap]
  uint16_t* att;             // [B][Hq*128]
  int q_heads, kv_heads, cap;
  float eps, scale;
  // Row b is at position ctl->position + b * pos_step: 0 when the rows are
  // sequences at one position (decode), 1 when they are consecutive
  // positions of one sequence (cache_seq_stride 0, chunked prompt pass).
  int pos_step;
};


// Grid (kv head, 64-key tile, sequence); block 256 = 4 waves, one per query
// head of the group.  Scores use 8 lanes per key, each an FMA chain over 16
// contiguous features, merged at offsets 4,2,1 (attention.cu:231-300).  The
// tile's 64 cached key rows do not depend on this token: they are issued at
// entry, with the head operands, so one memory latency covers both.
__global__ __launch_bounds__(kBlock) void k_attn_qk(AttnArgs a) {
  __shared__ float qs[4][kHeadDim];
  __shared__ float ks[kHeadDim];
  const int g = blockIdx.x, key0 = blockIdx.y * 64, b = blockIdx.z;
  const int wave = threadIdx.x / 64, lane = threadIdx.x % 64;
  const int kl = lane / 8, l = lane % 8;
  const int group = a.q_heads / a.kv_heads;
  const uint64_t qw = static_cast<uint64_t>(a.q_heads) * kHeadDim, kw = static_cast<uint64_t>(a.kv_heads) * kHeadDim;
  uint16_t* kc = a.k_cache + b * a.cache_seq_stride + static_cast<uint64_t>(g) * a.cap * kHeadDim;
  // Rows key0 .. key0 + 63 lie inside the cache (its capacity is a multiple
  // of 64); rows at or past the position are loaded but never used.
  u32x4 kpre[2][2];
#pragma unroll
  for (int it = 0; it < 2; ++it) {
    const u32x4* src =
        reinterpret_cast<const u32x4*>(kc + static_cast<uint64_t>(key0 + wave * 16 + it * 8 + kl) * kHeadDim + 16 * l);
    kpre[it][0] = src[0];
    kpre[it][1] = src[1];
  }
  HeadOperands qh{}, kh{};
  {
    const uint16_t* x = a.q_raw + b * qw + static_cast<uint64_t>(g * group + wave) * kHeadDim;
    qh.xa = dl_bf16_to_f32(x[lane]);
    qh.xb = dl_bf16_to_f32(x[lane + 64]);
    qh.ga = dl_bf16_to_f32(a.q_norm[lane]);
    qh.gb = dl_bf16_to_f32(a.q_norm[lane + 64]);
  }
  if (wave == 0) {
    const uint16_t* x = a.k_raw + b * kw + static_cast<uint64_t>(g) * kHeadDim;
    kh.xa = dl_bf16_to_f32(x[lane]);
    kh.xb = dl_bf16_to_f32(x[lane + 64]);
    kh.ga = dl_bf16_to_f32(a.k_norm[lane]);
    kh.gb = dl_bf16_to_f32(a.k_norm[lane + 64]);
  }
  if (!a.ctl->active) return;
  const uint64_t pos = a.ctl->position + static_cast<uint64_t>(b) * a.pos_step;
  const int count = static_cast<int>(pos) + 1;
  if (key0 >= count) return;
  const float* rope_pos = a.rope + pos * kHeadDim;
  qh.cosine = kh.cosine = rope_pos[2 * lane];
  qh.sine = kh.sine = rope_pos[2 * lane + 1];
  head_norm_rope(qh, lane, a.eps, qs[wave]);
  const bool has_new = pos >= static_cast<uint64_t>(key0) && pos < static_cast<uint64_t>(key0) + 64;
  if (has_new && wave == 0) {
    head_norm_rope(kh, lane, a.eps, ks);
    kc[pos * kHeadDim + lane] = bf16_bits(ks[lane]);
    kc[pos * kHeadDim + lane + 64] = bf16_bits(ks[lane + 64]);
  }
  __syncthreads();
  float q[4][16];
#pragma unroll
  for (int h = 0; h < 4; ++h)
#pragma unroll
    for (int i = 0; i < 16; ++i) q[h][i] = qs[h][16 * l + i];
#pragma unroll
  for (int it = 0; it < 2; ++it) {
    const int j = key0 + wave * 16 + it * 8 + kl;
    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    if (j < count) {
      float kf[16];
      if (static_cast<uint64_t>(j) == pos) {
#pragma unroll
        for (int i = 0; i < 16; ++i) kf[i] = ks[16 * l + i];
      } else {
        const u32x4 w0 = kpre[it][0], w1 = kpre[it][1];
        kf[0] = dl_bf16_lo(w0.x); kf[1] = dl_bf16_hi(w0.x); kf[2] = dl_bf16_lo(w0.y); kf[3] = dl_bf16_hi(w0.y);
        kf[4] = dl_bf16_lo(w0.z); kf[5] = dl_bf16_hi(w0.z); kf[6] = dl_bf16_lo(w0.w); kf[7] = dl_bf16_hi(w0.w);
        kf[8] = dl_bf16_lo(w1.x); kf[9] = dl_bf16_hi(w1.x); kf[10] = dl_bf16_lo(w1.y); kf[11] = dl_bf16_hi(w1.y);
        kf[12] = dl_bf16_lo(w1.z); kf[13] = dl_bf16_hi(w1.z); kf[14] = dl_bf16_lo(w1.w); kf[15] = dl_bf16_hi(w1.w);
      }
#pragma unroll
      for (int h = 0; h < 4; ++h)
#pragma unroll
        for (int i = 0; i < 16; ++i) acc[h] = fma_rn(q[h][i], kf[i], acc[h]);
    }
#pragma unroll
    for (int h = 0; h < 4; ++h) {
      acc[h] = acc[h] + row_down<4>(acc[h]);
      acc[h] = acc[h] + row_down<2>(acc[h]);
      acc[h] = acc[h] + row_down<1>(acc[h]);
    }
    if (l == 0 && j < count) {
#pragma unroll
      for (int h = 0; h < 4; ++h)
        a.scores[(static_cast<uint64_t>(b) * a.q_heads + g * group + h) * a.cap + j] = acc[h] * a.scale;
    }
  }
}

// k_attn_qk for the rows of the chunked prompt pass (consecutive positions
// of one sequence, pos_step 1, every row's rotated key already in the cache
// by k_append_keys): grid (kv head, 64-key tile, block of kQkRows rows).
// The tile's key rows are loaded and widened once for all the block's rows,
// and the group's query heads of those rows are normalized and rotated up
// front (wave w takes head w of every row).  Each score is k_attn_qk's:
// 8 lanes per key, an FMA chain over 16 contiguous features each, merged at
// offsets 4, 2, 1, times the scale (attention.cu:231-300).
constexpr int kQkRows = 8;

__global__ __launch_bounds__(kBlock) void k_attn_qk_rows(AttnArgs a, int rows) {
  __shared__ float qs[kQkRows][4][kHeadDim];
  const int g = blockIdx.x, key0 = blockIdx.y * 64, rb = blockIdx.z * kQkRows;
  const int wave = threadIdx.x / 64, lane = threadIdx.x % 64;
  const int kl = lane / 8, l = lane % 8;
  const int group = a.q_heads / a.kv_heads;
  const int n = min(kQkRows, rows - rb);
  const uint64_t qw = static_cast<uint64_t>(a.q_heads) * kHeadDim;
  const uint16_t* kc = a.k_cache + static_cast<uint64_t>(g) * a.cap * kHeadDim;
  // Rows key0 .. key0 + 63 lie inside the cache (its capacity is a multiple
  // of 64); rows past a query's position are loaded but never used.
  u32x4 kpre[2][2];
#pragma unroll
  for (int it = 0; it < 2; ++it) {
    const u32x4* src =
        reinterpret_cast<const u32x4*>(kc + static_cast<uint64_t>(key0 + wave * 16 + it * 8 + kl) * kHeadDim + 16 * l);
    kpre[it][0] = src[0];
    kpre[it][1] = src[1];
  }
  if (!a.ctl->active) return;
  const uint64_t pos0 = a.ctl->position + static_cast<uint64_t>(rb);
  if (static_cast<uint64_t>(key0) > pos0 + n - 1) return;  // past every row's last key
  for (int rr = 0; rr < n; ++rr) {
    const uint64_t pos = pos0 + rr;
    const uint16_t* x = a.q_raw + (rb + rr) * qw + static_cast<uint64_t>(g * group + wave) * kHeadDim;
    head_norm_rope(x, a.q_norm, a.rope + pos * kHeadDim, lane, a.eps, qs[rr][wave]);
  }
  float kf[2][16];
#pragma unroll
  for (int it = 0; it < 2; ++it) {
    const u32x4 w0 = kpre[it][0], w1 = kpre[it][1];
    kf[it][0] = dl_bf16_lo(w0.x); kf[it][1] = dl_bf16_hi(w0.x); kf[it][2] = dl_bf16_lo(w0.y); kf[it][3] = dl_bf16_hi(w0.y);
    kf[it][4] = dl_bf16_lo(w0.z); kf[it][5] = dl_bf16_hi(w0.z); kf[it][6] = dl_bf16_lo(w0.w); kf[it][7] = dl_bf16_hi(w0.w);
    kf[it][8] = dl_bf16_lo(w1.x); kf[it][9] = dl_bf16_hi(w1.x); kf[it][10] = dl_bf16_lo(w1.y); kf[it][11] = dl_bf16_hi(w1.y);
    kf[it][12] = dl_bf16_lo(w1.z); kf[it][13] = dl_bf16_hi(w1.z); kf[it][14] = dl_bf16_lo(w1.w); kf[it][15] = dl_bf16_hi(w1.w);
  }
  __syncthreads();
  for (int rr = 0; rr < n; ++rr) {
    const int count = static_cast<int>(pos0 + rr) + 1;
    const int b = rb + rr;
    float q[4][16];
#pragma unroll
    for (int h = 0; h < 4; ++h)
#pragma unroll
      for (int i = 0; i < 16; ++i) q[h][i] = qs[rr][h][16 * l + i];
#pragma unroll
    for (int it = 0; it < 2; ++it) {
      const int j = key0 + wave * 16 + it * 8 + kl;
      float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
      if (j < count) {
#pragma unroll
        for (int h = 0; h < 4; ++h)
#pragma unroll
          for (int i = 0; i < 16; ++i) acc[h] = fma_rn(q[h][i], kf[it][i], acc[h]);
      }
#pragma unroll
      for (int h = 0; h < 4; ++h) {
        acc[h] = acc[h] + row_down<4>(acc[h]);
        acc[h] = acc[h] + row_down<2>(acc[h]);
        acc[h] = acc[h] + row_down<1>(acc[h]);
      }
      if (l == 0 && j < count) {
#pragma unroll
        for (int h = 0; h < 4; ++h)
          a.scores[(static_cast<uint64_t>(b) * a.q_heads + g * group + h) * a.cap + j] = acc[h] * a.scale;
      }
    }
  }
}

// Grid (query head, sequence), 1024 threads.  m = max, e = exp(s - m),
// denominator from 32 partials owning j mod 32 merged at offsets 16..1,
// p = e / l (attention.cu:301-330).  Every thread issues all of its score
// loads before using any (indices clamped to the last key, which leaves the
// max unchanged); each partial reads its terms from LDS 16 at a time and
// adds them in ascending key order.
constexpr int kSoftmaxChunk = 16;
constexpr int kSoftmaxThreads = 1024;
constexpr int kSoftmaxLoads = 8;  // scores per thread in flight: 8192 keys per pass

__global__ __launch_bounds__(kSoftmaxThreads) void k_attn_softmax(AttnArgs a) {
  extern __shared__ float es[];
  __shared__ float wave_max[kSoftmaxThreads / 64];
  __shared__ float denominator_shared;
  if (!a.ctl->active) return;
  const int h = blockIdx.x, b = blockIdx.y, tid = threadIdx.x;
  const int count = static_cast<int>(a.ctl->position + static_cast<uint64_t>(b) * a.pos_step) + 1;
  const uint64_t row = (static_cast<uint64_t>(b) * a.q_heads + h) * a.cap;
  const float* sc = a.scores + row;
  float m = -INFINITY;
  for (int base = 0; base < count; base += kSoftmaxThreads * kSoftmaxLoads) {
    float s[kSoftmaxLoads];
#pragma unroll
    for (int i = 0; i < kSoftmaxLoads; ++i) s[i] = sc[min(base + tid + i * kSoftmaxThreads, count - 1)];
#pragma unroll
    for (int i = 0; i < kSoftmaxLoads; ++i) {
      m = fmaxf(m, s[i]);
      const int j = base + tid + i * kSoftmaxThreads;
      if (j < count) es[j] = s[i];
    }
  }
#pragma unroll
  for (int off = 32; off; off >>= 1) m = fmaxf(m, __shfl_xor(m, off));
  if (tid % 64 == 0) wave_max[tid / 64] = m;
  __syncthreads();
#pragma unroll
  for (int w = 0; w < kSoftmaxThreads / 64; ++w) m = fmaxf(m, wave_max[w]);
  for (int j = tid; j < count; j += kSoftmaxThreads) es[j] = dl_expf(es[j] - m);
  __syncthreads();
  if (tid < 32) {
    float p = 0.0f;
    int j = tid;
    for (; j + 32 * (kSoftmaxChunk - 1) < count; j += 32 * kSoftmaxChunk) {
      float e[kSoftmaxChunk];
#pragma unroll
      for (int i = 0; i < kSoftmaxChunk; ++i) e[i] = es[j + 32 * i];
#pragma unroll
      for (int i = 0; i < kSoftmaxChunk; ++i) p = p + e[i];
    }
    for (; j < count; j += 32) p = p + es[j];
#pragma unroll
    for (int off = 16; off; off >>= 1) p = p + __shfl_down(p, off, 32);
    if (tid == 0) denominator_shared = p;
  }
  __syncthreads();
  const float l = denominator_shared;
  for (int j = tid; j < count; j += kSoftmaxThreads) a.probs[row + j] = es[j] / l;
}

// k_attn_softmax for many rows (the chunked prompt pass, batched decode):
// one wavefront per (query head, row), grid (query head, row), so that a
// short row is not spread over 1024 threads and three workgroup barriers.
// The same arithmetic: m = max (order-free), e = exp(s - m) kept in the
// wavefront's LDS, the 32 partials owning j mod 32 in ascending key order
// (lanes 0-31, reads eight at a time), merged at offsets 16..1, p = e / l
// (attention.cu:301-330).
__global__ __launch_bounds__(64) void k_attn_softmax_rows(AttnArgs a) {
  extern __shared__ float es[];
  if (!a.ctl->active) return;
  const int h = blockIdx.x, b = blockIdx.y, lane = threadIdx.x;
  const int count = static_cast<int>(a.ctl->position + static_cast<uint64_t>(b) * a.pos_step) + 1;
  const uint64_t row = (static_cast<uint64_t>(b) * a.q_heads + h) * a.cap;
  const float* sc = a.scores + row;
  float m = -INFINITY;
  for (int base = 0; base < count; base += 64 * kSoftmaxLoads) {
    float s[kSoftmaxLoads];
#pragma unroll
    for (int i = 0; i < kSoftmaxLoads; ++i) s[i] = sc[min(base + lane + 64 * i, count - 1)];
#pragma unroll
    for (int i = 0; i < kSoftmaxLoads; ++i) {
      m = fmaxf(m, s[i]);
      const int j = base + lane + 64 * i;
      if (j < count) es[j] = s[i];
    }
  }
  m = dl::wave_max(m);
  wave_lds_sync();
  for (int j = lane; j < count; j += 64) es[j] = dl_expf(es[j] - m);
  wave_lds_sync();
  float partial = 0.0f;
  if (lane < 32) {
    int j = lane;
    for (; j + 7 * 32 < count; j += 8 * 32) {
      float e[8];
#pragma unroll
      for (int k = 0; k < 8; ++k) e[k] = es[j + 32 * k];
#pragma unroll
      for (int k = 0; k < 8; ++k) partial = partial + e[k];
    }
    for (; j < count; j += 32) partial = partial + es[j];
  }
  // Offsets 16, 8, 4, 2, 1 as __shfl_down(partial, off, 32); below 16 the
  // lanes that feed lane 0 read within their row (DPP).
  partial = partial + __shfl_down(partial, 16, 32);
  partial = partial + row_down<8>(partial);
  partial = partial + row_down<4>(partial);
  partial = partial + row_down<2>(partial);
  partial = partial + row_down<1>(partial);
  const float l = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(partial), 0));
  for (int j = lane; j < count; j += 64) a.probs[row + j] = es[j] / l;
}

// Grid (kv head * 32 feature blocks, sequence), 192 threads.  Wave 0 runs
// both PV key ranges (the first ceil(n/2) keys and the rest) for the group's
// 4 query heads x 4 features: lane = (range, head, feature) in lanes 0-31;
// each output feature is round(A + B), A and B ascending FMA chains
// (attention.cu:331-375).  One wave holds both ranges, so the kernel's VALU
// time is one wave's chain however the waves are placed on SIMDs.
//
// A wave issues at most one instruction per issue cycle of its SIMD, so the
// chain wave's time is its instruction count per key: one FMA (its
// probability broadcast within the lane's quad by DPP), a quarter of a
// 16-byte LDS read for V, a sixteenth of one for the probabilities, and its
// waits.
// The other two waves keep everything else off it:
// - wave 1 copies: each chunk's 8 V rows (BF16, both ranges) and 8
//   probability rows (FP32) go from global memory straight into a
//   kPvSlots-slot LDS ring (global_load_lds, no registers in flight),
//   kPvSlots - 1 chunks ahead of the chains, with explicit vmcnt waits and
//   plain barriers (a fenced barrier would wait for every copy in flight);
// - wave 2 widens the V rows of the next chunk to FP32 into one of two
//   buffers while the chains run the current one.
// The copy rate of a workgroup is bounded by the bytes it keeps in flight,
// so the work is spread over 256 workgroups, one per CU.  A copy instruction
// writes 64 x 16 bytes contiguously; its lanes fetch the rows interleaved 16
// bytes at a time and its block is padded; the widened rows are padded by
// 16 bytes, so the rows the chain wave reads at one key fall in distinct
// banks.
constexpr int kPvFeatures = 4;
constexpr int kPvThreads = 192;
constexpr int kPvChunk = 128;
constexpr int kPvSlots = 12;            // chunks in the copy ring
constexpr int kPvVBlocks = 2;           // V blocks per chunk (4 rows each)
constexpr int kPvCopies = 6;            // global_load_lds per chunk: 2 V blocks + 4 probability blocks
constexpr int kPvBlock = 1024 + 64;     // bytes per copy block in LDS (64 lanes x 16 bytes + pad)
constexpr int kPvSlotBytes = kPvCopies * kPvBlock;
constexpr int kPvInFlight = (kPvSlots - 3) * kPvCopies;  // copies a step leaves outstanding
constexpr int kPvWideRow = kPvChunk * 4 + 16;              // bytes per widened V row (FP32, padded)
constexpr int kPvWideBytes = 2 * kPvFeatures * kPvWideRow;  // one chunk's 8 widened rows
constexpr size_t kPvLds = size_t(kPvSlots) * kPvSlotBytes + 2 * kPvWideBytes;

typedef __attribute__((address_space(3))) void pv_lds_void;
typedef __attribute__((address_space(1))) void pv_global_void;

// s_waitcnt immediate waiting until at most n vector-memory operations of
// this wave are outstanding (vmcnt bits 3:0 and 15:14; expcnt and lgkmcnt
// left at their no-wait maxima).
constexpr unsigned pv_vmcnt(unsigned n) { return 0x0f70u | (n & 0xfu) | ((n >> 4) << 14); }
// s_waitcnt immediate waiting until no LDS operation of this wave is
// outstanding (lgkmcnt bits 11:8 zero; vmcnt and expcnt at their maxima).
constexpr unsigned kPvLdsDone = 0xc07fu;

// acc = fma(p_key, v[key], acc) for key = 4k + j, k and j = 0..3 ascending:
// p component j of quad lane k (DPP quad_perm broadcast), v[k] component j.
// v_fmac_f32 is the single-rounding FMA (fma_rn); the s_nop covers the two
// wait states a DPP read needs after a VALU write of its source.
__device__ __forceinline__ float fma16_quad_bcast(float acc, const float4& p, const float4 (&v)[4]) {
  asm volatile(
      "s_nop 1\n"
      "v_fmac_f32_dpp %0, %1, %5 quad_perm:[0,0,0,0] row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f32_dpp %0, %2, %6 quad_perm:[0,0,0,0] row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f32_dpp %0, %3, %7 quad_perm:[0,0,0,0] row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f32_dpp %0, %4, %8 quad_perm:[0,0,0,0] row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f32_dpp %0, %1, %9 quad_perm:[1,1,1,1] row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f32_dpp %0, %2, %10 quad_perm:[1,1,1,1] row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f32_dpp %0, %3, %11 quad_perm:[1,1,1,1] row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f32_dpp %0, %4, %12 quad_perm:[1,1,1,1] row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f32_dpp %0, %1, %13 quad_perm:[2,2,2,2] row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f32_dpp %0, %2, %14 quad_perm:[2,2,2,2] row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f32_dpp %0, %3, %15 quad_perm:[2,2,2,2] row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f32_dpp %0, %4, %16 quad_perm:[2,2,2,2] row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f32_dpp %0, %1, %17 quad_perm:[3,3,3,3] row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f32_dpp %0, %2, %18 quad_perm:[3,3,3,3] row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f32_dpp %0, %3, %19 quad_perm:[3,3,3,3] row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f32_dpp %0, %4, %20 quad_perm:[3,3,3,3] row_mask:0xf bank_mask:0xf\n"
      : "+v"(acc)
      : "v"(p.x), "v"(p.y), "v"(p.z), "v"(p.w), "v"(v[0].x), "v"(v[0].y), "v"(v[0].z), "v"(v[0].w), "v"(v[1].x),
        "v"(v[1].y), "v"(v[1].z), "v"(v[1].w), "v"(v[2].x), "v"(v[2].y), "v"(v[2].z), "v"(v[2].w), "v"(v[3].x),
        "v"(v[3].y), "v"(v[3].z), "v"(v[3].w));
  return acc;
}

__global__ __launch_bounds__(kPvThreads) void k_attn_pv(AttnArgs a) {
  extern __shared__ __align__(16) uint8_t pv_lds[];
  uint8_t* ring = pv_lds;
  uint8_t* wide = pv_lds + kPvSlots * kPvSlotBytes;
  if (!a.ctl->active) return;
  // Group-minor numbering keeps the feature blocks of one K/V group on one
  // XCD (workgroups are dealt to the XCDs round-robin): its L2 serves the
  // group's probability rows once for all of them.
  const int g = blockIdx.x % a.kv_heads, fb = blockIdx.x / a.kv_heads, b = blockIdx.y;
  const int count = static_cast<int>(a.ctl->position + static_cast<uint64_t>(b) * a.pos_step) + 1;
  const int split = (count - 1) / 2 + 1;
  // Wave-uniform values in scalar registers.
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / 64), lane = threadIdx.x % 64;
  const int group = a.q_heads / a.kv_heads;
  const uint16_t* vbase =
      a.v_cache + b * a.cache_seq_stride + static_cast<uint64_t>(g * kHeadDim + fb * kPvFeatures) * a.cap;
  const float* pbase = a.probs + (static_cast<uint64_t>(b) * a.q_heads + g * group) * a.cap;
  // Range r covers keys [begin_r, end_r), staged from the 8-aligned key below
  // begin_r; chunk c of range r holds keys jb0_r + kPvChunk c + [0, kPvChunk).
  const int end0 = split, begin1 = split, end1 = count;
  const int jb0_1 = begin1 & ~7;
  const int chunks0 = (end0 + kPvChunk - 1) / kPvChunk;
  const int chunks1 = end1 > begin1 ? (end1 - jb0_1 + kPvChunk - 1) / kPvChunk : 0;
  const int chunks = max(chunks0, chunks1);
  auto slot_of = [&](int c) { return ring + (c % kPvSlots) * kPvSlotBytes; };

  // Copy k (0..5) of a chunk fills block k of its slot.  k < 2: V rows
  // 4k .. 4k + 3 (row = range * 4 + feature); lane L fetches row 4k + L % 4,
  // keys 8 (L / 4) .. + 7.  k >= 2: probability rows 2(k - 2) + {0, 1}
  // (row = range * 4 + head); lane L fetches row 2(k - 2) + L % 2, keys
  // 4 (L / 2) .. + 3.  Sources past a range are clamped to its last 8 (4)
  // keys, inside the cache rows; the chains never use those values.  The
  // chunk index is clamped to the last chunk, so every step issues the same
  // number of copies and waits with the same count.
  auto copy = [&](int c) {
    uint8_t* slot = slot_of(c);
    c = min(c, chunks - 1);
#pragma unroll
    for (int k = 0; k < kPvCopies; ++k) {
      if (k < kPvVBlocks) {
        const int row = 4 * k + lane % 4, r = row / kPvFeatures, f = row % kPvFeatures;
        const int jb0 = r ? jb0_1 : 0, last8 = ((r ? end1 : end0) - 1) & ~7;
        const int key = max(0, min(jb0 + kPvChunk * c + 8 * (lane / 4), last8));
        __builtin_amdgcn_global_load_lds((const pv_global_void*)(vbase + static_cast<uint64_t>(f) * a.cap + key),
                                         (pv_lds_void*)(slot + k * kPvBlock), 16, 0, 0);
      } else {
        const int row = 2 * (k - kPvVBlocks) + lane % 2, r = row / 4, hl = row % 4;
        const int jb0 = r ? jb0_1 : 0, last4 = ((r ? end1 : end0) - 1) & ~3;
        const int key = max(0, min(jb0 + kPvChunk * c + 4 * (lane / 2), last4));
        __builtin_amdgcn_global_load_lds((const pv_global_void*)(pbase + static_cast<uint64_t>(hl) * a.cap + key),
                                         (pv_lds_void*)(slot + k * kPvBlock), 16, 0, 0);
      }
    }
  };
  // Widens the V blocks of a landed chunk: lane L of block k holds row
  // 4k + L % 4, keys 8 (L / 4) .. + 7, which go to that row of buffer c % 2
  // at key offset 8 (L / 4).
  auto widen = [&](int c) {
    const uint8_t* slot = slot_of(c);
    uint8_t* to = wide + (c & 1) * kPvWideBytes;
#pragma unroll
    for (int k = 0; k < kPvVBlocks; ++k) {
      const u32x4 w = *reinterpret_cast<const u32x4*>(slot + k * kPvBlock + 16 * lane);
      const float4 lo = make_float4(dl_bf16_lo(w.x), dl_bf16_hi(w.x), dl_bf16_lo(w.y), dl_bf16_hi(w.y));
      const float4 hi = make_float4(dl_bf16_lo(w.z), dl_bf16_hi(w.z), dl_bf16_lo(w.w), dl_bf16_hi(w.w));
      float4* dst = reinterpret_cast<float4*>(to + (4 * k + lane % 4) * kPvWideRow + 32 * (lane / 4));
      dst[0] = lo;
      dst[1] = hi;
    }
    __builtin_amdgcn_s_waitcnt(kPvLdsDone);
  };

  // Before step -1 the copy wave has chunks 0 .. kPvSlots - 3 in flight and
  // chunk 0 landed.
  if (wave == 1) {
    for (int c = 0; c <= kPvSlots - 3; ++c) copy(c);
    __builtin_amdgcn_s_waitcnt(pv_vmcnt(kPvInFlight));
  }

  // Chain lane L (lanes 32-63 repeat lanes 0-31 and write nothing): range
  // r = L / 16 % 2, head hl, feature f.  Widened V row r * 4 + f holds key
  // group q (8 keys) at byte 32 q; probability row r * 4 + hl lives in block
  // 2 + (r * 4 + hl) / 2 at piece 2 q + hl % 2 for key group q (4 keys).
  const int r = (lane / 16) & 1, hl = (lane % 16) / kPvFeatures, f = lane % kPvFeatures;
  const int begin = r ? begin1 : 0, end = r ? end1 : end0, jb0 = r ? jb0_1 : 0;
  const int prow = r * 4 + hl;
  const int voff = (r * kPvFeatures + f) * kPvWideRow;
  const int poff = (kPvVBlocks + prow / 2) * kPvBlock + (prow % 2) * 16;
  float acc = 0.0f;
  // Step c (from -1): after the barrier the chains run chunk c (its
  // probabilities in its slot, its V in buffer c % 2), wave 2 widens chunk
  // c + 1 (landed by the copy wave's wait of step c - 1), and the copy wave
  // copies chunk c + kPvSlots - 1 into the slot of chunk c - 1 (done with in
  // step c - 1) and waits until chunk c + 2 has landed.  The step count is
  // uniform, so all waves meet every barrier.
  for (int c = -1; c < chunks; ++c) {
    __builtin_amdgcn_s_barrier();
    if (wave == 1) {
      copy(c + kPvSlots - 1);
      __builtin_amdgcn_s_waitcnt(pv_vmcnt(kPvInFlight));
    } else if (wave == 2) {
      widen(c + 1);
    } else if (c >= 0) {
      const uint8_t* vb = wide + (c & 1) * kPvWideBytes + voff;
      const uint8_t* pb = slot_of(c) + poff;
      // Both ranges' chunk c full: the unmasked path (wave-uniform).
      const int cs0 = kPvChunk * c, cs1 = jb0_1 + kPvChunk * c;
      const bool full = cs0 + kPvChunk <= end0 && begin1 <= cs1 && cs1 + kPvChunk <= end1;
      if (full) {
        // 16-key groups m: four 16-byte reads of the lane's widened V row
        // and one of its head's probabilities, keys 16 m + 4 f .. + 3 (the
        // lanes of a quad share the head, so each quad holds the 16 keys'
        // probabilities and fma16_quad_bcast broadcasts them).  The reads
        // of group m + kAhead are issued before the FMAs of group m (the
        // order is pinned with scheduling barriers), so the LDS latency
        // hides behind the chain and the waits stay partial (at most
        // 5 kAhead reads are outstanding; the wait counter has 4 bits).
        constexpr int kGroups = kPvChunk / 16, kAhead = 2;
        float4 v4[kGroups][4], p4[kGroups];
        auto read = [&](int m) {
#pragma unroll
          for (int i = 0; i < 4; ++i) v4[m][i] = *reinterpret_cast<const float4*>(vb + 64 * m + 16 * i);
          p4[m] = *reinterpret_cast<const float4*>(pb + 128 * m + 32 * f);
        };
#pragma unroll
        for (int m = 0; m < kAhead; ++m) read(m);
#pragma unroll
        for (int m = 0; m < kGroups; ++m) {
          __builtin_amdgcn_sched_barrier(0);
          if (m + kAhead < kGroups) read(m + kAhead);
          __builtin_amdgcn_sched_barrier(0);
          acc = fma16_quad_bcast(acc, p4[m], v4[m]);
        }
      } else {
        // Keys [lo, hi) of this lane's range in the chunk (empty once the
        // range is done); the group loop bounds are the union over ranges.
        const int cs = jb0 + kPvChunk * c;
        const int lo = max(begin - cs, 0), hi = min(end - cs, kPvChunk);
        const int q_end = (min(max(end0 - cs0, end1 - cs1), kPvChunk) + 7) / 8;
        for (int q = 0; q < q_end; ++q) {
          const float4 va = *reinterpret_cast<const float4*>(vb + 32 * q);
          const float4 vc = *reinterpret_cast<const float4*>(vb + 32 * q + 16);
          const float4 pa = *reinterpret_cast<const float4*>(pb + 32 * (2 * q));
          const float4 pc = *reinterpret_cast<const float4*>(pb + 32 * (2 * q + 1));
          const float vv[8] = {va.x, va.y, va.z, va.w, vc.x, vc.y, vc.z, vc.w};
          const float pp[8] = {pa.x, pa.y, pa.z, pa.w, pc.x, pc.y, pc.z, pc.w};
#pragma unroll
          for (int e = 0; e < 8; ++e)
            if (8 * q + e >= lo && 8 * q + e < hi) acc = fma_rn(pp[e], vv[e], acc);
        }
      }
    }
  }
  static_assert((kPvSlots - 2) * kPvCopies <= 63, "the wait counter holds at most 63 outstanding copies");
  static_assert(kPvVBlocks * 4 == 2 * kPvFeatures && (kPvCopies - kPvVBlocks) * 2 == 2 * 4,
                "blocks of 4 V rows for two ranges of kPvFeatures, of 2 probability rows for two ranges of 4 heads");
  if (wave != 0) {
    if (wave == 1) __builtin_amdgcn_s_waitcnt(pv_vmcnt(0));  // no copy outstanding at exit
    return;
  }
  const float second = __shfl_down(acc, 16);
  if (lane < 16)
    a.att[static_cast<uint64_t>(b) * a.q_heads * kHeadDim + (g * group + hl) * kHeadDim + fb * kPvFeatures + f] =
        bf16_bits(acc + second);
}

// acc = fma(p_k, v[k], acc) for k = 0..15 in order, p_k taken from lane k
// of the lane's 16-lane row of `p` (DPP row_newbcast): one VGPR carries the
// probabilities of 16 keys, so a PV chain wave needs no LDS read per key.
// v_fmac_f32 is the single-rounding FMA, the same operation as fma_rn.  The
// s_nop covers the two wait states a DPP read needs after a VALU write of its
// source.
__device__ __forceinline__ float fma16_row_bcast(float acc, float p, const float (&v)[16]) {
  asm volatile(
      "s_nop 1\n"
      "v_fmac_f32_dpp %0, %1, %2 row_newbcast:0 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f32_dpp %0, %1, %3 row_newbcast:1 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f32_dpp %0, %1, %4 row_newbcast:2 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f32_dpp %0, %1, %5 row_newbcast:3 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f32_dpp %0, %1, %6 row_newbcast:4 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f32_dpp %0, %1, %7 row_newbcast:5 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f32_dpp %0, %1, %8 row_newbcast:6 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f32_dpp %0, %1, %9 row_newbcast:7 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f32_dpp %0, %1, %10 row_newbcast:8 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f32_dpp %0, %1, %11 row_newbcast:9 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f32_dpp %0, %1, %12 row_newbcast:10 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f32_dpp %0, %1, %13 row_newbcast:11 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f32_dpp %0, %1, %14 row_newbcast:12 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f32_dpp %0, %1, %15 row_newbcast:13 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f32_dpp %0, %1, %16 row_newbcast:14 row_mask:0xf bank_mask:0xf\n"
      "v_fmac_f32_dpp %0, %1, %17 row_newbcast:15 row_mask:0xf bank_mask:0xf"
      : "+v"(acc)
      : "v"(p), "v"(v[0]), "v"(v[1]), "v"(v[2]), "v"(v[3]), "v"(v[4]), "v"(v[5]), "v"(v[6]), "v"(v[7]), "v"(v[8]),
        "v"(v[9]), "v"(v[10]), "v"(v[11]), "v"(v[12]), "v"(v[13]), "v"(v[14]), "v"(v[15]));
  return acc;
}

// Several rows per launch (the chunked prompt pass): k_attn_pv's work in 64
// workgroups per row, so that 8 rows still fit the GPU in one round.  Grid
// (kv head * 8 feature blocks, row), 256 threads.  Waves 0 and 2 run the two
// PV key ranges (the first ceil(n/2) keys and the rest) for the
// group's 4 query heads x 16 features, lane = (head, feature); each output
// feature is round(A + B), A and B ascending FMA chains (attention.cu:331-375).
//
// The keys go through LDS in chunks of kPwChunk.  Waves 1 and 3 only copy:
// each chunk's 32 V rows (BF16, both ranges) and 8 probability rows (FP32)
// go from global memory straight into a kPwSlots-slot LDS ring
// (global_load_lds, no registers in flight), kPwSlots - 1 chunks ahead of
// the chains, with explicit vmcnt waits and plain barriers (a fenced
// barrier would wait for every copy in flight).  A copy instruction writes
// 64 x 16 bytes contiguously; its lanes fetch the rows interleaved 16 bytes
// at a time and its block is padded, so the 16 V rows (and the 4
// probability rows) a chain wave reads at one key fall in distinct banks.
constexpr int kPwFeatures = 16;
constexpr int kPwThreads = 256;
constexpr int kPwChunk = 128;
constexpr int kPwSlots = 6;             // chunks in the copy ring
constexpr int kPwCopies = 6;            // global_load_lds per producer wave per chunk
constexpr int kPwBlock = 1024 + 64;     // bytes per copy block in LDS (64 lanes x 16 bytes + pad)
constexpr int kPwSlotBytes = 12 * kPwBlock;  // 8 V blocks (4 rows each) + 4 probability blocks (2 rows each)


struct PwSlot {
  uint8_t bytes[kPwSlotBytes];
};

__global__ __launch_bounds__(kPwThreads) void k_attn_pv_rows(AttnArgs a) {
  __shared__ __align__(16) PwSlot s0, s1, s2, s3, s4, s5;
  __shared__ float second[64];
  if (!a.ctl->active) return;
  // Group-minor numbering keeps the feature blocks of one K/V group on one
  // XCD (workgroups are dealt to the XCDs round-robin): its L2 serves the
  // group's probability rows once for all of them.
  const int g = blockIdx.x % a.kv_heads, fb = blockIdx.x / a.kv_heads, b = blockIdx.y;
  const int count = static_cast<int>(a.ctl->position + static_cast<uint64_t>(b) * a.pos_step) + 1;
  const int split = (count - 1) / 2 + 1;
  // Wave-uniform values in scalar registers.
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / 64), lane = threadIdx.x % 64;
  const int group = a.q_heads / a.kv_heads;
  const uint16_t* vbase =
      a.v_cache + b * a.cache_seq_stride + static_cast<uint64_t>(g * kHeadDim + fb * kPwFeatures) * a.cap;
  const float* pbase = a.probs + (static_cast<uint64_t>(b) * a.q_heads + g * group) * a.cap;
  // Range r covers keys [begin_r, end_r), staged from the 8-aligned key below
  // begin_r; chunk c of range r holds keys jb0_r + kPwChunk c + [0, kPwChunk).
  const int end0 = split, begin1 = split, end1 = count;
  const int jb0_1 = begin1 & ~7;
  const int chunks0 = (end0 + kPwChunk - 1) / kPwChunk;
  const int chunks1 = end1 > begin1 ? (end1 - jb0_1 + kPwChunk - 1) / kPwChunk : 0;
  const int chunks = max(chunks0, chunks1);
  // Waves 0 and 2 run the chains (ranges 0 and 1), waves 1 and 3 copy, so
  // that the two chains do not share a SIMD when a workgroup's consecutive
  // waves are paired on SIMDs.
  const bool producer = (wave & 1) != 0;

  // Copy k (0..11) of a chunk fills block k of its slot.  k < 8: V rows
  // 4k .. 4k + 3 (row = range * 16 + feature); lane L fetches row 4k + L % 4,
  // keys 8 (L / 4) .. + 7.  k >= 8: probability rows 2(k - 8) + {0, 1}
  // (row = range * 4 + head); lane L fetches row 2(k - 8) + L % 2, keys
  // 4 (L / 2) .. + 3.  Sources past a range are clamped to its last 8 (4)
  // keys, inside the cache rows; the chains never use those values.  The
  // chunk index is clamped to the last chunk, so every step issues the same
  // number of copies and waits with the same count.  Producer wave w takes
  // the copies k = w / 2 + 2 n.
  auto copy = [&](PwSlot& slot, int c) {
    c = min(c, chunks - 1);
#pragma unroll
    for (int n = 0; n < kPwCopies; ++n) {
      const int k = wave / 2 + 2 * n;
      if (k < 8) {
        const int row = 4 * k + lane % 4, r = row / kPwFeatures, f = row % kPwFeatures;
        const int jb0 = r ? jb0_1 : 0, last8 = ((r ? end1 : end0) - 1) & ~7;
        const int key = max(0, min(jb0 + kPwChunk * c + 8 * (lane / 4), last8));
        __builtin_amdgcn_global_load_lds((const pv_global_void*)(vbase + static_cast<uint64_t>(f) * a.cap + key),
                                         (pv_lds_void*)(slot.bytes + k * kPwBlock), 16, 0, 0);
      } else {
        const int row = 2 * (k - 8) + lane % 2, r = row / 4, hl = row % 4;
        const int jb0 = r ? jb0_1 : 0, last4 = ((r ? end1 : end0) - 1) & ~3;
        const int key = max(0, min(jb0 + kPwChunk * c + 4 * (lane / 2), last4));
        __builtin_amdgcn_global_load_lds((const pv_global_void*)(pbase + static_cast<uint64_t>(hl) * a.cap + key),
                                         (pv_lds_void*)(slot.bytes + k * kPwBlock), 16, 0, 0);
      }
    }
  };

  if (producer && chunks > 0) {
    copy(s0, 0);
    copy(s1, 1);
    copy(s2, 2);
    copy(s3, 3);
    copy(s4, 4);
    __builtin_amdgcn_s_waitcnt(pv_vmcnt((kPwSlots - 2) * kPwCopies));  // chunk 0 is in s0
  }

  // Chains: wave r runs range r; lane = (head hl, feature f).  V row
  // r * 16 + f lives in block (r * 16 + f) / 4 at 16-byte piece
  // 4 g + f % 4 for key group g (8 keys); probability row r * 4 + hl in
  // block 8 + (r * 4 + hl) / 2 at piece 2 q + hl % 2 for key group q (4 keys).
  const int hl = lane / kPwFeatures, f = lane % kPwFeatures;
  const int r = wave / 2;
  const int begin = r ? begin1 : 0, end = r ? end1 : end0, jb0 = r ? jb0_1 : 0;
  const int mine = r ? chunks1 : chunks0;
  const int vrow = r * kPwFeatures + f, prow = r * 4 + hl;
  const int voff = (vrow / 4) * kPwBlock + (vrow % 4) * 16;
  const int poff = (8 + prow / 2) * kPwBlock + (prow % 2) * 16;
  float acc = 0.0f;
  // Step c: after the barrier the chains run chunk c from slot c % kPwSlots
  // while the producers copy chunk c + kPwSlots - 1 into chunk c - 1's slot
  // and wait until chunk c + 1 has landed.  `chunks` is uniform, so every
  // wave meets every barrier.
  auto step = [&](int c, const PwSlot& cur, PwSlot& ahead) {
    __builtin_amdgcn_s_barrier();  // chunk c is in `cur`; every chain is done with chunk c - 1
    if (producer) {
      copy(ahead, c + kPwSlots - 1);
      __builtin_amdgcn_s_waitcnt(pv_vmcnt((kPwSlots - 2) * kPwCopies));
      return;
    }
    if (c >= mine) return;
    const uint8_t* vb = cur.bytes + voff;
    const uint8_t* pb = cur.bytes + poff;
    const int cs = jb0 + kPwChunk * c;
    const int lo = max(begin - cs, 0), hi = min(end - cs, kPwChunk);
    auto eight = [&](int q, bool masked) {
      const u32x4 w = *reinterpret_cast<const u32x4*>(vb + 64 * q);
      const float4 pa = *reinterpret_cast<const float4*>(pb + 32 * (2 * q));
      const float4 pc = *reinterpret_cast<const float4*>(pb + 32 * (2 * q + 1));
      const float vv[8] = {dl_bf16_lo(w.x), dl_bf16_hi(w.x), dl_bf16_lo(w.y), dl_bf16_hi(w.y),
                           dl_bf16_lo(w.z), dl_bf16_hi(w.z), dl_bf16_lo(w.w), dl_bf16_hi(w.w)};
      const float pp[8] = {pa.x, pa.y, pa.z, pa.w, pc.x, pc.y, pc.z, pc.w};
      if (!masked) {
#pragma unroll
        for (int e = 0; e < 8; ++e) acc = fma_rn(pp[e], vv[e], acc);
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e)
          if (8 * q + e >= lo && 8 * q + e < hi) acc = fma_rn(pp[e], vv[e], acc);
      }
    };
    if (lo == 0 && hi == kPwChunk) {
      // The reads of group q + kAhead are issued before the FMAs of group
      // q (the order is pinned with scheduling barriers), so the LDS
      // latency hides behind the chain and the waits stay partial (at most
      // 3 kAhead reads are outstanding; the wait counter has 4 bits).  The
      // chain then runs at the rate of its two VALU instructions per key
      // (widen, FMA).
      constexpr int kGroups = kPwChunk / 8, kAhead = 3;
      u32x4 w[kGroups];
      float4 pa[kGroups], pc[kGroups];
      auto read = [&](int q) {
        w[q] = *reinterpret_cast<const u32x4*>(vb + 64 * q);
        pa[q] = *reinterpret_cast<const float4*>(pb + 32 * (2 * q));
        pc[q] = *reinterpret_cast<const float4*>(pb + 32 * (2 * q + 1));
      };
#pragma unroll
      for (int q = 0; q < kAhead; ++q) read(q);
#pragma unroll
      for (int q = 0; q < kGroups; ++q) {
        __builtin_amdgcn_sched_barrier(0);
        if (q + kAhead < kGroups) read(q + kAhead);
        __builtin_amdgcn_sched_barrier(0);
        const float vv[8] = {dl_bf16_lo(w[q].x), dl_bf16_hi(w[q].x), dl_bf16_lo(w[q].y), dl_bf16_hi(w[q].y),
                             dl_bf16_lo(w[q].z), dl_bf16_hi(w[q].z), dl_bf16_lo(w[q].w), dl_bf16_hi(w[q].w)};
        const float pp[8] = {pa[q].x, pa[q].y, pa[q].z, pa[q].w, pc[q].x, pc[q].y, pc[q].z, pc[q].w};
#pragma unroll
        for (int e = 0; e < 8; ++e) acc = fma_rn(pp[e], vv[e], acc);
      }
    } else {
      for (int q = lo / 8; q * 8 < hi; ++q) eight(q, true);
    }
  };
  static_assert(kPwSlots == 6 && (kPwSlots - 2) * kPwCopies <= 63, "the ring below is unrolled for 6 slots");
  for (int c0 = 0; c0 < chunks; c0 += kPwSlots) {
    step(c0, s0, s5);
    if (c0 + 1 < chunks) step(c0 + 1, s1, s0);
    if (c0 + 2 < chunks) step(c0 + 2, s2, s1);
    if (c0 + 3 < chunks) step(c0 + 3, s3, s2);
    if (c0 + 4 < chunks) step(c0 + 4, s4, s3);
    if (c0 + 5 < chunks) step(c0 + 5, s5, s4);
  }
  if (producer) __builtin_amdgcn_s_waitcnt(pv_vmcnt(0));  // no copy outstanding at exit
  if (wave == 2) second[lane] = acc;
  __syncthreads();
  if (wave == 0)
    a.att[static_cast<uint64_t>(b) * a.q_heads * kHeadDim + (g * group + hl) * kHeadDim + fb * kPwFeatures + f] =
        bf16_bits(acc + second[lane]);
}

// k_attn_pv_rows for the rows of the chunked prompt pass (consecutive
// positions of one sequence, pos_step 1): a workgroup runs kPbRows rows of
// half the features of one K/V group.  Grid (kv head * 2 feature halves, row
// blocks), 256 threads.  Waves 0 and 2 run the two PV key ranges: for row r
// with n_r keys, range 0 is [0, ceil(n_r / 2)) and range 1 the rest.  Lane
// (head, feature group) owns 4 features of one head for every row of the
// block, one accumulator per (row, feature), so each output feature is
// round(A + B) of the same two ascending FMA chains as in k_attn_pv_rows
// (attention.cu:331-375), while each widened V value feeds kPbRows FMAs and
// each probability 4.  A wave runs the union of its rows' ranges; a key
// group inside every row's range runs unmasked, the groups at the range
// ends masked per row (wave-uniform: a wave's rows are its lanes' rows).
// The lanes read their V rows (BF16, 8 keys per 16-byte load, two groups
// ahead) straight from memory; waves 1 and 3 copy the probability rows of
// the block's rows into a kPbSlots-slot LDS ring (global_load_lds),
// kPbSlots - 1 chunks ahead, as k_attn_pv_rows does.
constexpr int kPbRows = 4;
constexpr int kPbSlots = 4;
constexpr int kPbFeat = 4;                          // features per chain lane
constexpr int kPbHalf = 64;                         // features per workgroup
constexpr int kPbPBlocks = 2 * kPbRows * 4 / 2;     // 2 ranges x kPbRows rows x 4 heads, 2 rows per block
constexpr int kPbCopies = kPbPBlocks / 2;           // per copy wave and chunk
constexpr int kPbSlotBytes = kPbPBlocks * kPwBlock;
constexpr size_t kPbLds = size_t(kPbSlots) * kPbSlotBytes;

__global__ __launch_bounds__(kPwThreads) void k_attn_pv_block(AttnArgs a, int rows) {
  extern __shared__ __align__(16) uint8_t pb_lds[];
  __shared__ float second[kPbRows][kPbFeat][64];
  static_assert((kPbSlots - 1) * kPbCopies <= 63, "the wait counter holds at most 63 outstanding copies");
  static_assert(4 * (kPbHalf / kPbFeat) == 64, "lane = (head, feature group)");
  if (!a.ctl->active) return;
  const int g = blockIdx.x / 2, fh = blockIdx.x % 2, rb = blockIdx.y * kPbRows;
  const int n = min(kPbRows, rows - rb);
  const int pos0 = static_cast<int>(a.ctl->position) + rb;
  // Row rr attends to keys [0, pos0 + rr]; its ranges split at
  // ceil(count / 2).  The union of range 0 is [0, split of the last row),
  // of range 1 [split of the first row, count of the last row).
  auto count_of = [&](int rr) { return pos0 + rr + 1; };
  auto split_of = [&](int rr) { return (count_of(rr) - 1) / 2 + 1; };
  const int end0 = split_of(n - 1), begin1 = split_of(0), end1 = count_of(n - 1);
  const int jb0_1 = begin1 & ~7;
  const int chunks0 = (end0 + kPwChunk - 1) / kPwChunk;
  const int chunks1 = end1 > begin1 ? (end1 - jb0_1 + kPwChunk - 1) / kPwChunk : 0;
  const int chunks = max(chunks0, chunks1);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / 64), lane = threadIdx.x % 64;
  const int group = a.q_heads / a.kv_heads;
  const float* pbase = a.probs + (static_cast<uint64_t>(rb) * a.q_heads + g * group) * a.cap;
  const bool producer = (wave & 1) != 0;
  auto slot_of = [&](int c) { return pb_lds + (c % kPbSlots) * kPbSlotBytes; };

  // Copy k of a chunk fills block k of its slot: probability rows
  // 2 k + {0, 1} (row = (range * kPbRows + rr) * 4 + head); lane L fetches
  // row 2 k + L % 2, keys 4 (L / 2) .. + 3.  Sources past a range are clamped
  // to its last 4 keys, rows past the block's last row repeat it; the chains
  // never use those values.  Producer wave w takes the copies k = w / 2 + 2 m.
  auto copy = [&](int c) {
    uint8_t* slot = slot_of(c);
    c = min(c, chunks - 1);
#pragma unroll
    for (int m = 0; m < kPbCopies; ++m) {
      const int k = wave / 2 + 2 * m;
      const int prow = 2 * k + lane % 2;
      const int r = prow / (4 * kPbRows), rr = min((prow / 4) % kPbRows, n - 1), hl = prow % 4;
      const int jb0 = r ? jb0_1 : 0, last4 = ((r ? end1 : end0) - 1) & ~3;
      const int key = max(0, min(jb0 + kPwChunk * c + 4 * (lane / 2), last4));
      __builtin_amdgcn_global_load_lds(
          (const pv_global_void*)(pbase + (static_cast<uint64_t>(rr) * a.q_heads + hl) * a.cap + key),
          (pv_lds_void*)(slot + k * kPwBlock), 16, 0, 0);
    }
  };

  if (producer) {
    for (int c = 0; c < kPbSlots - 1; ++c) copy(c);
    __builtin_amdgcn_s_waitcnt(pv_vmcnt((kPbSlots - 2) * kPbCopies));  // chunk 0 has landed
  }

  // Chains: wave 2 r runs range r; lane = (head hl, feature group fg), the
  // features fh * 64 + 4 fg .. + 3.  Probability row (r * kPbRows + rr) * 4
  // + hl lives in block row / 2 at piece 2 q + row % 2 for key group q (4
  // keys).
  const int hl = lane / (kPbHalf / kPbFeat), fg = lane % (kPbHalf / kPbFeat);
  const int r = wave / 2;
  const int jb0 = r ? jb0_1 : 0;
  const int f0 = fh * kPbHalf + kPbFeat * fg;
  const uint16_t* vrow = a.v_cache + static_cast<uint64_t>(g * kHeadDim + f0) * a.cap;
  int poff[kPbRows];
#pragma unroll
  for (int rr = 0; rr < kPbRows; ++rr) {
    const int prow = (r * kPbRows + rr) * 4 + hl;
    poff[rr] = (prow / 2) * kPwBlock + (prow % 2) * 16;
  }
  auto begin_of = [&](int rr) { return r ? split_of(rr) : 0; };
  auto end_of = [&](int rr) { return r ? count_of(rr) : split_of(rr); };
  // The last 8 keys of the wave's union range: V loads past it are clamped
  // there (inside the cache rows) and never used.
  const int last8 = ((r ? end1 : end0) - 1) & ~7;
  float acc[kPbRows][kPbFeat];
#pragma unroll
  for (int rr = 0; rr < kPbRows; ++rr)
#pragma unroll
    for (int i = 0; i < kPbFeat; ++i) acc[rr][i] = 0.0f;
  // V of the key group starting at key `key`: 8 keys of each of the lane's
  // 4 feature rows.
  struct VGroup {
    u32x4 w[kPbFeat];
  };
  auto load_v = [&](VGroup& x, int key) {
    const int k = min(max(key, 0), last8);
#pragma unroll
    for (int i = 0; i < kPbFeat; ++i) x.w[i] = *reinterpret_cast<const u32x4*>(vrow + static_cast<uint64_t>(i) * a.cap + k);
  };

  for (int c = 0; c < chunks; ++c) {
    __builtin_amdgcn_s_barrier();  // chunk c is in its slot; every chain is done with chunk c - 1
    if (producer) {
      copy(c + kPbSlots - 1);
      __builtin_amdgcn_s_waitcnt(pv_vmcnt((kPbSlots - 2) * kPbCopies));
      continue;
    }
    const uint8_t* cur = slot_of(c);
    const int cs = jb0 + kPwChunk * c;
    // Keys [lo, hi) of the chunk lie in every row's range; [lo_any, hi_any)
    // in some row's (wave-uniform: the rows and ranges are).
    int lo = 0, hi = kPwChunk, lo_any = kPwChunk, hi_any = 0;
#pragma unroll
    for (int rr = 0; rr < kPbRows; ++rr) {
      if (rr < n) {
        const int l0 = max(begin_of(rr) - cs, 0), h0 = min(end_of(rr) - cs, kPwChunk);
        lo = max(lo, l0);
        hi = min(hi, h0);
        if (h0 > l0) {
          lo_any = min(lo_any, l0);
          hi_any = max(hi_any, h0);
        }
      }
    }
    const int q0 = lo_any / 8, q1 = (hi_any + 7) / 8;
    if (q1 <= q0) continue;
    auto run = [&](const VGroup& x, int q) {
      const bool masked = !(8 * q >= lo && 8 * q + 8 <= hi);
      float pp[kPbRows][8];
#pragma unroll
      for (int rr = 0; rr < kPbRows; ++rr) {
        const float4 pa = *reinterpret_cast<const float4*>(cur + poff[rr] + 32 * (2 * q));
        const float4 pc = *reinterpret_cast<const float4*>(cur + poff[rr] + 32 * (2 * q + 1));
        pp[rr][0] = pa.x; pp[rr][1] = pa.y; pp[rr][2] = pa.z; pp[rr][3] = pa.w;
        pp[rr][4] = pc.x; pp[rr][5] = pc.y; pp[rr][6] = pc.z; pp[rr][7] = pc.w;
      }
      auto widen = [&](int e, float (&vf)[kPbFeat]) {
#pragma unroll
        for (int i = 0; i < kPbFeat; ++i) {
          const uint32_t word = (e >> 1) == 0 ? x.w[i].x : (e >> 1) == 1 ? x.w[i].y : (e >> 1) == 2 ? x.w[i].z : x.w[i].w;
          vf[i] = (e & 1) ? dl_bf16_hi(word) : dl_bf16_lo(word);
        }
      };
      if (!masked) {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          float vf[kPbFeat];
          widen(e, vf);
#pragma unroll
          for (int rr = 0; rr < kPbRows; ++rr)
#pragma unroll
            for (int i = 0; i < kPbFeat; ++i) acc[rr][i] = fma_rn(pp[rr][e], vf[i], acc[rr][i]);
        }
      } else {
        // Each step kept only where the key lies in the row's range (a
        // select, so the chain is unchanged elsewhere).
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int j = cs + 8 * q + e;
          float vf[kPbFeat];
          widen(e, vf);
#pragma unroll
          for (int rr = 0; rr < kPbRows; ++rr) {
            const bool in = rr < n && j >= begin_of(rr) && j < end_of(rr);
#pragma unroll
            for (int i = 0; i < kPbFeat; ++i) {
              const float t = fma_rn(pp[rr][e], vf[i], acc[rr][i]);
              acc[rr][i] = in ? t : acc[rr][i];
            }
          }
        }
      }
    };
    // Two key groups of V in flight ahead of the one being multiplied.
    VGroup x0, x1, x2;
    load_v(x0, cs + 8 * q0);
    load_v(x1, cs + 8 * (q0 + 1));
    int q = q0;
    for (; q + 3 <= q1; q += 3) {
      load_v(x2, cs + 8 * (q + 2));
      run(x0, q);
      load_v(x0, cs + 8 * (q + 3));
      run(x1, q + 1);
      load_v(x1, cs + 8 * (q + 4));
      run(x2, q + 2);
    }
    if (q < q1) run(x0, q);
    if (q + 1 < q1) run(x1, q + 1);
  }
  if (producer) {
    __builtin_amdgcn_s_waitcnt(pv_vmcnt(0));  // no copy outstanding at exit
  }
  if (wave == 2) {
#pragma unroll
    for (int rr = 0; rr < kPbRows; ++rr)
#pragma unroll
      for (int i = 0; i < kPbFeat; ++i) second[rr][i][lane] = acc[rr][i];
  }
  __syncthreads();
  if (wave == 0) {
#pragma unroll
    for (int rr = 0; rr < kPbRows; ++rr)
      if (rr < n) {
#pragma unroll
        for (int i = 0; i < kPbFeat; ++i)
          a.att[static_cast<uint64_t>(rb + rr) * a.q_heads * kHeadDim + (g * group + hl) * kHeadDim + f0 + i] =
              bf16_bits(acc[rr][i] + second[rr][i][lane]);
      }
  }
}

// Short-context attention in one kernel (the reference's retained-score
// kernel shape, attention.cu:231-383): grid (query head, sequence), 256
// threads.  Wave 0 applies the head's RMSNorm + RoPE to q; wave 1 does the
// same for the group's new key (written to the cache by the first head of
// the group).  32 groups of 8 lanes score keys (ranges merged at 4,2,1),
// scores stay in LDS, the max and the 32-partial denominator follow, and
// the two PV key ranges run as 2 x 128 threads over the transposed V rows.
// Below kFusedKeys keys one launch (and its fused QKV / O forms) beats the
// three-kernel split: measured per decode step on MI355X, the crossover lies
// between 1536 and 1800 keys (1280 keys: 3345 against 3432 us; 1536: 3409
// against 3458; 1800: 3554 against 3524).
constexpr int kFusedKeys = 1536;
constexpr int kAttnThreads = 512;
constexpr int kAttnKeysPerPass = kAttnThreads / 8;
constexpr int kAttnKeyPasses = 8;     // key rows issued at kernel entry: 512 keys
constexpr int kAttnValueBlocks = 16;  // 8-key V blocks per PV chain issued at entry (two 64-key blocks)

// The attention of query head slot `slot` (group-minor numbering) of row
// `b`; false when the loop is stopped (nothing is written).  kHandoff writes
// the output with device-coherent stores and waits for them, for a reader
// in the same launch (no cache writeback needed).
// Hand-off words between the workgroup roles of one launch: uint32 words,
// one 128-byte line (32 words) each, zero between launches.  `go` is the
// first of 8 go-flag lines (a waiting workgroup polls the line of its XCD,
// so the polling spreads over 8 lines), `exit` counts the last role's
// finished workgroups (the last one zeroes lines [0, exit]), `failure`
// records an expired wait.
struct Handoff {
  uint32_t* words;
  int go, exit, failure;
};
constexpr uint32_t kHandoffPolls = 1u << 22;

__device__ __forceinline__ uint32_t* handoff_line(const Handoff& hs, int line) { return hs.words + 32 * line; }

// Thread 0 polls its XCD's go line (relaxed device-coherent loads, no cache
// invalidation); a wait that expires records the failure and goes on.
__device__ __forceinline__ void handoff_wait(const Handoff& hs) {
  if (threadIdx.x == 0) {
    const uint32_t* go = handoff_line(hs, hs.go + blockIdx.x % 8);
    uint32_t polls = 0;
    while (__hip_atomic_load(go, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == 0u) {
      __builtin_amdgcn_s_sleep(4);
      if (++polls == kHandoffPolls) {
        __hip_atomic_store(handoff_line(hs, hs.failure), 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        break;
      }
    }
  }
  __syncthreads();
}

// Raises the 8 go lines starting at `go`.
__device__ __forceinline__ void handoff_raise(const Handoff& hs, int go) {
  for (int x = 0; x < 8; ++x)
    __hip_atomic_store(handoff_line(hs, go + x), 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Tagged hand-off words: each 64-bit word carries two BF16 values in its low
// half and the writing launch's tag in its high half, stored and loaded as
// one naturally aligned 64-bit atomic (single-copy atomic, device-coherent:
// `global_store_dwordx2 ... sc1` / `global_load_dwordx2 ... sc1`).  A reader
// polls its own words until every tag is the launch's, so it needs neither
// the writer's store acknowledgements nor a counter or a go flag: the values
// are in the word that tells it they are current.  The tag is the launch's
// epoch + 1; the epoch word is advanced once per live launch by its last
// workgroup, so a word left over from any earlier launch carries another tag.
struct Tagged {
  uint64_t* words;
  uint32_t tag;
  int k, v, att;  // word offsets of the k row, the new v row and the attention output (q at 0)
  int row;        // words per row (row b's words start at words + b * row)
};

__device__ __forceinline__ void tagged_put(uint64_t* w, uint32_t data, uint32_t tag) {
  __hip_atomic_store(w, static_cast<uint64_t>(data) | (static_cast<uint64_t>(tag) << 32), __ATOMIC_RELAXED,
                     __HIP_MEMORY_SCOPE_AGENT);
}

// Reads the N words src[k] once each is tagged `tag`: all loads are issued
// first, then only the stale ones are read again.  A wait that expires
// records the failure and goes on.
template <int N>
__device__ __forceinline__ void tagged_gather(const uint64_t* const (&src)[N], uint32_t tag, uint32_t* failure,
                                              uint32_t (&out)[N]) {
  uint64_t x[N];
#pragma unroll
  for (int k = 0; k < N; ++k) x[k] = __hip_atomic_load(src[k], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  uint32_t polls = 0;
  for (;;) {
    bool ready = true;
#pragma unroll
    for (int k = 0; k < N; ++k) ready = ready && static_cast<uint32_t>(x[k] >> 32) == tag;
    if (ready) break;
    if (++polls == kHandoffPolls) {
      __hip_atomic_store(failure, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      break;
    }
    __builtin_amdgcn_s_sleep(1);
#pragma unroll
    for (int k = 0; k < N; ++k)
      if (static_cast<uint32_t>(x[k] >> 32) != tag)
        x[k] = __hip_atomic_load(src[k], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
#pragma unroll
  for (int k = 0; k < N; ++k) out[k] = static_cast<uint32_t>(x[k]);
}

// kFromQkv: q, k and the new v row are written in this launch (by the QKV
// workgroups before the attention ones in the grid) as the tagged words of
// `tg`: the head rows are read from them once tagged, the chain holding the
// current position takes its value from the tagged v row (the V cache column
// is written in this launch too), and the output goes out as tagged words
// (an expired wait records its failure on `hs`'s failure line).
//
// kSplit > 1 spreads one head's PV over kSplit workgroups: `slot` then runs
// over q_heads x kSplit, and part slot / q_heads owns features
// [part F, part F + F), F = 128 / kSplit, as one wavefront per chain half.
// Every part computes the head's scores and softmax itself (identical
// values), so no part waits for another; the parts' PV chains run on
// different compute units.
template <bool kHandoff = false, bool kFromQkv = false, int kSplit = 1>
__device__ __forceinline__ bool attn_fused_body(const AttnArgs& a, int slot, int b, const Handoff* hs = nullptr,
                                                const Tagged* tg = nullptr) {
  static_assert(kSplit == 1 || kSplit == 2 || kSplit == 4, "a head splits into 1, 2 or 4 feature parts");
  __shared__ float qs[kHeadDim];
  __shared__ float ks[kHeadDim];
  __shared__ __align__(16) float sc[kFusedKeys];
  __shared__ float red[kAttnThreads];
  __shared__ float wave_max[kAttnThreads / 64];
  __shared__ float denominator_shared;
  // Workgroups are dealt to the XCDs round-robin by linear id: numbering the
  // query heads group-minor puts the heads of one K/V group on one XCD, whose
  // L2 then serves the group's key and value rows once for all of them.
  const int group = a.q_heads / a.kv_heads;
  const int part = slot / a.q_heads, head_slot = slot % a.q_heads;
  const int g = head_slot % a.kv_heads, h = g * group + head_slot / a.kv_heads;
  const int tid = threadIdx.x;
  const int wave = tid / 64, lane = tid % 64;
  const uint64_t qw = static_cast<uint64_t>(a.q_heads) * kHeadDim, kw = static_cast<uint64_t>(a.kv_heads) * kHeadDim;
  // This token's q/k rows and their norm gains do not depend on the loop
  // state: they are issued before the control block is read, and the rope
  // row of the position right after it.  Loads retire in order, so anything
  // issued before them would delay the head norms.
  HeadOperands head{};
  const uint16_t* head_row = wave == 0 ? a.q_raw + b * qw + static_cast<uint64_t>(h) * kHeadDim
                                       : a.k_raw + b * kw + static_cast<uint64_t>(g) * kHeadDim;
  if (wave < 2) {
    const uint16_t* gain = wave == 0 ? a.q_norm : a.k_norm;
    if constexpr (!kFromQkv) {
      head.xa = dl_bf16_to_f32(head_row[lane]);
      head.xb = dl_bf16_to_f32(head_row[lane + 64]);
    }
    head.ga = dl_bf16_to_f32(gain[lane]);
    head.gb = dl_bf16_to_f32(gain[lane + 64]);
  }
  if (!a.ctl->active) return false;
  const uint64_t pos = a.ctl->position + static_cast<uint64_t>(b) * a.pos_step;
  const int count = static_cast<int>(pos) + 1;
  const float* rope_pos = a.rope + pos * kHeadDim;
  uint16_t* kc = a.k_cache + b * a.cache_seq_stride + static_cast<uint64_t>(g) * a.cap * kHeadDim;
  if (wave < 2) {
    head.cosine = rope_pos[2 * lane];
    head.sine = rope_pos[2 * lane + 1];
  }

  // Cached K rows and V blocks do not depend on this token: issue the first
  // kAttnKeyPasses passes of key rows and kAttnValueBlocks 8-key blocks of
  // each PV chain before the head norms, so their latency overlaps them.
  __builtin_amdgcn_sched_barrier(0);
  const int kg = tid / 8, l = tid % 8;
  u32x4 kpre[kAttnKeyPasses][2];
#pragma unroll
  for (int p = 0; p < kAttnKeyPasses; ++p) {
    const int j = min(p * kAttnKeysPerPass + kg, count - 1);
    const u32x4* src = reinterpret_cast<const u32x4*>(kc + static_cast<uint64_t>(j) * kHeadDim + 16 * l);
    kpre[p][0] = src[0];
    kpre[p][1] = src[1];
  }
  // PV chains: one chain per lane of feature f and half (half 0: keys
  // [0, split), half 1: [split, count)).  Whole heads: waves 0-1 and 2-3
  // hold the halves (64 features each); parts: wave 0 and wave 1.
  const int split = (count - 1) / 2 + 1;
  // Wave-uniform chain half, so the PV loop bounds stay in scalar registers.
  constexpr int kPartFeatures = kHeadDim / kSplit;
  constexpr int kHalfWaves = kSplit == 1 ? 2 : 1;
  const int half = __builtin_amdgcn_readfirstlane(wave) / kHalfWaves;
  const int fl = (wave % kHalfWaves) * 64 + lane;  // feature within the part
  const int f = part * kPartFeatures + fl % kPartFeatures;
  const bool chain = wave < 2 * kHalfWaves && fl < kPartFeatures;
  const int begin = half ? split : 0, end = half ? count : split;
  const int first_block = begin & ~7;
  const uint16_t* v = a.v_cache + b * a.cache_seq_stride + static_cast<uint64_t>(g * kHeadDim + f) * a.cap;
  u32x4 vpre[kAttnValueBlocks];
  if (chain) {
#pragma unroll
    for (int i = 0; i < kAttnValueBlocks; ++i) {
      const int jb = min(first_block + 8 * i, a.cap - 8);
      vpre[i] = *reinterpret_cast<const u32x4*>(v + jb);
    }
  }
  float v_pos = 0.0f;  // the new value at `pos` of this lane's feature (kFromQkv)
  if constexpr (kFromQkv) {
    // A lane of a head wave reads values lane and lane + 64 of its head row
    // (words lane / 2 and 32 + lane / 2); a chain lane reads its feature's
    // new value.  The waves that do neither go straight to the barrier.
    __builtin_amdgcn_sched_barrier(0);
    uint32_t* failure = handoff_line(*hs, hs->failure);
    const int c = g * kHeadDim + f;
    if (wave < 2) {
      const uint64_t* row = tg->words + (wave == 0 ? h * (kHeadDim / 2) : tg->k + g * (kHeadDim / 2)) + lane / 2;
      const uint64_t* src[3] = {row, row + 32, chain ? tg->words + tg->v + c / 2 : row};
      uint32_t x[3];
      tagged_gather<3>(src, tg->tag, failure, x);
      head.xa = (lane & 1) ? dl_bf16_hi(x[0]) : dl_bf16_lo(x[0]);
      head.xb = (lane & 1) ? dl_bf16_hi(x[1]) : dl_bf16_lo(x[1]);
      if (chain) v_pos = (c & 1) ? dl_bf16_hi(x[2]) : dl_bf16_lo(x[2]);
    } else if (chain) {
      const uint64_t* src[1] = {tg->words + tg->v + c / 2};
      uint32_t x[1];
      tagged_gather<1>(src, tg->tag, failure, x);
      v_pos = (c & 1) ? dl_bf16_hi(x[0]) : dl_bf16_lo(x[0]);
    }
  }

  __builtin_amdgcn_sched_barrier(0);
  if (wave == 0) head_norm_rope(head, lane, a.eps, qs);
  if (wave == 1) {
    head_norm_rope(head, lane, a.eps, ks);
    if (h % group == 0 && part == 0) {
      kc[pos * kHeadDim + lane] = bf16_bits(ks[lane]);
      kc[pos * kHeadDim + lane + 64] = bf16_bits(ks[lane + 64]);
    }
  }
  __syncthreads();

  // Scores: 8 lanes per key, each an FMA chain over 16 contiguous features,
  // merged at offsets 4, 2, 1 (attention.cu:231-300).  The row at `pos` is
  // the freshly rotated key (its cache row may not be written yet).
  {
    float q[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) q[i] = qs[16 * l + i];
    auto score = [&](int j, const u32x4 w0, const u32x4 w1) {
      float kf[16];
      if (static_cast<uint64_t>(j) == pos) {
#pragma unroll
        for (int i = 0; i < 16; ++i) kf[i] = ks[16 * l + i];
      } else {
        kf[0] = dl_bf16_lo(w0.x); kf[1] = dl_bf16_hi(w0.x); kf[2] = dl_bf16_lo(w0.y); kf[3] = dl_bf16_hi(w0.y);
        kf[4] = dl_bf16_lo(w0.z); kf[5] = dl_bf16_hi(w0.z); kf[6] = dl_bf16_lo(w0.w); kf[7] = dl_bf16_hi(w0.w);
        kf[8] = dl_bf16_lo(w1.x); kf[9] = dl_bf16_hi(w1.x); kf[10] = dl_bf16_lo(w1.y); kf[11] = dl_bf16_hi(w1.y);
        kf[12] = dl_bf16_lo(w1.z); kf[13] = dl_bf16_hi(w1.z); kf[14] = dl_bf16_lo(w1.w); kf[15] = dl_bf16_hi(w1.w);
      }
      float acc = 0.0f;
#pragma unroll
      for (int i = 0; i < 16; ++i) acc = fma_rn(q[i], kf[i], acc);
      acc = acc + row_down<4>(acc);
      acc = acc + row_down<2>(acc);
      acc = acc + row_down<1>(acc);
      if (l == 0 && j < count) sc[j] = acc * a.scale;
    };
    // A ring of kAttnKeyPasses passes: consuming pass p issues pass
    // p + kAttnKeyPasses into the same registers, so that many key rows stay
    // in flight over the whole row.
    constexpr int kRing = kAttnKeyPasses * kAttnKeysPerPass;
    for (int base0 = 0; base0 < count; base0 += kRing) {
#pragma unroll
      for (int p = 0; p < kAttnKeyPasses; ++p) {
        const int base = base0 + p * kAttnKeysPerPass;
        if (base < count) {
          const u32x4 w0 = kpre[p][0], w1 = kpre[p][1];
          if (base + kRing < count) {
            const int j = min(base + kRing + kg, count - 1);
            const u32x4* src = reinterpret_cast<const u32x4*>(kc + static_cast<uint64_t>(j) * kHeadDim + 16 * l);
            kpre[p][0] = src[0];
            kpre[p][1] = src[1];
          }
          score(base + kg, w0, w1);
        }
      }
    }
  }
  __syncthreads();

  // Softmax: exact maximum, e = exp(s - m), 32 strided partial sums merged
  // 16..1, p = e / l (attention.cu:301-360).
  float m = -INFINITY;
  for (int j = tid; j < count; j += kAttnThreads) m = fmaxf(m, sc[j]);
  m = dl::wave_max(m);
  if (lane == 0) wave_max[wave] = m;
  __syncthreads();
  m = wave_max[0];
#pragma unroll
  for (int w = 1; w < kAttnThreads / 64; ++w) m = fmaxf(m, wave_max[w]);
  for (int j = tid; j < count; j += kAttnThreads) sc[j] = dl_expf(sc[j] - m);
  __syncthreads();
  if (tid < 32) {
    // The partial's additions in ascending key order, its LDS reads issued
    // eight at a time (the last, partial batch too: reads past the keys are
    // clamped and their additions skipped).
    float partial = 0.0f;
    int j = tid;
    for (; j + 7 * 32 < count; j += 8 * 32) {
      float e[8];
#pragma unroll
      for (int k = 0; k < 8; ++k) e[k] = sc[j + 32 * k];
#pragma unroll
      for (int k = 0; k < 8; ++k) partial = partial + e[k];
    }
    if (j < count) {
      float e[7];
#pragma unroll
      for (int k = 0; k < 7; ++k) e[k] = sc[min(j + 32 * k, count - 1)];
#pragma unroll
      for (int k = 0; k < 7; ++k) partial = j + 32 * k < count ? partial + e[k] : partial;
    }
    // Offsets 16, 8, 4, 2, 1 as __shfl_down(partial, off, 32); below 16 the
    // lanes that feed lane 0 read within their row (DPP).
    partial = partial + __shfl_down(partial, 16, 32);
    partial = partial + row_down<8>(partial);
    partial = partial + row_down<4>(partial);
    partial = partial + row_down<2>(partial);
    partial = partial + row_down<1>(partial);
    if (tid == 0) denominator_shared = partial;
  }
  __syncthreads();
  const float denominator = denominator_shared;
  for (int j = tid; j < count; j += kAttnThreads) sc[j] = sc[j] / denominator;
  __syncthreads();

  // PV: two ascending FMA chains over [0, split) and [split, count), in
  // 64-key blocks from the 8-aligned key below `begin`; the first and last
  // block mask the keys outside the chain.  A block's 64 probabilities are
  // read from LDS as 16 float4s before its FMAs, and the next block's V
  // rows are in flight meanwhile (two register buffers, uniform trip count).
  // Loads past the chain are clamped to its last 8 keys (4 for the
  // probabilities) and never used.
  if (chain) {
    float acc = 0.0f;
    const int blocks = end > begin ? (end - first_block + 63) / 64 : 0;
    const int last8 = (end - 1) & ~7, last4 = (end - 1) & ~3;
    auto load = [&](u32x4* vb, int x) {
      const int jb = first_block + 64 * min(x, blocks - 1);
#pragma unroll
      for (int i = 0; i < 8; ++i) vb[i] = *reinterpret_cast<const u32x4*>(v + min(jb + 8 * i, last8));
    };
    auto run = [&](const u32x4* vb, int x) {
      const int jb = first_block + 64 * x;
      const int lo = max(begin - jb, 0), hi = min(end - jb, 64);
      // kFromQkv: the block holding `pos` takes the new value there
      // (wave-uniform: pos, jb and the chain's range are).
      const int pi = static_cast<int>(pos) - jb;
      const bool patch = kFromQkv && pi >= lo && pi < hi;
      if (hi <= lo) return;
      if (kPartFeatures % 64 == 0 && lo == 0 && hi == 64 && !patch) {
        // A block wholly inside the chain: the 64 probabilities as four
        // VGPRs of 16 (lane l holds key jb + 16 q + l % 16), each FMA taking
        // its key's value by DPP broadcast.  Every lane of the wave is a
        // chain lane of one half here (one or two parts per head), as the
        // broadcast needs.
        float pq[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) pq[q] = sc[jb + 16 * q + (lane & 15)];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const u32x4 w0 = vb[2 * q], w1 = vb[2 * q + 1];
          const float vf[16] = {dl_bf16_lo(w0.x), dl_bf16_hi(w0.x), dl_bf16_lo(w0.y), dl_bf16_hi(w0.y),
                                dl_bf16_lo(w0.z), dl_bf16_hi(w0.z), dl_bf16_lo(w0.w), dl_bf16_hi(w0.w),
                                dl_bf16_lo(w1.x), dl_bf16_hi(w1.x), dl_bf16_lo(w1.y), dl_bf16_hi(w1.y),
                                dl_bf16_lo(w1.z), dl_bf16_hi(w1.z), dl_bf16_lo(w1.w), dl_bf16_hi(w1.w)};
          acc = fma16_row_bcast(acc, pq[q], vf);
        }
        return;
      }
      float4 pc[16];
#pragma unroll
      for (int i = 0; i < 16; ++i) pc[i] = *reinterpret_cast<const float4*>(sc + min(jb + 4 * i, last4));
      // Wave-uniform branches: a block wholly inside the chain runs its 64
      // steps straight; in the chain's first and last blocks (and the one
      // holding `pos`) each 8-key group is skipped, run straight or run
      // masked; a block past the chain does nothing.
      if (hi <= lo) return;
      auto group = [&](int i, bool full) {
        float vf[8] = {dl_bf16_lo(vb[i].x), dl_bf16_hi(vb[i].x), dl_bf16_lo(vb[i].y), dl_bf16_hi(vb[i].y),
                       dl_bf16_lo(vb[i].z), dl_bf16_hi(vb[i].z), dl_bf16_lo(vb[i].w), dl_bf16_hi(vb[i].w)};
        const float pf[8] = {pc[2 * i].x, pc[2 * i].y, pc[2 * i].z, pc[2 * i].w,
                             pc[2 * i + 1].x, pc[2 * i + 1].y, pc[2 * i + 1].z, pc[2 * i + 1].w};
        if (full) {
#pragma unroll
          for (int e = 0; e < 8; ++e) acc = fma_rn(pf[e], vf[e], acc);
        } else {
          if (patch) {
#pragma unroll
            for (int e = 0; e < 8; ++e) vf[e] = 8 * i + e == pi ? v_pos : vf[e];
          }
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const float t = fma_rn(pf[e], vf[e], acc);
            acc = (8 * i + e >= lo && 8 * i + e < hi) ? t : acc;
          }
        }
      };
      if (lo == 0 && hi == 64 && !patch) {
#pragma unroll
        for (int i = 0; i < 8; ++i) group(i, true);
      } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const int g0 = 8 * i;
          if (g0 >= hi || g0 + 8 <= lo) continue;
          const bool holds_pos = patch && pi >= g0 && pi < g0 + 8;
          if (g0 >= lo && g0 + 8 <= hi && !holds_pos)
            group(i, true);
          else
            group(i, false);
        }
      }
    };
    if (blocks > 0) {
      // Blocks 0 and 1 come from the entry prefetch.
      static_assert(kAttnValueBlocks == 16, "the entry prefetch holds two 64-key blocks");
      u32x4 va[8], vb[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) va[i] = vpre[i];
#pragma unroll
      for (int i = 0; i < 8; ++i) vb[i] = vpre[8 + i];
      run(va, 0);
      int x = 1;
      if (blocks > 1) {
        load(va, 2);
        __builtin_amdgcn_sched_barrier(0);
        run(vb, 1);
        __builtin_amdgcn_sched_barrier(0);
        x = 2;
      }
      for (; x + 2 <= blocks; x += 2) {
        load(vb, x + 1);
        __builtin_amdgcn_sched_barrier(0);
        run(va, x);
        __builtin_amdgcn_sched_barrier(0);
        load(va, x + 2);
        __builtin_amdgcn_sched_barrier(0);
        run(vb, x + 1);
        __builtin_amdgcn_sched_barrier(0);
      }
      if (x < blocks) run(va, x);
    }
    red[half * kHeadDim + fl] = acc;
  }
  __syncthreads();
  uint16_t* att = a.att + static_cast<uint64_t>(b) * qw + h * kHeadDim + part * kPartFeatures;
  if constexpr (kFromQkv) {
    if (tid < kPartFeatures / 2) {
      const uint32_t lo = bf16_bits(red[2 * tid] + red[2 * tid + kHeadDim]);
      const uint32_t hi = bf16_bits(red[2 * tid + 1] + red[2 * tid + 1 + kHeadDim]);
      tagged_put(tg->words + tg->att + (h * kHeadDim + part * kPartFeatures) / 2 + tid, lo | (hi << 16), tg->tag);
    }
  } else if constexpr (kHandoff) {
    if (tid < kPartFeatures / 2) {
      const uint32_t lo = bf16_bits(red[2 * tid] + red[2 * tid + kHeadDim]);
      const uint32_t hi = bf16_bits(red[2 * tid + 1] + red[2 * tid + 1 + kHeadDim]);
      __hip_atomic_store(reinterpret_cast<uint32_t*>(att) + tid, lo | (hi << 16), __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
      __builtin_amdgcn_s_waitcnt(pv_vmcnt(0));
    }
  } else {
    if (tid < kPartFeatures) att[tid] = bf16_bits(red[tid] + red[tid + kHeadDim]);
  }
  return true;
}

template <int kSplit>
__global__ __launch_bounds__(kAttnThreads) void k_attn_fused(AttnArgs a) {
  attn_fused_body<false, false, kSplit>(a, blockIdx.x, blockIdx.y);
}

// ------------------------------------------------- residual GEMV (O, down)
struct ResidualArgs {
  const Control* ctl;
  const uint16_t* x;     // [B][I]
  const u32x4* w;        // packed [D][I]
  uint16_t* h;           // [B][D], updated in place
  uint16_t* capture;     // [B][cap][D] or null
  const float* steer;    // [B][D] or null
  int I, D, cap, layer;
  int row0;              // first row of this launch's row group
  // Rows are sequences (decode: row r is sequence r at ctl->position), or,
  // with same_sequence, consecutive positions of sequence `sequence`
  // (row r at ctl->position + r; chunked prompt pass).
  int same_sequence, sequence;
  // Rows from row0 that exist (a launch of a larger row template for fewer
  // rows reads and writes only these).
  int rows = 1 << 30;
};


// Residual epilogue of one tile: output row tile * RW + i of sequence row b
// is h = round(h + round(y)), then the optional steering and capture.  With
// several rows the merged sums (in lanes i * P) go through the wavefront's
// LDS area `ep` (RW * B floats) so that lane i * B + b finishes (i, b) and
// all the h updates of a tile are issued together.
// Output `row` of step row `b` (launch-relative): h = round(h + round(y)),
// then the optional steering and capture.
__device__ __forceinline__ void residual_store(const ResidualArgs& a, int row, int b, float y, uint64_t pos,
                                               bool steer, bool capture, uint32_t steer_mask) {
  const int r = a.row0 + b;
  const int seq = a.same_sequence ? a.sequence : r;
  const uint64_t at = static_cast<uint64_t>(r) * a.D + row;
  float value = rbf(dl_bf16_to_f32(a.h[at]) + rbf(y));
  if (steer && ((steer_mask >> seq) & 1u)) value = rbf(value + a.steer[static_cast<uint64_t>(seq) * a.D + row]);
  a.h[at] = bf16_bits(value);
  if (capture) {
    const uint64_t at_pos = a.same_sequence ? pos + r : pos;
    a.capture[(static_cast<uint64_t>(seq) * a.cap + at_pos) * a.D + row] = bf16_bits(value);
  }
}

template <int P, int B>
__device__ __forceinline__ void residual_outputs(const ResidualArgs& a, const float (&acc)[B], int tile, int lane,
                                                 float* ep, uint64_t pos, bool steer, bool capture,
                                                 uint32_t steer_mask) {
  constexpr int RW = 64 / P;
  auto finish = [&](int i, int b, float y) {
    residual_store(a, tile * RW + i, b, y, pos, steer, capture, steer_mask);
  };
  if constexpr (B == 1) {
    if (lane % P == 0) finish(lane / P, 0, acc[0]);
  } else {
    if (lane % P == 0) {
#pragma unroll
      for (int b = 0; b < B; ++b) ep[(lane / P) * B + b] = acc[b];
    }
    wave_lds_sync();
    if (lane < RW * B && lane % B < live_rows<B>(a.rows)) finish(lane / B, lane % B, ep[lane]);
    wave_lds_sync();
  }
}

// y = round(x W^T); h = round(h + y); optionally h = round(h + steer) and a
// copy of h into the capture arena at the current position.
// Split as in k_qkv: each tile's rows as Split work items of B / Split rows.
template <int P, int B, int Split = 1>
__global__ __launch_bounds__(gemv_waves(B) * 64) void k_residual(ResidualArgs a) {
  constexpr int W = gemv_waves(B);
  constexpr int BR = B / Split;
  static_assert(B % Split == 0, "rows split evenly");
  extern __shared__ float xs[];
  __shared__ float epi[W * (64 / P) * BR];
  const int wave = threadIdx.x / 64, lane = threadIdx.x % 64;
  constexpr int RW = 64 / P;
  const int tiles = a.D / RW;
  const int items = tiles * Split;
  const int S = a.I / (8 * P);
  const uint64_t chunks = static_cast<uint64_t>(S) * 64;
  const int first = blockIdx.x * W + wave;
  FirstBatch fb{};
  // The prologue returns, after issuing its loads, when the loop is stopped
  // (grid-uniform flag).
  if (!stage_rows<P>(
          a.x + static_cast<uint64_t>(a.row0) * a.I, a.I, B, xs,
          [&] {
            if (first < items) issue_first(a.w + (first / Split) * chunks, lane, fb);
          },
          0, &a.ctl->active, live_rows<B>(a.rows)))
    return;
  __syncthreads();
  const uint64_t pos = a.ctl->position;
  const bool steer = a.steer != nullptr && a.layer == a.ctl->steer_layer;
  const bool capture = a.capture != nullptr && a.layer == a.ctl->capture_layer;
  const uint32_t steer_mask = a.ctl->steer_mask;
  for (int item = first; item < items; item += gridDim.x * W) {
    const int tile = item / Split, b0 = (item % Split) * BR;
    float acc[BR];
    const int next = item + gridDim.x * W;
    // One tile per wavefront at B = 1 leaves one or two wavefronts per SIMD:
    // two batches in flight per wavefront keep more of HBM busy.
    chain_tile<P, BR, true>(a.w + tile * chunks, xs + b0 * staged_floats(P, a.I), a.I, lane, acc, &fb,
                            next < items ? a.w + (next / Split) * chunks : nullptr);
    if constexpr (Split == 1) {
      residual_outputs<P, BR>(a, acc, tile, lane, epi + wave * RW * BR, pos, steer, capture, steer_mask);
    } else {
      ResidualArgs part = a;
      part.row0 += b0;
      part.rows -= b0;
      residual_outputs<P, BR>(part, acc, tile, lane, epi + wave * RW * BR, pos, steer, capture, steer_mask);
    }
  }
}

// k_residual for rows whose staged inputs do not fit in LDS at once (the
// down projection, I = 12288, at four or more rows): the inputs are staged
// kChunkInputs at a time and every wavefront carries its chains across the
// blocks in ascending input order, so each partial is the same FMA chain as
// in k_residual.  Each wavefront owns one tile per pass; all wavefronts of a
// workgroup take part in every staging barrier (uniform trip counts).
constexpr int kChunkInputs = 4096;

template <int P, int B>
__global__ __launch_bounds__(gemv_waves(B) * 64) void k_residual_chunked(ResidualArgs a) {
  constexpr int W = gemv_waves(B);
  constexpr int kChunkSteps = kChunkInputs / (8 * P);
  extern __shared__ float xs[];
  __shared__ float epi[W * (64 / P) * B];
  if (!a.ctl->active) return;
  const uint64_t pos = a.ctl->position;
  const int wave = threadIdx.x / 64, lane = threadIdx.x % 64;
  constexpr int RW = 64 / P;
  const int tiles = a.D / RW;
  const int S = a.I / (8 * P);
  const uint64_t chunks = static_cast<uint64_t>(S) * 64;
  const int blocks = a.I / kChunkInputs;
  const bool steer = a.steer != nullptr && a.layer == a.ctl->steer_layer;
  const bool capture = a.capture != nullptr && a.layer == a.ctl->capture_layer;
  const uint32_t steer_mask = a.ctl->steer_mask;
  for (int base = blockIdx.x * W; base < tiles; base += gridDim.x * W) {
    const int tile = base + wave;
    const bool active = tile < tiles;
    const u32x4* src = a.w + static_cast<uint64_t>(active ? tile : base) * chunks;
    float acc[B];
#pragma unroll
    for (int b = 0; b < B; ++b) acc[b] = 0.0f;
    FirstBatch fb{};
    for (int c = 0; c < blocks; ++c) {
      __syncthreads();  // every wavefront is done with the previous block
      stage_block<P, B, kChunkInputs, W * 64>(a.x + static_cast<uint64_t>(a.row0) * a.I + c * kChunkInputs, a.I, xs,
                                             [&] {
                                               if (c == 0 && active) issue_first(src, lane, fb);
                                             },
                                             live_rows<B>(a.rows));
      __syncthreads();
      if (active) {
        // The block width is passed as a run-time value (a.I / blocks): a
        // compile-time width lets the compiler unroll the whole block and
        // hoist its LDS reads past the register file.
        const u32x4* at = src + static_cast<uint64_t>(c) * kChunkSteps * 64;
        chain_body<P, B>(at, xs, a.I / blocks, lane, acc, &fb, c + 1 < blocks ? at + kChunkSteps * 64 : nullptr);
      }
    }
    chain_merge<P, B>(acc);
    if (active) residual_outputs<P, B>(a, acc, tile, lane, epi + wave * RW * B, pos, steer, capture, steer_mask);
  }
}

// --------------------------------------- attention + O projection, batch 1
// One launch for a short-context step's attention and O projection of a
// single row.  Workgroups [0, q_heads kAttnSplit) run the fused attention,
// kAttnSplit per query head (each the PV chains of its part of the head's
// features); the others each own 8 O tiles (one per wavefront).  An O
// wavefront issues its whole weight tile (kOChunks 16-byte chunks per lane)
// at entry, so the O weights stream from HBM while the attention runs, then
// waits for the attention output, stages it and runs the tile's chains from
// registers: the same chain steps, in the same order, as k_residual.
//
// Hand-off: the attention output goes through device-coherent stores (each
// wavefront waits until its stores are done), each attention workgroup then
// counts itself; the last one raises the go lines, every O workgroup polls
// the line of its XCD and reads the output with device-coherent loads.  All
// hand-off traffic meets at the device's coherence point, so no cache
// writeback or invalidation (which scans a whole XCD's L2) is needed.  The
// waiting workgroups come after the ones they wait for in the grid, which
// are dispatched first, and the waits are bounded (handoff_wait).
constexpr int kOChunks = 32;           // 16-byte weight chunks per lane: I / (8 P) with I = 4096, P = 16
// Workgroups per query head (feature parts of its PV): 2 measured better
// than 1 and 4 in both fused launches.
constexpr int kAttnSplit = 2;
constexpr int kOWaves = kAttnThreads / 64;
// k_attn_o's lines: attention count 0, go 1-8, O exit 9, failure 10.
constexpr Handoff kAttnOLayout{nullptr, 1, 9, 10};
constexpr int kAttnOCount = 0;
constexpr int kSyncWords = 32 * 11;

struct AttnOArgs {
  AttnArgs attn;
  ResidualArgs o;
  uint32_t* sync;
};

// The O workgroup `wg` of `o_workgroups`: waits on hs's go lines (or, with
// `tg`, reads the attention output as tagged words); the last to finish
// zeroes lines [0, hs.exit] (and with `tg` advances the epoch word `epoch`).
template <bool kTagged = false, int B = 1>
__device__ __forceinline__ void o_prefetched(const ResidualArgs& a, int wg, int o_workgroups, const Handoff& hs,
                                             const Tagged* tg = nullptr, uint32_t* epoch = nullptr) {
  static_assert(B == 1 || kTagged, "several rows come as tagged words");
  constexpr int P = 16, RW = 64 / P;
  // 16-byte aligned: the attention's static arrays come first, and the chain
  // reads the staged inputs 16 bytes at a time.
  extern __shared__ __align__(16) float xs[];
  __shared__ float epi[kOWaves * RW * B];
  const int wave = threadIdx.x / 64, lane = threadIdx.x % 64;
  const int tile = wg * kOWaves + wave;
  const u32x4* src = a.w + static_cast<uint64_t>(tile) * (kOChunks * 64) + lane;
  u32x4 w[kOChunks];
#pragma unroll
  for (int s = 0; s < kOChunks; ++s) w[s] = load_stream(src + s * 64);
  if (!a.ctl->active) return;
  const uint64_t pos = a.ctl->position;
  // The attention output, read device-coherently (it was written in this
  // launch), staged as stage_rows does; all of a thread's loads are issued
  // before any is used.
  constexpr int kWords = kOChunks * 8 * P / 2 / kAttnThreads;
  static_assert(kWords * 2 * kAttnThreads == kOChunks * 8 * P, "the O input row splits evenly over the threads");
  // Row b's words follow row 0's at b * qkvo_tagged_words (the per-row
  // stride `tg->row`).
  uint32_t v[B * kWords];
  if constexpr (kTagged) {
    const uint64_t* src[B * kWords];
#pragma unroll
    for (int b = 0; b < B; ++b)
#pragma unroll
      for (int k = 0; k < kWords; ++k)
        src[b * kWords + k] = tg->words + b * tg->row + tg->att + threadIdx.x + k * kAttnThreads;
    tagged_gather<B * kWords>(src, tg->tag, handoff_line(hs, hs.failure), v);
  } else {
    handoff_wait(hs);
    const uint32_t* x32 = reinterpret_cast<const uint32_t*>(a.x);
#pragma unroll
    for (int k = 0; k < kWords; ++k)
      v[k] = __hip_atomic_load(x32 + threadIdx.x + k * kAttnThreads, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
#pragma unroll
  for (int b = 0; b < B; ++b)
#pragma unroll
    for (int k = 0; k < kWords; ++k) {
      const int wi = threadIdx.x + k * kAttnThreads;
      stage_put<P>(xs, a.I, b, 2 * wi, dl_bf16_lo(v[b * kWords + k]));
      stage_put<P>(xs, a.I, b, 2 * wi + 1, dl_bf16_hi(v[b * kWords + k]));
    }
  __syncthreads();
  const int L = a.I / P, stride = L + kXsPad, bstride = P * stride;
  const float* xt = xs + (lane % P) * stride;
  float acc[B];
#pragma unroll
  for (int b = 0; b < B; ++b) acc[b] = 0.0f;
#pragma unroll
  for (int s = 0; s < kOChunks; ++s) chain_step<B>(w[s], xt, bstride, s, acc);
  chain_merge<P, B>(acc);
  residual_outputs<P, B>(a, acc, tile, lane, epi + wave * RW * B, pos, false, false, 0u);
  __syncthreads();
  if (threadIdx.x == 0) {
    const uint32_t done = __hip_atomic_fetch_add(handoff_line(hs, hs.exit), 1u, __ATOMIC_RELAXED,
                                                 __HIP_MEMORY_SCOPE_AGENT);
    if (done == static_cast<uint32_t>(o_workgroups) - 1u) {
      // Every workgroup of this launch is past its wait: clear for the next.
      if constexpr (kTagged) {
        // Every tagged word was read (each is some O workgroup's input or
        // was read by an attention workgroup whose output this one read),
        // so every workgroup has read the epoch: the next launch may use
        // the next tag.
        __hip_atomic_store(handoff_line(hs, hs.exit), 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(epoch, tg->tag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      } else {
        for (int line = 0; line <= hs.exit; ++line)
          __hip_atomic_store(handoff_line(hs, line), 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
  }
}

// Counts one finished workgroup on `count`; the last of `total` raises the
// go lines `go`.
__device__ __forceinline__ void handoff_signal(const Handoff& hs, int count, uint32_t total, int go) {
  if (threadIdx.x == 0) {
    const uint32_t n = __hip_atomic_fetch_add(handoff_line(hs, count), 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (n == total - 1u) handoff_raise(hs, go);
  }
}

__global__ __launch_bounds__(kAttnThreads) void k_attn_o(AttnOArgs a) {
  const uint32_t heads = static_cast<uint32_t>(a.attn.q_heads) * kAttnSplit;
  Handoff hs = kAttnOLayout;
  hs.words = a.sync;
  if (blockIdx.x < heads) {
    if (!attn_fused_body<true, false, kAttnSplit>(a.attn, blockIdx.x, 0)) return;
    __syncthreads();  // every output word of this workgroup has been written
    handoff_signal(hs, kAttnOCount, heads, hs.go);
    return;
  }
  o_prefetched(a.o, blockIdx.x - heads, gridDim.x - heads, hs);
}

// ------------------------------------ QKV + attention + O projection, batch 1
// One launch for a short-context step's QKV projection, attention and O
// projection of a single row: workgroups [0, qkv_workgroups) own one QKV
// tile per wavefront (held in registers, as k_qkv's batch-1 path), then the
// attention workgroups (kAttnSplit per query head), then the O workgroups
// (as in k_attn_o).  Every hand-off goes through tagged words (Tagged): the
// QKV workgroups write q, k and the new V values as tagged words (the new V
// values also into the cache column, for later steps) and exit; each
// attention workgroup issues its key and value prefetch, then reads its own
// head's q row, its group's k row and its features' new V values once they
// carry this launch's tag, and writes its output as tagged words; each O
// workgroup reads the whole attention output the same way.  So no role
// waits for another's store acknowledgements, counters or go flags, and a
// head starts as soon as its own rows are written.  Sync lines: O exit
// count 0, failure 1, epoch 2.
constexpr Handoff kQkvoLayout{nullptr, -1, 0, 1};
constexpr int kQkvoEpoch = 2;
constexpr int kQkvoSyncWords = 32 * 3;
constexpr int kQkvWaves = kAttnThreads / 64;

// Tagged words of one k_qkv_attn_o launch: q (QW / 2), k (KW / 2), the new
// V values (KW / 2), the attention output (QW / 2).
__host__ __device__ constexpr int qkvo_tagged_words(int QW, int KW) { return QW + KW; }

struct QkvAttnOArgs {
  QkvArgs qkv;
  AttnArgs attn;
  ResidualArgs o;
  uint64_t* tagged;
  uint32_t* sync;
};

template <int B>
__device__ __forceinline__ void qkv_phase(const QkvArgs& a, const Tagged& tg) {
  constexpr int W = kQkvWaves;
  extern __shared__ __align__(16) float lds[];
  float* xs16 = lds;
  float* xs32 = lds + B * staged_floats(16, kWholeTileInputs);
  __shared__ float scratch[W * 40];
  const int wave = threadIdx.x / 64, lane = threadIdx.x % 64;
  const int q_tiles = a.QW / 4, k_tiles = a.KW / 2;
  const uint64_t q_chunks = static_cast<uint64_t>(a.D / 128) * 64, k_chunks = static_cast<uint64_t>(a.D / 256) * 64;
  const int tile = blockIdx.x * W + wave;
  const bool is_q = tile < q_tiles;
  int kt = tile - q_tiles;
  const bool is_v = !is_q && kt >= k_tiles;
  if (is_v) kt -= k_tiles;
  const u32x4* src = (is_q ? a.w + tile * q_chunks
                           : a.w + q_tiles * q_chunks + (is_v ? k_tiles : 0) * k_chunks + kt * k_chunks) + lane;
  constexpr int SQ = kWholeTileInputs / 128, SK = kWholeTileInputs / 256;
  u32x4 w[SQ];
  if (!norm_stage<B, true, true, W / 2>(
          a.h, a.norm, a.eps, xs16, xs32, scratch,
          [&] {
#pragma unroll
            for (int s = 0; s < SK; ++s) w[s] = load_stream(src + s * 64);
          },
          &a.ctl->active))
    return;
  if (is_q) {
#pragma unroll
    for (int s = SK; s < SQ; ++s) w[s] = load_stream(src + s * 64);
  }
  __syncthreads();
  float acc[B];
#pragma unroll
  for (int b = 0; b < B; ++b) acc[b] = 0.0f;
  if (is_q) {
    constexpr int P = 16, stride = kWholeTileInputs / P + kXsPad;
    const float* xt = xs16 + (lane % P) * stride;
#pragma unroll
    for (int s = 0; s < SQ; ++s) chain_step<B>(w[s], xt, P * stride, s, acc);
    chain_merge<P, B>(acc);
    // Lanes 0, 16, 32, 48 hold rows 4 t .. 4 t + 3: two words per row.
#pragma unroll
    for (int b = 0; b < B; ++b) {
      const uint32_t y = bf16_bits(acc[b]);
      const uint32_t y1 = __shfl_down(y, 16, 64);
      if (lane == 0 || lane == 32) tagged_put(tg.words + b * tg.row + tile * 2 + lane / 32, y | (y1 << 16), tg.tag);
    }
  } else {
    constexpr int P = 32, stride = kWholeTileInputs / P + kXsPad;
    const float* xt = xs32 + (lane % P) * stride;
#pragma unroll
    for (int s = 0; s < SK; ++s) chain_step<B>(w[s], xt, P * stride, s, acc);
    chain_merge<P, B>(acc);
    // Lanes 0 and 32 hold rows 2 kt and 2 kt + 1: one word per row.  Row b's
    // new V values go to its cache column as k_qkv writes them.
#pragma unroll
    for (int b = 0; b < B; ++b) {
      const uint32_t y = bf16_bits(acc[b]);
      const uint32_t y1 = __shfl_down(y, 32, 64);
      if (is_v && lane % P == 0)
        a.v_cache[b * a.cache_seq_stride + static_cast<uint64_t>(kt * 2 + lane / P) * a.cap + a.ctl->position] =
            static_cast<uint16_t>(y);
      if (lane == 0) tagged_put(tg.words + b * tg.row + (is_v ? tg.v : tg.k) + kt, y | (y1 << 16), tg.tag);
    }
  }
}

template <int B>
__global__ __launch_bounds__(kAttnThreads) __attribute__((amdgpu_waves_per_eu(2))) void k_qkv_attn_o(QkvAttnOArgs a) {
  const uint32_t heads = static_cast<uint32_t>(a.attn.q_heads) * kAttnSplit;
  const uint32_t nq = static_cast<uint32_t>(a.qkv.QW / 4 + a.qkv.KW) / kQkvWaves;
  Handoff hs = kQkvoLayout;
  hs.words = a.sync;
  uint32_t* epoch = handoff_line(hs, kQkvoEpoch);
  Tagged tg{a.tagged, __hip_atomic_load(epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + 1u, a.qkv.QW / 2,
            a.qkv.QW / 2 + a.qkv.KW / 2, a.qkv.QW / 2 + a.qkv.KW, qkvo_tagged_words(a.qkv.QW, a.qkv.KW)};
  if (blockIdx.x < nq) {
    qkv_phase<B>(a.qkv, tg);
    return;
  }
  if (blockIdx.x < nq + B * heads) {
    // Row-major over (row, head slot): row b's heads read and write row b's
    // tagged words.
    const uint32_t i = blockIdx.x - nq, b = i / heads;
    tg.words += b * tg.row;
    attn_fused_body<true, true, kAttnSplit>(a.attn, i % heads, b, &hs, &tg);
    return;
  }
  o_prefetched<true, B>(a.o, blockIdx.x - nq - B * heads, gridDim.x - nq - B * heads, hs, &tg, epoch);
}

// ------------------------------------------------------------ gate/up GEMV
struct GateUpArgs {
  const Control* ctl;
  const uint16_t* h;
  const uint16_t* norm;
  const u32x4* w;        // packed interleaved rows [g 2j, g 2j+1, u 2j, u 2j+1]
  uint16_t* act;         // [B][F]
  int D, F;
  float eps;
  int rows = 1 << 30;    // rows that exist (see QkvArgs::rows)
};

template <int B>
__global__ __launch_bounds__(gemv_waves(B) * 64) void k_gateup(GateUpArgs a) {
  constexpr int W = gemv_waves(B);
  extern __shared__ float xs[];
  __shared__ float scratch[W * 40];
  __shared__ float epi[W * 4 * B];
  const int wave = threadIdx.x / 64, lane = threadIdx.x % 64;
  const int tiles = a.F / 2;
  const int S = a.D / 128;
  const uint64_t chunks = static_cast<uint64_t>(S) * 64;
  const int first = blockIdx.x * W + wave;
  FirstBatch fb{};
  // The prologue returns, after issuing its loads, when the loop is stopped
  // (grid-uniform flag).
  if (!norm_stage<B, true, false, W / 2>(
          a.h, a.norm, a.eps, xs, nullptr, scratch,
          [&] {
            if (first < tiles) issue_first(a.w + first * chunks, lane, fb);
          },
          &a.ctl->active, live_rows<B>(a.rows)))
    return;
  __syncthreads();
  (void)S;
  for (int tile = first; tile < tiles; tile += gridDim.x * W) {
    float acc[B];
    const int next = tile + gridDim.x * W;
    chain_tile<16, B>(a.w + tile * chunks, xs, a.D, lane, acc, &fb, next < tiles ? a.w + next * chunks : nullptr);
    // Lanes 0, 16, 32, 48 hold gate 2t, gate 2t+1, up 2t, up 2t+1.  With
    // several rows the sums go through LDS so that lane o * B + b evaluates
    // SiLU(gate) * up of output 2t + o for row b: one SiLU per lane.
    if constexpr (B == 1) {
      const float up = __shfl_down(acc[0], 32, 64);
      if (lane == 0 || lane == 16)
        a.act[tile * 2 + lane / 16] = bf16_bits(silu_times(rbf(acc[0]), rbf(up)));
    } else {
      float* ep = epi + wave * 4 * B;
      if (lane % 16 == 0) {
#pragma unroll
        for (int b = 0; b < B; ++b) ep[(lane / 16) * B + b] = acc[b];
      }
      wave_lds_sync();
      if (lane < 2 * B && lane % B < live_rows<B>(a.rows)) {
        const int o = lane / B, b = lane % B;
        a.act[static_cast<uint64_t>(b) * a.F + tile * 2 + o] =
            bf16_bits(silu_times(rbf(ep[o * B + b]), rbf(ep[(2 + o) * B + b])));
      }
      wave_lds_sync();
    }
  }
}

// ---------------------------------------------- exact GEMM over many rows
// The projections of the chunked prompt pass when a chunk holds many rows
// (positions of one sequence).  Every output is the same P-partial FMA chain
// and upper-into-lower merge as in the GEMV kernels (projection.cu:139-482):
// partial t of output f is the FMA chain over inputs t, t + P, ... in
// ascending order.  Only the assignment of chains to lanes differs: lane
// (g, t) of a wavefront owns partial t of kXgFeat consecutive outputs for
// kXgPos rows, so each staged input feeds kXgFeat FMAs and each widened
// weight kXgPos, and the weights are read once per kXgRows rows instead of
// once per step row.
//
// Workgroup: 8 wavefronts = kXgWN output blocks x kXgWP row blocks, tile
// kXgWN * (64 / P) * kXgFeat outputs x kXgRows rows.  The rows' inputs pass
// through LDS kXgChunk inputs at a time as FP32 in the GEMV's staged layout
// (partial-major rows padded by kXsPad floats, so the P lanes of a read hit
// distinct banks); the next pass's inputs are loaded into registers while
// the current one is multiplied.  The weights come straight from memory in
// the packed layout, one 8-element step ahead.  Workgroups that share
// weights (same blockIdx.x) land on one XCD when gridDim.x is a multiple of
// 8, so its L2 serves the weights to the row blocks.
constexpr int kXgThreads = 512;
constexpr int kXgWN = 4, kXgWP = 2;
constexpr int kXgFeat = 4;                  // outputs per lane (one P = 16 tile, two P = 32 tiles)
constexpr int kXgPos = 16;                  // rows per lane
constexpr int kXgRows = kXgWP * kXgPos;     // rows per workgroup
constexpr int kXgChunk = 1024;              // inputs staged per pass
constexpr int kXgMinRows = 16;              // fewer rows run through the batched GEMVs

enum XgEpilogue : int {
  kXgQ = 0,         // out[b][f] = BF16(acc): Q rows
  kXgKV = 1,        // K rows (f < kw) to out[b][f], V rows to the transposed cache column of row b
  kXgResidual = 2,  // residual_store (O and down)
  kXgGateUp = 3,    // interleaved [g 2j, g 2j+1, u 2j, u 2j+1] -> SiLU(g) * u, P32-permuted act rows
};

struct XgemmArgs {
  const Control* ctl;
  const uint16_t* x;     // [B][K] BF16 input rows: P-permuted (`permuted`) or natural order
  const u32x4* w;        // packed rows with P partials
  int B, N, K, permuted;
  uint16_t* out;         // kXgQ [B][N]; kXgKV k rows [B][kw]; kXgGateUp act [B][N / 2]
  uint16_t* v_cache;     // kXgKV: V^T of this layer; row b's column is position + b * v_stride
  uint64_t v_stride;
  int kw, cap;
  ResidualArgs res;      // kXgResidual
};

__host__ __device__ constexpr size_t xgemm_lds(int P) {
  return size_t(kXgRows) * P * (kXgChunk / P + kXsPad) * sizeof(float);
}

template <int P, int EPI>
__global__ __launch_bounds__(kXgThreads) void k_xgemm(XgemmArgs a) {
  constexpr int G = 64 / P;                    // lane groups of a wavefront
  constexpr int RW = 64 / P;                   // outputs per packed tile
  constexpr int WF = G * kXgFeat;              // outputs per wavefront
  constexpr int TF = kXgWN * WF;               // outputs per workgroup
  constexpr int stride = kXgChunk / P + kXsPad;
  constexpr int row_floats = P * stride;       // staged floats per row
  constexpr int steps = kXgChunk / (8 * P);    // 8-element chain steps per pass
  constexpr int kPieces = kXgRows * kXgChunk / 8 / kXgThreads;  // 16-byte input pieces per thread per pass
  static_assert(kXgFeat % RW == 0 || RW % kXgFeat == 0, "whole tiles per lane");
  static_assert(kXgWN * kXgWP * 64 == kXgThreads, "one wavefront per (output block, row block)");
  extern __shared__ float xs[];                // [kXgRows][P][stride]
  if (!a.ctl->active) return;
  const int wave = threadIdx.x / 64, lane = threadIdx.x % 64;
  const int g = lane / P, t = lane % P;
  const int f0 = blockIdx.x * TF + (wave % kXgWN) * WF + g * kXgFeat;  // first output of this lane
  const int b0 = blockIdx.y * kXgRows;                                 // first row of the workgroup
  const int pb = (wave / kXgWN) * kXgPos;                              // first row of this lane in the tile
  const int S = a.K / (8 * P), passes = a.K / kXgChunk;
  const uint64_t pos = a.ctl->position;

  // Packed chunk of output f, step s, partial t: ((f / RW) S + s) 64 + (f % RW) P + t.
  const u32x4* wsrc[kXgFeat];
#pragma unroll
  for (int j = 0; j < kXgFeat; ++j) {
    const int f = f0 + j;
    wsrc[j] = a.w + static_cast<uint64_t>(f / RW) * S * 64 + (f % RW) * P + t;
  }
  // Weights of a step: kXgFeat 16-byte chunks; two register sets alternate
  // (a pass has an even number of steps), each loaded one step ahead.
  u32x4 wa[kXgFeat], wb[kXgFeat];
  auto load_w = [&](u32x4* w, int sg) {
    const uint64_t at = static_cast<uint64_t>(sg < S ? sg : S - 1) * 64;  // past the end: reload the last step
#pragma unroll
    for (int j = 0; j < kXgFeat; ++j) w[j] = wsrc[j][at];
  };
  load_w(wa, 0);

  // Piece q of row r of a pass: inputs 8q .. 8q + 7 of the pass (rows past
  // B repeat row B - 1 and are never stored).
  u32x4 xr[kPieces];
  auto load_x = [&](int c) {
#pragma unroll
    for (int j = 0; j < kPieces; ++j) {
      const int piece = threadIdx.x + j * kXgThreads, r = piece / (kXgChunk / 8), q = piece % (kXgChunk / 8);
      const int b = min(b0 + r, a.B - 1);
      xr[j] = *reinterpret_cast<const u32x4*>(a.x + static_cast<uint64_t>(b) * a.K + c * kXgChunk + 8 * q);
    }
  };
  auto store_x = [&] {
#pragma unroll
    for (int j = 0; j < kPieces; ++j) {
      const int piece = threadIdx.x + j * kXgThreads, r = piece / (kXgChunk / 8), q = piece % (kXgChunk / 8);
      const float v[8] = {dl_bf16_lo(xr[j].x), dl_bf16_hi(xr[j].x), dl_bf16_lo(xr[j].y), dl_bf16_hi(xr[j].y),
                          dl_bf16_lo(xr[j].z), dl_bf16_hi(xr[j].z), dl_bf16_lo(xr[j].w), dl_bf16_hi(xr[j].w)};
      float* row = xs + r * row_floats;
      if (a.permuted) {
        // P-permuted: piece q holds chain elements 8 (q / P) .. + 7 of
        // partial q % P (the pass starts on a block of 8 P inputs).
        float4* dst = reinterpret_cast<float4*>(row + (q % P) * stride + 8 * (q / P));
        dst[0] = make_float4(v[0], v[1], v[2], v[3]);
        dst[1] = make_float4(v[4], v[5], v[6], v[7]);
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int i = 8 * q + e;
          row[(i % P) * stride + i / P] = v[e];
        }
      }
    }
  };

  float acc[kXgFeat * kXgPos];
#pragma unroll
  for (int i = 0; i < kXgFeat * kXgPos; ++i) acc[i] = 0.0f;
  // One chain step (8 elements) of every (output, row) pair of the lane.
  auto step = [&](const u32x4* w, int s) {
    float wf[kXgFeat][8];
#pragma unroll
    for (int j = 0; j < kXgFeat; ++j) {
      wf[j][0] = dl_bf16_lo(w[j].x); wf[j][1] = dl_bf16_hi(w[j].x);
      wf[j][2] = dl_bf16_lo(w[j].y); wf[j][3] = dl_bf16_hi(w[j].y);
      wf[j][4] = dl_bf16_lo(w[j].z); wf[j][5] = dl_bf16_hi(w[j].z);
      wf[j][6] = dl_bf16_lo(w[j].w); wf[j][7] = dl_bf16_hi(w[j].w);
    }
#pragma unroll
    for (int i = 0; i < kXgPos; ++i) {
      const float* xp = xs + (pb + i) * row_floats + t * stride + 8 * s;
      const float4 xa = *reinterpret_cast<const float4*>(xp);
      const float4 xb = *reinterpret_cast<const float4*>(xp + 4);
#pragma unroll
      for (int j = 0; j < kXgFeat; ++j) {
        float v = acc[j * kXgPos + i];
        v = fma_rn(xa.x, wf[j][0], v);
        v = fma_rn(xa.y, wf[j][1], v);
        v = fma_rn(xa.z, wf[j][2], v);
        v = fma_rn(xa.w, wf[j][3], v);
        v = fma_rn(xb.x, wf[j][4], v);
        v = fma_rn(xb.y, wf[j][5], v);
        v = fma_rn(xb.z, wf[j][6], v);
        v = fma_rn(xb.w, wf[j][7], v);
        acc[j * kXgPos + i] = v;
      }
    }
  };
  static_assert(steps % 2 == 0, "the weight register sets alternate within a pass");
  load_x(0);
  for (int c = 0; c < passes; ++c) {
    __syncthreads();  // every wavefront is done with the previous pass
    store_x();
    if (c + 1 < passes) load_x(c + 1);
    __syncthreads();
#pragma unroll
    for (int s = 0; s < steps; s += 2) {
      const int sg = c * steps + s;
      load_w(wb, sg + 1);
      step(wa, s);
      load_w(wa, sg + 2);
      step(wb, s + 1);
    }
  }
  chain_merge<P, kXgFeat * kXgPos>(acc);
  if (t != 0) return;

  bool steer = false, capture = false;
  uint32_t steer_mask = 0;
  if constexpr (EPI == kXgResidual) {
    steer = a.res.steer != nullptr && a.res.layer == a.ctl->steer_layer;
    capture = a.res.capture != nullptr && a.res.layer == a.ctl->capture_layer;
    steer_mask = a.ctl->steer_mask;
  }
#pragma unroll
  for (int i = 0; i < kXgPos; ++i) {
    const int b = b0 + pb + i;
    if (b >= a.B) break;
    if constexpr (EPI == kXgGateUp) {
      // One P = 16 tile: [g 2j, g 2j+1, u 2j, u 2j+1], j = f0 / 4.
#pragma unroll
      for (int o = 0; o < 2; ++o) {
        const uint32_t n = static_cast<uint32_t>(f0 / 2 + o);
        a.out[static_cast<uint64_t>(b) * (a.N / 2) + prefill::permuted(n, 32)] =
            bf16_bits(silu_times(rbf(acc[o * kXgPos + i]), rbf(acc[(2 + o) * kXgPos + i])));
      }
    } else {
#pragma unroll
      for (int j = 0; j < kXgFeat; ++j) {
        const int f = f0 + j;
        const float y = acc[j * kXgPos + i];
        if constexpr (EPI == kXgQ) {
          a.out[static_cast<uint64_t>(b) * a.N + f] = bf16_bits(y);
        } else if constexpr (EPI == kXgKV) {
          if (f < a.kw)
            a.out[static_cast<uint64_t>(b) * a.kw + f] = bf16_bits(y);
          else
            a.v_cache[static_cast<uint64_t>(b) * a.v_stride + static_cast<uint64_t>(f - a.kw) * a.cap + pos] =
                bf16_bits(y);
        } else {
          residual_store(a.res, f, b, y, pos, steer, capture, steer_mask);
        }
      }
    }
  }
}

// ------------------------------------------------------------------ LM head
struct HeadArgs {
  const Control* ctl;
  const uint16_t* h;
  const uint16_t* norm;
  const u32x4* w;          // packed [V][D], P = 16
  uint16_t* logits;        // [B][V]
  uint64_t* partial_keys;  // [B][gridDim.x]
  uint32_t* partial_flags; // [B][gridDim.x]
  int D;
  uint32_t V;
  float eps;
  int row0;                // first sequence of this launch's row group
  int rows = 1 << 30;      // rows from row0 that exist (see QkvArgs::rows)
};

// Orders BF16 logits: key = (ordered value << 32) | ~id, so the maximum key
// is the largest value with the lowest id (categorical.cpp:168-173).
// Flags: bit 0 NaN or +inf seen, bit 1 a finite candidate seen.
__device__ __forceinline__ void logit_key(uint16_t bits, uint32_t id, uint64_t* key, uint32_t* flags) {
  const uint32_t magnitude = bits & 0x7fffu;
  if (magnitude > 0x7f80u || bits == 0x7f80u) {
    *flags |= 1u;
    return;
  }
  if (bits == 0xff80u) return;
  *flags |= 2u;
  const uint32_t canonical = bits == 0x8000u ? 0u : bits;
  const uint32_t ordered = (canonical & 0x8000u) ? (~canonical & 0xffffu) : (canonical | 0x8000u);
  const uint64_t k = (static_cast<uint64_t>(ordered) << 32) | (0xffffffffu - id);
  if (k > *key) *key = k;
}

__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) {
#pragma unroll
  for (int off = 32; off; off >>= 1) {
    const uint32_t lo = __shfl_xor(static_cast<uint32_t>(v), off);
    const uint32_t hi = __shfl_xor(static_cast<uint32_t>(v >> 32), off);
    const uint64_t o = (static_cast<uint64_t>(hi) << 32) | lo;
    v = o > v ? o : v;
  }
  return v;
}

template <int B>
__global__ __launch_bounds__(gemv_waves(B) * 64) void k_lm_head(HeadArgs a) {
  constexpr int W = gemv_waves(B);
  extern __shared__ float xs[];
  __shared__ float scratch[W * 40];
  __shared__ uint64_t wave_keys[W][B];
  __shared__ uint32_t wave_flags[W][B];
  if (!a.ctl->active || !selecting(a.ctl)) return;
  const int wave = threadIdx.x / 64, lane = threadIdx.x % 64;
  const int tiles = static_cast<int>(a.V / 4);
  const int S = a.D / 128;
  const uint64_t chunks = static_cast<uint64_t>(S) * 64;
  const int first = blockIdx.x * W + wave;
  (void)S;
  FirstBatch fb{};
  const int rows = live_rows<B>(a.rows);
  norm_stage<B, true, false, W / 2>(a.h + static_cast<uint64_t>(a.row0) * a.D, a.norm, a.eps, xs, nullptr, scratch,
                                    [&] {
    if (first < tiles) issue_first(a.w + first * chunks, lane, fb);
  }, nullptr, rows);
  __syncthreads();
  uint64_t best[B];
  uint32_t flags[B];
#pragma unroll
  for (int b = 0; b < B; ++b) {
    best[b] = 0;
    flags[b] = 0;
  }
  for (int tile = first; tile < tiles; tile += gridDim.x * W) {
    float acc[B];
    const int next = tile + gridDim.x * W;
    chain_tile<16, B>(a.w + tile * chunks, xs, a.D, lane, acc, &fb, next < tiles ? a.w + next * chunks : nullptr);
    if (lane % 16 == 0) {
      const uint32_t row = static_cast<uint32_t>(tile * 4 + lane / 16);
#pragma unroll
      for (int b = 0; b < B; ++b) {
        if (b >= rows) break;
        const uint16_t bits = bf16_bits(acc[b]);
        a.logits[static_cast<uint64_t>(a.row0 + b) * a.V + row] = bits;
        logit_key(bits, row, &best[b], &flags[b]);
      }
    }
  }
#pragma unroll
  for (int b = 0; b < B; ++b) {
    const uint64_t k = wave_max_u64(best[b]);
    uint32_t f = flags[b];
#pragma unroll
    for (int off = 32; off; off >>= 1) f |= __shfl_xor(f, off);
    if (lane == 0) {
      wave_keys[wave][b] = k;
      wave_flags[wave][b] = f;
    }
  }
  __syncthreads();
  if (static_cast<int>(threadIdx.x) < rows) {
    const int b = threadIdx.x;
    uint64_t k = 0;
    uint32_t f = 0;
    for (int w = 0; w < W; ++w) {
      k = wave_keys[w][b] > k ? wave_keys[w][b] : k;
      f |= wave_flags[w][b];
    }
    a.partial_keys[static_cast<uint64_t>(a.row0 + b) * gridDim.x + blockIdx.x] = k;
    a.partial_flags[static_cast<uint64_t>(a.row0 + b) * gridDim.x + blockIdx.x] = f;
  }
}

// ---------------------------------------------------------------- step end
struct EndArgs {
  Control* ctl;
  const uint64_t* partial_keys;
  const uint32_t* partial_flags;
  int partials;
  uint32_t* selected;       // [B]
  uint32_t* out_tokens;     // [B][out_capacity]
  uint32_t out_capacity;
  const uint8_t* stop_mask; // [V]
  const uint32_t* intervention_state;  // [status, count], or null
  int batch;
  Journal journal;
};

// Greedy selection from the argmax partials (categorical rows were selected
// by the device sampler before this kernel), per-sequence token streams,
// stop latches and position advance (decode.cu finish_selection /
// finish_consumption).  A sequence that emitted a stop id emits nothing more.
__global__ __launch_bounds__(kBlock) void k_step_end(EndArgs a) {
  __shared__ uint64_t keys[kBlock];
  __shared__ uint32_t flags[kBlock];
  Control* c = a.ctl;
  if (!c->active) return;
  const bool select = selecting(c);
  if (select && c->mode == 0) {
    for (int b = 0; b < a.batch; ++b) {
      if (!row_selects(c, b)) continue;
      uint64_t k = 0;
      uint32_t f = 0;
      for (int i = threadIdx.x; i < a.partials; i += blockDim.x) {
        const uint64_t v = a.partial_keys[static_cast<uint64_t>(b) * a.partials + i];
        k = v > k ? v : k;
        f |= a.partial_flags[static_cast<uint64_t>(b) * a.partials + i];
      }
      keys[threadIdx.x] = k;
      flags[threadIdx.x] = f;
      __syncthreads();
      for (int off = kBlock / 2; off; off >>= 1) {
        if (threadIdx.x < off) {
          keys[threadIdx.x] = keys[threadIdx.x + off] > keys[threadIdx.x] ? keys[threadIdx.x + off] : keys[threadIdx.x];
          flags[threadIdx.x] |= flags[threadIdx.x + off];
        }
        __syncthreads();
      }
      if (threadIdx.x == 0) {
        if (flags[0] & 1u) {
          c->status |= 1u;
        } else if (!(flags[0] & 2u)) {
          c->status |= 2u;
        } else {
          const uint32_t id = 0xffffffffu - static_cast<uint32_t>(keys[0] & 0xffffffffu);
          a.selected[b] = id;
          const uint32_t emitted = c->row_generated[b];
          if (emitted < a.out_capacity) a.out_tokens[static_cast<uint64_t>(b) * a.out_capacity + emitted] = id;
          c->row_generated[b] = emitted + 1;
          if (a.stop_mask[id]) c->finished_mask |= 1u << b;
        }
      }
      __syncthreads();
    }
  }
  if (threadIdx.x != 0) return;
  const uint64_t pos = c->position;
  // Events of this step (decode.cu finish_prompt / finish_consumption /
  // finish_selection): every running sequence consumed `pos`; the selecting
  // ones chose the token of `pos + 1`; a sequence whose stop id was
  // selected earlier has now consumed it and ends with reason eos.
  for (int b = 0; b < a.batch; ++b)
    if (!((c->terminal_mask >> b) & 1u)) journal_write(a.journal, c, b, kConsumed, 0, pos, 1, 0, 0.0f);
  if (select && c->status == 0) {
    for (int b = 0; b < a.batch; ++b)
      if ((c->select_mask >> b) & 1u) journal_write(a.journal, c, b, kSelected, 0, pos + 1, 1, a.selected[b], 0.0f);
  }
  for (int b = 0; b < a.batch; ++b) {
    if (((c->finished_before & ~c->terminal_mask) >> b) & 1u) {
      journal_write(a.journal, c, b, kTerminal, kEos, pos + 1, c->row_generated[b], 0, 0.0f);
      c->terminal_mask |= 1u << b;
    }
  }
  if (select) {
    c->generated += 1;
    if (c->generated >= c->max_new || (c->finished_mask & c->all_mask) == c->all_mask) c->stop_pending = 1;
  } else if (c->stop_pending && pos + 1 >= c->prompt_length) {
    // The final selection has now been consumed (decode.cu finish_consumption).
    c->active = 0;
    c->reason = c->cancel_pending ? 2u
                                  : (c->max_new > 0 && (c->finished_mask & c->all_mask) == c->all_mask) ? 1u : 0u;
  }
  // decode.cu finish_consumption / finish_sequence: a latched intervention
  // failure ends the loop, and a loop that ends with its whole prompt
  // consumed must have applied the intervention exactly once.
  if (const uint32_t* iv = a.intervention_state) {
    if (iv[0] || (!c->active && pos + 1 >= c->prompt_length && iv[1] != 1)) c->status |= 16u;
  }
  if (c->status) {
    c->active = 0;
    c->reason = 3;
  }
  c->position = pos + 1;
  c->steps += 1;
  if (!c->active) journal_finish(a.journal, c, a.batch, pos + 1);
  journal_publish(a.journal, c, a.batch);
}

// Row-major seeded N(0, std) fill (untied embedding table).
__global__ void k_fill_rowmajor(uint16_t* p, uint64_t n, uint64_t seed, uint64_t stream, float scale) {
  const uint64_t step = static_cast<uint64_t>(gridDim.x) * blockDim.x;
  for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += step)
    p[i] = dl_normal_bf16(seed, stream, i, scale);
}

// Partial count of the reference projection rule (projection.cu:277-318).
int partials_for(uint64_t in_w, uint64_t out_w) { return (in_w <= 4096 && out_w > 1024) ? 16 : 32; }

__global__ void k_bench_control(const Control* live, Control* bench) {
  Control c = *live;
  c.active = 1;
  c.select_row = 1;
  c.capture_layer = -1;
  c.steer_layer = -1;
  if (c.position >= 1) c.position -= 1;
  *bench = c;
}

// Control of one chunk of the exact prompt pass: the live control with the
// loop active at `position` and the plan's capture / steering settings.
__global__ void k_chunk_control(const Control* live, Control* chunk, uint64_t position, int32_t capture_layer,
                                int32_t steer_layer, uint32_t steer_mask) {
  Control c = *live;
  c.active = 1;
  c.position = position;
  c.capture_layer = capture_layer;
  c.steer_layer = steer_layer;
  c.steer_mask = steer_mask;
  *chunk = c;
}

// Rotated keys of the rows of a chunk (consecutive positions of one
// sequence) written to the cache before the chunk's attention, which reads
// its predecessors' keys from there (rotary.cu:84-126).  Grid (kv head, row),
// one wavefront.
__global__ __launch_bounds__(64) void k_append_keys(AttnArgs a) {
  __shared__ float ks[kHeadDim];
  if (!a.ctl->active) return;
  const int g = blockIdx.x, b = blockIdx.y, lane = threadIdx.x;
  const uint64_t pos = a.ctl->position + static_cast<uint64_t>(b) * a.pos_step;
  const uint64_t kw = static_cast<uint64_t>(a.kv_heads) * kHeadDim;
  head_norm_rope(a.k_raw + b * kw + static_cast<uint64_t>(g) * kHeadDim, a.k_norm, a.rope + pos * kHeadDim, lane,
                 a.eps, ks);
  __syncthreads();
  uint16_t* kc = a.k_cache + b * a.cache_seq_stride + static_cast<uint64_t>(g) * a.cap * kHeadDim;
  kc[pos * kHeadDim + lane] = bf16_bits(ks[lane]);
  kc[pos * kHeadDim + lane + 64] = bf16_bits(ks[lane + 64]);
}

__global__ void k_seek(Control* c, uint64_t position) {
  c->position = position;
  c->active = 0;
}

// Reference-layout cache rows [count][Hkv][128] <-> the plan's layout:
// K head-major [Hkv][cap][128], V transposed [Hkv*128][cap].
__global__ void k_cache_rows(uint16_t* k_cache, uint16_t* v_cache, int cap, int kv_heads, uint64_t first,
                             uint64_t count, uint16_t* keys, uint16_t* values, int read) {
  const uint64_t n = count * kv_heads * kHeadDim;
  const uint64_t step = static_cast<uint64_t>(gridDim.x) * blockDim.x;
  for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += step) {
    const uint64_t j = first + i / (kv_heads * kHeadDim);
    const uint64_t g = (i / kHeadDim) % kv_heads, f = i % kHeadDim;
    uint16_t* kp = k_cache + (g * cap + j) * kHeadDim + f;
    uint16_t* vp = v_cache + (g * kHeadDim + f) * cap + j;
    if (read) {
      keys[i] = *kp;
      values[i] = *vp;
    } else {
      *kp = keys[i];
      *vp = values[i];
    }
  }
}

// ---------------------------------------------------- MFMA prefill helpers
// Embedding rows of prefill positions [first, first + rows) into h
// [padded][D]; rows past `rows` are zeroed.  The embedding override row
// replaces its position when the sequence is masked in.
struct PrefillEmbedArgs {
  const uint32_t* tokens;      // absolute-position history
  const uint16_t* lm_packed;   // tied: packed LM head (P = 16)
  const uint16_t* embedding;   // untied: row-major [V][D]
  const uint16_t* override_row;
  uint16_t* h;
  uint32_t rows, D;
  uint64_t first;
  int tied, override_row_active;
  uint64_t override_position;
};

__global__ __launch_bounds__(kBlock) void k_prefill_embed(PrefillEmbedArgs a) {
  const uint32_t r = blockIdx.x;
  uint16_t* out = a.h + static_cast<uint64_t>(r) * a.D;
  if (r >= a.rows) {
    for (uint32_t k = threadIdx.x; k < a.D; k += blockDim.x) out[k] = 0;
    return;
  }
  const uint64_t pos = a.first + r;
  const uint32_t token = a.tokens[pos];
  if (a.override_row_active && pos == a.override_position) {
    for (uint32_t k = threadIdx.x; k < a.D; k += blockDim.x) out[k] = a.override_row[k];
  } else if (a.tied) {
    for (uint32_t k = threadIdx.x; k < a.D; k += blockDim.x) out[k] = a.lm_packed[packed_index(token, k, 16, a.D)];
  } else {
    const uint16_t* row = a.embedding + static_cast<uint64_t>(token) * a.D;
    for (uint32_t k = threadIdx.x; k < a.D; k += blockDim.x) out[k] = row[k];
  }
}

// h <- BF16(FP32(h) + v) over prefill rows (all-position steering), then an
// optional copy of each row into the capture arena at its position.
__global__ __launch_bounds__(kBlock) void k_prefill_steer_capture(uint16_t* h, const float* steer, uint16_t* capture,
                                                                  uint32_t D, uint64_t first) {
  const uint32_t r = blockIdx.x;
  uint16_t* row = h + static_cast<uint64_t>(r) * D;
  for (uint32_t k = threadIdx.x; k < D; k += blockDim.x) {
    float value = dl_bf16_to_f32(row[k]);
    if (steer) {
      value = rbf(value + steer[k]);
      row[k] = bf16_bits(value);
    }
    if (capture) capture[(first + r) * D + k] = bf16_bits(value);
  }
}

// The plan's residual intervention (steering.cu:107-159) on the block output
// of `layer`, the Qwen3 intervention boundary after the second residual add
// (src/models/qwen3/model.h:7): of the launch's rows, the one holding
// sequence `sequence` at absolute position `position` gets
// h <- BF16(h + (strength * ||h||) * u).  Row r is at first + r * pos_step of
// sequence (same_sequence ? row_sequence : r), with first the control's
// position when a control is given (the loop must then be active).  A
// capture of the same layer is rewritten with the intervened row, as the
// reference copies captures after the boundary's producer step.  A failed
// application also latches the control's status and cancels the step's
// selection.  One workgroup.
struct InterveneArgs {
  Control* ctl;            // null: a prompt pass without a control
  uint16_t* h;             // [rows][D]
  const float* direction;  // [D] unit FP32 direction
  uint32_t* state;         // [status, count]
  uint16_t* capture;       // [batch][cap][D] or null
  uint64_t first, position, cap;
  uint32_t rows, D, sequence;
  int pos_step, same_sequence, row_sequence, layer, capture_layer;
  float strength;
};

__global__ __launch_bounds__(nla::kThreads) void k_plan_intervene(InterveneArgs a) {
  __shared__ float sums[nla::kLanes + 2];
  __shared__ uint32_t invalid;
  uint64_t first = a.first;
  int capture_layer = a.capture_layer;
  if (a.ctl) {
    if (!a.ctl->active) return;
    first = a.ctl->position;
    capture_layer = a.ctl->capture_layer;
  }
  uint64_t r;
  if (a.same_sequence) {
    if (static_cast<uint32_t>(a.row_sequence) != a.sequence || a.position < first) return;
    const uint64_t offset = a.position - first;
    if (a.pos_step == 0) {
      if (offset != 0) return;
      r = 0;
    } else {
      if (offset % a.pos_step != 0 || offset / a.pos_step >= a.rows) return;
      r = offset / a.pos_step;
    }
  } else {
    r = a.sequence;
    if (r >= a.rows || first + r * a.pos_step != a.position) return;
  }
  uint16_t* row = a.h + r * a.D;
  nla::intervene_row(row, a.direction, a.state, a.D, a.strength, sums, &invalid);
  if (a.capture && capture_layer == a.layer) {
    // Each thread reads back the elements it wrote in intervene_row.
    uint16_t* dst = a.capture + (static_cast<uint64_t>(a.sequence) * a.cap + a.position) * a.D;
    for (uint32_t k = threadIdx.x; k < a.D; k += blockDim.x) dst[k] = row[k];
  }
  if (a.ctl && threadIdx.x == 0 && a.state[0]) {
    a.ctl->status |= 16u;
    a.ctl->select_row = 0;
  }
}

}  // namespace
}  // namespace dl

// ===================================================================== host
using dl::guard;
using dl::require;

struct dl_qwen3 {
  dl_device* device = nullptr;
  dl_qwen3_config cfg{};
  int p_q = 16, p_kv = 32, p_o = 16, p_gu = 16, p_down = 32, p_lm = 16;
  uint64_t qkv_elems = 0, o_elems = 0, gu_elems = 0, down_elems = 0;
  std::vector<uint16_t*> qkv, o, gu, down, input_norm, post_norm, q_norm, k_norm;
  uint16_t* final_norm = nullptr;
  uint16_t* lm_head = nullptr;    // packed
  uint16_t* embedding = nullptr;  // row-major, untied only
  uint64_t resident = 0;
  std::vector<void*> allocations;

  uint16_t* alloc(uint64_t elements) {
    void* p = nullptr;
    const hipError_t e = hipMalloc(&p, elements * 2);
    if (e != hipSuccess) {
      (void)hipGetLastError();
      dl::fail(DL_LENGTH_ERROR, std::string("model allocation failed: ") + hipGetErrorString(e));
    }
    allocations.push_back(p);
    resident += elements * 2;
    return static_cast<uint16_t*>(p);
  }

  // The view of one logical parameter inside the packed storage.
  dl::PackedView view(int role, uint32_t layer, uint64_t* rows, uint64_t* cols) const {
    const uint64_t D = cfg.hidden, QW = uint64_t(cfg.q_heads) * cfg.head_dim,
                   KW = uint64_t(cfg.kv_heads) * cfg.head_dim, F = cfg.ffn;
    switch (role) {
      case DL_ROLE_Q: *rows = QW; *cols = D; return {qkv[layer], p_q, D, 0};
      case DL_ROLE_K: *rows = KW; *cols = D; return {qkv[layer] + QW * D, p_kv, D, 0};
      case DL_ROLE_V: *rows = KW; *cols = D; return {qkv[layer] + (QW + KW) * D, p_kv, D, 0};
      case DL_ROLE_O: *rows = D; *cols = QW; return {o[layer], p_o, QW, 0};
      case DL_ROLE_GATE: *rows = F; *cols = D; return {gu[layer], p_gu, D, 1};
      case DL_ROLE_UP: *rows = F; *cols = D; return {gu[layer], p_gu, D, 2};
      case DL_ROLE_DOWN: *rows = D; *cols = F; return {down[layer], p_down, F, 0};
      case DL_ROLE_LM_HEAD: *rows = cfg.vocab; *cols = D; return {lm_head, p_lm, D, 0};
      default: dl::fail(DL_INVALID_ARGUMENT, "role has no packed view");
    }
  }

  // Row-major vectors and tables.
  uint16_t* plain(int role, uint32_t layer, uint64_t* elements) const {
    const uint64_t D = cfg.hidden;
    switch (role) {
      case DL_ROLE_FINAL_NORM: *elements = D; return final_norm;
      case DL_ROLE_INPUT_NORM: *elements = D; return input_norm[layer];
      case DL_ROLE_POST_NORM: *elements = D; return post_norm[layer];
      case DL_ROLE_Q_NORM: *elements = cfg.head_dim; return q_norm[layer];
      case DL_ROLE_K_NORM: *elements = cfg.head_dim; return k_norm[layer];
      case DL_ROLE_EMBEDDING:
        if (cfg.tied_embeddings) return nullptr;
        *elements = uint64_t(cfg.vocab) * D;
        return embedding;
      default: return nullptr;
    }
  }

  ~dl_qwen3() {
    for (void* p : allocations) (void)hipFree(p);
  }
};

namespace {
void validate_config(const dl_qwen3_config& c) {
  require(c.layers > 0 && c.hidden > 0 && c.q_heads > 0 && c.kv_heads > 0 && c.ffn > 0 && c.vocab > 0,
          "empty Qwen3 dimension");
  require(c.head_dim == 128, "this backend requires head_dim 128");
  require(c.q_heads == 4 * c.kv_heads, "this backend requires 4 query heads per KV head");
  require(c.hidden % 256 == 0 && c.ffn % 256 == 0, "hidden and ffn widths must be multiples of 256");
  // Register-resident RMSNorm prologue (128 lanes x 32 features) and
  // 16-byte staging (8 chunks per lane of 256) bound the widths.
  require(c.hidden == static_cast<uint32_t>(dl::kNormWidth) && c.ffn <= 16384 &&
              uint64_t(c.q_heads) * c.head_dim <= 16384,
          "hidden must be 4096 and ffn / query widths at most 16384");
  require(uint64_t(c.q_heads) * c.head_dim % 256 == 0, "query width must be a multiple of 256");
  require(c.vocab % 4 == 0, "vocabulary must be a multiple of 4");
  require(c.rms_eps > 0.0f, "rms epsilon must be positive");
  require(c.rope_theta > 0.0 && std::isfinite(c.rope_theta), "rope theta must be positive");
}

unsigned fill_grid(uint64_t n) { return static_cast<unsigned>(std::min<uint64_t>(dl::ceil_div(n, 256), 65535)); }
}  // namespace

extern "C" {

int dl_qwen3_create(dl_device* device, dl_queue* queue, const dl_qwen3_config* config, dl_qwen3** out) {
  return guard([&] {
    require(device && config && out, "null argument");
    dl::enter(queue);
    validate_config(*config);
    auto m = std::make_unique<dl_qwen3>();
    m->device = device;
    m->cfg = *config;
    const auto& c = m->cfg;
    const uint64_t D = c.hidden, QW = uint64_t(c.q_heads) * c.head_dim, KW = uint64_t(c.kv_heads) * c.head_dim,
                   F = c.ffn, V = c.vocab;
    // P from the reference rule (projection.cu:277-318), per logical projection.
    m->p_q = dl::partials_for(D, QW);
    m->p_kv = dl::partials_for(D, KW);
    m->p_o = dl::partials_for(QW, D);
    m->p_gu = dl::partials_for(D, F);
    m->p_down = dl::partials_for(F, D);
    m->p_lm = dl::partials_for(D, V);
    require(m->p_q == 16 && m->p_kv == 32 && m->p_o == 16 && m->p_gu == 16 && m->p_down == 32 && m->p_lm == 16,
            "shape selects a partial count the fused kernels do not implement");
    m->qkv_elems = (QW + 2 * KW) * D;
    m->o_elems = D * QW;
    m->gu_elems = 2 * F * D;
    m->down_elems = D * F;
    for (uint32_t l = 0; l < c.layers; ++l) {
      m->qkv.push_back(m->alloc(m->qkv_elems));
      m->o.push_back(m->alloc(m->o_elems));
      m->gu.push_back(m->alloc(m->gu_elems));
      m->down.push_back(m->alloc(m->down_elems));
      m->input_norm.push_back(m->alloc(D));
      m->post_norm.push_back(m->alloc(D));
      m->q_norm.push_back(m->alloc(c.head_dim));
      m->k_norm.push_back(m->alloc(c.head_dim));
    }
    m->final_norm = m->alloc(D);
    m->lm_head = m->alloc(V * D);
    if (!c.tied_embeddings) m->embedding = m->alloc(V * D);
    *out = m.release();
  });
}

int dl_qwen3_destroy(dl_qwen3* model) {
  return guard([&] {
    if (!model) return;
    model->device->activate();
    (void)hipDeviceSynchronize();
    delete model;
  });
}

int dl_qwen3_resident_bytes(dl_qwen3* model, uint64_t* bytes) {
  return guard([&] {
    require(model && bytes, "null argument");
    *bytes = model->resident;
  });
}

int dl_qwen3_fill_synthetic(dl_qwen3* model, dl_queue* queue, uint64_t seed, float weight_std) {
  return guard([&] {
    require(model != nullptr, "null model");
    dl::enter(queue);
    require(weight_std > 0.0f && std::isfinite(weight_std), "weight_std must be positive");
    const auto& c = model->cfg;
    hipStream_t s = queue->stream;
    const int roles[] = {DL_ROLE_Q, DL_ROLE_K, DL_ROLE_V, DL_ROLE_O, DL_ROLE_GATE, DL_ROLE_UP, DL_ROLE_DOWN};
    for (uint32_t l = 0; l < c.layers; ++l) {
      for (int role : roles) {
        uint64_t rows, cols;
        const dl::PackedView v = model->view(role, l, &rows, &cols);
        dl::k_fill_view<<<fill_grid(rows * cols), 256, 0, s>>>(v, rows, seed, uint64_t(l) * 16 + role, weight_std);
      }
      const int norms[] = {DL_ROLE_INPUT_NORM, DL_ROLE_POST_NORM, DL_ROLE_Q_NORM, DL_ROLE_K_NORM};
      for (int role : norms) {
        uint64_t n;
        uint16_t* p = model->plain(role, l, &n);
        dl::k_fill_const<<<fill_grid(n), 256, 0, s>>>(p, n, 0x3f80);
      }
    }
    dl::k_fill_const<<<fill_grid(c.hidden), 256, 0, s>>>(model->final_norm, c.hidden, 0x3f80);
    uint64_t rows, cols;
    const dl::PackedView lm = model->view(DL_ROLE_LM_HEAD, 0, &rows, &cols);
    // The tied table is the embedding (stream of role 0); the untied head uses role 1.
    dl::k_fill_view<<<fill_grid(rows * cols), 256, 0, s>>>(lm, rows, seed,
                                                            c.tied_embeddings ? DL_ROLE_EMBEDDING : DL_ROLE_LM_HEAD,
                                                            weight_std);
    if (!c.tied_embeddings) {
      const uint64_t n = uint64_t(c.vocab) * c.hidden;
      dl::k_fill_rowmajor<<<fill_grid(n), 256, 0, s>>>(model->embedding, n, seed, DL_ROLE_EMBEDDING, weight_std);
    }
    dl::check_launch(queue, "synthetic fill");
  });
}

static int transfer_tensor(dl_qwen3* model, dl_queue* queue, int role, uint32_t layer, uint16_t* host,
                           uint64_t elements, bool write) {
  return guard([&] {
    require(model != nullptr && host != nullptr, "null argument");
    dl::enter(queue);
    const auto& c = model->cfg;
    const bool global = role == DL_ROLE_EMBEDDING || role == DL_ROLE_LM_HEAD || role == DL_ROLE_FINAL_NORM;
    require(global || layer < c.layers, "layer out of range");
    if (role == DL_ROLE_EMBEDDING && c.tied_embeddings) role = DL_ROLE_LM_HEAD;
    uint64_t n = 0;
    if (uint16_t* p = model->plain(role, layer, &n)) {
      require(elements == n, "element count does not match the parameter", DL_LENGTH_ERROR);
      dl::check_hip(hipMemcpyAsync(write ? static_cast<void*>(p) : static_cast<void*>(host),
                                   write ? static_cast<const void*>(host) : static_cast<const void*>(p), n * 2,
                                   write ? hipMemcpyHostToDevice : hipMemcpyDeviceToHost, queue->stream),
                    "tensor transfer");
      dl::check_hip(hipStreamSynchronize(queue->stream), "tensor transfer wait");
      return;
    }
    uint64_t rows, cols;
    const dl::PackedView v = model->view(role, layer, &rows, &cols);
    require(elements == rows * cols, "element count does not match the parameter", DL_LENGTH_ERROR);
    void* tmp = nullptr;
    dl::check_hip(hipMalloc(&tmp, elements * 2), "staging allocation");
    hipError_t e = hipSuccess;
    if (write) {
      e = hipMemcpyAsync(tmp, host, elements * 2, hipMemcpyHostToDevice, queue->stream);
      if (e == hipSuccess)
        dl::k_pack_view<<<fill_grid(elements), 256, 0, queue->stream>>>(v, rows, static_cast<uint16_t*>(tmp), 0,
                                                                          nullptr);
    } else {
      dl::k_pack_view<<<fill_grid(elements), 256, 0, queue->stream>>>(v, rows, nullptr, 1,
                                                                        static_cast<uint16_t*>(tmp));
      e = hipMemcpyAsync(host, tmp, elements * 2, hipMemcpyDeviceToHost, queue->stream);
    }
    const hipError_t w = hipStreamSynchronize(queue->stream);
    (void)hipFree(tmp);
    dl::check_hip(e, "tensor transfer");
    dl::check_hip(w, "tensor transfer wait");
  });
}

// Places one row-major BF16 parameter held in device memory at `src` into
// its resident form: a copy for vectors and tables, the packing kernel for
// GEMV operands.
static void place_parameter(dl_qwen3* model, hipStream_t s, int role, uint32_t layer, const uint16_t* src,
                            uint64_t elements) {
  if (role == DL_ROLE_EMBEDDING && model->cfg.tied_embeddings) role = DL_ROLE_LM_HEAD;
  uint64_t n = 0;
  if (uint16_t* p = model->plain(role, layer, &n)) {
    require(elements == n, "element count does not match the parameter", DL_LENGTH_ERROR);
    dl::check_hip(hipMemcpyAsync(p, src, n * 2, hipMemcpyDeviceToDevice, s), "parameter copy");
    return;
  }
  uint64_t rows, cols;
  const dl::PackedView v = model->view(role, layer, &rows, &cols);
  require(elements == rows * cols, "element count does not match the parameter", DL_LENGTH_ERROR);
  dl::k_pack_view<<<fill_grid(elements), 256, 0, s>>>(v, rows, const_cast<uint16_t*>(src), 0, nullptr);
  dl::check_hip(hipGetLastError(), "parameter packing");
}

namespace {
// Bounded transfer staging of a checkpoint upload: one device buffer for the
// largest tensor and two pinned host chunks that alternate, so the host copy
// out of the file mapping overlaps the previous chunk's DMA.
struct UploadStaging {
  static constexpr uint64_t kChunk = uint64_t{64} << 20;
  hipStream_t stream = nullptr;
  void* device = nullptr;
  void* host[2] = {nullptr, nullptr};
  hipEvent_t done[2] = {nullptr, nullptr};
  explicit UploadStaging(hipStream_t s, uint64_t largest) : stream(s) {
    dl::check_hip(hipMalloc(&device, std::max<uint64_t>(largest, 2)), "upload staging");
    for (int i = 0; i < 2; ++i) {
      dl::check_hip(hipHostMalloc(&host[i], kChunk, hipHostMallocDefault), "pinned upload staging");
      dl::check_hip(hipEventCreateWithFlags(&done[i], hipEventDisableTiming), "upload event");
    }
  }
  ~UploadStaging() {
    (void)hipStreamSynchronize(stream);
    for (int i = 0; i < 2; ++i) {
      if (done[i]) (void)hipEventDestroy(done[i]);
      if (host[i]) (void)hipHostFree(host[i]);
    }
    if (device) (void)hipFree(device);
  }
};

// memcpy split over a few host threads (the mapped pages fault in from the
// file as they are read).
void parallel_copy(void* dst, const void* src, uint64_t bytes) {
  constexpr uint64_t kPiece = uint64_t{8} << 20;
  const uint64_t parts = std::min<uint64_t>(8, std::max<uint64_t>(1, bytes / kPiece));
  if (parts == 1) {
    std::memcpy(dst, src, bytes);
    return;
  }
  std::vector<std::thread> threads;
  const uint64_t step = dl::ceil_div(bytes, parts);
  for (uint64_t k = 0; k < parts; ++k) {
    const uint64_t begin = k * step, end = std::min(bytes, begin + step);
    if (begin >= end) break;
    threads.emplace_back([=] {
      std::memcpy(static_cast<uint8_t*>(dst) + begin, static_cast<const uint8_t*>(src) + begin, end - begin);
    });
  }
  for (auto& t : threads) t.join();
}
}  // namespace

int dl_qwen3_load(dl_qwen3* model, dl_queue* queue, const dl_archive* archive, const char* configuration_artifact) {
  return guard([&] {
    require(model && archive && configuration_artifact, "null argument");
    dl::enter(queue);
    std::vector<dl::qwen3::Binding> bindings;
    const auto settings = dl::qwen3::bind_causal_lm(*archive, configuration_artifact, &bindings);
    const auto& c = model->cfg;
    const auto& a = settings.config;
    require(settings.weight_dtype == DL_BF16, "this backend holds BF16 weights (no type conversion)");
    require(!c.tied_embeddings, "a Qwen3 checkpoint binds an untied embedding and LM head");
    require(c.layers == a.layers && c.hidden == a.hidden && c.q_heads == a.q_heads && c.kv_heads == a.kv_heads &&
                c.head_dim == a.head_dim && c.ffn == a.ffn && c.vocab == a.vocab && c.rms_eps == a.rms_eps &&
                c.rope_theta == a.rope_theta,
            "archive configuration differs from the resident model");
    uint64_t largest = 0;
    for (const auto& b : bindings) {
      require(b.tensor->payload != nullptr || b.tensor->byte_count == 0, "archive holds no tensor payloads");
      largest = std::max(largest, b.tensor->byte_count);
    }
    hipStream_t stream = queue->stream;
    UploadStaging staging(stream, largest);
    uint64_t chunk = 0;
    for (const auto& b : bindings) {
      const uint8_t* src = b.tensor->payload;
      const uint64_t n = b.tensor->byte_count;
      for (uint64_t off = 0; off < n; off += UploadStaging::kChunk, ++chunk) {
        const uint64_t len = std::min(UploadStaging::kChunk, n - off);
        const int slot = static_cast<int>(chunk % 2);
        if (chunk >= 2) dl::check_hip(hipEventSynchronize(staging.done[slot]), "upload staging wait");
        parallel_copy(staging.host[slot], src + off, len);
        dl::check_hip(hipMemcpyAsync(static_cast<uint8_t*>(staging.device) + off, staging.host[slot], len,
                                     hipMemcpyHostToDevice, stream),
                      "parameter upload");
        dl::check_hip(hipEventRecord(staging.done[slot], stream), "upload event");
      }
      place_parameter(model, stream, b.role, b.layer, static_cast<const uint16_t*>(staging.device), n / 2);
    }
    dl::check_hip(hipStreamSynchronize(stream), "checkpoint upload");
  });
}

int dl_qwen3_write_tensor(dl_qwen3* model, dl_queue* queue, int role, uint32_t layer, const uint16_t* host,
                          uint64_t elements) {
  return transfer_tensor(model, queue, role, layer, const_cast<uint16_t*>(host), elements, true);
}

int dl_qwen3_read_tensor(dl_qwen3* model, dl_queue* queue, int role, uint32_t layer, uint16_t* host,
                         uint64_t elements) {
  return transfer_tensor(model, queue, role, layer, host, elements, false);
}

}  // extern "C"

// ===================================================================== plan
// Steps per window of the default bounded step window (at most 32 idle step
// replays, ~20 ms on Qwen3-8B, after a stop).
constexpr uint32_t kDefaultWindow = 16;

struct dl_plan {
  dl_qwen3* model = nullptr;
  dl_queue* queue = nullptr;
  uint32_t batch = 1, capacity = 0, cap = 0;  // cap: padded to 64
  // LM head workgroups (also the argmax partials per row): 256, or 192 for
  // plans of 2 to 4 rows (MI355X sweep: 20 us per batch-2 step faster).
  int head_blocks = 256;
  uint64_t compute_units = 256;  // queried at creation
  std::vector<void*> allocations;
  std::vector<uint64_t> allocation_bytes;
  dl::Control* ctl = nullptr;
  dl::Control* bench_ctl = nullptr;
  uint16_t *h = nullptr, *q_raw = nullptr, *k_raw = nullptr, *att = nullptr, *act = nullptr, *logits = nullptr;
  uint16_t *k_cache = nullptr, *v_cache = nullptr, *capture = nullptr, *override_row = nullptr;
  float *scores = nullptr, *probs = nullptr, *rope = nullptr, *steer = nullptr;
  // Hand-off words of the fused attention + O launch (zero between launches;
  // word 2 records an expired hand-off wait).
  uint32_t* attn_sync = nullptr;
  // Hand-off words of the fused QKV + attention + O launch, and its new V row.
  uint32_t* qkvo_sync = nullptr;
  uint64_t* qkvo_tagged = nullptr;
  uint64_t* partial_keys = nullptr;
  uint32_t *partial_flags = nullptr, *tokens = nullptr, *selected = nullptr, *out_tokens = nullptr;
  uint8_t* stop_mask = nullptr;
  uint32_t* cancel_host = nullptr;
  uint32_t* cancel_device = nullptr;
  // DeviceSequence event journal in pinned, host-mapped memory: per-sequence
  // publication words, the loop mirror, then kMaxBatch x capacity events.
  void* journal_host = nullptr;
  dl::Journal journal{};  // device addresses of the same memory
  dl::Publication* publication_host = nullptr;
  dl::Mirror* mirror_host = nullptr;
  dl::Event* events_host = nullptr;
  // Bounded step window: n (default kDefaultWindow) keeps at most 2n steps
  // ahead of the device and enqueues no more once the loop has stopped, so a
  // stop costs at most 2n idle step replays; 0 enqueues every step of a
  // generation at once (the loop then completes without the host).
  uint32_t window = kDefaultWindow;
  uint64_t steps_total = 0, steps_enqueued = 0;
  uint64_t cache_seq_stride = 0, cache_layer_stride = 0;
  hipGraph_t graphs[2] = {nullptr, nullptr};  // [0] long context, [1] short context
  hipGraphExec_t execs[2] = {nullptr, nullptr};
  uint64_t host_position = 0;                 // position the next enqueued step consumes
  bool eager = false;
  dl::sampling::Settings sampling{0, 0, 1.0, 1.0};  // law recorded into the step graphs
  dl::sampling::Workspace sampler{};                // per-sequence device sampler state
  // Workgroups per decode-step kernel (0: one tile per wavefront).
  // Defaults from the workgroup sweep on MI355X (grid-stride over tiles).
  uint32_t grid_override[8] = {512, 0, 0, 0, 256, 768, 512, 0};
  // The same for launches of two to four rows where the sweep differs (0:
  // as grid_override): gate/up at 2 and 4 rows streams faster from 192
  // workgroups than from one or three per compute unit (at 8 rows, one per
  // compute unit, the LDS-resident count, is faster).
  uint32_t grid_override_rows[8] = {0, 0, 0, 0, 0, 192, 0, 0};
  // Workgroups of `waves` wavefronts for `tiles` tiles of a `rows`-row
  // launch: the tuned override (or one tile per wavefront), capped at what
  // stays resident at once when the staged rows' LDS limits residency, so no
  // workgroup repeats the staging prologue in a second round.
  unsigned grid_for(int which, uint64_t tiles, size_t lds = 0, int waves = dl::kWaves, int rows = 1) const {
    const uint64_t full = dl::ceil_div(tiles, static_cast<uint64_t>(waves));
    const bool few = rows >= 2 && rows <= 4;
    const uint32_t tuned = few && grid_override_rows[which] ? grid_override_rows[which] : grid_override[which];
    uint64_t g = tuned ? tuned : full;
    if (lds > 0) {
      const uint64_t resident = std::max<uint64_t>(1, dl::kLdsPerCu / (lds + 1024));
      g = std::min<uint64_t>(g, resident * compute_units);
    }
    return static_cast<unsigned>(g < full ? g : full);
  }
  // Host mirror of settings.
  uint64_t position = 0;
  int32_t capture_layer = -1;
  int32_t steer_layer = -1;
  uint32_t steer_mask = 0;
  bool override_active = false;
  uint32_t override_mask = 0;
  uint64_t override_position = 0;
  // An installed injection replaces the override row with its BF16 output
  // (storage + 8) and gates the loop on its status word (storage + 4); the
  // storage belongs to the caller and must outlive its use.
  const uint16_t* injection_row = nullptr;
  const uint32_t* injection_status = nullptr;
  const float* injection_norm = nullptr;
  // One-row residual intervention (steering.cu:107-159) on the output of
  // block `layer` for sequence `sequence` at `position`.
  struct Intervention {
    bool active = false;
    uint32_t sequence = 0;
    int32_t layer = -1;
    uint64_t position = 0;
    float strength = 0.0f;
    float* direction = nullptr;  // [D], plan-owned copy
    uint32_t* state = nullptr;   // [status, count]
  } intervention;
  const uint16_t* override_source() const { return injection_row ? injection_row : override_row; }
  const uint32_t* intervention_state() const { return intervention.active ? intervention.state : nullptr; }
  uint32_t max_new = 0;
  // MFMA prefill: row buffers (allocated on first use for the capacity) and
  // the prompt whose positions [0, prefilled) the caches hold.
  struct Prefill {
    uint16_t *h = nullptr, *x16 = nullptr, *x32 = nullptr, *q = nullptr, *k = nullptr, *q_rot = nullptr,
             *att = nullptr, *act = nullptr;
    uint32_t rows = 0;  // allocated rows (multiple of 128)
  } pf;
  // Exact chunked prompt pass: row buffers for `rows` consecutive positions
  // of one sequence (the longest chunk a pass has needed so far, at most
  // kExactChunk) and the chunk's control.
  struct Chunk {
    uint16_t *h = nullptr, *q = nullptr, *k = nullptr, *att = nullptr, *act = nullptr, *x16 = nullptr,
             *x32 = nullptr;
    float *scores = nullptr, *probs = nullptr;
    dl::Control* ctl = nullptr;
    uint32_t rows = 0;
  } ex;
  std::vector<uint32_t> prefilled_prompt;
  uint32_t prefilled = 0;
  uint64_t start_position = 0;  // position the prepared generation starts at

  template <class T>
  T* alloc(uint64_t count) {
    void* p = nullptr;
    const hipError_t e = hipMalloc(&p, count * sizeof(T));
    if (e != hipSuccess) {
      (void)hipGetLastError();
      dl::fail(DL_LENGTH_ERROR, std::string("plan allocation failed: ") + hipGetErrorString(e));
    }
    allocations.push_back(p);
    allocation_bytes.push_back(count * sizeof(T));
    return static_cast<T*>(p);
  }
  // Frees one allocation of this plan (the stream must be idle).
  void release(void* p) {
    for (size_t i = 0; i < allocations.size(); ++i) {
      if (allocations[i] == p) {
        (void)hipFree(p);
        allocations.erase(allocations.begin() + static_cast<long>(i));
        allocation_bytes.erase(allocation_bytes.begin() + static_cast<long>(i));
        return;
      }
    }
  }
  uint64_t device_bytes() const {
    uint64_t total = 0;
    for (uint64_t b : allocation_bytes) total += b;
    return total;
  }

  ~dl_plan() {
    for (int i = 0; i < 2; ++i) {
      if (execs[i]) (void)hipGraphExecDestroy(execs[i]);
      if (graphs[i]) (void)hipGraphDestroy(graphs[i]);
    }
    for (void* p : allocations) (void)hipFree(p);
    if (cancel_host) (void)hipHostFree(cancel_host);
    if (journal_host) (void)hipHostFree(journal_host);
  }

  void record_step(hipStream_t s, bool short_context);
  void prepare_kernels();
  void capture_step();
};

namespace {

template <class K>
void allow_lds(K kernel, size_t bytes) {
  if (bytes > 64 * 1024)
    dl::check_hip(hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                                      hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(bytes)),
                  "hipFuncSetAttribute");
}

// Largest rows per launch of each GEMV kernel: the staged FP32 inputs of
// a row group must fit the 160 KiB LDS (QKV stages D twice, for P = 16 and
// P = 32; down stages F = 12288 for P = 32).  Wider batches launch several
// row groups, each streaming the weights once.
constexpr int kQkvRows = 8;   // eight rows run as a Q launch and a K/V launch
constexpr int kDownRows = 8;  // from four rows the inputs are staged in blocks
constexpr int kWideRows = 8;

size_t qkv_lds(int rows, int D, int part = dl::kQkvAll) {
  const size_t q = part == dl::kQkvKV ? 0 : dl::staged_floats(16, D);
  const size_t kv = part == dl::kQkvQ ? 0 : dl::staged_floats(32, D);
  return size_t(rows) * (q + kv) * 4;
}
size_t p16_lds(int rows, int I) { return size_t(rows) * dl::staged_floats(16, I) * 4; }
size_t p32_lds(int rows, int I) { return size_t(rows) * dl::staged_floats(32, I) * 4; }

// Calls f(row0, g, rows) over row groups: `limit` rows at a time, then the
// remaining rows as one launch of the smallest templated size g (1, 2, 4
// or 8, at most `limit`) that holds them, whose kernels read and write only
// its `rows` rows.  So every group streams the weights once: 3 rows run the
// 4-row kernels, 5 to 7 rows the 8-row kernels.
template <class F>
void for_row_groups(uint32_t batch, int limit, F&& f) {
  uint32_t row0 = 0;
  while (row0 < batch) {
    const uint32_t rest = batch - row0;
    int g = 1;
    while (static_cast<uint32_t>(g) < rest && g < limit) g *= 2;
    const uint32_t rows = rest < static_cast<uint32_t>(g) ? rest : static_cast<uint32_t>(g);
    f(row0, g, static_cast<int>(rows));
    row0 += rows;
  }
}

// Dynamic LDS above 64 KiB needs an explicit opt-in per kernel; this runs
// before stream capture begins.
void prepare_kernels_all(dl_plan* p) {
  using namespace dl;
  const auto& c = p->model->cfg;
  const int D = c.hidden, QW = c.q_heads * c.head_dim, F = c.ffn;
  allow_lds(k_attn_pv, kPvLds);
  allow_lds(k_attn_pv_block, kPbLds);
  allow_lds(k_xgemm<16, kXgQ>, xgemm_lds(16));
  allow_lds(k_xgemm<32, kXgKV>, xgemm_lds(32));
  allow_lds(k_xgemm<16, kXgResidual>, xgemm_lds(16));
  allow_lds(k_xgemm<32, kXgResidual>, xgemm_lds(32));
  allow_lds(k_xgemm<16, kXgGateUp>, xgemm_lds(16));
  allow_lds(k_qkv<1>, qkv_lds(1, D));
  allow_lds(k_qkv<2>, qkv_lds(2, D));
  allow_lds(k_qkv<4>, qkv_lds(4, D));
  allow_lds(k_qkv_roles<8, 2>, std::max(qkv_lds(8, D, kQkvQ), qkv_lds(8, D, kQkvKV)));
  allow_lds(k_residual_chunked<32, 4>, p32_lds(4, kChunkInputs));
  allow_lds(k_residual_chunked<32, 8>, p32_lds(8, kChunkInputs));
  allow_lds(k_residual<16, 1>, p16_lds(1, QW));
  allow_lds(k_residual<16, 2>, p16_lds(2, QW));
  allow_lds(k_residual<16, 4>, p16_lds(4, QW));
  allow_lds(k_residual<16, 8, 2>, p16_lds(8, QW));
  allow_lds(k_gateup<1>, p16_lds(1, D));
  allow_lds(k_gateup<2>, p16_lds(2, D));
  allow_lds(k_gateup<4>, p16_lds(4, D));
  allow_lds(k_gateup<8>, p16_lds(8, D));
  allow_lds(k_residual<32, 1>, p32_lds(1, F));
  allow_lds(k_residual<32, 2>, p32_lds(2, F));
  allow_lds(k_lm_head<1>, p16_lds(1, D));
  allow_lds(k_lm_head<2>, p16_lds(2, D));
  allow_lds(k_lm_head<4>, p16_lds(4, D));
  allow_lds(k_lm_head<8>, p16_lds(8, D));
  allow_lds(k_attn_softmax, size_t(p->cap) * sizeof(float));
  allow_lds(k_attn_softmax_rows, size_t(p->cap) * sizeof(float));
  allow_lds(k_qkv_attn_o<2>, qkv_lds(2, D));
}

// Row groups per tile for launches with one tile per wavefront (O and the
// split Q, K/V launches, 1024 tiles each): at eight rows two groups of four,
// so 256 workgroups cover the chip and each chain is half as long.
constexpr int kRowSplit(int rows, int one_tile_per_wave) { return rows == 8 && one_tile_per_wave ? 2 : 1; }

template <int G, int Part = dl::kQkvAll>
void launch_qkv(dl_plan* p, hipStream_t s, const dl::QkvArgs& a) {
  const uint64_t tiles = Part == dl::kQkvQ ? a.QW / 4 : Part == dl::kQkvKV ? a.KW : a.QW / 4 + a.KW;
  const size_t lds = qkv_lds(G, a.D, Part);
  constexpr int waves = dl::qkv_waves(G, Part);
  constexpr int split = kRowSplit(G, Part == dl::kQkvAll ? 0 : 1);
  dl::k_qkv<G, Part, split><<<p->grid_for(0, tiles * split, lds, waves), waves * 64, lds, s>>>(a);
}
// The Q and K/V parts of G rows as one launch (k_qkv_roles), each part with
// the grid launch_qkv gives it.
template <int G>
void launch_qkv_roles(dl_plan* p, hipStream_t s, const dl::QkvArgs& a) {
  constexpr int waves = dl::qkv_waves(G, dl::kQkvQ);
  constexpr int split = kRowSplit(G, 1);
  const size_t lds = std::max(qkv_lds(G, a.D, dl::kQkvQ), qkv_lds(G, a.D, dl::kQkvKV));
  // Both parts run at once, each on half the workgroups that stay resident
  // (measured at 8 rows: config 5 5140 -> 4952 us per step against a
  // resident grid per part, which runs the parts one after the other; a
  // split in proportion to the parts' weight rows, 170 + 86, 4951-4977 us).
  const uint64_t resident = std::max<uint64_t>(2, dl::kLdsPerCu / (lds + 1024) * p->compute_units);
  const uint64_t q_share = resident / 2, kv_share = resident - q_share;
  const unsigned q_blocks = static_cast<unsigned>(
      std::min<uint64_t>(q_share, p->grid_for(0, uint64_t(a.QW / 4) * split, qkv_lds(G, a.D, dl::kQkvQ), waves)));
  const unsigned kv_blocks = static_cast<unsigned>(
      std::min<uint64_t>(kv_share, p->grid_for(0, uint64_t(a.KW) * split, qkv_lds(G, a.D, dl::kQkvKV), waves)));
  dl::k_qkv_roles<G, split><<<q_blocks + kv_blocks, waves * 64, lds, s>>>(a, static_cast<int>(q_blocks));
}
template <int G>
void launch_down_chunked(dl_plan* p, hipStream_t s, const dl::ResidualArgs& a) {
  const size_t lds = p32_lds(G, dl::kChunkInputs);
  constexpr int waves = dl::gemv_waves(G);
  dl::k_residual_chunked<32, G><<<p->grid_for(6, a.D / 2, lds, waves), waves * 64, lds, s>>>(a);
}
template <int P, int G>
void launch_residual(dl_plan* p, hipStream_t s, int which, const dl::ResidualArgs& a) {
  const size_t lds = P == 16 ? p16_lds(G, a.I) : p32_lds(G, a.I);
  constexpr int split = kRowSplit(G, P == 16 ? 1 : 0);
  dl::k_residual<P, G, split><<<p->grid_for(which, a.D / (64 / P) * split, lds, dl::gemv_waves(G)),
                                dl::gemv_waves(G) * 64, lds, s>>>(a);
}

template <int G>
void launch_gateup(dl_plan* p, hipStream_t s, const dl::GateUpArgs& a) {
  dl::k_gateup<G><<<p->grid_for(5, a.F / 2, p16_lds(G, a.D), dl::gemv_waves(G), G), dl::gemv_waves(G) * 64,
                     p16_lds(G, a.D), s>>>(a);
}
template <int G>
void launch_head(dl_plan* p, hipStream_t s, const dl::HeadArgs& a) {
  dl::k_lm_head<G><<<p->head_blocks, dl::gemv_waves(G) * 64, p16_lds(G, a.D), s>>>(a);
}
// The many-row exact GEMM: grid (output blocks, row blocks).
template <int P, int EPI>
void launch_xgemm(hipStream_t s, const dl::XgemmArgs& a) {
  constexpr int tile_outputs = dl::kXgWN * (64 / P) * dl::kXgFeat;
  require(a.N % tile_outputs == 0 && a.K % dl::kXgChunk == 0 && a.B > 0, "exact GEMM shape");
  const dim3 grid(a.N / tile_outputs, (a.B + dl::kXgRows - 1) / dl::kXgRows);
  dl::k_xgemm<P, EPI><<<grid, dl::kXgThreads, dl::xgemm_lds(P), s>>>(a);
}

// The rows one step works on.  For the token loop they are the plan's
// sequences at one position; for the exact chunked prompt pass they are up
// to kMaxBatch consecutive positions of one sequence, in their own buffers.
struct StepRows {
  uint16_t *h, *q_raw, *k_raw, *att, *act;
  float *scores, *probs;
  uint32_t rows;
  uint64_t cache_base;       // element offset of row 0's sequence in the K and V caches
  uint64_t v_append_stride;  // QKV epilogue: V element offset from row r to row r + 1
  uint64_t attn_seq_stride;  // attention: cache offset from row r to row r + 1
  int pos_step;              // row r is at ctl->position + r * pos_step
  int same_sequence, sequence;
  // Normalized rows in P16 / P32 order for the many-row exact GEMM (null
  // where the step never has kXgMinRows rows).
  uint16_t *x16, *x32;
};

StepRows plan_rows(const dl_plan* p) {
  return StepRows{p->h, p->q_raw, p->k_raw, p->att, p->act, p->scores, p->probs, p->batch, 0,
                  p->cache_seq_stride, p->cache_seq_stride, 0, 0, 0};
}

// Whether step rows `r` run their projections through the many-row exact
// GEMM (its shapes: widths that are whole passes of staged inputs).
bool use_xgemm(const dl_plan* p, const StepRows& r) {
  const auto& c = p->model->cfg;
  const dl_qwen3* m = p->model;
  return r.rows >= static_cast<uint32_t>(dl::kXgMinRows) && r.x16 != nullptr && r.x32 != nullptr &&
         m->p_q == 16 && m->p_kv == 32 && m->p_o == 16 && m->p_gu == 16 && m->p_down == 32 &&
         c.hidden % dl::kXgChunk == 0 && (uint64_t(c.q_heads) * c.head_dim) % dl::kXgChunk == 0 &&
         c.ffn % dl::kXgChunk == 0;
}

// Launches one decode-step kernel `which` of layer `l` with control `ctl`
// over the rows `r` (every sequence of the plan unless given).
void launch_step_kernel(dl_plan* p, hipStream_t s, int which, uint32_t l, dl::Control* ctl, const StepRows& r) {
  using namespace dl;
  const dl_qwen3* m = p->model;
  const auto& c = m->cfg;
  const int D = c.hidden, QW = c.q_heads * c.head_dim, KW = c.kv_heads * c.head_dim, F = c.ffn;
  const uint32_t V = c.vocab, B = r.rows;
  const float scale = static_cast<float>(1.0 / std::sqrt(static_cast<double>(c.head_dim)));
  uint16_t* kc = p->k_cache + uint64_t(l) * p->cache_layer_stride + r.cache_base;
  uint16_t* vc = p->v_cache + uint64_t(l) * p->cache_layer_stride + r.cache_base;
  AttnArgs aa{ctl, r.q_raw, r.k_raw, m->q_norm[l], m->k_norm[l], p->rope, kc, vc, r.attn_seq_stride,
              r.scores, r.probs, r.att, static_cast<int>(c.q_heads), static_cast<int>(c.kv_heads),
              static_cast<int>(p->cap), c.rms_eps, scale, r.pos_step};
  const bool xg = use_xgemm(p, r);
  switch (which) {
    case 0:
      if (xg) {
        prefill::launch_norm(s, prefill::NormArgs{r.h, m->input_norm[l], r.x16, r.x32, static_cast<int>(B), D,
                                                  c.rms_eps});
        XgemmArgs qa{ctl, r.x16, reinterpret_cast<const u32x4*>(m->qkv[l]), static_cast<int>(B), QW, D, 1,
                     r.q_raw, nullptr, 0, KW, static_cast<int>(p->cap), {}};
        launch_xgemm<16, kXgQ>(s, qa);
        XgemmArgs kva{ctl, r.x32, reinterpret_cast<const u32x4*>(m->qkv[l] + uint64_t(QW) * D),
                      static_cast<int>(B), 2 * KW, D, 1, r.k_raw, vc, r.v_append_stride, KW,
                      static_cast<int>(p->cap), {}};
        launch_xgemm<32, kXgKV>(s, kva);
        break;
      }
      for_row_groups(B, kQkvRows, [&](uint32_t r0, int g, int rows) {
        QkvArgs qa{ctl, r.h + uint64_t(r0) * D, m->input_norm[l], reinterpret_cast<const u32x4*>(m->qkv[l]),
                   r.q_raw + uint64_t(r0) * QW, r.k_raw + uint64_t(r0) * KW, vc + r0 * r.v_append_stride,
                   r.v_append_stride, D, QW, KW, static_cast<int>(p->cap), c.rms_eps, rows};
        if (g == 8) {
          launch_qkv_roles<8>(p, s, qa);
        } else if (g == 4) {
          launch_qkv<4>(p, s, qa);
        } else if (g == 2) {
          launch_qkv<2>(p, s, qa);
        } else {
          launch_qkv<1>(p, s, qa);
        }
      });
      break;
    case 1:
      // Consecutive positions of one sequence (their keys appended first)
      // share each key tile over a block of rows.
      if (r.pos_step == 1 && B >= static_cast<uint32_t>(kQkRows))
        k_attn_qk_rows<<<dim3(c.kv_heads, p->cap / 64, (B + kQkRows - 1) / kQkRows), kBlock, 0, s>>>(
            aa, static_cast<int>(B));
      else
        k_attn_qk<<<dim3(c.kv_heads, p->cap / 64, B), kBlock, 0, s>>>(aa);
      break;
    case 2:
      // Several rows: one wavefront per (query head, row).
      if (B > 1)
        k_attn_softmax_rows<<<dim3(c.q_heads, B), 64, size_t(p->cap) * sizeof(float), s>>>(aa);
      else
        k_attn_softmax<<<dim3(c.q_heads, B), kSoftmaxThreads, size_t(p->cap) * sizeof(float), s>>>(aa);
      break;
    case 3:
      if (B == 1)
        k_attn_pv<<<dim3(c.kv_heads * (kHeadDim / kPvFeatures), 1), kPvThreads, kPvLds, s>>>(aa);
      else if (r.pos_step == 1 && B >= static_cast<uint32_t>(2 * kPbRows))
        k_attn_pv_block<<<dim3(c.kv_heads * (kHeadDim / kPbHalf), (B + kPbRows - 1) / kPbRows), kPwThreads, kPbLds,
                          s>>>(aa, static_cast<int>(B));
      else
        k_attn_pv_rows<<<dim3(c.kv_heads * (kHeadDim / kPwFeatures), B), kPwThreads, 0, s>>>(aa);
      break;
    case 8:
      // Up to four rows, two workgroups per query head (see kAttnSplit);
      // eight rows already fill the GPU with one.
      if (B <= 4)
        k_attn_fused<2><<<dim3(c.q_heads * 2, B), kAttnThreads, 0, s>>>(aa);
      else
        k_attn_fused<1><<<dim3(c.q_heads, B), kAttnThreads, 0, s>>>(aa);
      break;
    case 12: {
      // QKV + attention + O of one or two rows (fused_qkv_attention_o decides
      // when it applies).
      QkvArgs qa{ctl, r.h, m->input_norm[l], reinterpret_cast<const u32x4*>(m->qkv[l]), r.q_raw, r.k_raw, vc,
                 r.v_append_stride, D, QW, KW, static_cast<int>(p->cap), c.rms_eps};
      ResidualArgs oa{ctl, r.att, reinterpret_cast<const u32x4*>(m->o[l]), r.h, nullptr, nullptr, QW, D,
                      static_cast<int>(p->cap), static_cast<int>(l), 0, r.same_sequence, r.sequence};
      const int qkv_workgroups = (QW / 4 + KW) / kQkvWaves;
      const int o_workgroups = D / (64 / 16) / kOWaves;
      const int grid = qkv_workgroups + static_cast<int>(B) * c.q_heads * kAttnSplit + o_workgroups;
      const size_t lds = qkv_lds(static_cast<int>(B), D);
      const QkvAttnOArgs args{qa, aa, oa, p->qkvo_tagged, p->qkvo_sync};
      if (B == 1)
        k_qkv_attn_o<1><<<grid, kAttnThreads, lds, s>>>(args);
      else
        k_qkv_attn_o<2><<<grid, kAttnThreads, lds, s>>>(args);
      break;
    }
    case 10: {
      // Attention + O of one row (fused_attention_o decides when it applies).
      ResidualArgs oa{ctl, r.att, reinterpret_cast<const u32x4*>(m->o[l]), r.h, nullptr, nullptr, QW, D,
                      static_cast<int>(p->cap), static_cast<int>(l), 0, r.same_sequence, r.sequence};
      const int o_workgroups = D / (64 / 16) / kOWaves;
      k_attn_o<<<c.q_heads * kAttnSplit + o_workgroups, kAttnThreads, p16_lds(1, QW), s>>>(
          AttnOArgs{aa, oa, p->attn_sync});
      break;
    }
    case 9: k_append_keys<<<dim3(c.kv_heads, B), 64, 0, s>>>(aa); break;
    case 4:
      if (xg) {
        ResidualArgs oa{ctl, r.att, reinterpret_cast<const u32x4*>(m->o[l]), r.h, nullptr, nullptr, QW, D,
                        static_cast<int>(p->cap), static_cast<int>(l), 0, r.same_sequence, r.sequence};
        launch_xgemm<16, kXgResidual>(
            s, XgemmArgs{ctl, r.att, oa.w, static_cast<int>(B), D, QW, 0, nullptr, nullptr, 0, 0, 0, oa});
        break;
      }
      for_row_groups(B, kWideRows, [&](uint32_t r0, int g, int rows) {
        ResidualArgs oa{ctl, r.att, reinterpret_cast<const u32x4*>(m->o[l]), r.h, nullptr, nullptr, QW, D,
                        static_cast<int>(p->cap), static_cast<int>(l), static_cast<int>(r0), r.same_sequence,
                        r.sequence, rows};
        if (g == 8) launch_residual<16, 8>(p, s, 4, oa);
        else if (g == 4) launch_residual<16, 4>(p, s, 4, oa);
        else if (g == 2) launch_residual<16, 2>(p, s, 4, oa);
        else launch_residual<16, 1>(p, s, 4, oa);
      });
      break;
    case 5:
      if (xg) {
        prefill::launch_norm(s, prefill::NormArgs{r.h, m->post_norm[l], r.x16, nullptr, static_cast<int>(B), D,
                                                  c.rms_eps});
        // SiLU(g) * u rows go to act in P32 order, the order the down GEMM stages.
        launch_xgemm<16, kXgGateUp>(s, XgemmArgs{ctl, r.x16, reinterpret_cast<const u32x4*>(m->gu[l]),
                                                 static_cast<int>(B), 2 * F, D, 1, r.act, nullptr, 0, 0, 0, {}});
        break;
      }
      for_row_groups(B, kWideRows, [&](uint32_t r0, int g, int rows) {
        GateUpArgs ga{ctl, r.h + uint64_t(r0) * D, m->post_norm[l], reinterpret_cast<const u32x4*>(m->gu[l]),
                      r.act + uint64_t(r0) * F, D, F, c.rms_eps, rows};
        if (g == 8) launch_gateup<8>(p, s, ga);
        else if (g == 4) launch_gateup<4>(p, s, ga);
        else if (g == 2) launch_gateup<2>(p, s, ga);
        else launch_gateup<1>(p, s, ga);
      });
      break;
    case 6:
      if (xg) {
        ResidualArgs da{ctl, r.act, reinterpret_cast<const u32x4*>(m->down[l]), r.h, p->capture, p->steer, F, D,
                        static_cast<int>(p->cap), static_cast<int>(l), 0, r.same_sequence, r.sequence};
        launch_xgemm<32, kXgResidual>(
            s, XgemmArgs{ctl, r.act, da.w, static_cast<int>(B), D, F, 1, nullptr, nullptr, 0, 0, 0, da});
        break;
      }
      // Staging in blocks needs whole blocks of inputs; other widths keep
      // two-row launches.
      for_row_groups(B, F % kChunkInputs == 0 ? kDownRows : 2, [&](uint32_t r0, int g, int rows) {
        ResidualArgs da{ctl, r.act, reinterpret_cast<const u32x4*>(m->down[l]), r.h, p->capture, p->steer, F, D,
                        static_cast<int>(p->cap), static_cast<int>(l), static_cast<int>(r0), r.same_sequence,
                        r.sequence, rows};
        if (g == 8) launch_down_chunked<8>(p, s, da);
        else if (g == 4) launch_down_chunked<4>(p, s, da);
        else if (g == 2) launch_residual<32, 2>(p, s, 6, da);
        else launch_residual<32, 1>(p, s, 6, da);
      });
      break;
    case 7:
      for_row_groups(B, kWideRows, [&](uint32_t r0, int g, int rows) {
        HeadArgs ha{ctl, r.h, m->final_norm, reinterpret_cast<const u32x4*>(m->lm_head), p->logits,
                    p->partial_keys, p->partial_flags, D, V, c.rms_eps, static_cast<int>(r0), rows};
        if (g == 8) launch_head<8>(p, s, ha);
        else if (g == 4) launch_head<4>(p, s, ha);
        else if (g == 2) launch_head<2>(p, s, ha);
        else launch_head<1>(p, s, ha);
      });
      break;
    default: fail(DL_INVALID_ARGUMENT, "unknown step kernel");
  }
}

// The plan's intervention after block `l` over the rows `r` (nothing when
// no intervention is set or `l` is not its layer).  Without a control the
// rows start at `first` and the plan's capture layer applies.
void launch_intervention(dl_plan* p, hipStream_t s, uint32_t l, dl::Control* ctl, const StepRows& r,
                         uint64_t first = 0) {
  const auto& iv = p->intervention;
  if (!iv.active || static_cast<int32_t>(l) != iv.layer) return;
  dl::InterveneArgs a{ctl, r.h, iv.direction, iv.state, p->capture, first, iv.position, p->cap, r.rows,
                      p->model->cfg.hidden, iv.sequence, r.pos_step, r.same_sequence, r.sequence,
                      static_cast<int>(l), p->capture_layer, iv.strength};
  dl::k_plan_intervene<<<1, dl::nla::kThreads, 0, s>>>(a);
}

// Whether a short-context step of this plan runs attention and the O
// projection as one launch (k_attn_o): one row, and the O tile shape the
// kernel holds in registers (I = 4096 inputs at P = 16, whole workgroups of
// O tiles).
bool fused_attention_o(const dl_plan* p) {
  const auto& c = p->model->cfg;
  const int QW = c.q_heads * c.head_dim, tiles = c.hidden / (64 / 16);
  return p->batch == 1 && QW / (8 * 16) == dl::kOChunks && tiles % dl::kOWaves == 0;
}

// Whether a short-context step runs QKV, attention and O as one launch
// (k_qkv_attn_o): one or two rows, the O tile shape of k_attn_o and the QKV
// tile shapes of the batch-1 whole-tile path (hidden width
// kWholeTileInputs) in whole workgroups.
bool fused_qkv_attention_o(const dl_plan* p) {
  const auto& c = p->model->cfg;
  const int QW = c.q_heads * c.head_dim, KW = c.kv_heads * c.head_dim, tiles = c.hidden / (64 / 16);
  return (p->batch == 1 || p->batch == 2) && QW / (8 * 16) == dl::kOChunks && tiles % dl::kOWaves == 0 &&
         c.hidden == dl::kWholeTileInputs && (QW / 4 + KW) % dl::kQkvWaves == 0;
}

// Records one decode step.  `short_context` selects the fused attention
// kernel (positions below kFusedKeys) instead of the three-kernel split;
// categorical generation adds the device sampler after the LM head.
void record_step_all(dl_plan* p, hipStream_t s, bool short_context) {
  using namespace dl;
  const dl_qwen3* m = p->model;
  const auto& c = m->cfg;
  BeginArgs begin{p->ctl, p->tokens, p->selected, p->h, m->lm_head, m->embedding, p->override_source(),
                  p->cancel_device, p->injection_status, p->intervention_state(), static_cast<int>(c.hidden),
                  c.vocab, c.tied_embeddings ? 1 : 0, p->journal, static_cast<int>(p->batch)};
  k_step_begin<<<p->batch, kBlock, 0, s>>>(begin);
  const bool fused_attn = fused_attention_o(p), fused_qkv = fused_qkv_attention_o(p);
  for (uint32_t l = 0; l < c.layers; ++l) {
    if (short_context && fused_qkv) {
      launch_step_kernel(p, s, 12, l, p->ctl, plan_rows(p));
    } else if (short_context && fused_attn) {
      launch_step_kernel(p, s, 0, l, p->ctl, plan_rows(p));
      launch_step_kernel(p, s, 10, l, p->ctl, plan_rows(p));
    } else {
      launch_step_kernel(p, s, 0, l, p->ctl, plan_rows(p));
      if (short_context)
        launch_step_kernel(p, s, 8, l, p->ctl, plan_rows(p));
      else
        for (int which : {1, 2, 3}) launch_step_kernel(p, s, which, l, p->ctl, plan_rows(p));
      launch_step_kernel(p, s, 4, l, p->ctl, plan_rows(p));
    }
    launch_step_kernel(p, s, 5, l, p->ctl, plan_rows(p));
    launch_step_kernel(p, s, 6, l, p->ctl, plan_rows(p));
    launch_intervention(p, s, l, p->ctl, plan_rows(p));
  }
  launch_step_kernel(p, s, 7, 0, p->ctl, plan_rows(p));
  if (p->sampling.mode == 1) {
    sampling::RowsArgs ra{};
    ra.logits = p->logits;
    ra.row_stride = c.vocab;
    ra.n = c.vocab;
    ra.rows = static_cast<int>(p->batch);
    ra.settings = p->sampling;
    ra.ws = p->sampler;
    ra.loop_rng = 1;
    ra.loop = sampling::LoopOutput{p->ctl, p->selected, p->out_tokens, p->cap, p->stop_mask};
    sampling::launch_count(s, ra);
    sampling::launch_select(s, ra);
  }
  EndArgs ea{p->ctl, p->partial_keys, p->partial_flags, p->head_blocks, p->selected, p->out_tokens, p->cap,
             p->stop_mask, p->intervention_state(), static_cast<int>(p->batch), p->journal};
  k_step_end<<<1, kBlock, 0, s>>>(ea);
}

}  // namespace

void dl_plan::record_step(hipStream_t s, bool short_context) { record_step_all(this, s, short_context); }

void dl_plan::prepare_kernels() { prepare_kernels_all(this); }

void dl_plan::capture_step() {
  hipStream_t s = queue->stream;
  const char* env = std::getenv("DL_EAGER");
  eager = env != nullptr && env[0] == '1';
  for (int i = 0; i < 2; ++i) {
    if (execs[i]) (void)hipGraphExecDestroy(execs[i]);
    if (graphs[i]) (void)hipGraphDestroy(graphs[i]);
    execs[i] = nullptr;
    graphs[i] = nullptr;
  }
  prepare_kernels();
  if (eager) return;
  for (int i = 0; i < 2; ++i) {
    if (i == 0 && cap <= static_cast<uint32_t>(dl::kFusedKeys)) continue;  // short graph covers every position
    dl::check_hip(hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal), "begin capture");
    try {
      record_step(s, i == 1);
    } catch (...) {
      hipGraph_t g = nullptr;
      (void)hipStreamEndCapture(s, &g);
      if (g) (void)hipGraphDestroy(g);
      throw;
    }
    dl::check_hip(hipStreamEndCapture(s, &graphs[i]), "end capture");
    dl::check_hip(hipGraphInstantiate(&execs[i], graphs[i], nullptr, nullptr, 0), "graph instantiate");
  }
}

namespace {
// Graph replay per step; with DL_EAGER=1 in the environment the same
// kernels are launched directly on the stream (for profilers that cannot
// trace graph launches).
// The host tracks the position each enqueued step will consume (the device
// position advances by one per step while the loop is active) and picks the
// short-context graph below kFusedKeys.  A step launched after the loop
// stopped exits at once in either graph.
// Zeroes the intervention's status and count (a new pass over the prompt).
void reset_intervention(dl_plan* p) {
  dl::check_hip(hipMemsetAsync(p->intervention.state, 0, 8, p->queue->stream), "intervention reset");
}

void launch_steps(dl_plan* p, uint32_t steps) {
  p->steps_enqueued += steps;
  for (uint32_t i = 0; i < steps; ++i) {
    // A plan whose cache ends at or below kFusedKeys has only the short
    // graph (capture_step); its steps past the capacity find the loop
    // stopped and replay that one.  The choice depends on the capacity, not
    // on which graphs exist: eager launches capture none.
    const bool short_context = p->host_position < static_cast<uint64_t>(dl::kFusedKeys) ||
                               p->cap <= static_cast<uint32_t>(dl::kFusedKeys);
    if (p->eager)
      p->record_step(p->queue->stream, short_context);
    else
      dl::check_hip(hipGraphLaunch(p->execs[short_context ? 1 : 0], p->queue->stream), "hipGraphLaunch");
    ++p->host_position;
  }
  if (p->eager) dl::check_launch(p->queue, "decode step");
}

// Starts a loop at `position`.  The queue must be idle: the journal's host
// words are reset here, before the device writes them again.
void init_control(dl_plan* p, uint64_t position, uint32_t prompt_length, uint32_t max_new, uint32_t mode) {
  p->host_position = position;
  p->steps_enqueued = 0;
  p->steps_total = prompt_length > position ? prompt_length - position + uint64_t(max_new) : 0;
  for (int b = 0; b < dl::kMaxBatch; ++b) __atomic_store_n(&p->publication_host[b].completed, 0u, __ATOMIC_RELAXED);
  __atomic_store_n(&p->mirror_host->steps, 0u, __ATOMIC_RELAXED);
  __atomic_store_n(&p->mirror_host->active, 1u, __ATOMIC_RELEASE);
  // An injection replaces a prompt row only (executor.cpp: the embedding
  // replacement is submitted with the prompt body).
  const bool override_on = p->override_active && !(p->injection_row && p->override_position >= prompt_length);
  dl::InitArgs a{p->ctl, position, prompt_length, max_new, p->batch, mode, p->capture_layer, p->steer_layer,
                 p->steer_mask, override_on ? 1u : 0u, p->override_mask, p->override_position, p->journal,
                 p->injection_status, p->injection_norm};
  dl::k_init_control<<<1, 1, 0, p->queue->stream>>>(a);
  dl::check_launch(p->queue, "init control");
}

// Window pacing: enqueues further steps of the running generation while
// fewer than two windows are ahead of the device and the loop is live.
void pump(dl_plan* p) {
  if (!p->window || p->steps_enqueued >= p->steps_total) return;
  if (!__atomic_load_n(&p->mirror_host->active, __ATOMIC_ACQUIRE)) return;
  const uint64_t done = __atomic_load_n(&p->mirror_host->steps, __ATOMIC_ACQUIRE);
  // A window is added only while at most one is ahead, so never more than
  // two windows run past the last step the host saw.
  while (p->steps_enqueued < p->steps_total && p->steps_enqueued - std::min(done, p->steps_enqueued) <= p->window) {
    launch_steps(p, static_cast<uint32_t>(std::min<uint64_t>(p->window, p->steps_total - p->steps_enqueued)));
  }
}

// True while a windowed generation still has steps to enqueue.
bool pumping(const dl_plan* p) {
  return p->window && p->steps_enqueued < p->steps_total &&
         __atomic_load_n(&p->mirror_host->active, __ATOMIC_ACQUIRE) != 0;
}
}  // namespace

extern "C" {

int dl_plan_create(dl_qwen3* model, dl_queue* queue, uint32_t batch, uint32_t capacity, dl_plan** out) {
  return guard([&] {
    require(model && out, "null argument");
    dl::enter(queue);
    require(batch >= 1 && batch <= static_cast<uint32_t>(dl::kMaxBatch), "batch must be in [1, 8]",
            DL_LENGTH_ERROR);
    require(capacity >= 1 && capacity <= 32768, "capacity must be in [1, 32768]", DL_LENGTH_ERROR);
    auto p = std::make_unique<dl_plan>();
    p->model = model;
    p->queue = queue;
    p->batch = batch;
    p->capacity = capacity;
    p->cap = static_cast<uint32_t>(dl::ceil_div(capacity, 64) * 64);
    {
      int device = 0, cus = 0;
      dl::check_hip(hipGetDevice(&device), "current device");
      dl::check_hip(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device), "compute units");
      p->compute_units = static_cast<uint64_t>(std::max(cus, 1));
    }
    if (batch >= 2 && batch <= 4) p->head_blocks = 192;
    const auto& c = model->cfg;
    const uint64_t B = batch, D = c.hidden, QW = uint64_t(c.q_heads) * c.head_dim,
                   KW = uint64_t(c.kv_heads) * c.head_dim, F = c.ffn, V = c.vocab, L = c.layers, cap = p->cap;
    p->ctl = p->alloc<dl::Control>(1);
    p->bench_ctl = p->alloc<dl::Control>(1);
    p->h = p->alloc<uint16_t>(B * D);
    p->q_raw = p->alloc<uint16_t>(B * QW);
    p->k_raw = p->alloc<uint16_t>(B * KW);
    p->att = p->alloc<uint16_t>(B * QW);
    p->act = p->alloc<uint16_t>(B * F);
    p->logits = p->alloc<uint16_t>(B * V);
    p->cache_layer_stride = KW * cap;
    p->cache_seq_stride = L * p->cache_layer_stride;
    p->k_cache = p->alloc<uint16_t>(B * p->cache_seq_stride);
    p->v_cache = p->alloc<uint16_t>(B * p->cache_seq_stride);
    dl::check_hip(hipMemsetAsync(p->v_cache, 0, B * p->cache_seq_stride * 2, queue->stream), "cache clear");
    dl::check_hip(hipMemsetAsync(p->k_cache, 0, B * p->cache_seq_stride * 2, queue->stream), "cache clear");
    p->scores = p->alloc<float>(B * c.q_heads * cap);
    p->probs = p->alloc<float>(B * c.q_heads * cap);
    dl::check_hip(hipMemsetAsync(p->probs, 0, B * c.q_heads * cap * 4, queue->stream), "probs clear");
    p->rope = p->alloc<float>(cap * c.head_dim);
    p->attn_sync = p->alloc<uint32_t>(dl::kSyncWords);
    dl::check_hip(hipMemsetAsync(p->attn_sync, 0, dl::kSyncWords * 4, queue->stream), "hand-off clear");
    p->qkvo_sync = p->alloc<uint32_t>(dl::kQkvoSyncWords);
    dl::check_hip(hipMemsetAsync(p->qkvo_sync, 0, dl::kQkvoSyncWords * 4, queue->stream), "hand-off clear");
    p->qkvo_tagged = p->alloc<uint64_t>(B * dl::qkvo_tagged_words(QW, KW));
    dl::check_hip(hipMemsetAsync(p->qkvo_tagged, 0, B * dl::qkvo_tagged_words(QW, KW) * 8, queue->stream),
                  "hand-off clear");
    p->partial_keys = p->alloc<uint64_t>(B * 1024);
    p->partial_flags = p->alloc<uint32_t>(B * 1024);
    p->tokens = p->alloc<uint32_t>(cap);
    p->selected = p->alloc<uint32_t>(B);
    p->out_tokens = p->alloc<uint32_t>(B * cap);
    p->stop_mask = p->alloc<uint8_t>(V);
    p->override_row = p->alloc<uint16_t>(D);
    p->steer = p->alloc<float>(B * D);
    p->intervention.direction = p->alloc<float>(D);
    p->intervention.state = p->alloc<uint32_t>(2);
    dl::check_hip(hipMemsetAsync(p->intervention.state, 0, 8, queue->stream), "intervention clear");
    p->sampler = dl::sampling::carve_workspace(p->alloc<uint8_t>(dl::sampling::workspace_bytes(batch, 0)),
                                               static_cast<int>(batch), 0);
    dl::sampling::launch_clear(queue->stream, p->sampler, static_cast<int>(batch));
    dl::check_launch(queue, "sampler clear");
    dl::check_hip(hipMemsetAsync(p->stop_mask, 0, V, queue->stream), "stop mask clear");
    dl::check_hip(hipMemsetAsync(p->selected, 0, B * 4, queue->stream), "selection clear");
    dl::check_hip(hipMemsetAsync(p->tokens, 0, cap * 4, queue->stream), "token clear");
    dl::check_hip(hipHostMalloc(reinterpret_cast<void**>(&p->cancel_host), 64, hipHostMallocMapped), "cancel word");
    *p->cancel_host = 0;
    dl::check_hip(hipHostGetDevicePointer(reinterpret_cast<void**>(&p->cancel_device), p->cancel_host, 0),
                  "cancel word mapping");
    {
      // The journal: P + 2G + 3 events at most per sequence (an injection,
      // the consumed positions, one selection and one consumption per
      // token, the terminal) with P + G <= capacity.
      const uint64_t per_sequence = 2ull * p->cap + 4;
      const uint64_t head = sizeof(dl::Publication) * dl::kMaxBatch + sizeof(dl::Mirror);
      const uint64_t bytes = head + uint64_t(B) * per_sequence * sizeof(dl::Event);
      dl::check_hip(hipHostMalloc(&p->journal_host, bytes, hipHostMallocMapped | hipHostMallocCoherent), "journal");
      std::memset(p->journal_host, 0, bytes);
      void* device = nullptr;
      dl::check_hip(hipHostGetDevicePointer(&device, p->journal_host, 0), "journal mapping");
      auto* host = static_cast<uint8_t*>(p->journal_host);
      auto* dev = static_cast<uint8_t*>(device);
      p->publication_host = reinterpret_cast<dl::Publication*>(host);
      p->mirror_host = reinterpret_cast<dl::Mirror*>(host + sizeof(dl::Publication) * dl::kMaxBatch);
      p->events_host = reinterpret_cast<dl::Event*>(host + head);
      p->journal = dl::Journal{reinterpret_cast<dl::Publication*>(dev),
                               reinterpret_cast<dl::Mirror*>(dev + sizeof(dl::Publication) * dl::kMaxBatch),
                               reinterpret_cast<dl::Event*>(dev + head), static_cast<uint32_t>(per_sequence)};
    }
    dl::k_rope_table<<<fill_grid(cap * c.head_dim / 2), 256, 0, queue->stream>>>(p->rope, cap, c.head_dim,
                                                                                  c.rope_theta);
    dl::check_launch(queue, "rope table");
    // Inactive control until a forward or generation starts.
    dl::check_hip(hipMemsetAsync(p->ctl, 0, sizeof(dl::Control), queue->stream), "control clear");
    dl::check_hip(hipStreamSynchronize(queue->stream), "plan setup");
    // Capture one step into a graph.
    p->capture_step();
    *out = p.release();
  });
}

int dl_plan_bench_prepare(dl_plan* plan) {
  return guard([&] {
    require(plan != nullptr, "null plan");
    dl::enter(plan->queue);
    dl::k_bench_control<<<1, 1, 0, plan->queue->stream>>>(plan->ctl, plan->bench_ctl);
    dl::check_launch(plan->queue, "bench control");
  });
}

int dl_plan_launch_kernel(dl_plan* plan, uint32_t which, uint32_t first_layer, uint32_t count) {
  return guard([&] {
    require(plan != nullptr, "null plan");
    dl::enter(plan->queue);
    require(which <= 8 || (which == 10 && fused_attention_o(plan)) || (which == 12 && fused_qkv_attention_o(plan)),
            "unknown step kernel");
    const uint32_t L = plan->model->cfg.layers;
    require(first_layer < L, "layer out of range");
    for (uint32_t i = 0; i < count; ++i) {
      const uint32_t l = (first_layer + i) % L;
      launch_step_kernel(plan, plan->queue->stream, static_cast<int>(which), l, plan->bench_ctl, plan_rows(plan));
    }
    dl::check_launch(plan->queue, "step kernel");
  });
}

int dl_plan_set_grid(dl_plan* plan, uint32_t which, uint32_t blocks) {
  return guard([&] {
    require(plan != nullptr, "null plan");
    require(which <= 7, "unknown step kernel");
    dl::enter(plan->queue);
    if (which == 7) {
      require(blocks >= 1 && blocks <= 1024, "LM head workgroups must be in [1, 1024]");
      plan->head_blocks = static_cast<int>(blocks);
    } else {
      plan->grid_override[which] = blocks;
      plan->grid_override_rows[which] = 0;  // the value set applies at every row count
    }
    dl::check_hip(hipStreamSynchronize(plan->queue->stream), "set grid wait");
    plan->capture_step();
  });
}

int dl_plan_destroy(dl_plan* plan) {
  return guard([&] {
    if (!plan) return;
    plan->queue->device->activate();
    (void)hipStreamSynchronize(plan->queue->stream);
    delete plan;
  });
}

int dl_plan_reset(dl_plan* plan) {
  return guard([&] {
    require(plan != nullptr, "null plan");
    dl::enter(plan->queue);
    dl::check_hip(hipStreamSynchronize(plan->queue->stream), "reset wait");
    dl::check_hip(hipMemsetAsync(plan->ctl, 0, sizeof(dl::Control), plan->queue->stream), "control clear");
    *plan->cancel_host = 0;
    plan->position = 0;
    plan->host_position = 0;
    plan->prefilled = 0;
    dl::check_hip(hipStreamSynchronize(plan->queue->stream), "reset");
  });
}

int dl_plan_position(dl_plan* plan, uint64_t* position) {
  return guard([&] {
    require(plan && position, "null argument");
    dl::enter(plan->queue);
    dl::Control c;
    dl::check_hip(hipMemcpyAsync(&c, plan->ctl, sizeof c, hipMemcpyDeviceToHost, plan->queue->stream), "read control");
    dl::check_hip(hipStreamSynchronize(plan->queue->stream), "read control wait");
    *position = c.position;
  });
}

int dl_plan_forward(dl_plan* plan, const uint32_t* tokens, uint32_t rows) {
  return guard([&] {
    require(plan && tokens, "null argument");
    dl::enter(plan->queue);
    require(rows > 0, "empty forward");
    plan->prefilled = 0;
    dl::Control c;
    hipStream_t s = plan->queue->stream;
    dl::check_hip(hipMemcpyAsync(&c, plan->ctl, sizeof c, hipMemcpyDeviceToHost, s), "read control");
    dl::check_hip(hipStreamSynchronize(s), "read control wait");
    const uint64_t pos = c.position;
    require(pos + rows <= plan->capacity, "forward exceeds the cache capacity", DL_LENGTH_ERROR);
    // All sequences consume the same rows in this diagnostic path.
    dl::check_hip(hipMemcpyAsync(plan->tokens + pos, tokens, rows * 4, hipMemcpyHostToDevice, s), "token upload");
    plan->max_new = 1;
    if (pos == 0) reset_intervention(plan);
    init_control(plan, pos, static_cast<uint32_t>(pos + rows), 1, 0);
    launch_steps(plan, rows);
    dl::check_hip(hipStreamSynchronize(s), "forward");
  });
}

int dl_plan_read_logits(dl_plan* plan, uint32_t seq, uint16_t* host) {
  return guard([&] {
    require(plan && host, "null argument");
    require(seq < plan->batch, "sequence out of range");
    dl::enter(plan->queue);
    const uint64_t V = plan->model->cfg.vocab;
    dl::check_hip(hipMemcpyAsync(host, plan->logits + uint64_t(seq) * V, V * 2, hipMemcpyDeviceToHost,
                                 plan->queue->stream),
                  "read logits");
    dl::check_hip(hipStreamSynchronize(plan->queue->stream), "read logits wait");
  });
}

int dl_plan_logits_address(dl_plan* plan, uint32_t seq, void** out) {
  return guard([&] {
    require(plan && out, "null argument");
    require(seq < plan->batch, "sequence out of range");
    *out = plan->logits + uint64_t(seq) * plan->model->cfg.vocab;
  });
}

int dl_plan_set_capture(dl_plan* plan, int32_t layer) {
  return guard([&] {
    require(plan != nullptr, "null plan");
    dl::enter(plan->queue);
    require(layer < static_cast<int32_t>(plan->model->cfg.layers), "capture layer out of range");
    if (layer >= 0 && !plan->capture) {
      plan->capture = plan->alloc<uint16_t>(uint64_t(plan->batch) * plan->cap * plan->model->cfg.hidden);
      // The recorded graph holds the capture pointer: record it again.
      dl::check_hip(hipStreamSynchronize(plan->queue->stream), "capture setup");
      plan->capture_step();
    }
    // A prefilled prompt wrote no capture rows for a layer chosen after it.
    if (layer != plan->capture_layer) plan->prefilled = 0;
    plan->capture_layer = layer;
  });
}

int dl_plan_read_capture(dl_plan* plan, uint32_t seq, uint64_t first_position, uint64_t count, uint16_t* host) {
  return guard([&] {
    require(plan && host, "null argument");
    require(plan->capture != nullptr, "capture is not enabled");
    require(seq < plan->batch, "sequence out of range");
    require(count <= plan->cap && first_position <= plan->cap - count, "capture range outside the cache",
            DL_LENGTH_ERROR);
    dl::enter(plan->queue);
    const uint64_t D = plan->model->cfg.hidden;
    dl::check_hip(hipMemcpyAsync(host, plan->capture + (uint64_t(seq) * plan->cap + first_position) * D,
                                 count * D * 2, hipMemcpyDeviceToHost, plan->queue->stream),
                  "read capture");
    dl::check_hip(hipStreamSynchronize(plan->queue->stream), "read capture wait");
  });
}

int dl_plan_set_steering(dl_plan* plan, uint32_t seq, int32_t layer, const float* vector) {
  return guard([&] {
    require(plan != nullptr, "null plan");
    require(seq < plan->batch, "sequence out of range");
    dl::enter(plan->queue);
    const auto& c = plan->model->cfg;
    // A prefilled prompt's caches hold the steering state of its pass.
    plan->prefilled = 0;
    if (!vector) {
      plan->steer_mask &= ~(1u << seq);
      return;
    }
    require(layer >= 0 && layer < static_cast<int32_t>(c.layers), "steering layer out of range");
    require(plan->steer_layer < 0 || plan->steer_layer == layer || plan->steer_mask == 0,
            "all steered sequences must use one layer");
    for (uint32_t i = 0; i < c.hidden; ++i) require(std::isfinite(vector[i]), "steering vector must be finite");
    dl::check_hip(hipMemcpyAsync(plan->steer + uint64_t(seq) * c.hidden, vector, c.hidden * 4, hipMemcpyHostToDevice,
                                 plan->queue->stream),
                  "steering upload");
    dl::check_hip(hipStreamSynchronize(plan->queue->stream), "steering upload wait");
    plan->steer_layer = layer;
    plan->steer_mask |= 1u << seq;
  });
}

// Drops an installed injection; the recorded steps hold its pointers, so
// they are recorded again.
static void clear_injection(dl_plan* plan) {
  if (!plan->injection_row) return;
  plan->injection_row = nullptr;
  plan->injection_status = nullptr;
  plan->injection_norm = nullptr;
  plan->override_active = false;
  dl::check_hip(hipStreamSynchronize(plan->queue->stream), "injection clear");
  plan->capture_step();
}

int dl_plan_set_embedding_override(dl_plan* plan, uint64_t position, const uint16_t* row, uint32_t seq_mask) {
  return guard([&] {
    require(plan != nullptr, "null plan");
    dl::enter(plan->queue);
    clear_injection(plan);
    // A prefilled prompt's caches hold the embedding rows of its pass.
    plan->prefilled = 0;
    if (!row || seq_mask == 0) {
      plan->override_active = false;
      return;
    }
    require(position < plan->capacity, "override position outside the cache", DL_LENGTH_ERROR);
    dl::check_hip(hipMemcpyAsync(plan->override_row, row, plan->model->cfg.hidden * 2, hipMemcpyHostToDevice,
                                 plan->queue->stream),
                  "override upload");
    dl::check_hip(hipStreamSynchronize(plan->queue->stream), "override upload wait");
    plan->override_active = true;
    plan->override_position = position;
    plan->override_mask = seq_mask;
  });
}

int dl_plan_set_injection(dl_plan* plan, uint64_t position, const void* storage, int output_dtype,
                          uint32_t seq_mask) {
  return guard([&] {
    require(plan != nullptr, "null plan");
    dl::enter(plan->queue);
    if (!storage || seq_mask == 0) {
      clear_injection(plan);
      return;
    }
    require(output_dtype == DL_BF16, "injection type differs from the activation storage");
    require(reinterpret_cast<uintptr_t>(storage) % 4 == 0, "misaligned injection region");
    require(position < plan->capacity, "injection position outside the cache", DL_LENGTH_ERROR);
    const auto* base = static_cast<const uint8_t*>(storage);
    dl::check_hip(hipStreamSynchronize(plan->queue->stream), "injection setup");
    plan->injection_norm = reinterpret_cast<const float*>(base);
    plan->injection_status = reinterpret_cast<const uint32_t*>(base + sizeof(float));
    plan->injection_row = reinterpret_cast<const uint16_t*>(base + sizeof(float) + sizeof(uint32_t));
    plan->override_active = true;
    plan->override_position = position;
    plan->override_mask = seq_mask;
    plan->prefilled = 0;  // a prefilled prompt did not see the injection
    plan->capture_step();
  });
}

int dl_plan_set_intervention(dl_plan* plan, uint32_t seq, int32_t layer, uint64_t position, const float* direction,
                             float strength) {
  return guard([&] {
    require(plan != nullptr, "null plan");
    dl::enter(plan->queue);
    const auto& c = plan->model->cfg;
    auto& iv = plan->intervention;
    const bool was_active = iv.active;
    require(std::isfinite(strength) && strength >= 0.0f, "intervention preparation state");
    if (!direction || layer < 0 || strength == 0.0f) {
      // executor.cpp prepare_intervention: strength zero prepares nothing.
      iv.active = false;
    } else {
      require(seq < plan->batch, "sequence out of range");
      require(layer < static_cast<int32_t>(c.layers), "unsupported intervention boundary");
      require(position < plan->capacity, "intervention preparation state", DL_LENGTH_ERROR);
      require(reinterpret_cast<uintptr_t>(direction) % 4 == 0, "misaligned direction region");
      // Stream order places the copy after the kernel that wrote the direction.
      dl::check_hip(hipMemcpyAsync(iv.direction, direction, uint64_t(c.hidden) * 4, hipMemcpyDefault,
                                   plan->queue->stream),
                    "direction copy");
      iv.active = true;
      iv.sequence = seq;
      iv.layer = layer;
      iv.position = position;
      iv.strength = strength;
    }
    dl::check_hip(hipStreamSynchronize(plan->queue->stream), "intervention setup");
    reset_intervention(plan);
    plan->prefilled = 0;  // a prefilled prompt did not see the intervention
    if (iv.active || was_active) plan->capture_step();
  });
}

int dl_plan_read_intervention(dl_plan* plan, uint32_t* status, uint32_t* count) {
  return guard([&] {
    require(plan && status && count, "null argument");
    dl::enter(plan->queue);
    uint32_t state[2];
    dl::check_hip(hipMemcpyAsync(state, plan->intervention.state, sizeof state, hipMemcpyDeviceToHost,
                                 plan->queue->stream),
                  "read intervention");
    dl::check_hip(hipStreamSynchronize(plan->queue->stream), "read intervention wait");
    *status = state[0];
    *count = state[1];
  });
}

static int cache_transfer(dl_plan* plan, uint32_t seq, uint32_t layer, uint64_t first, uint64_t count,
                          uint16_t* keys, uint16_t* values, bool read) {
  return guard([&] {
    require(plan && keys && values, "null argument");
    dl::enter(plan->queue);
    const auto& c = plan->model->cfg;
    require(seq < plan->batch && layer < c.layers, "sequence or layer out of range");
    require(count > 0 && count <= plan->capacity && first <= plan->capacity - count,
            "cache rows outside the capacity", DL_LENGTH_ERROR);
    const uint64_t elements = count * c.kv_heads * c.head_dim;
    void* tk = nullptr;
    void* tv = nullptr;
    dl::check_hip(hipMalloc(&tk, elements * 2), "cache staging");
    if (hipMalloc(&tv, elements * 2) != hipSuccess) {
      (void)hipFree(tk);
      dl::fail(DL_LENGTH_ERROR, "cache staging allocation failed");
    }
    hipStream_t s = plan->queue->stream;
    const uint64_t base = seq * plan->cache_seq_stride + uint64_t(layer) * plan->cache_layer_stride;
    hipError_t e = hipSuccess;
    if (!read) {
      e = hipMemcpyAsync(tk, keys, elements * 2, hipMemcpyHostToDevice, s);
      if (e == hipSuccess) e = hipMemcpyAsync(tv, values, elements * 2, hipMemcpyHostToDevice, s);
    }
    if (e == hipSuccess)
      dl::k_cache_rows<<<fill_grid(elements), 256, 0, s>>>(plan->k_cache + base, plan->v_cache + base,
                                                           static_cast<int>(plan->cap), c.kv_heads, first, count,
                                                           static_cast<uint16_t*>(tk), static_cast<uint16_t*>(tv),
                                                           read ? 1 : 0);
    if (e == hipSuccess && read) {
      e = hipMemcpyAsync(keys, tk, elements * 2, hipMemcpyDeviceToHost, s);
      if (e == hipSuccess) e = hipMemcpyAsync(values, tv, elements * 2, hipMemcpyDeviceToHost, s);
    }
    const hipError_t w = hipStreamSynchronize(s);
    (void)hipFree(tk);
    (void)hipFree(tv);
    dl::check_hip(e, "cache transfer");
    dl::check_hip(w, "cache transfer wait");
  });
}

int dl_plan_write_cache(dl_plan* plan, uint32_t seq, uint32_t layer, uint64_t first_position, uint64_t count,
                        const uint16_t* keys, const uint16_t* values) {
  return cache_transfer(plan, seq, layer, first_position, count, const_cast<uint16_t*>(keys),
                        const_cast<uint16_t*>(values), false);
}

int dl_plan_read_cache(dl_plan* plan, uint32_t seq, uint32_t layer, uint64_t first_position, uint64_t count,
                       uint16_t* keys, uint16_t* values) {
  return cache_transfer(plan, seq, layer, first_position, count, keys, values, true);
}

int dl_plan_device_bytes(dl_plan* plan, uint64_t* bytes) {
  return guard([&] {
    require(plan && bytes, "null argument");
    *bytes = plan->device_bytes();
  });
}

int dl_plan_seek(dl_plan* plan, uint64_t position) {
  return guard([&] {
    require(plan != nullptr, "null plan");
    dl::enter(plan->queue);
    require(position < plan->capacity, "position outside the capacity", DL_LENGTH_ERROR);
    dl::k_seek<<<1, 1, 0, plan->queue->stream>>>(plan->ctl, position);
    plan->host_position = position;
    plan->prefilled = 0;
    dl::check_launch(plan->queue, "seek");
    dl::check_hip(hipStreamSynchronize(plan->queue->stream), "seek wait");
  });
}

int dl_plan_read_hidden(dl_plan* plan, uint32_t seq, uint16_t* host) {
  return guard([&] {
    require(plan && host, "null argument");
    require(seq < plan->batch, "sequence out of range");
    dl::enter(plan->queue);
    const uint64_t D = plan->model->cfg.hidden;
    dl::check_hip(hipMemcpyAsync(host, plan->h + uint64_t(seq) * D, D * 2, hipMemcpyDeviceToHost, plan->queue->stream),
                  "read hidden");
    dl::check_hip(hipStreamSynchronize(plan->queue->stream), "read hidden wait");
  });
}

int dl_plan_generate(dl_plan* plan, const uint32_t* prompt, uint32_t prompt_length, uint32_t max_new,
                     const dl_sampling* sampling, const uint64_t* seeds, const uint32_t* stop_ids,
                     uint32_t stop_count) {
  const int status =
      dl_plan_prepare_generation(plan, prompt, prompt_length, max_new, sampling, seeds, stop_ids, stop_count);
  if (status != DL_OK) return status;
  return guard([&] {
    dl::enter(plan->queue);
    if (plan->window)
      pump(plan);
    else
      launch_steps(plan, static_cast<uint32_t>(plan->steps_total));
  });
}

int dl_plan_prepare_generation(dl_plan* plan, const uint32_t* prompt, uint32_t prompt_length, uint32_t max_new,
                               const dl_sampling* sampling, const uint64_t* seeds, const uint32_t* stop_ids,
                               uint32_t stop_count) {
  return guard([&] {
    require(plan && prompt, "null argument");
    dl::enter(plan->queue);
    require(prompt_length > 0, "empty prompt");
    require(uint64_t(prompt_length) + max_new <= plan->capacity, "generation exceeds the cache capacity",
            DL_LENGTH_ERROR);
    dl::sampling::Settings law{0, 0, 1.0, 1.0};
    if (sampling) {
      require(sampling->mode == 0 || sampling->mode == 1, "invalid sampling settings");
      require(std::isfinite(sampling->temperature) && sampling->temperature > 0, "invalid sampling settings");
      require(std::isfinite(sampling->top_p) && sampling->top_p > 0 && sampling->top_p <= 1,
              "invalid sampling settings");
      if (sampling->mode == 0)
        require(sampling->temperature == 1 && sampling->top_k == 0 && sampling->top_p == 1,
                "invalid sampling settings");
      law = dl::sampling::Settings{sampling->mode, sampling->top_k, sampling->temperature, sampling->top_p};
    }
    const uint32_t mode = law.mode;
    const uint32_t V = plan->model->cfg.vocab;
    require(law.top_k <= V, "sampling shape or top-k mismatch");
    for (uint32_t i = 0; i < prompt_length; ++i) require(prompt[i] < V, "prompt id outside the vocabulary");
    for (uint32_t i = 0; i < stop_count; ++i) require(stop_ids && stop_ids[i] < V, "stop id outside the vocabulary");
    require(!plan->intervention.active || plan->intervention.position < prompt_length,
            "intervention must belong to replay prefix");
    hipStream_t s = plan->queue->stream;
    dl::check_hip(hipStreamSynchronize(s), "generate wait");
    const dl::sampling::Settings& had = plan->sampling;
    const bool recapture = had.mode != law.mode || (law.mode == 1 && (had.top_k != law.top_k ||
                                                                     had.temperature != law.temperature ||
                                                                     had.top_p != law.top_p));
    if (recapture) {
      plan->sampling = law;
      plan->capture_step();
    }
    if (mode == 1) {
      dl::sampling::Seeds sd{};
      for (uint32_t b = 0; b < plan->batch; ++b) sd.seed[b] = seeds ? seeds[b] : 0;
      dl::sampling::launch_seed(s, plan->sampler.state, static_cast<int>(plan->batch), sd);
      dl::check_launch(plan->queue, "sampler seed");
    }
    *plan->cancel_host = 0;
    dl::check_hip(hipMemcpyAsync(plan->tokens, prompt, prompt_length * 4ull, hipMemcpyHostToDevice, s), "prompt");
    dl::check_hip(hipMemsetAsync(plan->stop_mask, 0, V, s), "stop mask");
    if (stop_count) {
      std::vector<uint8_t> mask(V, 0);
      for (uint32_t i = 0; i < stop_count; ++i) mask[stop_ids[i]] = 1;
      dl::check_hip(hipMemcpyAsync(plan->stop_mask, mask.data(), V, hipMemcpyHostToDevice, s), "stop mask");
      dl::check_hip(hipStreamSynchronize(s), "stop mask wait");
    }
    plan->max_new = max_new;
    // A prompt whose leading positions were prefilled resumes after them.
    const bool resume = plan->prefilled > 0 && plan->prefilled_prompt.size() == prompt_length &&
                        std::equal(prompt, prompt + prompt_length, plan->prefilled_prompt.begin());
    plan->start_position = resume ? plan->prefilled : 0;
    if (!resume) {
      plan->prefilled = 0;
      reset_intervention(plan);
    }
    init_control(plan, plan->start_position, prompt_length, max_new, mode);
  });
}

int dl_plan_decode_steps(dl_plan* plan, uint32_t steps) {
  return guard([&] {
    require(plan != nullptr, "null plan");
    dl::enter(plan->queue);
    launch_steps(plan, steps);
  });
}

int dl_plan_collect(dl_plan* plan, uint32_t* tokens, uint32_t max_new, dl_generation_result* results) {
  return guard([&] {
    require(plan != nullptr, "null plan");
    dl::enter(plan->queue);
    hipStream_t s = plan->queue->stream;
    // A windowed generation advances while it is collected.
    while (pumping(plan)) {
      pump(plan);
      const hipError_t q = hipStreamQuery(s);
      if (q != hipSuccess && q != hipErrorNotReady) {
        plan->queue->device->poisoned = true;
        dl::check_hip(q, "generation");
      }
      if (q == hipErrorNotReady) std::this_thread::sleep_for(std::chrono::microseconds(50));
    }
    const hipError_t e = hipStreamSynchronize(s);
    if (e != hipSuccess) {
      plan->queue->device->poisoned = true;
      dl::check_hip(e, "generation");
    }
    uint32_t handoff = 0, qkvo_handoff = 0;
    dl::check_hip(hipMemcpy(&handoff, plan->attn_sync + 32 * dl::kAttnOLayout.failure, 4, hipMemcpyDeviceToHost),
                  "read hand-off word");
    dl::check_hip(hipMemcpy(&qkvo_handoff, plan->qkvo_sync + 32 * dl::kQkvoLayout.failure, 4, hipMemcpyDeviceToHost),
                  "read hand-off word");
    if (handoff != 0 || qkvo_handoff != 0) {
      plan->queue->device->poisoned = true;
      dl::fail(DL_RUNTIME_ERROR, "attention to O hand-off wait expired; the results are invalid");
    }
    dl::Control c;
    dl::check_hip(hipMemcpy(&c, plan->ctl, sizeof c, hipMemcpyDeviceToHost), "read control");
    for (uint32_t b = 0; b < plan->batch; ++b) {
      const uint32_t n = std::min(c.row_generated[b], max_new);
      if (tokens && n)
        dl::check_hip(hipMemcpy(tokens + uint64_t(b) * max_new, plan->out_tokens + uint64_t(b) * plan->cap, n * 4ull,
                                hipMemcpyDeviceToHost),
                      "read tokens");
      if (results) {
        results[b].generated = c.row_generated[b];
        results[b].reason = c.active ? 0u : c.reason;
        if (!c.active && c.reason == 0 && ((c.finished_mask >> b) & 1u)) results[b].reason = 1;
        results[b].status = c.status;
        results[b].reserved = c.active;
        results[b].position = c.position;
        // A sequence's terminal event, when published, is its outcome
        // (a sequence that stopped early ends at its own position).
        const uint32_t count = __atomic_load_n(&plan->publication_host[b].completed, __ATOMIC_ACQUIRE);
        if (count > 0) {
          const dl::Event& last = plan->events_host[uint64_t(b) * plan->journal.capacity + count - 1];
          if ((last.kind & 0xffu) == dl::kTerminal) {
            results[b].reason = last.status;
            results[b].generated = static_cast<uint32_t>(last.count);
            results[b].position = last.position;
          }
        }
      }
    }
  });
}

int dl_plan_collect_event(dl_plan* plan, uint32_t seq, uint64_t index, int wait, dl_sequence_event* event,
                          int* ready) {
  return guard([&] {
    require(plan && event && ready, "null argument");
    require(seq < plan->batch, "sequence out of range");
    require(index < plan->journal.capacity, "event outside sequence", DL_LENGTH_ERROR);
    dl::enter(plan->queue);
    *ready = 0;
    hipStream_t s = plan->queue->stream;
    const dl::Event* slot = plan->events_host + uint64_t(seq) * plan->journal.capacity + index;
    for (;;) {
      pump(plan);
      if (__atomic_load_n(&plan->publication_host[seq].completed, __ATOMIC_ACQUIRE) > index) {
        std::memcpy(event, slot, sizeof *event);
        *ready = 1;
        return;
      }
      // An idle queue with nothing left to enqueue ends the journal, and a
      // failed queue fails the wait, whether or not the caller blocks.
      const hipError_t q = hipStreamQuery(s);
      if (q == hipSuccess) {
        if (__atomic_load_n(&plan->publication_host[seq].completed, __ATOMIC_ACQUIRE) > index) continue;
        if (pumping(plan)) continue;
        dl::fail(DL_RUNTIME_ERROR, "sequence ended without event");
      }
      if (q != hipErrorNotReady) {
        plan->queue->device->poisoned = true;
        dl::check_hip(q, "generation");
      }
      if (!wait) return;
      std::this_thread::sleep_for(std::chrono::microseconds(50));
    }
  });
}

int dl_plan_event_count(dl_plan* plan, uint32_t seq, uint64_t* count) {
  return guard([&] {
    require(plan && count, "null argument");
    require(seq < plan->batch, "sequence out of range");
    *count = __atomic_load_n(&plan->publication_host[seq].completed, __ATOMIC_ACQUIRE);
  });
}

int dl_plan_set_step_window(dl_plan* plan, uint32_t steps) {
  return guard([&] {
    require(plan != nullptr, "null plan");
    // A windowed generation that still has steps to enqueue keeps its window
    // (switching to 0 would leave those steps unenqueued).
    require(!pumping(plan), "step window change while a windowed generation is live");
    plan->window = steps;
  });
}

int dl_plan_steps_enqueued(dl_plan* plan, uint64_t* steps) {
  return guard([&] {
    require(plan && steps, "null argument");
    *steps = plan->steps_enqueued;
  });
}

int dl_plan_request_stop(dl_plan* plan) {
  return guard([&] {
    require(plan != nullptr, "null plan");
    __atomic_store_n(plan->cancel_host, 1u, __ATOMIC_RELEASE);
  });
}


// True when the prompt pass differs between the plan's sequences (steering,
// an intervention or an embedding override applied to some of them, or
// capture, which writes every sequence's arena), so each sequence needs its
// own pass.
static bool sequences_differ(const dl_plan* plan) {
  const uint32_t all = (1u << plan->batch) - 1u;
  const bool override_differs =
      plan->override_active && (plan->override_mask & all) != 0 && (plan->override_mask & all) != all;
  return plan->batch > 1 &&
         (plan->steer_mask != 0 || plan->capture_layer >= 0 || override_differs || plan->intervention.active);
}

// Copies sequence 0's cached positions [0, rows) into the other sequences'
// caches (a prompt shared by every sequence).
static void copy_prefix_to_other_sequences(dl_plan* plan, uint32_t rows) {
  const auto& c = plan->model->cfg;
  const uint64_t KW = uint64_t(c.kv_heads) * c.head_dim;
  hipStream_t s = plan->queue->stream;
  for (uint32_t b = 1; b < plan->batch; ++b) {
    const uint64_t off = uint64_t(b) * plan->cache_seq_stride;
    // The cache of one sequence: for every layer, K [Hkv][cap][128] then the
    // layer's V^T [Hkv*128][cap] at the same layer offset.
    dl::check_hip(hipMemcpy2DAsync(plan->k_cache + off, uint64_t(plan->cap) * c.head_dim * 2, plan->k_cache,
                                   uint64_t(plan->cap) * c.head_dim * 2, uint64_t(rows) * c.head_dim * 2,
                                   uint64_t(c.layers) * c.kv_heads, hipMemcpyDeviceToDevice, s),
                  "prefill K copy");
    dl::check_hip(hipMemcpy2DAsync(plan->v_cache + off, uint64_t(plan->cap) * 2, plan->v_cache,
                                   uint64_t(plan->cap) * 2, uint64_t(rows) * 2, uint64_t(c.layers) * KW,
                                   hipMemcpyDeviceToDevice, s),
                  "prefill V copy");
  }
}

int dl_plan_prefill_mfma(dl_plan* plan, const uint32_t* prompt, uint32_t prompt_length) {
  return guard([&] {
    require(plan && prompt, "null argument");
    dl::enter(plan->queue);
    const dl_qwen3* m = plan->model;
    const auto& c = m->cfg;
    require(prompt_length > 0, "empty prompt");
    require(prompt_length <= plan->capacity, "prompt exceeds the cache capacity", DL_LENGTH_ERROR);
    for (uint32_t i = 0; i < prompt_length; ++i) require(prompt[i] < c.vocab, "prompt id outside the vocabulary");
    hipStream_t s = plan->queue->stream;
    dl::check_hip(hipStreamSynchronize(s), "prefill wait");
    require(!plan->intervention.active || plan->intervention.position < prompt_length,
            "intervention must belong to replay prefix");
    plan->prefilled = 0;
    plan->prefilled_prompt.assign(prompt, prompt + prompt_length);
    reset_intervention(plan);
    // The last prompt position is consumed by the exact decode step, which
    // also selects the first token.
    const uint32_t rows = prompt_length - 1;
    if (rows == 0) return;
    const uint32_t D = c.hidden, QW = c.q_heads * c.head_dim, KW = c.kv_heads * c.head_dim, F = c.ffn;
    const uint32_t M = static_cast<uint32_t>(dl::ceil_div(rows, dl::prefill::kTileM) * dl::prefill::kTileM);
    auto& pf = plan->pf;
    if (pf.rows < M) {
      const uint32_t R = static_cast<uint32_t>(dl::ceil_div(plan->capacity, dl::prefill::kTileM) * dl::prefill::kTileM);
      pf.h = plan->alloc<uint16_t>(uint64_t(R) * D);
      pf.x16 = plan->alloc<uint16_t>(uint64_t(R) * D);
      pf.x32 = plan->alloc<uint16_t>(uint64_t(R) * D);
      pf.q = plan->alloc<uint16_t>(uint64_t(R) * QW);
      pf.k = plan->alloc<uint16_t>(uint64_t(R) * KW);
      pf.q_rot = plan->alloc<uint16_t>(uint64_t(R) * QW);
      pf.att = plan->alloc<uint16_t>(uint64_t(R) * QW);
      pf.act = plan->alloc<uint16_t>(uint64_t(R) * F);
      dl::check_hip(hipMemsetAsync(pf.att, 0, uint64_t(R) * QW * 2, s), "prefill clear");
      pf.rows = R;
    }
    dl::check_hip(hipMemcpyAsync(plan->tokens, prompt, prompt_length * 4ull, hipMemcpyHostToDevice, s), "prompt");
    const float scale = static_cast<float>(1.0 / std::sqrt(static_cast<double>(c.head_dim)));
    // Sequences share the prompt: prefill each separately only when
    // steering, capture or an embedding override differs between them,
    // else copy sequence 0.
    const bool per_sequence = sequences_differ(plan);
    const uint32_t runs = per_sequence ? plan->batch : 1;
    for (uint32_t seq = 0; seq < runs; ++seq) {
      dl::PrefillEmbedArgs ea{plan->tokens, m->lm_head, m->embedding, plan->override_source(), pf.h, rows, D, 0,
                              c.tied_embeddings ? 1 : 0,
                              (plan->override_active && ((plan->override_mask >> seq) & 1u)) ? 1 : 0,
                              plan->override_position};
      dl::k_prefill_embed<<<M, dl::kBlock, 0, s>>>(ea);
      for (uint32_t l = 0; l < c.layers; ++l) {
        uint16_t* kc = plan->k_cache + uint64_t(seq) * plan->cache_seq_stride + uint64_t(l) * plan->cache_layer_stride;
        uint16_t* vc = plan->v_cache + uint64_t(seq) * plan->cache_seq_stride + uint64_t(l) * plan->cache_layer_stride;
        dl::prefill::launch_norm(s, {pf.h, m->input_norm[l], pf.x16, pf.x32, static_cast<int>(M), static_cast<int>(D),
                                     c.rms_eps});
        dl::prefill::GemmArgs g{};
        g.a = pf.x16;
        g.a_alt = pf.x32;
        g.w = m->qkv[l];
        g.w_alt = m->qkv[l] + uint64_t(QW) * D;
        g.M = static_cast<int>(M);
        g.N = static_cast<int>(QW + 2 * KW);
        g.K = static_cast<int>(D);
        g.n_split = static_cast<int>(QW);
        g.P = m->p_q;
        g.P_alt = m->p_kv;
        g.epilogue = dl::prefill::kStoreQkv;
        g.m_valid = static_cast<int>(rows);
        g.out = pf.q;
        g.out2 = pf.k;
        g.v_cache = vc;
        g.q_width = static_cast<int>(QW);
        g.kv_width = static_cast<int>(KW);
        g.cap = static_cast<int>(plan->cap);
        g.first_position = 0;
        dl::prefill::launch_gemm(s, g);
        dl::prefill::launch_heads(s, {pf.q, pf.k, m->q_norm[l], m->k_norm[l], plan->rope, pf.q_rot, kc,
                                      static_cast<int>(rows), static_cast<int>(c.q_heads),
                                      static_cast<int>(c.kv_heads), static_cast<int>(plan->cap), 0, c.rms_eps});
        dl::prefill::launch_attention(s, {pf.q_rot, kc, vc, pf.att, static_cast<int>(rows),
                                          static_cast<int>(c.q_heads), static_cast<int>(c.kv_heads),
                                          static_cast<int>(plan->cap), 0, scale});
        dl::prefill::GemmArgs o{};
        o.a = o.a_alt = pf.att;
        o.w = o.w_alt = m->o[l];
        o.M = static_cast<int>(M);
        o.N = o.n_split = static_cast<int>(D);
        o.K = static_cast<int>(QW);
        o.P = o.P_alt = m->p_o;
        o.epilogue = dl::prefill::kResidual;
        o.m_valid = static_cast<int>(rows);
        o.out = pf.h;
        dl::prefill::launch_gemm(s, o);
        dl::prefill::launch_norm(s, {pf.h, m->post_norm[l], pf.x16, nullptr, static_cast<int>(M),
                                     static_cast<int>(D), c.rms_eps});
        dl::prefill::GemmArgs gu{};
        gu.a = gu.a_alt = pf.x16;
        gu.w = gu.w_alt = m->gu[l];
        gu.M = static_cast<int>(M);
        gu.N = gu.n_split = static_cast<int>(2 * F);
        gu.K = static_cast<int>(D);
        gu.P = gu.P_alt = m->p_gu;
        gu.epilogue = dl::prefill::kGateUp;
        gu.m_valid = static_cast<int>(rows);
        gu.out = pf.act;
        dl::prefill::launch_gemm(s, gu);
        dl::prefill::GemmArgs dn{};
        dn.a = dn.a_alt = pf.act;
        dn.w = dn.w_alt = m->down[l];
        dn.M = static_cast<int>(M);
        dn.N = dn.n_split = static_cast<int>(D);
        dn.K = static_cast<int>(F);
        dn.P = dn.P_alt = m->p_down;
        dn.epilogue = dl::prefill::kResidual;
        dn.m_valid = static_cast<int>(rows);
        dn.out = pf.h;
        dl::prefill::launch_gemm(s, dn);
        const bool steer = plan->steer_layer == static_cast<int32_t>(l) && ((plan->steer_mask >> seq) & 1u);
        const bool capture = plan->capture && plan->capture_layer == static_cast<int32_t>(l);
        if (steer || capture)
          dl::k_prefill_steer_capture<<<rows, dl::kBlock, 0, s>>>(
              pf.h, steer ? plan->steer + uint64_t(seq) * D : nullptr,
              capture ? plan->capture + uint64_t(seq) * plan->cap * D : nullptr, D, 0);
        const StepRows pr{pf.h, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, rows, 0, 0, 0, 1, 1,
                          static_cast<int>(seq)};
        launch_intervention(plan, s, l, nullptr, pr, 0);
      }
      dl::check_launch(plan->queue, "prefill");
    }
    if (!per_sequence) copy_prefix_to_other_sequences(plan, rows);
    dl::check_hip(hipStreamSynchronize(s), "prefill");
    plan->prefilled = rows;
  });
}

// The exact prompt pass: positions [0, prompt_length - 1) in chunks of up to
// kExactChunk consecutive positions through the decode kernels, rows =
// positions (StepRows with pos_step 1).  Every projection row is the same FMA
// chain as a single-position step (many-row exact GEMMs from 16 rows, each
// weight read once per chunk), the chunk's keys are in the cache before its
// attention, and each row attends to keys [0, its position], so the caches
// are bit-identical to consuming the prompt one position per step.  The
// chunk's score and probability rows take rows x q_heads x capacity floats
// each: 64 KiB each per cache position at 512 rows and 32 heads, sized to
// the longest chunk a pass has needed (at most kExactChunk rows) and counted
// by dl_plan_device_bytes.
constexpr uint32_t kExactChunk = 512;

int dl_plan_prefill(dl_plan* plan, const uint32_t* prompt, uint32_t prompt_length) {
  return guard([&] {
    require(plan && prompt, "null argument");
    dl::enter(plan->queue);
    const dl_qwen3* m = plan->model;
    const auto& c = m->cfg;
    require(prompt_length > 0, "empty prompt");
    require(prompt_length <= plan->capacity, "prompt exceeds the cache capacity", DL_LENGTH_ERROR);
    for (uint32_t i = 0; i < prompt_length; ++i) require(prompt[i] < c.vocab, "prompt id outside the vocabulary");
    hipStream_t s = plan->queue->stream;
    dl::check_hip(hipStreamSynchronize(s), "prefill wait");
    require(!plan->intervention.active || plan->intervention.position < prompt_length,
            "intervention must belong to replay prefix");
    plan->prefilled = 0;
    plan->prefilled_prompt.assign(prompt, prompt + prompt_length);
    reset_intervention(plan);
    const uint32_t rows = prompt_length - 1;
    if (rows == 0) return;
    const uint64_t D = c.hidden, QW = uint64_t(c.q_heads) * c.head_dim, KW = uint64_t(c.kv_heads) * c.head_dim,
                   F = c.ffn, R = kExactChunk;
    auto& ex = plan->ex;
    const uint32_t need = std::min<uint32_t>(kExactChunk, rows);
    if (ex.rows < need) {
      for (void* old : {static_cast<void*>(ex.h), static_cast<void*>(ex.q), static_cast<void*>(ex.k),
                        static_cast<void*>(ex.att), static_cast<void*>(ex.act), static_cast<void*>(ex.x16),
                        static_cast<void*>(ex.x32), static_cast<void*>(ex.scores), static_cast<void*>(ex.probs),
                        static_cast<void*>(ex.ctl)})
        if (old) plan->release(old);
      ex = {};
      const uint64_t R = need;
      ex.h = plan->alloc<uint16_t>(R * D);
      ex.q = plan->alloc<uint16_t>(R * QW);
      ex.k = plan->alloc<uint16_t>(R * KW);
      ex.att = plan->alloc<uint16_t>(R * QW);
      ex.act = plan->alloc<uint16_t>(R * F);
      ex.x16 = plan->alloc<uint16_t>(R * D);
      ex.x32 = plan->alloc<uint16_t>(R * D);
      ex.scores = plan->alloc<float>(R * c.q_heads * plan->cap);
      ex.probs = plan->alloc<float>(R * c.q_heads * plan->cap);
      ex.ctl = plan->alloc<dl::Control>(1);
      ex.rows = need;
    }
    dl::check_hip(hipMemcpyAsync(plan->tokens, prompt, prompt_length * 4ull, hipMemcpyHostToDevice, s), "prompt");
    const bool per_sequence = sequences_differ(plan);
    const uint32_t runs = per_sequence ? plan->batch : 1;
    for (uint32_t seq = 0; seq < runs; ++seq) {
      for (uint32_t p0 = 0; p0 < rows; p0 += R) {
        const uint32_t n = std::min<uint32_t>(static_cast<uint32_t>(R), rows - p0);
        dl::k_chunk_control<<<1, 1, 0, s>>>(plan->ctl, ex.ctl, p0, plan->capture_layer, plan->steer_layer,
                                            plan->steer_mask);
        dl::PrefillEmbedArgs ea{plan->tokens, m->lm_head, m->embedding, plan->override_source(), ex.h, n,
                                static_cast<uint32_t>(D), p0, c.tied_embeddings ? 1 : 0,
                                (plan->override_active && ((plan->override_mask >> seq) & 1u)) ? 1 : 0,
                                plan->override_position};
        dl::k_prefill_embed<<<n, dl::kBlock, 0, s>>>(ea);
        const StepRows r{ex.h, ex.q, ex.k, ex.att, ex.act, ex.scores, ex.probs, n,
                         uint64_t(seq) * plan->cache_seq_stride, 1, 0, 1, 1, static_cast<int>(seq), ex.x16, ex.x32};
        // Chunks of 8 rows or more share key tiles and V rows across rows in
        // the split kernels (k_attn_qk_rows, k_attn_pv_block) at any context;
        // fewer rows run the one-kernel attention below kFusedKeys.
        const bool short_context = n < static_cast<uint32_t>(2 * dl::kPbRows) &&
                                   p0 + n <= static_cast<uint32_t>(dl::kFusedKeys);
        for (uint32_t l = 0; l < c.layers; ++l) {
          launch_step_kernel(plan, s, 0, l, ex.ctl, r);  // Q, K, V (V into the cache)
          launch_step_kernel(plan, s, 9, l, ex.ctl, r);  // rotated K into the cache
          if (short_context) {
            launch_step_kernel(plan, s, 8, l, ex.ctl, r);
          } else {
            for (int which : {1, 2, 3}) launch_step_kernel(plan, s, which, l, ex.ctl, r);
          }
          for (int which : {4, 5, 6}) launch_step_kernel(plan, s, which, l, ex.ctl, r);
          launch_intervention(plan, s, l, ex.ctl, r);
        }
      }
      dl::check_launch(plan->queue, "exact prefill");
    }
    if (!per_sequence) copy_prefix_to_other_sequences(plan, rows);
    dl::check_hip(hipStreamSynchronize(s), "exact prefill");
    plan->prefilled = rows;
  });
}


int dl_plan_read_prefill_hidden(dl_plan* plan, uint64_t first_row, uint64_t count, uint16_t* host) {
  uint64_t D = 0;
  const int status = guard([&] {
    require(plan && host, "null argument");
    D = plan->model->cfg.hidden;
    require(count <= plan->pf.rows && first_row <= plan->pf.rows - count, "no prefill rows", DL_LENGTH_ERROR);
  });
  if (status != DL_OK) return status;
  return dl_plan_read_prefill_buffer(plan, 0, first_row * D, count * D, host);
}

int dl_plan_read_prefill_buffer(dl_plan* plan, uint32_t which, uint64_t first, uint64_t count, uint16_t* host) {
  return guard([&] {
    require(plan && host, "null argument");
    dl::enter(plan->queue);
    const auto& c = plan->model->cfg;
    const uint64_t R = plan->pf.rows, D = c.hidden, QW = uint64_t(c.q_heads) * c.head_dim,
                   KW = uint64_t(c.kv_heads) * c.head_dim, F = c.ffn;
    const uint16_t* bufs[8] = {plan->pf.h, plan->pf.x16, plan->pf.x32, plan->pf.q,
                               plan->pf.k, plan->pf.q_rot, plan->pf.att, plan->pf.act};
    const uint64_t sizes[8] = {R * D, R * D, R * D, R * QW, R * KW, R * QW, R * QW, R * F};
    require(which < 8, "unknown prefill buffer");
    require(bufs[which] != nullptr && count <= sizes[which] && first <= sizes[which] - count, "no prefill rows",
            DL_LENGTH_ERROR);
    dl::check_hip(hipMemcpyAsync(host, bufs[which] + first, count * 2, hipMemcpyDeviceToHost, plan->queue->stream),
                  "read prefill buffer");
    dl::check_hip(hipStreamSynchronize(plan->queue->stream), "read prefill buffer wait");
  });
}

}  // extern "C"
