// MFMA prefill path for long prompts (BF16 MFMA projections and causal
// attention with FP32 softmax).  Results follow the reference's operator
// sequence (src/models/qwen3/model.cpp:343-409) within tolerance: the MFMA
// units accumulate in their own order, so the prefilled KV cache is not
// bit-identical to the exact decode path's.
//
// Activation layout.  The resident projection weights keep the packed
// exact-chain layout: within each block of 8P inputs a row stores input
// P*e + t at position 8t + e.  The GEMM contracts over positions, so the
// activations it reads are stored in that same "P-permuted" order and every
// MFMA operand of either side is one contiguous 16-byte load; no second copy
// of the weights exists.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace dl::prefill {

constexpr int kTileM = 128;  // rows (positions) per GEMM tile
constexpr int kTileN = 128;  // output features per GEMM tile
constexpr int kAttnRows = 64;  // query rows per attention workgroup

// Position of input k in the P-permuted order.
__host__ __device__ inline uint32_t permuted(uint32_t k, uint32_t P) {
  const uint32_t block = 8 * P;
  return (k / block) * block + (k % P) * 8 + (k % block) / P;
}

enum Epilogue : int {
  kStore = 0,     // out[m][n] = BF16(acc)
  kStoreQkv = 1,  // q | k rows, V columns straight into the transposed V cache
  kResidual = 2,  // out[m][n] = BF16(out[m][n] + BF16(acc))
  kGateUp = 3,    // interleaved gate/up columns -> SiLU(g) * u in P32 order
};

struct GemmArgs {
  const uint16_t* a;      // [M][K], P-permuted, for columns < n_split
  const uint16_t* a_alt;  // [M][K], P_alt-permuted, for columns >= n_split
  const uint16_t* w;      // packed rows [0, n_split) with P partials
  const uint16_t* w_alt;  // packed rows [n_split, N) with P_alt partials
  int M, N, K, n_split, P, P_alt;
  int epilogue;
  int m_valid;            // rows >= m_valid are padding (never stored to caches)
  uint16_t* out;          // kStore/kResidual [M][N]; kStoreQkv q [M][q_width]; kGateUp act [M][N/2]
  uint16_t* out2;         // kStoreQkv k [M][kv_width]
  uint16_t* v_cache;      // kStoreQkv: this layer's V^T [kv_width][cap]
  int q_width, kv_width, cap;
  int first_position;     // absolute position of row 0 (multiple of 4)
};

// Exact RMSNorm rows (normalization.cu:134-186) written in P16 order (x16)
// and optionally P32 order (x32).
struct NormArgs {
  const uint16_t* h;
  const uint16_t* gain;
  uint16_t* x16;
  uint16_t* x32;
  int rows, width;
  float eps;
};

// Per-head QK RMSNorm + RoPE of prefill rows (rotary.cu:84-126); rotated
// keys go to the K cache, rotated queries to q_rot [rows][q_heads*128].
struct HeadArgs {
  const uint16_t* q;      // [rows][q_heads*128]
  const uint16_t* k;      // [rows][kv_heads*128]
  const uint16_t* q_norm;
  const uint16_t* k_norm;
  const float* rope;      // [cap][64][2]
  uint16_t* q_rot;
  uint16_t* k_cache;      // this layer: [kv_heads][cap][128]
  int rows, q_heads, kv_heads, cap, first_position;
  float eps;
};

// Causal attention of prefill rows over the cached keys [0, position].  The
// kernel addresses a head's K and V^T rows with 32-bit element offsets
// (capacity x 128 < 2^31).
constexpr uint64_t kMaxAttnCapacity = uint64_t(1) << 24;
struct AttnArgs {
  const uint16_t* q_rot;    // [rows][q_heads*128]
  const uint16_t* k_cache;  // this layer: [kv_heads][cap][128]
  const uint16_t* v_cache;  // this layer: [kv_heads*128][cap]
  uint16_t* out;            // [rows][q_heads*128], P16-permuted per row
  int rows, q_heads, kv_heads, cap, first_position;
  float scale;
};

void launch_permute(hipStream_t stream, const uint16_t* x, uint16_t* out, uint64_t rows, uint32_t width,
                    uint32_t P);
void launch_gemm(hipStream_t stream, const GemmArgs& args);
void launch_norm(hipStream_t stream, const NormArgs& args);
void launch_heads(hipStream_t stream, const HeadArgs& args);
void launch_attention(hipStream_t stream, const AttnArgs& args);

}  // namespace dl::prefill
