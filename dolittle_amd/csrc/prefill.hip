// MFMA prefill kernels for gfx950: projections as BF16 GEMMs over the packed
// resident weights, exact row norms written in the GEMM's permuted input
// order, per-head QK norm + RoPE, and causal flash attention with FP32
// softmax.  The probabilities enter the PV product at full FP32 precision:
// each p is split exactly into three BF16 parts (p = hi + mid + lo) and
// every part runs through a BF16 MFMA accumulating in FP32, so no
// probability is rounded to BF16 (numerical-portability.md:8-10).
#include <algorithm>
#include <cmath>
#include <mutex>
#include <type_traits>
#include <vector>

#include "dl_device.h"
#include "dl_internal.h"
#include "heads.h"
#include "prefill.h"

namespace dl::prefill {

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef float floatx16 __attribute__((ext_vector_type(16)));

constexpr int kTK = 64;              // GEMM positions per K chunk
constexpr int kRow = kTK + 8;        // LDS row stride in BF16 (144 B staggers banks)
constexpr int kGemmThreads = 256;    // 4 waves, each a 64 x 64 quarter of the tile
constexpr int kHd = 128;
constexpr int kKeyTile = 64;
// K tile rows are 256 bytes, unpadded, with 16-byte piece p of key row r at
// p ^ key_swizzle(r % 16); V^T tile rows are 136 bytes (8-byte aligned,
// written as 8-byte halves).  Both keep the fragment reads of the attention
// kernel off shared banks (measured with the LDS bank-conflict counter on
// gfx950).
constexpr int kQRow = kHd;
constexpr int kVRow = kKeyTile + 4;
constexpr int kXcds = 8;             // XCDs per MI355X; workgroups are dealt round-robin
constexpr int kAttnThreads = 256;    // 4 waves x 16 queries

__device__ __forceinline__ bf16x8 as_bf16x8(u32x4 v) { return __builtin_bit_cast(bf16x8, v); }
__device__ __forceinline__ int key_swizzle(int r) { return ((r & 3) << 1) | (r & 8); }

// Element offset of packed position `kpos` of weight row n (P partials,
// K inputs): the row's 8P positions of block kpos / 8P are contiguous.
__device__ __forceinline__ uint64_t packed_offset(int n, int P, int K, int kpos) {
  const int RW = 64 / P, S = K / (8 * P), block = 8 * P;
  const int s = kpos / block, local = kpos % block;
  return (static_cast<uint64_t>((n / RW) * S + s) * 64 + (n % RW) * P) * 8 + local;
}

// SiluMultiply on BF16-rounded operands (elementwise.cu:62-87), two-sided
// as there, with the decode path's correctly rounded exponential, so an
// activation row equals the exact chain's whenever its gate and up inputs do:
// the activation is silu_round(gate) * up.
__device__ __forceinline__ float silu_round(float a) {
  const float e = dl_expf(a >= 0.0f ? -a : a);
  const float sigmoid = a >= 0.0f ? 1.0f / (1.0f + e) : e / (1.0f + e);
  return dl_round_bf16(a * sigmoid);
}

// silu_round of every BF16 value, by bit pattern, built once per device
// (k_silu_table): the GEMM epilogue looks its activations up instead of
// evaluating the FP64-accurate exponential per element, with the same
// values.  In a 256 x 256 gate/up tile the evaluation took ~20% of the launch.
__device__ uint16_t g_silu_table[65536];

__global__ void k_silu_table() {
  const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
  g_silu_table[i] = dl_f32_to_bf16(silu_round(dl_bf16_to_f32(static_cast<uint16_t>(i))));
}

// exp(x) for x <= 0 within about 2 ulp: 2^(x log2 e) with the product split
// into its rounded value t and its rounding error (an FMA recovers it; the
// tail of log2 e adds the rest), so exp(x) = 2^t (1 + err ln 2 + O(err^2)),
// |err| < 2^-17, and the hardware 2^t (v_exp_f32, 1 ulp) is corrected by one
// FMA.  Used for the probabilities of the MFMA pass; the exact pass uses the
// correctly rounded dl_expf.
__device__ __forceinline__ float exp_nonpositive(float x) {
  constexpr float kLog2e = 0x1.715476p+0f;          // log2(e) rounded to binary32
  constexpr float kLog2eTail = 0x1.4ae0c0p-26f;     // log2(e) - kLog2e
  constexpr float kLn2 = 0x1.62e430p-1f;
  const float t = x * kLog2e;
  const float err = __builtin_fmaf(x, kLog2e, -t) + x * kLog2eTail;
  const float p = __builtin_amdgcn_exp2f(t);
  return __builtin_fmaf(p, err * kLn2, p);
}

// ------------------------------------------------------------------ GEMM
// Output element (m, n) of a GEMM tile through the store, residual or QKV
// epilogue.
template <int EPI>
__device__ __forceinline__ void gemm_epilogue(const GemmArgs& a, int m, int n, float v) {
  if constexpr (EPI == kStore) {
    a.out[static_cast<uint64_t>(m) * a.N + n] = dl_f32_to_bf16(v);
  } else if constexpr (EPI == kResidual) {
    uint16_t* o = a.out + static_cast<uint64_t>(m) * a.N + n;
    *o = dl_f32_to_bf16(dl_bf16_to_f32(*o) + dl_round_bf16(v));
  } else if constexpr (EPI == kStoreQkv) {
    if (n < a.q_width) {
      a.out[static_cast<uint64_t>(m) * a.q_width + n] = dl_f32_to_bf16(v);
    } else if (n < a.q_width + a.kv_width) {
      a.out2[static_cast<uint64_t>(m) * a.kv_width + (n - a.q_width)] = dl_f32_to_bf16(v);
    } else if (m < a.m_valid) {
      a.v_cache[static_cast<uint64_t>(n - a.q_width - a.kv_width) * a.cap + a.first_position + m] =
          dl_f32_to_bf16(v);
    }
  }
}

// Epilogue of one wave's (32 WM) x (32 WN) block of 32x32 accumulators, rows
// from mb, columns from nb.  Lane layout of a 32x32 accumulator: column
// lane % 32, row 8 (r / 4) + 4 (lane / 32) + r % 4 for r < 16.  For the
// gate/up epilogue the four lanes of a quad hold gate 2j, gate 2j+1, up 2j,
// up 2j+1 of the same rows; the gate lanes finish rows r < 8 and the up lanes
// rows r >= 8, each taking the other operand from the lane two over, and
// per row of MFMA tiles every SiLU is looked up before any activation is
// stored (so the lookups are not ordered behind the stores).
template <int EPI, int WM, int WN>
__device__ __forceinline__ void gemm_tile_epilogue(const GemmArgs& a, const floatx16 (&acc)[WM][WN], int mb, int nb,
                                                   int lane) {
  if constexpr (EPI == kResidual) {
    // Per row of MFMA tiles, every residual value is loaded before any sum
    // is stored: the stores may alias later loads as far as the compiler
    // knows, so element by element each load would wait for a full memory
    // round trip.
#pragma unroll
    for (int i = 0; i < WM; ++i) {
      const int rows = mb + 32 * i + 4 * (lane / 32);
      uint16_t old[WN][16];
#pragma unroll
      for (int j = 0; j < WN; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r)
          old[j][r] = a.out[static_cast<uint64_t>(rows + 8 * (r / 4) + r % 4) * a.N + nb + 32 * j + lane % 32];
#pragma unroll
      for (int j = 0; j < WN; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r)
          a.out[static_cast<uint64_t>(rows + 8 * (r / 4) + r % 4) * a.N + nb + 32 * j + lane % 32] =
              dl_f32_to_bf16(dl_bf16_to_f32(old[j][r]) + dl_round_bf16(acc[i][j][r]));
    }
    return;
  }
  if constexpr (EPI == kGateUp) {
    const bool gate_lane = (lane & 3) < 2;
#pragma unroll
    for (int i = 0; i < WM; ++i) {
      const int rows = mb + 32 * i + 4 * (lane / 32);
      uint16_t silu[WN][8];
      float other[WN][8];
#pragma unroll
      for (int j = 0; j < WN; ++j) {
#pragma unroll
        for (int k = 0; k < 8; ++k) {
          const float send = gate_lane ? acc[i][j][8 + k] : acc[i][j][k];
          const float recv = __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(send), 0x4e, 0xf, 0xf, false));
          const float gate = gate_lane ? acc[i][j][k] : recv;
          other[j][k] = dl_round_bf16(gate_lane ? recv : acc[i][j][8 + k]);
          silu[j][k] = g_silu_table[dl_f32_to_bf16(gate)];
        }
      }
#pragma unroll
      for (int j = 0; j < WN; ++j) {
        const int n = nb + 32 * j + lane % 32;
        uint16_t* out = a.out + permuted(2 * (n / 4) + (lane & 1), 32);
#pragma unroll
        for (int k = 0; k < 8; ++k) {
          const int r = gate_lane ? k : 8 + k;
          const int m = rows + 8 * (r / 4) + r % 4;
          out[static_cast<uint64_t>(m) * (a.N / 2)] = dl_f32_to_bf16(dl_bf16_to_f32(silu[j][k]) * other[j][k]);
        }
      }
    }
    return;
  }
#pragma unroll
  for (int i = 0; i < WM; ++i) {
#pragma unroll
    for (int j = 0; j < WN; ++j) {
      const int n = nb + 32 * j + lane % 32;
      const int rows = mb + 32 * i + 4 * (lane / 32);
#pragma unroll
      for (int r = 0; r < 16; ++r) gemm_epilogue<EPI>(a, rows + 8 * (r / 4) + r % 4, n, acc[i][j][r]);
    }
  }
}

// C[M x N] = A[M x K] W[N x K]^T over permuted positions, 32x32x16 BF16
// MFMA.  Four waves in a 2 x 2 grid; each wave owns a 64 x (32 WN) block of
// 2 x WN MFMA tiles, so a 16-deep K step reads 2 + WN operand fragments
// from LDS for 2 WN MFMAs.  WN = 2: tile 128 x 128 in K chunks of 64;
// WN = 4: tile 128 x 256 in K chunks of 32 (two workgroups per CU still fit
// in LDS), which halves the fragment reads per MFMA of the A side.  Chunks
// are double-buffered through LDS and come through two register sets, so
// each chunk's loads are issued two chunks before they are stored.
template <int EPI, int WN>
__global__ __launch_bounds__(kGemmThreads) __attribute__((amdgpu_waves_per_eu(2))) void k_gemm(GemmArgs a) {
  constexpr int TN = 64 * WN;
  constexpr int TK = WN == 2 ? 64 : 32;
  constexpr int RS = TK + 8;                  // LDS row stride in BF16 (staggers banks)
  constexpr int PR = TK / 8;                  // 16-byte pieces per row per chunk
  constexpr int NA = kTileM * PR / kGemmThreads, NB = TN * PR / kGemmThreads, NR = NA + NB;
  __shared__ __align__(16) uint16_t As[2][kTileM * RS];
  __shared__ __align__(16) uint16_t Bs[2][TN * RS];
  const int n0 = blockIdx.x * TN, m0 = blockIdx.y * kTileM;
  const bool alt = n0 >= a.n_split;
  const uint16_t* A = alt ? a.a_alt : a.a;
  const uint16_t* W = alt ? a.w_alt : a.w;
  const int P = alt ? a.P_alt : a.P;
  const int nb = alt ? n0 - a.n_split : n0;
  const int K = a.K, chunks = K / TK;
  const int tid = threadIdx.x, wave = tid / 64, lane = tid % 64;
  const int wm = wave >> 1, wn = wave & 1;

  // Piece i = tid + 256 j of a tile covers row i / PR, positions 8 (i % PR)
  // .. + 7 of the chunk.
  const u32x4* a_src[NA];
  const uint16_t* w_row[NB];
  int a_off[NA], b_off[NB];
#pragma unroll
  for (int j = 0; j < NA; ++j) {
    const int i = tid + kGemmThreads * j, row = i / PR, col = (i % PR) * 8;
    a_src[j] = reinterpret_cast<const u32x4*>(A + static_cast<uint64_t>(m0 + row) * K + col);
    a_off[j] = row * RS + col;
  }
#pragma unroll
  for (int j = 0; j < NB; ++j) {
    const int i = tid + kGemmThreads * j, row = i / PR, col = (i % PR) * 8;
    w_row[j] = W + packed_offset(nb + row, P, K, 0) + col;
    b_off[j] = row * RS + col;
  }
  const int block = 8 * P;
  // Packed position kpos of a row: consecutive 8P-blocks of a row sit
  // 64 * 8 elements apart.
  const uint64_t block_stride = static_cast<uint64_t>(64) * 8;
  u32x4 r0[NR], r1[NR];
#define DL_GEMM_LOAD(set, c)                                                                          \
  do {                                                                                                \
    const int kp = (c) * TK;                                                                          \
    _Pragma("unroll") for (int j = 0; j < NA; ++j) set[j] = a_src[j][kp / 8];                         \
    _Pragma("unroll") for (int j = 0; j < NB; ++j) set[NA + j] =                                      \
        *reinterpret_cast<const u32x4*>(w_row[j] + (kp / block) * block_stride + (kp % block));       \
  } while (0)
#define DL_GEMM_STORE(set, buf)                                                                       \
  do {                                                                                                \
    _Pragma("unroll") for (int j = 0; j < NA; ++j) *reinterpret_cast<u32x4*>(&As[buf][a_off[j]]) = set[j]; \
    _Pragma("unroll") for (int j = 0; j < NB; ++j) *reinterpret_cast<u32x4*>(&Bs[buf][b_off[j]]) = set[NA + j]; \
  } while (0)
#define DL_GEMM_COMPUTE(buf)                                                                          \
  do {                                                                                                \
    _Pragma("unroll") for (int ks = 0; ks < TK / 16; ++ks) {                                          \
      bf16x8 af[2], bw[WN];                                                                           \
      _Pragma("unroll") for (int i = 0; i < 2; ++i) af[i] = as_bf16x8(*reinterpret_cast<const u32x4*>(   \
          &As[buf][(64 * wm + 32 * i + lane % 32) * RS + ks * 16 + 8 * (lane / 32)]));                  \
      _Pragma("unroll") for (int j = 0; j < WN; ++j) bw[j] = as_bf16x8(*reinterpret_cast<const u32x4*>(  \
          &Bs[buf][(32 * WN * wn + 32 * j + lane % 32) * RS + ks * 16 + 8 * (lane / 32)]));             \
      _Pragma("unroll") for (int i = 0; i < 2; ++i)                                                   \
      _Pragma("unroll") for (int j = 0; j < WN; ++j)                                                  \
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[i], bw[j], acc[i][j], 0, 0, 0);        \
    }                                                                                                 \
  } while (0)

  floatx16 acc[2][WN];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < WN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

  DL_GEMM_LOAD(r0, 0);
  if (chunks > 1) DL_GEMM_LOAD(r1, 1);
  DL_GEMM_STORE(r0, 0);
  __syncthreads();
  // Chunk c sits in LDS buffer c & 1 and came through register set c & 1.
  // Loads past the last chunk reload the last one (never stored).
  int c = 0;
  for (; c + 1 < chunks; c += 2) {
    DL_GEMM_LOAD(r0, min(c + 2, chunks - 1));
    DL_GEMM_COMPUTE(0);
    DL_GEMM_STORE(r1, 1);
    __syncthreads();
    DL_GEMM_LOAD(r1, min(c + 3, chunks - 1));
    DL_GEMM_COMPUTE(1);
    if (c + 2 < chunks) DL_GEMM_STORE(r0, 0);
    __syncthreads();
  }
  if (c < chunks) DL_GEMM_COMPUTE(0);
#undef DL_GEMM_LOAD
#undef DL_GEMM_STORE
#undef DL_GEMM_COMPUTE

  gemm_tile_epilogue<EPI, 2, WN>(a, acc, m0 + 64 * wm, n0 + 32 * WN * wn, lane);
}

// The 128 x 256 tile fed by direct global-to-LDS loads: each wave
// instruction moves 64 lanes x 16 bytes into 1 KB of LDS, so chunks (32
// positions) go through three LDS stages with no register staging and one
// barrier per chunk; chunk c + 2 is in flight while chunk c is multiplied.
// LDS rows are 64 bytes, unpadded; the four 16-byte pieces of row r sit at
// piece p ^ ((r / 4) & 3), which puts the 16-byte fragment reads of a 32-row
// block on distinct banks (measured with the LDS bank-conflict counter on
// gfx950).  Each stage is its own LDS object, so the explicit vmcnt waits
// below are the only ones the loads need.
constexpr int kDmaTK = 32;
constexpr int kDmaTN = 256;
constexpr int kGemmGroupM = 8;  // M tiles per group of the tile order
constexpr int kDmaLoads = (kTileM + kDmaTN) * kDmaTK / 8 / kGemmThreads;  // 16-byte loads per thread per chunk

__device__ __forceinline__ int dma_swizzle(int r) { return (r >> 2) & 3; }

// s_waitcnt immediate that waits until at most n vector-memory operations are
// outstanding (gfx9 encoding: vmcnt bits 3:0 and 15:14; expcnt and lgkmcnt
// left at their no-wait maxima).
constexpr unsigned vmcnt_wait(unsigned n) { return 0x0f70u | (n & 0xfu) | ((n >> 4) << 14); }

typedef __attribute__((address_space(3))) void lds_void;
typedef __attribute__((address_space(1))) void global_void;

template <int EPI>
__global__ __launch_bounds__(kGemmThreads) __attribute__((amdgpu_waves_per_eu(2))) void k_gemm_dma(GemmArgs a) {
  __shared__ __align__(1024) uint16_t A0[kTileM * kDmaTK], A1[kTileM * kDmaTK], A2[kTileM * kDmaTK];
  __shared__ __align__(1024) uint16_t B0[kDmaTN * kDmaTK], B1[kDmaTN * kDmaTK], B2[kDmaTN * kDmaTK];
  // Tile order.  Workgroups are dealt to the XCDs round-robin by linear id;
  // XCD x takes the x-th eighth of a grouped raster (kGemmGroupM M tiles per
  // group, walked N tile by N tile), so the ~64 workgroups resident on one
  // XCD at a time cover a compact block of tiles and share their A rows and
  // weight rows in that XCD's L2.
  const int nN = gridDim.x, nM = gridDim.y, total = nN * nM;
  const int id = blockIdx.x + blockIdx.y * nN;
  const int v = total % kXcds == 0 ? (id % kXcds) * (total / kXcds) + id / kXcds : id;
  const int group = v / (kGemmGroupM * nN), first_m = group * kGemmGroupM;
  const int gm = min(nM - first_m, kGemmGroupM), rest = v - group * kGemmGroupM * nN;
  const int n0 = (rest / gm) * kDmaTN, m0 = (first_m + rest % gm) * kTileM;
  const bool alt = n0 >= a.n_split;
  const uint16_t* A = alt ? a.a_alt : a.a;
  const uint16_t* W = alt ? a.w_alt : a.w;
  const int P = alt ? a.P_alt : a.P;
  const int nb = alt ? n0 - a.n_split : n0;
  const int K = a.K, chunks = K / kDmaTK;
  const int tid = threadIdx.x, lane = tid % 64;
  const int wave = __builtin_amdgcn_readfirstlane(tid / 64);
  const int wm = wave >> 1, wn = wave & 1;

  // Load j of this wave fills rows 16 (4 j + wave) .. + 15 of its stage
  // (j < 2: A, else B); lane L of it brings row + L / 4, physical piece L % 4.
  const int lr = lane / 4, lp = lane % 4;
  const uint16_t* src[2 + 4];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int r = 16 * (4 * j + wave) + lr;
    src[j] = A + static_cast<uint64_t>(m0 + r) * K + 8 * (lp ^ dma_swizzle(r));
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int r = 16 * (4 * j + wave) + lr;
    src[2 + j] = W + packed_offset(nb + r, P, K, 0) + 8 * (lp ^ dma_swizzle(r));
  }
  // Packed position kp of a row: 8P-blocks sit 64 x 8 elements apart.
  const int block_shift = __builtin_ctz(8 * P), block_mask = 8 * P - 1;
  auto issue = [&](int c, uint16_t* As, uint16_t* Bs) {
    const int kp = c * kDmaTK;
    const uint64_t woff = (static_cast<uint64_t>(kp >> block_shift) << 9) + (kp & block_mask);
#pragma unroll
    for (int j = 0; j < 2; ++j)
      __builtin_amdgcn_global_load_lds((const global_void*)(src[j] + kp), (lds_void*)(As + 16 * (4 * j + wave) * kDmaTK),
                                       16, 0, 0);
#pragma unroll
    for (int j = 0; j < 4; ++j)
      __builtin_amdgcn_global_load_lds((const global_void*)(src[2 + j] + woff),
                                       (lds_void*)(Bs + 16 * (4 * j + wave) * kDmaTK), 16, 0, 0);
  };

  // Fragment offsets: row base + lane % 32 (bases are multiples of 32, so
  // the swizzle depends on lane % 32 only), logical piece 2 ks + lane / 32.
  const int sw = dma_swizzle(lane % 32);
  int frag[2];
#pragma unroll
  for (int ks = 0; ks < 2; ++ks) frag[ks] = (lane % 32) * kDmaTK + 8 * ((2 * ks + lane / 32) ^ sw);

  floatx16 acc[2][4];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

  // Both 16-deep K steps' fragments are read before the first product.
  auto compute = [&](const uint16_t* As, const uint16_t* Bs) {
    bf16x8 af[2][2], bw[2][4];
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
#pragma unroll
      for (int i = 0; i < 2; ++i)
        af[ks][i] = as_bf16x8(*reinterpret_cast<const u32x4*>(&As[(64 * wm + 32 * i) * kDmaTK + frag[ks]]));
#pragma unroll
      for (int j = 0; j < 4; ++j)
        bw[ks][j] = as_bf16x8(*reinterpret_cast<const u32x4*>(&Bs[(128 * wn + 32 * j) * kDmaTK + frag[ks]]));
    }
#pragma unroll
    for (int ks = 0; ks < 2; ++ks)
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[ks][i], bw[ks][j], acc[i][j], 0, 0, 0);
  };
  // Schedule of one step: the 12 fragment reads, then the 16 products in
  // fours with the next chunk's loads (two at a time) between them.
  auto schedule = [] {
    __builtin_amdgcn_sched_group_barrier(0x100, 12, 0);  // LDS reads
#pragma unroll
    for (int t = 0; t < 3; ++t) {
      __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);  // MFMA
      __builtin_amdgcn_sched_group_barrier(0x020, 2, 0);  // global-to-LDS loads
    }
    __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);
  };

  // Step c: wait for this thread's loads of chunk c (those of chunk c + 1
  // may stay in flight), barrier (every wave's chunk c is in LDS and every
  // wave is done with chunk c - 1, whose stage chunk c + 2 reuses), issue
  // chunk c + 2, multiply chunk c.  Past the last chunk the loads repeat it
  // into the free stage, so every step issues the same number of loads and
  // waits with the same count.
  issue(0, A0, B0);
  issue(min(1, chunks - 1), A1, B1);
  int c = 0;
#define DL_DMA_STEP(Ac, Bc, An, Bn)                                      \
  do {                                                                   \
    __builtin_amdgcn_s_waitcnt(vmcnt_wait(kDmaLoads));                  \
    __builtin_amdgcn_s_barrier();                                        \
    __builtin_amdgcn_sched_barrier(0);                                   \
    issue(min(c + 2, chunks - 1), An, Bn);                               \
    compute(Ac, Bc);                                                     \
    schedule();                                                          \
    __builtin_amdgcn_sched_barrier(0);                                   \
    ++c;                                                                 \
  } while (0)
  for (; c + 3 <= chunks;) {
    DL_DMA_STEP(A0, B0, A2, B2);
    DL_DMA_STEP(A1, B1, A0, B0);
    DL_DMA_STEP(A2, B2, A1, B1);
  }
  if (c < chunks) DL_DMA_STEP(A0, B0, A2, B2);
  if (c < chunks) DL_DMA_STEP(A1, B1, A0, B0);
#undef DL_DMA_STEP
  __builtin_amdgcn_s_waitcnt(vmcnt_wait(0));  // no load outlives the wave
#undef DL_DMA_STEP
  gemm_tile_epilogue<EPI, 2, 4>(a, acc, m0 + 64 * wm, n0 + 128 * wn, lane);
}

// 256 x 256 tiles for the wide GEMMs (gate/up, O, down): eight waves of
// 64 x 128 (2 x 4 MFMA tiles, 128 FP32 accumulators per lane), two per
// SIMD, so one wave's barrier and fragment waits overlap the other's
// products (four waves of 128 x 128, one per SIMD, took 77.4 against 75.7
// ms for the 4096-id prompt, the same outputs); a 16-deep K step reads 6
// operand fragments from LDS for 8 products, and a workgroup brings 64 KB
// per 32 K positions for twice k_gemm_dma's work.  K chunks of 32
// positions go through a ring of four 32 KB LDS stages by direct
// global-to-LDS loads, three chunks ahead.  Per chunk, each wave
//   - reads the second K step's fragments (F1) of chunk c,
//   - issues chunk c + 3 into the stage chunk c - 1 left, between the
//     products of the first K step (F0, read in the previous chunk),
//   - waits for its loads of chunk c + 1 and its fragment reads, then one
//     workgroup barrier (every wave's chunk c + 1 is in LDS; every wave is
//     done reading chunk c - 1's stage before any load into it is issued),
//   - reads chunk c + 1's F0 while the products of F1 run,
// so the matrix cores see no fragment-read latency and one barrier per 32
// products.  Stage rows use k_gemm_dma's 64-byte swizzled rows.
constexpr int kBigM = 256;
constexpr int kBigStageElems = (kBigM + kDmaTN) * kDmaTK;  // A rows then W rows

// s_waitcnt immediate: at most n vector-memory operations outstanding and no
// LDS operation outstanding (lgkmcnt 0; expcnt at its no-wait maximum).
constexpr unsigned vm_lds_wait(unsigned n) { return 0x0070u | (n & 0xfu) | ((n >> 4) << 14); }

constexpr int kBigThreads = 512;
constexpr int kBigLoads = kBigStageElems / 8 / kBigThreads;  // 16-byte loads per thread per chunk: 4

struct BigFrags {
  bf16x8 a[2], b[4];
};

template <int EPI>
__global__ __launch_bounds__(kBigThreads) __attribute__((amdgpu_waves_per_eu(2))) void k_gemm_big(GemmArgs a) {
  __shared__ __align__(1024) uint16_t S0[kBigStageElems], S1[kBigStageElems], S2[kBigStageElems],
      S3[kBigStageElems];
  const int nN = gridDim.x, nM = gridDim.y, total = nN * nM;
  const int id = blockIdx.x + blockIdx.y * nN;
  const int v = total % kXcds == 0 ? (id % kXcds) * (total / kXcds) + id / kXcds : id;
  constexpr int kGroup = kGemmGroupM / 2;
  const int group = v / (kGroup * nN), first_m = group * kGroup;
  const int gm = min(nM - first_m, kGroup), rest = v - group * kGroup * nN;
  const int n0 = (rest / gm) * kDmaTN, m0 = (first_m + rest % gm) * kBigM;
  const bool alt = n0 >= a.n_split;
  const uint16_t* A = alt ? a.a_alt : a.a;
  const uint16_t* W = alt ? a.w_alt : a.w;
  const int P = alt ? a.P_alt : a.P;
  const int nb = alt ? n0 - a.n_split : n0;
  const int K = a.K, chunks = K / kDmaTK;
  const int tid = threadIdx.x, lane = tid % 64;
  const int wave = __builtin_amdgcn_readfirstlane(tid / 64);
  const int wm = wave >> 1, wn = wave & 1;
  // Load j of this wave fills stage rows 16 (8 j + wave) .. + 15 of A (j < 2)
  // or of W (j >= 2).
  const int lr = lane / 4, lp = lane % 4;
  const uint16_t* src[4];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int r = 16 * (8 * j + wave) + lr;
    src[j] = A + static_cast<uint64_t>(m0 + r) * K + 8 * (lp ^ dma_swizzle(r));
    src[2 + j] = W + packed_offset(nb + r, P, K, 0) + 8 * (lp ^ dma_swizzle(r));
  }
  const int block_shift = __builtin_ctz(8 * P), block_mask = 8 * P - 1;
  auto issue = [&](int c, uint16_t* S) {
    const int kp = c * kDmaTK;
    const uint64_t woff = (static_cast<uint64_t>(kp >> block_shift) << 9) + (kp & block_mask);
#pragma unroll
    for (int j = 0; j < 2; ++j)
      __builtin_amdgcn_global_load_lds((const global_void*)(src[j] + kp), (lds_void*)(S + 16 * (8 * j + wave) * kDmaTK),
                                       16, 0, 0);
#pragma unroll
    for (int j = 0; j < 2; ++j)
      __builtin_amdgcn_global_load_lds((const global_void*)(src[2 + j] + woff),
                                       (lds_void*)(S + (kBigM + 16 * (8 * j + wave)) * kDmaTK), 16, 0, 0);
  };
  const int sw = dma_swizzle(lane % 32);
  int frag[2];
#pragma unroll
  for (int ks = 0; ks < 2; ++ks) frag[ks] = (lane % 32) * kDmaTK + 8 * ((2 * ks + lane / 32) ^ sw);
  auto read = [&](const uint16_t* S, int ks, BigFrags& f) {
#pragma unroll
    for (int i = 0; i < 2; ++i)
      f.a[i] = as_bf16x8(*reinterpret_cast<const u32x4*>(&S[(64 * wm + 32 * i) * kDmaTK + frag[ks]]));
#pragma unroll
    for (int j = 0; j < 4; ++j)
      f.b[j] = as_bf16x8(*reinterpret_cast<const u32x4*>(&S[(kBigM + 128 * wn + 32 * j) * kDmaTK + frag[ks]]));
  };
  floatx16 acc[2][4];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;
  auto products = [&](const BigFrags& f) {
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(f.a[i], f.b[j], acc[i][j], 0, 0, 0);
  };
  auto first_schedule = [] {
#pragma unroll
    for (int t = 0; t < 3; ++t) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
      __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);  // LDS reads
    }
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);  // global-to-LDS load
    }
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
  };
  auto second_schedule = [] {
#pragma unroll
    for (int t = 0; t < 3; ++t) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x008, 5, 0);
  };
  issue(0, S0);
  issue(min(1, chunks - 1), S1);
  issue(min(2, chunks - 1), S2);
  __builtin_amdgcn_s_waitcnt(vm_lds_wait(2 * kBigLoads));
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_sched_barrier(0);
  BigFrags f0, f1;
  read(S0, 0, f0);
  int c = 0;
#define DL_BIG_STEP(Sc, Sn, Sf)                                           \
  do {                                                                     \
    read(Sc, 1, f1);                                                       \
    issue(min(c + 3, chunks - 1), Sf);                                     \
    products(f0);                                                          \
    first_schedule();                                                      \
    __builtin_amdgcn_sched_barrier(0);                                     \
    __builtin_amdgcn_s_waitcnt(vm_lds_wait(2 * kBigLoads));              \
    __builtin_amdgcn_s_barrier();                                          \
    __builtin_amdgcn_sched_barrier(0);                                     \
    read(Sn, 0, f0);                                                       \
    products(f1);                                                          \
    second_schedule();                                                     \
    __builtin_amdgcn_sched_barrier(0);                                     \
    ++c;                                                                   \
  } while (0)
  for (; c + 4 <= chunks;) {
    DL_BIG_STEP(S0, S1, S3);
    DL_BIG_STEP(S1, S2, S0);
    DL_BIG_STEP(S2, S3, S1);
    DL_BIG_STEP(S3, S0, S2);
  }
  if (c < chunks) DL_BIG_STEP(S0, S1, S3);
  if (c < chunks) DL_BIG_STEP(S1, S2, S0);
  if (c < chunks) DL_BIG_STEP(S2, S3, S1);
#undef DL_BIG_STEP
  __builtin_amdgcn_s_waitcnt(vmcnt_wait(0));  // no load outlives the wave
  gemm_tile_epilogue<EPI, 2, 4>(a, acc, m0 + 64 * wm, n0 + 128 * wn, lane);
}

// ------------------------------------------------------------- row norms
// One workgroup per row; thread i < 128 owns features i + 128k, the
// reference tree of normalization.cu:134-186, output in P16 / P32 order.
constexpr int kNormK = 32;

__global__ __launch_bounds__(256) void k_norm(NormArgs a) {
  __shared__ float scratch[40];
  const int row = blockIdx.x, tid = threadIdx.x;
  const uint16_t* h = a.h + static_cast<uint64_t>(row) * a.width;
  const int K = a.width / 128;
  float hv[kNormK], gv[kNormK];
  if (tid < 128) {
#pragma unroll
    for (int k = 0; k < kNormK; ++k) {
      const int kk = k < K ? k : 0;
      hv[k] = dl_bf16_to_f32(h[tid + 128 * kk]);
      gv[k] = dl_bf16_to_f32(a.gain[tid + 128 * kk]);
    }
    float comp = 0.0f;
#pragma unroll
    for (int k = 0; k < kNormK; ++k)
      if (k < K) comp = comp + hv[k] * hv[k];
    const float second = __shfl_down(comp, 1, 4);
    const float third = __shfl_down(comp, 2, 4);
    const float fourth = __shfl_down(comp, 3, 4);
    if ((tid & 3) == 0) scratch[tid >> 2] = ((comp + second) + third) + fourth;
  }
  __syncthreads();
  if (tid < 32) {
    float s = scratch[tid];
#pragma unroll
    for (int off = 1; off < 32; off *= 2) s = s + __shfl_down(s, off, 32);
    if (tid == 0) scratch[32] = inverse_sqrt(s * (1.0f / static_cast<float>(a.width)) + a.eps);
  }
  __syncthreads();
  if (tid < 128) {
    const float inverse = scratch[32];
    uint16_t* x16 = a.x16 + static_cast<uint64_t>(row) * a.width;
    uint16_t* x32 = a.x32 ? a.x32 + static_cast<uint64_t>(row) * a.width : nullptr;
#pragma unroll
    for (int k = 0; k < kNormK; ++k) {
      if (k < K) {
        const uint32_t col = tid + 128 * k;
        const uint16_t n = dl_f32_to_bf16(dl_round_bf16(hv[k] * inverse) * gv[k]);
        x16[permuted(col, 16)] = n;
        if (x32) x32[permuted(col, 32)] = n;
      }
    }
  }
}

// --------------------------------------------------- head norms and RoPE
// Grid (rows, q_heads + kv_heads), one wavefront per head.
__global__ __launch_bounds__(64) void k_heads(HeadArgs a) {
  __shared__ float out[kHd];
  const int row = blockIdx.x, head = blockIdx.y, lane = threadIdx.x;
  const int position = a.first_position + row;
  const float* rope_pos = a.rope + static_cast<uint64_t>(position) * kHd;
  if (head < a.q_heads) {
    const uint64_t base = static_cast<uint64_t>(row) * a.q_heads * kHd + static_cast<uint64_t>(head) * kHd;
    head_norm_rope(a.q + base, a.q_norm, rope_pos, lane, a.eps, out);
    a.q_rot[base + lane] = dl_f32_to_bf16(out[lane]);
    a.q_rot[base + lane + 64] = dl_f32_to_bf16(out[lane + 64]);
  } else {
    const int g = head - a.q_heads;
    const uint64_t base = static_cast<uint64_t>(row) * a.kv_heads * kHd + static_cast<uint64_t>(g) * kHd;
    head_norm_rope(a.k + base, a.k_norm, rope_pos, lane, a.eps, out);
    uint16_t* dst = a.k_cache + (static_cast<uint64_t>(g) * a.cap + position) * kHd;
    dst[lane] = dl_f32_to_bf16(out[lane]);
    dst[lane + 64] = dl_f32_to_bf16(out[lane + 64]);
  }
}

// ------------------------------------------------------------- attention
// One workgroup per (query tile of 64 rows, query head); 4 waves of 16
// queries each.  Workgroups are dealt to the XCDs round-robin, so the flat
// index is renumbered to give each XCD a contiguous run of query heads (one
// GQA group per XCD when there are 8 KV heads, whose keys and values then stay
// in that XCD's L2), each head's tiles heaviest (longest causal span) first.
// Scores are computed transposed, S^T = K Q^T (16x16x32 MFMA), so each lane
// owns one query: lane l holds keys 4 (l / 16) + t of every 16-key block for
// query l % 16, and O^T += V^T E^T takes the exponentials straight from
// registers.
//
// The softmax follows the reference's order (transformer-execution.md:
// 149-170, attention.cu:231-383): a first pass over the keys finds the exact
// maximum m of the query's visible scores; a second pass recomputes the same
// scores (the same products in the same order, so the same bits), forms
// e_j = exp(s_j - m) and sums them in 32 strided partials (partial j mod 32,
// ascending j), merged by the descending half tree (offsets 16, 8, 4, 2, 1).
// Partial j mod 32 of a 64-key tile is 16 (sub & 1) + 4 lg + t, so lane group
// lg keeps partials 4 lg + t and 16 + 4 lg + t; the tree's first step is in
// the lane, the next two across lane groups (xor 32, then xor 16), the last
// two in the lane again.  In the PV product the 32 keys of a K step are taken
// in the order the lane holds them (keys 4g..4g+3 of two 16-key blocks for
// lane group g) on both operands, each e is split exactly into three BF16
// parts, and the output is (sum e v) / l: the one division per feature takes
// the place of the reference's per-key p = e / l, since the MFMA sum has its
// own order anyway.
__global__ __launch_bounds__(kAttnThreads) __attribute__((amdgpu_waves_per_eu(2))) void k_attention(AttnArgs a) {
  __shared__ __align__(16) uint16_t Ks[kKeyTile * kQRow];
  __shared__ __align__(16) uint16_t Vs[kHd * kVRow];
  const int tiles = (a.rows + kAttnRows - 1) / kAttnRows;
  const int total = tiles * a.q_heads;
  int item = blockIdx.x;
  if (total % kXcds == 0) item = (item % kXcds) * (total / kXcds) + item / kXcds;
  const int h = item / tiles, g = h / (a.q_heads / a.kv_heads);
  const int q0 = (tiles - 1 - item % tiles) * kAttnRows;
  const int tid = threadIdx.x, wave = tid / 64, lane = tid % 64;
  const int lg = lane / 16, lq = lane % 16;
  const uint64_t qw = static_cast<uint64_t>(a.q_heads) * kHd;
  // Physical piece of the lane's K fragment in step ks: (4 ks + lg) ^
  // key_swizzle(lq), with 4 ks and lg on disjoint bits.
  const int kpiece = lg ^ key_swizzle(lq);

  // The lane's B operand of S^T = K Q^T: query row 16 wave + lq, features
  // 32 ks + 8 lg .. +7.
  bf16x8 qb[kHd / 32];
  {
    const int row = q0 + 16 * wave + lq;
    const uint16_t* src = a.q_rot + static_cast<uint64_t>(min(row, a.rows - 1)) * qw + h * kHd + 8 * lg;
#pragma unroll
    for (int ks = 0; ks < kHd / 32; ++ks) {
      const u32x4 v = *reinterpret_cast<const u32x4*>(src + 32 * ks);
      qb[ks] = as_bf16x8(row < a.rows ? v : u32x4{0u, 0u, 0u, 0u});
    }
  }
  const uint16_t* kc = a.k_cache + static_cast<uint64_t>(g) * a.cap * kHd;
  const uint16_t* vc = a.v_cache + static_cast<uint64_t>(g) * kHd * a.cap;

  // This lane's query; o[d] holds O^T rows 16 d + 4 lg + t (features) for it.
  const int qrow = 16 * wave + lq;
  const int qpos = a.first_position + q0 + qrow;
  const int wave_first = a.first_position + q0 + 16 * wave;
  floatx4 o[8];
#pragma unroll
  for (int d = 0; d < 8; ++d) o[d] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};

  const int last_row = min(q0 + kAttnRows, a.rows) - 1;
  const int key_end = a.first_position + last_row + 1;
  // K (and in the second pass V) tiles go through registers: the next
  // tile's loads are issued before this tile's products and stored to LDS
  // once every wave is done with this tile.  Two workgroups share a CU (the
  // second pass holds 178 VGPRs; at three waves per SIMD it spilled).
  u32x4 kr[4], vr[4];
  auto load_keys = [&](int kt0) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int i = tid + kAttnThreads * j;
      const int key = i / 16, col = (i % 16) * 8;
      const int kk = min(kt0 + key, a.cap - 1);
      kr[j] = *reinterpret_cast<const u32x4*>(kc + (kk * kHd + col));  // offsets fit 32 bits
    }
  };
  auto load_values = [&](int kt0) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int i = tid + kAttnThreads * j;
      const int d = i / 8, vcol = (i % 8) * 8;
      vr[j] = *reinterpret_cast<const u32x4*>(vc + (d * a.cap + min(kt0 + vcol, a.cap - 8)));
    }
  };
  auto store_keys = [&] {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int i = tid + kAttnThreads * j;
      const int key = i / 16, col = (i % 16) * 8;
      *reinterpret_cast<u32x4*>(&Ks[key * kQRow + 8 * ((col / 8) ^ key_swizzle(key % 16))]) = kr[j];
    }
  };
  auto store_values = [&](int kt0) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int i = tid + kAttnThreads * j;
      const int d = i / 8, vcol = (i % 8) * 8;
      u32x4 vv = vr[j];
      // Keys at or past key_end are masked for every query of this tile
      // (e = 0); zero them so stale cache contents cannot turn 0 * v into NaN.
      const int left = key_end - (kt0 + vcol);
      if (left < 8) {
        uint32_t w[4] = {vv.x, vv.y, vv.z, vv.w};
#pragma unroll
        for (int e = 0; e < 8; ++e)
          if (e >= left) w[e / 2] &= (e & 1) ? 0x0000ffffu : 0xffff0000u;
        vv = u32x4{w[0], w[1], w[2], w[3]};
      }
      uint2* vdst = reinterpret_cast<uint2*>(&Vs[d * kVRow + vcol]);
      vdst[0] = uint2{vv.x, vv.y};
      vdst[1] = uint2{vv.z, vv.w};
    }
  };
  // Scaled scores of the tile's 64 keys for the lane's query: s[sub][t] is
  // key kt0 + 16 sub + 4 lg + t.  Both passes run exactly this.
  auto tile_scores = [&](floatx4 (&s)[4]) {
#pragma unroll
    for (int sub = 0; sub < 4; ++sub) s[sub] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int ks = 0; ks < kHd / 32; ++ks)
#pragma unroll
      for (int sub = 0; sub < 4; ++sub) {
        const bf16x8 ka = as_bf16x8(
            *reinterpret_cast<const u32x4*>(&Ks[(16 * sub + lq) * kQRow + 8 * (kpiece ^ (4 * ks))]));
        s[sub] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ka, qb[ks], s[sub], 0, 0, 0);
      }
#pragma unroll
    for (int sub = 0; sub < 4; ++sub)
#pragma unroll
      for (int t = 0; t < 4; ++t) s[sub][t] = s[sub][t] * a.scale;
  };
  // Key kt0 + 16 sub + 4 lg + t is visible to the lane's query when
  // 16 sub + t <= lim; only a tile reaching past the wave's first query
  // masks anything.
  auto visible = [&](int kt0, int sub, int t) { return 16 * sub + t <= qpos - kt0 - 4 * lg; };

  // Pass 1: the exact maximum of the visible scores (order-free).
  float m = -INFINITY;
  load_keys(0);
  for (int kt0 = 0; kt0 < key_end; kt0 += kKeyTile) {
    if (kt0 > 0) __syncthreads();
    store_keys();
    __syncthreads();
    if (kt0 + kKeyTile < key_end) load_keys(kt0 + kKeyTile);
    floatx4 s[4];
    tile_scores(s);
    const bool masking = kt0 + kKeyTile - 1 > wave_first;
#pragma unroll
    for (int sub = 0; sub < 4; ++sub)
#pragma unroll
      for (int t = 0; t < 4; ++t)
        if (!masking || visible(kt0, sub, t)) m = fmaxf(m, s[sub][t]);
  }
  // Key 0 is visible to every query, so m is finite.
  m = fmaxf(m, __shfl_xor(m, 16));
  m = fmaxf(m, __shfl_xor(m, 32));

  // Pass 2: e = exp(s - m), the strided partials, and O^T += V^T E^T.
  float part[8];  // partials 4 lg + t (t < 4) and 16 + 4 lg + (t - 4)
#pragma unroll
  for (int i = 0; i < 8; ++i) part[i] = 0.0f;
  __syncthreads();  // every wave is done with the last key tile of pass 1
  load_keys(0);
  load_values(0);
  for (int kt0 = 0; kt0 < key_end; kt0 += kKeyTile) {
    if (kt0 > 0) __syncthreads();
    store_keys();
    store_values(kt0);
    __syncthreads();
    if (kt0 + kKeyTile < key_end) {
      load_keys(kt0 + kKeyTile);
      load_values(kt0 + kKeyTile);
    }
    floatx4 s[4];
    tile_scores(s);
    const bool masking = kt0 + kKeyTile - 1 > wave_first;
    // Partial (sub & 1, t) takes key 16 sub + 4 lg + t of sub 0, then 2
    // (even) or 1, then 3 (odd): ascending keys within every partial.
#pragma unroll
    for (int sub = 0; sub < 4; ++sub)
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const float e = (!masking || visible(kt0, sub, t)) ? exp_nonpositive(s[sub][t] - m) : 0.0f;
        s[sub][t] = e;
        part[4 * (sub & 1) + t] = part[4 * (sub & 1) + t] + e;
      }

    // O^T += V^T E^T, one 32-key K step per pair of 16-key blocks.
#pragma unroll
    for (int ks = 0; ks < kKeyTile / 32; ++ks) {
      const float p[8] = {s[2 * ks][0], s[2 * ks][1], s[2 * ks][2], s[2 * ks][3],
                          s[2 * ks + 1][0], s[2 * ks + 1][1], s[2 * ks + 1][2], s[2 * ks + 1][3]};
      // e = hi + mid + lo exactly: hi is e cut to its top 8 significant
      // bits, mid the residual cut the same way, and lo the rest, which has
      // at most 8 significant bits left; both subtractions are exact.  The
      // parts are the upper halves of the FP32 words, packed by byte permute.
      uint32_t hi[4], mid[4], lo[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint32_t b0 = __float_as_uint(p[2 * e]), b1 = __float_as_uint(p[2 * e + 1]);
        hi[e] = __builtin_amdgcn_perm(b1, b0, 0x07060302u);
        const float r0 = p[2 * e] - __uint_as_float(b0 & 0xffff0000u);
        const float r1 = p[2 * e + 1] - __uint_as_float(b1 & 0xffff0000u);
        const uint32_t c0 = __float_as_uint(r0), c1 = __float_as_uint(r1);
        mid[e] = __builtin_amdgcn_perm(c1, c0, 0x07060302u);
        const float l0 = r0 - __uint_as_float(c0 & 0xffff0000u);
        const float l1 = r1 - __uint_as_float(c1 & 0xffff0000u);
        lo[e] = __builtin_amdgcn_perm(__float_as_uint(l1), __float_as_uint(l0), 0x07060302u);
      }
      const bf16x8 ph = as_bf16x8(u32x4{hi[0], hi[1], hi[2], hi[3]});
      const bf16x8 pm = as_bf16x8(u32x4{mid[0], mid[1], mid[2], mid[3]});
      const bf16x8 pl = as_bf16x8(u32x4{lo[0], lo[1], lo[2], lo[3]});
      const int k0 = 32 * ks + 4 * lg;  // keys k0..k0+3 and k0+16..k0+19 of the tile
#pragma unroll
      for (int d = 0; d < 8; ++d) {
        const uint16_t* vrow = &Vs[(16 * d + lq) * kVRow];
        const uint2 va = *reinterpret_cast<const uint2*>(vrow + k0);
        const uint2 vb = *reinterpret_cast<const uint2*>(vrow + k0 + 16);
        const bf16x8 vt = as_bf16x8(u32x4{va.x, va.y, vb.x, vb.y});
        o[d] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vt, ph, o[d], 0, 0, 0);
        o[d] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vt, pm, o[d], 0, 0, 0);
        o[d] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vt, pl, o[d], 0, 0, 0);
      }
    }
  }

  // The half tree: offset 16 in the lane, 8 across lane groups lg ^ 2, 4
  // across lg ^ 1, then 2 and 1 in the lane (every lane ends with l).
  float q4[4];
#pragma unroll
  for (int t = 0; t < 4; ++t) q4[t] = part[t] + part[4 + t];
#pragma unroll
  for (int t = 0; t < 4; ++t) q4[t] = q4[t] + __shfl_xor(q4[t], 32);
#pragma unroll
  for (int t = 0; t < 4; ++t) q4[t] = q4[t] + __shfl_xor(q4[t], 16);
  const float l = (q4[0] + q4[2]) + (q4[1] + q4[3]);

  const int row = q0 + qrow;
  if (row < a.rows) {
    uint16_t* dst = a.out + static_cast<uint64_t>(row) * qw;
#pragma unroll
    for (int d = 0; d < 8; ++d)
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const uint32_t feature = h * kHd + 16 * d + 4 * lg + t;
        dst[permuted(feature, 16)] = dl_f32_to_bf16(o[d][t] / l);
      }
  }
}

// x_perm[m][permuted(k, P)] = x[m][k].
__global__ void k_permute(const uint16_t* x, uint16_t* out, uint64_t rows, uint32_t width, uint32_t P) {
  const uint64_t n = rows * width;
  const uint64_t step = static_cast<uint64_t>(gridDim.x) * blockDim.x;
  for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += step) {
    const uint64_t m = i / width;
    const uint32_t k = static_cast<uint32_t>(i % width);
    out[m * width + permuted(k, P)] = x[i];
  }
}

}  // namespace

void launch_permute(hipStream_t stream, const uint16_t* x, uint16_t* out, uint64_t rows, uint32_t width,
                    uint32_t P) {
  const uint64_t n = rows * width;
  const unsigned grid = static_cast<unsigned>(std::min<uint64_t>((n + 255) / 256, 65535));
  hipLaunchKernelGGL(k_permute, dim3(grid), dim3(256), 0, stream, x, out, rows, width, P);
}

// Builds g_silu_table on the current device before its first gate/up GEMM
// (and waits for it, so a GEMM on any other stream of the device finds it).
void ensure_silu_table(hipStream_t stream) {
  static std::mutex mu;
  static std::vector<bool> built;
  int device = 0;
  check_hip(hipGetDevice(&device), "current device");
  std::lock_guard<std::mutex> lock(mu);
  if (built.size() <= static_cast<size_t>(device)) built.resize(device + 1, false);
  if (built[device]) return;
  hipLaunchKernelGGL(k_silu_table, dim3(65536 / 256), dim3(256), 0, stream);
  check_hip(hipGetLastError(), "SiLU table");
  check_hip(hipStreamSynchronize(stream), "SiLU table");
  built[device] = true;
}

void launch_gemm(hipStream_t stream, const GemmArgs& a) {
  if (a.epilogue == kGateUp) ensure_silu_table(stream);
  // 256 x 256 tiles where they fill the GPU in whole rounds (gate/up, O,
  // down at 4096 rows); the QKV epilogue keeps the 128 x 256 tiles.
  if (a.N % 256 == 0 && a.n_split % 256 == 0 && a.M % kBigM == 0 && a.epilogue != kStoreQkv &&
      (a.N / 256) * (a.M / kBigM) >= 256) {
    const dim3 grid(a.N / kDmaTN, a.M / kBigM);
    switch (a.epilogue) {
      case kStore: hipLaunchKernelGGL((k_gemm_big<kStore>), grid, dim3(kBigThreads), 0, stream, a); break;
      case kResidual: hipLaunchKernelGGL((k_gemm_big<kResidual>), grid, dim3(kBigThreads), 0, stream, a); break;
      default: hipLaunchKernelGGL((k_gemm_big<kGateUp>), grid, dim3(kBigThreads), 0, stream, a); break;
    }
    return;
  }
  // The 256-wide tile needs whole tiles on both sides of the Q | K/V split.
  if (a.N % 256 == 0 && a.n_split % 256 == 0) {
    const dim3 grid(a.N / kDmaTN, a.M / kTileM);
    switch (a.epilogue) {
      case kStore: hipLaunchKernelGGL((k_gemm_dma<kStore>), grid, dim3(kGemmThreads), 0, stream, a); break;
      case kStoreQkv: hipLaunchKernelGGL((k_gemm_dma<kStoreQkv>), grid, dim3(kGemmThreads), 0, stream, a); break;
      case kResidual: hipLaunchKernelGGL((k_gemm_dma<kResidual>), grid, dim3(kGemmThreads), 0, stream, a); break;
      default: hipLaunchKernelGGL((k_gemm_dma<kGateUp>), grid, dim3(kGemmThreads), 0, stream, a); break;
    }
    return;
  }
  const dim3 grid(a.N / kTileN, a.M / kTileM);
  switch (a.epilogue) {
    case kStore: hipLaunchKernelGGL((k_gemm<kStore, 2>), grid, dim3(kGemmThreads), 0, stream, a); break;
    case kStoreQkv: hipLaunchKernelGGL((k_gemm<kStoreQkv, 2>), grid, dim3(kGemmThreads), 0, stream, a); break;
    case kResidual: hipLaunchKernelGGL((k_gemm<kResidual, 2>), grid, dim3(kGemmThreads), 0, stream, a); break;
    default: hipLaunchKernelGGL((k_gemm<kGateUp, 2>), grid, dim3(kGemmThreads), 0, stream, a); break;
  }
}

void launch_norm(hipStream_t stream, const NormArgs& a) {
  hipLaunchKernelGGL(k_norm, dim3(a.rows), dim3(256), 0, stream, a);
}

void launch_heads(hipStream_t stream, const HeadArgs& a) {
  hipLaunchKernelGGL(k_heads, dim3(a.rows, a.q_heads + a.kv_heads), dim3(64), 0, stream, a);
}

void launch_attention(hipStream_t stream, const AttnArgs& a) {
  hipLaunchKernelGGL(k_attention, dim3((a.rows + kAttnRows - 1) / kAttnRows * a.q_heads), dim3(kAttnThreads), 0,
                     stream, a);
}

}  // namespace dl::prefill

// ------------------------------------------------------------------ C ABI
extern "C" int dl_prefill_projection(dl_queue* queue, const void* input, const void* packed, void* output,
                                     void* workspace, uint64_t rows, uint64_t input_width,
                                     uint64_t output_width) {
  return dl::guard([&] {
    dl::require(queue && input && packed && output && workspace, "null argument");
    dl::require(rows > 0 && rows % dl::prefill::kTileM == 0, "rows must be a positive multiple of 128");
    dl::require(output_width > 0 && output_width % dl::prefill::kTileN == 0,
                "output width must be a positive multiple of 128");
    const int P = (input_width <= 4096 && output_width > 1024) ? 16 : 32;
    dl::require(input_width > 0 && input_width % (8 * P) == 0 && input_width % 64 == 0,
                "input width must be a multiple of 8P and of 64");
    dl::enter(queue);
    hipStream_t s = queue->stream;
    uint16_t* perm = static_cast<uint16_t*>(workspace);
    dl::prefill::launch_permute(s, static_cast<const uint16_t*>(input), perm, rows,
                                static_cast<uint32_t>(input_width), static_cast<uint32_t>(P));
    dl::prefill::GemmArgs g{};
    g.a = g.a_alt = perm;
    g.w = g.w_alt = static_cast<const uint16_t*>(packed);
    g.M = static_cast<int>(rows);
    g.N = static_cast<int>(output_width);
    g.K = static_cast<int>(input_width);
    g.n_split = g.N;
    g.P = g.P_alt = P;
    g.epilogue = dl::prefill::kStore;
    g.m_valid = g.M;
    g.out = static_cast<uint16_t*>(output);
    dl::prefill::launch_gemm(s, g);
    dl::check_launch(queue, "prefill projection");
  });
}

extern "C" int dl_prefill_attention(dl_queue* queue, const void* q_rot, const void* k_cache, const void* v_cache,
                                    void* output, uint64_t rows, uint64_t q_heads, uint64_t kv_heads,
                                    uint64_t capacity, uint64_t first_position) {
  return dl::guard([&] {
    dl::require(queue && q_rot && k_cache && v_cache && output, "null argument");
    dl::require(rows > 0 && q_heads > 0 && kv_heads > 0 && q_heads % kv_heads == 0, "invalid attention shape");
    dl::require(capacity % 64 == 0 && first_position + rows <= capacity, "rows exceed the cache capacity",
                DL_LENGTH_ERROR);
    dl::require(capacity <= dl::prefill::kMaxAttnCapacity, "cache capacity too large for prefill attention",
                DL_LENGTH_ERROR);
    dl::enter(queue);
    dl::prefill::AttnArgs a{static_cast<const uint16_t*>(q_rot), static_cast<const uint16_t*>(k_cache),
                            static_cast<const uint16_t*>(v_cache), static_cast<uint16_t*>(output),
                            static_cast<int>(rows), static_cast<int>(q_heads), static_cast<int>(kv_heads),
                            static_cast<int>(capacity), static_cast<int>(first_position),
                            static_cast<float>(1.0 / std::sqrt(128.0))};
    dl::prefill::launch_attention(queue->stream, a);
    dl::check_launch(queue, "prefill attention");
  });
}

extern "C" int dl_prefill_gate_up(dl_queue* queue, const void* input, const void* packed, void* output,
                                  void* workspace, uint64_t rows, uint64_t hidden, uint64_t ffn) {
  return dl::guard([&] {
    dl::require(queue && input && packed && output && workspace, "null argument");
    dl::require(rows > 0 && rows % dl::prefill::kTileM == 0 && (2 * ffn) % dl::prefill::kTileN == 0 &&
                    hidden % 128 == 0 && hidden <= 4096 && ffn % 256 == 0,
                "invalid gate/up shape");
    dl::enter(queue);
    hipStream_t s = queue->stream;
    uint16_t* perm = static_cast<uint16_t*>(workspace);
    dl::prefill::launch_permute(s, static_cast<const uint16_t*>(input), perm, rows, static_cast<uint32_t>(hidden),
                                16);
    dl::prefill::GemmArgs g{};
    g.a = g.a_alt = perm;
    g.w = g.w_alt = static_cast<const uint16_t*>(packed);
    g.M = static_cast<int>(rows);
    g.N = g.n_split = static_cast<int>(2 * ffn);
    g.K = static_cast<int>(hidden);
    g.P = g.P_alt = 16;
    g.epilogue = dl::prefill::kGateUp;
    g.m_valid = g.M;
    g.out = static_cast<uint16_t*>(output);
    dl::prefill::launch_gemm(s, g);
    dl::check_launch(queue, "prefill gate/up");
  });
}
