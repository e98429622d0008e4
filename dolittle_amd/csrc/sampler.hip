// Device categorical selection (the law of
// src/inference/sampling/categorical.cpp:146-201) and the standalone
// DeviceCategorical C ABI (src/inference/sampling/device.h:58-85).
//
// k_sample_count   one pass over each BF16 row: NaN/+inf and finite flags,
//                  argmax partials (largest value, lowest id) and, for
//                  categorical rows, the per-value histogram over the 16-bit
//                  order key (descending value == descending key; -0 joins +0)
// k_sample_select  one 1024-lane workgroup per row: FP64 weight per distinct
//                  value, prefix estimates, guarded cutoff and draw decisions
//                  (exact serial replay when a decision falls inside the error
//                  band), id lookup of the chosen value's j-th occurrence, and
//                  the histogram cleared for the next selection
//
// Error band.  Let E_k be the exact sum of the first k weights.  The host
// fold F_k differs from E_k by at most (k - 1) * 2^-53 * E_k (positive
// summands), the host's exp from this build's by at most 2 ulp per weight
// (the CPU restatement's math checks), and every estimate formed here (64-term
// running sums, a 10-level scan, two roundings per candidate) by at most
// 143 * 2^-53 * E_k.  g = (n + 256) * 2^-52 bounds their sum with a factor 2
// to spare; a comparison that holds after widening by g is decided exactly as
// the host decides it.
#include <algorithm>
#include <cmath>
#include <cstring>
#include <memory>
#include <mutex>
#include <vector>

#include "dl_device.h"
#include "dl_internal.h"
#include "sampler.h"

namespace dl::sampling {

namespace {

constexpr uint32_t kNone = 0xffffffffu;
constexpr int kLookupTile = kSelectThreads * 16;
constexpr uint64_t kMtUpper = 0xffffffff80000000ull;
constexpr uint64_t kMtLower = 0x7fffffffull;
constexpr uint64_t kMtMatrix = 0xb5026f5aa96619e9ull;

// BF16 classification on raw bits.
__device__ __forceinline__ bool bf16_rejected(uint32_t x) {
  return (x & 0x7fffu) > 0x7f80u || x == 0x7f80u;  // NaN or +inf
}
__device__ __forceinline__ bool bf16_is_finite(uint32_t x) { return (x & 0x7f80u) != 0x7f80u; }

// Order key of a finite BF16 value: larger value, larger key; -0 equals +0.
__device__ __forceinline__ uint32_t bf16_order(uint32_t x) {
  if (x == 0x8000u) x = 0;
  return (x & 0x8000u) ? (~x & 0xffffu) : (x | 0x8000u);
}
__device__ __forceinline__ float order_value(uint32_t key) {
  const uint32_t bits = (key & 0x8000u) ? (key & 0x7fffu) : (~key & 0xffffu);
  return dl_bf16_to_f32(static_cast<uint16_t>(bits));
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

__device__ __forceinline__ uint32_t wave_or(uint32_t v) {
#pragma unroll
  for (int off = 32; off; off >>= 1) v |= __shfl_xor(v, off);
  return v;
}

__device__ __forceinline__ uint32_t wave_min_u32(uint32_t v) {
#pragma unroll
  for (int off = 32; off; off >>= 1) v = min(v, static_cast<uint32_t>(__shfl_xor(v, off)));
  return v;
}

template <class T>
__device__ __forceinline__ T wave_inclusive_scan(T v) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const T o = __shfl_up(v, off, 64);
    if (lane >= off) v = v + o;
  }
  return v;
}

// Exclusive prefix of v over the workgroup in thread order; *total gets the
// workgroup sum.  Every thread calls; lds holds one value per wavefront.
template <class T>
__device__ T block_exclusive_scan(T v, T* total, T* lds) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, waves = blockDim.x >> 6;
  const T inclusive = wave_inclusive_scan(v);
  T before = __shfl_up(inclusive, 1, 64);
  if (lane == 0) before = T(0);
  if (lane == 63) lds[wave] = inclusive;
  __syncthreads();
  if (wave == 0) {
    T t = lane < waves ? lds[lane] : T(0);
    t = wave_inclusive_scan(t);
    if (lane < waves) lds[lane] = t;
  }
  __syncthreads();
  const T base = wave ? lds[wave - 1] : T(0);
  *total = lds[waves - 1];
  __syncthreads();
  return base + before;
}

__device__ uint32_t block_min(uint32_t v, uint32_t* lds) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, waves = blockDim.x >> 6;
  v = wave_min_u32(v);
  if (lane == 0) lds[wave] = v;
  __syncthreads();
  uint32_t m = kNone;
  for (int w = 0; w < waves; ++w) m = min(m, lds[w]);
  __syncthreads();
  return m;
}

// ------------------------------------------------------------ MT19937-64
__device__ __forceinline__ uint64_t twist_word(uint64_t current, uint64_t next, uint64_t far) {
  const uint64_t x = (current & kMtUpper) | (next & kMtLower);
  return far ^ (x >> 1) ^ ((x & 1u) ? kMtMatrix : 0ull);
}

// The next MT19937-64 output of `state` (std::mt19937_64, sampler.h:52),
// computed by the whole workgroup (at least 312 lanes).  The in-place twist
// (word i takes old words i, i+1 and word i+156 mod 312, the latter already
// renewed when i >= 156) runs in three dependency phases: i < 156 reads only
// old words, 156 <= i < 311 reads the renewed i - 156, and i = 311 reads the
// renewed words 0 and 155.  Returns the same value to every thread.
__device__ uint64_t block_mt_next(RowState* state, uint64_t* words, uint64_t* out) {
  const int tid = threadIdx.x;
  const uint32_t index = state->index;
  __syncthreads();
  const bool twist = index >= kMtWords;
  if (twist) {
    for (int i = tid; i < kMtWords; i += blockDim.x) words[i] = state->words[i];
    __syncthreads();
    uint64_t v = 0;
    if (tid < 156) v = twist_word(words[tid], words[tid + 1], words[tid + 156]);
    __syncthreads();
    if (tid < 156) words[tid] = v;
    __syncthreads();
    if (tid >= 156 && tid < 311) v = twist_word(words[tid], words[tid + 1], words[tid - 156]);
    __syncthreads();
    if (tid >= 156 && tid < 311) words[tid] = v;
    __syncthreads();
    if (tid == 0) words[311] = twist_word(words[311], words[0], words[155]);
    __syncthreads();
    for (int i = tid; i < kMtWords; i += blockDim.x) state->words[i] = words[i];
  }
  if (tid == 0) {
    const uint32_t at = twist ? 0u : index;
    uint64_t y = twist ? words[0] : state->words[at];
    y ^= (y >> 29) & 0x5555555555555555ull;
    y ^= (y << 17) & 0x71d67fffeda60000ull;
    y ^= (y << 37) & 0xfff7eee000000000ull;
    y ^= y >> 43;
    state->index = at + 1;
    *out = y;
  }
  __syncthreads();
  const uint64_t y = *out;
  __syncthreads();
  return y;
}

__device__ __forceinline__ double draw_unit(uint64_t bits) {
  return static_cast<double>(bits >> 11) * 0x1p-53;
}

__device__ __forceinline__ bool row_live(const RowsArgs& a, int row) {
  return !a.loop.ctl || (row_selects(a.loop.ctl, row) && a.loop.ctl->mode == 1);
}

// ------------------------------------------------------------- counting
__global__ __launch_bounds__(kCountThreads) void k_sample_count(RowsArgs a) {
  __shared__ uint64_t wave_keys[kCountThreads / 64];
  __shared__ uint32_t wave_flags[kCountThreads / 64];
  // Consecutive workgroups go to different XCDs; taking the row from the
  // low digit keeps each row's histogram atomics on one XCD when rows | 8.
  const int row = static_cast<int>(blockIdx.x % a.rows);
  const int part = static_cast<int>(blockIdx.x / a.rows);
  if (!row_live(a, row)) return;
  const bool categorical = a.settings.mode == 1;
  const uint16_t* x = a.logits + static_cast<uint64_t>(row) * a.row_stride;
  const uint32_t chunk = (a.n + kCountBlocks - 1) / kCountBlocks;
  const uint32_t begin = min(a.n, static_cast<uint32_t>(part) * chunk);
  const uint32_t end = min(a.n, begin + chunk);
  uint32_t* hist = a.ws.hist + static_cast<uint64_t>(row) * kBins;
  uint64_t best = 0;
  uint32_t flags = 0;
  for (uint32_t i = begin + threadIdx.x; i < end; i += kCountThreads) {
    const uint32_t v = x[i];
    if (bf16_rejected(v)) {
      flags |= 1u;
    } else if (bf16_is_finite(v)) {
      flags |= 2u;
      const uint32_t key = bf16_order(v);
      const uint64_t k = (static_cast<uint64_t>(key) << 32) | (0xffffffffu - i);
      best = k > best ? k : best;
      if (categorical) atomicAdd(hist + key, 1u);
    }
  }
  best = wave_max_u64(best);
  flags = wave_or(flags);
  const int wave = threadIdx.x / 64;
  if ((threadIdx.x & 63) == 0) {
    wave_keys[wave] = best;
    wave_flags[wave] = flags;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < kCountThreads / 64; ++w) {
      best = wave_keys[w] > best ? wave_keys[w] : best;
      flags |= wave_flags[w];
    }
    a.ws.partial_keys[static_cast<uint64_t>(row) * kCountBlocks + part] = best;
    a.ws.partial_flags[static_cast<uint64_t>(row) * kCountBlocks + part] = flags;
  }
}

// ------------------------------------------------------------ selection
struct Found {
  uint32_t k;     // 1-based index among kept candidates, kNone if none
  uint32_t key;   // order key of its value
  uint32_t j;     // 1-based occurrence of that value (ascending id)
  double value;   // prefix estimate of the first k weights
};

__device__ __forceinline__ bool reaches(double v, double threshold, bool strict) {
  return strict ? v > threshold : v >= threshold;
}

// First kept candidate in this thread's bins whose prefix estimate reaches
// `threshold`.  The estimates form this thread's canonical non-decreasing
// sequence: A starts at the thread's scanned prefix, grows by count * weight
// per bin, and candidate j of a bin is estimated as A + j * weight.
__device__ __forceinline__ Found walk(const uint32_t (&count)[kBinsPerThread], uint32_t top, double A,
                                      uint32_t k, uint32_t kept_left, const double* w_row, double threshold,
                                      bool strict) {
  int hit = -1;
  double hit_a = 0.0, hit_w = 0.0;
  uint32_t hit_k = 0, hit_count = 0;
#pragma unroll
  for (int q = 0; q < kBinsPerThread; ++q) {
    const uint32_t kq = min(count[q], kept_left);
    kept_left -= kq;
    if (kq && hit < 0) {
      const double w = w_row[top - q];
      const double end = A + static_cast<double>(kq) * w;
      if (reaches(end, threshold, strict)) {
        hit = q;
        hit_a = A;
        hit_w = w;
        hit_k = k;
        hit_count = kq;
      } else {
        A = end;
        k += kq;
      }
    }
  }
  if (hit < 0) return Found{kNone, 0, 0, 0.0};
  uint32_t lo = 1, hi = hit_count;
  while (lo < hi) {
    const uint32_t mid = lo + (hi - lo) / 2;
    if (reaches(hit_a + static_cast<double>(mid) * hit_w, threshold, strict))
      hi = mid;
    else
      lo = mid + 1;
  }
  return Found{hit_k + lo, top - static_cast<uint32_t>(hit), lo, hit_a + static_cast<double>(lo) * hit_w};
}

// The host law folded serially over the histogram, one lane
// (categorical.cpp:178-200).  Returns the chosen value's key and occurrence.
__device__ void exact_replay(const uint32_t* hist, const double* w_row, uint32_t kept, double top_p, double u,
                             uint32_t* out_key, uint32_t* out_j) {
  double total = 0.0;
  uint32_t left = kept;
  for (int key = kBins - 1; key >= 0 && left; --key) {
    const uint32_t c = min(hist[key], left);
    if (!c) continue;
    left -= c;
    const double w = w_row[key];
    for (uint32_t i = 0; i < c; ++i) total = total + w;
  }
  double retained = 0.0;
  uint32_t count = 0, cut_key = 0, cut_j = 0;
  bool cut = false;
  left = kept;
  for (int key = kBins - 1; key >= 0 && left && !cut; --key) {
    const uint32_t c = min(hist[key], left);
    if (!c) continue;
    left -= c;
    const double w = w_row[key];
    for (uint32_t j = 1; j <= c; ++j) {
      retained = retained + w;
      ++count;
      if (!(count < kept && retained / total < top_p)) {
        cut = true;
        cut_key = static_cast<uint32_t>(key);
        cut_j = j;
        break;
      }
    }
  }
  *out_key = cut_key;
  *out_j = cut_j;
  double cumulative = 0.0;
  uint32_t seen = 0;
  left = kept;
  for (int key = kBins - 1; key >= 0 && left && seen < count; --key) {
    const uint32_t c = min(hist[key], left);
    if (!c) continue;
    left -= c;
    const double share = w_row[key] / retained;
    for (uint32_t j = 1; j <= c && seen < count; ++j) {
      ++seen;
      cumulative = cumulative + share;
      if (u < cumulative) {
        *out_key = static_cast<uint32_t>(key);
        *out_j = j;
        return;
      }
    }
  }
}

__global__ __launch_bounds__(kSelectThreads) void k_sample_select(RowsArgs a) {
  __shared__ uint64_t s_words[kMtWords];
  __shared__ uint64_t s_u64;
  __shared__ double s_dscan[kSelectThreads / 64];
  __shared__ uint32_t s_uscan[kSelectThreads / 64];
  __shared__ Found s_found[4];
  __shared__ uint32_t s_token;
  __shared__ uint32_t s_pick[2];
  __shared__ uint16_t s_tile[kLookupTile];

  const int row = blockIdx.x;
  const int tid = threadIdx.x;
  if (!row_live(a, row)) return;
  const Settings set = a.settings;
  const bool categorical = set.mode == 1;
  RowState* state = a.ws.state + row;
  uint32_t* hist = a.ws.hist + static_cast<uint64_t>(row) * kBins;
  double* w_row = a.ws.weights + static_cast<uint64_t>(row) * kBins;
  const uint16_t* x = a.logits + static_cast<uint64_t>(row) * a.row_stride;

  // Argmax partials and flags.
  if (tid < 64) {
    uint64_t key = a.ws.partial_keys[static_cast<uint64_t>(row) * kCountBlocks + tid];
    uint32_t flags = a.ws.partial_flags[static_cast<uint64_t>(row) * kCountBlocks + tid];
    key = wave_max_u64(key);
    flags = wave_or(flags);
    if (tid == 0) {
      s_found[0].value = 0.0;
      s_u64 = key;
      s_pick[0] = flags;
    }
  }
  __syncthreads();
  const uint64_t best = s_u64;
  const uint32_t flags = s_pick[0];
  __syncthreads();
  const uint32_t status = (flags & 1u) ? 1u : (!(flags & 2u) ? 2u : 0u);

  double u = a.draw ? *a.draw : a.draw_value;
  if (categorical && a.loop_rng) u = draw_unit(block_mt_next(state, s_words, &s_u64));

  uint32_t token = status ? 0u : 0xffffffffu - static_cast<uint32_t>(best & 0xffffffffu);
  const uint32_t top = kBins - 1 - kBinsPerThread * tid;
  if (categorical && status == 0) {
    // Per-value counts of this thread's bins, in descending value order.
    uint32_t count[kBinsPerThread];
    const u32x4* src = reinterpret_cast<const u32x4*>(hist + top - (kBinsPerThread - 1));
#pragma unroll
    for (int v = 0; v < kBinsPerThread / 4; ++v) {
      const u32x4 c = src[v];
      count[kBinsPerThread - 1 - 4 * v] = c.x;
      count[kBinsPerThread - 2 - 4 * v] = c.y;
      count[kBinsPerThread - 3 - 4 * v] = c.z;
      count[kBinsPerThread - 4 - 4 * v] = c.w;
    }
    uint32_t mine = 0;
#pragma unroll
    for (int q = 0; q < kBinsPerThread; ++q) mine += count[q];
    uint32_t size = 0;
    const uint32_t before = block_exclusive_scan<uint32_t>(mine, &size, s_uscan);
    const uint32_t kept = (set.top_k && size > set.top_k) ? set.top_k : size;
    const uint32_t kept_left = kept > before ? kept - before : 0u;

    // One weight per distinct kept value (categorical.cpp:178-181).
    const double z0 = static_cast<double>(order_value(static_cast<uint32_t>(best >> 32)));
    double mass = 0.0;
    {
      uint32_t left = kept_left;
#pragma unroll
      for (int q = 0; q < kBinsPerThread; ++q) {
        const uint32_t kq = min(count[q], left);
        left -= kq;
        if (kq) {
          const uint32_t key = top - q;
          const double w = dl_exp((static_cast<double>(order_value(key)) - z0) / set.temperature);
          w_row[key] = w;
          mass = mass + static_cast<double>(kq) * w;
        }
      }
    }
    double total = 0.0;
    const double prefix = block_exclusive_scan<double>(mass, &total, s_dscan);

    // Cutoff: the smallest c with F_c / F_n >= top_p lies in [c_lo, c_hi].
    const double g = (static_cast<double>(kept) + 256.0) * 0x1p-52;
    const double p = set.top_p;
    const double t_lo = p * total * ((1.0 - g) / (1.0 + g)) * (1.0 - 0x1p-50);
    const double t_hi = p * total * ((1.0 + g) / (1.0 - g)) * (1.0 + 0x1p-50);
    const Found f0 = walk(count, top, prefix, before, kept_left, w_row, t_lo, false);
    const Found f1 = walk(count, top, prefix, before, kept_left, w_row, t_hi, false);
    const uint32_t c_lo = block_min(f0.k, s_uscan);
    const uint32_t c_hi_found = block_min(f1.k, s_uscan);
    if (f0.k != kNone && f0.k == c_lo) s_found[0] = f0;
    if (f1.k != kNone && f1.k == c_hi_found) s_found[1] = f1;
    __syncthreads();
    const bool lost = c_lo == kNone;
    const uint32_t c_hi = c_hi_found == kNone ? kept : c_hi_found;
    const double e_lo = lost ? 0.0 : s_found[0].value;
    const double e_hi = c_hi_found == kNone ? total : s_found[1].value;

    // Draw: the first i with G_i > u lies in [s_lo, s_hi] (G_i the host's
    // fold of w / F_c, F_c within [R_lo, R_hi]).
    const double r_lo = e_lo * (1.0 - g) * (1.0 - 0x1p-50);
    const double r_hi = e_hi * (1.0 + g) * (1.0 + 0x1p-50);
    const double g2 = 2.0 * g;
    const double d_lo = u * r_lo / (1.0 + g2) * (1.0 - 0x1p-50);
    const double d_hi = u * r_hi / (1.0 - g2) * (1.0 + 0x1p-50);
    const Found f2 = walk(count, top, prefix, before, kept_left, w_row, d_lo, false);
    const Found f3 = walk(count, top, prefix, before, kept_left, w_row, d_hi, true);
    const uint32_t s_lo = block_min(f2.k, s_uscan);
    const uint32_t s_hi = block_min(f3.k, s_uscan);
    if (f3.k != kNone && f3.k == s_hi) s_found[3] = f3;
    __syncthreads();

    int pick = -1;  // 0: candidate c_lo, 3: candidate s_hi
    if (!lost && !a.exact) {
      const bool draw_known = s_lo == s_hi && s_hi != kNone;
      if (c_lo == c_hi) {
        if (draw_known && s_hi <= c_lo)
          pick = 3;
        else if (s_lo == kNone || s_lo > c_lo)
          pick = 0;
      } else if (draw_known && s_hi <= c_lo) {
        pick = 3;
      }
    }
    if (tid == 0) {
      s_token = 0;
      if (pick >= 0) {
        s_pick[0] = s_found[pick].key;
        s_pick[1] = s_found[pick].j;
      } else {
        exact_replay(hist, w_row, kept, p, u, &s_pick[0], &s_pick[1]);
        state->exact_replays += 1;
      }
    }
    __syncthreads();
    const uint32_t key = s_pick[0];
    uint32_t wanted = s_pick[1];

    // The wanted-th smallest id holding that value.
    for (uint32_t base = 0; base < a.n; base += kLookupTile) {
      const uint32_t len = min(static_cast<uint32_t>(kLookupTile), a.n - base);
      for (uint32_t i = tid; i < len; i += kSelectThreads) s_tile[i] = x[base + i];
      __syncthreads();
      uint32_t mine_hits = 0;
      const uint32_t first = tid * 16;
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const uint32_t i = first + e;
        if (i < len) {
          const uint32_t v = s_tile[i];
          mine_hits += (bf16_is_finite(v) && bf16_order(v) == key) ? 1u : 0u;
        }
      }
      uint32_t tile_hits = 0;
      const uint32_t earlier = block_exclusive_scan<uint32_t>(mine_hits, &tile_hits, s_uscan);
      if (wanted > earlier && wanted <= earlier + mine_hits) {
        uint32_t left = wanted - earlier;
        for (int e = 0; e < 16; ++e) {
          const uint32_t i = first + e;
          if (i < len) {
            const uint32_t v = s_tile[i];
            if (bf16_is_finite(v) && bf16_order(v) == key && --left == 0) {
              s_token = base + i;
              break;
            }
          }
        }
      }
      __syncthreads();
      if (wanted <= tile_hits) break;
      wanted -= tile_hits;
    }
    __syncthreads();
    token = s_token;
  }

  if (tid == 0) {
    const Result r{status ? 0u : token, status};
    if (a.loop.ctl) {
      Control* c = a.loop.ctl;
      if (status) {
        atomicOr(&c->status, status);
      } else {
        a.loop.selected[row] = r.token;
        const uint32_t emitted = c->row_generated[row];
        if (emitted < a.loop.out_capacity)
          a.loop.out_tokens[static_cast<uint64_t>(row) * a.loop.out_capacity + emitted] = r.token;
        c->row_generated[row] = emitted + 1;
        if (a.loop.stop_mask[r.token]) atomicOr(&c->finished_mask, 1u << row);
      }
    } else if (a.result_out) {
      *a.result_out = r;
    } else {
      state->result = r;
    }
  }
  if (categorical) {
    __syncthreads();
    u32x4* dst = reinterpret_cast<u32x4*>(hist + top - (kBinsPerThread - 1));
    const u32x4 zero = {0u, 0u, 0u, 0u};
#pragma unroll
    for (int v = 0; v < kBinsPerThread / 4; ++v) dst[v] = zero;
  }
}

__global__ void k_rng_seed(RowState* state, Seeds seeds) {
  RowState* s = state + blockIdx.x;
  uint64_t prev = seeds.seed[blockIdx.x];
  s->words[0] = prev;
  for (uint32_t i = 1; i < kMtWords; ++i) {
    prev = 6364136223846793005ull * (prev ^ (prev >> 62)) + i;
    s->words[i] = prev;
  }
  s->index = kMtWords;
  s->terminal = 0;
  s->draw = 0.0;
  s->result = Result{0, 0};
  s->previous = Result{0, 0};
}

// DeviceCategorical live draw (sampling.cu next_random): none once the
// stream is terminal or for greedy selection.
__global__ __launch_bounds__(512) void k_rng_next(RowState* state, int greedy) {
  __shared__ uint64_t words[kMtWords];
  __shared__ uint64_t out;
  if (state->terminal || greedy) return;
  const uint64_t y = block_mt_next(state, words, &out);
  if (threadIdx.x == 0) state->draw = draw_unit(y);
}

// DeviceCategorical terminal latch (sampling.cu commit_selection).
__global__ void k_rng_commit(RowState* state, const uint8_t* stop_mask) {
  if (state->terminal) {
    state->result = state->previous;
    return;
  }
  state->previous = state->result;
  state->terminal = state->result.status || stop_mask[state->result.token];
}

__global__ void k_clear_hist(uint32_t* hist, uint64_t words) {
  const uint64_t step = static_cast<uint64_t>(gridDim.x) * blockDim.x;
  for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < words; i += step) hist[i] = 0;
}

__global__ void k_clear_state(RowState* state, int rows) {
  const int r = threadIdx.x;
  if (r < rows) {
    state[r].index = kMtWords;
    state[r].terminal = 0;
    state[r].draw = 0.0;
    state[r].result = Result{0, 0};
    state[r].previous = Result{0, 0};
    state[r].exact_replays = 0;
  }
}

constexpr uint64_t align_up(uint64_t v, uint64_t a) { return (v + a - 1) / a * a; }

}  // namespace

std::size_t workspace_bytes(int rows, uint64_t vocabulary) {
  uint64_t b = 0;
  b += align_up(uint64_t(rows) * kBins * sizeof(uint32_t), 256);
  b += align_up(uint64_t(rows) * kBins * sizeof(double), 256);
  b += align_up(uint64_t(rows) * kCountBlocks * sizeof(uint64_t), 256);
  b += align_up(uint64_t(rows) * kCountBlocks * sizeof(uint32_t), 256);
  b += align_up(uint64_t(rows) * sizeof(RowState), 256);
  b += align_up(vocabulary, 256);
  return b;
}

Workspace carve_workspace(void* base, int rows, uint64_t vocabulary) {
  (void)vocabulary;
  auto* p = static_cast<uint8_t*>(base);
  Workspace w{};
  w.hist = reinterpret_cast<uint32_t*>(p);
  p += align_up(uint64_t(rows) * kBins * sizeof(uint32_t), 256);
  w.weights = reinterpret_cast<double*>(p);
  p += align_up(uint64_t(rows) * kBins * sizeof(double), 256);
  w.partial_keys = reinterpret_cast<uint64_t*>(p);
  p += align_up(uint64_t(rows) * kCountBlocks * sizeof(uint64_t), 256);
  w.partial_flags = reinterpret_cast<uint32_t*>(p);
  p += align_up(uint64_t(rows) * kCountBlocks * sizeof(uint32_t), 256);
  w.state = reinterpret_cast<RowState*>(p);
  p += align_up(uint64_t(rows) * sizeof(RowState), 256);
  w.stop_mask = p;
  return w;
}

void launch_count(hipStream_t stream, const RowsArgs& args) {
  hipLaunchKernelGGL(k_sample_count, dim3(args.rows * kCountBlocks), dim3(kCountThreads), 0, stream, args);
}

void launch_select(hipStream_t stream, const RowsArgs& args) {
  hipLaunchKernelGGL(k_sample_select, dim3(args.rows), dim3(kSelectThreads), 0, stream, args);
}

void launch_seed(hipStream_t stream, RowState* state, int rows, const Seeds& seeds) {
  hipLaunchKernelGGL(k_rng_seed, dim3(rows), dim3(1), 0, stream, state, seeds);
}

void launch_clear(hipStream_t stream, const Workspace& ws, int rows) {
  hipLaunchKernelGGL(k_clear_hist, dim3(256), dim3(256), 0, stream, ws.hist, uint64_t(rows) * kBins);
  hipLaunchKernelGGL(k_clear_state, dim3(1), dim3(64), 0, stream, ws.state, rows);
}

}  // namespace dl::sampling

// ------------------------------------------------------------------ C ABI
using namespace dl::sampling;

struct dl_sampler {
  dl_device* device = nullptr;
  dl_queue* queue = nullptr;
  uint64_t vocabulary = 0;
  void* arena = nullptr;
  Workspace ws{};
  Settings settings{};
  bool started = false;
  bool has_result = false;
  int exact = 0;
};

namespace {

constexpr uint64_t kMaxVocabulary = 1ull << 28;

Settings checked_settings(const dl_sampling* s) {
  dl::require(s != nullptr, "null sampling settings");
  const bool valid = (s->mode == 0 || s->mode == 1) && std::isfinite(s->temperature) && s->temperature > 0 &&
                     std::isfinite(s->top_p) && s->top_p > 0 && s->top_p <= 1 &&
                     !(s->mode == 0 && (s->temperature != 1 || s->top_k != 0 || s->top_p != 1));
  dl::require(valid, "invalid sampling settings");
  return Settings{s->mode, s->top_k, s->temperature, s->top_p};
}

RowsArgs row_args(dl_sampler* s, const void* row, const Settings& settings) {
  RowsArgs a{};
  a.logits = static_cast<const uint16_t*>(row);
  a.row_stride = s->vocabulary;
  a.n = static_cast<uint32_t>(s->vocabulary);
  a.rows = 1;
  a.settings = settings;
  a.ws = s->ws;
  a.exact = s->exact;
  return a;
}

void check_row(dl_sampler* s, const void* row, uint64_t row_bytes) {
  dl::require(row != nullptr && row_bytes == s->vocabulary * 2, "invalid device sampling row");
}

// ---------------------------------------------- allocation-free selection
// Scratch of dl_sample_noalloc: the workspace of one selection row (the
// 65,536-bin histogram, the FP64 weight of each distinct value, the argmax
// partials and one row state), carved exactly as carve_workspace(base, 1, 0)
// carves an allocated arena.  Each GPU holds its own copy until the process
// ends.  Host code never passes the array's name to a kernel: its device
// address comes from hipGetSymbolAddress, once per device.
constexpr uint64_t kNoAllocScratchBytes =
    align_up(uint64_t(kBins) * sizeof(uint32_t), 256) + align_up(uint64_t(kBins) * sizeof(double), 256) +
    align_up(uint64_t(kCountBlocks) * sizeof(uint64_t), 256) + align_up(uint64_t(kCountBlocks) * sizeof(uint32_t), 256) +
    align_up(sizeof(RowState), 256);
__device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];

std::mutex scratch_mutex;
std::vector<void*> scratch_address;  // per device ordinal, from hipGetSymbolAddress

// The current device's address of `scratch` (the device is current: the
// caller went through dl::enter).
void* scratch_on(int ordinal) {
  std::lock_guard<std::mutex> lock(scratch_mutex);
  if (scratch_address.size() <= static_cast<size_t>(ordinal)) scratch_address.resize(ordinal + 1, nullptr);
  if (!scratch_address[ordinal]) {
    void* ptr = nullptr;
    dl::check_hip(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)), "sampler scratch address");
    dl::require(ptr != nullptr, "sampler scratch address", DL_RUNTIME_ERROR);
    scratch_address[ordinal] = ptr;
  }
  return scratch_address[ordinal];
}

}  // namespace

extern "C" {

int dl_sample_noalloc(dl_queue* queue, const void* logits, uint64_t row_bytes, uint64_t vocabulary,
                      const dl_sampling* settings, uint64_t draw_bits, uint32_t* result) {
  return dl::guard([&] {
    const Settings st = checked_settings(settings);
    dl::require(vocabulary > 0, "unsupported sampling vocabulary");
    dl::require(vocabulary <= kMaxVocabulary, "vocabulary above the allocation-free sampler's maximum of 2^28 ids",
                DL_LENGTH_ERROR);
    dl::require(logits != nullptr && row_bytes == vocabulary * 2, "invalid device sampling row");
    dl::require(result != nullptr && reinterpret_cast<uintptr_t>(result) % alignof(uint32_t) == 0,
                "invalid device result region");
    dl::require(st.top_k <= vocabulary, "invalid device sampling row");
    dl::enter(queue);
    const Workspace ws = carve_workspace(scratch_on(queue->device->ordinal), 1, 0);
    // The count kernel adds into the histogram, which must start at zero
    // (a fill kernel, so the call can be recorded into a graph).
    hipLaunchKernelGGL(k_clear_hist, dim3(64), dim3(256), 0, queue->stream, ws.hist, uint64_t(kBins));
    RowsArgs a{};
    a.logits = static_cast<const uint16_t*>(logits);
    a.row_stride = vocabulary;
    a.n = static_cast<uint32_t>(vocabulary);
    a.rows = 1;
    a.settings = st;
    a.ws = ws;
    a.draw_value = static_cast<double>(draw_bits >> 11) * 0x1p-53;
    a.result_out = reinterpret_cast<Result*>(result);
    launch_count(queue->stream, a);
    launch_select(queue->stream, a);
    dl::check_launch(queue, "allocation-free selection");
  });
}

int dl_sampler_required_bytes(uint64_t vocabulary, uint64_t* bytes) {
  return dl::guard([&] {
    dl::require(bytes != nullptr, "null argument");
    dl::require(vocabulary > 0 && vocabulary <= kMaxVocabulary, "unsupported sampling vocabulary");
    *bytes = workspace_bytes(1, vocabulary);
  });
}

int dl_sampler_create(dl_device* device, dl_queue* queue, uint64_t vocabulary, int dtype, uint64_t budget,
                      dl_sampler** out) {
  return dl::guard([&] {
    dl::require(device && queue && out, "null argument");
    dl::require(queue->device == device, "queue belongs to another device");
    dl::require(vocabulary > 0 && vocabulary <= kMaxVocabulary, "unsupported sampling vocabulary");
    const uint64_t bytes = workspace_bytes(1, vocabulary);
    dl::require(bytes <= budget, "device sampling exceeds budget", DL_LENGTH_ERROR);
    dl::require(dtype == DL_BF16 || dtype == DL_F32, "unsupported sampling storage");
    dl::require(dtype == DL_BF16, "FP32 logits rows are not supported by the gfx950 sampler");
    dl::enter(queue);
    auto s = std::make_unique<dl_sampler>();
    s->device = device;
    s->queue = queue;
    s->vocabulary = vocabulary;
    dl::check_hip(hipMalloc(&s->arena, bytes), "sampler workspace");
    s->ws = carve_workspace(s->arena, 1, vocabulary);
    launch_clear(queue->stream, s->ws, 1);
    dl::check_launch(queue, "sampler clear");
    *out = s.release();
  });
}

int dl_sampler_destroy(dl_sampler* sampler) {
  if (!sampler) return DL_OK;
  (void)hipSetDevice(sampler->device->ordinal);
  (void)hipStreamSynchronize(sampler->queue->stream);
  (void)hipFree(sampler->arena);
  delete sampler;
  return DL_OK;
}

int dl_sampler_submit(dl_sampler* s, const void* logits, uint64_t row_bytes, const dl_sampling* settings,
                      uint64_t draw_bits) {
  return dl::guard([&] {
    dl::require(s != nullptr, "null sampler");
    const Settings st = checked_settings(settings);
    check_row(s, logits, row_bytes);
    dl::require(st.top_k <= s->vocabulary, "invalid device sampling row");
    dl::enter(s->queue);
    RowsArgs a = row_args(s, logits, st);
    a.draw_value = static_cast<double>(draw_bits >> 11) * 0x1p-53;
    launch_count(s->queue->stream, a);
    launch_select(s->queue->stream, a);
    dl::check_launch(s->queue, "device selection");
  });
}

int dl_sampler_start(dl_sampler* s, const dl_sampling* settings, uint64_t seed, const uint32_t* stop_ids,
                     uint32_t stop_count) {
  return dl::guard([&] {
    dl::require(s != nullptr, "null sampler");
    const Settings st = checked_settings(settings);
    dl::require(!s->started && st.top_k <= s->vocabulary, "invalid or repeated device sampler start");
    for (uint32_t i = 0; i < stop_count; ++i)
      dl::require(stop_ids && stop_ids[i] < s->vocabulary, "stop ID outside vocabulary");
    dl::enter(s->queue);
    hipStream_t stream = s->queue->stream;
    std::vector<uint8_t> mask(s->vocabulary, 0);
    for (uint32_t i = 0; i < stop_count; ++i) mask[stop_ids[i]] = 1;
    dl::check_hip(hipMemcpyAsync(s->ws.stop_mask, mask.data(), mask.size(), hipMemcpyHostToDevice, stream),
                  "stop mask");
    Seeds seeds{};
    seeds.seed[0] = seed;
    launch_seed(stream, s->ws.state, 1, seeds);
    dl::check_launch(s->queue, "sampler seed");
    dl::check_hip(hipStreamSynchronize(stream), "sampler start");
    s->settings = st;
    s->started = true;
  });
}

int dl_sampler_submit_next(dl_sampler* s, const void* logits, uint64_t row_bytes) {
  return dl::guard([&] {
    dl::require(s != nullptr, "null sampler");
    dl::require(s->started, "device sampler not started");
    check_row(s, logits, row_bytes);
    dl::enter(s->queue);
    hipStream_t stream = s->queue->stream;
    RowsArgs a = row_args(s, logits, s->settings);
    a.draw = &s->ws.state->draw;
    hipLaunchKernelGGL(k_rng_next, dim3(1), dim3(512), 0, stream, s->ws.state, s->settings.mode == 0 ? 1 : 0);
    launch_count(stream, a);
    launch_select(stream, a);
    hipLaunchKernelGGL(k_rng_commit, dim3(1), dim3(1), 0, stream, s->ws.state, s->ws.stop_mask);
    dl::check_launch(s->queue, "device selection");
    s->has_result = true;
  });
}

int dl_sampler_result(dl_sampler* s, uint32_t* token, uint32_t* status) {
  return dl::guard([&] {
    dl::require(s && token && status, "null argument");
    dl::enter(s->queue);
    Result r{};
    dl::check_hip(hipMemcpyAsync(&r, &s->ws.state->result, sizeof r, hipMemcpyDeviceToHost, s->queue->stream),
                  "read selection");
    dl::check_hip(hipStreamSynchronize(s->queue->stream), "selection");
    *token = r.token;
    *status = r.status;
  });
}

int dl_sampler_result_address(dl_sampler* s, void** out) {
  return dl::guard([&] {
    dl::require(s && out, "null argument");
    *out = &s->ws.state->result;
  });
}

int dl_sampler_terminal_address(dl_sampler* s, void** out) {
  return dl::guard([&] {
    dl::require(s && out, "null argument");
    *out = &s->ws.state->terminal;
  });
}

int dl_sampler_current_token_address(dl_sampler* s, void** out) {
  return dl::guard([&] {
    dl::require(s && out, "null argument");
    dl::require(s->started && s->has_result, "device sampler has no preceding selection");
    *out = &s->ws.state->result.token;
  });
}

int dl_sampler_set_exact(dl_sampler* s, int exact) {
  return dl::guard([&] {
    dl::require(s != nullptr, "null sampler");
    s->exact = exact ? 1 : 0;
  });
}

int dl_sampler_exact_replays(dl_sampler* s, uint64_t* count) {
  return dl::guard([&] {
    dl::require(s && count, "null argument");
    dl::enter(s->queue);
    dl::check_hip(hipMemcpyAsync(count, &s->ws.state->exact_replays, sizeof *count, hipMemcpyDeviceToHost,
                                 s->queue->stream),
                  "read replays");
    dl::check_hip(hipStreamSynchronize(s->queue->stream), "replays");
  });
}

}  // extern "C"
