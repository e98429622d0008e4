// Per-head QK RMSNorm + RoPE of one 128-wide head by one wavefront, shared
// by the decode attention kernels and the prefill head kernel.
#pragma once

#include "dl_device.h"

namespace dl {

// Per-head RMSNorm (width 128: lane t, component c holds feature t+32c;
// normalization.cu:82-132) followed by RoPE (rotary.cu:84-126) for one head,
// computed by one wavefront; lane i owns the RoPE pair (i, i+64).  The
// operands are loaded first (head_load) so callers can issue them ahead of
// other memory traffic.
struct HeadOperands {
  float xa, xb, ga, gb, cosine, sine;
};

__device__ __forceinline__ HeadOperands head_load(const uint16_t* __restrict__ x, const uint16_t* __restrict__ gain,
                                                  const float* __restrict__ rope_pos, int lane) {
  return HeadOperands{dl_bf16_to_f32(x[lane]), dl_bf16_to_f32(x[lane + 64]), dl_bf16_to_f32(gain[lane]),
                      dl_bf16_to_f32(gain[lane + 64]), rope_pos[2 * lane], rope_pos[2 * lane + 1]};
}

__device__ __forceinline__ void head_norm_rope(const HeadOperands& o, int lane, float eps, float* out) {
  const float xa = o.xa, xb = o.xb;
  const float xa_hi = __shfl(xa, (lane + 32) & 63);
  const float xb_hi = __shfl(xb, (lane + 32) & 63);
  const float s = tree_sum32(((xa * xa + xa_hi * xa_hi) + xb * xb) + xb_hi * xb_hi);
  const float total = __shfl(s, 0);
  const float inverse = inverse_sqrt(total * (1.0f / 128.0f) + eps);
  const float na = dl_round_bf16(dl_round_bf16(xa * inverse) * o.ga);
  const float nb = dl_round_bf16(dl_round_bf16(xb * inverse) * o.gb);
  out[lane] = dl_round_bf16(dl_round_bf16(na * o.cosine) - dl_round_bf16(nb * o.sine));
  out[lane + 64] = dl_round_bf16(dl_round_bf16(nb * o.cosine) + dl_round_bf16(na * o.sine));
}

__device__ __forceinline__ void head_norm_rope(const uint16_t* __restrict__ x, const uint16_t* __restrict__ gain,
                                               const float* __restrict__ rope_pos, int lane, float eps,
                                               float* out) {
  head_norm_rope(head_load(x, gain, rope_pos, lane), lane, eps, out);
}

}  // namespace dl
