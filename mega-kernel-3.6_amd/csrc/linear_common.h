// Arithmetic shared by the Qwen3.6 linear-attention kernels: the causal conv
// update of one channel and the gated RMSNorm of one row.  The separate ops
// (csrc/linear_step.hip) and the one-launch step (csrc/linear_attention.hip)
// both call these, so the step is bit-identical to composing the ops.
#pragma once

#include "mkq_device.h"

namespace mkq {

constexpr int kMaxConvTaps = 8;  // conv width S + 1 <= 8

// One channel of causal_conv1d_update: win = [state[0..S-1], x] (zero past
// S) and w = the channel's S + 1 taps (zero past S), NT >= S + 1 entries.
// acc = bias + sum_t w[t] * win[t] as an FMA chain in tap order, rounded to
// T, then SiLU rounded to T when `act`: the roundings of a T-typed
// convolution followed by a T-typed SiLU.  Returns the T value as FP32.
template <typename T, int NT>
__device__ __forceinline__ float conv_channel(const float (&win)[NT], const float (&w)[NT], float bias, int s_len,
                                              bool act) {
  float acc = bias;
#pragma unroll
  for (int t = 0; t < NT; ++t)
    if (t <= s_len) acc = fmaf(w[t], win[t], acc);
  float y = to_f(from_f<T>(acc));
  if (act) y = to_f(from_f<T>(silu(y)));
  return y;
}

// Gated RMSNorm (norm before gate) of one row of d values by one wave:
//     n = T(x * rsqrt(mean(x^2) + eps));  t = T(w * n);  out = T(t * silu(z))
// The sum of squares runs over i = lane, lane + 64, ... as an FMA chain, then
// a wave sum; gated_norm_inv takes that sum, gated_norm_value gives out[i].
__device__ __forceinline__ float gated_norm_inv(float lane_ss, int d, float eps) {
  return 1.0f / sqrtf(wave_sum(lane_ss) / float(d) + eps);
}
template <typename T>
__device__ __forceinline__ T gated_norm_value(float x, float inv, float w, float z) {
  const float n = to_f(from_f<T>(x * inv));
  const float t = to_f(from_f<T>(w * n));
  return from_f<T>(t * silu(z));
}

// The whole row from memory; `xv(i)` returns x[i] as FP32.
template <typename T, typename XV>
__device__ __forceinline__ void gated_norm_row(XV xv, const T* __restrict__ zr, const T* __restrict__ w,
                                               T* __restrict__ orow, int d, float eps, int lane) {
  float ss = 0.f;
  for (int i = lane; i < d; i += kWave) {
    const float v = xv(i);
    ss = fmaf(v, v, ss);
  }
  const float inv = gated_norm_inv(ss, d, eps);
  for (int i = lane; i < d; i += kWave) orow[i] = gated_norm_value<T>(xv(i), inv, to_f(w[i]), to_f(zr[i]));
}

}  // namespace mkq
