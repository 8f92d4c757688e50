// The element-wise ops around the gated delta recurrence in the Qwen3.6
// linear-attention decode step (the model's causal_conv1d_update and
// RMSNormGated), for gfx950.
//
// causal_conv1d_update: depthwise causal convolution of one new token per
// channel, width S + 1 (4 in Qwen3.6), with the S previous inputs kept in
// conv_state [B, C, S]:
//     win = [state[b, c, 0..S-1], x[b, c]]
//     out[b, c] = act(sum_t w[c, t] * win[t] + bias[c]);  state[b, c] <- win[1..S]
// The sum is rounded to T before the activation and the activation's result
// again, as a T-typed convolution followed by a T-typed SiLU round them.
//
// gated_rms_norm (norm before gate): per row of D values
//     n = T(x * rsqrt(mean(x^2) + eps));  t = T(w * n);  out = T(t * silu(z))
// with the mean and rsqrt in FP32, the roundings of the model's module.
//
// Both are a few KB per step: latency-bound single launches.
#include "linear_common.h"
#include "mkq_host.h"

using namespace mkq;

namespace {

constexpr int kThreads = 256;

// grid: (ceil(C / 256), B); one thread per (b, c).
template <typename T>
__global__ __launch_bounds__(kThreads) void conv1d_update_kernel(const T* __restrict__ x, T* __restrict__ conv_state,
                                                                 const T* __restrict__ w, const T* __restrict__ bias,
                                                                 T* __restrict__ out, int c_dim, int s_len,
                                                                 int silu_act) {
  const int c = blockIdx.x * kThreads + threadIdx.x;
  const int b = blockIdx.y;
  if (c >= c_dim) return;
  const size_t row = size_t(b) * c_dim + c;
  T* st = conv_state + row * s_len;
  const T* wc = w + size_t(c) * (s_len + 1);
  // Fully unrolled over the maximum width so the window stays in registers.
  const float xv = to_f(x[row]);
  float win[kMaxConvTaps], wv[kMaxConvTaps];
#pragma unroll
  for (int t = 0; t < kMaxConvTaps; ++t) {
    win[t] = t < s_len ? to_f(st[t]) : (t == s_len ? xv : 0.f);
    wv[t] = t <= s_len ? to_f(wc[t]) : 0.f;
  }
  const float y = conv_channel<T, kMaxConvTaps>(win, wv, bias ? to_f(bias[c]) : 0.f, s_len, silu_act != 0);
#pragma unroll
  for (int t = 0; t + 1 < kMaxConvTaps; ++t)
    if (t < s_len) st[t] = from_f<T>(win[t + 1]);
  out[row] = from_f<T>(y);
}

// grid: (ceil(rows / 4)); block 256, one wave per row.
template <typename T>
__global__ __launch_bounds__(kThreads) void gated_rms_norm_kernel(const T* __restrict__ x, const T* __restrict__ z,
                                                                  const T* __restrict__ w, T* __restrict__ out,
                                                                  int rows, int d, float eps) {
  const int lane = threadIdx.x % kWave;
  const int r = blockIdx.x * (kThreads / kWave) + wave_id();
  if (r >= rows) return;  // wave-uniform
  const T* xr = x + size_t(r) * d;
  gated_norm_row<T>([&](int i) { return to_f(xr[i]); }, z + size_t(r) * d, w, out + size_t(r) * d, d, eps, lane);
}

template <typename T>
int conv_typed(const void* x, void* st, const void* w, const void* bias, void* out, int batch, int c_dim, int s_len,
               int act, hipStream_t stream) {
  dim3 grid((c_dim + kThreads - 1) / kThreads, batch);
  conv1d_update_kernel<T><<<grid, kThreads, 0, stream>>>(static_cast<const T*>(x), static_cast<T*>(st),
                                                         static_cast<const T*>(w), static_cast<const T*>(bias),
                                                         static_cast<T*>(out), c_dim, s_len, act);
  MKQ_LAUNCH_CHECK("conv1d_update_kernel");
  return MKQ_OK;
}

template <typename T>
int norm_typed(const void* x, const void* z, const void* w, void* out, int rows, int d, float eps,
               hipStream_t stream) {
  const int per = kThreads / kWave;
  gated_rms_norm_kernel<T><<<(rows + per - 1) / per, kThreads, 0, stream>>>(
      static_cast<const T*>(x), static_cast<const T*>(z), static_cast<const T*>(w), static_cast<T*>(out), rows, d,
      eps);
  MKQ_LAUNCH_CHECK("gated_rms_norm_kernel");
  return MKQ_OK;
}

}  // namespace

extern "C" int mkq_causal_conv1d_update(int dtype, const void* x, void* conv_state, const void* weight,
                                        const void* bias, void* out, int batch, int channels, int state_len,
                                        int silu_activation, void* stream) {
  clear_error();
  MKQ_REQUIRE(batch > 0 && channels > 0 && state_len > 0, "causal_conv1d_update: sizes must be positive");
  MKQ_REQUIRE(state_len < kMaxConvTaps, "causal_conv1d_update: state_len %d > %d", state_len, kMaxConvTaps - 1);
  MKQ_REQUIRE(batch <= 65535, "causal_conv1d_update: batch too large");
  MKQ_REQUIRE(x && conv_state && weight && out, "causal_conv1d_update: null tensor pointer");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int act = silu_activation ? 1 : 0;
  switch (dtype) {
    case MKQ_DTYPE_BF16: return conv_typed<bf16_t>(x, conv_state, weight, bias, out, batch, channels, state_len, act, s);
    case MKQ_DTYPE_F16: return conv_typed<f16_t>(x, conv_state, weight, bias, out, batch, channels, state_len, act, s);
    case MKQ_DTYPE_F32: return conv_typed<float>(x, conv_state, weight, bias, out, batch, channels, state_len, act, s);
    default: return set_error(MKQ_ERR_INVALID, "causal_conv1d_update: unknown dtype %d", dtype);
  }
}

extern "C" int mkq_gated_rms_norm(int dtype, const void* x, const void* gate, const void* weight, void* out,
                                  int rows, int dim, float eps, void* stream) {
  clear_error();
  MKQ_REQUIRE(rows > 0 && dim > 0, "gated_rms_norm: sizes must be positive");
  MKQ_REQUIRE(x && gate && weight && out, "gated_rms_norm: null tensor pointer");
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (dtype) {
    case MKQ_DTYPE_BF16: return norm_typed<bf16_t>(x, gate, weight, out, rows, dim, eps, s);
    case MKQ_DTYPE_F16: return norm_typed<f16_t>(x, gate, weight, out, rows, dim, eps, s);
    case MKQ_DTYPE_F32: return norm_typed<float>(x, gate, weight, out, rows, dim, eps, s);
    default: return set_error(MKQ_ERR_INVALID, "gated_rms_norm: unknown dtype %d", dtype);
  }
}
