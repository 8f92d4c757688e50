// Small-batch GEMV y[b, n] = sum_k w[n, k] x[b, k] (+ residual[b, n]) for the
// projections of decode_layer.  x is staged in LDS as FP32; each wave streams
// whole weight rows with 128-bit loads.  The two-output form also writes
// sum[b, n] = residual[b, n] + y[b, n] with y rounded to T first, the same two
// roundings as a separate elementwise add.  The normalised form first turns
// the staged x into rms_norm(x) * norm_weight (FP32 statistics, the result
// rounded to T as reference.py:10-13 does), so an input RMSNorm and the
// projection after it are one launch.
#include "mkq_host.h"

using namespace mkq;

namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / kWave;
constexpr int kMaxNb = 4;
constexpr int kUnroll = 4;

template <typename T, int NB, bool VEC>
__global__ __launch_bounds__(kThreads) void gemv_kernel(const T* __restrict__ x, const T* __restrict__ w,
                                                        const T* __restrict__ residual, T* __restrict__ y,
                                                        T* __restrict__ sum, const T* __restrict__ nw, float eps,
                                                        int kdim, int n, int rows_per_wg) {
  constexpr int EPC = Epc<T>::value;
  extern __shared__ float xs[];  // [NB][kp], then the norm's partial sums [kWaves][NB]
  const int kp = (kdim + EPC - 1) / EPC * EPC;
  float* red = xs + NB * kp;
  const int lane = threadIdx.x % kWave, wave = wave_id();
  float ss[NB];
#pragma unroll
  for (int b = 0; b < NB; ++b) ss[b] = 0.f;
  for (int i = threadIdx.x; i < kp; i += kThreads)
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      const float v = i < kdim ? to_f(x[size_t(b) * kdim + i]) : 0.f;
      xs[b * kp + i] = v;
      ss[b] = fmaf(v, v, ss[b]);
    }
  if (nw != nullptr) {
    // Every workgroup normalises the whole of x itself (a few KB): no
    // hand-off between workgroups.
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      const float t = wave_sum(ss[b]);
      if (lane == 0) red[wave * NB + b] = t;
    }
    __syncthreads();
    float inv[NB];
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      float t = 0.f;
#pragma unroll
      for (int v = 0; v < kWaves; ++v) t += red[v * NB + b];
      inv[b] = 1.0f / sqrtf(t / float(kdim) + eps);
    }
    for (int i = threadIdx.x; i < kdim; i += kThreads) {
      const float g = to_f(nw[i]);
#pragma unroll
      for (int b = 0; b < NB; ++b) xs[b * kp + i] = to_f(from_f<T>(xs[b * kp + i] * inv[b] * g));
    }
  }
  __syncthreads();
  const int nch = kp / EPC;
  const int r0 = blockIdx.x * rows_per_wg, r1 = min(n, r0 + rows_per_wg);
  for (int r = r0 + wave; r < r1; r += kWaves) {
    const T* row = w + size_t(r) * kdim;
    float acc[NB];
#pragma unroll
    for (int b = 0; b < NB; ++b) acc[b] = 0.f;
    for (int j0 = lane; j0 < nch; j0 += kWave * kUnroll) {
      u32x4 c[kUnroll];
#pragma unroll
      for (int u = 0; u < kUnroll; ++u)
        if (j0 + u * kWave < nch) c[u] = load_chunk_nt<T, VEC>(row, j0 + u * kWave, kdim);
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) {
        const int j = j0 + u * kWave;
        if (j < nch) {
          float f[EPC];
          unpack(c[u], f, T{});
#pragma unroll
          for (int b = 0; b < NB; ++b)
#pragma unroll
            for (int e = 0; e < EPC; ++e) acc[b] = fmaf(f[e], xs[b * kp + j * EPC + e], acc[b]);
        }
      }
    }
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      const float s = wave_sum(acc[b]);
      if (lane == 0) {
        const size_t o = size_t(b) * n + r;
        if (sum) {
          const T yv = from_f<T>(s);
          y[o] = yv;
          sum[o] = from_f<T>(to_f(residual[o]) + to_f(yv));
        } else {
          y[o] = from_f<T>(residual ? s + to_f(residual[o]) : s);
        }
      }
    }
  }
}

template <typename T, int NB>
int launch(const T* x, const T* w, const T* residual, T* y, T* sum, const T* nw, float eps, int kdim, int n,
           hipStream_t stream) {
  constexpr int EPC = Epc<T>::value;
  const size_t lds = sizeof(float) * (NB * size_t((kdim + EPC - 1) / EPC * EPC) + kWaves * NB);
  if (lds > size_t(max_lds_per_block()))
    return set_error(MKQ_ERR_UNSUPPORTED, "gemv: in_features=%d too large for LDS staging", kdim);
  const bool vec = (kdim % EPC == 0) && aligned16(w);
  static bool attr_set = false;
  if (!attr_set) {
    MKQ_HIP_TRY(hipFuncSetAttribute(reinterpret_cast<const void*>(&gemv_kernel<T, NB, true>),
                                    hipFuncAttributeMaxDynamicSharedMemorySize, max_lds_per_block()));
    MKQ_HIP_TRY(hipFuncSetAttribute(reinterpret_cast<const void*>(&gemv_kernel<T, NB, false>),
                                    hipFuncAttributeMaxDynamicSharedMemorySize, max_lds_per_block()));
    attr_set = true;
  }
  const int rows = 2 * kWaves;
  const int grid = (n + rows - 1) / rows;
  if (vec)
    gemv_kernel<T, NB, true><<<grid, kThreads, lds, stream>>>(x, w, residual, y, sum, nw, eps, kdim, n, rows);
  else
    gemv_kernel<T, NB, false><<<grid, kThreads, lds, stream>>>(x, w, residual, y, sum, nw, eps, kdim, n, rows);
  MKQ_LAUNCH_CHECK("gemv_kernel");
  return MKQ_OK;
}

template <typename T>
int gemv_typed(const void* xv, const void* wv, const void* rv, void* yv, void* sv, const void* nv, float eps,
               int batch, int kdim, int n, hipStream_t stream) {
  const T* nw = static_cast<const T*>(nv);
  const T* x = static_cast<const T*>(xv);
  const T* w = static_cast<const T*>(wv);
  const T* r = static_cast<const T*>(rv);
  T* y = static_cast<T*>(yv);
  T* sm = static_cast<T*>(sv);
  for (int b0 = 0; b0 < batch; b0 += kMaxNb) {
    const int nb = batch - b0 < kMaxNb ? batch - b0 : kMaxNb;
    const T* xb = x + size_t(b0) * kdim;
    const T* rb = r ? r + size_t(b0) * n : nullptr;
    T* yb = y + size_t(b0) * n;
    T* sb = sm ? sm + size_t(b0) * n : nullptr;
    int rc;
    switch (nb) {
      case 1: rc = launch<T, 1>(xb, w, rb, yb, sb, nw, eps, kdim, n, stream); break;
      case 2: rc = launch<T, 2>(xb, w, rb, yb, sb, nw, eps, kdim, n, stream); break;
      case 3: rc = launch<T, 3>(xb, w, rb, yb, sb, nw, eps, kdim, n, stream); break;
      default: rc = launch<T, 4>(xb, w, rb, yb, sb, nw, eps, kdim, n, stream); break;
    }
    if (rc != MKQ_OK) return rc;
  }
  return MKQ_OK;
}

}  // namespace

static int gemv_dispatch(int dtype, const void* x, const void* w, const void* residual, void* y, void* sum,
                         const void* nw, float eps, int batch, int in_features, int out_features, hipStream_t s) {
  switch (dtype) {
    case MKQ_DTYPE_BF16:
      return gemv_typed<bf16_t>(x, w, residual, y, sum, nw, eps, batch, in_features, out_features, s);
    case MKQ_DTYPE_F16:
      return gemv_typed<f16_t>(x, w, residual, y, sum, nw, eps, batch, in_features, out_features, s);
    case MKQ_DTYPE_F32:
      return gemv_typed<float>(x, w, residual, y, sum, nw, eps, batch, in_features, out_features, s);
    default: return set_error(MKQ_ERR_INVALID, "gemv: unknown dtype %d", dtype);
  }
}

extern "C" int mkq_gemv(int dtype, const void* x, const void* w, const void* residual, void* y, int batch,
                        int in_features, int out_features, void* stream) {
  clear_error();
  MKQ_REQUIRE(batch > 0 && in_features > 0 && out_features > 0, "gemv: sizes must be positive");
  MKQ_REQUIRE(x && w && y, "gemv: null tensor pointer");
  return gemv_dispatch(dtype, x, w, residual, y, nullptr, nullptr, 0.f, batch, in_features, out_features,
                       static_cast<hipStream_t>(stream));
}

extern "C" int mkq_gemv_add(int dtype, const void* x, const void* w, const void* residual, void* y, void* sum,
                            int batch, int in_features, int out_features, void* stream) {
  clear_error();
  MKQ_REQUIRE(batch > 0 && in_features > 0 && out_features > 0, "gemv_add: sizes must be positive");
  MKQ_REQUIRE(x && w && residual && y && sum, "gemv_add: null tensor pointer");
  return gemv_dispatch(dtype, x, w, residual, y, sum, nullptr, 0.f, batch, in_features, out_features,
                       static_cast<hipStream_t>(stream));
}

extern "C" int mkq_rms_norm_gemv(int dtype, const void* x, const void* norm_weight, float eps, const void* w,
                                 void* y, int batch, int in_features, int out_features, void* stream) {
  clear_error();
  MKQ_REQUIRE(batch > 0 && in_features > 0 && out_features > 0, "rms_norm_gemv: sizes must be positive");
  MKQ_REQUIRE(x && norm_weight && w && y, "rms_norm_gemv: null tensor pointer");
  MKQ_REQUIRE(eps >= 0.f, "rms_norm_gemv: eps must be non-negative");
  return gemv_dispatch(dtype, x, w, nullptr, y, nullptr, norm_weight, eps, batch, in_features, out_features,
                       static_cast<hipStream_t>(stream));
}
