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

// Work items are (row, segment): a segment is up to 64 * CPL 16-byte chunks of
// a weight row, loaded as CPL chunks per lane through one buffer descriptor
// sized to the segment (chunks past it read as zero, with no branch), so all
// of an item's loads are in flight at once.  Each wave keeps two items in
// flight; the first two are issued before x is staged.  Segment partial sums
// meet in LDS and one thread per (batch row, output row) finishes, in a fixed
// order.
template <typename T, int NB, int CPL>
__global__ __launch_bounds__(kThreads) void gemv_kernel(const T* __restrict__ x, const T* __restrict__ w,
                                                        const T* __restrict__ residual, T* __restrict__ y,
                                                        T* __restrict__ sum, const T* __restrict__ nw, float eps,
                                                        int kdim, int n, int rows_per_wg) {
  constexpr int EPC = Epc<T>::value;
  constexpr int kSeg = kWave * CPL;  // chunks per segment
  extern __shared__ float smem[];    // x [NB][kp], norm partials [kWaves][NB], item sums [items][NB]
  const int kp = (kdim + EPC - 1) / EPC * EPC;
  const int nch = kp / EPC;
  const int nseg = (nch + kSeg - 1) / kSeg;
  float* xs = smem;
  float* red = xs + NB * kp;
  float* part = red + kWaves * NB;
  const int tid = threadIdx.x, lane = tid % kWave, wave = wave_id();
  const int r0 = blockIdx.x * rows_per_wg;
  const int nr = max(0, min(rows_per_wg, n - r0));
  const int nitems = nr * nseg;

  auto issue = [&](int item, u32x4 (&c)[CPL]) {
    const bool ok = item < nitems;
    const int it = ok ? item : 0;
    const int row = r0 + it / nseg, c0 = (it % nseg) * kSeg;
    const uint32_t bytes = ok ? uint32_t(min(kSeg, nch - c0)) * 16u : 0u;
    const rsrc_t rs = make_rsrc(w + size_t(row) * kdim + size_t(c0) * EPC, bytes);
#pragma unroll
    for (int j = 0; j < CPL; ++j) c[j] = buf_load16<kAuxStream>(rs, uint32_t(lane + kWave * j) * 16u);
  };
  u32x4 ca[CPL], cb[CPL];
  issue(wave, ca);
  issue(wave + kWaves, cb);
  pin_loads();

  // x -> LDS (FP32) with 16-byte loads, all of a thread's issued at once,
  // and its sum of squares for the optional norm.
  constexpr int kStage = 8;  // chunks per thread per pass (a pass covers kStage * 256 chunks)
  const int xch = nch;       // chunks per batch row
  const rsrc_t xr = make_rsrc(x, uint32_t(NB) * uint32_t(kdim) * uint32_t(sizeof(T)));
  float ss[NB];
#pragma unroll
  for (int b = 0; b < NB; ++b) ss[b] = 0.f;
  // With the norm, the first pass of x and of the norm weight is peeled off
  // its loop: at a loop header the compiler waits for every load in flight
  // (the weight rows above) before issuing the loop's loads, which
  // serialised x, then the norm weight, behind the weight rows (rms_norm_gemv
  // 2048 -> 8192: 10.3-10.7 -> 9.5-9.9 us cold).  Without the norm, peeling
  // measured no faster (out_proj 4096 -> 2048, within +-0.3 us).
  auto stage_x = [&](int f0) __attribute__((always_inline)) {
    u32x4 v[kStage];
#pragma unroll
    for (int r = 0; r < kStage; ++r) {
      const int f = f0 + r * kThreads;
      v[r] = buf_load16(xr, f < NB * xch ? uint32_t(f) * 16u : 0xFFFFFFF0u);
    }
#pragma unroll
    for (int r = 0; r < kStage; ++r) {
      const int f = f0 + r * kThreads;
      if (f < NB * xch) {
        const int b = f / xch, c = f % xch;
        float e[EPC];
        unpack(v[r], e, T{});
        float sq = 0.f;
        float4* dst = reinterpret_cast<float4*>(xs + b * kp + c * EPC);
#pragma unroll
        for (int h = 0; h < EPC / 4; ++h) {
          dst[h] = make_float4(e[4 * h], e[4 * h + 1], e[4 * h + 2], e[4 * h + 3]);
          sq = fmaf(e[4 * h], e[4 * h], sq);
          sq = fmaf(e[4 * h + 1], e[4 * h + 1], sq);
          sq = fmaf(e[4 * h + 2], e[4 * h + 2], sq);
          sq = fmaf(e[4 * h + 3], e[4 * h + 3], sq);
        }
#pragma unroll
        for (int bb = 0; bb < NB; ++bb) ss[bb] += bb == b ? sq : 0.f;
      }
    }
  };
  const int f_first = nw != nullptr ? tid + kStage * kThreads : tid;
  if (nw != nullptr) stage_x(tid);
  for (int f0 = f_first; f0 < NB * xch; f0 += kStage * kThreads) stage_x(f0);
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
    const rsrc_t nr = make_rsrc(nw, uint32_t(kdim) * uint32_t(sizeof(T)));
    auto norm_pass = [&](int c0) __attribute__((always_inline)) {
      u32x4 g[kStage];
#pragma unroll
      for (int r = 0; r < kStage; ++r) g[r] = buf_load16(nr, c0 + r * kThreads < xch ? uint32_t(c0 + r * kThreads) * 16u
                                                                                       : 0xFFFFFFF0u);
#pragma unroll
      for (int r = 0; r < kStage; ++r) {
        const int c = c0 + r * kThreads;
        if (c < xch) {
          float gf[EPC];
          unpack(g[r], gf, T{});
#pragma unroll
          for (int b = 0; b < NB; ++b)
#pragma unroll
            for (int e = 0; e < EPC; ++e) {
              float* px = xs + b * kp + c * EPC + e;
              *px = to_f(from_f<T>(*px * inv[b] * gf[e]));
            }
        }
      }
    };
    norm_pass(tid);
    for (int c0 = tid + kStage * kThreads; c0 < xch; c0 += kStage * kThreads) norm_pass(c0);
  }
  __syncthreads();

  auto consume = [&](int item, const u32x4 (&c)[CPL]) {
    if (item >= nitems) return;
    const int c0 = (item % nseg) * kSeg;
    const int last = nch - 1;
    float acc[NB];
#pragma unroll
    for (int b = 0; b < NB; ++b) acc[b] = 0.f;
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
      // chunks past the row were loaded as zero; pair them with a clamped
      // (finite) x position instead of branching
      const int q = min(c0 + lane + kWave * j, last);
      float f[EPC];
      unpack(c[j], f, T{});
#pragma unroll
      for (int b = 0; b < NB; ++b) {
        const float4* pv = reinterpret_cast<const float4*>(xs + b * kp + q * EPC);
#pragma unroll
        for (int h = 0; h < EPC / 4; ++h) {
          const float4 v = pv[h];
          acc[b] = fmaf(f[4 * h], v.x, acc[b]);
          acc[b] = fmaf(f[4 * h + 1], v.y, acc[b]);
          acc[b] = fmaf(f[4 * h + 2], v.z, acc[b]);
          acc[b] = fmaf(f[4 * h + 3], v.w, acc[b]);
        }
      }
    }
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      const float t = wave_sum_u(acc[b]);
      if (lane == 0) part[item * NB + b] = t;
    }
  };
  for (int it = wave; it < nitems; it += 2 * kWaves) {
    consume(it, ca);
    if (it + 2 * kWaves < nitems) issue(it + 2 * kWaves, ca);
    pin_loads();
    if (it + kWaves >= nitems) break;
    consume(it + kWaves, cb);
    if (it + 3 * kWaves < nitems) issue(it + 3 * kWaves, cb);
    pin_loads();
  }
  __syncthreads();
  for (int t = tid; t < nr * NB; t += kThreads) {
    const int rl = t / NB, b = t % NB;
    float s = 0.f;
    for (int g = 0; g < nseg; ++g) s += part[(rl * nseg + g) * NB + b];
    const size_t o = size_t(b) * n + r0 + rl;
    if (sum) {
      const T yv = from_f<T>(s);
      y[o] = yv;
      sum[o] = from_f<T>(to_f(residual[o]) + to_f(yv));
    } else {
      y[o] = from_f<T>(residual ? s + to_f(residual[o]) : s);
    }
  }
}

// Element-wise variant for rows that are not whole 16-byte chunks (or
// unaligned weights): one wave per row, any length.
template <typename T, int NB>
__global__ __launch_bounds__(kThreads) void gemv_scalar_kernel(const T* __restrict__ x, const T* __restrict__ w,
                                                               const T* __restrict__ residual, T* __restrict__ y,
                                                               T* __restrict__ sum, const T* __restrict__ nw,
                                                               float eps, int kdim, int n) {
  extern __shared__ float xs[];
  float* red = xs + NB * kdim;
  const int tid = threadIdx.x, lane = tid % kWave, wave = wave_id();
  float ss[NB];
#pragma unroll
  for (int b = 0; b < NB; ++b) ss[b] = 0.f;
  for (int i = tid; i < kdim; i += kThreads)
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      const float v = to_f(x[size_t(b) * kdim + i]);
      xs[b * kdim + i] = v;
      ss[b] = fmaf(v, v, ss[b]);
    }
  if (nw != nullptr) {
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
    for (int i = tid; i < kdim; i += kThreads) {
      const float g = to_f(nw[i]);
#pragma unroll
      for (int b = 0; b < NB; ++b) xs[b * kdim + i] = to_f(from_f<T>(xs[b * kdim + i] * inv[b] * g));
    }
  }
  __syncthreads();
  const int r = blockIdx.x * kWaves + wave;
  if (r >= n) return;
  float acc[NB];
#pragma unroll
  for (int b = 0; b < NB; ++b) acc[b] = 0.f;
  for (int i = lane; i < kdim; i += kWave) {
    const float f = to_f(w[size_t(r) * kdim + i]);
#pragma unroll
    for (int b = 0; b < NB; ++b) acc[b] = fmaf(f, xs[b * kdim + i], acc[b]);
  }
#pragma unroll
  for (int b = 0; b < NB; ++b) {
    const float s = wave_sum_u(acc[b]);
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

template <typename K>
int set_max_lds(K* kern, bool& done) {
  if (!done) {
    MKQ_HIP_TRY(hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize,
                                    max_lds_per_block()));
    done = true;
  }
  return MKQ_OK;
}

template <typename T, int NB>
int launch(const T* x, const T* w, const T* residual, T* y, T* sum, const T* nw, float eps, int kdim, int n,
           hipStream_t stream) {
  constexpr int EPC = Epc<T>::value;
  const bool vec = (kdim % EPC == 0) && aligned16(w) && aligned16(x) && (nw == nullptr || aligned16(nw));
  if (!vec) {
    const size_t lds = sizeof(float) * (size_t(NB) * kdim + kWaves * NB);
    if (lds > size_t(max_lds_per_block()))
      return set_error(MKQ_ERR_UNSUPPORTED, "gemv: in_features=%d too large for LDS staging", kdim);
    static bool attr = false;
    const int rc = set_max_lds(&gemv_scalar_kernel<T, NB>, attr);
    if (rc != MKQ_OK) return rc;
    gemv_scalar_kernel<T, NB><<<(n + kWaves - 1) / kWaves, kThreads, lds, stream>>>(x, w, residual, y, sum, nw, eps,
                                                                                    kdim, n);
    MKQ_LAUNCH_CHECK("gemv_scalar_kernel");
    return MKQ_OK;
  }
  const int nch = kdim / EPC;
  // 8 chunks per lane (8 KB of bf16 per item) for long rows, 4 for short ones.
  const bool wide = nch > 4 * kWave;
  const int seg = kWave * (wide ? 8 : 4);
  const int nseg = (nch + seg - 1) / seg;
  // About two workgroups per CU: each keeps 8 items in flight.
  const int ncu = cu_count();
  const int rows_per_wg = max(1, (n + 2 * ncu - 1) / (2 * ncu));
  const int grid = (n + rows_per_wg - 1) / rows_per_wg;
  const size_t lds = sizeof(float) * (size_t(NB) * kdim + kWaves * NB + size_t(rows_per_wg) * nseg * NB);
  if (lds > size_t(max_lds_per_block()))
    return set_error(MKQ_ERR_UNSUPPORTED, "gemv: in_features=%d too large for LDS staging", kdim);
  if (wide) {
    static bool attr = false;
    const int rc = set_max_lds(&gemv_kernel<T, NB, 8>, attr);
    if (rc != MKQ_OK) return rc;
    gemv_kernel<T, NB, 8><<<grid, kThreads, lds, stream>>>(x, w, residual, y, sum, nw, eps, kdim, n, rows_per_wg);
  } else {
    static bool attr = false;
    const int rc = set_max_lds(&gemv_kernel<T, NB, 4>, attr);
    if (rc != MKQ_OK) return rc;
    gemv_kernel<T, NB, 4><<<grid, kThreads, lds, stream>>>(x, w, residual, y, sum, nw, eps, kdim, n, rows_per_wg);
  }
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
