// Dense SwiGLU FFN decode for gfx950.
//
//   x_norm = x * rsqrt(mean(x^2) + eps) * norm_weight          (FP32)
//   act    = silu(x_norm . gate_row) * (x_norm . up_row)       (FP32, workspace)
//   out    = act . down_row (+ x)                              (rounded to dtype)
//
// Semantics of reference.py:65-88 (dense_ffn_decode_reference); replaces the
// torch composite of ops.py:202-218.  Two launches:
//   K1 ffn_gateup_kernel : RMSNorm fused into the gate/up GEMVs + SwiGLU.
//                          Each workgroup recomputes the norm (x is a few KB,
//                          read from L2), keeps x_norm in LDS as FP32 and its
//                          waves stream gate/up row pairs with 128-bit loads.
//   K2 ffn_down_kernel   : the whole act vector is staged once per workgroup
//                          in LDS; all 256 threads split each group of rows
//                          along K, so a workgroup's share of the weight matrix
//                          is read with full-width coalesced loads.
// Both kernels are HBM-bound GEMVs (every weight byte is read exactly once).
#include "mkq_host.h"

using namespace mkq;

namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / kWave;
constexpr int kUnroll = 4;       // 128-bit loads in flight per matrix per lane (K1)
constexpr int kDownRows = 4;     // rows processed together in K2
constexpr int kMaxBatchPerLaunch = 2;

__host__ __device__ inline int round_up(int a, int b) { return (a + b - 1) / b * b; }

// Writes x_norm = x * inv_rms * nw for NB rows into lds_xn ([NB][hp] FP32,
// zero-padded from h to hp).  lds_red needs kWaves*NB floats.
template <typename T, int NB>
__device__ void stage_xnorm(const T* __restrict__ x, const T* __restrict__ nw, int h, int hp, float eps,
                            float* lds_xn, float* lds_red) {
  const int tid = threadIdx.x, lane = tid % kWave, wave = tid / kWave;
  float ss[NB];
#pragma unroll
  for (int b = 0; b < NB; ++b) ss[b] = 0.f;
  for (int k = tid; k < hp; k += kThreads) {
    const float w = k < h ? to_f(nw[k]) : 0.f;
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      const float v = k < h ? to_f(x[size_t(b) * h + k]) : 0.f;
      ss[b] += v * v;
      lds_xn[b * hp + k] = v * w;
    }
  }
#pragma unroll
  for (int b = 0; b < NB; ++b) {
    ss[b] = wave_sum(ss[b]);
    if (lane == 0) lds_red[wave * NB + b] = ss[b];
  }
  __syncthreads();
  float inv[NB];
#pragma unroll
  for (int b = 0; b < NB; ++b) {
    float t = 0.f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) t += lds_red[w * NB + b];
    inv[b] = 1.0f / sqrtf(t / float(h) + eps);
  }
  for (int k = tid; k < hp; k += kThreads) {
#pragma unroll
    for (int b = 0; b < NB; ++b) lds_xn[b * hp + k] *= inv[b];
  }
  __syncthreads();
}

// dot of one 16-byte weight chunk (EPC elements) with EPC FP32 values in LDS.
template <typename T>
__device__ __forceinline__ float chunk_dot(const u32x4& c, const float* __restrict__ xv) {
  constexpr int EPC = Epc<T>::value;
  float f[EPC];
  unpack(c, f, T{});
  float s = 0.f;
  if constexpr (EPC == 8) {
    const float4 a = *reinterpret_cast<const float4*>(xv);
    const float4 b = *reinterpret_cast<const float4*>(xv + 4);
    s = f[0] * a.x;
    s = fmaf(f[1], a.y, s);
    s = fmaf(f[2], a.z, s);
    s = fmaf(f[3], a.w, s);
    s = fmaf(f[4], b.x, s);
    s = fmaf(f[5], b.y, s);
    s = fmaf(f[6], b.z, s);
    s = fmaf(f[7], b.w, s);
  } else {
    const float4 a = *reinterpret_cast<const float4*>(xv);
    s = f[0] * a.x;
    s = fmaf(f[1], a.y, s);
    s = fmaf(f[2], a.z, s);
    s = fmaf(f[3], a.w, s);
  }
  return s;
}

// K1: grid.x = ceil(I / rows_per_wg); block = 256.
// LDS: NB*hp floats (x_norm) + kWaves*NB floats.
template <typename T, int NB, bool VEC>
__global__ __launch_bounds__(kThreads) void ffn_gateup_kernel(const T* __restrict__ x, const T* __restrict__ nw,
                                                              const T* __restrict__ wg, const T* __restrict__ wu,
                                                              float* __restrict__ act, int h, int inter, float eps,
                                                              int rows_per_wg, int act_ld) {
  constexpr int EPC = Epc<T>::value;
  extern __shared__ float smem[];
  const int hp = round_up(h, EPC);
  float* xn = smem;
  float* red = smem + NB * hp;
  stage_xnorm<T, NB>(x, nw, h, hp, eps, xn, red);

  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
  const int nch = hp / EPC;
  const int r0 = blockIdx.x * rows_per_wg;
  const int r1 = min(inter, r0 + rows_per_wg);
  for (int r = r0 + wave; r < r1; r += kWaves) {
    const T* grow = wg + size_t(r) * h;
    const T* urow = wu + size_t(r) * h;
    float ag[NB], au[NB];
#pragma unroll
    for (int b = 0; b < NB; ++b) ag[b] = au[b] = 0.f;
    for (int j0 = lane; j0 < nch; j0 += kWave * kUnroll) {
      u32x4 cg[kUnroll], cu[kUnroll];
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) {
        const int j = j0 + u * kWave;
        if (j < nch) {
          cg[u] = load_chunk_nt<T, VEC>(grow, j, h);
          cu[u] = load_chunk_nt<T, VEC>(urow, j, h);
        }
      }
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) {
        const int j = j0 + u * kWave;
        if (j < nch) {
#pragma unroll
          for (int b = 0; b < NB; ++b) {
            const float* xv = xn + b * hp + j * EPC;
            ag[b] += chunk_dot<T>(cg[u], xv);
            au[b] += chunk_dot<T>(cu[u], xv);
          }
        }
      }
    }
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      const float g = wave_sum(ag[b]);
      const float u = wave_sum(au[b]);
      if (lane == 0) act[size_t(b) * act_ld + r] = silu(g) * u;
    }
  }
}

// K2: grid.x = ceil(H / rows_per_wg); block = 256.
// LDS: NB*ip floats (act) + 2*kWaves*kDownRows*NB floats.
template <typename T, int NB, bool VEC>
__global__ __launch_bounds__(kThreads) void ffn_down_kernel(const float* __restrict__ act, const T* __restrict__ wd,
                                                            const T* __restrict__ x, T* __restrict__ out, int h,
                                                            int inter, int add_residual, int rows_per_wg,
                                                            int act_ld) {
  constexpr int EPC = Epc<T>::value;
  extern __shared__ float smem[];
  const int ip = round_up(inter, EPC);
  float* a = smem;
  float* red = smem + NB * ip;
  const int tid = threadIdx.x, lane = tid % kWave, wave = tid / kWave;
  for (int k = tid; k < ip; k += kThreads) {
#pragma unroll
    for (int b = 0; b < NB; ++b) a[b * ip + k] = k < inter ? act[size_t(b) * act_ld + k] : 0.f;
  }
  __syncthreads();

  const int nch = ip / EPC;
  const int r0 = blockIdx.x * rows_per_wg;
  const int r1 = min(h, r0 + rows_per_wg);
  int parity = 0;
  for (int rg = r0; rg < r1; rg += kDownRows, parity ^= 1) {
    const int nr = min(kDownRows, r1 - rg);
    float acc[kDownRows][NB];
#pragma unroll
    for (int i = 0; i < kDownRows; ++i)
#pragma unroll
      for (int b = 0; b < NB; ++b) acc[i][b] = 0.f;
    for (int j0 = tid; j0 < nch; j0 += kThreads * 2) {
      u32x4 c[2][kDownRows];
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const int j = j0 + u * kThreads;
#pragma unroll
        for (int i = 0; i < kDownRows; ++i)
          if (i < nr && j < nch) c[u][i] = load_chunk_nt<T, VEC>(wd + size_t(rg + i) * inter, j, inter);
      }
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const int j = j0 + u * kThreads;
        if (j < nch) {
#pragma unroll
          for (int i = 0; i < kDownRows; ++i)
            if (i < nr) {
#pragma unroll
              for (int b = 0; b < NB; ++b) acc[i][b] += chunk_dot<T>(c[u][i], a + b * ip + j * EPC);
            }
        }
      }
    }
    float* rb = red + parity * (kWaves * kDownRows * NB);
#pragma unroll
    for (int i = 0; i < kDownRows; ++i)
#pragma unroll
      for (int b = 0; b < NB; ++b) {
        const float s = wave_sum(acc[i][b]);
        if (lane == 0) rb[(wave * kDownRows + i) * NB + b] = s;
      }
    __syncthreads();
    if (tid < nr * NB) {
      const int i = tid / NB, b = tid % NB;
      float s = 0.f;
#pragma unroll
      for (int w = 0; w < kWaves; ++w) s += rb[(w * kDownRows + i) * NB + b];
      const size_t o = size_t(b) * h + rg + i;
      if (add_residual) s += to_f(x[o]);
      out[o] = from_f<T>(s);
    }
    // The next group writes the other half of `red`, so one barrier per group
    // suffices: a wave can only reach this group's slot again after the
    // barrier of the following group.
  }
}

template <typename T, int NB, bool VEC>
int launch_nb(const T* x, const T* nw, const T* wg, const T* wu, const T* wd, T* out, int h, int inter, float eps,
              int add_residual, float* act, hipStream_t stream) {
  constexpr int EPC = Epc<T>::value;
  const int ncu = cu_count();
  const int max_lds = max_lds_per_block();
  const int hp = round_up(h, EPC), ip = round_up(inter, EPC);

  const size_t lds1 = sizeof(float) * (size_t(NB) * hp + kWaves * NB);
  const size_t lds2 = sizeof(float) * (size_t(NB) * ip + 2 * kWaves * kDownRows * NB);
  if (lds1 > size_t(max_lds) || lds2 > size_t(max_lds))
    return set_error(MKQ_ERR_UNSUPPORTED, "dense_ffn_decode: hidden=%d / intermediate=%d too large for LDS staging", h,
                     inter);
  static bool attr_set = false;
  if (!attr_set) {
    MKQ_HIP_TRY(hipFuncSetAttribute(reinterpret_cast<const void*>(&ffn_gateup_kernel<T, NB, VEC>),
                                    hipFuncAttributeMaxDynamicSharedMemorySize, max_lds));
    MKQ_HIP_TRY(hipFuncSetAttribute(reinterpret_cast<const void*>(&ffn_down_kernel<T, NB, VEC>),
                                    hipFuncAttributeMaxDynamicSharedMemorySize, max_lds));
    attr_set = true;
  }

  // K1: 4 rows per wave -> 16 gate/up row pairs per workgroup.
  const int rows1 = 4 * kWaves;
  const int grid1 = (inter + rows1 - 1) / rows1;
  ffn_gateup_kernel<T, NB, VEC><<<grid1, kThreads, lds1, stream>>>(x, nw, wg, wu, act, h, inter, eps, rows1, inter);
  MKQ_LAUNCH_CHECK("ffn_gateup_kernel");

  // K2: two workgroups per CU, rows split evenly.
  int grid2 = 2 * ncu;
  int rows2 = (h + grid2 - 1) / grid2;
  if (rows2 < 1) rows2 = 1;
  grid2 = (h + rows2 - 1) / rows2;
  ffn_down_kernel<T, NB, VEC><<<grid2, kThreads, lds2, stream>>>(act, wd, x, out, h, inter, add_residual, rows2, inter);
  MKQ_LAUNCH_CHECK("ffn_down_kernel");
  return MKQ_OK;
}

template <typename T>
int dense_ffn_typed(const void* xv, const void* nwv, const void* gv, const void* uv, const void* dv, void* outv,
                    int batch, int h, int inter, float eps, int add_residual, float* act, hipStream_t stream) {
  constexpr int EPC = Epc<T>::value;
  const T* x = static_cast<const T*>(xv);
  const T* nw = static_cast<const T*>(nwv);
  const T* wg = static_cast<const T*>(gv);
  const T* wu = static_cast<const T*>(uv);
  const T* wd = static_cast<const T*>(dv);
  T* out = static_cast<T*>(outv);
  const bool vec = (h % EPC == 0) && (inter % EPC == 0) && aligned16(wg) && aligned16(wu) && aligned16(wd);
  for (int b0 = 0; b0 < batch; b0 += kMaxBatchPerLaunch) {
    const int nb = batch - b0 >= 2 ? 2 : 1;
    const T* xb = x + size_t(b0) * h;
    T* ob = out + size_t(b0) * h;
    float* ab = act + size_t(b0) * inter;
    int rc;
    if (nb == 2)
      rc = vec ? launch_nb<T, 2, true>(xb, nw, wg, wu, wd, ob, h, inter, eps, add_residual, ab, stream)
               : launch_nb<T, 2, false>(xb, nw, wg, wu, wd, ob, h, inter, eps, add_residual, ab, stream);
    else
      rc = vec ? launch_nb<T, 1, true>(xb, nw, wg, wu, wd, ob, h, inter, eps, add_residual, ab, stream)
               : launch_nb<T, 1, false>(xb, nw, wg, wu, wd, ob, h, inter, eps, add_residual, ab, stream);
    if (rc != MKQ_OK) return rc;
  }
  return MKQ_OK;
}

}  // namespace

extern "C" size_t mkq_dense_ffn_decode_workspace_bytes(int batch, int hidden, int intermediate) {
  (void)hidden;
  if (batch <= 0 || intermediate <= 0) return 0;
  return sizeof(float) * size_t(batch) * size_t(intermediate);
}

extern "C" int mkq_dense_ffn_decode(int dtype, const void* x, const void* norm_weight, const void* gate_weight,
                                    const void* up_weight, const void* down_weight, void* out, int batch, int hidden,
                                    int intermediate, float eps, int add_residual, void* workspace,
                                    size_t workspace_bytes, void* stream) {
  clear_error();
  MKQ_REQUIRE(batch > 0 && hidden > 0 && intermediate > 0, "dense_ffn_decode: sizes must be positive");
  MKQ_REQUIRE(x && norm_weight && gate_weight && up_weight && down_weight && out,
              "dense_ffn_decode: null tensor pointer");
  MKQ_REQUIRE(workspace && workspace_bytes >= mkq_dense_ffn_decode_workspace_bytes(batch, hidden, intermediate),
              "dense_ffn_decode: workspace too small");
  hipStream_t s = static_cast<hipStream_t>(stream);
  float* act = static_cast<float*>(workspace);
  switch (dtype) {
    case MKQ_DTYPE_BF16:
      return dense_ffn_typed<bf16_t>(x, norm_weight, gate_weight, up_weight, down_weight, out, batch, hidden,
                                     intermediate, eps, add_residual, act, s);
    case MKQ_DTYPE_F16:
      return dense_ffn_typed<f16_t>(x, norm_weight, gate_weight, up_weight, down_weight, out, batch, hidden,
                                    intermediate, eps, add_residual, act, s);
    case MKQ_DTYPE_F32:
      return dense_ffn_typed<float>(x, norm_weight, gate_weight, up_weight, down_weight, out, batch, hidden,
                                    intermediate, eps, add_residual, act, s);
    default:
      return set_error(MKQ_ERR_INVALID, "dense_ffn_decode: unknown dtype %d", dtype);
  }
}
