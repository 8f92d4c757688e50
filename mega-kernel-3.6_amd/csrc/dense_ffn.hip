// Dense SwiGLU FFN decode for gfx950.
//
//   x_norm = x * rsqrt(mean(x^2) + eps) * norm_weight          (FP32)
//   act    = silu(x_norm . gate_row) * (x_norm . up_row)       (FP32, workspace)
//   out    = act . down_row (+ x)                              (rounded to dtype)
//
// Semantics of reference.py:65-88 (dense_ffn_decode_reference); replaces the
// torch composite of ops.py:202-218.  Two launches, both HBM-bound GEMVs that
// read every weight byte exactly once:
//
//   K1 ffn_gateup_kernel: about two workgroups per CU, each owning a
//      contiguous block of intermediate rows; the workgroup computes the
//      RMSNorm once (x is a few KB, served from L2) into LDS as FP32, and its
//      waves stream (row, gate|up) items.  An item is CPL 16-byte chunks per
//      lane loaded through one buffer descriptor per row (no branches, all
//      loads in flight at once); two items per wave are always in flight.
//   K2 ffn_down_kernel: a workgroup owns a contiguous block of output rows;
//      the work items are (row, quarter of the row), so every wave gets the
//      same number of items.  The first items' weight loads are issued before
//      the act vector is staged in LDS, the quarter sums meet in LDS, and one
//      barrier finishes the block.
#include "mkq_host.h"

using namespace mkq;

namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / kWave;
constexpr int kQuarters = 4;       // K2 items per row
constexpr int kMaxBatchPerLaunch = 2;

__host__ __device__ inline int round_up(int a, int b) { return (a + b - 1) / b * b; }

// dot of the lane's chunks (chunk j = first + lane + 64 j of a vector segment)
// with FP32 values in LDS; chunks past the segment were loaded as zero and
// are paired with a clamped (finite) LDS position, so no branch is needed.
template <typename T, int CPL>
__device__ __forceinline__ float chunks_dot(const u32x4 (&c)[CPL], const float* __restrict__ v, int first, int last,
                                            int lane) {
  constexpr int EPC = Epc<T>::value;
  float s = 0.f;
#pragma unroll
  for (int j = 0; j < CPL; ++j) {
    const int q = min(first + lane + kWave * j, last);
    float f[EPC];
    unpack(c[j], f, T{});
    const float4* p = reinterpret_cast<const float4*>(v + q * EPC);
    if constexpr (EPC == 8) {
      const float4 a = p[0], b = p[1];
      s = fmaf(f[0], a.x, s);
      s = fmaf(f[1], a.y, s);
      s = fmaf(f[2], a.z, s);
      s = fmaf(f[3], a.w, s);
      s = fmaf(f[4], b.x, s);
      s = fmaf(f[5], b.y, s);
      s = fmaf(f[6], b.z, s);
      s = fmaf(f[7], b.w, s);
    } else {
      const float4 a = p[0];
      s = fmaf(f[0], a.x, s);
      s = fmaf(f[1], a.y, s);
      s = fmaf(f[2], a.z, s);
      s = fmaf(f[3], a.w, s);
    }
  }
  return s;
}

template <typename T, int CPL>
__device__ __forceinline__ void load_seg(rsrc_t r, int lane, u32x4 (&c)[CPL]) {
#pragma unroll
  for (int j = 0; j < CPL; ++j) c[j] = buf_load16<kAuxStream>(r, uint32_t(lane + kWave * j) * 16u);
}

// Element loads for rows that are not 16-byte granular.
template <typename T, int CPL>
__device__ __forceinline__ void load_seg_scalar(const T* row, int n, int first, int lane, u32x4 (&c)[CPL]) {
#pragma unroll
  for (int j = 0; j < CPL; ++j) c[j] = load_chunk<T, false>(row, first + lane + kWave * j, n);
}

// Writes x_norm = x * inv_rms * nw for NB rows into lds_xn ([NB][hp] FP32,
// zero-padded from h to hp).  lds_red needs kWaves*NB floats.  Vector path:
// 16-byte buffer loads, kNormUnroll per thread issued together.
constexpr int kNormUnroll = 4;
template <typename T, int NB, bool VEC>
__device__ void stage_xnorm(const T* __restrict__ x, const T* __restrict__ nw, int h, int hp, float eps,
                            float* lds_xn, float* lds_red) {
  constexpr int EPC = Epc<T>::value;
  const int tid = threadIdx.x, lane = tid % kWave, wave = wave_id();
  float ss[NB];
#pragma unroll
  for (int b = 0; b < NB; ++b) ss[b] = 0.f;
  if constexpr (VEC) {
    const int hq = hp / EPC;
    const rsrc_t nr = make_rsrc(nw, uint32_t(h) * uint32_t(sizeof(T)));
    for (int q0 = tid; q0 < hq; q0 += kNormUnroll * kThreads) {
      u32x4 nc[kNormUnroll], xc[NB][kNormUnroll];
#pragma unroll
      for (int r = 0; r < kNormUnroll; ++r) {
        const uint32_t off = uint32_t(q0 + r * kThreads) * 16u;
        nc[r] = buf_load16(nr, off);
#pragma unroll
        for (int b = 0; b < NB; ++b)
          xc[b][r] = buf_load16(make_rsrc(x + size_t(b) * h, uint32_t(h) * uint32_t(sizeof(T))), off);
      }
#pragma unroll
      for (int r = 0; r < kNormUnroll; ++r) {
        const int q = q0 + r * kThreads;
        if (q < hq) {
          float nf[EPC];
          unpack(nc[r], nf, T{});
#pragma unroll
          for (int b = 0; b < NB; ++b) {
            float xf[EPC];
            unpack(xc[b][r], xf, T{});
#pragma unroll
            for (int e = 0; e < EPC; ++e) {
              ss[b] = fmaf(xf[e], xf[e], ss[b]);
              lds_xn[b * hp + q * EPC + e] = xf[e] * nf[e];
            }
          }
        }
      }
    }
  } else {
    for (int k = tid; k < hp; k += kThreads) {
      const float w = k < h ? to_f(nw[k]) : 0.f;
#pragma unroll
      for (int b = 0; b < NB; ++b) {
        const float v = k < h ? to_f(x[size_t(b) * h + k]) : 0.f;
        ss[b] = fmaf(v, v, ss[b]);
        lds_xn[b * hp + k] = v * w;
      }
    }
  }
#pragma unroll
  for (int b = 0; b < NB; ++b) {
    ss[b] = wave_sum_u(ss[b]);
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

// K1: grid.x = ceil(I / rows_per_wg); block = 256.  A workgroup owns a
// contiguous block of intermediate rows; the work items are (row, gate|up),
// so every wave gets the same number of items.  Two items per wave are in
// flight before the norm is computed, and each finished item is replaced by
// the one two steps ahead.
// LDS: NB*hp floats (x_norm) + kWaves*NB floats + 2*rows_per_wg*NB floats.
template <typename T, int NB, bool VEC, int CPL>
__global__ __launch_bounds__(kThreads) void ffn_gateup_kernel(const T* __restrict__ x, const T* __restrict__ nw,
                                                              const T* __restrict__ wg, const T* __restrict__ wu,
                                                              float* __restrict__ act, int h, int inter, float eps,
                                                              int act_ld, int rows_per_wg) {
  constexpr int EPC = Epc<T>::value;
  extern __shared__ float smem[];
  const int hp = round_up(h, EPC);
  const int lane = threadIdx.x % kWave, wave = wave_id();
  const int last = hp / EPC - 1;
  const int rb = blockIdx.x * rows_per_wg;
  const int nr = min(rows_per_wg, inter - rb);
  const int nitems = 2 * nr;
  const uint32_t row_bytes = uint32_t(h) * uint32_t(sizeof(T));

  u32x4 ca[CPL], cb[CPL];
  auto issue = [&](int item, u32x4 (&c)[CPL]) {
    const bool ok = item < nitems;
    const int it = ok ? item : 0;
    const T* w = (it & 1) ? wu : wg;
    const int row = rb + (it >> 1);  // always a real row
    if constexpr (VEC) {
      load_seg<T, CPL>(make_rsrc(w + size_t(row) * h, ok ? row_bytes : 0u), lane, c);
    } else {
      load_seg_scalar<T, CPL>(w + size_t(row) * h, h, 0, lane, c);
    }
  };
  issue(wave, ca);
  issue(wave + kWaves, cb);
  pin_loads();

  float* xn = smem;
  float* red = smem + NB * hp;
  float* part = red + kWaves * NB;
  stage_xnorm<T, NB, VEC>(x, nw, h, hp, eps, xn, red);

  auto finish = [&](int item, const u32x4 (&c)[CPL]) {
    if (item >= nitems) return;
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      const float s = wave_sum_u(chunks_dot<T, CPL>(c, xn + b * hp, 0, last, lane));
      if (lane == 0) part[item * NB + b] = s;
    }
  };
  for (int item = wave; item < nitems; item += 2 * kWaves) {
    finish(item, ca);
    issue(item + 2 * kWaves, ca);
    pin_loads();
    finish(item + kWaves, cb);
    issue(item + 3 * kWaves, cb);
    pin_loads();
  }
  __syncthreads();
  for (int t = threadIdx.x; t < nr * NB; t += kThreads) {
    const int i = t / NB, b = t % NB;
    act[size_t(b) * act_ld + rb + i] = silu(part[2 * i * NB + b]) * part[(2 * i + 1) * NB + b];
  }
}

// K2: grid.x = ceil(H / rows_per_wg); block = 256.
// LDS: NB*ip floats (act) + rows_per_wg*kQuarters*NB floats (quarter sums).
template <typename T, int NB, bool VEC, int CPL>
__global__ __launch_bounds__(kThreads) void ffn_down_kernel(const float* __restrict__ act, const T* __restrict__ wd,
                                                            const T* __restrict__ x, T* __restrict__ out, int h,
                                                            int inter, int add_residual, int rows_per_wg,
                                                            int act_ld) {
  constexpr int EPC = Epc<T>::value;
  extern __shared__ float smem[];
  const int ip = round_up(inter, EPC);
  const int nch = ip / EPC;                          // chunks per row
  const int qch = (nch + kQuarters - 1) / kQuarters;  // chunks per quarter (last one may be shorter)
  float* a = smem;
  float* part = smem + NB * ip;
  const int tid = threadIdx.x, lane = tid % kWave, wave = wave_id();
  const int rb = blockIdx.x * rows_per_wg;
  const int nr = min(rows_per_wg, h - rb);
  const int nitems = nr * kQuarters;

  u32x4 ca[CPL], cb[CPL];
  auto issue = [&](int item, u32x4 (&c)[CPL]) {
    const bool ok = item < nitems;
    const int it = ok ? item : 0;
    const int row = rb + it / kQuarters, qt = it % kQuarters;
    const int c0 = qt * qch;
    const int cnt = max(0, min(qch, nch - c0));
    if constexpr (VEC) {
      load_seg<T, CPL>(make_rsrc(wd + size_t(row) * inter + size_t(c0) * EPC, ok ? uint32_t(cnt) * 16u : 0u), lane,
                       c);
    } else {
      // positions past the quarter read as zero via the element bound
      const int n_lim = min(inter, (c0 + cnt) * EPC);
#pragma unroll
      for (int j = 0; j < CPL; ++j) c[j] = ok ? load_chunk<T, false>(wd + size_t(row) * inter, c0 + lane + kWave * j, n_lim)
                                              : u32x4{0u, 0u, 0u, 0u};
    }
  };
  // Weight loads of the first two items go out before act is staged.
  issue(wave, ca);
  issue(wave + kWaves, cb);
  pin_loads();

  // act -> LDS: 16-byte buffer loads, kActUnroll per thread in flight (act
  // rows are 16-byte aligned: act_ld == inter and inter % EPC == 0 on the
  // vector path).
  if constexpr (VEC) {
    constexpr int kActUnroll = 16;
    const int q4 = ip / 4;
    // One descriptor over all NB rows (a per-row descriptor would depend on the
    // lane's row and force a readfirstlane loop around every load).
    const rsrc_t ar = make_rsrc(act, uint32_t(NB - 1) * uint32_t(act_ld) * 4u + uint32_t(inter) * 4u);
    for (int f0 = tid; f0 < NB * q4; f0 += kActUnroll * kThreads) {
      u32x4 v[kActUnroll];
#pragma unroll
      for (int r = 0; r < kActUnroll; ++r) {
        const int f = f0 + r * kThreads;
        const int b = f / q4, c4 = f % q4;
        v[r] = buf_load16(ar, f < NB * q4 ? (uint32_t(b) * uint32_t(act_ld) + uint32_t(c4) * 4u) * 4u : 0xFFFFFFF0u);
      }
#pragma unroll
      for (int r = 0; r < kActUnroll; ++r) {
        const int f = f0 + r * kThreads;
        if (f < NB * q4) *reinterpret_cast<u32x4*>(a + size_t(f) * 4) = v[r];
      }
    }
  } else {
    for (int k = tid; k < ip; k += kThreads) {
#pragma unroll
      for (int b = 0; b < NB; ++b) a[b * ip + k] = k < inter ? act[size_t(b) * act_ld + k] : 0.f;
    }
  }
  __syncthreads();

  auto finish = [&](int item, const u32x4 (&c)[CPL]) {
    if (item >= nitems) return;
    const int qt = item % kQuarters;
    const int c0 = qt * qch;
    const int last = nch - 1;
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      const float s = wave_sum_u(chunks_dot<T, CPL>(c, a + b * ip, c0, last, lane));
      if (lane == 0) part[item * NB + b] = s;
    }
  };
  for (int item = wave; item < nitems; item += 2 * kWaves) {
    finish(item, ca);
    issue(item + 2 * kWaves, ca);
    pin_loads();
    finish(item + kWaves, cb);
    issue(item + 3 * kWaves, cb);
    pin_loads();
  }
  __syncthreads();
  for (int t = tid; t < nr * NB; t += kThreads) {
    const int i = t / NB, b = t % NB;
    float s = 0.f;
#pragma unroll
    for (int qt = 0; qt < kQuarters; ++qt) s += part[(i * kQuarters + qt) * NB + b];
    const size_t o = size_t(b) * h + rb + i;
    if (add_residual) s += to_f(x[o]);
    out[o] = from_f<T>(s);
  }
}

template <typename K>
int set_lds_limit(K kernel) {
  MKQ_HIP_TRY(hipFuncSetAttribute(reinterpret_cast<const void*>(kernel), hipFuncAttributeMaxDynamicSharedMemorySize,
                                  max_lds_per_block()));
  return MKQ_OK;
}

template <typename T, int NB, bool VEC, int CPL1, int CPL2>
int launch_nb(const T* x, const T* nw, const T* wg, const T* wu, const T* wd, T* out, int h, int inter, float eps,
              int add_residual, float* act, hipStream_t stream) {
  constexpr int EPC = Epc<T>::value;
  const int ncu = cu_count();
  const int max_lds = max_lds_per_block();
  const int hp = round_up(h, EPC), ip = round_up(inter, EPC);

  // Both kernels: two workgroups per CU, rows split evenly.
  const int rows1 = (inter + 2 * ncu - 1) / (2 * ncu);
  const int grid1 = (inter + rows1 - 1) / rows1;
  const int rows2 = (h + 2 * ncu - 1) / (2 * ncu);
  const int grid2 = (h + rows2 - 1) / rows2;

  const size_t lds1 = sizeof(float) * (size_t(NB) * hp + kWaves * NB + size_t(2) * rows1 * NB);
  const size_t lds2 = sizeof(float) * (size_t(NB) * ip + size_t(rows2) * kQuarters * NB);
  if (lds1 > size_t(max_lds) || lds2 > size_t(max_lds))
    return set_error(MKQ_ERR_UNSUPPORTED, "dense_ffn_decode: hidden=%d / intermediate=%d too large for LDS staging", h,
                     inter);
  static bool attr_set = false;
  if (!attr_set) {
    if (int rc = set_lds_limit(&ffn_gateup_kernel<T, NB, VEC, CPL1>)) return rc;
    if (int rc = set_lds_limit(&ffn_down_kernel<T, NB, VEC, CPL2>)) return rc;
    attr_set = true;
  }
  ffn_gateup_kernel<T, NB, VEC, CPL1><<<grid1, kThreads, lds1, stream>>>(x, nw, wg, wu, act, h, inter, eps, inter,
                                                                        rows1);
  MKQ_LAUNCH_CHECK("ffn_gateup_kernel");
  ffn_down_kernel<T, NB, VEC, CPL2><<<grid2, kThreads, lds2, stream>>>(act, wd, x, out, h, inter, add_residual, rows2,
                                                                      inter);
  MKQ_LAUNCH_CHECK("ffn_down_kernel");
  return MKQ_OK;
}

// Chunks per lane: K1 covers a hidden-long row, K2 a quarter of an
// intermediate-long row.  Instantiated sizes (16-bit types): hidden <= 5120
// and intermediate <= 18432 on the fast sizes, up to 16384 / 65536 generally.
constexpr int kCpl[] = {2, 4, 10, 16, 32};

template <typename T, int NB, bool VEC>
int dispatch_cpl(const T* x, const T* nw, const T* wg, const T* wu, const T* wd, T* out, int h, int inter, float eps,
                 int add_residual, float* act, hipStream_t stream) {
  constexpr int EPC = Epc<T>::value;
  const int need1 = (round_up(h, EPC) / EPC + kWave - 1) / kWave;
  const int need2 = ((round_up(inter, EPC) / EPC + kQuarters - 1) / kQuarters + kWave - 1) / kWave;
  const int n1 = need1 <= 2 ? 0 : need1 <= 4 ? 1 : need1 <= 10 ? 2 : need1 <= 16 ? 3 : need1 <= 32 ? 4 : 5;
  const int n2 = need2 <= 2 ? 0 : need2 <= 4 ? 1 : need2 <= 10 ? 2 : need2 <= 16 ? 3 : need2 <= 32 ? 4 : 5;
  if (n1 > 4 || n2 > 4)
    return set_error(MKQ_ERR_UNSUPPORTED, "dense_ffn_decode: hidden=%d / intermediate=%d exceed the kernel sizes", h,
                     inter);
#define MKQ_CPL_CASE(A, B)                                                                                         \
  if (n1 == A && n2 == B)                                                                                          \
    return launch_nb<T, NB, VEC, kCpl[A], kCpl[B]>(x, nw, wg, wu, wd, out, h, inter, eps, add_residual, act, stream);
  // The 27B shape (10, 10) and the small test shapes; others take the next larger instantiation.
  MKQ_CPL_CASE(0, 0)
  MKQ_CPL_CASE(0, 1)
  MKQ_CPL_CASE(1, 1)
  MKQ_CPL_CASE(2, 2)
  MKQ_CPL_CASE(1, 2)
  MKQ_CPL_CASE(2, 1)
#undef MKQ_CPL_CASE
  return launch_nb<T, NB, VEC, 32, 32>(x, nw, wg, wu, wd, out, h, inter, eps, add_residual, act, stream);
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
      rc = vec ? dispatch_cpl<T, 2, true>(xb, nw, wg, wu, wd, ob, h, inter, eps, add_residual, ab, stream)
               : dispatch_cpl<T, 2, false>(xb, nw, wg, wu, wd, ob, h, inter, eps, add_residual, ab, stream);
    else
      rc = vec ? dispatch_cpl<T, 1, true>(xb, nw, wg, wu, wd, ob, h, inter, eps, add_residual, ab, stream)
               : dispatch_cpl<T, 1, false>(xb, nw, wg, wu, wd, ob, h, inter, eps, add_residual, ab, stream);
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
