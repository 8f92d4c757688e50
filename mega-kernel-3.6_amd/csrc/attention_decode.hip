// GQA full-attention decode (one query token) for gfx950: split-K flash-decode
// on MFMA.
//
// out[b, qh] = softmax(q[b,qh] . K[b,:,kvh]^T * scale) V[b,:,kvh],  kvh = qh / G
// (reference.py:117-145; replaces attention_decode.cu:33-218).
//
// Work split: workgroup = (token chunk, kv head [, group of 16 q heads], batch
// row); its 4 waves take 32-token tiles of the chunk in turn.  Per tile a wave
//   * loads the K tile straight into MFMA A-operand registers (16 tokens x 32
//     dims per v_mfma_f32_16x16x32, 16 bytes per lane) and computes S^T = K Q^T
//     for all q heads of the group at once -- the G (=6) q heads that share a
//     kv head reuse one read of K and V;
//   * stages the V tile in wave-private LDS (row stride padded so the
//     transposed 16-bit reads below are bank-conflict free);
//   * runs an online softmax in the base-2 domain; the probabilities stay in
//     registers in exactly the token order the PV product needs as its B
//     operand (the S^T output of lane l covers tokens 4*(l/16)+i of each
//     16-token half, which is the K-group of lane l in the PV MFMA);
//   * accumulates O^T = V^T P^T with 16 MFMAs per 32 tokens (A operand read
//     transposed from LDS).
// The 4 waves merge in LDS; each workgroup writes one partial (m, l, O) and a
// small merge kernel combines the chunks with the log-sum-exp rule.
//
// HBM-bound: every K/V byte is read once (4*T*Hkv*D bytes per batch row).
#include <math.h>

#include "mkq_host.h"

using namespace mkq;

namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / kWave;
constexpr int kTile = 32;   // tokens per wave iteration
constexpr int kMaxD = 256;
constexpr int kMaxSteps = kMaxD / 32;   // QK^T MFMA steps over head_dim
constexpr int kMaxDTiles = kMaxD / 16;  // PV MFMA tiles over head_dim
constexpr int kMaxVChunks = kTile * kMaxD / 8 / kWave;  // 16-byte V chunks per lane per tile
constexpr float kNegInf = -INFINITY;

template <typename T>
struct Mfma;
template <>
struct Mfma<bf16_t> {
  typedef bf16x8 vec;
  static __device__ __forceinline__ f32x4 mma(vec a, vec b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ short from_float(float f) { return short(f2bf_bits(f)); }
};
template <>
struct Mfma<f16_t> {
  typedef f16x8 vec;
  static __device__ __forceinline__ f32x4 mma(vec a, vec b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ _Float16 from_float(float f) { return _Float16(f); }
};

// LDS row stride (in 16-bit elements) of the staged V tile: D/2 dwords padded
// to 2 mod 8 dwords, so the four token rows a transposed read touches land in
// four disjoint groups of 8 banks.
__host__ __device__ inline int v_stride(int d) {
  const int dw = d / 2;
  const int pad = ((2 - dw) % 8 + 8) % 8;
  return 2 * (dw + pad);
}

__host__ __device__ inline size_t chunk_lds_bytes(int d) {
  const size_t stage = size_t(kWaves) * kTile * v_stride(d) * 2;
  const size_t merge = size_t(kWaves) * (32 + 16 * size_t(d)) * 4;
  return stage > merge ? stage : merge;
}

// grid: (nchunks, kv_heads * head_groups, batch); block 256.
template <typename T>
__global__ __launch_bounds__(kThreads) void attn_chunk_kernel(const T* __restrict__ q, const T* __restrict__ kc,
                                                              const T* __restrict__ vc, float* __restrict__ part_o,
                                                              float* __restrict__ part_m, float* __restrict__ part_l,
                                                              int hq, int hkv, int d, int seq, int group, int ngroups,
                                                              int nchunks, int chunk_tokens, float scale_log2) {
  typedef typename Mfma<T>::vec V8;
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
  const int col = lane & 15, grp = lane >> 4;
  const int c = blockIdx.x, b = blockIdx.z;
  const int kvh = blockIdx.y / ngroups, hg = blockIdx.y % ngroups;
  const int heads_here = min(16, group - hg * 16);
  const int qh0 = kvh * group + hg * 16;
  const int nsteps = (d + 31) / 32;
  const int ndt = (d + 15) / 16;
  const int vstr = v_stride(d);
  const int cpr = d / 8;  // 16-byte chunks per token row
  uint16_t* vt = reinterpret_cast<uint16_t*>(smem) + size_t(wave) * kTile * vstr;

  // Q^T as the B operand: lane (head col, k-group grp) holds dims 32s+8grp..+8.
  V8 qop[kMaxSteps];
#pragma unroll
  for (int s = 0; s < kMaxSteps; ++s) {
    const int d0 = 32 * s + 8 * grp;
    u32x4 v = u32x4{0u, 0u, 0u, 0u};
    if (s < nsteps && col < heads_here && d0 < d)
      v = *reinterpret_cast<const u32x4*>(q + (size_t(b) * hq + qh0 + col) * d + d0);
    qop[s] = __builtin_bit_cast(V8, v);
  }

  f32x4 oacc[kMaxDTiles];
#pragma unroll
  for (int n = 0; n < kMaxDTiles; ++n) oacc[n] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m_run = kNegInf, l_run = 0.f;

  const int t_begin = c * chunk_tokens;
  const int t_end = min(seq, t_begin + chunk_tokens);
  const size_t tok_stride = size_t(hkv) * d;
  const T* kb = kc + (size_t(b) * seq * hkv + kvh) * d;
  const T* vb = vc + (size_t(b) * seq * hkv + kvh) * d;

  for (int t0 = t_begin + wave * kTile; t0 < t_end; t0 += kWaves * kTile) {
    // K tile -> A operands (token = 16*hh + col, dims 32s + 8grp).
    V8 kop[2][kMaxSteps];
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
      const int tok = t0 + 16 * hh + col;
#pragma unroll
      for (int s = 0; s < kMaxSteps; ++s) {
        const int d0 = 32 * s + 8 * grp;
        u32x4 v = u32x4{0u, 0u, 0u, 0u};
        if (s < nsteps && tok < t_end && d0 < d)
          v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(kb + size_t(tok) * tok_stride + d0));
        kop[hh][s] = __builtin_bit_cast(V8, v);
      }
    }
    // V tile -> registers (coalesced 16-byte chunks; invalid tokens read as 0).
    u32x4 vreg[kMaxVChunks];
#pragma unroll
    for (int i = 0; i < kMaxVChunks; ++i) {
      const int qi = lane + kWave * i;
      vreg[i] = u32x4{0u, 0u, 0u, 0u};
      if (qi < kTile * cpr) {
        const int row = qi / cpr, dc = qi % cpr;
        const int tok = t0 + row;
        if (tok < t_end)
          vreg[i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(vb + size_t(tok) * tok_stride + dc * 8));
      }
    }
    // S^T = K Q^T: sacc[hh][i] = score(token t0+16hh+4grp+i, head col).
    f32x4 sacc[2] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}};
#pragma unroll
    for (int s = 0; s < kMaxSteps; ++s) {
      if (s < nsteps) {
        sacc[0] = Mfma<T>::mma(kop[0][s], qop[s], sacc[0]);
        sacc[1] = Mfma<T>::mma(kop[1][s], qop[s], sacc[1]);
      }
    }
    // Stage V in LDS (two 8-byte stores per chunk: the padded stride is 8-byte aligned).
#pragma unroll
    for (int i = 0; i < kMaxVChunks; ++i) {
      const int qi = lane + kWave * i;
      if (qi < kTile * cpr) {
        const int row = qi / cpr, dc = qi % cpr;
        uint2* dst = reinterpret_cast<uint2*>(vt + row * vstr + dc * 8);
        dst[0] = make_uint2(vreg[i].x, vreg[i].y);
        dst[1] = make_uint2(vreg[i].z, vreg[i].w);
      }
    }
    // Online softmax (base 2).  Element j of this lane's 8 scores is token
    // tau(j) = (j < 4 ? 4grp + j : 16 + 4grp + j - 4) of the tile.
    float sv[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int hh = j >> 2, i = j & 3;
      const int tok = t0 + 16 * hh + 4 * grp + i;
      sv[j] = tok < t_end ? sacc[hh][i] * scale_log2 : kNegInf;
    }
    float mx = sv[0];
#pragma unroll
    for (int j = 1; j < 8; ++j) mx = fmaxf(mx, sv[j]);
    mx = fmaxf(mx, xor_lane(mx, 16));
    mx = fmaxf(mx, xor_lane(mx, 32));
    const float m_new = fmaxf(m_run, mx);
    const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
    V8 pop;
    float psum = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float p = __builtin_amdgcn_exp2f(sv[j] - m_new);
      psum += p;
      pop[j] = Mfma<T>::from_float(p);
    }
    l_run = l_run * alpha + psum;
    m_run = m_new;
    // O^T = V^T P^T, A operand read transposed from LDS: dim 16n + col, tokens tau(j).
#pragma unroll
    for (int n = 0; n < kMaxDTiles; ++n) {
      if (n < ndt) {
        const int dim = 16 * n + col;
        union {
          V8 v;
          uint16_t u[8];
        } va;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const int tok = (j < 4 ? 4 * grp + j : 16 + 4 * grp + (j - 4));
          va.u[j] = vt[tok * vstr + dim];
        }
        oacc[n] = Mfma<T>::mma(va.v, pop, oacc[n] * alpha);
      }
    }
  }

  // Per-head l over the 4 lane groups (m is already uniform across them).
  l_run += xor_lane(l_run, 16);
  l_run += xor_lane(l_run, 32);

  __syncthreads();  // V staging area becomes the merge area
  float* mw = reinterpret_cast<float*>(smem) + size_t(wave) * (32 + 16 * d);
  float* lw = mw + 16;
  float* ow = mw + 32;  // [16 heads][d]
  if (grp == 0) {
    mw[col] = m_run;
    lw[col] = l_run;
  }
#pragma unroll
  for (int n = 0; n < kMaxDTiles; ++n) {
    if (n < ndt) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int dim = 16 * n + 4 * grp + i;
        if (dim < d) ow[col * d + dim] = oacc[n][i];
      }
    }
  }
  __syncthreads();
  const float* m0 = reinterpret_cast<const float*>(smem);
  const size_t wstride = 32 + 16 * size_t(d);
  for (int idx = threadIdx.x; idx < heads_here * d; idx += kThreads) {
    const int hd = idx / d, dim = idx % d;
    float M = kNegInf;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) M = fmaxf(M, m0[w * wstride + hd]);
    float o = 0.f, L = 0.f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
      const float mwv = m0[w * wstride + hd];
      const float f = mwv == kNegInf ? 0.f : __builtin_amdgcn_exp2f(mwv - M);
      o += f * m0[w * wstride + 32 + hd * d + dim];
      L += f * m0[w * wstride + 16 + hd];
    }
    const size_t pi = (size_t(b) * hq + qh0 + hd) * nchunks + c;
    part_o[pi * d + dim] = o;
    if (dim == 0) {
      part_m[pi] = M;
      part_l[pi] = L;
    }
  }
}

// grid: (batch*q_heads, ceil(d/64)); block 256 = 64 dims x 4 chunk slices.
template <typename T>
__global__ __launch_bounds__(kThreads) void attn_merge_kernel(const float* __restrict__ part_o,
                                                              const float* __restrict__ part_m,
                                                              const float* __restrict__ part_l, T* __restrict__ out,
                                                              int d, int nchunks) {
  __shared__ float red[kThreads];
  __shared__ float bcast[2];
  const int bq = blockIdx.x;
  const int tid = threadIdx.x, dl = tid & 63, cs = tid >> 6;
  const int dim = blockIdx.y * 64 + dl;
  const float* pm = part_m + size_t(bq) * nchunks;
  const float* pl = part_l + size_t(bq) * nchunks;

  float M = kNegInf;
  for (int c = tid; c < nchunks; c += kThreads) M = fmaxf(M, pm[c]);
  M = wave_max(M);
  if ((tid & 63) == 0) red[tid >> 6] = M;
  __syncthreads();
  if (tid == 0) {
    float mm = red[0];
    for (int w = 1; w < kWaves; ++w) mm = fmaxf(mm, red[w]);
    bcast[0] = mm;
  }
  __syncthreads();
  M = bcast[0];
  float L = 0.f;
  for (int c = tid; c < nchunks; c += kThreads) L += pl[c] * __builtin_amdgcn_exp2f(pm[c] - M);
  L = wave_sum(L);
  __syncthreads();
  if ((tid & 63) == 0) red[tid >> 6] = L;
  __syncthreads();
  if (tid == 0) bcast[1] = red[0] + red[1] + red[2] + red[3];

  float o = 0.f;
  if (dim < d)
    for (int c = cs; c < nchunks; c += kWaves)
      o += part_o[(size_t(bq) * nchunks + c) * d + dim] * __builtin_amdgcn_exp2f(pm[c] - M);
  __syncthreads();
  red[tid] = o;
  __syncthreads();
  if (cs == 0 && dim < d) {
    const float s = red[dl] + red[64 + dl] + red[128 + dl] + red[192 + dl];
    out[size_t(bq) * d + dim] = from_f<T>(s / bcast[1]);
  }
}

// Fallback for float32 inputs or head_dim not a multiple of 8: three passes
// over the keys with the probabilities kept in the workspace.
// grid: (q_heads, batch); block 256.
template <typename T>
__global__ __launch_bounds__(kThreads) void attn_generic_kernel(const T* __restrict__ q, const T* __restrict__ kc,
                                                                const T* __restrict__ vc, T* __restrict__ out,
                                                                float* __restrict__ probs, int hq, int hkv, int d,
                                                                int seq, float scale) {
  __shared__ float qs[kMaxD];
  __shared__ float red[kWaves];
  __shared__ float bc;
  const int qh = blockIdx.x, b = blockIdx.y, tid = threadIdx.x;
  const int kvh = qh / (hq / hkv);
  for (int i = tid; i < d; i += kThreads) qs[i] = to_f(q[(size_t(b) * hq + qh) * d + i]);
  __syncthreads();
  float* p = probs + (size_t(b) * hq + qh) * seq;
  const size_t ts = size_t(hkv) * d;
  const T* kb = kc + (size_t(b) * seq * hkv + kvh) * d;
  const T* vb = vc + (size_t(b) * seq * hkv + kvh) * d;
  float mx = kNegInf;
  for (int t = tid; t < seq; t += kThreads) {
    float s = 0.f;
    for (int i = 0; i < d; ++i) s = fmaf(to_f(kb[size_t(t) * ts + i]), qs[i], s);
    s *= scale;
    p[t] = s;
    mx = fmaxf(mx, s);
  }
  mx = wave_max(mx);
  if ((tid & 63) == 0) red[tid >> 6] = mx;
  __syncthreads();
  if (tid == 0) bc = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  __syncthreads();
  const float M = bc;
  float sum = 0.f;
  for (int t = tid; t < seq; t += kThreads) {
    const float e = expf(p[t] - M);
    p[t] = e;
    sum += e;
  }
  sum = wave_sum(sum);
  __syncthreads();
  if ((tid & 63) == 0) red[tid >> 6] = sum;
  __syncthreads();
  if (tid == 0) bc = red[0] + red[1] + red[2] + red[3];
  __syncthreads();
  const float inv = 1.0f / bc;
  for (int i = tid; i < d; i += kThreads) {
    float o = 0.f;
    for (int t = 0; t < seq; ++t) o = fmaf(p[t], to_f(vb[size_t(t) * ts + i]), o);
    out[(size_t(b) * hq + qh) * d + i] = from_f<T>(o * inv);
  }
}

int num_chunks(int batch, int hkv, int ngroups, int seq) {
  const int max_chunks = (seq + kWaves * kTile - 1) / (kWaves * kTile);  // >= one tile per wave
  const int want = (2 * cu_count() + batch * hkv * ngroups - 1) / (batch * hkv * ngroups);
  int n = want < max_chunks ? want : max_chunks;
  return n < 1 ? 1 : n;
}

size_t fast_ws_floats(int batch, int hq, int d, int seq) {
  const int max_chunks = (seq + kWaves * kTile - 1) / (kWaves * kTile);
  return size_t(batch) * hq * max_chunks * (size_t(d) + 2);
}

template <typename T>
int launch_fast(const void* q, const void* k, const void* v, void* out, int batch, int hq, int hkv, int d, int seq,
                float scale, float* ws, hipStream_t stream) {
  const int group = hq / hkv;
  const int ngroups = (group + 15) / 16;
  const int nchunks = num_chunks(batch, hkv, ngroups, seq);
  int chunk_tokens = (seq + nchunks - 1) / nchunks;
  chunk_tokens = (chunk_tokens + kTile - 1) / kTile * kTile;
  const int nch = (seq + chunk_tokens - 1) / chunk_tokens;
  const size_t lds = chunk_lds_bytes(d);
  static bool attr_set = false;
  if (!attr_set) {
    MKQ_HIP_TRY(hipFuncSetAttribute(reinterpret_cast<const void*>(&attn_chunk_kernel<T>),
                                    hipFuncAttributeMaxDynamicSharedMemorySize, int(chunk_lds_bytes(kMaxD))));
    attr_set = true;
  }
  float* part_o = ws;
  float* part_m = part_o + size_t(batch) * hq * nch * d;
  float* part_l = part_m + size_t(batch) * hq * nch;
  dim3 g1(nch, hkv * ngroups, batch);
  attn_chunk_kernel<T><<<g1, kThreads, lds, stream>>>(static_cast<const T*>(q), static_cast<const T*>(k),
                                                      static_cast<const T*>(v), part_o, part_m, part_l, hq, hkv, d,
                                                      seq, group, ngroups, nch, chunk_tokens, scale * kLog2e);
  MKQ_LAUNCH_CHECK("attn_chunk_kernel");
  dim3 g2(batch * hq, (d + 63) / 64);
  attn_merge_kernel<T><<<g2, kThreads, 0, stream>>>(part_o, part_m, part_l, static_cast<T*>(out), d, nch);
  MKQ_LAUNCH_CHECK("attn_merge_kernel");
  return MKQ_OK;
}

template <typename T>
int launch_generic(const void* q, const void* k, const void* v, void* out, int batch, int hq, int hkv, int d,
                   int seq, float scale, float* ws, hipStream_t stream) {
  dim3 g(hq, batch);
  attn_generic_kernel<T><<<g, kThreads, 0, stream>>>(static_cast<const T*>(q), static_cast<const T*>(k),
                                                     static_cast<const T*>(v), static_cast<T*>(out), ws, hq, hkv, d,
                                                     seq, scale);
  MKQ_LAUNCH_CHECK("attn_generic_kernel");
  return MKQ_OK;
}

}  // namespace

extern "C" size_t mkq_full_attention_decode_workspace_bytes(int batch, int q_heads, int kv_heads, int head_dim,
                                                            int seq_len) {
  (void)kv_heads;
  if (batch <= 0 || q_heads <= 0 || head_dim <= 0 || seq_len <= 0) return 0;
  const size_t fast = fast_ws_floats(batch, q_heads, head_dim, seq_len);
  const size_t generic = size_t(batch) * q_heads * seq_len;
  return sizeof(float) * (fast > generic ? fast : generic);
}

extern "C" int mkq_full_attention_decode(int dtype, const void* q, const void* k_cache, const void* v_cache,
                                         void* out, int batch, int q_heads, int kv_heads, int head_dim, int seq_len,
                                         float scale, void* workspace, size_t workspace_bytes, void* stream) {
  clear_error();
  MKQ_REQUIRE(batch > 0 && q_heads > 0 && kv_heads > 0 && head_dim > 0, "full_attention_decode: sizes must be positive");
  MKQ_REQUIRE(seq_len > 0, "seq_len must be positive");
  MKQ_REQUIRE(q_heads % kv_heads == 0, "query_heads must be divisible by kv_heads");
  MKQ_REQUIRE(head_dim <= kMaxD, "head_dim > 256 is not supported by this kernel");
  MKQ_REQUIRE(q && k_cache && v_cache && out, "full_attention_decode: null tensor pointer");
  MKQ_REQUIRE(batch <= 65535 && q_heads <= 65535, "full_attention_decode: batch/heads too large");
  MKQ_REQUIRE(workspace && workspace_bytes >= mkq_full_attention_decode_workspace_bytes(batch, q_heads, kv_heads,
                                                                                        head_dim, seq_len),
              "full_attention_decode: workspace too small");
  hipStream_t s = static_cast<hipStream_t>(stream);
  float* ws = static_cast<float*>(workspace);
  const bool fast_ok = (head_dim % 8 == 0) && aligned16(q) && aligned16(k_cache) && aligned16(v_cache);
  switch (dtype) {
    case MKQ_DTYPE_BF16:
      return fast_ok ? launch_fast<bf16_t>(q, k_cache, v_cache, out, batch, q_heads, kv_heads, head_dim, seq_len,
                                           scale, ws, s)
                     : launch_generic<bf16_t>(q, k_cache, v_cache, out, batch, q_heads, kv_heads, head_dim, seq_len,
                                              scale, ws, s);
    case MKQ_DTYPE_F16:
      return fast_ok ? launch_fast<f16_t>(q, k_cache, v_cache, out, batch, q_heads, kv_heads, head_dim, seq_len,
                                          scale, ws, s)
                     : launch_generic<f16_t>(q, k_cache, v_cache, out, batch, q_heads, kv_heads, head_dim, seq_len,
                                             scale, ws, s);
    case MKQ_DTYPE_F32:
      return launch_generic<float>(q, k_cache, v_cache, out, batch, q_heads, kv_heads, head_dim, seq_len, scale, ws,
                                   s);
    default:
      return set_error(MKQ_ERR_INVALID, "full_attention_decode: unknown dtype %d", dtype);
  }
}
