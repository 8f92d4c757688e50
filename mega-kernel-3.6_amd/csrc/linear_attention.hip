// Recurrent linear-attention decode for gfx950: the reference rule and the
// gated delta rule, FP32 state.
//
// Reference rule (reference.py:148-166, linear_attention_decode.cu:10-42):
//     S' = decay * S + k (x) v;            o = S'^T q
// Gated delta rule (Qwen3.6 linear attention; v head j reads q/k head j/rep):
//     S  = exp(g) * S;  u = v - S^T k;  S' = S + beta * k (x) u;  o = S'^T q
//
// Column j of S (all key rows i for one value index j) evolves independently,
// so a workgroup owns a 64-column slice of one (batch, v-head) state: lane =
// column (64 consecutive floats = one coalesced 256-byte row segment), the 4
// waves split the key rows, and the two reductions over key rows (S^T k and
// S'^T q) cross the waves through LDS.  The slice stays in VGPRs between the
// single HBM read and the single HBM write of the state.
//
// With qk_norm, q and k are L2-normalised in FP32 as they are staged,
// x / sqrt(sum x^2 + 1e-6), and q is then multiplied by q_scale: the
// use_qk_l2norm_in_kernel form of the Qwen3.6 linear-attention step.
#include "mkq_host.h"

using namespace mkq;

namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / kWave;
constexpr int kMaxKeyDim = 256;
constexpr int kRowsPerWave = kMaxKeyDim / kWaves;  // 64 state values per lane at most

// grid: (ceil(Dv/64), Hv, B); block 256.
template <typename T, bool GATED>
__global__ __launch_bounds__(kThreads) void linear_attention_kernel(
    const T* __restrict__ q, const T* __restrict__ k, const T* __restrict__ v, const float* state,
    const float* __restrict__ g, const float* __restrict__ beta, T* __restrict__ out, float* new_state, int hk,
    int hv, int dk, int dv, float decay, int qk_norm, float q_scale, int qk_bs, int v_bs) {
  static_assert(kMaxKeyDim == kThreads, "one staged q/k element per thread");
  __shared__ float qs[kMaxKeyDim];
  __shared__ float ks[kMaxKeyDim];
  __shared__ float red[kWaves][kWave];
  __shared__ float nrm[kWaves][2];

  const int lane = threadIdx.x % kWave, wave = wave_id();
  const int j = blockIdx.x * kWave + lane;  // value column
  const int vh = blockIdx.y;
  const int b = blockIdx.z;
  const int rep = hv / hk;
  const int qh = vh / rep;
  const bool col_ok = j < dv;

  // One descriptor over this head's state: rows i >= dk fall past its end and
  // read as zero, so all loads issue back to back with no branches.  Lanes
  // past the last column use an out-of-range offset.
  const size_t base = (size_t(b) * hv + vh) * size_t(dk) * dv;
  const rsrc_t srd = make_rsrc(state + base, uint32_t(size_t(dk) * dv * 4));
  const rsrc_t swr = make_rsrc(new_state + base, uint32_t(size_t(dk) * dv * 4));

  // q, k and v first (unconditional loads at clamped indices, zeroed after,
  // so no branch waits on them), then the state slice: the state loads are
  // in flight while q/k are staged (and normalised).
  const int ti = threadIdx.x;  // staged q/k element, zero past dk
  const bool kin = ti < dk;
  const size_t qo = size_t(b) * qk_bs + size_t(qh) * dk + (kin ? ti : 0);  // qk_bs: batch stride
  float qv = to_f(q[qo]);
  float kv = to_f(k[qo]);
  const float vraw = to_f(v[size_t(b) * v_bs + size_t(vh) * dv + (col_ok ? j : 0)]);
  float d = decay, bt = 1.0f;
  if constexpr (GATED) {
    d = expf(g[size_t(b) * hv + vh]);
    bt = beta[size_t(b) * hv + vh];
  }
  float s[kRowsPerWave];
#pragma unroll
  for (int r = 0; r < kRowsPerWave; ++r) {
    const int i = wave + r * kWaves;
    const uint32_t off = col_ok ? uint32_t((i * dv + j) * 4) : 0xFFFFFFF0u;
    s[r] = buf_loadf(srd, off);
  }

  qv = kin ? qv : 0.f;
  kv = kin ? kv : 0.f;
  const float vj = col_ok ? vraw : 0.f;
  if (qk_norm) {  // uniform over the launch
    const float sq = wave_sum(qv * qv), sk = wave_sum(kv * kv);
    if (lane == 0) {
      nrm[wave][0] = sq;
      nrm[wave][1] = sk;
    }
    __syncthreads();
    float tq = 0.f, tk = 0.f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
      tq += nrm[w][0];
      tk += nrm[w][1];
    }
    qv = qv / sqrtf(tq + 1e-6f) * q_scale;
    kv = kv / sqrtf(tk + 1e-6f);
  }
  qs[ti] = qv;
  ks[ti] = kv;
  __syncthreads();
#pragma unroll
  for (int r = 0; r < kRowsPerWave; ++r) s[r] *= d;

  float add = vj;  // reference rule: S += k (x) v
  if constexpr (GATED) {
    float p = 0.f;
#pragma unroll
    for (int r = 0; r < kRowsPerWave; ++r) {
      const int i = wave + r * kWaves;
      p = fmaf(s[r], ks[i], p);
    }
    red[wave][lane] = p;
    __syncthreads();
    float sk = 0.f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) sk += red[w][lane];
    add = bt * (vj - sk);  // S += k (x) beta*(v - S^T k)
    __syncthreads();
  }

  float o = 0.f;
#pragma unroll
  for (int r = 0; r < kRowsPerWave; ++r) {
    const int i = wave + r * kWaves;
    // ks/qs are zero past dk, so rows i >= dk add nothing; their stores fall
    // past the descriptor and are dropped.
    s[r] = fmaf(ks[i], add, s[r]);
    o = fmaf(s[r], qs[i], o);
    buf_storef(swr, col_ok ? uint32_t((i * dv + j) * 4) : 0xFFFFFFF0u, s[r]);
  }
  red[wave][lane] = o;
  __syncthreads();
  if (wave == 0 && col_ok) {
    float t = 0.f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) t += red[w][lane];
    out[(size_t(b) * hv + vh) * dv + j] = from_f<T>(t);
  }
}

template <typename T, bool GATED>
int launch(const void* q, const void* k, const void* v, const float* state, const float* g, const float* beta,
           void* out, float* new_state, int batch, int hk, int hv, int dk, int dv, float decay, int qk_norm,
           float q_scale, int qk_bs, int v_bs, hipStream_t stream) {
  dim3 grid((dv + kWave - 1) / kWave, hv, batch);
  linear_attention_kernel<T, GATED><<<grid, kThreads, 0, stream>>>(
      static_cast<const T*>(q), static_cast<const T*>(k), static_cast<const T*>(v), state, g, beta,
      static_cast<T*>(out), new_state, hk, hv, dk, dv, decay, qk_norm, q_scale, qk_bs, v_bs);
  MKQ_LAUNCH_CHECK("linear_attention_kernel");
  return MKQ_OK;
}

template <bool GATED>
int dispatch(int dtype, const void* q, const void* k, const void* v, const float* state, const float* g,
             const float* beta, void* out, float* new_state, int batch, int hk, int hv, int dk, int dv, float decay,
             int qk_norm, float q_scale, void* stream, int qk_bs = 0, int v_bs = 0) {
  if (qk_bs == 0) qk_bs = hk * dk;  // contiguous [B, H, D] by default
  if (v_bs == 0) v_bs = hv * dv;
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (dtype) {
    case MKQ_DTYPE_BF16:
      return launch<bf16_t, GATED>(q, k, v, state, g, beta, out, new_state, batch, hk, hv, dk, dv, decay, qk_norm,
                                   q_scale, qk_bs, v_bs, s);
    case MKQ_DTYPE_F16:
      return launch<f16_t, GATED>(q, k, v, state, g, beta, out, new_state, batch, hk, hv, dk, dv, decay, qk_norm,
                                  q_scale, qk_bs, v_bs, s);
    case MKQ_DTYPE_F32:
      return launch<float, GATED>(q, k, v, state, g, beta, out, new_state, batch, hk, hv, dk, dv, decay, qk_norm,
                                  q_scale, qk_bs, v_bs, s);
    default:
      return set_error(MKQ_ERR_INVALID, "linear attention: unknown dtype %d", dtype);
  }
}

}  // namespace

extern "C" int mkq_linear_attention_decode(int dtype, const void* q, const void* k, const void* v, const float* state,
                                           void* out, float* new_state, int batch, int heads, int key_dim,
                                           int value_dim, float decay, void* stream) {
  clear_error();
  MKQ_REQUIRE(batch > 0 && heads > 0 && key_dim > 0 && value_dim > 0, "linear_attention_decode: sizes must be positive");
  MKQ_REQUIRE(q && k && v && state && out && new_state, "linear_attention_decode: null tensor pointer");
  if (key_dim > kMaxKeyDim)
    return set_error(MKQ_ERR_UNSUPPORTED, "linear_attention_decode: key_dim %d > %d", key_dim, kMaxKeyDim);
  MKQ_REQUIRE(batch <= 65535 && heads <= 65535, "linear_attention_decode: batch/heads too large");
  return dispatch<false>(dtype, q, k, v, state, nullptr, nullptr, out, new_state, batch, heads, heads, key_dim,
                         value_dim, decay, 0, 1.0f, stream);
}

namespace {

int gated_entry(const char* fn, int dtype, const void* q, const void* k, const void* v, const float* state,
                const float* g, const float* beta, void* out, float* new_state, int batch, int k_heads, int v_heads,
                int key_dim, int value_dim, int qk_norm, float q_scale, void* stream) {
  clear_error();
  MKQ_REQUIRE(batch > 0 && k_heads > 0 && v_heads > 0 && key_dim > 0 && value_dim > 0, "%s: sizes must be positive",
              fn);
  MKQ_REQUIRE(v_heads % k_heads == 0, "%s: v_heads must be a multiple of k_heads", fn);
  MKQ_REQUIRE(q && k && v && state && g && beta && out && new_state, "%s: null tensor pointer", fn);
  if (key_dim > kMaxKeyDim) return set_error(MKQ_ERR_UNSUPPORTED, "%s: key_dim %d > %d", fn, key_dim, kMaxKeyDim);
  MKQ_REQUIRE(batch <= 65535 && v_heads <= 65535, "%s: batch/heads too large", fn);
  return dispatch<true>(dtype, q, k, v, state, g, beta, out, new_state, batch, k_heads, v_heads, key_dim, value_dim,
                        1.0f, qk_norm, q_scale, stream);
}

}  // namespace

extern "C" int mkq_gated_delta_decode(int dtype, const void* q, const void* k, const void* v, const float* state,
                                      const float* g, const float* beta, void* out, float* new_state, int batch,
                                      int k_heads, int v_heads, int key_dim, int value_dim, void* stream) {
  return gated_entry("gated_delta_decode", dtype, q, k, v, state, g, beta, out, new_state, batch, k_heads, v_heads,
                     key_dim, value_dim, 0, 1.0f, stream);
}

extern "C" int mkq_gated_delta_decode_qknorm(int dtype, const void* q, const void* k, const void* v,
                                             const float* state, const float* g, const float* beta, void* out,
                                             float* new_state, int batch, int k_heads, int v_heads, int key_dim,
                                             int value_dim, float q_scale, void* stream) {
  return gated_entry("gated_delta_decode_qknorm", dtype, q, k, v, state, g, beta, out, new_state, batch, k_heads,
                     v_heads, key_dim, value_dim, 1, q_scale, stream);
}

namespace {

size_t align256(size_t n) { return (n + 255) / 256 * 256; }

size_t elt_size(int dtype) {
  return dtype == MKQ_DTYPE_F32 ? 4 : (dtype == MKQ_DTYPE_BF16 || dtype == MKQ_DTYPE_F16) ? 2 : 0;
}

}  // namespace

extern "C" size_t mkq_linear_attention_step_workspace_bytes(int dtype, int batch, int k_heads, int v_heads,
                                                            int key_dim, int value_dim) {
  const size_t elt = elt_size(dtype);
  if (elt == 0 || batch <= 0 || k_heads <= 0 || v_heads <= 0 || key_dim <= 0 || value_dim <= 0) return 0;
  const size_t channels = 2 * size_t(k_heads) * key_dim + size_t(v_heads) * value_dim;
  return align256(size_t(batch) * channels * elt) + align256(size_t(batch) * v_heads * value_dim * elt);
}

// The three launches of one Qwen3.6 linear-attention step on one stream: the
// conv update writes the mixed q/k/v row into the workspace, the recurrence
// reads q, k and v from it in place (batch stride = the channel count) and
// updates the state in place, and the gated norm writes `out`.
extern "C" int mkq_linear_attention_step(int dtype, const void* x_mixed, void* conv_state, const void* conv_weight,
                                         const void* conv_bias, int conv_state_len, float* state, const float* g,
                                         const float* beta, const void* z, const void* norm_weight, void* out,
                                         int batch, int k_heads, int v_heads, int key_dim, int value_dim,
                                         float q_scale, float eps, void* workspace, size_t workspace_bytes,
                                         void* stream) {
  clear_error();
  const char* fn = "linear_attention_step";
  MKQ_REQUIRE(batch > 0 && k_heads > 0 && v_heads > 0 && key_dim > 0 && value_dim > 0 && conv_state_len > 0,
              "%s: sizes must be positive", fn);
  MKQ_REQUIRE(v_heads % k_heads == 0, "%s: v_heads must be a multiple of k_heads", fn);
  MKQ_REQUIRE(x_mixed && conv_state && conv_weight && state && g && beta && z && norm_weight && out,
              "%s: null tensor pointer", fn);
  if (key_dim > kMaxKeyDim) return set_error(MKQ_ERR_UNSUPPORTED, "%s: key_dim %d > %d", fn, key_dim, kMaxKeyDim);
  MKQ_REQUIRE(batch <= 65535 && v_heads <= 65535, "%s: batch/heads too large", fn);
  const size_t need = mkq_linear_attention_step_workspace_bytes(dtype, batch, k_heads, v_heads, key_dim, value_dim);
  MKQ_REQUIRE(need > 0, "%s: unknown dtype %d", fn, dtype);
  MKQ_REQUIRE(workspace && workspace_bytes >= need, "%s: workspace too small", fn);
  MKQ_REQUIRE((reinterpret_cast<uintptr_t>(workspace) & 255u) == 0, "%s: workspace must be 256-byte aligned", fn);
  const size_t elt = elt_size(dtype);
  const int channels = 2 * k_heads * key_dim + v_heads * value_dim;
  unsigned char* mixed = static_cast<unsigned char*>(workspace);
  unsigned char* o = mixed + align256(size_t(batch) * channels * elt);
  int rc = mkq_causal_conv1d_update(dtype, x_mixed, conv_state, conv_weight, conv_bias, mixed, batch, channels,
                                    conv_state_len, 1, stream);
  if (rc != MKQ_OK) return rc;
  const size_t kd = size_t(k_heads) * key_dim * elt;
  rc = dispatch<true>(dtype, mixed, mixed + kd, mixed + 2 * kd, state, g, beta, o, state, batch, k_heads, v_heads,
                      key_dim, value_dim, 1.0f, 1, q_scale, stream, channels, channels);
  if (rc != MKQ_OK) return rc;
  return mkq_gated_rms_norm(dtype, o, z, norm_weight, out, batch * v_heads, value_dim, eps, stream);
}
