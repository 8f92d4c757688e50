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
// waves split the key rows in contiguous blocks, and the two reductions over
// key rows (S^T k and S'^T q) cross the waves through LDS.  The slice stays in VGPRs between the
// single HBM read and the single HBM write of the state.
//
// With qk_norm, q and k are L2-normalised in FP32 as they are staged,
// x / sqrt(sum x^2 + 1e-6), and q is then multiplied by q_scale: the
// use_qk_l2norm_in_kernel form of the Qwen3.6 linear-attention step.
#include "linear_common.h"
#include "mkq_host.h"

using namespace mkq;

namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / kWave;
constexpr int kMaxKeyDim = 256;
constexpr int kNormPre = 4;  // step: z / norm weight values per lane held for the row norm (value_dim <= 256)

// The conv and norm side of the one-launch step (NT > 0).
template <typename T>
struct StepArgs {
  const T* x = nullptr;          // x_mixed [B, C]
  T* conv_state = nullptr;       // [B, C, S], updated in place
  const T* conv_w = nullptr;     // [C, S + 1]
  const T* conv_b = nullptr;     // [C] or null
  const T* z = nullptr;          // [B, Hv, Dv]
  const T* norm_w = nullptr;     // [Dv]
  float* obuf = nullptr;         // [B, Hv, Dv]: the recurrence output (T-rounded) handed to the row's norm
  unsigned* cnt_qk = nullptr;    // [B, Hk]: arrivals of the workgroups that read a q/k head's channels
  unsigned* cnt_row = nullptr;   // [B, Hv]: arrivals of a row's column slices
  int channels = 0, s_len = 0;
  float eps = 0.f;
};

// grid: (ceil(Dv/64), Hv, B); block 256.
//
// NT > 0 (the one-launch Qwen3.6 step, GATED with qk_norm; NT = conv taps
// held, S + 1 <= NT): q, k and v are not read from memory but computed by the
// causal conv update from x_mixed, as the conv op computes them.  Thread t
// computes q and k channel t of head qh (every workgroup reading that head
// does, so rep * ncol workgroups compute the same values) and wave 0 lane l
// the v channel of column j0 + l, which only this workgroup reads.  The v
// channels' conv state is written at once; a q/k channel's state is written
// by the last of the workgroups that read it (an arrival count per (b, qh)),
// since any earlier write could reach a workgroup that has not loaded the
// old state yet.  At the end each workgroup hands its T-rounded output
// columns over agent-coherent stores, and the last column slice of a row to
// arrive runs the gated RMSNorm over the whole row.  Both counts are put
// back at zero by their last arrival.
template <typename T, bool GATED, int NT, int RW>
__global__ __launch_bounds__(kThreads) void linear_attention_kernel(
    const T* __restrict__ q, const T* __restrict__ k, const T* __restrict__ v, const float* state,
    const float* __restrict__ g, const float* __restrict__ beta, T* __restrict__ out, float* new_state, int hk,
    int hv, int dk, int dv, float decay, int qk_norm, float q_scale, int qk_bs, int v_bs, StepArgs<T> sa) {
  static_assert(kMaxKeyDim == kThreads, "one staged q/k element per thread");
  static_assert(RW * kWaves <= kMaxKeyDim, "RW key rows per wave");
  constexpr bool STEP = NT > 0;
  static_assert(!STEP || GATED, "the step runs the gated rule");
  __shared__ float qs[kMaxKeyDim];
  __shared__ float ks[kMaxKeyDim];
  __shared__ float vs[kWave];
  __shared__ float red[kWaves][kWave];
  __shared__ float nrm[kWaves][2];
  __shared__ int last_qk;

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
  float qv = 0.f, kv = 0.f, vraw = 0.f;
  // STEP: the conv windows and taps of this thread's q, k and v channels.
  float win_q[NT > 0 ? NT : 1], tap_q[NT > 0 ? NT : 1], win_k[NT > 0 ? NT : 1], tap_k[NT > 0 ? NT : 1];
  float win_v[NT > 0 ? NT : 1], tap_v[NT > 0 ? NT : 1], bq = 0.f, bk = 0.f, bv = 0.f;
  const int s_len = sa.s_len;
  const size_t xrow = size_t(b) * sa.channels;
  const int cq = qh * dk + (kin ? ti : 0), ck = hk * dk + cq;
  const bool vown = ti < kWave && blockIdx.x * kWave + ti < dv;
  const int cv = 2 * hk * dk + vh * dv + (vown ? blockIdx.x * kWave + ti : 0);
  if constexpr (STEP) {
    // The bias is read from conv_w when there is none (in range, discarded),
    // so that no load sits in a branch.
    const T* bp = sa.conv_b ? sa.conv_b : sa.conv_w;
    auto window = [&](int c, float (&win)[NT], float (&taps)[NT], float& bias) __attribute__((always_inline)) {
      const T* st = sa.conv_state + (xrow + c) * s_len;
      const T* wc = sa.conv_w + size_t(c) * (s_len + 1);
      const float xv = to_f(sa.x[xrow + c]);
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        const float sv = to_f(st[t < s_len ? t : s_len - 1]);
        const float tw = to_f(wc[t <= s_len ? t : s_len]);
        win[t] = t < s_len ? sv : (t == s_len ? xv : 0.f);
        taps[t] = t <= s_len ? tw : 0.f;
      }
      const float bb = to_f(bp[c]);
      bias = sa.conv_b ? bb : 0.f;
    };
    window(cq, win_q, tap_q, bq);
    window(ck, win_k, tap_k, bk);
    window(cv, win_v, tap_v, bv);
  } else {
    const size_t qo = size_t(b) * qk_bs + size_t(qh) * dk + (kin ? ti : 0);  // qk_bs: batch stride
    qv = to_f(q[qo]);
    kv = to_f(k[qo]);
    vraw = to_f(v[size_t(b) * v_bs + size_t(vh) * dv + (col_ok ? j : 0)]);
  }
  // STEP: z and the norm weight of columns lane + 64 m (value_dim <= 256),
  // loaded now for the row's norm at the end, before the state loads.
  float zpre[kNormPre], wpre[kNormPre];
  if constexpr (STEP) {
    const T* zr = sa.z + (size_t(b) * hv + vh) * dv;
#pragma unroll
    for (int m = 0; m < kNormPre; ++m) {
      const int i = lane + kWave * m, ic = i < dv ? i : dv - 1;
      zpre[m] = to_f(zr[ic]);
      wpre[m] = to_f(sa.norm_w[ic]);
    }
  }
  float d = decay, bt = 1.0f;
  if constexpr (GATED) {
    d = expf(g[size_t(b) * hv + vh]);
    bt = beta[size_t(b) * hv + vh];
  }
  // Wave w holds key rows w * RW .. w * RW + RW - 1 (RW * 4 >= dk), so the
  // q/k values a wave reads from LDS are contiguous.
  // Byte offset of (row wave * RW, column j); lanes past the last column
  // start at 2^31, past any descriptor, and stay there for every row.
  const uint32_t off0 = col_ok ? uint32_t((wave * RW * dv + j) * 4) : 0x80000000u;
  float s[RW];
#pragma unroll
  for (int r = 0; r < RW; ++r) s[r] = buf_loadf(srd, off0 + uint32_t(r * dv * 4));

  if constexpr (STEP) {
    qv = conv_channel<T, NT>(win_q, tap_q, bq, s_len, true);
    kv = conv_channel<T, NT>(win_k, tap_k, bk, s_len, true);
    const float vc = conv_channel<T, NT>(win_v, tap_v, bv, s_len, true);
    if (vown) {
      vs[ti] = vc;
      T* st = sa.conv_state + (xrow + cv) * s_len;
#pragma unroll
      for (int t = 0; t + 1 < NT; ++t)
        if (t < s_len) st[t] = from_f<T>(win_v[t + 1]);
    }
  }
  qv = kin ? qv : 0.f;
  kv = kin ? kv : 0.f;
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
  // STEP: every thread has used its conv loads, so this workgroup counts as a
  // reader of head qh's conv state; the count's result is used at the end.
  unsigned qk_prev = 0;
  if constexpr (STEP) {
    if (threadIdx.x == 0)
      qk_prev = __hip_atomic_fetch_add(sa.cnt_qk + size_t(b) * hk + qh, 1u, __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
  }
  const float vj = col_ok ? (STEP ? vs[lane] : vraw) : 0.f;
#pragma unroll
  for (int r = 0; r < RW; ++r) s[r] *= d;

  float add = vj;  // reference rule: S += k (x) v
  if constexpr (GATED) {
    float p = 0.f;
#pragma unroll
    for (int r = 0; r < RW; ++r) p = fmaf(s[r], ks[wave * RW + r], p);
    red[wave][lane] = p;
    __syncthreads();
    float sk = 0.f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) sk += red[w][lane];
    add = bt * (vj - sk);  // S += k (x) beta*(v - S^T k)
    __syncthreads();
  }

  // STEP: wave 0 stores its state rows after handing its output over, so
  // that the wait for the hand-off's stores does not include them.
  // ks/qs are zero past dk, so rows i >= dk add nothing; their stores fall
  // past the descriptor and are dropped.
  auto store_rows = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int r = 0; r < RW; ++r)
      buf_storef(swr, off0 + uint32_t(r * dv * 4), s[r]);
  };
  float o = 0.f;
#pragma unroll
  for (int r = 0; r < RW; ++r) {
    s[r] = fmaf(ks[wave * RW + r], add, s[r]);
    o = fmaf(s[r], qs[wave * RW + r], o);
  }
  if (!STEP || wave != 0) store_rows();
  red[wave][lane] = o;
  const unsigned qk_readers = unsigned(rep) * gridDim.x;
  if constexpr (STEP) {
    if (threadIdx.x == 0) last_qk = qk_prev == qk_readers - 1u ? 1 : 0;
  }
  __syncthreads();
  if constexpr (!STEP) {
    if (wave == 0 && col_ok) {
      float t = 0.f;
#pragma unroll
      for (int w = 0; w < kWaves; ++w) t += red[w][lane];
      out[(size_t(b) * hv + vh) * dv + j] = from_f<T>(t);
    }
  } else {
    if (last_qk) {  // the last reader of head qh writes its q/k conv state
      if (kin) {
        T* sq = sa.conv_state + (xrow + cq) * s_len;
        T* sk = sa.conv_state + (xrow + ck) * s_len;
#pragma unroll
        for (int t = 0; t + 1 < NT; ++t)
          if (t < s_len) {
            sq[t] = from_f<T>(win_q[t + 1]);
            sk[t] = from_f<T>(win_k[t + 1]);
          }
      }
      if (threadIdx.x == 0)
        __hip_atomic_store(sa.cnt_qk + size_t(b) * hk + qh, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    if (wave == 0) {
      const size_t row = size_t(b) * hv + vh;
      float t = 0.f;
#pragma unroll
      for (int w = 0; w < kWaves; ++w) t += red[w][lane];
      if (col_ok) store_partial(sa.obuf + row * dv + j, to_f(from_f<T>(t)));
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the row's columns are in memory before the count
      unsigned prev = 0;
      if (lane == 0)
        prev = __hip_atomic_fetch_add(sa.cnt_row + row, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      store_rows();
      prev = __builtin_amdgcn_readfirstlane(prev);
      if (prev == gridDim.x - 1u) {  // the row's last column slice: its gated RMSNorm
        const float* orow = sa.obuf + row * dv;
        if (dv <= kWave * kNormPre) {
          float xs[kNormPre], ss = 0.f;
#pragma unroll
          for (int m = 0; m < kNormPre; ++m) {
            const int i = lane + kWave * m;
            const float x = load_partial(orow + (i < dv ? i : 0));
            xs[m] = i < dv ? x : 0.f;
          }
#pragma unroll
          for (int m = 0; m < kNormPre; ++m)
            if (lane + kWave * m < dv) ss = fmaf(xs[m], xs[m], ss);
          const float inv = gated_norm_inv(ss, dv, sa.eps);
#pragma unroll
          for (int m = 0; m < kNormPre; ++m) {
            const int i = lane + kWave * m;
            if (i < dv) out[row * dv + i] = gated_norm_value<T>(xs[m], inv, wpre[m], zpre[m]);
          }
        } else {
          gated_norm_row<T>([&](int i) { return load_partial(orow + i); }, sa.z + row * dv, sa.norm_w,
                            out + row * dv, dv, sa.eps, lane);
        }
        if (lane == 0) __hip_atomic_store(sa.cnt_row + row, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
  }
}

template <typename T, bool GATED>
int launch(const void* q, const void* k, const void* v, const float* state, const float* g, const float* beta,
           void* out, float* new_state, int batch, int hk, int hv, int dk, int dv, float decay, int qk_norm,
           float q_scale, int qk_bs, int v_bs, hipStream_t stream) {
  dim3 grid((dv + kWave - 1) / kWave, hv, batch);
  auto* kern = dk <= 32 * kWaves ? linear_attention_kernel<T, GATED, 0, 32> : linear_attention_kernel<T, GATED, 0, 64>;
  kern<<<grid, kThreads, 0, stream>>>(static_cast<const T*>(q), static_cast<const T*>(k), static_cast<const T*>(v),
                                      state, g, beta, static_cast<T*>(out), new_state, hk, hv, dk, dv, decay, qk_norm,
                                      q_scale, qk_bs, v_bs, StepArgs<T>{});
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
  MKQ_REQUIRE(size_t(kMaxKeyDim) * value_dim * 4 < (size_t(1) << 31), "linear_attention_decode: value_dim too large");
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
  MKQ_REQUIRE(size_t(kMaxKeyDim) * value_dim * 4 < (size_t(1) << 31), "%s: value_dim too large", fn);
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

// Workspace of the one-launch step: the q/k-head and row arrival counts at
// fixed offsets for every shape (a workspace reused with another shape still
// finds them at zero), then the recurrence output handed to the rows' norms
// (FP32 [B, Hv, Dv]).
constexpr int kMaxStepCounts = 16384;  // per count array: B * Hk and B * Hv
struct StepWs {
  size_t cnt_qk, cnt_row, obuf, total;
};
StepWs step_ws(int batch, int v_heads, int value_dim) {
  StepWs w;
  w.cnt_qk = 0;
  w.cnt_row = size_t(kMaxStepCounts) * sizeof(unsigned);
  w.obuf = 2 * size_t(kMaxStepCounts) * sizeof(unsigned);
  w.total = w.obuf + align256(size_t(batch) * v_heads * value_dim * sizeof(float));
  return w;
}

template <typename T, int NT>
int launch_step(const StepArgs<T>& sa, float* state, const float* g, const float* beta, void* out, int batch,
                int hk, int hv, int dk, int dv, float q_scale, hipStream_t stream) {
  dim3 grid((dv + kWave - 1) / kWave, hv, batch);
  auto* kern = dk <= 32 * kWaves ? linear_attention_kernel<T, true, NT, 32> : linear_attention_kernel<T, true, NT, 64>;
  kern<<<grid, kThreads, 0, stream>>>(nullptr, nullptr, nullptr, state, g, beta, static_cast<T*>(out), state, hk, hv,
                                      dk, dv, 1.0f, 1, q_scale, 0, 0, sa);
  MKQ_LAUNCH_CHECK("linear_attention_kernel (step)");
  return MKQ_OK;
}

template <typename T>
int step_typed(const void* x_mixed, void* conv_state, const void* conv_weight, const void* conv_bias, int s_len,
               float* state, const float* g, const float* beta, const void* z, const void* norm_weight, void* out,
               int batch, int hk, int hv, int dk, int dv, float q_scale, float eps, unsigned char* ws,
               hipStream_t stream) {
  const StepWs w = step_ws(batch, hv, dv);
  StepArgs<T> sa;
  sa.x = static_cast<const T*>(x_mixed);
  sa.conv_state = static_cast<T*>(conv_state);
  sa.conv_w = static_cast<const T*>(conv_weight);
  sa.conv_b = static_cast<const T*>(conv_bias);
  sa.z = static_cast<const T*>(z);
  sa.norm_w = static_cast<const T*>(norm_weight);
  sa.obuf = reinterpret_cast<float*>(ws + w.obuf);
  sa.cnt_qk = reinterpret_cast<unsigned*>(ws + w.cnt_qk);
  sa.cnt_row = reinterpret_cast<unsigned*>(ws + w.cnt_row);
  sa.channels = 2 * hk * dk + hv * dv;
  sa.s_len = s_len;
  sa.eps = eps;
  if (s_len + 1 <= 4) return launch_step<T, 4>(sa, state, g, beta, out, batch, hk, hv, dk, dv, q_scale, stream);
  return launch_step<T, kMaxConvTaps>(sa, state, g, beta, out, batch, hk, hv, dk, dv, q_scale, stream);
}

}  // namespace

extern "C" size_t mkq_linear_attention_step_workspace_bytes(int dtype, int batch, int k_heads, int v_heads,
                                                            int key_dim, int value_dim) {
  if (elt_size(dtype) == 0 || batch <= 0 || k_heads <= 0 || v_heads <= 0 || key_dim <= 0 || value_dim <= 0) return 0;
  return step_ws(batch, v_heads, value_dim).total;
}

// One launch: the conv update, the gated delta rule with q/k L2 norm and the
// gated RMSNorm (linear_attention_kernel with NT > 0).  The workspace holds
// arrival counts that each call leaves at zero, so it is zero-filled once
// before its first use.
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
  MKQ_REQUIRE(conv_state_len < kMaxConvTaps, "%s: conv_state_len %d > %d", fn, conv_state_len, kMaxConvTaps - 1);
  MKQ_REQUIRE(batch <= 65535 && v_heads <= 65535, "%s: batch/heads too large", fn);
  MKQ_REQUIRE(size_t(kMaxKeyDim) * value_dim * 4 < (size_t(1) << 31), "%s: value_dim too large", fn);
  MKQ_REQUIRE(size_t(2) * k_heads * key_dim + size_t(v_heads) * value_dim < (size_t(1) << 31),
              "%s: too many channels", fn);
  if (size_t(batch) * v_heads > size_t(kMaxStepCounts))
    return set_error(MKQ_ERR_UNSUPPORTED, "%s: batch * v_heads %zu > %d", fn, size_t(batch) * v_heads,
                     kMaxStepCounts);
  const size_t need = mkq_linear_attention_step_workspace_bytes(dtype, batch, k_heads, v_heads, key_dim, value_dim);
  MKQ_REQUIRE(need > 0, "%s: unknown dtype %d", fn, dtype);
  MKQ_REQUIRE(workspace && workspace_bytes >= need, "%s: workspace too small", fn);
  MKQ_REQUIRE((reinterpret_cast<uintptr_t>(workspace) & 255u) == 0, "%s: workspace must be 256-byte aligned", fn);
  hipStream_t s = static_cast<hipStream_t>(stream);
  unsigned char* ws = static_cast<unsigned char*>(workspace);
  switch (dtype) {
    case MKQ_DTYPE_BF16:
      return step_typed<bf16_t>(x_mixed, conv_state, conv_weight, conv_bias, conv_state_len, state, g, beta, z,
                                norm_weight, out, batch, k_heads, v_heads, key_dim, value_dim, q_scale, eps, ws, s);
    case MKQ_DTYPE_F16:
      return step_typed<f16_t>(x_mixed, conv_state, conv_weight, conv_bias, conv_state_len, state, g, beta, z,
                               norm_weight, out, batch, k_heads, v_heads, key_dim, value_dim, q_scale, eps, ws, s);
    default:
      return step_typed<float>(x_mixed, conv_state, conv_weight, conv_bias, conv_state_len, state, g, beta, z,
                               norm_weight, out, batch, k_heads, v_heads, key_dim, value_dim, q_scale, eps, ws, s);
  }
}
