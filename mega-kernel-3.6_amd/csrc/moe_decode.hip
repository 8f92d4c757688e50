// Persistent single-launch MoE decode for gfx950 (Qwen3.6-35B-A3B shape:
// hidden 2048, 256 experts, top-8, SwiGLU intermediate 512, one shared expert
// optionally scaled by sigmoid(x_norm . w_sg)).
//
// Semantics of reference.py:16-62 (moe_decode_reference); replaces the
// cooperative kernel of persistent_moe_decode.cu:229-581 and its host wrapper
// :648-860.  One launch, one workgroup per CU, no grid barrier: the phases are
// chained by per-workgroup flags in the workspace.
//
//   phase 0  every WG: issue its router row and shared-expert gate/up rows;
//            RMSNorm of x (FP32, recomputed per WG from L2) into LDS; router
//            logits for its expert rows -> workspace; publish router flag;
//            shared-expert act = silu(g)*u for its shared rows -> workspace.
//   phase 1  wait until every WG's router flag is up; top-k (descending
//            logit, ties to the lower index) + softmax per batch row, one
//            wave per row, repeated in every WG so no result has to be sent
//            back; distinct experts of the batch are listed in expert order.
//   phase 2  issue the first group of routed gate/up rows AND the first group
//            of down-projection rows of this WG's output rows (both known from
//            the routing alone), then compute act = w_route * silu(g) * u for
//            each (expert row, batch row using it); publish act flag.
//   phase 3  wait until every WG's act flag is up; stage act and the shared
//            act in LDS; out[b, h] for this WG's output rows = sum over experts
//            (fixed order) + sigmoid gate * shared down + residual.
//
// Cross-WG data (logits, act, shared act) is written and read with agent-scope
// atomic accesses, which are coherent across the 8 XCD L2s without
// invalidating them; each flag is published with a release store after the
// data.  Flags carry a generation number that every launch derives from the
// workspace itself (WG 0 advances it once all WGs have read it), so repeated
// launches and graph replays need no host-side reset.  Spin-waits are bounded:
// after kSpinLimit polls the kernel records an error code in the workspace
// and finishes without waiting.
//
// Every weight byte is read from HBM once per launch: router, shared expert,
// and the gate/up/down rows of each distinct selected expert (once even when
// several batch rows select it).
#include <math.h>

#include "mkq_host.h"

using namespace mkq;

namespace {

constexpr int kThreads = 512;
constexpr int kWaves = kThreads / kWave;
constexpr int kMaxB = 8;             // batch rows per launch (larger batches are split on the host)
constexpr int kMaxWg = 1024;         // flag slots
constexpr int kMaxHC = 8;            // max 16-byte chunks per lane for a hidden-long row (H <= 512*EPC)
constexpr int kMaxIC = 2;            // max 16-byte chunks per lane for an intermediate-long row (I <= 128*EPC)
constexpr int kGU = 2;               // routed gate/up row pairs in flight per wave
constexpr int kDN = 8;               // down rows in flight per wave
constexpr int kActWindowBytes = 64 * 1024;
constexpr unsigned kSpinLimit = 1u << 22;

// Workspace layout (bytes).
constexpr size_t kOffGen = 0;          // uint32 generation
constexpr size_t kOffErr = 4;          // uint32 error code (1 = spin limit hit)
constexpr size_t kOffRFlag = 256;      // uint32[kMaxWg]
constexpr size_t kOffAFlag = kOffRFlag + 4 * kMaxWg;
constexpr size_t kOffData = kOffAFlag + 4 * kMaxWg;

__host__ __device__ inline int round_up(int a, int b) { return (a + b - 1) / b * b; }

template <typename T>
struct MoeArgs {
  const T* x;
  const T* nw;
  const T* router;
  const T* eg;
  const T* eu;
  const T* ed;
  const T* sg;
  const T* su;
  const T* sd;
  const T* wsg;  // may be null
  T* out;
  int64_t* idx;
  float* wts;
  unsigned char* ws;
  int B, H, E, I, Is, K;
  float eps;
  int add_residual;
  int nwg;
  int rows_per_wg;  // output rows per WG in phase 3
};

struct WsPtrs {
  unsigned* gen;
  unsigned* err;
  unsigned* rflag;
  unsigned* aflag;
  float* logits;  // [B][E]
  float* act;     // [B*K][I]   (b, slot) entries, route weight folded in
  float* sact;    // [B][Is]
};

__host__ __device__ inline WsPtrs ws_ptrs(unsigned char* ws, int B, int E, int I, int K) {
  WsPtrs p;
  p.gen = reinterpret_cast<unsigned*>(ws + kOffGen);
  p.err = reinterpret_cast<unsigned*>(ws + kOffErr);
  p.rflag = reinterpret_cast<unsigned*>(ws + kOffRFlag);
  p.aflag = reinterpret_cast<unsigned*>(ws + kOffAFlag);
  p.logits = reinterpret_cast<float*>(ws + kOffData);
  p.act = p.logits + size_t(B) * E;
  p.sact = p.act + size_t(B) * K * I;
  return p;
}

__device__ __forceinline__ void st_agent(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float ld_agent(const float* p) {
  return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Wave-level wait until flags[0..n) all equal `tag` (bounded).  Returns false
// on timeout.  Followed by a workgroup-scope acquire fence, so later loads are
// issued only after the flags were seen; the data itself is read with
// agent-scope atomic loads.
__device__ bool wait_flags(unsigned* flags, int n, unsigned tag, int lane) {
  unsigned polls = 0;
  while (true) {
    bool ok = true;
    for (int i = lane; i < n; i += kWave) {
      const unsigned f = __hip_atomic_load(flags + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      ok = ok && (f == tag);
    }
    if (__all(ok)) break;
    if (++polls >= kSpinLimit) return false;
    __builtin_amdgcn_s_sleep(1);
  }
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
  return true;
}

// Loads up to MAXC 16-byte chunks per lane of a row of length n (chunk j of
// the lane is chunk lane + 64*j of the row); chunks past the row read as 0.
template <typename T, bool VEC, int MAXC>
__device__ __forceinline__ void load_row(const T* __restrict__ row, int n, int lane, u32x4 (&c)[MAXC]) {
  constexpr int EPC = Epc<T>::value;
  const int nch = (n + EPC - 1) / EPC;
#pragma unroll
  for (int j = 0; j < MAXC; ++j) {
    const int q = lane + kWave * j;
    c[j] = q < nch ? load_chunk_nt<T, VEC>(row, q, n) : u32x4{0u, 0u, 0u, 0u};
  }
}

// Lane-partial dot of the chunks with an FP32 vector in LDS (zero-padded to a
// multiple of EPC).
template <typename T, int MAXC>
__device__ __forceinline__ float dot_row(const u32x4 (&c)[MAXC], const float* __restrict__ v, int n, int lane) {
  constexpr int EPC = Epc<T>::value;
  const int nch = (n + EPC - 1) / EPC;
  float s = 0.f;
#pragma unroll
  for (int j = 0; j < MAXC; ++j) {
    const int q = lane + kWave * j;
    if (q < nch) {
      float f[EPC];
      unpack(c[j], f, T{});
#pragma unroll
      for (int e = 0; e < EPC; ++e) s = fmaf(f[e], v[q * EPC + e], s);
    }
  }
  return s;
}

// Wave argmax over (value desc, index asc).
__device__ __forceinline__ void wave_argmax(float& v, int& i) {
#pragma unroll
  for (int m = 1; m < kWave; m <<= 1) {
    const float ov = __shfl_xor(v, m, kWave);
    const int oi = __shfl_xor(i, m, kWave);
    if (ov > v || (ov == v && oi < i)) {
      v = ov;
      i = oi;
    }
  }
}

// HC / IC: 16-byte chunks per lane of a hidden-long / intermediate-long row.
template <typename T, bool VEC, int HC, int IC>
__global__ __launch_bounds__(kThreads, 1) void moe_decode_kernel(MoeArgs<T> a) {
  constexpr int EPC = Epc<T>::value;
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid / kWave;
  const int wg = blockIdx.x, nwg = a.nwg;
  const int B = a.B, H = a.H, E = a.E, I = a.I, Is = a.Is, K = a.K;
  const int Hp = round_up(H, EPC), Ip = round_up(I, EPC), Isp = round_up(Is, EPC);
  const WsPtrs w = ws_ptrs(a.ws, B, E, I, K);

  // ---- LDS carve-up --------------------------------------------------------
  // region A (phases 0-2): x_norm [B][Hp] ; region A reused in phase 3 for the
  // act window and the shared act.  Small bookkeeping arrays follow.
  const int ulimit = min(E, B * K);
  float* xn = reinterpret_cast<float*>(smem);
  const size_t region_a = size_t(max(B * Hp, kActWindowBytes / 4 + B * Isp));
  float* act_l = xn;                        // [win entries][Ip]
  float* sact_l = xn + kActWindowBytes / 4;  // [B][Isp]
  float* red = xn + region_a;                // [kWaves][2*kMaxB]
  float* sgf = red + kWaves * 2 * kMaxB;     // [kMaxB]
  float* sel_w = sgf + kMaxB;                // [B*K]
  int* sel_e = reinterpret_cast<int*>(sel_w + kMaxB * K);  // [B*K]
  unsigned* emask = reinterpret_cast<unsigned*>(sel_e + kMaxB * K);  // [E]
  int* ulist = reinterpret_cast<int*>(emask + E);                    // [ulimit]
  unsigned* umask = reinterpret_cast<unsigned*>(ulist + ulimit);     // [ulimit]
  int* uslot = reinterpret_cast<int*>(umask + ulimit);               // [ulimit][kMaxB]
  int* misc = uslot + ulimit * kMaxB;                                // [0]=U, [1..kWaves] wave counts, [16] timeout
  float* part = reinterpret_cast<float*>(misc + 32);                 // [rows_per_wg][U+1][B]

  const unsigned gen = __hip_atomic_load(w.gen, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  const unsigned tag = gen + 1;

  // ---- phase 0: issue router / shared gate-up rows --------------------------
  const int e0 = wg + nwg * wave;  // first router row of this wave
  u32x4 rrow[HC];
  if (e0 < E) load_row<T, VEC, HC>(a.router + size_t(e0) * H, H, lane, rrow);
  const int s0 = wg + nwg * (kWaves - 1 - wave);  // first shared gate/up row of this wave
  u32x4 sgr[HC], sur[HC];
  if (s0 < Is) {
    load_row<T, VEC, HC>(a.sg + size_t(s0) * H, H, lane, sgr);
    load_row<T, VEC, HC>(a.su + size_t(s0) * H, H, lane, sur);
  }

  // RMSNorm (FP32) into LDS; x * nw first, then scaled by 1/rms.
  if (tid < E) emask[tid] = 0u;
  for (int e = tid + kThreads; e < E; e += kThreads) emask[e] = 0u;
  {
    float ss[kMaxB];
#pragma unroll
    for (int b = 0; b < kMaxB; ++b) ss[b] = 0.f;
    for (int h = tid; h < Hp; h += kThreads) {
      const float nwv = h < H ? to_f(a.nw[h]) : 0.f;
#pragma unroll
      for (int b = 0; b < kMaxB; ++b)
        if (b < B) {
          const float v = h < H ? to_f(a.x[size_t(b) * H + h]) : 0.f;
          ss[b] = fmaf(v, v, ss[b]);
          xn[b * Hp + h] = v * nwv;
        }
    }
#pragma unroll
    for (int b = 0; b < kMaxB; ++b) {
      const float t = wave_sum(ss[b]);
      if (lane == 0) red[wave * 2 * kMaxB + b] = t;
    }
    __syncthreads();
    float inv[kMaxB];
#pragma unroll
    for (int b = 0; b < kMaxB; ++b) {
      float t = 0.f;
#pragma unroll
      for (int v = 0; v < kWaves; ++v) t += red[v * 2 * kMaxB + b];
      inv[b] = 1.0f / sqrtf(t / float(H) + a.eps);
    }
    float gs[kMaxB];
#pragma unroll
    for (int b = 0; b < kMaxB; ++b) gs[b] = 0.f;
    for (int h = tid; h < Hp; h += kThreads) {
      const float wg_ = (a.wsg != nullptr && h < H) ? to_f(a.wsg[h]) : 0.f;
#pragma unroll
      for (int b = 0; b < kMaxB; ++b)
        if (b < B) {
          const float v = xn[b * Hp + h] * inv[b];
          xn[b * Hp + h] = v;
          gs[b] = fmaf(v, wg_, gs[b]);
        }
    }
#pragma unroll
    for (int b = 0; b < kMaxB; ++b) {
      const float t = wave_sum(gs[b]);
      if (lane == 0) red[wave * 2 * kMaxB + kMaxB + b] = t;
    }
    __syncthreads();
    if (tid < B) {
      float t = 0.f;
      for (int v = 0; v < kWaves; ++v) t += red[v * 2 * kMaxB + kMaxB + tid];
      sgf[tid] = a.wsg != nullptr ? 1.0f / (1.0f + expf(-t)) : 1.0f;
    }
  }

  // Router logits of this wave's rows.
  for (int e = e0, r = 0; e < E; e += nwg * kWaves, ++r) {
    if (r > 0) load_row<T, VEC, HC>(a.router + size_t(e) * H, H, lane, rrow);
#pragma unroll
    for (int b = 0; b < kMaxB; ++b)
      if (b < B) {
        const float s = wave_sum(dot_row<T, HC>(rrow, xn + b * Hp, H, lane));
        if (lane == 0) st_agent(w.logits + size_t(b) * E + e, s);
      }
  }
  // Each wave makes its own stores visible at agent scope before the barrier;
  // only then does one thread raise the WG's flag.
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
  __syncthreads();
  if (tid == 0) __hip_atomic_store(w.rflag + wg, tag, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);

  // Shared-expert gate/up of this wave's rows (published with the act flag).
  for (int s = s0, r = 0; s < Is; s += nwg * kWaves, ++r) {
    if (r > 0) {
      load_row<T, VEC, HC>(a.sg + size_t(s) * H, H, lane, sgr);
      load_row<T, VEC, HC>(a.su + size_t(s) * H, H, lane, sur);
    }
#pragma unroll
    for (int b = 0; b < kMaxB; ++b)
      if (b < B) {
        const float g = wave_sum(dot_row<T, HC>(sgr, xn + b * Hp, H, lane));
        const float u = wave_sum(dot_row<T, HC>(sur, xn + b * Hp, H, lane));
        if (lane == 0) st_agent(w.sact + size_t(b) * Is + s, silu(g) * u);
      }
  }

  // ---- phase 1: wait for all router logits, top-k ---------------------------
  if (wave == 0) {
    const bool ok = wait_flags(w.rflag, nwg, tag, lane);
    if (lane == 0) misc[16] = ok ? 0 : 1;
    if (!ok && lane == 0) __hip_atomic_store(w.err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  __syncthreads();
  bool timed_out = misc[16] != 0;
  if (wg == 0 && tid == 0 && !timed_out) {
    // Every WG read `gen` before raising its router flag: advance it for the next launch.
    __hip_atomic_store(w.gen, tag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  if (wave < B) {
    const int b = wave;
    constexpr int kMaxEL = 16;  // experts per lane (E <= 1024)
    float v[kMaxEL];
#pragma unroll
    for (int j = 0; j < kMaxEL; ++j) {
      const int e = lane + kWave * j;
      v[j] = (e < E && !timed_out) ? ld_agent(w.logits + size_t(b) * E + e) : -INFINITY;
    }
    unsigned taken = 0u;
    float first = 0.f, denom = 0.f;
    for (int s = 0; s < K; ++s) {
      float bv = -INFINITY;
      int bi = 0x7fffffff;
#pragma unroll
      for (int j = 0; j < kMaxEL; ++j) {
        const int e = lane + kWave * j;
        if (e < E && !((taken >> j) & 1u) && (v[j] > bv || (v[j] == bv && e < bi))) {
          bv = v[j];
          bi = e;
        }
      }
      wave_argmax(bv, bi);
      if (bi < E && (bi & (kWave - 1)) == lane) taken |= 1u << (bi / kWave);
      if (s == 0) first = bv;
      const float ex = expf(bv - first);
      denom += ex;
      if (lane == 0) {
        sel_e[b * K + s] = bi < E ? bi : 0;
        sel_w[b * K + s] = ex;
      }
    }
    if (lane == 0) {
      const float inv = 1.0f / denom;
      for (int s = 0; s < K; ++s) {
        sel_w[b * K + s] *= inv;
        atomicOr(&emask[sel_e[b * K + s]], 1u << b);
        if (wg == 0) {
          a.idx[size_t(b) * K + s] = sel_e[b * K + s];
          a.wts[size_t(b) * K + s] = sel_w[b * K + s];
        }
      }
    }
  }
  __syncthreads();
  // Compact the selected experts in expert order (ballot prefix per wave).
  {
    int cnt_before = 0;
    for (int base = 0; base < E; base += kThreads) {
      const int e = base + tid;
      const bool used = e < E && emask[e] != 0u;
      const unsigned long long bal = __ballot(used);
      if (lane == 0) misc[1 + wave] = __popcll(bal);
      __syncthreads();
      int off = cnt_before;
      for (int v = 0; v < wave; ++v) off += misc[1 + v];
      int tot = cnt_before;
      for (int v = 0; v < kWaves; ++v) tot += misc[1 + v];
      if (used) {
        const int pos = off + __popcll(bal & ((1ull << lane) - 1ull));
        ulist[pos] = e;
        umask[pos] = emask[e];
      }
      cnt_before = tot;
      __syncthreads();
    }
    if (tid == 0) misc[0] = cnt_before;
  }
  __syncthreads();
  const int U = misc[0];
  // slot of expert u in batch row b (route weight lives in sel_w[b*K+slot]).
  for (int t = tid; t < U * kMaxB; t += kThreads) {
    const int u = t / kMaxB, b = t % kMaxB;
    int slot = -1;
    if (b < B)
      for (int s = 0; s < K; ++s)
        if (sel_e[b * K + s] == ulist[u]) slot = s;
    uslot[t] = slot;
  }
  __syncthreads();

  // ---- phase 2: routed gate/up (+ early issue of the down rows) -------------
  const int nw_total = nwg * kWaves;
  const int gw = wave * nwg + wg;  // global wave id, consecutive ids on different WGs
  const int ntask = U * I;
  // down pairs of this WG: (output row hl, expert u) for u < U, index p = hl*U + u
  const int h0 = wg * a.rows_per_wg;
  const int nrows = max(0, min(a.rows_per_wg, H - h0));
  const int npairs = nrows * U;

  u32x4 dn[kDN][IC];
#pragma unroll
  for (int j = 0; j < kDN; ++j) {
    const int p = wave + kWaves * j;
    if (p < npairs) {
      const int hl = p / U, u = p % U;
      load_row<T, VEC, IC>(a.ed + (size_t(ulist[u]) * H + h0 + hl) * I, I, lane, dn[j]);
    }
  }
  // shared down row of this wave (one output row per wave, rest later)
  u32x4 sdn[IC];
  if (wave < nrows) load_row<T, VEC, IC>(a.sd + size_t(h0 + wave) * Is, Is, lane, sdn);

  for (int t0 = gw; t0 < ntask; t0 += nw_total * kGU) {
    u32x4 gr[kGU][HC], ur[kGU][HC];
#pragma unroll
    for (int q = 0; q < kGU; ++q) {
      const int t = t0 + q * nw_total;
      if (t < ntask) {
        const int u = t / I, i = t % I;
        const size_t ro = (size_t(ulist[u]) * I + i) * H;
        load_row<T, VEC, HC>(a.eg + ro, H, lane, gr[q]);
        load_row<T, VEC, HC>(a.eu + ro, H, lane, ur[q]);
      }
    }
#pragma unroll
    for (int q = 0; q < kGU; ++q) {
      const int t = t0 + q * nw_total;
      if (t < ntask) {
        const int u = t / I, i = t % I;
        const unsigned mask = umask[u];
#pragma unroll
        for (int b = 0; b < kMaxB; ++b)
          if ((mask >> b) & 1u) {
            const float g = wave_sum(dot_row<T, HC>(gr[q], xn + b * Hp, H, lane));
            const float u_ = wave_sum(dot_row<T, HC>(ur[q], xn + b * Hp, H, lane));
            if (lane == 0) {
              const int slot = uslot[u * kMaxB + b];
              const float rw = sel_w[b * K + slot];
              st_agent(w.act + (size_t(b) * K + slot) * I + i, rw * silu(g) * u_);
            }
          }
      }
    }
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
  __syncthreads();
  if (tid == 0) __hip_atomic_store(w.aflag + wg, tag, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);

  // ---- phase 3: wait for all act, down projection ---------------------------
  if (wave == 0) {
    const bool ok = timed_out ? false : wait_flags(w.aflag, nwg, tag, lane);
    if (lane == 0) misc[17] = ok ? 0 : 1;
    if (!ok && lane == 0) __hip_atomic_store(w.err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  __syncthreads();
  timed_out = misc[17] != 0;

  // shared act -> LDS
  for (int t = tid; t < B * Isp; t += kThreads) {
    const int b = t / Isp, i = t % Isp;
    sact_l[t] = (i < Is && !timed_out) ? ld_agent(w.sact + size_t(b) * Is + i) : 0.f;
  }
  // act windows: experts [u_lo, u_hi) whose (b, slot) entries fit the window
  const int win_entries = max(1, (kActWindowBytes / 4) / Ip);
  int u_lo = 0, jdone = 0;
  // entry index of (u, b) inside a window: running count of set mask bits
  while (u_lo < U) {
    int u_hi = u_lo, ent = 0;
    while (u_hi < U && (ent + __popc(umask[u_hi]) <= win_entries || u_hi == u_lo)) {
      ent += __popc(umask[u_hi]);
      ++u_hi;
    }
    __syncthreads();  // previous window fully consumed
    // stage entries of experts [u_lo, u_hi): entry order = (u, b ascending)
    for (int t = tid; t < ent * Ip; t += kThreads) {
      const int en = t / Ip, i = t % Ip;
      int u = u_lo, cnt = 0, bsel = 0;
      for (; u < u_hi; ++u) {
        const int pc = __popc(umask[u]);
        if (en < cnt + pc) break;
        cnt += pc;
      }
      unsigned m = umask[u];
      for (int k2 = en - cnt; k2 > 0; --k2) m &= m - 1u;
      bsel = __ffs(m) - 1;
      const int slot = uslot[u * kMaxB + bsel];
      act_l[t] = (i < I && !timed_out) ? ld_agent(w.act + (size_t(bsel) * K + slot) * I + i) : 0.f;
    }
    __syncthreads();
    // pairs of this window handled by this wave: p = wave + kWaves*j over all
    // pairs (hl, u); only u in [u_lo, u_hi) are computed now.
    for (int j = 0;; ++j) {
      const int p = wave + kWaves * j;
      if (p >= npairs) break;
      const int hl = p / U, u = p % U;
      if (u < u_lo || u >= u_hi) continue;
      u32x4 c[IC];
      if (j < kDN) {
#pragma unroll
        for (int jj = 0; jj < kDN; ++jj)
          if (jj == j)
#pragma unroll
            for (int q = 0; q < IC; ++q) c[q] = dn[jj][q];
      } else {
        load_row<T, VEC, IC>(a.ed + (size_t(ulist[u]) * H + h0 + hl) * I, I, lane, c);
      }
      // window entry offset of expert u
      int en = 0;
      for (int v = u_lo; v < u; ++v) en += __popc(umask[v]);
      const unsigned mask = umask[u];
#pragma unroll
      for (int b = 0; b < kMaxB; ++b)
        if ((mask >> b) & 1u) {
          const float s = wave_sum(dot_row<T, IC>(c, act_l + size_t(en) * Ip, I, lane));
          if (lane == 0) part[(hl * (U + 1) + u) * kMaxB + b] = s;
          ++en;
        }
    }
    u_lo = u_hi;
    ++jdone;
  }
  // shared down rows
  for (int hl = wave; hl < nrows; hl += kWaves) {
    u32x4 c[IC];
    if (hl == wave) {
#pragma unroll
      for (int q = 0; q < IC; ++q) c[q] = sdn[q];
    } else {
      load_row<T, VEC, IC>(a.sd + size_t(h0 + hl) * Is, Is, lane, c);
    }
#pragma unroll
    for (int b = 0; b < kMaxB; ++b)
      if (b < B) {
        const float s = wave_sum(dot_row<T, IC>(c, sact_l + b * Isp, Is, lane));
        if (lane == 0) part[(hl * (U + 1) + U) * kMaxB + b] = s;
      }
  }
  __syncthreads();
  // combine: out[b, h] = sum_u part (expert order) + gate * shared + residual
  for (int t = tid; t < nrows * B; t += kThreads) {
    const int hl = t / B, b = t % B;
    float s = 0.f;
    for (int u = 0; u < U; ++u)
      if ((umask[u] >> b) & 1u) s += part[(hl * (U + 1) + u) * kMaxB + b];
    s = fmaf(sgf[b], part[(hl * (U + 1) + U) * kMaxB + b], s);
    const size_t o = size_t(b) * H + h0 + hl;
    if (a.add_residual) s += to_f(a.x[o]);
    a.out[o] = from_f<T>(timed_out ? NAN : s);
  }
}

size_t lds_bytes(int B, int H, int E, int I, int Is, int K, int epc, int rows_per_wg) {
  const int Hp = round_up(H, epc), Isp = round_up(Is, epc);
  const int ulimit = E < B * K ? E : B * K;
  size_t region_a = size_t(B) * Hp;
  const size_t r3 = size_t(kActWindowBytes / 4) + size_t(B) * Isp;
  if (r3 > region_a) region_a = r3;
  size_t n = region_a + kWaves * 2 * kMaxB + kMaxB + kMaxB * K;  // floats
  n += kMaxB * K + E + ulimit + ulimit + size_t(ulimit) * kMaxB + 32;  // ints
  n += size_t(rows_per_wg) * (ulimit + 1) * kMaxB;
  (void)I;
  return n * 4;
}

template <typename T>
int launch(const MoeArgs<T>& args0, int batch, hipStream_t stream) {
  constexpr int EPC = Epc<T>::value;
  MoeArgs<T> a = args0;
  const int ncu = cu_count();
  int nwg = ncu < kMaxWg ? ncu : kMaxWg;
  a.nwg = nwg;
  a.rows_per_wg = (a.H + nwg - 1) / nwg;
  const bool vec = (a.H % EPC == 0) && (a.I % EPC == 0) && (a.Is % EPC == 0) && aligned16(a.router) &&
                   aligned16(a.eg) && aligned16(a.eu) && aligned16(a.ed) && aligned16(a.sg) && aligned16(a.su) &&
                   aligned16(a.sd);
  const size_t lds = lds_bytes(kMaxB, a.H, a.E, a.I, a.Is, a.K, EPC, a.rows_per_wg);
  if (lds > size_t(max_lds_per_block()))
    return set_error(MKQ_ERR_UNSUPPORTED, "moe_decode: shape needs %zu bytes of LDS (> %d)", lds, max_lds_per_block());
  // Chunk counts per lane: the smallest instantiation that covers the rows.
  const int hc_need = (a.H + EPC * kWave - 1) / (EPC * kWave);
  const int ic_need = (max(a.I, a.Is) + EPC * kWave - 1) / (EPC * kWave);
  void (*kern)(MoeArgs<T>) = nullptr;
  if (vec && hc_need <= 4 && ic_need <= 1)
    kern = &moe_decode_kernel<T, true, 4, 1>;
  else if (vec)
    kern = &moe_decode_kernel<T, true, kMaxHC, kMaxIC>;
  else
    kern = &moe_decode_kernel<T, false, kMaxHC, kMaxIC>;
  static bool attr_set[3] = {false, false, false};
  const int which = (vec && hc_need <= 4 && ic_need <= 1) ? 0 : (vec ? 1 : 2);
  if (!attr_set[which]) {
    MKQ_HIP_TRY(hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize,
                                    max_lds_per_block()));
    attr_set[which] = true;
  }
  for (int b0 = 0; b0 < batch; b0 += kMaxB) {
    a.B = batch - b0 < kMaxB ? batch - b0 : kMaxB;
    a.x = args0.x + size_t(b0) * a.H;
    a.out = args0.out + size_t(b0) * a.H;
    a.idx = args0.idx + size_t(b0) * a.K;
    a.wts = args0.wts + size_t(b0) * a.K;
    kern<<<nwg, kThreads, lds, stream>>>(a);
    MKQ_LAUNCH_CHECK("moe_decode_kernel");
  }
  return MKQ_OK;
}

}  // namespace

extern "C" size_t mkq_moe_decode_workspace_bytes(int batch, int hidden, int experts, int intermediate,
                                                 int shared_intermediate, int top_k) {
  (void)batch;
  (void)hidden;
  if (experts <= 0 || intermediate <= 0 || shared_intermediate <= 0 || top_k <= 0) return 0;
  const size_t data = sizeof(float) * (size_t(kMaxB) * experts + size_t(kMaxB) * top_k * intermediate +
                                       size_t(kMaxB) * shared_intermediate);
  return kOffData + data;
}

extern "C" int mkq_moe_decode(int dtype, const void* x, const void* norm_weight, const void* router_weight,
                              const void* expert_gate, const void* expert_up, const void* expert_down,
                              const void* shared_gate, const void* shared_up, const void* shared_down,
                              const void* shared_expert_gate, void* out, int64_t* indices, float* weights, int batch,
                              int hidden, int experts, int intermediate, int shared_intermediate, int top_k,
                              float eps, int add_residual, void* workspace, size_t workspace_bytes, void* stream) {
  clear_error();
  MKQ_REQUIRE(batch > 0 && hidden > 0 && experts > 0 && intermediate > 0 && shared_intermediate > 0,
              "moe_decode: sizes must be positive");
  MKQ_REQUIRE(top_k > 0 && top_k <= experts, "top_k must be in [1, experts]");
  MKQ_REQUIRE(x && norm_weight && router_weight && expert_gate && expert_up && expert_down && shared_gate &&
                  shared_up && shared_down && out && indices && weights,
              "moe_decode: null tensor pointer");
  MKQ_REQUIRE(workspace && workspace_bytes >= mkq_moe_decode_workspace_bytes(batch, hidden, experts, intermediate,
                                                                              shared_intermediate, top_k),
              "moe_decode: workspace too small");
  MKQ_REQUIRE((reinterpret_cast<uintptr_t>(workspace) & 255u) == 0, "moe_decode: workspace must be 256-byte aligned");
  if (experts > 1024 || top_k > 64)
    return set_error(MKQ_ERR_UNSUPPORTED, "moe_decode: experts <= 1024 and top_k <= 64 are supported");
  const int maxh = 8 * kWave * kMaxHC / (dtype == MKQ_DTYPE_F32 ? 2 : 1);
  const int maxi = 8 * kWave * kMaxIC / (dtype == MKQ_DTYPE_F32 ? 2 : 1);
  if (hidden > maxh || intermediate > maxi || shared_intermediate > maxi)
    return set_error(MKQ_ERR_UNSUPPORTED, "moe_decode: hidden <= %d and intermediate <= %d are supported", maxh, maxi);
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (dtype) {
#define MKQ_MOE_CASE(CODE, TYPE)                                                                                   \
  case CODE: {                                                                                                     \
    MoeArgs<TYPE> a{};                                                                                             \
    a.x = static_cast<const TYPE*>(x);                                                                             \
    a.nw = static_cast<const TYPE*>(norm_weight);                                                                  \
    a.router = static_cast<const TYPE*>(router_weight);                                                            \
    a.eg = static_cast<const TYPE*>(expert_gate);                                                                  \
    a.eu = static_cast<const TYPE*>(expert_up);                                                                    \
    a.ed = static_cast<const TYPE*>(expert_down);                                                                  \
    a.sg = static_cast<const TYPE*>(shared_gate);                                                                  \
    a.su = static_cast<const TYPE*>(shared_up);                                                                    \
    a.sd = static_cast<const TYPE*>(shared_down);                                                                  \
    a.wsg = static_cast<const TYPE*>(shared_expert_gate);                                                          \
    a.out = static_cast<TYPE*>(out);                                                                               \
    a.idx = indices;                                                                                               \
    a.wts = weights;                                                                                               \
    a.ws = static_cast<unsigned char*>(workspace);                                                                 \
    a.H = hidden;                                                                                                  \
    a.E = experts;                                                                                                 \
    a.I = intermediate;                                                                                            \
    a.Is = shared_intermediate;                                                                                    \
    a.K = top_k;                                                                                                   \
    a.eps = eps;                                                                                                   \
    a.add_residual = add_residual;                                                                                 \
    return launch<TYPE>(a, batch, s);                                                                              \
  }
    MKQ_MOE_CASE(MKQ_DTYPE_BF16, bf16_t)
    MKQ_MOE_CASE(MKQ_DTYPE_F16, f16_t)
    MKQ_MOE_CASE(MKQ_DTYPE_F32, float)
#undef MKQ_MOE_CASE
    default:
      return set_error(MKQ_ERR_INVALID, "moe_decode: unknown dtype %d", dtype);
  }
}
