// Persistent single-launch MoE decode for gfx950 (Qwen3.6-35B-A3B shape:
// hidden 2048, 256 experts, top-8, SwiGLU intermediate 512, one shared expert
// optionally scaled by sigmoid(x_norm . w_sg)).
//
// Semantics of reference.py:16-62 (moe_decode_reference); replaces the
// cooperative kernel of persistent_moe_decode.cu:229-581 and its host wrapper
// :648-860.  One launch, one workgroup (8 waves) per CU, no grid barrier.
//
//   phase 0  every WG issues x, its router row and its shared-expert gate/up
//            rows; RMSNorm (FP32) into LDS; router logits of its rows and the
//            shared-expert act of its rows are published.
//   phase 1  one wave per batch row gathers all router logits, then top-k
//            (descending logit, ties to the lower index) and softmax over the
//            k logits.  Every WG repeats this, so nothing is sent back; the
//            distinct experts of the batch are listed in expert order.
//   phase 2  each wave issues its routed gate/up rows AND the down-projection
//            rows of its WG's output rows (both known from the routing alone)
//            before computing act = w_route * silu(g) * u, which it publishes.
//   phase 3  the WG gathers act and the shared act into LDS and finishes its
//            output rows: sum over experts (fixed order) + gate * shared
//            down + residual.
//
// Hand-off between WGs: every published value is one 64-bit word {float bits,
// generation tag}, written with a single agent-coherent store and read with
// agent-coherent (sc1) loads, which see other XCDs' stores without any cache
// invalidation.  A reader that sees the current tag has the current value (an
// aligned 8-byte store is seen whole), so there are no flags, no fences and
// no waits for store completion.  The tag is the workspace's generation word
// + 1; every WG also publishes a tagged presence word, and WG 0 advances the
// generation at its very end, once all presence words carry the tag (so every
// WG has read it).  Repeated launches and graph replays need no reset.  Waits are bounded (kSpinLimit polls); on timeout the
// kernel records an error code in the workspace, writes NaN and finishes.
//
// Every weight byte is read from HBM once per launch: router, shared expert,
// and the gate/up/down rows of each distinct selected expert (once even when
// several batch rows select it).
#include <math.h>

#include <mutex>

#include "mkq_host.h"

using namespace mkq;

namespace {

constexpr int kThreads = 512;
constexpr int kWaves = kThreads / kWave;
constexpr int kMaxB = 8;       // batch rows per launch (larger batches are split on the host)
constexpr int kMaxWg = 1024;   // workgroups
constexpr int kMaxHC = 8;      // max 16-byte chunks per lane for a hidden-long row (H <= 512*EPC)
constexpr int kMaxIC = 2;      // max 16-byte chunks per lane for an intermediate-long row (I <= 128*EPC)
constexpr int kGU = 2;         // routed gate/up row pairs per wave and load group (one-row path)
constexpr int kGUM = 1;        // the same for the multi-row path, whose per-row state needs the registers
constexpr int kDN = 8;         // down rows issued per wave before the act hand-off
constexpr int kRB = 8;         // output rows per block in the multi-row down phase (kRB * kMaxB == 64 lanes)
constexpr int kMaxEL = 16;     // router logits per lane (E <= 1024)
constexpr unsigned kSpinLimit = 1u << 21;
constexpr int kMaxDevCache = 64;  // devices whose residency check is cached

// Workspace layout (bytes).  The generation and error words live in their own
// 256-byte lines; the tagged arrays follow, each 256-byte aligned.
constexpr size_t kOffGen = 0;                         // uint32 generation
constexpr size_t kOffErr = 256;                       // uint32 error code (1 = a wait timed out)
constexpr size_t kOffPresence = 512;                  // uint64[kMaxWg] tagged
constexpr size_t kOffData = kOffPresence + 8 * kMaxWg;

// Phase timestamps, compiled only into profiling builds (-DMKQ_MOE_TRACE):
// lane 0 of every wave stores the 100 MHz real-time counter at numbered
// points into trace[(wg * kWaves + wave) * 16 + point], a kernel argument
// (held in scalar registers, so a mark adds no wait for earlier loads).
#ifdef MKQ_MOE_TRACE
#define MOE_MARK(n)                                                                 \
  do {                                                                              \
    if (lane == 0 && a.trace != nullptr)                                            \
      a.trace[(size_t(blockIdx.x) * kWaves + wave) * 16 + (n)] = wall_clock64();    \
  } while (0)
uint64_t* g_trace = nullptr;  // host side: the buffer given to mkq_moe_set_trace
#else
#define MOE_MARK(n) \
  do {              \
  } while (0)
#endif

__host__ __device__ inline int round_up(int a, int b) { return (a + b - 1) / b * b; }
__host__ __device__ inline size_t align256(size_t v) { return (v + 255) & ~size_t(255); }

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
  int win_floats;   // act window of the multi-row down phase (floats, a multiple of round_up(I, EPC))
#ifdef MKQ_MOE_TRACE
  uint64_t* trace;
#endif
};

// Every published array (router logits, act, shared act) is written in
// kCopies copies, one per XCD (workgroup wg runs on XCD wg % 8), each read by
// that XCD's workgroups only: every workgroup polls the whole array, and 256
// pollers of one array queue at the few memory channels that hold it.  The
// copies are an odd number of 256-byte lines apart, so they sit on different
// channels.  A copy's words are written by lanes 0..kCopies-1 of one store.
constexpr int kCopies = 8;
__host__ __device__ inline size_t copy_words(size_t bytes) { return (align256(bytes) + 256) / 8; }
__host__ __device__ inline size_t logit_copy_words(int E) { return copy_words(8 * size_t(kMaxB) * E); }
__host__ __device__ inline size_t act_copy_words(int K, int I) { return copy_words(8 * size_t(kMaxB) * K * I); }
__host__ __device__ inline size_t sact_copy_words(int Is) { return copy_words(8 * size_t(kMaxB) * Is); }

struct WsPtrs {
  unsigned* gen;
  unsigned* err;
  uint64_t* presence;  // [nwg]   tagged
  uint64_t* logits;  // [kCopies][B][E] tagged, copies logit_copy_words(E) apart
  uint64_t* act;     // [kCopies][B*K][I] tagged, (b, slot) rows, route weight folded in
  uint64_t* sact;    // [kCopies][B][Is]  tagged
};

__host__ __device__ inline WsPtrs ws_ptrs(unsigned char* ws, int E, int I, int Is, int K) {
  WsPtrs p;
  p.gen = reinterpret_cast<unsigned*>(ws + kOffGen);
  p.err = reinterpret_cast<unsigned*>(ws + kOffErr);
  p.presence = reinterpret_cast<uint64_t*>(ws + kOffPresence);
  size_t off = kOffData;
  p.logits = reinterpret_cast<uint64_t*>(ws + off);
  off = align256(off + 8 * kCopies * logit_copy_words(E));
  p.act = reinterpret_cast<uint64_t*>(ws + off);
  off = align256(off + 8 * kCopies * act_copy_words(K, I));
  p.sact = reinterpret_cast<uint64_t*>(ws + off);
  (void)Is;
  return p;
}

__host__ __device__ inline size_t ws_bytes(int E, int I, int Is, int K) {
  size_t off = kOffData;
  off = align256(off + 8 * kCopies * logit_copy_words(E));
  off = align256(off + 8 * kCopies * act_copy_words(K, I));
  off = align256(off + 8 * kCopies * sact_copy_words(Is));
  return off;
}



// Loads up to MAXC 16-byte chunks per lane of a row of length n (chunk j of
// the lane is chunk lane + 64*j of the row); chunks past the row, and every
// chunk of a row with valid == false, read as 0.  The vector path uses one
// buffer descriptor sized to the row, so there is no branch around the loads
// and all of them stay in flight together.
template <typename T, bool VEC, int MAXC>
__device__ __forceinline__ void load_row(const T* __restrict__ row, int n, bool valid, int lane, u32x4 (&c)[MAXC]) {
  constexpr int EPC = Epc<T>::value;
  if constexpr (VEC) {
    const rsrc_t r = make_rsrc(row, valid ? uint32_t(n) * uint32_t(sizeof(T)) : 0u);
#pragma unroll
    for (int j = 0; j < MAXC; ++j) c[j] = buf_load16<kAuxStream>(r, uint32_t(lane + kWave * j) * 16u);
  } else {
    const int nch = (n + EPC - 1) / EPC;
#pragma unroll
    for (int j = 0; j < MAXC; ++j) {
      const int q = lane + kWave * j;
      c[j] = (valid && q < nch) ? load_chunk<T, false>(row, q, n) : u32x4{0u, 0u, 0u, 0u};
    }
  }
}

// Lane-partial dot of the chunks with an FP32 vector in LDS (zero-padded to a
// multiple of EPC).  Branch-free: a chunk past the row was loaded as zeros,
// so it is multiplied with the (finite) last chunk of the vector instead of
// being skipped.
// One accumulator per chunk keeps the FMA chains short (they run in
// parallel); the chunk sums are added pairwise at the end.  The vector is read
// as float4s: every LDS vector handed in here is 16-byte aligned, and
// 16-byte reads keep the 32-byte lane stride to a 2-way bank conflict, where
// the 8-byte pair reads the compiler otherwise emits serialise much further.
template <typename T, int MAXC>
__device__ __forceinline__ float dot_row(const u32x4 (&c)[MAXC], const float* __restrict__ v, int n, int lane) {
  constexpr int EPC = Epc<T>::value;
  const int last = (n + EPC - 1) / EPC - 1;
  float s[MAXC];
#pragma unroll
  for (int j = 0; j < MAXC; ++j) {
    const int q = min(lane + kWave * j, last);
    float f[EPC];
    unpack(c[j], f, T{});
    const float4* p = reinterpret_cast<const float4*>(v + q * EPC);
    float vv[EPC];
#pragma unroll
    for (int h = 0; h < EPC / 4; ++h) {
      const float4 t = p[h];
      vv[4 * h] = t.x;
      vv[4 * h + 1] = t.y;
      vv[4 * h + 2] = t.z;
      vv[4 * h + 3] = t.w;
    }
    s[j] = 0.f;
#pragma unroll
    for (int e = 0; e < EPC; ++e) s[j] = fmaf(f[e], vv[e], s[j]);
  }
#pragma unroll
  for (int st = 1; st < MAXC; st *= 2)
#pragma unroll
    for (int j = 0; j + st < MAXC; j += 2 * st) s[j] += s[j + st];
  return s[0];
}

// Gathers `pairs` pairs of tagged words (word 2p, 2p+1 of the array behind
// `r`, pair p taken from pair index src(p)) into `dst` floats, waiting until
// every word carries `tag`.  Each thread waits only for its own words; the
// caller's barrier then makes the whole set visible to the workgroup.
// Returns false on timeout.
template <typename SrcFn>
__device__ bool gather_tagged_pairs(rsrc_t r, int pairs, SrcFn src, float* dst, unsigned tag, int tid) {
  bool ok = true;
  for (int f0 = tid; f0 < pairs; f0 += 4 * kThreads) {
    u32x4 v[4];
    uint32_t off[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int f = f0 + q * kThreads;
      off[q] = f < pairs ? src(f) : 0xFFFFFFF0u;
    }
    unsigned polls = 0;
    while (true) {
#pragma unroll
      for (int q = 0; q < 4; ++q) v[q] = buf_load16<kAuxCoherent>(r, off[q]);
      bool ready = true;
#pragma unroll
      for (int q = 0; q < 4; ++q)
        ready = ready & (off[q] == 0xFFFFFFF0u || (v[q].y == tag && v[q].w == tag));
      if (ready) break;
      if (++polls >= kSpinLimit) {
        ok = false;
        break;
      }
      __builtin_amdgcn_s_sleep(1);
    }
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int f = f0 + q * kThreads;
      if (f < pairs) {
        dst[2 * f] = __uint_as_float(v[q].x);
        dst[2 * f + 1] = __uint_as_float(v[q].z);
      }
    }
  }
  return ok;
}

// Routes one batch row (one wave): waits until the E tagged logits behind `lr`
// carry `tag`, then takes the top K by (logit descending, index ascending) --
// the reference's order and tie rule -- and the softmax over those K logits.
// Lane s < K returns slot s (expert, route weight).  Lane l holds the logits of
// experts EL*l .. EL*l + EL-1 (16-byte loads of two tagged words each), sorted
// in the lane; a round is then one wave-wide max of the lane heads and a
// ballot for the lowest lane holding it, after which that lane pops its head.
// on_slot(s, my_e) runs right after round s (lane s then holds slot s), so a
// caller can hand out a slot while the later rounds run.  Returns false
// (experts 0) if the wait timed out.
template <int EL, typename OnSlot>
__device__ bool route_row(rsrc_t lr, int E, int K, unsigned tag, int lane, int& my_e, float& my_w, OnSlot on_slot) {
  u32x4 word[EL / 2];
  bool ok = true;
  for (unsigned polls = 0;;) {
#pragma unroll
    for (int m = 0; m < EL / 2; ++m) word[m] = buf_load16<kAuxCoherent>(lr, uint32_t(EL * lane + 2 * m) * 8u);
    bool ready = true;
#pragma unroll
    for (int m = 0; m < EL / 2; ++m) {
      const int e = EL * lane + 2 * m;
      ready = ready & (e >= E || word[m].y == tag) & (e + 1 >= E || word[m].w == tag);
    }
    if (__all(ready)) break;
    if (++polls >= kSpinLimit) {
      ok = false;
      break;
    }
    __builtin_amdgcn_s_sleep(1);
  }
  uint32_t key[EL];
  int kid[EL];
#pragma unroll
  for (int m = 0; m < EL / 2; ++m) {
    const int e = EL * lane + 2 * m;
    key[2 * m] = (ok && e < E) ? ord_key(__uint_as_float(word[m].x)) : 0u;
    key[2 * m + 1] = (ok && e + 1 < E) ? ord_key(__uint_as_float(word[m].z)) : 0u;
    kid[2 * m] = e;
    kid[2 * m + 1] = e + 1;
  }
  // Odd-even transposition sort of the lane's EL keys.
#pragma unroll
  for (int r = 0; r < EL; ++r)
#pragma unroll
    for (int j = r & 1; j + 1 < EL; j += 2) {
      const bool sw = key[j + 1] > key[j] || (key[j + 1] == key[j] && kid[j + 1] < kid[j]);
      const uint32_t k0 = key[j], k1 = key[j + 1];
      const int i0 = kid[j], i1 = kid[j + 1];
      key[j] = sw ? k1 : k0;
      key[j + 1] = sw ? k0 : k1;
      kid[j] = sw ? i1 : i0;
      kid[j + 1] = sw ? i0 : i1;
    }
  float my_v = 0.f;
  my_e = 0;
  for (int s = 0; s < K; ++s) {
    const uint32_t best = wave_max_u32(key[0]);
    const unsigned long long m = __ballot(key[0] == best);
    const int L = m != 0ull ? int(__builtin_ctzll(m)) : 0;
    const int e = __builtin_amdgcn_readlane(kid[0], L);
    const bool pop = lane == L;
#pragma unroll
    for (int j = 0; j + 1 < EL; ++j) {
      key[j] = pop ? key[j + 1] : key[j];
      kid[j] = pop ? kid[j + 1] : kid[j];
    }
    key[EL - 1] = pop ? 0u : key[EL - 1];
    if (lane == s) {
      my_e = (best != 0u && e < E) ? e : 0;  // 0 = absent (timed-out wait)
      my_v = ord_value(best);
    }
    on_slot(s, my_e);
  }
  // Slot 0 holds the largest logit; exp(v_s - v_0) summed in slot order.
  const float first = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(my_v), 0));
  const float ex = lane < K ? expf(my_v - first) : 0.f;
  float denom = 0.f;
  for (int s = 0; s < K; ++s) denom += __int_as_float(__builtin_amdgcn_readlane(__float_as_int(ex), s));
  my_w = ex / denom;
  return ok;
}

// HC / IC: 16-byte chunks per lane of a hidden-long / intermediate-long row.
// MB: largest batch of this instantiation (1 = the single-token fast path).
// EL: router logits held per lane in the top-k (E <= 64*EL).
template <typename T, bool VEC, int HC, int IC, int MB, int EL>
__global__ __launch_bounds__(kThreads, 1) void moe_decode_kernel(MoeArgs<T> a) {
  constexpr int EPC = Epc<T>::value;
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = wave_id();
  const int wg = blockIdx.x, nwg = a.nwg;
  MOE_MARK(0);
  const int B = a.B, H = a.H, E = a.E, I = a.I, Is = a.Is, K = a.K;
  const int Hp = round_up(H, EPC), Ip = round_up(I, EPC), Isp = round_up(Is, EPC);
  const WsPtrs w = ws_ptrs(a.ws, E, I, Is, K);

  // ---- LDS carve-up --------------------------------------------------------
  // region A: x_norm [B][Hp] (phases 0-2); reused in phase 3 for the act
  // window [entries][Ip] and the shared act [B][Isp].
  const int ulimit = min(E, B * K);
  float* xn = reinterpret_cast<float*>(smem);
  const size_t region_a = size_t(max(B * Hp, a.win_floats + B * Isp));
  float* act_l = xn;
  float* sact_l = xn + a.win_floats;
  float* red = xn + region_a;                                        // [kWaves][2*MB]
  float* sgf = red + kWaves * 2 * MB;                             // [MB]
  float* sel_w = sgf + MB;                                        // [MB*K]
  int* sel_e = reinterpret_cast<int*>(sel_w + MB * K);            // [MB*K]
  unsigned* emask = reinterpret_cast<unsigned*>(sel_e + MB * K);  // [E]
  int* ulist = reinterpret_cast<int*>(emask + E);                    // [ulimit]
  unsigned* umask = reinterpret_cast<unsigned*>(ulist + ulimit);     // [ulimit]
  int* uslot = reinterpret_cast<int*>(umask + ulimit);               // [ulimit][MB]
  int* ent_src = uslot + ulimit * MB;                             // [MB*K] act rows of a window
  int* ent_of = ent_src + MB * K;                                 // [ulimit][MB] window entry of (u, b)
  int* misc = ent_of + ulimit * MB;  // [0]=U, [1..kWaves] counts, [16] error, [17] sticky error at launch,
                                     // [18] one-row routing progress
  float* part = reinterpret_cast<float*>(misc + 32);                 // [rows_per_wg][MB] running sums
  int* ent_base = reinterpret_cast<int*>(part + a.rows_per_wg * MB);  // [ulimit + 1] first entry of expert u

  // ---- phase 0 -------------------------------------------------------------

  // x and the norm weight first: loads complete in order, so the norm waits
  // only for these, not for the weight rows issued after them.
  const int hq = Hp / EPC;
  u32x4 xc[4], nc[4], gc[4];
  const rsrc_t gsr = make_rsrc(a.wsg, a.wsg != nullptr ? uint32_t(H) * uint32_t(sizeof(T)) : 0u);
  if constexpr (VEC) {
    const rsrc_t nr = make_rsrc(a.nw, uint32_t(H) * uint32_t(sizeof(T)));
    if constexpr (MB == 1) {
      const rsrc_t xr = make_rsrc(a.x, uint32_t(B) * uint32_t(H) * uint32_t(sizeof(T)));
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int q = tid + r * kThreads;
        xc[r] = buf_load16(xr, q < B * hq ? uint32_t(q) * 16u : 0xFFFFFFF0u);
        nc[r] = buf_load16(nr, uint32_t(q % hq) * 16u);
        gc[r] = buf_load16(gsr, uint32_t(q % hq) * 16u);
      }
    } else {
      // Several rows: wave b normalises batch row b (chunk lane + 64 r).
      const rsrc_t xr = make_rsrc(a.x + size_t(min(wave, B - 1)) * H, wave < B ? uint32_t(H) * uint32_t(sizeof(T)) : 0u);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const uint32_t off = uint32_t(lane + kWave * r) * 16u;
        xc[r] = buf_load16(xr, off);
        nc[r] = buf_load16(nr, off);
        gc[r] = buf_load16(gsr, off);
      }
    }
  }
  // Generation of this launch (advanced by WG 0 at the end of the previous
  // one).  Loaded by every thread (no branch) after x, so the norm does not
  // wait for it; the tag is first used after the norm.
  const unsigned gen = __hip_atomic_load(w.gen, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  // A wait of an earlier launch on this workspace timed out: its tagged words
  // and generation can no longer be trusted, so every launch writes NaN and
  // leaves without publishing anything until the host clears the workspace
  // (mkq_moe_decode_status with reset).  Taken through LDS after the first
  // barrier, so the whole workgroup takes the same branch.  Thread 0 stores
  // it into LDS only after the norm: a store under `tid == 0` here made the
  // compiler wait for every load issued so far (x, the norm weight, w_sg)
  // before wave 0 issued its router row.
  const unsigned err_at_start = __hip_atomic_load(w.err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  // The residual of this wave's (first) output row, fetched now: after the
  // expert weights have streamed through, x is no longer in the L2, and a
  // load at the end would add a cold round trip to the tail.  Several batch
  // rows: lane b holds batch row b's value (clamped in range, so no branch).
  float x_res = 0.f;
  if constexpr (MB == 1) {
    x_res = to_f(a.x[min(wg * a.rows_per_wg + wave, H - 1)]);
  } else {
    x_res = to_f(a.x[size_t(min(lane, B - 1)) * H + min(wg * a.rows_per_wg + wave, H - 1)]);
  }
  // Router and shared gate/up rows: one row per wave (rows wg + nwg * w) with
  // one batch row; with several batch rows, wave b takes every router and
  // shared row of the WG (rows wg + nwg * j) for batch row b.
  const int e0 = MB == 1 ? wg + nwg * wave : wg;  // first router row of this wave
  const int rstep = MB == 1 ? nwg * kWaves : nwg;
  const bool rows_on = MB == 1 || wave < B;
  u32x4 rrow[HC];
  load_row<T, VEC, HC>(a.router + size_t(min(e0, E - 1)) * H, H, e0 < E && rows_on, lane, rrow);
  const int s0 = MB == 1 ? wg + nwg * (kWaves - 1 - wave) : wg;  // first shared gate/up row of this wave
  const int h0 = wg * a.rows_per_wg;
  const int nrows = max(0, min(a.rows_per_wg, H - h0));
  // Shared-expert gate/up rows and the shared down row of this wave's first
  // output row are independent of the routing.  The multi-row path fetches
  // the gate/up rows now; the one-row path only once its router logits are
  // out, so that the router rows do not queue behind 6 MB of shared-expert
  // rows, and fetches its shared down row with them.  The multi-row path
  // fetches its down row at the end of the gate/up phase (held from here it
  // would stay live through every phase of that register-heavy instance).
  u32x4 sgr[HC], sur[HC], sdn[IC];
  auto issue_shared_gu = [&]() {
    load_row<T, VEC, HC>(a.sg + size_t(min(s0, Is - 1)) * H, H, s0 < Is && rows_on, lane, sgr);
    load_row<T, VEC, HC>(a.su + size_t(min(s0, Is - 1)) * H, H, s0 < Is && rows_on, lane, sur);
  };
  auto issue_shared_down = [&]() {
    load_row<T, VEC, IC>(a.sd + size_t(min(h0 + wave, H - 1)) * Is, Is, wave < nrows, lane, sdn);
  };
  if constexpr (MB > 1) issue_shared_gu();
  pin_loads();

  if constexpr (MB > 1) {
    for (int e = tid; e < E; e += kThreads) emask[e] = 0u;
    // Wave b: RMSNorm of batch row b into LDS and its shared-gate dot; no
    // other wave reads the row before the routing barrier.
    if (tid == 0) {
      misc[16] = 0;
      misc[17] = int(err_at_start);
    }
    if (wave < B) {
      float* xr_l = xn + wave * Hp;
      float ss = 0.f;
      auto sq_chunk = [&](int c, const u32x4& xq, const u32x4& nq) {
        float xf[EPC], nf[EPC];
        unpack(xq, xf, T{});
        unpack(nq, nf, T{});
#pragma unroll
        for (int e = 0; e < EPC; ++e) ss = fmaf(xf[e], xf[e], ss);
        if (c < hq) {
          float4* dst = reinterpret_cast<float4*>(xr_l + c * EPC);
#pragma unroll
          for (int h = 0; h < EPC / 4; ++h)
            dst[h] = make_float4(xf[4 * h] * nf[4 * h], xf[4 * h + 1] * nf[4 * h + 1], xf[4 * h + 2] * nf[4 * h + 2],
                                 xf[4 * h + 3] * nf[4 * h + 3]);
        }
      };
      if constexpr (VEC) {
#pragma unroll
        for (int r = 0; r < 4; ++r) sq_chunk(lane + kWave * r, xc[r], nc[r]);
        if constexpr (HC > 4) {
          const rsrc_t xr = make_rsrc(a.x + size_t(wave) * H, uint32_t(H) * uint32_t(sizeof(T)));
          const rsrc_t nr = make_rsrc(a.nw, uint32_t(H) * uint32_t(sizeof(T)));
          for (int c = lane + 4 * kWave; c < hq; c += kWave)
            sq_chunk(c, buf_load16(xr, uint32_t(c) * 16u), buf_load16(nr, uint32_t(c) * 16u));
        }
      } else {
        for (int h = lane; h < Hp; h += kWave) {
          const float v = h < H ? to_f(a.x[size_t(wave) * H + h]) : 0.f;
          const float nwv = h < H ? to_f(a.nw[h]) : 0.f;
          ss = fmaf(v, v, ss);
          xr_l[h] = v * nwv;
        }
      }
      const float inv = 1.0f / sqrtf(wave_sum_u(ss) / float(H) + a.eps);
      float dg = 0.f;
      if constexpr (VEC) {
        auto scale_chunk = [&](int c, const u32x4& gq) {
          if (c >= hq) return;
          float gf[EPC];
          unpack(gq, gf, T{});
          float4* xv = reinterpret_cast<float4*>(xr_l + c * EPC);
#pragma unroll
          for (int h = 0; h < EPC / 4; ++h) {
            float4 v = xv[h];
            v.x *= inv;
            v.y *= inv;
            v.z *= inv;
            v.w *= inv;
            xv[h] = v;
            dg = fmaf(v.x, gf[4 * h], dg);
            dg = fmaf(v.y, gf[4 * h + 1], dg);
            dg = fmaf(v.z, gf[4 * h + 2], dg);
            dg = fmaf(v.w, gf[4 * h + 3], dg);
          }
        };
#pragma unroll
        for (int r = 0; r < 4; ++r) scale_chunk(lane + kWave * r, gc[r]);
        if constexpr (HC > 4)
          for (int c = lane + 4 * kWave; c < hq; c += kWave) scale_chunk(c, buf_load16(gsr, uint32_t(c) * 16u));
      } else {
        for (int h = lane; h < Hp; h += kWave) {
          const float v = xr_l[h] * inv;
          xr_l[h] = v;
          dg = fmaf(v, (a.wsg != nullptr && h < H) ? to_f(a.wsg[h]) : 0.f, dg);
        }
      }
      const float t = wave_sum_u(dg);
      if (lane == 0) sgf[wave] = a.wsg != nullptr ? 1.0f / (1.0f + expf(-t)) : 1.0f;
    }
    __syncthreads();  // emask and misc cleared before phase 1
  } else   {
    float ss[MB], gs[MB];
#pragma unroll
    for (int b = 0; b < MB; ++b) ss[b] = gs[b] = 0.f;
    if constexpr (VEC) {
      // chunk q = (row q / hq, chunk q % hq); the first 4*512 chunks were
      // loaded above and are processed outside the loop (so their waits are
      // exact), any beyond (B*H > 16384 elements) are loaded in the loop.
      auto sq_batch = [&](int q0) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int q = q0 + r * kThreads;
          if (q < B * hq) {
            const int b = q / hq, c = q % hq;
            float xf[EPC], nf[EPC];
            unpack(xc[r], xf, T{});
            unpack(nc[r], nf, T{});
            float sq = 0.f;
            float4* dst = reinterpret_cast<float4*>(xn + b * Hp + c * EPC);
#pragma unroll
            for (int h = 0; h < EPC / 4; ++h) {
#pragma unroll
              for (int e = 4 * h; e < 4 * h + 4; ++e) sq = fmaf(xf[e], xf[e], sq);
              dst[h] = make_float4(xf[4 * h] * nf[4 * h], xf[4 * h + 1] * nf[4 * h + 1], xf[4 * h + 2] * nf[4 * h + 2],
                                   xf[4 * h + 3] * nf[4 * h + 3]);
            }
#pragma unroll
            for (int bb = 0; bb < MB; ++bb) ss[bb] += bb == b ? sq : 0.f;
          }
        }
      };
      sq_batch(tid);
      // With HC <= 4 (H <= 2048 for 16-bit types) and B <= 8 every chunk is
      // in the first batch; compiling the loop out keeps the waits exact.
      if constexpr (HC > 4)
      for (int q0 = tid + 4 * kThreads; q0 < B * hq; q0 += 4 * kThreads) {
        const rsrc_t xr = make_rsrc(a.x, uint32_t(B) * uint32_t(H) * uint32_t(sizeof(T)));
        const rsrc_t nr = make_rsrc(a.nw, uint32_t(H) * uint32_t(sizeof(T)));
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int q = q0 + r * kThreads;
          xc[r] = buf_load16(xr, q < B * hq ? uint32_t(q) * 16u : 0xFFFFFFF0u);
          nc[r] = buf_load16(nr, uint32_t(q % hq) * 16u);
        }
        sq_batch(q0);
      }
    } else {
      for (int h = tid; h < Hp; h += kThreads) {
        const float nwv = h < H ? to_f(a.nw[h]) : 0.f;
#pragma unroll
        for (int b = 0; b < MB; ++b)
          if (b < B) {
            const float v = h < H ? to_f(a.x[size_t(b) * H + h]) : 0.f;
            ss[b] = fmaf(v, v, ss[b]);
            xn[b * Hp + h] = v * nwv;
          }
      }
    }
#pragma unroll
    for (int b = 0; b < MB; ++b) {
      const float t = wave_sum_u(ss[b]);
      if (lane == 0) red[wave * 2 * MB + b] = t;
    }
    __syncthreads();
    float inv[MB];
#pragma unroll
    for (int b = 0; b < MB; ++b) {
      float t = 0.f;
#pragma unroll
      for (int v = 0; v < kWaves; ++v) t += red[v * 2 * MB + b];
      inv[b] = 1.0f / sqrtf(t / float(H) + a.eps);
    }
    // Scale to x_norm in place; dot with the shared-expert gate vector.
    if constexpr (VEC) {
      auto scale_batch = [&](int q0) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int q = q0 + r * kThreads;
          if (q < B * hq) {
            const int b = q / hq, c = q % hq;
            float gf[EPC];
            unpack(gc[r], gf, T{});
            float ib = 0.f;
#pragma unroll
            for (int bb = 0; bb < MB; ++bb) ib = bb == b ? inv[bb] : ib;
            float dg = 0.f;
            float4* xv = reinterpret_cast<float4*>(xn + b * Hp + c * EPC);
#pragma unroll
            for (int h = 0; h < EPC / 4; ++h) {
              float4 v = xv[h];
              v.x *= ib;
              v.y *= ib;
              v.z *= ib;
              v.w *= ib;
              xv[h] = v;
              dg = fmaf(v.x, gf[4 * h], dg);
              dg = fmaf(v.y, gf[4 * h + 1], dg);
              dg = fmaf(v.z, gf[4 * h + 2], dg);
              dg = fmaf(v.w, gf[4 * h + 3], dg);
            }
#pragma unroll
            for (int bb = 0; bb < MB; ++bb) gs[bb] += bb == b ? dg : 0.f;
          }
        }
      };
      scale_batch(tid);  // the first 4*512 chunks' gate vector was loaded at the start
      if constexpr (HC > 4)
      for (int q0 = tid + 4 * kThreads; q0 < B * hq; q0 += 4 * kThreads) {
#pragma unroll
        for (int r = 0; r < 4; ++r) gc[r] = buf_load16(gsr, uint32_t((q0 + r * kThreads) % hq) * 16u);
        scale_batch(q0);
      }
    } else {
      for (int h = tid; h < Hp; h += kThreads) {
        const float wg_ = (a.wsg != nullptr && h < H) ? to_f(a.wsg[h]) : 0.f;
#pragma unroll
        for (int b = 0; b < MB; ++b)
          if (b < B) {
            const float v = xn[b * Hp + h] * inv[b];
            xn[b * Hp + h] = v;
            gs[b] = fmaf(v, wg_, gs[b]);
          }
      }
    }
#pragma unroll
    for (int b = 0; b < MB; ++b) {
      const float t = wave_sum_u(gs[b]);
      if (lane == 0) red[wave * 2 * MB + MB + b] = t;
    }
    if (tid == 0) {
      misc[16] = 0;
      misc[17] = int(err_at_start);
      misc[18] = 0;  // one-row routing: K + 1 once the route weights are in LDS
    }
    if (MB == 1 && tid < K) sel_e[tid] = 0;  // one-row routing: slot tid's expert + 1, 0 until decided
    __syncthreads();
    MOE_MARK(1);
    if (tid < B) {
      float t = 0.f;
      for (int v = 0; v < kWaves; ++v) t += red[v * 2 * MB + MB + tid];
      sgf[tid] = a.wsg != nullptr ? 1.0f / (1.0f + expf(-t)) : 1.0f;
    }
  }
  if (misc[17] != 0) {
    for (int t = tid; t < B * nrows; t += kThreads) a.out[size_t(t / nrows) * H + h0 + t % nrows] = from_f<T>(NAN);
    if (wg == 0)
      for (int t = tid; t < B * K; t += kThreads) {
        a.idx[t] = 0;
        a.wts[t] = NAN;
      }
    return;
  }
  const unsigned tag = gen + 1u;
  if (tid == 0) put_tagged(w.presence + wg, 0.f, tag);
  // WG 0 advances the generation once every WG of this launch has read it
  // (its presence word carries the tag).  Nothing of this launch reads the
  // generation word after its start, so this may run as soon as every WG is
  // known to have started: the one-row instance runs it in wave 1 of WG 0,
  // which reaches the end of its gate/up rows ~1 us before the workgroup's
  // last wave, so the check's round trip is off the kernel's tail.
  auto advance_gen = [&]() {
    const rsrc_t pr = make_rsrc(w.presence, uint32_t(nwg) * 8u);
    bool seen = false;
    for (unsigned polls = 0; polls < kSpinLimit && !seen; ++polls) {
      bool ready = true;
      for (int q = lane; q < (nwg + 1) / 2; q += kWave) {
        const u32x4 v = buf_load16<kAuxCoherent>(pr, uint32_t(q) * 16u);
        ready = ready & (v.y == tag) & (2 * q + 1 >= nwg || v.w == tag);
      }
      seen = __all(ready);
      if (!seen) __builtin_amdgcn_s_sleep(1);
    }
    // After a timed-out wait the generation is left alone: the error word
    // keeps every later launch out of the tagged arrays until a reset.
    if (lane == 0) {
      if (!seen)
        __hip_atomic_store(w.err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      else
        __hip_atomic_store(w.gen, tag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  };
  // This XCD's copies of the published act and shared act.  The multi-row
  // path publishes B times as many act words and keeps one copy: there the
  // extra stores cost more than the shorter wait saves.
  constexpr int kActCopies = MB == 1 ? kCopies : 1;
  uint64_t* const act_r = w.act + (wg % kActCopies) * act_copy_words(K, I);
  uint64_t* const sact_r = w.sact + (wg % kActCopies) * sact_copy_words(Is);

  // Router logits of this wave's rows.  The one-row instance owns at most one
  // router row and one shared row per wave (the host checks E and Is against
  // the wave count), so its code has no loads here: loads in a branch that
  // most waves skip make the compiler wait at the join for the loads issued
  // before it.
  if constexpr (MB == 1) {
    if (e0 < E) {
      const float s = wave_sum_u(dot_row<T, HC>(rrow, xn, H, lane));
      if (lane < kCopies) put_tagged(w.logits + lane * logit_copy_words(E) + e0, s, tag);
      MOE_MARK(2);
    }
  } else if (wave < B) {
    for (int e = e0, r = 0; e < E; e += rstep, ++r) {
      if (r > 0) load_row<T, VEC, HC>(a.router + size_t(e) * H, H, true, lane, rrow);
      const float s = wave_sum_u(dot_row<T, HC>(rrow, xn + wave * Hp, H, lane));
      if (lane < kCopies) put_tagged(w.logits + lane * logit_copy_words(E) + size_t(wave) * E + e, s, tag);
    }
  }
  // Shared-expert gate/up of this wave's rows.  The one-row path runs this
  // after issuing its routed loads: the shared rows arrive behind the router
  // row, and the routing must not wait for them.
  auto publish_shared = [&]() {
    if constexpr (MB == 1) {
      if (s0 < Is) {
        float g = dot_row<T, HC>(sgr, xn, H, lane);
        float u = dot_row<T, HC>(sur, xn, H, lane);
        wave_sum2_u(g, u);
        if (lane < kActCopies) put_tagged(w.sact + lane * sact_copy_words(Is) + s0, silu(g) * u, tag);
      }
      return;
    }
    if (wave >= B) return;
    for (int s = s0, r = 0; s < Is; s += rstep, ++r) {
      if (r > 0) {
        load_row<T, VEC, HC>(a.sg + size_t(s) * H, H, true, lane, sgr);
        load_row<T, VEC, HC>(a.su + size_t(s) * H, H, true, lane, sur);
      }
      float g = dot_row<T, HC>(sgr, xn + wave * Hp, H, lane);
      float u = dot_row<T, HC>(sur, xn + wave * Hp, H, lane);
      wave_sum2_u(g, u);
      if (lane < kActCopies) put_tagged(w.sact + lane * sact_copy_words(Is) + size_t(wave) * Is + s, silu(g) * u, tag);
    }
  };
  // The multi-row instance publishes its shared-expert act in phase 2, after
  // its first routed gate/up rows are issued: the loop loads a second row
  // pair cold (Is > nwg), and waiting for it here held the routing back by
  // ~2 us at B = 8.

  if constexpr (MB == 1) {
    // Shared rows (and this wave's 1 KB shared down row, used in phase 3) are
    // fetched while the logits are exchanged, after the router rows are in --
    // except by wave 0, which polls for the logits: a wave's loads return in
    // issue order, so each of its polls would wait for every row issued before
    // it.  Waves without a shared row issue no placeholder loads (a load past
    // a descriptor's end reads zero but still takes a memory round trip).
    if (wave != 0) {
      if (s0 < Is) issue_shared_gu();
      issue_shared_down();
    }
    pin_loads();
    // ---- phases 1-2, one batch row ---------------------------------------------
    // Wave 0 gathers all logits and routes (one polling wave per WG keeps the
    // coherent read traffic of the exchange 8x lower than every wave polling;
    // the top-k rounds are bound by the SIMD's issue rate, so a second
    // routing wave on a SIMD would slow both).  Lane l holds the logits of
    // experts EL*l .. EL*l + EL-1 (16-byte loads of two tagged words each),
    // sorted in the lane by (logit descending, index ascending).  A top-k
    // round is then one wave-wide max of the lane heads and a ballot for the
    // lowest lane holding it -- the lowest expert index among equal logits,
    // the reference's tie rule -- after which that lane pops its head.
    // After round s wave 0 writes slot s's expert + 1 into the slot's LDS
    // word (one store, no ordering wait inside the round); each wave issues
    // its first group of gate/up rows as soon as the words of the group's
    // slots are set, while the later rounds run.  A counter reaches K + 1
    // once the route weights (softmax over the K selected logits) are in LDS
    // too.
    int* const ready = misc + 18;
    // The round after which every slot of this wave's first group is known.
    // Wave 0 runs the rounds, so it takes the groups of the last wave (the
    // last slot at the batch-1 shape) and issues no loads inside the rounds:
    // issuing there waited on the CU's memory queue (~0.3 us) and delayed
    // every later round.
    const int nw_total = nwg * kWaves;
    const int gw = ((wave + kWaves - 1) % kWaves) * nwg + wg;
    const int ntask = K * I;
    const int first_ready = min(K - 1, min(gw * kGU + kGU - 1, ntask - 1) / I);
    auto slot_expert = [&](int u) { return __builtin_amdgcn_readfirstlane(sel_e[u]) - 1; };
    auto slot_weight = [&](int u) { return sel_w[u]; };
    const size_t hrow = size_t(min(h0 + wave, H - 1));

    // Routed gate/up: tasks t = (slot t / I, row t % I) in groups of kGU
    // consecutive tasks; wave gw takes groups gw, gw + nw_total, ...  At the
    // batch-1 shape (K * I = 2 * nwg * kWaves) a wave's one group lies in one
    // slot: wave w of every WG reads rows of slot w.
    auto issue_gu = [&](int grp, u32x4 (&g)[kGU][HC], u32x4 (&u)[kGU][HC]) {
#pragma unroll
      for (int q = 0; q < kGU; ++q) {
        const int t = grp * kGU + q;
        const int tc = min(t, ntask - 1);
        const size_t ro = (size_t(slot_expert(tc / I)) * I + tc % I) * H;
        load_row<T, VEC, HC>(a.eg + ro, H, t < ntask, lane, g[q]);
        load_row<T, VEC, HC>(a.eu + ro, H, t < ntask, lane, u[q]);
      }
    };
    auto compute_gu = [&](int grp, const u32x4 (&g)[kGU][HC], const u32x4 (&u)[kGU][HC]) {
#pragma unroll
      for (int q = 0; q < kGU; ++q) {
        const int t = grp * kGU + q;
        if (t < ntask) {
          const int su = t / I, i = t % I;
          float gv = dot_row<T, HC>(g[q], xn, H, lane);
          float uv = dot_row<T, HC>(u[q], xn, H, lane);
          wave_sum2_u(gv, uv);
          if (lane < kActCopies)
            put_tagged(w.act + lane * act_copy_words(K, I) + size_t(su) * I + i, slot_weight(su) * silu(gv) * uv, tag);
        }
      }
    };
    // Waits (bounded; wave 0 always gets there) until the counter passes n.
    auto wait_ready = [&](int n) {
      for (unsigned polls = 0; polls < kSpinLimit; ++polls) {
        if (__hip_atomic_load(ready, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP) > n) break;
        __builtin_amdgcn_s_sleep(1);
      }
    };
    // Waits (bounded) until slots 0..n are decided.  Wave 0 writes the slot
    // words in order, and one wave's LDS stores land in issue order.
    auto wait_slot = [&](int n) {
      for (unsigned polls = 0; polls < kSpinLimit; ++polls) {
        if (__hip_atomic_load(sel_e + n, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) != 0) break;
        __builtin_amdgcn_s_sleep(1);
      }
    };
    u32x4 gA[kGU][HC], uA[kGU][HC], gB[kGU][HC], uB[kGU][HC];
    if (wave == 0) {
      int my_e;
      float my_w;
      const bool routed =
          route_row<EL>(make_rsrc(w.logits + (wg % kCopies) * logit_copy_words(E), uint32_t(E) * 8u), E, K, tag,
                        lane, my_e, my_w, [&](int s, int e) {
                          if (lane == s)  // lane s holds slot s's expert
                            __hip_atomic_store(sel_e + s, e + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
                        });
      if (!routed && lane == 0) misc[16] = 1;
      if (lane < K) sel_w[lane] = my_w;
      if (lane == 0) __hip_atomic_store(ready, K + 1, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
      if (wg == 0 && lane < K) {
        a.idx[lane] = my_e;
        a.wts[lane] = my_w;
      }
      // Wave 0's own rows only now: by this time the other waves' rows fill
      // the CU's memory queue, and an issue that waits for queue space must
      // not hold back the route weights every wave needs.
      issue_gu(gw, gA, uA);
      pin_loads();
      if (s0 < Is) issue_shared_gu();
      issue_shared_down();
      pin_loads();
    } else {
      wait_slot(first_ready);
      issue_gu(gw, gA, uA);
      pin_loads();
    }
    wait_ready(K);  // route weights in LDS (and every slot word)
    MOE_MARK(3);
    // Shared-expert act of the waves that own a shared row (its rows arrived
    // long ago), before their routed rows: phase 3 needs both.  This code
    // issues no loads (one shared row per wave), so it adds no wait for the
    // gate/up rows just issued.
    publish_shared();
    for (int grp = gw; grp * kGU < ntask; grp += 2 * nw_total) {
      if ((grp + nw_total) * kGU < ntask) issue_gu(grp + nw_total, gB, uB);
      pin_loads();
      compute_gu(grp, gA, uA);
      if ((grp + nw_total) * kGU >= ntask) break;
      if ((grp + 2 * nw_total) * kGU < ntask) issue_gu(grp + 2 * nw_total, gA, uA);
      pin_loads();
      compute_gu(grp + nw_total, gB, uB);
    }
    MOE_MARK(4);
    if (wg == 0 && wave == 1) advance_gen();
    // Down rows of (this wave's output row, expert of slot s): needed only
    // after the act exchange, so they are issued once the whole WG's gate/up
    // rows are consumed and stream during the exchange.  A CU serves its
    // loads at a bounded rate, so down rows issued by its early waves would
    // delay the gate/up rows of its late waves, which the exchange waits for
    // (-1.8 us at batch 1 with the barrier).
    __syncthreads();
    u32x4 dn[kDN][IC];
#pragma unroll
    for (int s = 0; s < kDN; ++s)
      load_row<T, VEC, IC>(a.ed + (size_t(slot_expert(min(s, K - 1))) * H + hrow) * I, I, s < K && wave < nrows, lane,
                           dn[s]);
    pin_loads();

    // ---- phase 3, one batch row ----------------------------------------------
    // act [K][Ip] and the shared act [Isp] sit after x_norm in LDS (the host
    // checks they fit), so no barrier is needed before gathering them.
    float* act1 = xn + Hp;
    float* sact1 = act1 + size_t(K) * Ip;
    bool ok3 = true;
    if constexpr (VEC) {
      const int hpi = Ip / 2, hps = Isp / 2;  // word pairs per row
      ok3 = gather_tagged_pairs(
          make_rsrc(sact_r, uint32_t(Is) * 8u), hps,
          [&](int f) -> uint32_t { return 2 * f < Is ? uint32_t(2 * f) * 8u : 0xFFFFFFF0u; }, sact1, tag, tid);
      ok3 = gather_tagged_pairs(
                make_rsrc(act_r, uint32_t(K) * uint32_t(I) * 8u), K * hpi,
                [&](int f) -> uint32_t {
                  const int en = f / hpi, c2 = (f % hpi) * 2;
                  return c2 < I ? uint32_t(en * I + c2) * 8u : 0xFFFFFFF0u;
                },
                act1, tag, tid) &&
            ok3;
    } else {
      for (int t = tid; t < Isp + K * Ip; t += kThreads) {
        const bool is_sact = t < Isp;
        const int en = is_sact ? 0 : (t - Isp) / Ip, i = is_sact ? t : (t - Isp) % Ip;
        const int n = is_sact ? Is : I;
        float val = 0.f;
        if (i < n) {
          const uint64_t* pw = is_sact ? sact_r + i : act_r + size_t(en) * I + i;
          uint64_t word64 = 0;
          for (unsigned polls = 0; polls < kSpinLimit; ++polls) {
            word64 = __hip_atomic_load(const_cast<uint64_t*>(pw), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            if (unsigned(word64 >> 32) == tag) break;
            __builtin_amdgcn_s_sleep(1);
          }
          ok3 = ok3 && unsigned(word64 >> 32) == tag;
          val = __uint_as_float(unsigned(word64));
        }
        if (is_sact)
          sact1[i] = val;
        else
          act1[size_t(en) * Ip + i] = val;
      }
    }
    if (!ok3) misc[16] = 1;
    __syncthreads();
    MOE_MARK(5);
    const bool timed_out = misc[16] != 0;
    if (timed_out && tid == 0) __hip_atomic_store(w.err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    // Wave w owns output rows h0 + w, h0 + w + kWaves, ...: experts in slot
    // order (the reference's order), then the gated shared expert and the
    // residual.
    // Lane-partial sums of all experts and of the gated shared expert, then a
    // single wave reduction (the per-expert partials are independent chains).
    for (int hl = wave; hl < nrows; hl += kWaves) {
      float part = 0.f;
      int u0 = 0;
      if (hl == wave) {
        // rows of slots >= K were loaded as zeros
        float pe[kDN];
#pragma unroll
        for (int uu = 0; uu < kDN; ++uu) pe[uu] = dot_row<T, IC>(dn[uu], act1 + size_t(min(uu, K - 1)) * Ip, I, lane);
#pragma unroll
        for (int st = 1; st < kDN; st *= 2)
#pragma unroll
          for (int j = 0; j + st < kDN; j += 2 * st) pe[j] += pe[j + st];
        part = pe[0];
        u0 = kDN;
      }
      for (int u = u0; u < K; ++u) {
        u32x4 c[IC];
        load_row<T, VEC, IC>(a.ed + (size_t(slot_expert(u)) * H + h0 + hl) * I, I, true, lane, c);
        part += dot_row<T, IC>(c, act1 + size_t(u) * Ip, I, lane);
      }
      u32x4 c[IC];
      if (hl == wave) {
#pragma unroll
        for (int q = 0; q < IC; ++q) c[q] = sdn[q];
      } else {
        load_row<T, VEC, IC>(a.sd + size_t(h0 + hl) * Is, Is, true, lane, c);
      }
      float s = wave_sum_u(fmaf(sgf[0], dot_row<T, IC>(c, sact1, Is, lane), part));
      const size_t o = size_t(h0 + hl);
      if (lane == 0) {
        if (a.add_residual) s += hl == wave ? x_res : to_f(a.x[o]);
        a.out[o] = from_f<T>(timed_out ? NAN : s);
      }
    }
    MOE_MARK(6);
  } else {

  // ---- phase 1: gather the router logits, top-k -----------------------------
  // Wave b routes batch row b.
  if (wave < B) {
    const int b = wave;
    int my_e;
    float my_w;
    if (!route_row<EL>(make_rsrc(w.logits + (wg % kCopies) * logit_copy_words(E) + size_t(b) * E,
                                 uint32_t(E) * 8u),
                       E, K, tag, lane, my_e, my_w, [](int, int) {}) &&
        lane == 0) {
      misc[16] = 1;
      __hip_atomic_store(w.err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    if (lane < K) {
      sel_e[b * K + lane] = my_e;
      sel_w[b * K + lane] = my_w;
      if constexpr (MB > 1) atomicOr(&emask[my_e], 1u << b);
      if (wg == 0) {
        a.idx[size_t(b) * K + lane] = my_e;
        a.wts[size_t(b) * K + lane] = my_w;
      }
    }
  }
  __syncthreads();
  // Distinct experts of the batch.  One row: the K selected experts in slot
  // order.  Several rows: compacted in expert order (ballot prefix per wave).
  if constexpr (MB == 1) {
    if (tid < K) {
      ulist[tid] = sel_e[tid];
      umask[tid] = 1u;
    }
    if (tid == 0) misc[0] = K;
  } else {
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
  bool timed_out = misc[16] != 0;
  // slot of expert u in batch row b (route weight lives in sel_w[b*K+slot]).
  for (int t = tid; t < U * MB; t += kThreads) {
    const int u = t / MB, b = t % MB;
    int slot = -1;
    if constexpr (MB == 1) {
      slot = u;
    } else {
      if (b < B)
        for (int s = 0; s < K; ++s)
          if (sel_e[b * K + s] == ulist[u]) slot = s;
    }
    uslot[t] = slot;
  }
  __syncthreads();
  // Act entries (u, b) in expert order, then batch-row order: entry of
  // (u, b) = ent_base[u] + rank of b among expert u's rows.  The prefix sum
  // over the experts' row counts runs in one wave; the table is filled by all.
  if (wave == 0) {
    int carry = 0;
    for (int u0 = 0; u0 < U; u0 += kWave) {
      const int u = u0 + lane;
      int c = u < U ? __popc(umask[u]) : 0;
      for (int d = 1; d < kWave; d <<= 1) {
        const int v = __shfl_up(c, d, kWave);
        c += lane >= d ? v : 0;
      }
      if (u < U) ent_base[u + 1] = carry + c;
      carry += __shfl(c, kWave - 1, kWave);
    }
    if (lane == 0) ent_base[0] = 0;
  }
  __syncthreads();
  for (int t = tid; t < U * MB; t += kThreads) {
    const int u = t / MB, b = t % MB;
    const unsigned m = umask[u];
    if ((m >> b) & 1u) {
      const int en = ent_base[u] + __popc(m & ((1u << b) - 1u));
      ent_src[en] = b * K + uslot[t];
      ent_of[t] = en;
    }
  }
  __syncthreads();

  // ---- phase 2: routed gate/up (+ early issue of the down rows) -------------
  const int nw_total = nwg * kWaves;
  const int gw = wave * nwg + wg;  // global wave id, consecutive ids on different WGs
  const int ntask = U * I;
  // output rows of this WG in phase 3

  // Task t = (expert u, row i) of the routed gate/up, t = gw + nw_total * m.
  // Loads complete in issue order, so the first gate/up group is issued before
  // the down rows: act is published as soon as its own rows arrive, while the
  // down rows keep streaming during the hand-off.
  const int step = nw_total * kGUM;
  auto issue_gu = [&](int t0, u32x4 (&g)[kGUM][HC], u32x4 (&u)[kGUM][HC]) {
#pragma unroll
    for (int q = 0; q < kGUM; ++q) {
      const int t = t0 + q * nw_total;
      const int tc = min(t, ntask - 1);
      const size_t ro = (size_t(ulist[tc / I]) * I + tc % I) * H;
      load_row<T, VEC, HC>(a.eg + ro, H, t < ntask, lane, g[q]);
      load_row<T, VEC, HC>(a.eu + ro, H, t < ntask, lane, u[q]);
    }
  };
  auto compute_gu = [&](int t0, const u32x4 (&g)[kGUM][HC], const u32x4 (&u)[kGUM][HC]) {
#pragma unroll
    for (int q = 0; q < kGUM; ++q) {
      const int t = t0 + q * nw_total;
      if (t < ntask) {
        const int ue = t / I, i = t % I;
        const unsigned mask = umask[ue];
#pragma unroll
        for (int b = 0; b < MB; ++b)
          if ((mask >> b) & 1u) {
            const float gv = wave_sum_u(dot_row<T, HC>(g[q], xn + b * Hp, H, lane));
            const float uv = wave_sum_u(dot_row<T, HC>(u[q], xn + b * Hp, H, lane));
            if (lane < kActCopies) {
              const int slot = uslot[ue * MB + b];
              put_tagged(w.act + lane * act_copy_words(K, I) + (size_t(b) * K + slot) * I + i,
                         sel_w[b * K + slot] * silu(gv) * uv, tag);
            }
          }
      }
    }
  };
  u32x4 gA[kGUM][HC], uA[kGUM][HC], gB[kGUM][HC], uB[kGUM][HC];
  issue_gu(gw, gA, uA);
  pin_loads();
  publish_shared();

  // Double-buffered: the next group is in flight while this one is reduced.
  // Groups are issued unconditionally (tasks past ntask are zero-size loads),
  // so the waits before a group's use cover only that group.
  for (int t0 = gw; t0 < ntask; t0 += 2 * step) {
    issue_gu(t0 + step, gB, uB);
    pin_loads();
    compute_gu(t0, gA, uA);
    issue_gu(t0 + 2 * step, gA, uA);
    pin_loads();
    compute_gu(t0 + step, gB, uB);
  }
  // Down rows of this wave's first expert (u = wave) for the WG's first block
  // of output rows, issued only now: they stream while act is handed over
  // instead of competing with the gate/up rows on which act depends.
  u32x4 dn[kRB][IC];
#pragma unroll
  for (int r = 0; r < kRB; ++r)
    load_row<T, VEC, IC>(a.ed + (size_t(ulist[min(wave, U - 1)]) * H + min(h0 + r, H - 1)) * I, I,
                         wave < U && r < nrows, lane, dn[r]);
  issue_shared_down();
  pin_loads();
  __syncthreads();  // x_norm (region A) is dead from here on

  // ---- phase 3: gather act, down projection --------------------------------
  // shared act -> LDS [B][Isp]
  bool ok3 = true;
  if constexpr (VEC) {
    const rsrc_t sr = make_rsrc(sact_r, uint32_t(B) * uint32_t(Is) * 8u);
    const int hp = Isp / 2;  // word pairs per row
    ok3 = gather_tagged_pairs(
        sr, B * hp,
        [&](int f) -> uint32_t {
          const int b = f / hp, c2 = (f % hp) * 2;
          return c2 < Is ? uint32_t(b * Is + c2) * 8u : 0xFFFFFFF0u;
        },
        sact_l, tag, tid);
  } else {
    for (int t = tid; t < B * Isp; t += kThreads) {
      const int b = t / Isp, i = t % Isp;
      float val = 0.f;
      if (i < Is) {
        uint64_t word = 0;
        for (unsigned polls = 0; polls < kSpinLimit; ++polls) {
          word = __hip_atomic_load(sact_r + size_t(b) * Is + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          if (unsigned(word >> 32) == tag) break;
          __builtin_amdgcn_s_sleep(1);
        }
        ok3 = ok3 && unsigned(word >> 32) == tag;
        val = __uint_as_float(unsigned(word));
      }
      sact_l[t] = val;
    }
  }
  // Down projection by experts: wave w takes experts u_lo + w, u_lo + w + 8,
  // ... of each act window and, for each, the down rows of the WG's block of
  // kRB output rows -- kRB contiguous rows (kRB KB at I = 512), read as whole
  // cache lines.  Every lane keeps partials acc[r][b] for all rows and batch
  // rows over all windows; one butterfly reduction across the lanes at the end
  // leaves lane L with the total of accumulator bitrev(L), and the waves'
  // totals meet in LDS.  Usually nrows <= kRB (one block).
  for (int t = tid; t < a.rows_per_wg * MB; t += kThreads) part[t] = 0.f;
  const int win_entries = a.win_floats / Ip;
  for (int rb = 0; rb < nrows; rb += kRB) {
    const int nr = min(kRB, nrows - rb);
    float acc[kRB][MB];
#pragma unroll
    for (int r = 0; r < kRB; ++r)
#pragma unroll
      for (int b = 0; b < MB; ++b) acc[r][b] = 0.f;
    int u_lo = 0;
    while (u_lo < U) {
      int u_hi = u_lo + 1;
      while (u_hi < U && ent_base[u_hi + 1] - ent_base[u_lo] <= win_entries) ++u_hi;
      const int e_lo = ent_base[u_lo], ent = ent_base[u_hi] - e_lo;
      __syncthreads();  // previous window (and part[] zeroing) done
      if constexpr (VEC) {
        const rsrc_t ar = make_rsrc(act_r, uint32_t(B) * uint32_t(K) * uint32_t(I) * 8u);
        const int hp = Ip / 2;
        ok3 = gather_tagged_pairs(
                  ar, ent * hp,
                  [&](int f) -> uint32_t {
                    const int en = f / hp, c2 = (f % hp) * 2;
                    return c2 < I ? uint32_t(ent_src[e_lo + en] * I + c2) * 8u : 0xFFFFFFF0u;
                  },
                  act_l, tag, tid) &&
              ok3;
      } else {
        for (int t = tid; t < ent * Ip; t += kThreads) {
          const int en = t / Ip, i = t % Ip;
          float val = 0.f;
          if (i < I) {
            uint64_t word = 0;
            const uint64_t* pw = act_r + size_t(ent_src[e_lo + en]) * I + i;
            for (unsigned polls = 0; polls < kSpinLimit; ++polls) {
              word = __hip_atomic_load(const_cast<uint64_t*>(pw), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
              if (unsigned(word >> 32) == tag) break;
              __builtin_amdgcn_s_sleep(1);
            }
            ok3 = ok3 && unsigned(word >> 32) == tag;
            val = __uint_as_float(unsigned(word));
          }
          act_l[t] = val;
        }
      }
      if (!ok3) misc[16] = 1;
      __syncthreads();
      // Rows of expert u for the block (zero-size loads past the window or
      // past the block), issued unconditionally so that the waits before a
      // block's use cover only that block.
      auto issue_x = [&](int u, u32x4 (&c)[kRB][IC]) {
        const size_t base = (size_t(ulist[min(u, U - 1)]) * H + h0 + rb) * I;
#pragma unroll
        for (int r = 0; r < kRB; ++r)
          load_row<T, VEC, IC>(a.ed + base + size_t(min(r, nr - 1)) * I, I, u < u_hi && r < nr, lane, c[r]);
      };
      auto consume_x = [&](int u, const u32x4 (&c)[kRB][IC]) {
        if (u >= u_hi) return;
        const unsigned mask = umask[u];
#pragma unroll
        for (int b = 0; b < MB; ++b)
          if ((mask >> b) & 1u) {
            const float* av = act_l + size_t(ent_of[u * MB + b] - e_lo) * Ip;
#pragma unroll
            for (int r = 0; r < kRB; ++r) acc[r][b] += dot_row<T, IC>(c[r], av, I, lane);
          }
      };
      // The wave's j-th expert of the window (u_hi: none).  Waves 4-7 share
      // their SIMDs with waves 0-3 and stream ~20 % slower.  With at least 5
      // full rounds of experts and more than 4 in the last, partial round, that
      // round's experts past the 4th go to waves 0, 1, ... as one more each,
      // so that no slower wave streams an extra expert.
      const int nw8 = (u_hi - u_lo) / kWaves, nlast = (u_hi - u_lo) % kWaves;
      const int nmv = nw8 >= 5 && nlast > kWaves / 2 ? nlast - kWaves / 2 : 0;
      const int u_main = u_hi - nmv;
      const int j_extra = (u_main - u_lo - wave + kWaves - 1) / kWaves;  // strided experts of this wave
      auto seq = [&](int j) -> int {
        const int u = u_lo + wave + kWaves * j;
        return u < u_main ? u : (wave < nmv && j == j_extra) ? u_main + wave : u_hi;
      };
      u32x4 ca[kRB][IC], cb[kRB][IC];
      if (rb == 0 && u_lo == 0 && wave < u_hi) {  // prefetched in phase 2
#pragma unroll
        for (int r = 0; r < kRB; ++r)
#pragma unroll
          for (int q = 0; q < IC; ++q) ca[r][q] = dn[r][q];
      } else {
        issue_x(seq(0), ca);
      }
      pin_loads();
      for (int j = 0; seq(j) < u_hi; j += 2) {
        issue_x(seq(j + 1), cb);
        pin_loads();
        consume_x(seq(j), ca);
        issue_x(seq(j + 2), ca);
        pin_loads();
        consume_x(seq(j + 1), cb);
      }
      u_lo = u_hi;
    }
    // Butterfly: at step k the lane keeps the half of its accumulators picked
    // by lane bit k and adds the partner's (lane ^ 2^k) copy of that half.
    constexpr int NA = kRB * MB;  // == kWave
    static_assert(NA == kWave, "one accumulator per lane after the butterfly");
    float v[NA];
#pragma unroll
    for (int r = 0; r < kRB; ++r)
#pragma unroll
      for (int b = 0; b < MB; ++b) v[r * MB + b] = acc[r][b];
#pragma unroll
    for (int k = 0; (1 << k) < NA; ++k) {
      const int half = NA >> (k + 1);
      const bool hi = (lane >> k) & 1;
#pragma unroll
      for (int i = 0; i < half; ++i) {
        const float keep = hi ? v[i + half] : v[i];
        const float send = hi ? v[i] : v[i + half];
        v[i] = keep + __shfl_xor(send, 1 << k, kWave);
      }
    }
    int idx = 0;  // bit-reversed lane: the accumulator this lane now holds
#pragma unroll
    for (int k = 0; (1 << k) < NA; ++k) idx |= ((lane >> k) & 1) << (5 - k);
    __syncthreads();  // act window dead: its first kWaves * NA floats take the wave totals
    act_l[wave * NA + idx] = v[0];
    __syncthreads();
    if (tid < NA) {
      const int r = tid / MB, b = tid % MB;
      float t = 0.f;
#pragma unroll
      for (int ww = 0; ww < kWaves; ++ww) t += act_l[ww * NA + tid];
      if (r < nr) part[(rb + r) * MB + b] = t;
    }
  }
  __syncthreads();
  timed_out = misc[16] != 0;
  if (timed_out && tid == 0) __hip_atomic_store(w.err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  // shared expert (gated) + residual; the owning wave writes its rows
  for (int hl = wave; hl < nrows; hl += kWaves) {
    u32x4 c[IC];
    if (hl == wave) {
#pragma unroll
      for (int q = 0; q < IC; ++q) c[q] = sdn[q];
    } else {
      load_row<T, VEC, IC>(a.sd + size_t(h0 + hl) * Is, Is, true, lane, c);
    }
    if (B > kMaxB / 2) {
      // The MB shared-expert dots of this row are summed over the wave
      // together (from B = 5 on; below, one reduction per row costs less):
      // a butterfly halves the values a lane holds at each of log2(MB)
      // steps (lane bit k picks the half kept), then the lanes that hold
      // the same value add across the remaining lane bits.  Lane L ends with
      // the total of batch row bitrev(L mod MB).  Rows b >= B read row
      // B - 1's shared act and are not written.
      constexpr int LGB = MB == 2 ? 1 : MB == 4 ? 2 : 3;
      static_assert(MB == 2 || MB == 4 || MB == 8, "power-of-two batch rows");
      float dv[MB];
#pragma unroll
      for (int b = 0; b < MB; ++b) dv[b] = dot_row<T, IC>(c, sact_l + min(b, B - 1) * Isp, Is, lane);
#pragma unroll
      for (int k = 0; k < LGB; ++k) {
        const int half = MB >> (k + 1);
        const bool hi = (lane >> k) & 1;
#pragma unroll
        for (int i = 0; i < half; ++i) {
          const float keep = hi ? dv[i + half] : dv[i];
          const float send = hi ? dv[i] : dv[i + half];
          dv[i] = keep + __shfl_xor(send, 1 << k, kWave);
        }
      }
      float tot = dv[0];
#pragma unroll
      for (int m = MB; m < kWave; m <<= 1) tot += __shfl_xor(tot, m, kWave);
      int bb = 0;  // the batch row this lane's total belongs to
#pragma unroll
      for (int k = 0; k < LGB; ++k) bb |= ((lane >> k) & 1) << (LGB - 1 - k);
      const float xr = __shfl(x_res, bb, kWave);  // lane b of x_res holds batch row b's residual
      if (lane < MB && bb < B) {
        const size_t o = size_t(bb) * H + h0 + hl;
        float s = fmaf(sgf[bb], tot, part[hl * MB + bb]);
        if (a.add_residual) s += hl == wave ? xr : to_f(a.x[o]);
        a.out[o] = from_f<T>(timed_out ? NAN : s);
      }
    } else {
#pragma unroll
      for (int b = 0; b < MB; ++b)
        if (b < B) {
          float s = fmaf(sgf[b], wave_sum_u(dot_row<T, IC>(c, sact_l + b * Isp, Is, lane)), part[hl * MB + b]);
          const size_t o = size_t(b) * H + h0 + hl;
          const float xr = __shfl(x_res, b, kWave);  // prefetched for the wave's first row
          if (lane == 0) {
            if (a.add_residual) s += hl == wave ? xr : to_f(a.x[o]);
            a.out[o] = from_f<T>(timed_out ? NAN : s);
          }
        }
    }
  }
  }  // multi-row path
  if constexpr (MB > 1) {
    if (wg == 0 && wave == 0) advance_gen();
  }
  MOE_MARK(7);
}

// LDS floats besides region A (x_norm, later the act window and shared act),
// for kMaxB rows.
size_t lds_fixed_floats(int E, int K, int rows_per_wg) {
  const int ulimit = E < kMaxB * K ? E : kMaxB * K;
  size_t n = kWaves * 2 * kMaxB + kMaxB + kMaxB * K;                                            // floats
  n += kMaxB * K + E + ulimit + ulimit + size_t(ulimit) * kMaxB + kMaxB * K + size_t(ulimit) * kMaxB + 32;  // ints
  n += size_t(rows_per_wg) * kMaxB;  // part
  n += size_t(ulimit) + 1;           // ent_base
  return n;
}

template <typename T>
int launch(const MoeArgs<T>& args0, int batch, hipStream_t stream) {
  constexpr int EPC = Epc<T>::value;
  MoeArgs<T> a = args0;
#ifdef MKQ_MOE_TRACE
  a.trace = g_trace;
#endif
  const int ncu = cu_count();
  const int nwg = ncu < kMaxWg ? ncu : kMaxWg;
  a.nwg = nwg;
  a.rows_per_wg = (a.H + nwg - 1) / nwg;
  const bool vec = (a.H % EPC == 0) && (a.I % EPC == 0) && (a.Is % EPC == 0) && aligned16(a.x) &&
                   aligned16(a.nw) && aligned16(a.router) && aligned16(a.eg) && aligned16(a.eu) && aligned16(a.ed) &&
                   aligned16(a.sg) && aligned16(a.su) && aligned16(a.sd) && (a.wsg == nullptr || aligned16(a.wsg));
  // Region A holds x_norm [kMaxB][Hp], later the act window and the shared act
  // [kMaxB][Isp].  The window takes what the LDS leaves, up to every act row
  // of the launch (B * K rows of Ip), and at least kMaxB rows (one expert's
  // rows of every batch row).
  const size_t Hp = round_up(a.H, EPC), Ip = round_up(a.I, EPC), Isp = round_up(a.Is, EPC);
  const size_t fixed = lds_fixed_floats(a.E, a.K, a.rows_per_wg);
  const size_t limit = size_t(max_lds_per_block()) / 4;
  const size_t avail = limit > fixed ? limit - fixed : 0;
  const size_t want = size_t(kMaxB) * a.K * Ip;
  const size_t room = avail > size_t(kMaxB) * Isp ? avail - size_t(kMaxB) * Isp : 0;
  // The window area also takes the multi-row down phase's per-wave totals
  // (kWaves * kWave floats) once the last window is consumed.
  const size_t totals = (size_t(kWaves) * kWave + Ip - 1) / Ip * Ip;
  const size_t win = max(totals, (room < want ? room : want) / Ip * Ip);
  const size_t region_floats = max(size_t(kMaxB) * Hp, win + size_t(kMaxB) * Isp);
  const size_t lds = 4 * (fixed + region_floats);
  if (avail < size_t(kMaxB) * Hp || win < size_t(kMaxB) * Ip || fixed + region_floats > limit)
    return set_error(MKQ_ERR_UNSUPPORTED, "moe_decode: shape does not fit the %zu bytes of LDS", limit * 4);
  a.win_floats = int(win);
  // Chunk counts per lane: the smallest instantiation that covers the rows.
  const int hc_need = (a.H + EPC * kWave - 1) / (EPC * kWave);
  const int ic_need = (max(a.I, a.Is) + EPC * kWave - 1) / (EPC * kWave);
  // The one-row path keeps x_norm, act [K][Ip] and the shared act side by side
  // in the LDS region that the multi-row path shares between them.
  const size_t one_row_floats = Hp + size_t(a.K) * Ip + Isp;
  // Its routing keeps the E logit keys in the act area until the act gather.
  const bool one_row_ok = batch == 1 && one_row_floats <= max(Hp, win + Isp) &&  // region A as sized for B = 1
                          a.E <= nwg * kWaves && a.Is <= nwg * kWaves &&         // one router / shared row per wave
                          size_t(a.E) <= size_t(a.K) * Ip + Isp;
  const int which = (vec && hc_need <= 4 && ic_need <= 1) ? (one_row_ok ? 0 : 1) : (vec ? 2 : 3);
  const bool el4 = a.E <= 4 * kWave;
  void (*kern)(MoeArgs<T>) = which == 0   ? (el4 ? &moe_decode_kernel<T, true, 4, 1, 1, 4>
                                                 : &moe_decode_kernel<T, true, 4, 1, 1, kMaxEL>)
                             : which == 1 ? (el4 ? &moe_decode_kernel<T, true, 4, 1, kMaxB, 4>
                                                 : &moe_decode_kernel<T, true, 4, 1, kMaxB, kMaxEL>)
                             : which == 2 ? &moe_decode_kernel<T, true, kMaxHC, kMaxIC, kMaxB, kMaxEL>
                                          : &moe_decode_kernel<T, false, kMaxHC, kMaxIC, kMaxB, kMaxEL>;
  static bool attr_set[8] = {false, false, false, false, false, false, false, false};
  const int slot = which * 2 + (el4 ? 1 : 0);
  if (!attr_set[slot]) {
    MKQ_HIP_TRY(hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize,
                                    max_lds_per_block()));
    attr_set[slot] = true;
  }
  // The workgroups wait for each other, so all nwg (one per CU) must be
  // resident at once.  Checked once per (device, instance, LDS size).
  static size_t resident_ok[kMaxDevCache][8] = {};
  const int dev = current_device();
  if (dev < 0 || dev >= kMaxDevCache || resident_ok[dev][slot] != lds) {
    int per_cu = 0;
    MKQ_HIP_TRY(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, reinterpret_cast<const void*>(kern), kThreads,
                                                             lds));
    if (per_cu < 1 || int64_t(per_cu) * ncu < nwg)
      return set_error(MKQ_ERR_UNSUPPORTED,
                       "moe_decode: %d workgroups of %d threads and %zu bytes of LDS cannot all be resident "
                       "(%d per CU, %d CUs)",
                       nwg, kThreads, lds, per_cu, ncu);
    if (dev >= 0 && dev < kMaxDevCache) resident_ok[dev][slot] = lds;
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

#ifdef MKQ_MOE_TRACE
// Profiling builds only: where the kernel stores its phase timestamps.
extern "C" int mkq_moe_set_trace(void* buf) {
  g_trace = static_cast<uint64_t*>(buf);
  return MKQ_OK;
}
#endif

extern "C" size_t mkq_moe_decode_workspace_bytes(int batch, int hidden, int experts, int intermediate,
                                                 int shared_intermediate, int top_k) {
  (void)batch;
  (void)hidden;
  if (experts <= 0 || intermediate <= 0 || shared_intermediate <= 0 || top_k <= 0) return 0;
  return ws_bytes(experts, intermediate, shared_intermediate, top_k);
}

namespace {

// Argument checks and dtype dispatch shared by mkq_moe_decode and
// mkq_moe_decode_noalloc; `fn` names the entry point in error messages.
int moe_entry(const char* fn, int dtype, const void* x, const void* norm_weight, const void* router_weight,
              const void* expert_gate, const void* expert_up, const void* expert_down, const void* shared_gate,
              const void* shared_up, const void* shared_down, const void* shared_expert_gate, void* out,
              int64_t* indices, float* weights, int batch, int hidden, int experts, int intermediate,
              int shared_intermediate, int top_k, float eps, int add_residual, void* workspace,
              size_t workspace_bytes, void* stream) {
  MKQ_REQUIRE(workspace && workspace_bytes >= mkq_moe_decode_workspace_bytes(batch, hidden, experts, intermediate,
                                                                              shared_intermediate, top_k),
              "%s: workspace too small", fn);
  MKQ_REQUIRE((reinterpret_cast<uintptr_t>(workspace) & 255u) == 0, "%s: workspace must be 256-byte aligned", fn);
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (dtype) {
#define MKQ_MOE_CASE(CODE, TYPE)                                 \
  case CODE: {                                                   \
    MoeArgs<TYPE> a{};                                           \
    a.x = static_cast<const TYPE*>(x);                           \
    a.nw = static_cast<const TYPE*>(norm_weight);                \
    a.router = static_cast<const TYPE*>(router_weight);          \
    a.eg = static_cast<const TYPE*>(expert_gate);                \
    a.eu = static_cast<const TYPE*>(expert_up);                  \
    a.ed = static_cast<const TYPE*>(expert_down);                \
    a.sg = static_cast<const TYPE*>(shared_gate);                \
    a.su = static_cast<const TYPE*>(shared_up);                  \
    a.sd = static_cast<const TYPE*>(shared_down);                \
    a.wsg = static_cast<const TYPE*>(shared_expert_gate);        \
    a.out = static_cast<TYPE*>(out);                             \
    a.idx = indices;                                             \
    a.wts = weights;                                             \
    a.ws = static_cast<unsigned char*>(workspace);               \
    a.H = hidden;                                                \
    a.E = experts;                                               \
    a.I = intermediate;                                          \
    a.Is = shared_intermediate;                                  \
    a.K = top_k;                                                 \
    a.eps = eps;                                                 \
    a.add_residual = add_residual;                               \
    return launch<TYPE>(a, batch, s);                            \
  }
    MKQ_MOE_CASE(MKQ_DTYPE_BF16, bf16_t)
    MKQ_MOE_CASE(MKQ_DTYPE_F16, f16_t)
    MKQ_MOE_CASE(MKQ_DTYPE_F32, float)
#undef MKQ_MOE_CASE
    default:
      return set_error(MKQ_ERR_INVALID, "%s: unknown dtype %d", fn, dtype);
  }
}

// Checks that need no workspace: sizes, pointers, supported shapes.
int moe_check_args(const char* fn, int dtype, const void* x, const void* norm_weight, const void* router_weight,
                   const void* expert_gate, const void* expert_up, const void* expert_down, const void* shared_gate,
                   const void* shared_up, const void* shared_down, const void* out, const void* indices,
                   const void* weights, int batch, int hidden, int experts, int intermediate, int shared_intermediate,
                   int top_k) {
  MKQ_REQUIRE(batch > 0 && hidden > 0 && experts > 0 && intermediate > 0 && shared_intermediate > 0,
              "%s: sizes must be positive", fn);
  MKQ_REQUIRE(top_k > 0 && top_k <= experts, "top_k must be in [1, experts]");
  MKQ_REQUIRE(x && norm_weight && router_weight && expert_gate && expert_up && expert_down && shared_gate &&
                  shared_up && shared_down && out && indices && weights,
              "%s: null tensor pointer", fn);
  if (experts > kMaxEL * kWave || top_k > 64)
    return set_error(MKQ_ERR_UNSUPPORTED, "%s: experts <= %d and top_k <= 64 are supported", fn, kMaxEL * kWave);
  const int epc = dtype == MKQ_DTYPE_F32 ? 4 : 8;
  const int maxh = epc * kWave * kMaxHC, maxi = epc * kWave * kMaxIC;
  if (hidden > maxh || intermediate > maxi || shared_intermediate > maxi)
    return set_error(MKQ_ERR_UNSUPPORTED, "%s: hidden <= %d and intermediate <= %d are supported", fn, maxh, maxi);
  return MKQ_OK;
}

// Scratch of mkq_moe_decode_noalloc: the MoE workspace (generation and error
// words, tagged logits, act and shared act) as a static device array, one per
// GPU, held until the process ends.  Device globals start zeroed when the
// code object is loaded, which is the state a fresh workspace must have; the
// generation protocol then keeps it valid from call to call, so nothing is
// cleared per call.  Its address is taken once per device with
// hipGetSymbolAddress (host code never passes `scratch` itself).
constexpr size_t kNoAllocScratchBytes = MKQ_MOE_NOALLOC_SCRATCH_BYTES;
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevCache] = {};

// Device address of this device's `scratch`, looked up on first use.
int scratch_ptr(const char* fn, void** out) {
  const int dev = current_device();
  if (dev < 0 || dev >= kMaxDevCache)
    return set_error(MKQ_ERR_UNSUPPORTED, "%s: device %d is beyond the %d devices supported", fn, dev, kMaxDevCache);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr)
      return set_error(MKQ_ERR_HIP, "%s: hipGetSymbolAddress(scratch) failed: %s", fn, hipGetErrorString(e));
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return MKQ_OK;
}

}  // namespace

extern "C" int mkq_moe_decode(int dtype, const void* x, const void* norm_weight, const void* router_weight,
                              const void* expert_gate, const void* expert_up, const void* expert_down,
                              const void* shared_gate, const void* shared_up, const void* shared_down,
                              const void* shared_expert_gate, void* out, int64_t* indices, float* weights, int batch,
                              int hidden, int experts, int intermediate, int shared_intermediate, int top_k,
                              float eps, int add_residual, void* workspace, size_t workspace_bytes, void* stream) {
  clear_error();
  const char* fn = "moe_decode";
  const int rc = moe_check_args(fn, dtype, x, norm_weight, router_weight, expert_gate, expert_up, expert_down,
                                shared_gate, shared_up, shared_down, out, indices, weights, batch, hidden, experts,
                                intermediate, shared_intermediate, top_k);
  if (rc != MKQ_OK) return rc;
  return moe_entry(fn, dtype, x, norm_weight, router_weight, expert_gate, expert_up, expert_down, shared_gate,
                   shared_up, shared_down, shared_expert_gate, out, indices, weights, batch, hidden, experts,
                   intermediate, shared_intermediate, top_k, eps, add_residual, workspace, workspace_bytes, stream);
}

extern "C" int mkq_moe_decode_noalloc(int dtype, const void* x, const void* norm_weight, const void* router_weight,
                                      const void* expert_gate, const void* expert_up, const void* expert_down,
                                      const void* shared_gate, const void* shared_up, const void* shared_down,
                                      const void* shared_expert_gate, void* out, int64_t* indices, float* weights,
                                      int batch, int hidden, int experts, int intermediate, int shared_intermediate,
                                      int top_k, float eps, int add_residual, void* stream) {
  clear_error();
  const char* fn = "moe_decode_noalloc";
  int rc = moe_check_args(fn, dtype, x, norm_weight, router_weight, expert_gate, expert_up, expert_down, shared_gate,
                          shared_up, shared_down, out, indices, weights, batch, hidden, experts, intermediate,
                          shared_intermediate, top_k);
  if (rc != MKQ_OK) return rc;
  const size_t need = ws_bytes(experts, intermediate, shared_intermediate, top_k);
  if (need > kNoAllocScratchBytes)
    return set_error(MKQ_ERR_UNSUPPORTED,
                     "%s: this shape needs %zu bytes of scratch; the static scratch array holds %zu "
                     "(use mkq_moe_decode with a caller workspace)",
                     fn, need, kNoAllocScratchBytes);
  void* ws = nullptr;
  rc = scratch_ptr(fn, &ws);
  if (rc != MKQ_OK) return rc;
  return moe_entry(fn, dtype, x, norm_weight, router_weight, expert_gate, expert_up, expert_down, shared_gate,
                   shared_up, shared_down, shared_expert_gate, out, indices, weights, batch, hidden, experts,
                   intermediate, shared_intermediate, top_k, eps, add_residual, ws, kNoAllocScratchBytes, stream);
}

extern "C" int mkq_moe_decode_status(void* workspace, size_t workspace_bytes, int reset, int* error_code,
                                     void* stream) {
  clear_error();
  MKQ_REQUIRE(workspace && error_code, "moe_decode_status: null pointer");
  MKQ_REQUIRE(workspace_bytes >= kOffData, "moe_decode_status: workspace too small");
  hipStream_t s = static_cast<hipStream_t>(stream);
  unsigned word = 0;
  MKQ_HIP_TRY(hipMemcpyAsync(&word, static_cast<unsigned char*>(workspace) + kOffErr, sizeof(word),
                             hipMemcpyDeviceToHost, s));
  MKQ_HIP_TRY(hipStreamSynchronize(s));
  *error_code = int(word);
  if (reset && word != 0) {
    MKQ_HIP_TRY(hipMemsetAsync(workspace, 0, workspace_bytes, s));
    MKQ_HIP_TRY(hipStreamSynchronize(s));
  }
  return MKQ_OK;
}
