// GQA full-attention decode (one query token) for gfx950: split-K flash-decode
// on MFMA.
//
// out[b, qh] = softmax(q[b,qh] . K[b,:,kvh]^T * scale) V[b,:,kvh],  kvh = qh / G
// (reference.py:117-145; replaces attention_decode.cu:33-218).
//
// Work split.  A "unit" is (batch row, kv head, group of <= 16 q heads that
// share the kv head).  The token axis of each unit is cut into chunks; a
// workgroup owns one (chunk, unit) and its 4 waves take the chunk's 16-token
// tiles in turn, so at any moment the workgroup streams 64 adjacent tokens.
// Workgroups of the same chunk for consecutive units are adjacent in launch
// order, so the kv heads stored side by side in one token row are read
// together.  Per tile a wave
//   * loads the K tile as two 512-byte token rows per instruction (full cache
//     lines; the A-operand layout would take 16 tokens x 64 bytes), stages it
//     in wave-private LDS and reads it back as MFMA A operands (16 tokens x 32
//     dims per v_mfma_f32_16x16x32), computing S^T = K Q^T for all q heads of
//     the group at once -- the G q heads of a kv head reuse one read of K and V;
//   * runs an online softmax in the base-2 domain; the probabilities stay in
//     the registers of the S^T result, whose layout (lane (head c, group g)
//     holds tokens 4g..4g+3) is exactly the B operand of v_mfma_f32_16x16x16;
//   * stages the V tile in wave-private LDS (row stride padded so the
//     transposed 16-bit reads are bank-conflict free) and accumulates
//     O^T = V^T P^T with one 16x16x16 MFMA per 16 output dims.
// K and V loads go through buffer descriptors that cover exactly the chunk,
// so the tail of a chunk reads zeros with no branch, and the next tile's K and
// V are issued while the current tile is computed.  The 4 waves merge in LDS;
// each workgroup writes one partial (m, l, O) per q head and a merge kernel
// combines the chunks with the log-sum-exp rule (a single chunk writes the
// output directly).
//
// HBM-bound: every K/V byte is read once (4*T*Hkv*D bytes per batch row).
#include <math.h>

#include "mkq_host.h"

using namespace mkq;

namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / kWave;
constexpr int kTT = 16;                  // tokens per wave tile
constexpr int kWgTokens = kWaves * kTT;  // tokens per workgroup pass
constexpr int kMaxD = 256;
constexpr int kMaxChunks = 1024;
constexpr int kMergeBatch = 16;          // chunk loads in flight per merge lane
constexpr uint32_t kFar = 0x80000000u;   // pushes an offset past any descriptor (all < 2^31 bytes)
constexpr float kNegInf = -INFINITY;

template <typename T>
struct Mfma;
template <>
struct Mfma<bf16_t> {
  typedef bf16x8 vec8;
  typedef short vec4 __attribute__((ext_vector_type(4)));
  static __device__ __forceinline__ f32x4 qk(vec8 a, vec8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ f32x4 pv(vec4 a, vec4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ short cvt(float f) { return short(f2bf_bits(f)); }
};
template <>
struct Mfma<f16_t> {
  typedef f16x8 vec8;
  typedef _Float16 vec4 __attribute__((ext_vector_type(4)));
  static __device__ __forceinline__ f32x4 qk(vec8 a, vec8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ f32x4 pv(vec4 a, vec4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x16f16(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ _Float16 cvt(float f) { return _Float16(f); }
};

// 8 floats -> one 16-byte chunk of T (round to nearest even).
__device__ __forceinline__ u32x4 pack8(const float (&f)[8], bf16_t) {
  u32x4 r;
  r.x = f2bf2_bits(f[0], f[1]);
  r.y = f2bf2_bits(f[2], f[3]);
  r.z = f2bf2_bits(f[4], f[5]);
  r.w = f2bf2_bits(f[6], f[7]);
  return r;
}
__device__ __forceinline__ u32x4 pack8(const float (&f)[8], f16_t) {
  uint32_t w[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f16x2 h;
    h[0] = _Float16(f[2 * i]);
    h[1] = _Float16(f[2 * i + 1]);
    w[i] = __builtin_bit_cast(uint32_t, h);
  }
  return u32x4{w[0], w[1], w[2], w[3]};
}

// Rotate-half RoPE of one 16-byte chunk: x' = x cos + p sin', p = the partner
// chunk, cos / sin' = 8 values each (c0 c1 / s0 s1; sin' already negated for
// the lower half).  Two rounded products, a rounded sum, then the rounding to T,
// as reference.py:91-114's torch ops do: no contraction into an FMA and no
// fused f32->f16 mixed FMA (the register barriers keep each value FP32).
template <typename T>
__device__ __forceinline__ u32x4 rope8(u32x4 xq, u32x4 pq, f32x4 c0, f32x4 c1, f32x4 s0, f32x4 s1) {
  float xf[8], pf[8], of[8];
  unpack(xq, xf, T{});
  unpack(pq, pf, T{});
  const float cv[8] = {c0[0], c0[1], c0[2], c0[3], c1[0], c1[1], c1[2], c1[3]};
  const float sv[8] = {s0[0], s0[1], s0[2], s0[3], s1[0], s1[1], s1[2], s1[3]};
#pragma unroll
  for (int e = 0; e < 8; ++e) {
#pragma clang fp contract(off)
    float a = xf[e] * cv[e];
    float b = pf[e] * sv[e];
    asm volatile("" : "+v"(a), "+v"(b));
    float sum = a + b;
    asm volatile("" : "+v"(sum));
    of[e] = sum;
  }
  return pack8(of, T{});
}

// LDS row stride (16-bit elements) of a staged V tile: D/2 dwords padded to
// 2 mod 8 dwords, so the four token rows 4g+j (g = 0..3) that one transposed
// read touches start 8 banks apart and cover 32 distinct banks.
constexpr __host__ __device__ int v_stride(int d) { return 2 * (d / 2 + ((2 - d / 2) % 8 + 8) % 8); }
// LDS row stride (bytes) of a staged K tile: D * 2 + 16, so the 16-byte A
// operand reads of 8 consecutive tokens start 4 banks apart (conflict free).
constexpr __host__ __device__ int k_stride_bytes(int d) { return 2 * d + 16; }
// Staging bytes per wave: the K tile and then the V tile use the same area.
constexpr __host__ __device__ int stage_bytes(int d) {
  return kTT * (k_stride_bytes(d) > 2 * v_stride(d) ? k_stride_bytes(d) : 2 * v_stride(d));
}

// Row stride (floats) of a wave's O block in the merge area.
__host__ __device__ inline int o_stride(int d) { return d + 4; }

__host__ __device__ inline size_t merge_floats(int d, int heads) { return size_t(32) + size_t(heads) * o_stride(d); }

template <int DT>
size_t chunk_lds_bytes(int d, int heads) {
  const size_t stage = size_t(kWaves) * stage_bytes(DT);
  const size_t merge = (size_t(kWaves) * merge_floats(d, heads) + 16 * 8) * 4;  // + per-head weights
  return stage > merge ? stage : merge;
}

// grid: (nchunks * units); block 256.  blockIdx.x = chunk * units + unit.
//
// ROPE: the keys are rotated on the fly with the rotate-half rule of
// reference.py:91-114 and one (cos, sin) vector for every token -- the
// reference rotates the whole k_cache with the same broadcast vectors before
// its kernel.  Once a K tile is staged in LDS, its rotary 16-byte chunks are
// spread over the wave's lanes; each reads its chunk and the partner chunk
// (dims +-rot/2) and writes the rotated chunk back.  q is rotated the same
// way once, in registers.  Products and
// the sum are rounded separately and the result is rounded to T, as the
// reference's torch ops do, so the rotated q and keys are bit-identical to
// the reference's.
//
// APP (KV append): token seq - 1 is the new one.  Its key and value come from
// k_new/v_new [B, Hkv, D] rather than the cache: the workgroups of the last
// chunk load them with q, write them over the stale row of the staged tile
// (before any rotation), and the first head group's wave 0 stores them into
// the cache row (kw/vw, the cache pointers) at the end.  No workgroup of the
// launch reads that cache row and uses it.  `cap` is the cache's token
// capacity (batch stride in tokens); seq <= cap.
//
// PG (paged KV): kc/vc are pools of blocks [nblocks, bsz, hkv, d] and token t
// of batch row b lives in block btab[b * maxb + t / bsz]; bsz % 16 == 0, so a
// 16-token tile never straddles two blocks.  The chunk's block ids are staged
// in LDS once; every tile gets a descriptor over its own rows, and an id
// outside [0, nblocks) reads as zeros.
template <typename T, int DT, bool ROPE, bool APP, bool PG>
__global__ __launch_bounds__(kThreads, 2) void attn_chunk_kernel(
    const T* __restrict__ q, const T* __restrict__ kc, const T* __restrict__ vc, float* __restrict__ part_o,
    float* __restrict__ part_m, float* __restrict__ part_l, T* __restrict__ out, const float* __restrict__ rope_cs,
    const T* __restrict__ k_new, const T* __restrict__ v_new, T* kw, T* vw, int cap, const int* __restrict__ btab,
    int bsz, int maxb, int nblocks, int blk_lds_off, int rot, int rope_lds_off,
    int hq, int hkv, int d, int seq, int group, int ngroups, int units, int nch, int chunk_tokens,
    float scale_log2) {
  typedef typename Mfma<T>::vec8 V8;
  typedef typename Mfma<T>::vec4 V4;
  constexpr int NS = DT / 32;               // QK^T MFMA steps over head_dim
  constexpr int NDT = DT / 16;              // PV MFMA tiles over head_dim
  constexpr int CPR = DT / 8;               // 16-byte chunks per staged token row
  constexpr int VCH = kTT * CPR / kWave;    // V chunks per lane per tile
  constexpr int VSTR = v_stride(DT);
  static_assert(VCH >= 1 && kTT * CPR == VCH * kWave, "V tile must split evenly over the wave");

  const int lane = threadIdx.x % kWave, wave = wave_id();
  const int col = lane & 15, grp = lane >> 4;
  const int unit = blockIdx.x % units, c = blockIdx.x / units;
  const int b = unit / (hkv * ngroups);
  const int kvh = (unit / ngroups) % hkv, hg = unit % ngroups;
  const int heads_here = min(16, group - hg * 16);
  const int qh0 = kvh * group + hg * 16;
  const int t_begin = c * chunk_tokens;
  const int len = min(seq - t_begin, chunk_tokens);
  const uint32_t tsb = uint32_t(hkv) * d * sizeof(T);  // bytes between tokens

  // Descriptors over this unit's K/V rows of the chunk; anything past the
  // last row (tail tokens, the prefetch after the last tile) reads zero.
  const size_t base = (size_t(b) * cap + t_begin) * hkv * d + size_t(kvh) * d;
  const uint32_t bytes = (uint32_t(len) - 1) * tsb + uint32_t(d) * sizeof(T);
  const rsrc_t kr = make_rsrc(kc + base, bytes);
  const rsrc_t vr = make_rsrc(vc + base, bytes);

  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  int* blk_l = reinterpret_cast<int*>(smem + blk_lds_off);
  const int bi0 = PG ? t_begin / bsz : 0;
  if constexpr (PG) {
    const int nbl = (t_begin + len - 1) / bsz - bi0 + 1;
    for (int i = threadIdx.x; i < nbl; i += kThreads) {
      const int bi = bi0 + i;
      blk_l[i] = bi < maxb ? btab[size_t(b) * maxb + bi] : -1;
    }
    __syncthreads();
  }
  // The descriptor and base offset for the 16-token tile at chunk row t
  // (wave-uniform): the chunk-wide descriptor, or with PG one over the tile's
  // rows in its block.  Rows past the chunk read as zeros either way.
  auto tile_src = [&](const T* cache, const rsrc_t& whole, int t, uint32_t& ob)
                      __attribute__((always_inline)) -> rsrc_t {
    if constexpr (!PG) {
      ob = uint32_t(t) * tsb;
      return whole;
    } else {
      ob = 0;
      const int rows = min(len - t, kTT);
      if (rows <= 0) return make_rsrc(cache, 0u);
      const int tg = t_begin + t;
      const int blk = __builtin_amdgcn_readfirstlane(blk_l[tg / bsz - bi0]);
      if (blk < 0 || blk >= nblocks) return make_rsrc(cache, 0u);
      const T* p = cache + (size_t(blk) * bsz + tg % bsz) * hkv * d + size_t(kvh) * d;
      return make_rsrc(p, uint32_t(rows - 1) * tsb + uint32_t(d) * sizeof(T));
    }
  };

  // Q^T as the B operand: lane (head col, k-group grp) holds dims 32s+8grp..+8;
  // heads past the group read zero.
  const rsrc_t qr = make_rsrc(q + (size_t(b) * hq + qh0) * d, uint32_t(heads_here * d * sizeof(T)));
  V8 qop[NS];
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    const int d0 = 32 * s + 8 * grp;
    qop[s] = __builtin_bit_cast(V8, buf_load16(qr, d0 < d ? uint32_t(col * d + d0) * uint32_t(sizeof(T)) : kFar));
  }
  // ROPE: q's partner chunks (dims +-rot/2) and this thread's cos/sin values
  // are loaded here, before the K/V stream, and used after it is issued.
  u32x4 qpart[NS];
  float cs_ld[2] = {0.f, 0.f};
  if constexpr (ROPE) {
    const int half = rot / 2;
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      const int d0 = 32 * s + 8 * grp;
      const int pd = d0 < half ? d0 + half : d0 - half;
      qpart[s] = buf_load16(qr, d0 < rot ? uint32_t(col * d + pd) * uint32_t(sizeof(T)) : kFar);
    }
    const rsrc_t cr = make_rsrc(rope_cs, uint32_t(2 * rot) * 4u);
    cs_ld[0] = buf_loadf(cr, uint32_t(threadIdx.x) * 4u);
    cs_ld[1] = buf_loadf(cr, uint32_t(threadIdx.x + kThreads) * 4u);
  }
  // APP: lane l < D/8 of every wave of the last chunk holds dims 8l..8l+7 of
  // the new key and value (other workgroups read nothing: an empty range).
  const int arow = seq - 1 - t_begin;  // the new token's row in this chunk
  const bool owner = APP && arow < len;
  u32x4 kap = u32x4{0u, 0u, 0u, 0u}, vap = u32x4{0u, 0u, 0u, 0u};
  if constexpr (APP) {
    const uint32_t nb = owner ? uint32_t(d * sizeof(T)) : 0u;
    const uint32_t off = lane * 8 < d ? uint32_t(lane * 16) : kFar;
    kap = buf_load16(make_rsrc(k_new + (size_t(b) * hkv + kvh) * d, nb), off);
    vap = buf_load16(make_rsrc(v_new + (size_t(b) * hkv + kvh) * d, nb), off);
  }
  // K and V chunk i of a tile: token row qi / CPR, dims 8 * (qi % CPR),
  // qi = lane + 64 i (two 512-byte token rows per load at D = 256).
  uint32_t voff[VCH];
#pragma unroll
  for (int i = 0; i < VCH; ++i) {
    const int qi = lane + kWave * i;
    const int row = qi / CPR, dc = qi % CPR;
    voff[i] = uint32_t(row) * tsb + (dc * 8 < d ? uint32_t(dc * 16) : kFar);
  }
  // ROPE: cos and the signed sin (rotate_half negates the upper half) of the
  // rotary dims, in LDS after the staging/merge area.
  const int rhc = ROPE ? rot / 16 : 0;  // partner chunk distance
  // ROPE: rot/8 rotary chunks per row (a power of two, 2^rlg); this lane's
  // chunk of the row in the key rotation.
  const int rlg = ROPE ? __builtin_ctz(unsigned(rot / 8)) : 0;
  const int rc = lane & ((1 << rlg) - 1);
  float* rope_l = reinterpret_cast<float*>(smem + rope_lds_off);
  static_assert(2 * kMaxD <= 2 * kThreads, "two cos/sin values per thread fill the table");
  unsigned char* stage = smem + size_t(wave) * stage_bytes(DT);
  uint16_t* vt = reinterpret_cast<uint16_t*>(stage);
  constexpr int KSTR = k_stride_bytes(DT);

  f32x4 oacc[NDT];
#pragma unroll
  for (int n = 0; n < NDT; ++n) oacc[n] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m_run = kNegInf, l_run = 0.f;

  u32x4 kreg[VCH], vreg[VCH];
  int t0 = wave * kTT;
  {
    uint32_t ob;
    const rsrc_t rk = tile_src(kc, kr, t0, ob);
#pragma unroll
    for (int i = 0; i < VCH; ++i) kreg[i] = buf_load16<kAuxStream>(rk, ob + voff[i]);
    const rsrc_t rv = tile_src(vc, vr, t0, ob);
#pragma unroll
    for (int i = 0; i < VCH; ++i) vreg[i] = buf_load16<kAuxStream>(rv, ob + voff[i]);
  }
  pin_loads();

  // ROPE, once the first tile is in flight: the cos/sin table into LDS, then
  // q's rotary chunks rotated in place (q' = q cos + rotate_half(q) sin, the
  // same rounding as the keys); q's loads were issued before K/V, so this
  // waits for them alone.
  if constexpr (ROPE) {
    // Every entry of the 2 * kMaxD-float table is written (zeros past 2 * rot):
    // with the store under a condition, the compiler moved the cos/sin loads
    // into that branch, behind the K/V loads, and waited for all of them.
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int t = threadIdx.x + j * kThreads;
      rope_l[t] = t >= rot && t < rot + rot / 2 ? -cs_ld[j] : cs_ld[j];
    }
    __syncthreads();
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      const int d0 = 32 * s + 8 * grp;
      if (d0 < rot) {
        const f32x4* cp = reinterpret_cast<const f32x4*>(rope_l + d0);
        const f32x4* sp = reinterpret_cast<const f32x4*>(rope_l + rot + d0);
        qop[s] = __builtin_bit_cast(V8, rope8<T>(__builtin_bit_cast(u32x4, qop[s]), qpart[s], cp[0], cp[1], sp[0],
                                                 sp[1]));
      }
    }
  }

  // One 16-token tile whose K and V are in kreg/vreg; with `pf` the next
  // pass's tile is prefetched into them.  The last tile prefetches nothing:
  // loads past the chunk read zero but still take a memory round trip, which
  // the registers' reuse after the loop would wait for.
  auto tile = [&](int t0, bool pf) __attribute__((always_inline)) {
    // Stage K, then S^T = K Q^T: sacc[i] = score(token t0 + 4grp + i, head col);
    // lane (token col, grp) reads dims 32 s + 8 grp of its token row.
#pragma unroll
    for (int i = 0; i < VCH; ++i) {
      const int qi = lane + kWave * i;
      *reinterpret_cast<u32x4*>(stage + (qi / CPR) * KSTR + (qi % CPR) * 16) = kreg[i];
    }
    // The next pass's K into the freed registers before the staged tile is
    // patched (APP) and rotated (ROPE), so that work overlaps the loads.
    uint32_t nob;
    if (pf) {
      const rsrc_t nk = tile_src(kc, kr, t0 + kWgTokens, nob);
#pragma unroll
      for (int i = 0; i < VCH; ++i) kreg[i] = buf_load16<kAuxStream>(nk, nob + voff[i]);
      pin_loads();
    }
    // APP: the new token's key over its stale row (same wave, program order).
    const int ar = arow - t0;
    const bool arow_here = owner && ar >= 0 && ar < kTT;
    if constexpr (APP) {
      if (arow_here && lane * 8 < d) *reinterpret_cast<u32x4*>(stage + ar * KSTR + lane * 16) = kap;
    }
    if constexpr (ROPE) {
      // Rotary chunks, k' = k cos + rotate_half(k) sin: the tile's 16 * rot/8
      // of them spread over the wave's lanes, two per pass (chunks j and
      // j + 64; chunk j is row j >> rlg, chunk rc of the row, the same for
      // both since rot/8 divides 64).  A chunk and its partner (rc ^ rhc) fall
      // in the same group of 64 and groups are whole rows; each pass reads
      // its four chunks before it writes.  Past the last chunk the second of
      // the pair repeats the first, which writes the same value twice.
      const f32x4 c0 = reinterpret_cast<const f32x4*>(rope_l + rc * 8)[0];
      const f32x4 c1 = reinterpret_cast<const f32x4*>(rope_l + rc * 8)[1];
      const f32x4 s0 = reinterpret_cast<const f32x4*>(rope_l + rot + rc * 8)[0];
      const f32x4 s1 = reinterpret_cast<const f32x4*>(rope_l + rot + rc * 8)[1];
      const int nchk = kTT << rlg;
      for (int j = lane; j < nchk; j += kWave) {
        unsigned char* r0 = stage + (j >> rlg) * KSTR;
        const u32x4 own0 = *reinterpret_cast<const u32x4*>(r0 + rc * 16);
        const u32x4 pq0 = *reinterpret_cast<const u32x4*>(r0 + (rc ^ rhc) * 16);
        *reinterpret_cast<u32x4*>(r0 + rc * 16) = rope8<T>(own0, pq0, c0, c1, s0, s1);
      }
    }
    f32x4 sacc = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      const u32x4 ka = *reinterpret_cast<const u32x4*>(stage + col * KSTR + (32 * s + 8 * grp) * 2);
      sacc = Mfma<T>::qk(__builtin_bit_cast(V8, ka), qop[s], sacc);
    }

    // Online softmax (base 2); m is kept equal across the 4 lanes of a head.
    float sv[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) sv[i] = t0 + 4 * grp + i < len ? sacc[i] * scale_log2 : kNegInf;
    float mx = fmaxf(fmaxf(sv[0], sv[1]), fmaxf(sv[2], sv[3]));
    mx = fmaxf(mx, xor_lane(mx, 16));
    mx = fmaxf(mx, xor_lane(mx, 32));
    const float m_new = fmaxf(m_run, mx);
    const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
    V4 pop;
    float psum = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float p = __builtin_amdgcn_exp2f(sv[i] - m_new);
      psum += p;
      pop[i] = Mfma<T>::cvt(p);
    }
    l_run = l_run * alpha + psum;
    m_run = m_new;

    // Stage V (two 8-byte stores per chunk: the padded stride is 8-byte aligned),
    // then prefetch the next tile's V into the freed registers.
#pragma unroll
    for (int i = 0; i < VCH; ++i) {
      const int qi = lane + kWave * i;
      uint2* dst = reinterpret_cast<uint2*>(vt + (qi / CPR) * VSTR + (qi % CPR) * 8);
      dst[0] = make_uint2(vreg[i].x, vreg[i].y);
      dst[1] = make_uint2(vreg[i].z, vreg[i].w);
    }
    if constexpr (APP) {
      if (arow_here && lane * 8 < d) {
        uint2* dst = reinterpret_cast<uint2*>(vt + ar * VSTR + lane * 8);
        dst[0] = make_uint2(vap.x, vap.y);
        dst[1] = make_uint2(vap.z, vap.w);
      }
    }
    if (pf) {
      const rsrc_t nv = tile_src(vc, vr, t0 + kWgTokens, nob);
#pragma unroll
      for (int i = 0; i < VCH; ++i) vreg[i] = buf_load16<kAuxStream>(nv, nob + voff[i]);
      pin_loads();
    }

    // O^T += V^T P^T: A operand = V[tokens 4grp..4grp+3][dim 16n + col] read transposed.
#pragma unroll
    for (int n = 0; n < NDT; ++n) {
      union {
        V4 v;
        uint16_t u[4];
      } va;
#pragma unroll
      for (int j = 0; j < 4; ++j) va.u[j] = vt[(4 * grp + j) * VSTR + 16 * n + col];
      oacc[n] = Mfma<T>::pv(va.v, pop, oacc[n] * alpha);
    }
  };
  const int ntiles = len > t0 ? (len - t0 + kWgTokens - 1) / kWgTokens : 0;
  for (int it = 0; it + 1 < ntiles; ++it, t0 += kWgTokens) tile(t0, true);
  if (ntiles > 0) tile(t0, false);

  // Per-head l over the 4 lane groups (m is already equal across them).
  l_run += xor_lane(l_run, 16);
  l_run += xor_lane(l_run, 32);

  __syncthreads();  // the V staging area becomes the merge area
  const int ostr = o_stride(d);
  const size_t wstride = merge_floats(d, min(16, group));
  float* mw = reinterpret_cast<float*>(smem) + size_t(wave) * wstride;
  if (grp == 0 && col < heads_here) {
    mw[col] = m_run;
    mw[16 + col] = l_run;
  }
  if (col < heads_here) {
    float* ow = mw + 32 + col * ostr;
#pragma unroll
    for (int n = 0; n < NDT; ++n) {
      const int dim = 16 * n + 4 * grp;  // d % 8 == 0: all four dims valid or none
      if (dim < d) *reinterpret_cast<f32x4*>(ow + dim) = oacc[n];
    }
  }
  __syncthreads();
  // Per-head weights of the 4 waves' partials (lane = head of wave 0): f_w =
  // 2^(m_w - M), M and L = sum f_w l_w, kept in `stat` [16][8].
  const float* m0 = reinterpret_cast<const float*>(smem);
  float* stat = reinterpret_cast<float*>(smem) + kWaves * wstride;
  if (wave == 0 && lane < heads_here) {
    float mv[kWaves], M = kNegInf, L = 0.f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
      mv[w] = m0[w * wstride + lane];
      M = fmaxf(M, mv[w]);
    }
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
      const float f = mv[w] == kNegInf ? 0.f : __builtin_amdgcn_exp2f(mv[w] - M);
      stat[lane * 8 + w] = f;
      L += f * m0[w * wstride + 16 + lane];
    }
    stat[lane * 8 + 4] = M;
    stat[lane * 8 + 5] = L;
  }
  __syncthreads();
  // Wave w merges heads w, w + 4, ...; lane l takes dims 4l..4l+3 (d <= 256).
  const int dim = 4 * lane;
  for (int hd = wave; hd < heads_here; hd += kWaves) {
    if (dim >= d) continue;
    const f32x4 fw = *reinterpret_cast<const f32x4*>(stat + hd * 8);
    f32x4 o = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int w = 0; w < kWaves; ++w)
      o += fw[w] * *reinterpret_cast<const f32x4*>(m0 + w * wstride + 32 + hd * ostr + dim);
    const float M = stat[hd * 8 + 4], L = stat[hd * 8 + 5];
    const size_t bq = size_t(b) * hq + qh0 + hd;
    if (nch == 1) {
#pragma unroll
      for (int k = 0; k < 4; ++k) out[bq * d + dim + k] = from_f<T>(o[k] / L);
    } else {
      const size_t pi = bq * nch + c;
      *reinterpret_cast<f32x4*>(part_o + pi * d + dim) = o;
      if (dim == 0) {
        part_m[pi] = M;
        part_l[pi] = L;
      }
    }
  }
  if constexpr (APP) {
    if (owner && hg == 0 && wave == 0 && lane * 8 < d) {
      size_t row = (size_t(b) * cap + (seq - 1)) * hkv * d;
      bool ok = true;
      if constexpr (PG) {  // the new row's block id is staged (this chunk holds it)
        const int blk = blk_l[(seq - 1) / bsz - bi0];
        ok = blk >= 0 && blk < nblocks;
        row = (size_t(ok ? blk : 0) * bsz + (seq - 1) % bsz) * hkv * d;
      }
      row += size_t(kvh) * d + size_t(lane) * 8;
      if (ok) {
        *reinterpret_cast<u32x4*>(kw + row) = kap;
        *reinterpret_cast<u32x4*>(vw + row) = vap;
      }
    }
  }
}

// grid: (batch * q_heads, ceil(d / 64)); block 256.  Lane = output dim; wave
// w merges chunks [w * cpw, (w + 1) * cpw) online (running max, 16 chunks'
// partial O loaded per step, their m and l as uniform loads), then the 4
// waves' (m, l, O) are combined in LDS.  One memory latency per 16 chunks and
// a single barrier.
template <typename T>
__global__ __launch_bounds__(kThreads) void attn_merge_kernel(const float* __restrict__ part_o,
                                                              const float* __restrict__ part_m,
                                                              const float* __restrict__ part_l,
                                                              T* __restrict__ out, int d, int nch) {
  __shared__ float so[kWaves][kWave];
  __shared__ float sml[kWaves][2];
  const int bq = blockIdx.x;
  const int lane = threadIdx.x % kWave, wave = wave_id();
  const int dim = blockIdx.y * kWave + lane;
  const int cpw = (nch + kWaves - 1) / kWaves;
  const int c0 = wave * cpw, c1 = min(nch, c0 + cpw);
  const rsrc_t por = make_rsrc(part_o + size_t(bq) * nch * d, uint32_t(size_t(nch) * d * 4));
  const uint32_t doff = dim < d ? uint32_t(dim) * 4 : kFar;
  const float* pm = part_m + size_t(bq) * nch;
  const float* pl = part_l + size_t(bq) * nch;
  float M = kNegInf, L = 0.f, o = 0.f;
  for (int cb = c0; cb < c1; cb += kMergeBatch) {
    float pv[kMergeBatch], mv[kMergeBatch], lv[kMergeBatch];
#pragma unroll
    for (int k = 0; k < kMergeBatch; ++k) {
      const int cc = cb + k;
      pv[k] = buf_loadf(por, cc < c1 ? uint32_t(cc) * uint32_t(d) * 4u + doff : kFar);
      const int ci = cc < c1 ? cc : c1 - 1;  // uniform, in range
      mv[k] = pm[ci];
      lv[k] = pl[ci];
    }
    float mb = M;
#pragma unroll
    for (int k = 0; k < kMergeBatch; ++k) mb = cb + k < c1 ? fmaxf(mb, mv[k]) : mb;
    const float r = M == kNegInf ? 0.f : __builtin_amdgcn_exp2f(M - mb);
    o *= r;
    L *= r;
#pragma unroll
    for (int k = 0; k < kMergeBatch; ++k) {
      const float w = cb + k < c1 && mv[k] != kNegInf ? __builtin_amdgcn_exp2f(mv[k] - mb) : 0.f;
      o += w * pv[k];
      L += w * lv[k];
    }
    M = mb;
  }
  so[wave][lane] = o;
  if (lane == 0) {
    sml[wave][0] = M;
    sml[wave][1] = L;
  }
  __syncthreads();
  if (wave == 0 && dim < d) {
    float Mg = kNegInf;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) Mg = fmaxf(Mg, sml[w][0]);
    float os = 0.f, Ls = 0.f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
      const float f = sml[w][0] == kNegInf ? 0.f : __builtin_amdgcn_exp2f(sml[w][0] - Mg);
      os += f * so[w][lane];
      Ls += f * sml[w][1];
    }
    out[size_t(bq) * d + dim] = from_f<T>(os / Ls);
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

// Chunk geometry: enough workgroups per CU for about 64 KB of K/V in flight
// (each wave holds one 16-token K+V tile: one workgroup per CU at D = 256,
// two at 128, four at 64), at least one tile per wave, and every chunk's byte
// range addressable with 31-bit offsets (including the prefetch one pass past
// its end).  More bytes in flight than that only lengthens the HBM queue: with
// two workgroups per CU at D = 256 each tile takes ~4.5 us instead of ~2.2 us
// to arrive, and the waves' finishing times spread over ~12 us instead of ~5.
struct Chunking {
  int nch;
  int chunk_tokens;
};

int max_chunks(int seq) {
  const int m = (seq + kWgTokens - 1) / kWgTokens;
  return m < kMaxChunks ? m : kMaxChunks;
}

int wgs_per_cu(int d, size_t elt) {
  const int tile_bytes = 2 * kTT * d * int(elt);  // one wave's K+V tile
  const int fit = (64 << 10) / (kWaves * tile_bytes);
  return fit > 1 ? fit : 1;
}

int plan_chunks(int units, int hkv, int d, int seq, size_t elt, Chunking* out) {
  int nch = (wgs_per_cu(d, elt) * cu_count() + units - 1) / units;
  const int cap = (seq + kWgTokens - 1) / kWgTokens;
  nch = nch < cap ? nch : cap;
  nch = nch < 1 ? 1 : nch;
  int ct = (seq + nch - 1) / nch;
  ct = (ct + kWgTokens - 1) / kWgTokens * kWgTokens;
  const size_t tsb = size_t(hkv) * d * elt;
  const size_t limit_tokens = (size_t(1) << 31) / tsb;
  if (size_t(ct) + 2 * kWgTokens > limit_tokens) {
    if (limit_tokens < size_t(3 * kWgTokens))
      return set_error(MKQ_ERR_UNSUPPORTED, "full_attention_decode: token row of %zu bytes is too large", tsb);
    ct = int((limit_tokens - 2 * kWgTokens) / kWgTokens * kWgTokens);
  }
  nch = (seq + ct - 1) / ct;
  if (nch > kMaxChunks)
    return set_error(MKQ_ERR_UNSUPPORTED, "full_attention_decode: seq_len %d needs %d chunks (max %d)", seq, nch,
                     kMaxChunks);
  out->nch = nch;
  out->chunk_tokens = ct;
  return MKQ_OK;
}

size_t fast_ws_floats(int batch, int hq, int d, int seq) { return size_t(batch) * hq * max_chunks(seq) * (size_t(d) + 2); }

// Appending launches pass k_new/v_new (non-null) and the cache capacity.
struct Append {
  const void* k_new = nullptr;
  const void* v_new = nullptr;
  int cap = 0;
};

// Paged launches pass the block table [batch, max_blocks] (int32), the block
// size in tokens and the pool's block count.
struct Paged {
  const int* table = nullptr;
  int block_size = 0;
  int max_blocks = 0;
  int num_blocks = 0;
};

// A paged chunk stages at most this many block ids in LDS.
constexpr int kMaxChunkBlocks = 1024;

template <typename T, int DT>
int launch_fast(const void* q, const void* k, const void* v, void* out, int batch, int hq, int hkv, int d, int seq,
                float scale, const float* rope_cs, int rot, const Append& ap, const Paged& pg, float* ws,
                hipStream_t stream) {
  const int group = hq / hkv;
  const int ngroups = (group + 15) / 16;
  const int units = batch * hkv * ngroups;
  Chunking ch;
  const int rc = plan_chunks(units, hkv, d, seq, sizeof(T), &ch);
  if (rc != MKQ_OK) return rc;
  const bool paged = pg.table != nullptr;
  if (paged) {  // a chunk's block ids must fit the LDS table
    const int cap_tokens = (kMaxChunkBlocks - 2) * pg.block_size / kWgTokens * kWgTokens;
    if (ch.chunk_tokens > cap_tokens) {
      ch.chunk_tokens = cap_tokens;
      ch.nch = (seq + cap_tokens - 1) / cap_tokens;
      if (ch.nch > kMaxChunks)
        return set_error(MKQ_ERR_UNSUPPORTED, "full_attention_decode_paged: seq_len %d needs too many chunks", seq);
    }
  }
  const size_t lds = chunk_lds_bytes<DT>(d, group < 16 ? group : 16);
  static bool attr_set = false;
  if (!attr_set) {
    const int plain = int(chunk_lds_bytes<DT>(DT, 16));
    const int roped = int(chunk_lds_bytes<DT>(DT, 16) + 16 + 2 * kMaxD * sizeof(float));
    const int pagedb = int(chunk_lds_bytes<DT>(DT, 16) + 16 + kMaxChunkBlocks * sizeof(int));
    const int paged_roped = int(pagedb + 2 * kMaxD * sizeof(float));
    MKQ_HIP_TRY(hipFuncSetAttribute(reinterpret_cast<const void*>(&attn_chunk_kernel<T, DT, false, false, false>),
                                    hipFuncAttributeMaxDynamicSharedMemorySize, plain));
    MKQ_HIP_TRY(hipFuncSetAttribute(reinterpret_cast<const void*>(&attn_chunk_kernel<T, DT, true, false, false>),
                                    hipFuncAttributeMaxDynamicSharedMemorySize, roped));
    MKQ_HIP_TRY(hipFuncSetAttribute(reinterpret_cast<const void*>(&attn_chunk_kernel<T, DT, false, true, false>),
                                    hipFuncAttributeMaxDynamicSharedMemorySize, plain));
    MKQ_HIP_TRY(hipFuncSetAttribute(reinterpret_cast<const void*>(&attn_chunk_kernel<T, DT, true, true, false>),
                                    hipFuncAttributeMaxDynamicSharedMemorySize, roped));
    MKQ_HIP_TRY(hipFuncSetAttribute(reinterpret_cast<const void*>(&attn_chunk_kernel<T, DT, false, false, true>),
                                    hipFuncAttributeMaxDynamicSharedMemorySize, pagedb));
    MKQ_HIP_TRY(hipFuncSetAttribute(reinterpret_cast<const void*>(&attn_chunk_kernel<T, DT, false, true, true>),
                                    hipFuncAttributeMaxDynamicSharedMemorySize, pagedb));
    MKQ_HIP_TRY(hipFuncSetAttribute(reinterpret_cast<const void*>(&attn_chunk_kernel<T, DT, true, false, true>),
                                    hipFuncAttributeMaxDynamicSharedMemorySize, paged_roped));
    MKQ_HIP_TRY(hipFuncSetAttribute(reinterpret_cast<const void*>(&attn_chunk_kernel<T, DT, true, true, true>),
                                    hipFuncAttributeMaxDynamicSharedMemorySize, paged_roped));
    attr_set = true;
  }
  MKQ_REQUIRE(size_t(ch.nch) * units < (size_t(1) << 31), "full_attention_decode: grid too large");
  float* part_o = ws;
  float* part_m = part_o + size_t(batch) * hq * ch.nch * d;
  float* part_l = part_m + size_t(batch) * hq * ch.nch;
  const bool app = ap.k_new != nullptr;
  auto* kern = paged  ? (app ? (rot > 0 ? attn_chunk_kernel<T, DT, true, true, true>
                                       : attn_chunk_kernel<T, DT, false, true, true>)
                             : rot > 0 ? attn_chunk_kernel<T, DT, true, false, true>
                                       : attn_chunk_kernel<T, DT, false, false, true>)
               : rot > 0 ? (app ? attn_chunk_kernel<T, DT, true, true, false> : attn_chunk_kernel<T, DT, true, false, false>)
                         : (app ? attn_chunk_kernel<T, DT, false, true, false>
                                : attn_chunk_kernel<T, DT, false, false, false>);
  // The cos/sin table (ROPE) and then the block ids (PG) follow the
  // staging/merge area.
  const size_t rope_off = (lds + 15) / 16 * 16;
  const size_t blk_off = rope_off + (rot > 0 ? size_t(2 * kMaxD) * sizeof(float) : 0);
  const int nblk = paged ? (ch.chunk_tokens + pg.block_size - 1) / pg.block_size + 2 : 0;
  const size_t lds_all = paged ? blk_off + size_t(nblk) * sizeof(int) : rot > 0 ? blk_off : lds;
  kern<<<dim3(ch.nch * units), kThreads, lds_all, stream>>>(
      static_cast<const T*>(q), static_cast<const T*>(k), static_cast<const T*>(v), part_o, part_m, part_l,
      static_cast<T*>(out), rope_cs, static_cast<const T*>(ap.k_new), static_cast<const T*>(ap.v_new),
      app ? static_cast<T*>(const_cast<void*>(k)) : nullptr, app ? static_cast<T*>(const_cast<void*>(v)) : nullptr,
      app ? ap.cap : seq, pg.table, pg.block_size, pg.max_blocks, pg.num_blocks, int(blk_off), rot, int(rope_off), hq,
      hkv, d, seq, group, ngroups, units, ch.nch, ch.chunk_tokens, scale * kLog2e);
  MKQ_LAUNCH_CHECK("attn_chunk_kernel");
  if (ch.nch > 1) {
    dim3 g2(batch * hq, (d + kWave - 1) / kWave);
    attn_merge_kernel<T><<<g2, kThreads, 0, stream>>>(part_o, part_m, part_l, static_cast<T*>(out), d, ch.nch);
    MKQ_LAUNCH_CHECK("attn_merge_kernel");
  }
  return MKQ_OK;
}

template <typename T>
int launch_fast_d(const void* q, const void* k, const void* v, void* out, int batch, int hq, int hkv, int d, int seq,
                  float scale, const float* rope_cs, int rot, const Append& ap, const Paged& pg, float* ws,
                  hipStream_t stream) {
  if (d <= 64)
    return launch_fast<T, 64>(q, k, v, out, batch, hq, hkv, d, seq, scale, rope_cs, rot, ap, pg, ws, stream);
  if (d <= 128)
    return launch_fast<T, 128>(q, k, v, out, batch, hq, hkv, d, seq, scale, rope_cs, rot, ap, pg, ws, stream);
  return launch_fast<T, 256>(q, k, v, out, batch, hq, hkv, d, seq, scale, rope_cs, rot, ap, pg, ws, stream);
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

namespace {

int attention_entry(const char* fn, int dtype, const void* q, const void* k_cache, const void* v_cache, void* out,
                    int batch, int q_heads, int kv_heads, int head_dim, int seq_len, float scale,
                    const float* rope_cs, int rot, const Append& ap, const Paged& pg, void* workspace,
                    size_t workspace_bytes, void* stream) {
  clear_error();
  MKQ_REQUIRE(batch > 0 && q_heads > 0 && kv_heads > 0 && head_dim > 0, "%s: sizes must be positive", fn);
  MKQ_REQUIRE(seq_len > 0, "seq_len must be positive");
  MKQ_REQUIRE(q_heads % kv_heads == 0, "query_heads must be divisible by kv_heads");
  MKQ_REQUIRE(head_dim <= kMaxD, "head_dim > 256 is not supported by this kernel");
  MKQ_REQUIRE(q && k_cache && v_cache && out, "%s: null tensor pointer", fn);
  MKQ_REQUIRE(batch <= 65535 && q_heads <= 65535, "%s: batch/heads too large", fn);
  MKQ_REQUIRE(workspace && workspace_bytes >= mkq_full_attention_decode_workspace_bytes(batch, q_heads, kv_heads,
                                                                                        head_dim, seq_len),
              "%s: workspace too small", fn);
  MKQ_REQUIRE((reinterpret_cast<uintptr_t>(workspace) & 255u) == 0, "%s: workspace must be 256-byte aligned", fn);
  hipStream_t s = static_cast<hipStream_t>(stream);
  float* ws = static_cast<float*>(workspace);
  const bool fast_ok = (head_dim % 8 == 0) && aligned16(q) && aligned16(k_cache) && aligned16(v_cache);
  if (pg.table) {
    MKQ_REQUIRE(pg.block_size > 0 && pg.block_size % 16 == 0, "%s: block_size %d must be a positive multiple of 16",
                fn, pg.block_size);
    MKQ_REQUIRE(pg.num_blocks > 0 && pg.max_blocks > 0, "%s: num_blocks and max_blocks must be positive", fn);
    MKQ_REQUIRE(int64_t(pg.max_blocks) * pg.block_size >= seq_len, "%s: max_blocks * block_size < seq_len", fn);
    if (!fast_ok || (dtype != MKQ_DTYPE_BF16 && dtype != MKQ_DTYPE_F16))
      return set_error(MKQ_ERR_UNSUPPORTED,
                       "%s: the paged layout needs bf16/f16, head_dim %% 8 == 0 and 16-byte aligned tensors", fn);
  }
  if (ap.k_new) {
    MKQ_REQUIRE(ap.v_new, "%s: null tensor pointer", fn);
    MKQ_REQUIRE(ap.cap >= seq_len, "%s: capacity %d is below seq_len %d", fn, ap.cap, seq_len);
    if (!fast_ok || !aligned16(ap.k_new) || !aligned16(ap.v_new) ||
        (dtype != MKQ_DTYPE_BF16 && dtype != MKQ_DTYPE_F16))
      return set_error(MKQ_ERR_UNSUPPORTED,
                       "%s: the in-kernel append needs bf16/f16, head_dim %% 8 == 0 and 16-byte aligned tensors", fn);
  }
  if (rot > 0) {
    MKQ_REQUIRE(rope_cs, "%s: null cos/sin pointer", fn);
    if (!fast_ok || (dtype != MKQ_DTYPE_BF16 && dtype != MKQ_DTYPE_F16) || rot < 16 || rot > head_dim ||
        (rot & (rot - 1)) != 0)
      return set_error(MKQ_ERR_UNSUPPORTED,
                       "%s: rotary_dim %d needs a power of two in [16, head_dim], bf16/f16 and head_dim %% 8 == 0 "
                       "with 16-byte aligned tensors",
                       fn, rot);
  }
  switch (dtype) {
    case MKQ_DTYPE_BF16:
      return fast_ok ? launch_fast_d<bf16_t>(q, k_cache, v_cache, out, batch, q_heads, kv_heads, head_dim, seq_len,
                                             scale, rope_cs, rot, ap, pg, ws, s)
                     : launch_generic<bf16_t>(q, k_cache, v_cache, out, batch, q_heads, kv_heads, head_dim, seq_len,
                                              scale, ws, s);
    case MKQ_DTYPE_F16:
      return fast_ok ? launch_fast_d<f16_t>(q, k_cache, v_cache, out, batch, q_heads, kv_heads, head_dim, seq_len,
                                            scale, rope_cs, rot, ap, pg, ws, s)
                     : launch_generic<f16_t>(q, k_cache, v_cache, out, batch, q_heads, kv_heads, head_dim, seq_len,
                                             scale, ws, s);
    case MKQ_DTYPE_F32:
      return launch_generic<float>(q, k_cache, v_cache, out, batch, q_heads, kv_heads, head_dim, seq_len, scale, ws,
                                   s);
    default:
      return set_error(MKQ_ERR_INVALID, "%s: unknown dtype %d", fn, dtype);
  }
}

}  // namespace

extern "C" int mkq_full_attention_decode(int dtype, const void* q, const void* k_cache, const void* v_cache,
                                         void* out, int batch, int q_heads, int kv_heads, int head_dim, int seq_len,
                                         float scale, void* workspace, size_t workspace_bytes, void* stream) {
  return attention_entry("full_attention_decode", dtype, q, k_cache, v_cache, out, batch, q_heads, kv_heads,
                         head_dim, seq_len, scale, nullptr, 0, Append{}, Paged{}, workspace, workspace_bytes, stream);
}

extern "C" int mkq_full_attention_decode_rope(int dtype, const void* q, const void* k_cache, const void* v_cache,
                                              void* out, int batch, int q_heads, int kv_heads, int head_dim,
                                              int seq_len, float scale, const float* cos_sin, int rotary_dim,
                                              void* workspace, size_t workspace_bytes, void* stream) {
  return attention_entry("full_attention_decode_rope", dtype, q, k_cache, v_cache, out, batch, q_heads, kv_heads,
                         head_dim, seq_len, scale, cos_sin, rotary_dim, Append{}, Paged{}, workspace,
                         workspace_bytes, stream);
}

extern "C" int mkq_full_attention_decode_append(int dtype, const void* q, const void* k_new, const void* v_new,
                                                void* k_cache, void* v_cache, void* out, int batch, int q_heads,
                                                int kv_heads, int head_dim, int seq_len, int capacity, float scale,
                                                const float* cos_sin, int rotary_dim, void* workspace,
                                                size_t workspace_bytes, void* stream) {
  const char* fn = "full_attention_decode_append";
  if (!k_new || !v_new) {
    clear_error();
    return set_error(MKQ_ERR_INVALID, "%s: null tensor pointer", fn);
  }
  Append ap;
  ap.k_new = k_new;
  ap.v_new = v_new;
  ap.cap = capacity;
  return attention_entry(fn, dtype, q, k_cache, v_cache, out, batch, q_heads, kv_heads, head_dim, seq_len, scale,
                         cos_sin, cos_sin ? rotary_dim : 0, ap, Paged{}, workspace, workspace_bytes, stream);
}

extern "C" int mkq_full_attention_decode_paged(int dtype, const void* q, const void* k_blocks, const void* v_blocks,
                                               const int* block_table, void* out, int batch, int q_heads,
                                               int kv_heads, int head_dim, int seq_len, int block_size,
                                               int max_blocks, int num_blocks, float scale, void* workspace,
                                               size_t workspace_bytes, void* stream) {
  const char* fn = "full_attention_decode_paged";
  if (!block_table) {
    clear_error();
    return set_error(MKQ_ERR_INVALID, "%s: null tensor pointer", fn);
  }
  Paged pg;
  pg.table = block_table;
  pg.block_size = block_size;
  pg.max_blocks = max_blocks;
  pg.num_blocks = num_blocks;
  return attention_entry(fn, dtype, q, k_blocks, v_blocks, out, batch, q_heads, kv_heads, head_dim, seq_len, scale,
                         nullptr, 0, Append{}, pg, workspace, workspace_bytes, stream);
}

extern "C" int mkq_full_attention_decode_paged_rope(int dtype, const void* q, const void* k_blocks,
                                                    const void* v_blocks, const int* block_table, void* out,
                                                    int batch, int q_heads, int kv_heads, int head_dim, int seq_len,
                                                    int block_size, int max_blocks, int num_blocks, float scale,
                                                    const float* cos_sin, int rotary_dim, void* workspace,
                                                    size_t workspace_bytes, void* stream) {
  const char* fn = "full_attention_decode_paged_rope";
  if (!block_table || !cos_sin) {
    clear_error();
    return set_error(MKQ_ERR_INVALID, "%s: null tensor pointer", fn);
  }
  if (rotary_dim <= 0) {
    clear_error();
    return set_error(MKQ_ERR_INVALID, "%s: rotary_dim %d must be positive", fn, rotary_dim);
  }
  Paged pg;
  pg.table = block_table;
  pg.block_size = block_size;
  pg.max_blocks = max_blocks;
  pg.num_blocks = num_blocks;
  return attention_entry(fn, dtype, q, k_blocks, v_blocks, out, batch, q_heads, kv_heads, head_dim, seq_len, scale,
                         cos_sin, rotary_dim, Append{}, pg, workspace, workspace_bytes, stream);
}

extern "C" int mkq_full_attention_decode_paged_append(int dtype, const void* q, const void* k_new, const void* v_new,
                                                      void* k_blocks, void* v_blocks, const int* block_table,
                                                      void* out, int batch, int q_heads, int kv_heads, int head_dim,
                                                      int seq_len, int block_size, int max_blocks, int num_blocks,
                                                      float scale, void* workspace, size_t workspace_bytes,
                                                      void* stream) {
  const char* fn = "full_attention_decode_paged_append";
  if (!block_table || !k_new || !v_new) {
    clear_error();
    return set_error(MKQ_ERR_INVALID, "%s: null tensor pointer", fn);
  }
  Paged pg;
  pg.table = block_table;
  pg.block_size = block_size;
  pg.max_blocks = max_blocks;
  pg.num_blocks = num_blocks;
  Append ap;
  ap.k_new = k_new;
  ap.v_new = v_new;
  ap.cap = seq_len;  // unused by the paged store
  return attention_entry(fn, dtype, q, k_blocks, v_blocks, out, batch, q_heads, kv_heads, head_dim, seq_len, scale,
                         nullptr, 0, ap, pg, workspace, workspace_bytes, stream);
}

extern "C" int mkq_full_attention_decode_paged_append_rope(int dtype, const void* q, const void* k_new,
                                                           const void* v_new, void* k_blocks, void* v_blocks,
                                                           const int* block_table, void* out, int batch, int q_heads,
                                                           int kv_heads, int head_dim, int seq_len, int block_size,
                                                           int max_blocks, int num_blocks, float scale,
                                                           const float* cos_sin, int rotary_dim, void* workspace,
                                                           size_t workspace_bytes, void* stream) {
  const char* fn = "full_attention_decode_paged_append_rope";
  if (!block_table || !k_new || !v_new || !cos_sin) {
    clear_error();
    return set_error(MKQ_ERR_INVALID, "%s: null tensor pointer", fn);
  }
  if (rotary_dim <= 0) {
    clear_error();
    return set_error(MKQ_ERR_INVALID, "%s: rotary_dim %d must be positive", fn, rotary_dim);
  }
  Paged pg;
  pg.table = block_table;
  pg.block_size = block_size;
  pg.max_blocks = max_blocks;
  pg.num_blocks = num_blocks;
  Append ap;
  ap.k_new = k_new;
  ap.v_new = v_new;
  ap.cap = seq_len;  // unused by the paged store
  return attention_entry(fn, dtype, q, k_blocks, v_blocks, out, batch, q_heads, kv_heads, head_dim, seq_len, scale,
                         cos_sin, rotary_dim, ap, pg, workspace, workspace_bytes, stream);
}
