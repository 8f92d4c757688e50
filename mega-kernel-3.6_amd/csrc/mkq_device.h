// Device-side helpers for the gfx950 decode kernels: element types, 16-byte
// chunk unpacking, wave64 reductions.
//
// Counterpart of the reference's csrc/common.cuh:14-55 (mk_to_float,
// mk_from_float, mk_silu, mk_warp_sum, mk_block_sum), re-derived for 64-wide
// wavefronts: reductions use DPP within a 16-lane row and a lane permute across
// rows instead of 32-lane shuffles.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mkq {

constexpr int kWave = 64;

// Index of the calling wave in its workgroup, as a wave-uniform (scalar)
// value.  threadIdx.x / 64 is the same in every lane, but the compiler treats
// it as divergent; buffer descriptors and row addresses derived from it would
// then be built per lane and every buffer load wrapped in a readfirstlane
// loop.
__device__ __forceinline__ int wave_id() { return __builtin_amdgcn_readfirstlane(int(threadIdx.x) / kWave); }

// Keeps the loads issued above this point where they are.  The compiler sinks
// a load to the block of its first use when nothing in between may write the
// loaded memory -- across loops and barriers -- which turns an early prefetch
// into a load waited on immediately.  An empty asm that clobbers memory is a
// point no load may cross; it has no register operands, so it adds no wait.
__device__ __forceinline__ void pin_loads() { asm volatile("" ::: "memory"); }

// bfloat16 storage type (bit pattern).
struct bf16_t {
  uint16_t bits;
};
typedef _Float16 f16_t;

typedef float f32x4 __attribute__((ext_vector_type(4)));
// One 16-byte chunk of a row (native vector type, so the non-temporal and
// buffer builtins accept it).
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef short bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

// ---------------------------------------------------------------------------
// scalar conversions
// ---------------------------------------------------------------------------
__device__ __forceinline__ float to_f(bf16_t v) { return __uint_as_float(uint32_t(v.bits) << 16); }
__device__ __forceinline__ float to_f(f16_t v) { return float(v); }
__device__ __forceinline__ float to_f(float v) { return v; }

// float -> bfloat16, round to nearest even; NaN stays NaN.  Bit for bit the
// rule u' = (u + 0x7fff + ((u >> 16) & 1)) >> 16 for non-NaN u and
// (u >> 16) | 0x40 for NaN, which the compiler's float -> __bf16 conversion
// (gfx950's v_cvt_pk_bf16_f32) computes (checked against that rule on all
// 2^32 inputs, denormals and NaNs included).  The conversion is left to the
// compiler, which tracks the instruction's register hazards.
__device__ __forceinline__ uint16_t f2bf_bits(float f) { return __builtin_bit_cast(uint16_t, static_cast<__bf16>(f)); }
// Two of them packed: lo in bits 0..15, hi in bits 16..31.
__device__ __forceinline__ uint32_t f2bf2_bits(float lo, float hi) {
  return uint32_t(f2bf_bits(lo)) | (uint32_t(f2bf_bits(hi)) << 16);
}

template <typename T>
__device__ __forceinline__ T from_f(float f);
template <>
__device__ __forceinline__ bf16_t from_f<bf16_t>(float f) {
  bf16_t r;
  r.bits = f2bf_bits(f);
  return r;
}
template <>
__device__ __forceinline__ f16_t from_f<f16_t>(float f) {
  return f16_t(f);
}
template <>
__device__ __forceinline__ float from_f<float>(float f) {
  return f;
}

// Elements of T in one 16-byte chunk.
template <typename T>
struct Epc {
  static constexpr int value = 16 / int(sizeof(T));
};

// ---------------------------------------------------------------------------
// 16-byte chunk -> floats
// ---------------------------------------------------------------------------
__device__ __forceinline__ void unpack(const u32x4& c, float (&f)[8], bf16_t) {
  f[0] = __uint_as_float(c.x << 16);
  f[1] = __uint_as_float(c.x & 0xffff0000u);
  f[2] = __uint_as_float(c.y << 16);
  f[3] = __uint_as_float(c.y & 0xffff0000u);
  f[4] = __uint_as_float(c.z << 16);
  f[5] = __uint_as_float(c.z & 0xffff0000u);
  f[6] = __uint_as_float(c.w << 16);
  f[7] = __uint_as_float(c.w & 0xffff0000u);
}
__device__ __forceinline__ void unpack(const u32x4& c, float (&f)[8], f16_t) {
  const uint32_t w[4] = {c.x, c.y, c.z, c.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f16x2 h = __builtin_bit_cast(f16x2, w[i]);
    f[2 * i] = float(h[0]);
    f[2 * i + 1] = float(h[1]);
  }
}
__device__ __forceinline__ void unpack(const u32x4& c, float (&f)[4], float) {
  f[0] = __uint_as_float(c.x);
  f[1] = __uint_as_float(c.y);
  f[2] = __uint_as_float(c.z);
  f[3] = __uint_as_float(c.w);
}

// Load chunk `j` (elements [j*EPC, j*EPC+EPC)) of a row of length n.
// VEC: the row is 16-byte aligned and n is a multiple of EPC, so the chunk is
// one 128-bit load.  Otherwise elements are loaded one by one and positions
// >= n read as zero.
template <typename T, bool VEC>
__device__ __forceinline__ u32x4 load_chunk(const T* __restrict__ row, int j, int n) {
  constexpr int EPC = Epc<T>::value;
  if constexpr (VEC) {
    return *reinterpret_cast<const u32x4*>(row + size_t(j) * EPC);
  } else {
    union {
      u32x4 v;
      T e[EPC];
    } u;
    u.v = u32x4{0u, 0u, 0u, 0u};
#pragma unroll
    for (int i = 0; i < EPC; ++i) {
      int k = j * EPC + i;
      if (k < n) u.e[i] = row[k];
    }
    return u.v;
  }
}

// ---------------------------------------------------------------------------
// buffer-resource loads: branch-free and bounds-checked by the hardware
// ---------------------------------------------------------------------------
// A raw buffer descriptor (stride 0) covers `bytes` bytes from `base`; loads
// at offsets past the end return zero and stores there are dropped.  Code that
// guards each load with a branch makes the compiler wait for every load at the
// branch join; expressing the guard as the descriptor's size keeps all loads
// of a row in flight at once.  Word 3 = 0x00020000 is the gfx9 raw-buffer
// format word (32-bit data, no swizzle).
typedef __amdgpu_buffer_rsrc_t rsrc_t;

__device__ __forceinline__ rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}

// Cache-policy bits of a buffer access: bit 1 = nt (streaming, read once);
// bit 4 = sc1, the policy of an agent-scope atomic load, which reads data
// written by other XCDs in the same kernel coherently.
constexpr int kAuxNone = 0;
constexpr int kAuxStream = 2;
constexpr int kAuxCoherent = 16;

template <int AUX = kAuxNone>
__device__ __forceinline__ u32x4 buf_load16(rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, AUX));
}
template <int AUX = kAuxNone>
__device__ __forceinline__ uint32_t buf_load4(rsrc_t r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b32(r, (int)off, 0, AUX);
}
__device__ __forceinline__ float buf_loadf(rsrc_t r, uint32_t off) { return __uint_as_float(buf_load4(r, off)); }

// One agent-coherent 64-bit store of {float bits, tag}: a reader that loads the
// word with agent-coherent (sc1) loads and sees the current tag has the value
// (an aligned 8-byte store is seen whole), with no flag and no fence.
__device__ __forceinline__ void put_tagged(uint64_t* p, float v, unsigned tag) {
  const uint64_t word = (uint64_t(tag) << 32) | uint64_t(__float_as_uint(v));
  __hip_atomic_store(p, word, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void buf_storef(rsrc_t r, uint32_t off, float v) {
  __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v), r, (int)off, 0, 0);
}

// Partials cross workgroups (and XCDs) through agent-coherent accesses: the
// stores write through to memory and the loads bypass the XCD-private L2
// copies, so no cache writeback or invalidation (an agent-scope fence) is
// needed.
__device__ __forceinline__ void store_partial(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float load_partial(const float* p) {
  return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Per-pair arrival: each thread waits until its partial stores are complete
// (acknowledged by memory), the barrier gathers the workgroup, then one
// thread counts the arrival; the workgroup learns whether it came last.  A
// workgroup that reads the final count reads the partials only after it, so
// it sees every split's complete stores.
__device__ __forceinline__ bool arrive_last(unsigned* cnt, unsigned splits, int* flag) {
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  if (threadIdx.x == 0)
    *flag = __hip_atomic_fetch_add(cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == splits - 1u ? 1 : 0;
  __syncthreads();
  return *flag != 0;
}

// Streaming (read-once) variant for weights: non-temporal hint.
template <typename T, bool VEC>
__device__ __forceinline__ u32x4 load_chunk_nt(const T* __restrict__ row, int j, int n) {
  constexpr int EPC = Epc<T>::value;
  if constexpr (VEC) {
    return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(row + size_t(j) * EPC));
  } else {
    return load_chunk<T, false>(row, j, n);
  }
}

// ---------------------------------------------------------------------------
// wave64 reductions
// ---------------------------------------------------------------------------
// DPP controls: quad_perm [1,0,3,2] = 0xB1, quad_perm [2,3,0,1] = 0x4E,
// row_ror:4 = 0x124, row_ror:8 = 0x128.
template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}

__device__ __forceinline__ float xor_lane(float v, int mask) {
  return __shfl_xor(v, mask, kWave);
}

// Sum over the 16 lanes of each DPP row (result in every lane of the row).
__device__ __forceinline__ float row16_sum(float v) {
  v += dpp<0xB1>(v);
  v += dpp<0x4E>(v);
  v += dpp<0x124>(v);
  v += dpp<0x128>(v);
  return v;
}

// Sum over all 64 lanes (result in every lane).
__device__ __forceinline__ float wave_sum(float v) {
  v = row16_sum(v);
  v += xor_lane(v, 16);
  v += xor_lane(v, 32);
  return v;
}

// Sum over all 64 lanes, returned as a wave-uniform value.  DPP within each
// 16-lane row, then row_bcast:15 / row_bcast:31 carry the row sums into lane
// 63, which is read out with readlane -- no LDS permute on the way.
__device__ __forceinline__ float wave_sum_u(float v) {
  v = row16_sum(v);
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x142, 0xA, 0xF, false));
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x143, 0xC, 0xF, false));
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

// Two independent wave sums, their DPP steps interleaved so that each step's
// latency is hidden behind the other's; results wave-uniform.
__device__ __forceinline__ void wave_sum2_u(float& a, float& b) {
  a += dpp<0xB1>(a);
  b += dpp<0xB1>(b);
  a += dpp<0x4E>(a);
  b += dpp<0x4E>(b);
  a += dpp<0x124>(a);
  b += dpp<0x124>(b);
  a += dpp<0x128>(a);
  b += dpp<0x128>(b);
  a += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(a), 0x142, 0xA, 0xF, false));
  b += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(b), 0x142, 0xA, 0xF, false));
  a += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(a), 0x143, 0xC, 0xF, false));
  b += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(b), 0x143, 0xC, 0xF, false));
  a = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(a), 63));
  b = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(b), 63));
}

// (value, index) of the largest value over the wave, ties to the lower index;
// returned wave-uniform.  DPP steps inside each 16-lane row, then the four row
// results are compared through readlane.
template <int CTRL>
__device__ __forceinline__ void argmax_dpp_step(float& v, int& i) {
  const float ov = __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
  const int oi = __builtin_amdgcn_update_dpp(0, i, CTRL, 0xF, 0xF, false);
  const bool take = ov > v || (ov == v && oi < i);
  v = take ? ov : v;
  i = take ? oi : i;
}
__device__ __forceinline__ void wave_argmax_u(float& v, int& i) {
  argmax_dpp_step<0xB1>(v, i);
  argmax_dpp_step<0x4E>(v, i);
  argmax_dpp_step<0x124>(v, i);
  argmax_dpp_step<0x128>(v, i);
  float bv = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
  int bi = __builtin_amdgcn_readlane(i, 0);
#pragma unroll
  for (int r = 1; r < 4; ++r) {
    const float rv = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16 * r));
    const int ri = __builtin_amdgcn_readlane(i, 16 * r);
    if (rv > bv || (rv == bv && ri < bi)) {
      bv = rv;
      bi = ri;
    }
  }
  v = bv;
  i = bi;
}

// Order-preserving 32-bit key of a float: the unsigned order of the keys is
// the numeric order of the values (negatives reversed).  0 is below every
// key of a non-NaN value, so it can mark an empty slot.
__device__ __forceinline__ uint32_t ord_key(float v) {
  const uint32_t u = __float_as_uint(v);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ float ord_value(uint32_t k) {
  return __uint_as_float((k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
}

// Unsigned max over all 64 lanes, returned wave-uniform (DPP inside rows,
// row_bcast into lane 63, readlane); 0 is the identity.
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
  v = max(v, uint32_t(__builtin_amdgcn_update_dpp(0, int(v), 0xB1, 0xF, 0xF, false)));
  v = max(v, uint32_t(__builtin_amdgcn_update_dpp(0, int(v), 0x4E, 0xF, 0xF, false)));
  v = max(v, uint32_t(__builtin_amdgcn_update_dpp(0, int(v), 0x124, 0xF, 0xF, false)));
  v = max(v, uint32_t(__builtin_amdgcn_update_dpp(0, int(v), 0x128, 0xF, 0xF, false)));
  v = max(v, uint32_t(__builtin_amdgcn_update_dpp(0, int(v), 0x142, 0xA, 0xF, false)));
  v = max(v, uint32_t(__builtin_amdgcn_update_dpp(0, int(v), 0x143, 0xC, 0xF, false)));
  return uint32_t(__builtin_amdgcn_readlane(int(v), 63));
}

// Order-preserving 64-bit key of (value, index): larger value first, then the
// lower index.  A float's bits map to an unsigned integer with the same order
// (negatives reversed); the low word holds ~index.
__device__ __forceinline__ uint64_t rank_key(float v, int index) {
  const uint32_t u = __float_as_uint(v);
  const uint32_t hi = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
  return (uint64_t(hi) << 32) | uint64_t(~uint32_t(index));
}
__device__ __forceinline__ float key_value(uint64_t k) {
  const uint32_t hi = uint32_t(k >> 32);
  return __uint_as_float((hi & 0x80000000u) ? (hi & 0x7fffffffu) : ~hi);
}
__device__ __forceinline__ int key_index(uint64_t k) { return int(~uint32_t(k)); }

template <int CTRL>
__device__ __forceinline__ uint64_t max_dpp_step(uint64_t k) {
  const uint32_t hi = __builtin_amdgcn_update_dpp(0, uint32_t(k >> 32), CTRL, 0xF, 0xF, false);
  const uint32_t lo = __builtin_amdgcn_update_dpp(0, uint32_t(k), CTRL, 0xF, 0xF, false);
  const uint64_t o = (uint64_t(hi) << 32) | lo;
  return o > k ? o : k;
}
// Largest key over the wave, returned wave-uniform.
__device__ __forceinline__ uint64_t wave_max_key(uint64_t k) {
  k = max_dpp_step<0xB1>(k);
  k = max_dpp_step<0x4E>(k);
  k = max_dpp_step<0x124>(k);
  k = max_dpp_step<0x128>(k);
  uint64_t best = 0;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const uint64_t rk = (uint64_t(uint32_t(__builtin_amdgcn_readlane(int(k >> 32), 16 * r))) << 32) |
                        uint32_t(__builtin_amdgcn_readlane(int(uint32_t(k)), 16 * r));
    best = rk > best ? rk : best;
  }
  return best;
}

__device__ __forceinline__ float wave_max(float v) {
  v = fmaxf(v, dpp<0xB1>(v));
  v = fmaxf(v, dpp<0x4E>(v));
  v = fmaxf(v, dpp<0x124>(v));
  v = fmaxf(v, dpp<0x128>(v));
  v = fmaxf(v, xor_lane(v, 16));
  v = fmaxf(v, xor_lane(v, 32));
  return v;
}

// ---------------------------------------------------------------------------
// math
// ---------------------------------------------------------------------------
constexpr float kLog2e = 1.4426950408889634f;

// e^x through the hardware base-2 exponential.
__device__ __forceinline__ float exp_fast(float x) { return __builtin_amdgcn_exp2f(x * kLog2e); }

// silu(x) = x * sigmoid(x) = x / (1 + e^-x)
__device__ __forceinline__ float silu(float x) { return x / (1.0f + exp_fast(-x)); }

__device__ __forceinline__ float sigmoid(float x) { return 1.0f / (1.0f + exp_fast(-x)); }

}  // namespace mkq
