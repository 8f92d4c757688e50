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

// float -> bfloat16, round to nearest even; NaN stays NaN.
__device__ __forceinline__ uint16_t f2bf_bits(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return uint16_t((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return uint16_t(u >> 16);
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
