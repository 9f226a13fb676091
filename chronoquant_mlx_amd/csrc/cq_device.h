// cq_device.h — device-side helpers shared by the ChronoQuant HIP kernels
// (gfx950 / CDNA4, wave64).  Host code includes it only for the parameter
// structs and validation helpers.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/chronoquant.h"

namespace cq {

constexpr int kWave = 64;
constexpr int kMaxHeadDim = 256;  // same limit as the reference's fused path

// ---------------------------------------------------------------------------
// Packed rows.  Dim d's code is stored as the fb-bit field code + 2^(fb-1)
// at bits [fb*d, fb*d + fb) of the row's little-endian bit stream: fb = 4
// for INT4 lanes (the reference's layout), delta_bits for dense rows.
// ---------------------------------------------------------------------------
__host__ __device__ inline int field_bits(const cq_component &c) {
  return c.packing == CQ_PACK_DENSE ? c.delta_bits : 4;
}
__host__ __device__ inline int row_words_of(int D, int fb) { return (D * fb + 31) / 32; }
__host__ __device__ inline int row_words(const cq_component &c, int D) {
  return row_words_of(D, field_bits(c));
}
// n <= 32 stream bits starting at bit `bit` of a row of rw words (bits past
// n, and past the row, read 0)
__device__ __forceinline__ uint32_t stream_bits(const uint32_t *row, int rw, int bit, int n) {
  const int w = bit >> 5, o = bit & 31;
  uint32_t v = w < rw ? row[w] >> o : 0u;
  if (o && o + n > 32 && w + 1 < rw) v |= row[w + 1] << (32 - o);
  return n >= 32 ? v : v & ((1u << n) - 1u);
}
// an fb-bit field of a code: code + 2^(fb-1), clipped into the field
__device__ __forceinline__ uint32_t code_field(int code, int fb) {
  int u = code + (1 << (fb - 1));
  const int top = (1 << fb) - 1;
  return (uint32_t)(u < 0 ? 0 : (u > top ? top : u));
}

// ---------------------------------------------------------------------------
// dtype traits.  round() rounds a binary32 value to the dtype (nearest even)
// and returns it as binary32; every codec op is "compute in binary32, round"
// which equals the dtype's own correctly rounded op for + - * / (24 >= 2p+2).
// ---------------------------------------------------------------------------
__device__ __forceinline__ float h2f(uint16_t h) {
  return (float)__builtin_bit_cast(_Float16, h);
}
__device__ __forceinline__ uint16_t f2h(float f) {
  return __builtin_bit_cast(uint16_t, (_Float16)f);
}
__device__ __forceinline__ float bf2f(uint16_t b) {
  return __uint_as_float((uint32_t)b << 16);
}
__device__ __forceinline__ uint16_t f2bf(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

template <int DT> struct Dt;
template <> struct Dt<CQ_F16> {
  using storage = uint16_t;
  static __device__ __forceinline__ float load(const void *p, int64_t i) {
    return h2f(((const uint16_t *)p)[i]);
  }
  static __device__ __forceinline__ float round(float x) { return h2f(f2h(x)); }
  static __device__ __forceinline__ void store(void *p, int64_t i, float x) {
    ((uint16_t *)p)[i] = f2h(x);
  }
};
template <> struct Dt<CQ_BF16> {
  using storage = uint16_t;
  static __device__ __forceinline__ float load(const void *p, int64_t i) {
    return bf2f(((const uint16_t *)p)[i]);
  }
  static __device__ __forceinline__ float round(float x) { return bf2f(f2bf(x)); }
  static __device__ __forceinline__ void store(void *p, int64_t i, float x) {
    ((uint16_t *)p)[i] = f2bf(x);
  }
};
template <> struct Dt<CQ_F32> {
  using storage = float;
  static __device__ __forceinline__ float load(const void *p, int64_t i) {
    return ((const float *)p)[i];
  }
  static __device__ __forceinline__ float round(float x) { return x; }
  static __device__ __forceinline__ void store(void *p, int64_t i, float x) {
    ((float *)p)[i] = x;
  }
};

__device__ __forceinline__ float load_any(int dt, const void *p, int64_t i) {
  if (dt == CQ_F16) return Dt<CQ_F16>::load(p, i);
  if (dt == CQ_BF16) return Dt<CQ_BF16>::load(p, i);
  return Dt<CQ_F32>::load(p, i);
}
__device__ __forceinline__ float round_any(int dt, float x) {
  if (dt == CQ_F16) return Dt<CQ_F16>::round(x);
  if (dt == CQ_BF16) return Dt<CQ_BF16>::round(x);
  return x;
}
__device__ __forceinline__ void store_any(int dt, void *p, int64_t i, float x) {
  if (dt == CQ_F16) Dt<CQ_F16>::store(p, i, x);
  else if (dt == CQ_BF16) Dt<CQ_BF16>::store(p, i, x);
  else Dt<CQ_F32>::store(p, i, x);
}

// ---------------------------------------------------------------------------
// Cross-lane reductions on DPP (gfx9 encodings).  After the four in-row steps
// every lane of a 16-lane row holds the row result; row_bcast15/31 then fold
// rows into lane 63, which readlane broadcasts to the wave (an SGPR value).
// ---------------------------------------------------------------------------
enum : int {
  kDppQuadXor1 = 0xB1,     // quad_perm [1,0,3,2]
  kDppQuadXor2 = 0x4E,     // quad_perm [2,3,0,1]
  kDppRowHalfMirror = 0x141,
  kDppRowMirror = 0x140,
  kDppRowBcast15 = 0x142,
  kDppRowBcast31 = 0x143,
  kDppRowRor4 = 0x124,  // row_ror:4 (rotate within the 16-lane row)
  kDppRowRor8 = 0x128,
};
// quad_perm [r,r,r,r]: every lane reads lane r of its quad
template <int R>
constexpr int kDppQuadBcast = 0x55 * R;

template <int CTRL, int ROW_MASK = 0xf>
__device__ __forceinline__ float dpp_f(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(
      __float_as_int(v), __float_as_int(v), CTRL, ROW_MASK, 0xf, false));
}
template <int CTRL, int ROW_MASK = 0xf>
__device__ __forceinline__ uint32_t dpp_u(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, CTRL, ROW_MASK,
                                                0xf, false);
}

// max(a, b) of non-NaN values as one instruction: fmaxf in IEEE mode first
// canonicalises every operand the compiler cannot prove canonical (values
// moved across lanes, converted halves), one extra VALU each; the IEEE
// 754-2019 maximum (NaN-propagating) needs no canonical operands and is one
// v_maximum3_f32 on gfx950.
__device__ __forceinline__ float max_nn(float a, float b) {
  return __builtin_elementwise_maximum(a, b);
}
__device__ __forceinline__ float wave_max(float v) {
  v = fmaxf(v, dpp_f<kDppQuadXor1>(v));
  v = fmaxf(v, dpp_f<kDppQuadXor2>(v));
  v = fmaxf(v, dpp_f<kDppRowHalfMirror>(v));
  v = fmaxf(v, dpp_f<kDppRowMirror>(v));
  v = fmaxf(v, dpp_f<kDppRowBcast15, 0xa>(v));
  v = fmaxf(v, dpp_f<kDppRowBcast31, 0xc>(v));
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

__device__ __forceinline__ float wave_sum(float v) {
  v += dpp_f<kDppQuadXor1>(v);
  v += dpp_f<kDppQuadXor2>(v);
  v += dpp_f<kDppRowHalfMirror>(v);
  v += dpp_f<kDppRowMirror>(v);
  v += dpp_f<kDppRowBcast15, 0xa>(v);
  v += dpp_f<kDppRowBcast31, 0xc>(v);
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

// Over the 16 lanes of a row (the first four steps of wave_max / wave_sum):
// every lane of the row gets the result, the sum with the same bits in
// every lane (each step adds a pair of values in either order).
__device__ __forceinline__ float row16_max(float v) {
  v = fmaxf(v, dpp_f<kDppQuadXor1>(v));
  v = fmaxf(v, dpp_f<kDppQuadXor2>(v));
  v = fmaxf(v, dpp_f<kDppRowHalfMirror>(v));
  return fmaxf(v, dpp_f<kDppRowMirror>(v));
}
__device__ __forceinline__ float row16_sum(float v) {
  v += dpp_f<kDppQuadXor1>(v);
  v += dpp_f<kDppQuadXor2>(v);
  v += dpp_f<kDppRowHalfMirror>(v);
  return v + dpp_f<kDppRowMirror>(v);
}
// Max over the 4 lanes of a row congruent to this lane mod 4.
__device__ __forceinline__ float row16_mod4_max(float v) {
  v = max_nn(v, dpp_f<kDppRowRor4>(v));
  return max_nn(v, dpp_f<kDppRowRor8>(v));
}
__device__ __forceinline__ float row16_mod4_sum(float v) {
  v += dpp_f<kDppRowRor4>(v);
  return v + dpp_f<kDppRowRor8>(v);
}

// max / sum of v and v of lane ^ 16 (lane ^ 32) without the LDS crossbar:
// gfx950 v_permlane16_swap (v_permlane32_swap) of v with itself gives every
// lane the values of its even and odd 16-lane row (lower and upper half), in
// that order, so both lanes of a pair compute the same bits.
__device__ __forceinline__ float xor16_max(float v) {
  const auto q = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return max_nn(__uint_as_float(q[0]), __uint_as_float(q[1]));
}
__device__ __forceinline__ float xor32_max(float v) {
  const auto q = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return max_nn(__uint_as_float(q[0]), __uint_as_float(q[1]));
}
__device__ __forceinline__ float xor16_sum(float v) {
  const auto q = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(q[0]) + __uint_as_float(q[1]);
}
__device__ __forceinline__ float xor32_sum(float v) {
  const auto q = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(q[0]) + __uint_as_float(q[1]);
}

// OR over aligned groups of N lanes (N = 2, 4 or 8), result in every lane.
template <int N>
__device__ __forceinline__ uint32_t group_or(uint32_t v) {
  v |= dpp_u<kDppQuadXor1>(v);
  if (N >= 4) v |= dpp_u<kDppQuadXor2>(v);
  if (N >= 8) v |= dpp_u<kDppRowHalfMirror>(v);
  return v;
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// threadIdx.x as a value the optimiser cannot hoist: inside a loop of a long
// kernel body, addresses derived from the thread index would otherwise be
// computed once before the loop and all stay live across the body.
__device__ __forceinline__ int thread_id() {
  int t = threadIdx.x;
  asm volatile("" : "+v"(t));
  return t;
}

constexpr float kLog2e = 1.4426950408889634f;

}  // namespace cq
