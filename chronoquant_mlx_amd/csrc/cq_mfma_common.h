// cq_mfma_common.h — pieces shared by the gfx950 MFMA decode kernels
// (cq_decode_mfma.hip: 16 q heads per tile; cq_decode_g4.hip: GQA groups of
// up to 4 q heads): operand types, cache-stream buffer loads, nibble and
// anchor operand builders for v_mfma_f32_16x16x32_f16, and the merge of a
// workgroup's 8 wave tiles followed by the split epilogue.
//
// v_mfma_f32_16x16x32_f16 lane layout (lane = 16 kg + c, c < 16, kg < 4):
//   A: lane holds A[row c][k = 8kg .. 8kg+7]     (8 fp16)
//   B: lane holds B[k = 8kg .. 8kg+7][col c]     (8 fp16)
//   C: lane holds C[row 4kg + r][col c], r < 4   (4 fp32)
#pragma once

#include <hip/hip_runtime.h>
#include <math.h>

#include "cq_decode_common.h"

namespace cq {

typedef _Float16 h2_t __attribute__((ext_vector_type(2)));
typedef _Float16 h4_t __attribute__((ext_vector_type(4)));
typedef _Float16 h8_t __attribute__((ext_vector_type(8)));
typedef float f4_t __attribute__((ext_vector_type(4)));
typedef int i4_t __attribute__((ext_vector_type(4)));

constexpr int kHeads = 16;  // q heads per MFMA tile column set
constexpr int kChunk = 64;  // tokens per wave iteration
constexpr int kD = 128;
constexpr int kWaves = kThreadsMfma / 64;
constexpr float kTau = 8.f;               // lazy-rescale threshold, log2 units
constexpr float kTwo24 = 16777216.f;      // 2^24

// ---------------------------------------------------------------------------
// small helpers
// ---------------------------------------------------------------------------
__device__ __forceinline__ h2_t as_h2(uint32_t u) { return __builtin_bit_cast(h2_t, u); }
__device__ __forceinline__ h4_t h4_of(uint32_t lo, uint32_t hi) {
  const h2_t a = as_h2(lo), b = as_h2(hi);
  return h4_t{a.x, a.y, b.x, b.y};
}
__device__ __forceinline__ h8_t h8_of(uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
  const h2_t x = as_h2(a), y = as_h2(b), z = as_h2(c), w = as_h2(d);
  return h8_t{x.x, x.y, y.x, y.y, z.x, z.y, w.x, w.y};
}

// bf16 queries: q' = bf16(q * bf16(scale)) (attention.py:46 in bf16: the
// fp32 product of two bf16 values is exact, so one round-to-nearest-even to
// bf16 gives the bf16 product), then converted to fp16 for the MFMA operand.
// The conversion is exact for |q'| in fp16's normal range (bf16 carries 8
// significant bits, fp16 11); below 2^-14 fp16 subnormals keep fewer bits.
__device__ __forceinline__ float bf16_round(float f) {
  uint32_t u = __float_as_uint(f);
  u += 0x7FFFu + ((u >> 16) & 1u);
  return __uint_as_float(u & 0xFFFF0000u);
}
__device__ __forceinline__ h8_t bf16x8_scaled_to_f16(uint4 raw, float scb) {
  const uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
  h8_t r;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    r[2 * i] = (_Float16)bf16_round(__uint_as_float(w[i] << 16) * scb);
    r[2 * i + 1] = (_Float16)bf16_round(__uint_as_float(w[i] & 0xFFFF0000u) * scb);
  }
  return r;
}

// (x & m) | o.  With o an opaque VGPR value (the magic below) the compiler
// emits one v_and_or_b32 (mask in an SGPR: gfx9 VOP3 reads at most one
// SGPR/literal).  The instruction itself must stay compiler-generated: the
// hazard recognizer does not count an inline-asm VALU write before an MFMA
// read, and such a write feeding v_mfma_f32_16x16x16_f16 gave wrong sums.
__device__ __forceinline__ uint32_t and_or(uint32_t x, uint32_t m, uint32_t o) {
  return (x & m) | o;
}

// Cache-stream loads: every cache byte is read once per decode, so they are
// non-temporal (cache policy nt) and do not evict the kernel's code, the
// argument block or the split partials from L2.
constexpr int kPolicyStream = 2;
__device__ __forceinline__ uint32_t bload32(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(r, (int)off, 0, kPolicyStream);
}
__device__ __forceinline__ uint4 bload128(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  const i4_t v = __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, kPolicyStream);
  return uint4{(uint32_t)v[0], (uint32_t)v[1], (uint32_t)v[2], (uint32_t)v[3]};
}
// the default cache policy (lines that a later load of the same wave reads again)
__device__ __forceinline__ uint4 bload128_cached(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  const i4_t v = __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 0);
  return uint4{(uint32_t)v[0], (uint32_t)v[1], (uint32_t)v[2], (uint32_t)v[3]};
}
__device__ __forceinline__ uint32_t bload16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(r, (int)off, 0, kPolicyStream);
}

__device__ __forceinline__ f4_t mfma32(h8_t a, h8_t b, f4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

__device__ __forceinline__ float shfl_max_kg(float v) {  // over the 4 lanes sharing lane&15
  return xor32_max(xor16_max(v));
}
__device__ __forceinline__ float shfl_sum_kg(float v) { return xor32_sum(xor16_sum(v)); }

// K code word (8 nibbles) -> A operand: n * 2^-24 as fp16 denormals in the K
// order {d0, d4, d1, d5, d2, d6, d3, d7} of the word's dims.
__device__ __forceinline__ h8_t unpack_k(uint32_t w) {
  const uint32_t m = 0x000F000Fu;
  return h8_of(w & m, (w >> 4) & m, (w >> 8) & m, (w >> 12) & m);
}

// 8 fp16 values (natural order d0..d7 in 4 dwords) -> the K order above.
__device__ __forceinline__ h8_t korder(uint4 u) {
  return h8_of(__builtin_amdgcn_perm(u.z, u.x, 0x05040100u),
               __builtin_amdgcn_perm(u.z, u.x, 0x07060302u),
               __builtin_amdgcn_perm(u.w, u.y, 0x05040100u),
               __builtin_amdgcn_perm(u.w, u.y, 0x07060302u));
}

// B operand (16x16x16) from 4 fp16 rows r (lane holds dims 8c..8c+7 of each
// as u[r]): the values of dim 8c + 2k (odd = false) or 8c + 2k + 1 (odd).
__device__ __forceinline__ h4_t rows_operand(const uint4 (&u)[4], int k, bool odd) {
  const uint32_t sel = odd ? 0x07060302u : 0x05040100u;
  const uint32_t w0 = k == 0 ? u[0].x : k == 1 ? u[0].y : k == 2 ? u[0].z : u[0].w;
  const uint32_t w1 = k == 0 ? u[1].x : k == 1 ? u[1].y : k == 2 ? u[1].z : u[1].w;
  const uint32_t w2 = k == 0 ? u[2].x : k == 1 ? u[2].y : k == 2 ? u[2].z : u[2].w;
  const uint32_t w3 = k == 0 ? u[3].x : k == 1 ? u[3].y : k == 2 ? u[3].z : u[3].w;
  return h4_of(__builtin_amdgcn_perm(w1, w0, sel), __builtin_amdgcn_perm(w3, w2, sel));
}

constexpr int kMergeHeads = 8;  // q heads per merge pass

struct MergeScratch {
  float t[kWaves][kMergeHeads][kD];  // each wave's unnormalised output tile
  float m[kWaves][kHeads], l[kWaves][kHeads];
  float wm[kHeads], wl[kHeads];
  float o[kHeads][kD];
};

// Merge the 8 waves' (m, l, o) through LDS and run the split epilogue.
// o_val(nb, r) is this lane's unnormalised output for head 4kg+r, dim 8col+nb.
// Each wave stores its tile with 16-byte writes (lane col owns dims
// 8col..8col+7 of its 4 heads); after one barrier every thread sums the 8
// tiles of (head, 4 dims) with the log-sum-exp weights, reading the 8 waves'
// running maxima itself.  Up to kMergeHeads heads per pass.
template <typename OVal>
__device__ __forceinline__ void merge_and_finish(const DecodeArgs &a, MergeScratch &M, int b,
                                                 int h, int chunk, int j0, int gn, int slot,
                                                 int live, float m_run, float l_run, OVal o_val) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int col = lane & 15, kg = lane >> 4;
  __syncthreads();  // wave scratch becomes the merge area
  if (kg == 0) {
    M.m[wave][col] = m_run;
    M.l[wave][col] = l_run;
  }
  for (int p0 = 0; p0 < gn; p0 += kMergeHeads) {
    const int pn = min(kMergeHeads, gn - p0);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int hp = 4 * kg + r - p0;
      if (hp >= 0 && hp < pn) {
        float4 *dst = (float4 *)&M.t[wave][hp][8 * col];
        dst[0] = make_float4(o_val(0, r), o_val(1, r), o_val(2, r), o_val(3, r));
        dst[1] = make_float4(o_val(4, r), o_val(5, r), o_val(6, r), o_val(7, r));
      }
    }
    __syncthreads();
    for (int e = tid; e < pn * (kD / 4); e += kThreadsMfma) {
      const int hp = e / (kD / 4), d0 = 4 * (e - hp * (kD / 4));
      const int hh = p0 + hp;
      float mw[kWaves], mm = -INFINITY;
#pragma unroll
      for (int w = 0; w < kWaves; ++w) {
        mw[w] = M.m[w][hh];
        mm = fmaxf(mm, mw[w]);
      }
      float4 o = make_float4(0.f, 0.f, 0.f, 0.f);
      float L = 0.f;
#pragma unroll
      for (int w = 0; w < kWaves; ++w) {
        const float f = (mw[w] == -INFINITY) ? 0.f : fast_exp2(mw[w] - mm);
        const float4 t = *(const float4 *)&M.t[w][hp][d0];
        o.x += f * t.x;
        o.y += f * t.y;
        o.z += f * t.z;
        o.w += f * t.w;
        L += f * M.l[w][hh];
      }
      *(float4 *)&M.o[hh][d0] = o;
      if (d0 == 0) {
        M.wm[hh] = mm;
        M.wl[hh] = L;
      }
    }
    __syncthreads();
  }
  finish_workgroup(a, b, h, chunk, j0, gn, slot, live, M.wm, M.wl, &M.o[0][0], kD);
}

}  // namespace cq
