// cq_decode_mfma.hip — gfx950 MFMA split-K decode over the ChronoQuant cache
// (head_dim 128, fp16 queries, any GQA ratio in chunks of 16 q heads), and the
// same kernel's plain-fp16 mode used as the uncompressed flash-decode baseline.
//
// Reference semantics: the fused Metal kernel (kernels.py:79-228) — scores
// q'.(a + c*s) with q' = fp16(q*fp16(scale)), softmax, sum_t p_t (a + c*s).
// The contraction is factored so that both products are MFMA tiles:
//   score_t = q'.a_g(t) + s_t * (q'.c_t)
//   out     = sum_g P_g a_g + sum_t (p_t s_t) c_t,   P_g = sum_{t in g} p_t
// * q'.c_t: A = 16 tokens x 32 codes (nibbles made exact fp16 by a magic-number
//   OR), B = q'^T: v_mfma_f32_16x16x32_f16, exact products, fp32 sums.
//   q'.a_g: the same with 16 anchor rows as A; kept in a per-wave LDS table.
// * The score tile's output layout (lane = q head, 4 consecutive tokens) is
//   the A- and the B-operand layout of v_mfma_f32_16x16x16_f16, so:
//   - (p*s) against the V codes (nibbles as 1024+n or 1024+16n; the odd-nibble
//     tiles use p*s/16) gives sum (p s)(c + const), the constant removed at
//     the end with sum(p s);
//   - P_g^T = E^T p^T with E the 0/1 token->group matrix, accumulated per
//     64-token chunk, then P_g (as an fp16 hi/lo pair) against the V anchors.
//   All of it lands in one accumulator tile per 16 output dims.
// Softmax in the log2 domain with a lazy running max (rescale only when a
// tile's max exceeds it by more than 2^8), so weights stay <= 256 in fp16.
//
// Memory: each wave owns 64-token chunks of its split; every global load of a
// chunk (scales, K code rows, V code words, K/V anchor rows) is issued before
// the first wait.  Workgroups are 8 waves, so a split is 512 tokens.
//
// Plain mode (stride 1, no P-frames): every token is an anchor; the same
// anchor tiles compute q.k and p.V directly — a standard MFMA flash decode.
#include <hip/hip_runtime.h>
#include <math.h>

#include "cq_decode_common.h"

namespace cq {

typedef _Float16 h2_t __attribute__((ext_vector_type(2)));
typedef _Float16 h4_t __attribute__((ext_vector_type(4)));
typedef _Float16 h8_t __attribute__((ext_vector_type(8)));
typedef float f4_t __attribute__((ext_vector_type(4)));

constexpr int kHeads = 16;  // q heads per workgroup (MFMA tile width)
constexpr int kChunk = 64;  // tokens per wave iteration
constexpr int kD = 128;
constexpr int kWaves = kThreadsMfma / 64;
constexpr float kTau = 8.f;  // lazy-rescale threshold, log2 units

struct WaveScratch {
  float s_k[kChunk], s_v[kChunk];  // P-frame scales by token (0: I-frame / padding)
  float qa[kChunk][kHeads];        // q'.anchor_k by (chunk-local anchor, head)
};

struct MergeScratch {
  float m[kWaves][kHeads], l[kWaves][kHeads];
  float wm[kHeads], wl[kHeads];
  float o[kHeads][kD];
};

union DecodeLds {
  WaveScratch w[kWaves];
  MergeScratch mg;
  float combine[kCombineScratchFloats];
};

__device__ __forceinline__ h2_t as_h2(uint32_t u) { return __builtin_bit_cast(h2_t, u); }
__device__ __forceinline__ uint32_t and_or(uint32_t x, uint32_t m, uint32_t o) {
  return (x & m) | o;
}
__device__ __forceinline__ h4_t h4_of(uint32_t lo, uint32_t hi) {
  const h2_t a = as_h2(lo), b = as_h2(hi);
  return h4_t{a.x, a.y, b.x, b.y};
}

constexpr uint32_t kMagic = 0x64006400u;  // fp16 1024 in both halves

// One packed word (8 nibbles) -> the exact codes n-8 as fp16, in the K order
// {d0, d4, d1, d5, d2, d6, d3, d7} of the word's dims.
__device__ __forceinline__ h8_t unpack_codes8(uint32_t w) {
  const h2_t k1032 = {(_Float16)-1032.f, (_Float16)-1032.f};
  const h2_t k16th = {(_Float16)0.0625f, (_Float16)0.0625f};
  const h2_t k72 = {(_Float16)-72.f, (_Float16)-72.f};
  const uint32_t w8 = w >> 8;
  h2_t lo0 = as_h2(and_or(w, 0x000F000Fu, kMagic));   // 1024+n0, 1024+n4
  h2_t hi0 = as_h2(and_or(w, 0x00F000F0u, kMagic));   // 1024+16n1, 1024+16n5
  h2_t lo1 = as_h2(and_or(w8, 0x000F000Fu, kMagic));  // n2, n6
  h2_t hi1 = as_h2(and_or(w8, 0x00F000F0u, kMagic));  // n3, n7
  lo0 = lo0 + k1032;
  lo1 = lo1 + k1032;
  hi0 = __builtin_elementwise_fma(hi0, k16th, k72);
  hi1 = __builtin_elementwise_fma(hi1, k16th, k72);
  return h8_t{lo0.x, lo0.y, hi0.x, hi0.y, lo1.x, lo1.y, hi1.x, hi1.y};
}

__device__ __forceinline__ f4_t mfma32(h8_t a, h8_t b, f4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f4_t mfma16(h4_t a, h4_t b, f4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x16f16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// B operand (16x16x16) of anchor rows: lane holds 4 rows x dims 8c..8c+7 as
// av[r]; returns dims 8c + 2k (odd = false) or 8c + 2k + 1 (odd = true).
__device__ __forceinline__ h4_t anchor_operand(const uint4 (&av)[4], int k, bool odd) {
  const uint32_t sel = odd ? 0x07060302u : 0x05040100u;
  const uint32_t w0 = k == 0 ? av[0].x : k == 1 ? av[0].y : k == 2 ? av[0].z : av[0].w;
  const uint32_t w1 = k == 0 ? av[1].x : k == 1 ? av[1].y : k == 2 ? av[1].z : av[1].w;
  const uint32_t w2 = k == 0 ? av[2].x : k == 1 ? av[2].y : k == 2 ? av[2].z : av[2].w;
  const uint32_t w3 = k == 0 ? av[3].x : k == 1 ? av[3].y : k == 2 ? av[3].z : av[3].w;
  return h4_of(__builtin_amdgcn_perm(w1, w0, sel), __builtin_amdgcn_perm(w3, w2, sel));
}

template <bool kPlain>
__global__ __launch_bounds__(kThreadsMfma) void decode_mfma_kernel(DecodeArgs a) {
  __shared__ DecodeLds lds;
  const int split = blockIdx.x;
  const int h = blockIdx.y / a.n_chunks;
  const int chunk = blockIdx.y - h * a.n_chunks;
  const int b = blockIdx.z;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int col = lane & 15;  // q head (operand column) / 16-dim output column
  const int kg = lane >> 4;   // K group of the MFMA operands
  const int j0 = chunk * kHeads;
  const int gn = min(kHeads, a.G - j0);
  const int64_t bh = (int64_t)b * a.H + h;
  const int64_t T = seq_len_of(a, b);
  const int64_t t0 = (int64_t)split * a.split_len;
  const int64_t t1 = min(T, t0 + a.split_len);

  const uint16_t *__restrict__ kf_k = a.kf[0] + bh * a.cap_kf[0] * kD;
  const uint16_t *__restrict__ kf_v = a.kf[1] + bh * a.cap_kf[1] * kD;
  const uint32_t *__restrict__ pk_k = a.pk[0] + bh * a.cap_pf[0] * 16;
  const uint32_t *__restrict__ pk_v = a.pk[1] + bh * a.cap_pf[1] * 16;
  const uint16_t *__restrict__ sc_k = a.sc[0] + bh * a.cap_pf[0];
  const uint16_t *__restrict__ sc_v = a.sc[1] + bh * a.cap_pf[1];
  const int sk = a.stride[0], sv = a.stride[1];
  const float isk = a.inv_stride[0], isv = a.inv_stride[1];

  // q'^T operands (columns >= gn are zero): qn for anchor rows (dims
  // 32kb + 8kg + e), qc for code rows (dims 32kg + 8kb + {0,4,1,5,2,6,3,7}).
  // All loads are unconditional (clamped row) so none of them waits alone.
  h8_t qc[4], qn[4];
  {
    const bool qok = col < gn;
    const _Float16 sc16 = qok ? (_Float16)a.scale : (_Float16)0.f;  // 0 zeroes the column
    const uint16_t *qrow = (const uint16_t *)a.q +
                           ((int64_t)b * a.nq + h * a.G + j0 + (qok ? col : 0)) * kD;
    uint4 un[4], uc[4];
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
      un[kb] = *(const uint4 *)(qrow + 32 * kb + 8 * kg);
      uc[kb] = *(const uint4 *)(qrow + 32 * kg + 8 * kb);
    }
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
      qn[kb] = __builtin_bit_cast(h8_t, un[kb]) * sc16;  // fp16(q * fp16(scale))
      const h8_t v = __builtin_bit_cast(h8_t, uc[kb]) * sc16;
      qc[kb] = h8_t{v[0], v[4], v[1], v[5], v[2], v[6], v[3], v[7]};
    }
  }

  float m_run = -INFINITY;  // per head col, log2 units
  float l_run = 0.f;        // sum of fp16 p over this lane's tokens
  float w_run = 0.f;        // sum of fp16 p*s_v
  float w16_run = 0.f;      // sum of fp16 p*s_v/16
  f4_t acc[8];
#pragma unroll
  for (int nb = 0; nb < 8; ++nb) acc[nb] = f4_t{0.f, 0.f, 0.f, 0.f};

  WaveScratch &W = lds.w[wave];
  for (int64_t c0l = t0 + (int64_t)wave * kChunk; c0l < t1; c0l += kWaves * kChunk) {
    const int c0 = (int)c0l;
    const int nt = (int)min((int64_t)kChunk, t1 - c0l);

    // ---- issue every global load of the chunk --------------------------------
    // Addresses are clamped to valid rows and the values selected afterwards:
    // a load under a branch would be followed by its own wait.
    // per-token scalars, one token per lane
    const int tl = c0 + min(lane, nt - 1);
    int slk = -1, slv = -1;
    uint16_t rsk = 0, rsv = 0;
    if (!kPlain) {
      const int gk = div_stride(tl, sk, isk), gv = div_stride(tl, sv, isv);
      slk = (lane < nt && tl != gk * sk) ? tl - gk - 1 : -1;
      slv = (lane < nt && tl != gv * sv) ? tl - gv - 1 : -1;
      rsk = sc_k[max(slk, 0)];
      rsv = sc_v[max(slv, 0)];
    }
    const int gk_base = div_stride(c0, sk, isk);
    const int gk_last = div_stride(c0 + nt - 1, sk, isk);
    const int gv_base = div_stride(c0, sv, isv);
    const int gv_last = div_stride(c0 + nt - 1, sv, isv);
    // first K anchor tile: rows gk_base + col
    h8_t ka[4];
    {
      const int row = min(gk_base + col, gk_last);
      const uint16_t *p = kf_k + (int64_t)row * kD + 8 * kg;
#pragma unroll
      for (int kb = 0; kb < 4; ++kb) ka[kb] = *(const h8_t *)(p + 32 * kb);
    }
    // K code rows (token 16i + col, words 4kg..4kg+3) and V code words
    // (tokens 16i + 4kg + r, word col); slot -1 (I-frame, padding) reads slot 0
    uint4 kw[4];
    uint32_t vw[4][4];
    int kslot[4], vslot[4][4];
    if (!kPlain) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        kslot[i] = __shfl(slk, 16 * i + col, 64);
        kw[i] = *(const uint4 *)(pk_k + (int64_t)max(kslot[i], 0) * 16 + 4 * kg);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          vslot[i][r] = __shfl(slv, 16 * i + 4 * kg + r, 64);
          vw[i][r] = pk_v[(int64_t)max(vslot[i][r], 0) * 16 + col];
        }
      }
    }
    // first V anchor tile: rows gv_base + 4kg + r, dims 8col..8col+7
    uint4 va[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int vrow = min(gv_base + 4 * kg + r, gv_last);
      va[r] = *(const uint4 *)(kf_v + (int64_t)vrow * kD + 8 * col);
    }
    if (!kPlain) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        if (kslot[i] < 0) kw[i] = uint4{0u, 0u, 0u, 0u};
#pragma unroll
        for (int r = 0; r < 4; ++r)
          if (vslot[i][r] < 0) vw[i][r] = 0u;
      }
    }

    // ---- scales to LDS, q'.anchor_k table --------------------------------------
    if (!kPlain) {
      W.s_k[lane] = slk >= 0 ? h2f(rsk) : 0.f;
      W.s_v[lane] = slv >= 0 ? h2f(rsv) : 0.f;
    }
    const int nk_tiles = (gk_last - gk_base) / 16 + 1;
    for (int gt = 0; gt < nk_tiles; ++gt) {
      if (gt > 0) {
        const int row = min(gk_base + 16 * gt + col, gk_last);
        const uint16_t *p = kf_k + (int64_t)row * kD + 8 * kg;
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) ka[kb] = *(const h8_t *)(p + 32 * kb);
      }
      f4_t d = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kb = 0; kb < 4; ++kb) d = mfma32(ka[kb], qn[kb], d);
#pragma unroll
      for (int r = 0; r < 4; ++r) W.qa[16 * gt + 4 * kg + r][col] = d[r];  // d[r]: anchor 16gt+4kg+r
    }
    wave_lds_sync();

    // ---- per 16-token tile: scores, softmax weights, P.V ------------------------
    f4_t pg[4];  // P_g^T per 16-group V tile: lane holds groups 16gt+4kg+r, head col
#pragma unroll
    for (int gt = 0; gt < 4; ++gt) pg[gt] = f4_t{0.f, 0.f, 0.f, 0.f};
    const int nv_tiles = (gv_last - gv_base) / 16 + 1;

#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int tb = 16 * i + 4 * kg;  // this lane's 4 tokens: c0 + tb + r
      float sc[4];
      if (kPlain) {
        // anchors are the tokens: the q.k tile is the anchor tile i
#pragma unroll
        for (int r = 0; r < 4; ++r) sc[r] = W.qa[tb + r][col];
      } else {
        f4_t d = {0.f, 0.f, 0.f, 0.f};
        d = mfma32(unpack_codes8(kw[i].x), qc[0], d);
        d = mfma32(unpack_codes8(kw[i].y), qc[1], d);
        d = mfma32(unpack_codes8(kw[i].z), qc[2], d);
        d = mfma32(unpack_codes8(kw[i].w), qc[3], d);
        const float4 s4 = *(const float4 *)&W.s_k[tb];
        const float sr[4] = {s4.x, s4.y, s4.z, s4.w};
        int g = div_stride(c0 + tb, sk, isk);
        int rem = c0 + tb - g * sk;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          sc[r] = W.qa[g - gk_base][col] + sr[r] * d[r];
          if (++rem == sk) {
            rem = 0;
            ++g;
          }
        }
      }
#pragma unroll
      for (int r = 0; r < 4; ++r)
        sc[r] = (tb + r < nt && col < gn) ? sc[r] * kLog2e : -INFINITY;

      // lazy running max
      float mx = fmaxf(fmaxf(sc[0], sc[1]), fmaxf(sc[2], sc[3]));
      mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
      mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
      if (__any(mx > m_run + kTau)) {
        const float m_new = fmaxf(m_run, mx);
        const float f = (m_run == -INFINITY) ? 0.f : fast_exp2(m_run - m_new);
        l_run *= f;
        w_run *= f;
        w16_run *= f;
#pragma unroll
        for (int gt = 0; gt < 4; ++gt) pg[gt] *= f;  // layout [group][head col]
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float fr = __shfl(f, 4 * kg + r, 64);  // factor of head 4kg + r
#pragma unroll
          for (int nb = 0; nb < 8; ++nb) acc[nb][r] *= fr;
        }
        m_run = m_new;
      }

      // weights
      h4_t ap, aw, aw16;
      float svr[4] = {0.f, 0.f, 0.f, 0.f};
      if (!kPlain) {
        const float4 v4 = *(const float4 *)&W.s_v[tb];
        svr[0] = v4.x, svr[1] = v4.y, svr[2] = v4.z, svr[3] = v4.w;
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float p = (sc[r] == -INFINITY) ? 0.f : fast_exp2(sc[r] - m_run);
        const _Float16 ph = (_Float16)p;
        l_run += (float)ph;
        ap[r] = ph;
        if (!kPlain) {
          const _Float16 wh = (_Float16)((float)ph * svr[r]);
          const _Float16 wh16 = wh * (_Float16)0.0625f;
          w_run += (float)wh;
          w16_run += (float)wh16;
          aw[r] = wh;
          aw16[r] = wh16;
        }
      }

      if (kPlain) {
        // P.V over the 16 token rows of anchor tile i
        uint4 vv[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int vrow = min(c0 + tb + r, c0 + nt - 1);
          vv[r] = *(const uint4 *)(kf_v + (int64_t)vrow * kD + 8 * col);
        }
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          acc[2 * k] = mfma16(ap, anchor_operand(vv, k, false), acc[2 * k]);
          acc[2 * k + 1] = mfma16(ap, anchor_operand(vv, k, true), acc[2 * k + 1]);
        }
      } else {
        // codes: B = 4 tokens x dim 8col + nb (nibble nb of word col)
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const uint32_t sel =
              (uint32_t)k | (0x0cu << 8) | ((uint32_t)(4 + k) << 16) | (0x0cu << 24);
          const uint32_t p01 = __builtin_amdgcn_perm(vw[i][1], vw[i][0], sel);
          const uint32_t p23 = __builtin_amdgcn_perm(vw[i][3], vw[i][2], sel);
          const h4_t blo = h4_of(and_or(p01, 0x000F000Fu, kMagic), and_or(p23, 0x000F000Fu, kMagic));
          const h4_t bhi = h4_of(and_or(p01, 0x00F000F0u, kMagic), and_or(p23, 0x00F000F0u, kMagic));
          acc[2 * k] = mfma16(aw, blo, acc[2 * k]);
          acc[2 * k + 1] = mfma16(aw16, bhi, acc[2 * k + 1]);
        }
        // P_g^T += E^T p^T for the V group tiles this token tile touches
        int g = div_stride(c0 + tb, sv, isv);
        int rem = c0 + tb - g * sv;
        int gr[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          gr[r] = g - gv_base;
          if (++rem == sv) {
            rem = 0;
            ++g;
          }
        }
#pragma unroll
        for (int gt = 0; gt < 4; ++gt) {
          if (gt < nv_tiles) {
            h4_t e;
#pragma unroll
            for (int r = 0; r < 4; ++r) e[r] = (gr[r] == 16 * gt + col) ? (_Float16)1.f : (_Float16)0.f;
            pg[gt] = mfma16(e, ap, pg[gt]);
          }
        }
      }
    }

    // ---- anchor term: P_g against the V anchor rows ------------------------------
    if (!kPlain) {
      for (int gt = 0; gt < nv_tiles; ++gt) {
        if (gt > 0) {
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int vrow = min(gv_base + 16 * gt + 4 * kg + r, gv_last);
            va[r] = *(const uint4 *)(kf_v + (int64_t)vrow * kD + 8 * col);
          }
        }
        // P_g as an fp16 hi/lo pair: one rounding per group would be shared by
        // all of the group's tokens, so it is carried to ~22 bits instead
        h4_t pa, pl;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          pa[r] = (_Float16)pg[gt][r];
          pl[r] = (_Float16)(pg[gt][r] - (float)pa[r]);
        }
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const h4_t blo = anchor_operand(va, k, false), bhi = anchor_operand(va, k, true);
          acc[2 * k] = mfma16(pa, blo, acc[2 * k]);
          acc[2 * k] = mfma16(pl, blo, acc[2 * k]);
          acc[2 * k + 1] = mfma16(pa, bhi, acc[2 * k + 1]);
          acc[2 * k + 1] = mfma16(pl, bhi, acc[2 * k + 1]);
        }
      }
    }
    wave_lds_sync();
  }

  // ---- per-head totals and the workgroup merge ----------------------------------
  l_run += __shfl_xor(l_run, 16, 64);
  l_run += __shfl_xor(l_run, 32, 64);
  w_run += __shfl_xor(w_run, 16, 64);
  w_run += __shfl_xor(w_run, 32, 64);
  w16_run += __shfl_xor(w16_run, 16, 64);
  w16_run += __shfl_xor(w16_run, 32, 64);

  __syncthreads();  // wave scratch becomes the merge area
  MergeScratch &M = lds.mg;
  for (int e = tid; e < kHeads * kD; e += kThreadsMfma) (&M.o[0][0])[e] = 0.f;
  if (kg == 0) {
    M.m[wave][col] = m_run;
    M.l[wave][col] = l_run;
  }
  __syncthreads();
  if (tid < kHeads) {
    float mm = -INFINITY;
    for (int wv = 0; wv < kWaves; ++wv) mm = fmaxf(mm, M.m[wv][tid]);
    float L = 0.f;
    if (mm != -INFINITY)
      for (int wv = 0; wv < kWaves; ++wv)
        if (M.m[wv][tid] != -INFINITY) L += M.l[wv][tid] * fast_exp2(M.m[wv][tid] - mm);
    M.wm[tid] = mm;
    M.wl[tid] = L;
  }
  __syncthreads();
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int hh = 4 * kg + r;
    const float sw = __shfl(w_run, hh, 64);
    const float sw16 = __shfl(w16_run, hh, 64);
    const float mw = __shfl(m_run, hh, 64);
    if (hh < gn && mw != -INFINITY) {
      const float f = fast_exp2(mw - M.wm[hh]);
#pragma unroll
      for (int nb = 0; nb < 8; ++nb) {
        // code columns: x = 1032 + c (even nb, weight p s) or, for odd nb,
        // (1152 + 16c) with weight (p s)/16: subtract the constants
        const float corr = (nb & 1) ? 1024.f * sw16 + 8.f * sw : 1032.f * sw;
        const float v = kPlain ? acc[nb][r] : acc[nb][r] - corr;
        atomicAdd(&M.o[hh][8 * col + nb], v * f);
      }
    }
  }
  __syncthreads();
  finish_workgroup(a, b, h, chunk, j0, gn, split, M.wm, M.wl, &M.o[0][0], kD, lds.combine);
}

bool mfma_supported(const DecodeArgs &a) {
  if (a.D != kD || a.q_dtype != CQ_F16) return false;
  if (a.max_T >= (1 << 24)) return false;
  const uintptr_t al = (uintptr_t)a.kf[0] | (uintptr_t)a.kf[1] | (uintptr_t)a.pk[0] |
                       (uintptr_t)a.pk[1] | (uintptr_t)a.q;
  return (al & 15u) == 0;
}

int launch_decode_mfma(DecodeArgs &a, void *workspace, size_t ws_bytes, hipStream_t stream) {
  int st = prepare_launch(a, kHeads, workspace, ws_bytes);
  if (st) return st;
  const dim3 grid((unsigned)a.nsplit, (unsigned)(a.H * a.n_chunks), (unsigned)a.B);
  const bool plain = a.stride[0] == 1 && a.stride[1] == 1;
  if (plain)
    decode_mfma_kernel<true><<<grid, dim3(kThreadsMfma), 0, stream>>>(a);
  else
    decode_mfma_kernel<false><<<grid, dim3(kThreadsMfma), 0, stream>>>(a);
  return hipGetLastError() == hipSuccess ? CQ_OK : CQ_ERR_LAUNCH;
}

}  // namespace cq
