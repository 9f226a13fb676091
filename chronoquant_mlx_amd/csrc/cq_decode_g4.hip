// cq_decode_g4.hip — gfx950 MFMA split-K decode over the ChronoQuant cache for
// GQA groups of at most 4 q heads per kv head (head_dim 128, fp16 or bf16
// queries, power-of-two strides >= 4): the shape of every benchmark
// configuration (32 q / 8 kv heads).
//
// Reference semantics: the fused Metal kernel (kernels.py:79-228), with the
// factoring of the 16-head kernel (cq_decode_mfma.hip):
//   score_t = q'.a_g(t) + s_t * (q'.c_t)
//   out     = sum_g P_g a_g + sum_t (p_t s_t) c_t,   P_g = sum_{t in g} p_t
//
// What differs is the layout of the score product.  With 4 q heads a 16-column
// head tile leaves 12 columns idle, and every per-score instruction after the
// product (scale, anchor term, softmax, weights) would run 4 times over.  Here
// the 16 columns are (token block j, head h), j, h < 4, and the 32-deep K index
// of v_mfma_f32_16x16x32_f16 is (token block j', 8 dims of slab m):
//   A[i][(j', e)]       = code nibble of token 16 j' + i, dim e of slab m
//   B[(j', e)][(j, h)]  = q'_h of that dim if j == j', else 0
//   C[i][(j, h)]       += q'_h . c over slab m of token 16 j + i
// Lane 16 kg + i supplies the codes of token 16 kg + i (its own 64-byte row,
// one 32-bit word per slab) and receives the 4 scores of tokens 16 j + 4 kg + r
// (r < 4) of head h, (j, h) its column: every score is used once.  B is read
// from the workgroup's q table in LDS, whose zero half supplies the off-block
// entries.  Codes enter as fp16 denormals n * 2^-24 (exact in the product).
//
// The products over V keep the 16-row head tile of the 16-head kernel (rows
// = heads, 4 used): p, p*s_v and p*s_v/16 move from the score layout to that
// operand layout through a per-wave LDS table, and the V code, P_g and anchor
// products, the lazy running max and the merge are the 16-head kernel's.
#include <hip/hip_runtime.h>
#include <math.h>

#include <algorithm>

#include "cq_mfma_common.h"

namespace cq {

namespace {

constexpr int kG4 = 4;  // q heads per kv head this kernel serves

// Code rows of the chunk being computed, by token (row kChunk: junk), rows
// padded to 20 words so that 16 consecutive rows start on distinct 4-bank
// groups: the pipelined and balanced instances load a chunk's P-frame rows
// as contiguous blocks and scatter them here to their tokens.
constexpr int kRowWords = 20;
struct alignas(16) G4Rows {
  uint32_t k[kChunk + 1][kRowWords];
  uint32_t v[kChunk + 1][kRowWords];
};

template <bool kContig>
struct G4WaveRows {};
template <>
struct G4WaveRows<true> {
  G4Rows rows;
};

// Per-wave LDS.  s16 is double-buffered (the chunk being computed and the one
// whose loads are in flight).
template <bool kContig>
struct alignas(16) G4WaveScratch : G4WaveRows<kContig> {
  int slot_v[kChunk];            // V P-frame slot per token (-1: I-frame / padding)
  uint32_t s16[2][kChunk];       // fp16 K scale | fp16 V scale << 16 (0: none)
  float qa[16][kG4];             // log2e * q'.anchor_k - mref by (local anchor, head)
  // p, p*s_v, p*s_v/16 (fp16) by (head, 4-token group); rows padded to 34
  // dwords so the 4 heads of a 4-token group fall in different banks
  uint2 pw[3][kG4][kChunk / 4 + 1];
};

// Per-workgroup LDS: q' of the group's heads in the order of the score
// product's K operand (q[8 par + p][h]: the dims of parity par of slabs 2p and
// 2p + 1, see unpack_pair), and the zero region the score product's off-block
// lanes read.
struct alignas(16) G4GroupScratch {
  h8_t q[16][kG4];
  h8_t qn[16][kG4];  // q' of head h, dims 8m .. 8m + 7 (natural order): the anchor product's B
  h8_t pad[kG4];  // puts zero[m][h] 64 bytes off q[m][h]'s banks
  h8_t zero[16][kG4];
  float s8[kG4];  // 8 * sum_d q'_d per head
};

template <bool kContig>
struct G4Stage {
  G4GroupScratch g;
  G4WaveScratch<kContig> w[kWaves];
};

// The workgroup merge: every wave's unnormalised output tile and its (m, l)
// per head, heads-major so that a thread reads the 8 waves' values of one
// head as two 16-byte words.
struct alignas(16) G4Merge {
  float t[kWaves][kG4][kD];
  float m[kG4][kWaves], l[kG4][kWaves];
};

// The merge area is separate from the staging area, so a wave writes its
// tile as soon as its own chunks are done.
template <bool kContig>
struct G4Lds {
  G4Stage<kContig> s;
  G4Merge mg;
};

// The last workgroup's fold of the `live` partials: thread (unit u, slice
// sl) = (tid / 4, tid % 4) owns head u / 32, dims 4 (u % 32) .. +3, and
// splits sl, sl + 4, ...; all of its loads ((m, l) pairs and 16-byte partial
// vectors, kCombineBatch splits at a time) are in flight together, and the
// 4 slices of a unit, adjacent lanes, fold with DPP quad permutes.
__device__ __forceinline__ void merge_partials_g4(const DecodeArgs &a, __amdgpu_buffer_rsrc_t racc,
                                                  __amdgpu_buffer_rsrc_t rml, int64_t bq0, int gn,
                                                  int nsplit) {
  constexpr int kSlices = 4;
  static_assert(kThreadsMfma == kSlices * kG4 * (kD / 4), "one thread per (head, 4 dims, slice)");
  const int tid = threadIdx.x;
  const int u = tid >> 2, sl = tid & (kSlices - 1);
  const int j = u >> 5, d0 = 4 * (u & 31);
  const bool live_unit = j < gn;
  const uint32_t row0 = (uint32_t)((bq0 + (live_unit ? j : 0)) * a.nsplit);
  float M = -INFINITY, L = 0.f;
  float o[4] = {0.f, 0.f, 0.f, 0.f};
  for (int sp0 = sl; sp0 < nsplit; sp0 += kCombineBatch * kSlices) {
    f2v_t ml[kCombineBatch];
    f4v_t ov[kCombineBatch];
#pragma unroll
    for (int k = 0; k < kCombineBatch; ++k) {
      // splits past the end re-read the last live split and are masked below
      const uint32_t spo = row0 + (uint32_t)min(sp0 + k * kSlices, nsplit - 1);
      ml[k] = load_dev2(rml, spo * 8u);
      ov[k] = load_dev4(racc, (spo * (uint32_t)kD + (uint32_t)d0) * 4u);
    }
    float mb = M;
#pragma unroll
    for (int k = 0; k < kCombineBatch; ++k) {
      if (sp0 + k * kSlices >= nsplit) ml[k].x = -INFINITY;
      mb = fmaxf(mb, ml[k].x);
    }
    const float mref = (mb == -INFINITY) ? 0.f : mb;
    const float f = (M == -INFINITY) ? 0.f : fast_exp2(M - mref);
    L *= f;
#pragma unroll
    for (int c = 0; c < 4; ++c) o[c] *= f;
#pragma unroll
    for (int k = 0; k < kCombineBatch; ++k) {
      const float w = (ml[k].x == -INFINITY) ? 0.f : fast_exp2(ml[k].x - mref);
      L += w * ml[k].y;
      o[0] += w * ov[k].x;
      o[1] += w * ov[k].y;
      o[2] += w * ov[k].z;
      o[3] += w * ov[k].w;
    }
    M = mb;
  }
  // the unit's 4 slices (lanes 4u .. 4u + 3)
  float Mx = fmaxf(M, dpp_f<kDppQuadXor1>(M));
  Mx = fmaxf(Mx, dpp_f<kDppQuadXor2>(Mx));
  const float f = (M == -INFINITY) ? 0.f : fast_exp2(M - Mx);
  L *= f;
#pragma unroll
  for (int c = 0; c < 4; ++c) o[c] *= f;
  L += dpp_f<kDppQuadXor1>(L);
  L += dpp_f<kDppQuadXor2>(L);
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    o[c] += dpp_f<kDppQuadXor1>(o[c]);
    o[c] += dpp_f<kDppQuadXor2>(o[c]);
  }
  if (live_unit && sl == 0) {
    const float inv = L > 0.f ? 1.f / L : 0.f;
    const int64_t oi = (bq0 + j) * kD + d0;
    if (a.out_dtype == CQ_F16) {
      const h2v_t lo = h2v_t{(_Float16)(o[0] * inv), (_Float16)(o[1] * inv)};
      const h2v_t hi = h2v_t{(_Float16)(o[2] * inv), (_Float16)(o[3] * inv)};
      *(uint2 *)((uint16_t *)a.out + oi) =
          uint2{__builtin_bit_cast(uint32_t, lo), __builtin_bit_cast(uint32_t, hi)};
    } else {
#pragma unroll
      for (int c = 0; c < 4; ++c) store_any(a.out_dtype, a.out, oi + c, o[c] * inv);
    }
  }
}

// ---------------------------------------------------------------------------
// Fold records (grid plan, when its workgroups are one resident generation):
// every live split stores its partial as records of 12 words per (head, 8
// dims) unit (m, l, 2 unused, 8 outputs), each word the bit pattern + 1 (a
// zero word is "not written"; only the NaN pattern 0xffffffff maps to zero,
// and a record holding it is folded when the poll bound runs out).  Split f
// then folds the units u = f, f + live, f + 2 live, ...: each record is read
// by exactly one folder, which polls it until all ten words are non-zero,
// folds and writes the outputs, and stores zeros over it.  Data and readiness
// arrive in one round trip; no flag, no counter, no acknowledgement wait.
// ---------------------------------------------------------------------------
__device__ __forceinline__ uint4 load_rec4(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  const i4_t v = __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, kPolicyDevice);
  return uint4{(uint32_t)v[0], (uint32_t)v[1], (uint32_t)v[2], (uint32_t)v[3]};
}
__device__ __forceinline__ void store_rec1(__amdgpu_buffer_rsrc_t r, uint32_t off, float v) {
  __builtin_amdgcn_raw_buffer_store_b32((int)(__float_as_uint(v) + 1u), r, (int)off, 0, kPolicyDevice);
}
__device__ __forceinline__ float rec_value(uint32_t w) { return __uint_as_float(w - 1u); }

// max / sum over aligned groups of 2^lg lanes (lg <= 6, wave-uniform)
__device__ __forceinline__ float group_max(float v, int lg) {
  if (lg > 0) v = fmaxf(v, dpp_f<kDppQuadXor1>(v));
  if (lg > 1) v = fmaxf(v, dpp_f<kDppQuadXor2>(v));
  if (lg > 2) v = fmaxf(v, dpp_f<kDppRowHalfMirror>(v));
  if (lg > 3) v = fmaxf(v, dpp_f<kDppRowMirror>(v));
  if (lg > 4) v = fmaxf(v, __shfl_xor(v, 16, 64));
  if (lg > 5) v = fmaxf(v, __shfl_xor(v, 32, 64));
  return v;
}
__device__ __forceinline__ float group_sum(float v, int lg) {
  if (lg > 0) v += dpp_f<kDppQuadXor1>(v);
  if (lg > 1) v += dpp_f<kDppQuadXor2>(v);
  if (lg > 2) v += dpp_f<kDppRowHalfMirror>(v);
  if (lg > 3) v += dpp_f<kDppRowMirror>(v);
  if (lg > 4) v += __shfl_xor(v, 16, 64);
  if (lg > 5) v += __shfl_xor(v, 32, 64);
  return v;
}

// A split wait that ran out of poll rounds: set the workspace's sticky
// status (the fold goes ahead with what it has; cq_decode_status reports the
// event to the host and clears the zero region).  Lane 0 of the waiting wave.
__device__ __forceinline__ void note_poll_timeout(const DecodeArgs &a) {
  if ((threadIdx.x & 63) == 0)
    __hip_atomic_fetch_or(a.status, kStatusFoldTimeout, __ATOMIC_RELAXED,
                          __HIP_MEMORY_SCOPE_AGENT);
}

// Wave 0 of split f's workgroup folds its units; lane = (unit k of the pass,
// split s), 2^lg >= live lanes per unit.
__device__ __forceinline__ void fold_records_g4(const DecodeArgs &a, int b, int h, int gn, int f,
                                                int live) {
  if (threadIdx.x >= 64) return;
  const int lane = threadIdx.x;
  const int lg = live > 1 ? 32 - __builtin_clz((uint32_t)(live - 1)) : 0;
  const int s = lane & ((1 << lg) - 1), k = lane >> lg;
  const int per_pass = 64 >> lg;
  const int nunits = kD / 8 * gn;
  const __amdgpu_buffer_rsrc_t rr = make_rsrc(a.recs, (uint32_t)kRecBytes);
  const int64_t col = (int64_t)b * a.H + h;
  for (int j0 = 0; f + live * j0 < nunits; j0 += per_pass) {
    const int u = f + live * (j0 + k);
    const bool valid = s < live && u < nunits;
    const uint32_t off =
        (uint32_t)(((col * a.nsplit + s) * kRecUnits + (valid ? u : 0)) * (kRecWords * 4));
    uint4 hv = uint4{0u, 0u, 0u, 0u}, o0 = hv, o1 = hv;
    int round = 0;
    for (; round < a.poll_rounds; ++round) {
      if (valid) {
        hv = load_rec4(rr, off);
        o0 = load_rec4(rr, off + 16u);
        o1 = load_rec4(rr, off + 32u);
      }
      const bool ok = !valid || (hv.x && hv.y && o0.x && o0.y && o0.z && o0.w && o1.x && o1.y &&
                                 o1.z && o1.w);
      if (__all(ok)) break;
      __builtin_amdgcn_s_sleep(1);
    }
    if (round == a.poll_rounds) note_poll_timeout(a);
    const float m = valid ? rec_value(hv.x) : -INFINITY;
    const float M = group_max(m, lg);
    const float w = (m == -INFINITY) ? 0.f : fast_exp2(m - M);
    const float L = group_sum(valid ? w * rec_value(hv.y) : 0.f, lg);
    const uint32_t ow[8] = {o0.x, o0.y, o0.z, o0.w, o1.x, o1.y, o1.z, o1.w};
    float o[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = group_sum(valid ? w * rec_value(ow[e]) : 0.f, lg);
    if (valid) {
      const i4_t z = i4_t{0, 0, 0, 0};
      __builtin_amdgcn_raw_buffer_store_b128(z, rr, (int)off, 0, kPolicyDevice);
      __builtin_amdgcn_raw_buffer_store_b128(z, rr, (int)off + 16, 0, kPolicyDevice);
      __builtin_amdgcn_raw_buffer_store_b128(z, rr, (int)off + 32, 0, kPolicyDevice);
      if (s == 0) {
        const float inv = L > 0.f ? 1.f / L : 0.f;
        const int64_t oi = ((int64_t)b * a.nq + h * a.G + (u >> 4)) * kD + 8 * (u & 15);
        if (a.out_dtype == CQ_F16) {
          h2v_t hp[4];
#pragma unroll
          for (int e = 0; e < 4; ++e)
            hp[e] = h2v_t{(_Float16)(o[2 * e] * inv), (_Float16)(o[2 * e + 1] * inv)};
          *(uint4 *)((uint16_t *)a.out + oi) =
              uint4{__builtin_bit_cast(uint32_t, hp[0]), __builtin_bit_cast(uint32_t, hp[1]),
                    __builtin_bit_cast(uint32_t, hp[2]), __builtin_bit_cast(uint32_t, hp[3])};
        } else {
#pragma unroll
          for (int e = 0; e < 8; ++e) store_any(a.out_dtype, a.out, oi + e, o[e] * inv);
        }
      }
    }
  }
}

// Slot 0's wait for the split-ready flags fl[1 .. live-1]: wave 0 polls them
// with device-scope loads (one per lane per round) until every flag is set,
// sleeping between rounds; the other waves wait at the barrier.  The other
// splits of the sequence are running workgroups of the same grid (the plans
// launch one resident generation) that publish their partials without
// waiting on anything, so the wait ends; a.poll_rounds bounds it regardless
// (and a wait that runs out sets the workspace's sticky status).
__device__ __forceinline__ void wait_split_flags(const DecodeArgs &a, const uint32_t *fl,
                                                 int live) {
  if (threadIdx.x < 64) {
    const int lane = threadIdx.x;
    int round = 0;
    for (; round < a.poll_rounds; ++round) {
      bool ready = true;
      for (int sp = 1 + lane; sp < live; sp += 64)
        ready = ready && __hip_atomic_load(const_cast<uint32_t *>(fl) + sp, __ATOMIC_RELAXED,
                                           __HIP_MEMORY_SCOPE_AGENT) != 0u;
      if (__all(ready)) break;
      __builtin_amdgcn_s_sleep(1);
    }
    if (round == a.poll_rounds) note_poll_timeout(a);
  }
  __syncthreads();
}

// The workgroup merge and the split epilogue.  Lanes 0..15 of each wave hold
// the wave's unnormalised output of heads r < gn, dims 8 col .. 8 col + 7
// (o_val(nb, r)), and lanes col < 4 of them the running max and weight sum
// of head col.  After one barrier each of the 512 threads folds one (head,
// dim) element over the 8 waves with the log-sum-exp weights, then writes
// the output (the workgroup holds the whole sequence) or stores its split
// partial from registers and runs the split tail.
template <typename OVal>
__device__ __forceinline__ void merge_finish_g4(const DecodeArgs &a, G4Merge &M, int b, int h,
                                                int gn, int slot, int live, float m_run,
                                                float l_run, OVal o_val) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int col = lane & 15, kg = lane >> 4;
  if (kg == 0) {
#pragma unroll
    for (int r = 0; r < kG4; ++r) {
      if (r < gn) {
        float4 *dst = (float4 *)&M.t[wave][r][8 * col];
        dst[0] = make_float4(o_val(0, r), o_val(1, r), o_val(2, r), o_val(3, r));
        dst[1] = make_float4(o_val(4, r), o_val(5, r), o_val(6, r), o_val(7, r));
      }
    }
    if (col < kG4) {
      M.m[col][wave] = m_run;
      M.l[col][wave] = l_run;
    }
  }
  __syncthreads();
  static_assert(kThreadsMfma == kG4 * kD, "one thread per (head, dim) of the merge");
  const int hh = tid >> 7, d = tid & (kD - 1);
  const int64_t bq0 = (int64_t)b * a.nq + h * a.G;
  const bool single = live == kGridLive ? a.nsplit == 1 : live == 1;
  __amdgpu_buffer_rsrc_t racc, rml;
  if (!single && !a.recs) partial_rsrcs(a, racc, rml);
  if (hh < gn) {
    const float4 m0 = *(const float4 *)&M.m[hh][0], m1 = *(const float4 *)&M.m[hh][4];
    const float4 l0 = *(const float4 *)&M.l[hh][0], l1 = *(const float4 *)&M.l[hh][4];
    const float mw[kWaves] = {m0.x, m0.y, m0.z, m0.w, m1.x, m1.y, m1.z, m1.w};
    const float lw[kWaves] = {l0.x, l0.y, l0.z, l0.w, l1.x, l1.y, l1.z, l1.w};
    float mm = -INFINITY;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) mm = fmaxf(mm, mw[w]);
    float O = 0.f, L = 0.f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
      const float f = (mw[w] == -INFINITY) ? 0.f : fast_exp2(mw[w] - mm);
      O += f * M.t[w][hh][d];
      L += f * lw[w];
    }
    if (single) {
      store_any(a.out_dtype, a.out, (bq0 + hh) * kD + d, L > 0.f ? O / L : 0.f);
    } else if (a.recs) {
      const __amdgpu_buffer_rsrc_t rr = make_rsrc(a.recs, (uint32_t)kRecBytes);
      const uint32_t rec = (uint32_t)(((((int64_t)b * a.H + h) * a.nsplit + slot) * kRecUnits +
                                       hh * (kD / 8) + (d >> 3)) * (kRecWords * 4));
      store_rec1(rr, rec + 16u + 4u * (uint32_t)(d & 7), O);
      if ((d & 7) == 0) {
        store_rec1(rr, rec, mm);
        store_rec1(rr, rec + 4u, L);
      }
    } else {
      const uint32_t row = (uint32_t)((bq0 + hh) * a.nsplit + slot);
      store_dev1(racc, (row * (uint32_t)kD + (uint32_t)d) * 4u, O);
      if (d == 0) store_dev2(rml, row * 8u, f2v_t{mm, L});
    }
  }
  if (single) return;
  if (live == kGridLive) live = grid_live(a, seq_len_of(a, b));
  if (a.recs) {
    phase_mark(a, 4);  // records stored (issued)
    fold_records_g4(a, b, h, gn, slot, live);
    phase_mark(a, 5);  // fold done, outputs stored (issued)
    return;
  }
  if (a.flags) {
    // Split-ready flags: every split but slot 0 publishes its partial and
    // sets its flag; slot 0 waits for the flags and folds.  No atomics, so
    // the splits of a sequence do not queue on one counter (their tickets
    // arrive within about a microsecond of each other and serialise).
    uint32_t *fl = a.flags + ((int64_t)b * a.H + h) * a.nsplit;
    __builtin_amdgcn_s_waitcnt(0);  // this thread's partial stores are complete
    __syncthreads();
    if (slot != 0) {
      if (tid == 0) __hip_atomic_store(fl + slot, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      return;
    }
    wait_split_flags(a, fl, live);
    merge_partials_g4(a, racc, rml, bq0, gn, live);
    for (int sp = 1 + tid; sp < live; sp += kThreadsMfma)
      __hip_atomic_store(fl + sp, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return;
  }
  uint32_t *ctr;
  if (!split_ticket(a, b, h, 0, live, ctr)) return;
  merge_partials_g4(a, racc, rml, bq0, gn, live);
  reset_ticket(ctr);
}

// K operand of the score product from two code words (slabs 2p, 2p + 1).  A
// nibble enters as an fp16 denormal: bits 0-3 and 4-7 of each 16-bit half
// are read in place (n * 2^-24 and 16 n * 2^-24), bits 8-15 after one shift
// by 8.  Parity 0 takes the low nibble of each byte, dims {0, 4, 2, 6} of a
// slab in that order; parity 1 the high nibble, dims {1, 5, 3, 7} at 16 times
// their value (the product's accumulator is scaled by 1/16).  Five VALU per
// word for both parities.
__device__ __forceinline__ h8_t unpack_pair(uint32_t wa, uint32_t wb, uint32_t ta, uint32_t tb,
                                           uint32_t m) {
  return h8_of(wa & m, ta & m, wb & m, tb & m);
}

// The registers one chunk's loads land in.  kr and vw first hold the chunk's
// contiguous K and V code blocks (16 bytes of slot row base + 16q + lane / 4,
// quarter lane % 4, per register), then, once scattered through LDS, the
// layouts the products read:
struct G4Buf {
  uint4 kr[4];        // K code row of this lane's token (words 4q .. 4q+3 in kr[q])
  uint4 ka[4];        // K anchor row gk_base + col, dims 32kg + 8kb .. +7
  uint32_t vw[4][4];  // V code word col of token 16i + 4kg + r
  uint32_t sk, sv;    // this lane's token's fp16 K and V scales (0: none)
  int c0, nt;         // chunk start, valid tokens (0: nothing to compute)
};

}  // namespace

// kBalanced = false: grid plan, workgroup (split, kv head, sequence) takes
// tokens [split * split_len, +split_len) of one sequence (uniform batches,
// where it is as balanced as the partition below).  kBalanced = true: the
// balanced partition of the batch's units (cq_plan.h), one or more segments
// per workgroup.
//
// kDenseV: the V rows are dense 3-bit rows (48 bytes: dim d's field code + 4
// at stream bits 3d .. 3d + 2), see the V code products below.
template <bool kBalanced, bool kOneChunk = false, bool kDenseV = false>
__global__ __launch_bounds__(kThreadsMfma) void decode_g4_kernel(DecodeArgs a) {
  static_assert(!(kBalanced && kOneChunk), "one-chunk splits are a grid plan");
  static_assert(!(kDenseV && kOneChunk), "dense V rows take the block-load instances");
  // bytes of a V P-frame row, and its 1 KB blocks per 64-row chunk
  constexpr uint32_t kVRow = kDenseV ? 48u : 64u;
  constexpr int kVBlocks = kDenseV ? 3 : 4;
  // Code loads: contiguous blocks scattered through LDS (the chunk loops of
  // the pipelined and balanced instances, where they are off the critical
  // path), or each lane's own token rows (one-chunk splits, whose single
  // chunk would wait for the LDS round trip).
  constexpr bool kContig = !kOneChunk;
  __shared__ G4Lds<kContig> lds;
  __shared__ int32_t s_units[kBalanced ? kMaxTableSeqs + 1 : 1];
  // Balanced plan: workgroup p of the column takes units [floor(pU/P),
  // floor((p+1)U/P)) of the batch's units laid end to end, one segment per
  // sequence it touches.  Per-sequence lengths give the unit table;
  // otherwise every sequence has the units of the length bound.
  //
  // The loop state stays in LDS while a segment runs and is read back after
  // it (the cursor double-buffered by iteration parity: thread 0 writes the
  // next cursor while other waves may still read the current one), so the
  // segment body keeps the scalar registers of a one-segment kernel.
  __shared__ int32_t s_loop[8];  // cursor unit [2], cursor sequence [2], end unit, P, n
  prefetch_args();
  phase_mark(a, 0);  // workgroup started
  const int h = blockIdx.y;  // kv head: one q-head chunk (G <= 4)
  const bool table = kBalanced && a.seq_lens && a.B > 1 && a.B <= kMaxTableSeqs;
  if constexpr (kBalanced) {
    if (table) build_unit_table(a, s_units);
    UnitSpace us;
    us.start = table ? s_units : nullptr;
    us.n = units_of(a.max_T);
    us.B = a.B;
    const int64_t U = us.total();
    const int64_t P = min((int64_t)gridDim.x, U);  // every workgroup below P has units
    if ((int64_t)blockIdx.x >= P) return;
    if (threadIdx.x == 0) {
      const int64_t u0 = unit_begin(blockIdx.x, U, P);
      s_loop[0] = (int32_t)u0;
      s_loop[2] = us.seq_of(u0);
      s_loop[4] = (int32_t)unit_begin(blockIdx.x + 1, U, P);
      s_loop[5] = (int32_t)P;
      s_loop[6] = (int32_t)us.n;
    }
    __syncthreads();
  }
  for (int it = 0;; ++it) {
    // (balanced plan: the thread index is opaque per segment, so that the
    // lane-derived addresses are computed inside the loop, not hoisted and
    // kept live across the body)
    const int tid = kBalanced ? thread_id() : (int)threadIdx.x;
    __builtin_assume(tid >= 0 && tid < kThreadsMfma);
    // (the wave index in a scalar register: the chunk loop's bounds derive
    // from it, so its branches are uniform)
    const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int col = lane & 15, kg = lane >> 4;
    const int hq = col & 3;   // score layout: head of this lane's column
    const int jb = col >> 2;  // score layout: token block of this lane's column
    const int gn = a.G;
    const int lsk = __builtin_ctz(a.stride[0]), lsv = __builtin_ctz(a.stride[1]);
    const int mk = a.stride[0] - 1, mv = a.stride[1] - 1;
    int b, slot, live;
    int64_t t0, t1;
    if constexpr (kBalanced) {
      const volatile int32_t *sl = s_loop;
      const int32_t u = __builtin_amdgcn_readfirstlane(sl[it & 1]);
      if (u >= __builtin_amdgcn_readfirstlane(sl[4])) break;
      b = __builtin_amdgcn_readfirstlane(sl[2 + (it & 1)]);
      UnitSpace us;
      us.start = table ? s_units : nullptr;
      us.n = __builtin_amdgcn_readfirstlane(sl[6]);
      us.B = a.B;
      Segment sg;
      const int64_t u_next = segment_at(us, blockIdx.x, __builtin_amdgcn_readfirstlane(sl[5]), u,
                                        b, seq_len_of(a, b), sg);
      if (tid == 0) {
        s_loop[(it + 1) & 1] = (int32_t)u_next;
        s_loop[2 + ((it + 1) & 1)] = b + 1;
      }
      if (sg.live == 0) {  // past the sequence's end
        __syncthreads();
        continue;
      }
      t0 = sg.t0;
      t1 = sg.t1;
      slot = sg.slot;
      live = sg.live;
    } else {
      const int split = blockIdx.x;
      b = blockIdx.z;
      const int64_t T = seq_len_of(a, b);
      t0 = (int64_t)split * a.split_len;
      t1 = min(T, t0 + a.split_len);
      if (split_is_empty(split, t0, T)) return;
      slot = split;
      live = kGridLive;
    }
    const int64_t bh = (int64_t)b * a.H + h;

    const __amdgpu_buffer_rsrc_t r_kfk =
        make_rsrc(a.kf[0] + bh * a.cap_kf[0] * kD, (uint32_t)(a.cap_kf[0] * kD * 2));
    const __amdgpu_buffer_rsrc_t r_kfv =
        make_rsrc(a.kf[1] + bh * a.cap_kf[1] * kD, (uint32_t)(a.cap_kf[1] * kD * 2));
    const __amdgpu_buffer_rsrc_t r_pkk =
        make_rsrc(a.pk[0] + bh * a.cap_pf[0] * 16, (uint32_t)(a.cap_pf[0] * 64));
    const __amdgpu_buffer_rsrc_t r_pkv =
        make_rsrc(a.pk[1] + bh * a.cap_pf[1] * (kVRow / 4), (uint32_t)(a.cap_pf[1] * kVRow));
    const __amdgpu_buffer_rsrc_t r_sck = make_rsrc(a.sc[0] + bh * a.cap_pf[0], (uint32_t)(a.cap_pf[0] * 2));
    const __amdgpu_buffer_rsrc_t r_scv = make_rsrc(a.sc[1] + bh * a.cap_pf[1], (uint32_t)(a.cap_pf[1] * 2));

    G4GroupScratch &Gs = lds.s.g;
    G4WaveScratch<kContig> &W = lds.s.w[wave];

    // Stage the chunk at c0 into cb: the token phase (lane = token c0 + lane:
    // scales; per-token loads: own K code row, V slot to LDS), the code blocks
    // (contiguous loads), then the K anchor rows and (per-token loads) the V
    // code words.  A chunk past the end (nt = 0) gets offsets past every
    // buffer, so its loads return zeros without traffic; so do I-frame and
    // padding slots.
    // Scatter targets (LDS words) of this lane's pieces of the contiguous code
    // blocks: piece j holds slot row s = 16j + lane / 4 (relative to base),
    // quarter lane % 4.  A computed chunk starts at c0 = 0 mod 64 (splits
    // start at multiples of the split length, itself a multiple of 64, and
    // balanced segments at multiples of the 512-token unit), so
    // the P-frame token of row s depends on s alone: for strides below 64
    // (c0 an I-frame) t = s + (s - 1) / (stride - 1), s >= 1; for larger
    // strides t = s.  Rows of other tokens go to the junk row.  Rows of
    // I-frame and padding tokens keep whatever they held: their scales are 0,
    // so any finite nibbles there (every bit pattern is one) contribute 0.
    auto scatter_word = [&](int j, int ls) {
      const int sr = 16 * j + (lane >> 2);
      int t = sr;
      if (ls < 6) t = sr == 0 ? kChunk : sr + (sr - 1) / ((1 << ls) - 1);
      return min(t, kChunk) * kRowWords + 4 * (lane & 3);
    };
    int wk[4], wv[4];
    if constexpr (kContig) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        wk[j] = scatter_word(j, lsk);
        wv[j] = scatter_word(j, lsv);
      }
      if constexpr (kDenseV) {
        // 48-byte rows: piece j of lane l is third (64j + l) % 3 of slot row
        // (64j + l) / 3, written to words 4 * third of its token's row
#pragma unroll
        for (int j = 0; j < kVBlocks; ++j) {
          const int pc = 64 * j + lane, sr = pc / 3;
          int t = sr;
          if (lsv < 6) t = sr == 0 ? kChunk : sr + (sr - 1) / ((1 << lsv) - 1);
          wv[j] = min(t, kChunk) * kRowWords + 4 * (pc - 3 * sr);
        }
      }
    }
    // Lane constants.  Every computed chunk starts at a multiple of 64 tokens,
    // so for a power-of-two stride 2^s and 0 <= x < 64, (c0 + x) >> s =
    // (c0 >> s) + (x >> s), and (c0 + x) is a multiple of 2^s iff both c0 and
    // x are: token indices within the chunk split into a uniform part and a
    // lane constant.
    const int lane_sk = lane - (lane >> lsk), lane_sv = lane - (lane >> lsv);
    const bool lane_pk = (lane & mk) != 0, lane_pv = (lane & mv) != 0;
    auto stage = [&](int c0, G4Buf &cb) {
      const int nt = (int)max((int64_t)0, min((int64_t)kChunk, t1 - c0));
      cb.c0 = c0;
      cb.nt = nt;
      const int gk_base = c0 >> lsk;
      const int gk_last = nt ? (c0 + nt - 1) >> lsk : gk_base;
      // anchor offsets stay below 2^30; buffers are below 2^31 bytes (mfma_supported)
      const uint32_t dead = nt ? 0u : 0x80000000u;
      {
        // slot t - t / stride - 1 of token t = c0 + lane (a P-frame iff t is
        // not a multiple of the stride; a chunk without tokens reads nothing)
        const bool valid = lane < nt;
        const bool pk = (c0 & mk) != 0 || lane_pk, pv = (c0 & mv) != 0 || lane_pv;
        const int slk = (valid && pk) ? c0 - gk_base - 1 + lane_sk : -1;
        const int slv = (valid && pv) ? c0 - (c0 >> lsv) - 1 + lane_sv : -1;
        // slot -1 reads past the buffer: scale 0, codes 0
        cb.sk = bload16(r_sck, (uint32_t)slk * 2u);
        cb.sv = bload16(r_scv, (uint32_t)slv * 2u);
        if constexpr (!kContig) {
#pragma unroll
          // the row's 4 quarters: each load touches every 64-byte row of the chunk
          // once, so these stay cacheable for the next three (no nt policy)
          for (int q = 0; q < 4; ++q) {
            const i4_t v = __builtin_amdgcn_raw_buffer_load_b128(r_pkk, (int)((uint32_t)slk * 64u + 16u * q), 0, 0);
            cb.kr[q] = uint4{(uint32_t)v[0], (uint32_t)v[1], (uint32_t)v[2], (uint32_t)v[3]};
          }
          W.slot_v[lane] = slv;
        }
      }
      if constexpr (kContig) {
        // The chunk's code rows as contiguous 1 KB blocks: slot rows base ..
        // base + 63, base the slot token c0 would have (every P-frame row of
        // the chunk lies in them; rows before slot 0 or past the buffer read 0)
        const uint32_t bk = ((uint32_t)(c0 - gk_base - 1) * 64u + 16u * lane) | dead;
        const uint32_t bv = ((uint32_t)(c0 - (c0 >> lsv) - 1) * kVRow + 16u * lane) | dead;
#pragma unroll
        for (int q = 0; q < 4; ++q) cb.kr[q] = bload128(r_pkk, bk + 1024u * q);
#pragma unroll
        for (int i = 0; i < kVBlocks; ++i) {
          const uint4 w = bload128(r_pkv, bv + 1024u * i);
          cb.vw[i][0] = w.x;
          cb.vw[i][1] = w.y;
          cb.vw[i][2] = w.z;
          cb.vw[i][3] = w.w;
        }
      }
      {
        const uint32_t row = ((uint32_t)min(gk_base + col, gk_last) * 256u + 64u * kg) | dead;
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) cb.ka[kb] = bload128(r_kfk, row + 16u * kb);
      }
      if constexpr (!kContig) {
        // the slots other lanes stored above (no instruction at wave scope;
        // it orders the LDS store before the loads)
        wave_lds_sync();
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int4 sl4 = *(const int4 *)&W.slot_v[16 * i + 4 * kg];
          cb.vw[i][0] = bload32(r_pkv, (uint32_t)sl4.x * 64u + 4u * col);
          cb.vw[i][1] = bload32(r_pkv, (uint32_t)sl4.y * 64u + 4u * col);
          cb.vw[i][2] = bload32(r_pkv, (uint32_t)sl4.z * 64u + 4u * col);
          cb.vw[i][3] = bload32(r_pkv, (uint32_t)sl4.w * 64u + 4u * col);
        }
      }
    };
    // V anchor rows gv_base + 4kg + r of the chunk at c0, dims 8col .. 8col+7.
    uint4 va[4];
    if constexpr (kBalanced) va[0] = va[1] = va[2] = va[3] = uint4{0u, 0u, 0u, 0u};
    auto stage_va = [&](int c0) {
      const int nt = (int)max((int64_t)0, min((int64_t)kChunk, t1 - c0));
      const int gv_base = c0 >> lsv;
      // anchors gv_base + min(4kg + r, last - gv_base), last = (c0 + nt - 1) / stride
      const int dv = nt ? (nt - 1) >> lsv : 0;
      const uint32_t base = (((uint32_t)gv_base * 256u) | (nt ? 0u : 0x80000000u)) + 16u * col;
#pragma unroll
      for (int r = 0; r < 4; ++r) va[r] = bload128(r_kfv, (uint32_t)min(4 * kg + r, dv) * 256u + base);
    };

    // Wave 0's q rows are requested first, then every wave's first chunk:
    // the two round trips overlap, and the q table (and the barrier after
    // it) waits for the q rows only, not for wave 0's chunk behind them.
    uint4 q_raw = uint4{0u, 0u, 0u, 0u};
    if (tid < 64 && (tid >> 4) < gn)
      q_raw = *(const uint4 *)((const uint16_t *)a.q +
                               ((int64_t)b * a.nq + h * a.G + (tid >> 4)) * kD + 8 * (tid & 15));
    int64_t c0l = t0 + (int64_t)wave * kChunk;
    const bool has_work = c0l < t1;
    // (balanced plan: zero-initialised; left undefined on a segment without
    // work, they would be carried from the previous segment and stay live
    // across the whole body)
    G4Buf bufA, bufB;
    if constexpr (kBalanced) bufA = bufB = G4Buf{};
    // Unconditional, so that the count of loads in flight is the same on every
    // path and the q table's wait covers the q rows only: a wave without work
    // stages a chunk past the end (no traffic, zeros).
    stage((int)min(c0l, t1), bufA);
    stage_va((int)min(c0l, t1));
    phase_mark(a, 1);  // first chunk's loads issued

    // ---- q table: q' = fp16(q * fp16(scale)) (bf16 queries: bf16(q * bf16(scale)))
    // per (parity, slab pair, head) in the order unpack_pair gives a code
    // word pair's nibbles; heads >= gn are zero.
    if (tid < 64) {
      const int hh = tid >> 4, m = tid & 15;
      h8_t v = {};
      float part = 0.f;
      if (hh < gn) {
        const uint4 raw = q_raw;
        const h8_t x = a.q_dtype == CQ_BF16 ? bf16x8_scaled_to_f16(raw, bf16_round(a.scale))
                                            : __builtin_bit_cast(h8_t, raw) * (_Float16)a.scale;
        v = x;
#pragma unroll
        for (int e = 0; e < 8; ++e) part += (float)x[e];
      }
      // slab m is half m & 1 of pair m >> 1
      ((h4_t *)&Gs.q[m >> 1][hh])[m & 1] = h4_t{v[0], v[4], v[2], v[6]};
      ((h4_t *)&Gs.q[8 + (m >> 1)][hh])[m & 1] = h4_t{v[1], v[5], v[3], v[7]};
      Gs.qn[m][hh] = v;
      part = row16_sum(part);  // the 16 lanes m of head hh
      if (m == 0) Gs.s8[hh] = 8.f * part;
    } else if (tid < 128) {
      (&Gs.zero[0][0])[tid - 64] = h8_t{};
    }
    __syncthreads();
    phase_mark(a, 2);  // q table ready
    // score-layout B operand of (parity, pair): Gs.q[..][hq] on the diagonal blocks, else zeros
    const h8_t *qsrc = jb == kg ? &Gs.q[0][hq] : &Gs.zero[0][hq];
    // 16-head-layout B operand of the anchor product (q'^T, column = head)
    const h8_t *qcol = col < kG4 ? &Gs.qn[0][col] : &Gs.zero[0][0];
    // the anchor table row of this lane's score tokens 16 jb + 4 kg (+ r < 4)
    const int qa_row = (16 * jb + 4 * kg) >> lsk;
    // E^T operand dwords of the P_g product (group col against tokens 32P +
    // 4kg + e and 32P + 16 + 4kg + e): fp16 1.0 pairs or zero
    uint32_t eop[2][2];
#pragma unroll
    for (int P = 0; P < 2; ++P) {
      eop[P][0] = ((32 * P + 4 * kg) >> lsv) == col ? 0x3c003c00u : 0u;
      eop[P][1] = ((32 * P + 16 + 4 * kg) >> lsv) == col ? 0x3c003c00u : 0u;
    }
    const float s8l = Gs.s8[hq] * kLog2e;

    uint32_t magic;  // fp16 1024 in both halves, held in a VGPR for v_and_or_b32
    asm volatile("v_mov_b32 %0, 0x64006400" : "=v"(magic));
    // dense V rows: the fp16 exponent fields of 2^(10 - pos), pos = 0 .. 7, in
    // both halves (VGPRs, as magic)
    uint32_t mg3[8];
    if constexpr (kDenseV) {
      asm volatile("v_mov_b32 %0, 0x64006400" : "=v"(mg3[0]));
      asm volatile("v_mov_b32 %0, 0x60006000" : "=v"(mg3[1]));
      asm volatile("v_mov_b32 %0, 0x5c005c00" : "=v"(mg3[2]));
      asm volatile("v_mov_b32 %0, 0x58005800" : "=v"(mg3[3]));
      asm volatile("v_mov_b32 %0, 0x54005400" : "=v"(mg3[4]));
      asm volatile("v_mov_b32 %0, 0x50005000" : "=v"(mg3[5]));
      asm volatile("v_mov_b32 %0, 0x4c004c00" : "=v"(mg3[6]));
      asm volatile("v_mov_b32 %0, 0x48004800" : "=v"(mg3[7]));
    }

    // score layout: softmax state of head hq (identical across its 16 lanes)
    float m_run = -INFINITY;  // log2 units
    float l_run = 0.f;        // sum of fp16 p over this lane's tokens
    float w_run = 0.f;        // sum of fp16 p*s_v
    float x_run = 0.f;        // sum of fp16 p*s_v/16
    f4_t acc[8];
#pragma unroll
    for (int nb = 0; nb < 8; ++nb) acc[nb] = f4_t{0.f, 0.f, 0.f, 0.f};
    const h2_t ones = {(_Float16)1.f, (_Float16)1.f};
    const h2_t sixteenth = {(_Float16)0.0625f, (_Float16)0.0625f};

    auto compute = [&](G4Buf &cb, int sl) {
      const int c0 = cb.c0;
      const int gk_base = c0 >> lsk, gv_base = c0 >> lsv;
      W.s16[sl][lane] = cb.sk | (cb.sv << 16);
      if constexpr (kContig) {
        // code rows by token: K row of this lane's token, V word col of tokens
        // 16i + 4kg + r
#pragma unroll
        for (int j = 0; j < 4; ++j) *(uint4 *)&W.rows.k[0][wk[j]] = cb.kr[j];
#pragma unroll
        for (int j = 0; j < kVBlocks; ++j)
          *(uint4 *)&W.rows.v[0][wv[j]] = uint4{cb.vw[j][0], cb.vw[j][1], cb.vw[j][2], cb.vw[j][3]};
        wave_lds_sync();
#pragma unroll
        for (int q = 0; q < 4; ++q) cb.kr[q] = *(const uint4 *)&W.rows.k[lane][4 * q];
        if constexpr (kDenseV) {
          // the 24 stream bits of dims 8col .. 8col + 7 (bytes 3col .. 3col + 2
          // of the row) moved to bits 0 .. 23
          const int w0 = (3 * col) >> 2, sh = 8 * ((3 * col) & 3);
#pragma unroll
          for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              const uint32_t *row = W.rows.v[16 * i + 4 * kg + r];
              cb.vw[i][r] = __builtin_amdgcn_alignbit(row[w0 + 1], row[w0], sh);
            }
        } else {
#pragma unroll
          for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int r = 0; r < 4; ++r) cb.vw[i][r] = W.rows.v[16 * i + 4 * kg + r][col];
        }
      }
      // ---- anchor table: log2e * q'.a - mref for anchors gk_base + 4kg + r ----------
      // (C[anchor][head col]; the lanes col < 4 are head col's score lanes of
      // block 0, whose m_run is head col's)
      {
        f4_t d = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        // product kb: lane group kg supplies parity kb & 1 of slabs 4kg + 2(kb >> 1), +1
        // product kb: lane group kg supplies dims 32kg + 8kb .. + 7 (natural order)
        for (int kb = 0; kb < 4; ++kb)
          d = mfma32(__builtin_bit_cast(h8_t, cb.ka[kb]), qcol[(4 * kg + kb) * kG4], d);
        if (col < kG4) {
          const float mref = (m_run == -INFINITY) ? 0.f : m_run;
#pragma unroll
          for (int r = 0; r < 4; ++r) W.qa[4 * kg + r][col] = __builtin_fmaf(d[r], kLog2e, -mref);
        }
      }
      wave_lds_sync();

      // ---- scores of tokens 16 jb + 4 kg + r, head hq (log2 units, minus mref) -------
      // two accumulation chains, one per parity (the odd one at 16x scale);
      // the q' operands of a group of 4 slabs are read from LDS together
      f4_t d0 = {0.f, 0.f, 0.f, 0.f}, d1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const h8_t e0 = qsrc[(2 * q) * kG4], o0 = qsrc[(8 + 2 * q) * kG4];
        const h8_t e1 = qsrc[(2 * q + 1) * kG4], o1 = qsrc[(8 + 2 * q + 1) * kG4];
        const uint4 w = cb.kr[q];
        const uint32_t tx = w.x >> 8, ty = w.y >> 8, tz = w.z >> 8, tw = w.w >> 8;
        d0 = mfma32(unpack_pair(w.x, w.y, tx, ty, 0x000F000Fu), e0, d0);
        d1 = mfma32(unpack_pair(w.x, w.y, tx, ty, 0x00F000F0u), o0, d1);
        d0 = mfma32(unpack_pair(w.z, w.w, tz, tw, 0x000F000Fu), e1, d0);
        d1 = mfma32(unpack_pair(w.z, w.w, tz, tw, 0x00F000F0u), o1, d1);
      }
      f4_t d;
#pragma unroll
      for (int r = 0; r < 4; ++r) d[r] = __builtin_fmaf(d1[r], 0.0625f, d0[r]);
      const int tb = 16 * jb + 4 * kg;
      const uint4 s4 = *(const uint4 *)&W.s16[sl][tb];
      const uint32_t sr[4] = {s4.x, s4.y, s4.z, s4.w};
      // the 4 tokens share one K anchor (stride >= 4, token groups aligned to 4)
      const float qa = W.qa[qa_row][hq];
      float sc[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        // log2e * s * (q'.c) with q'.c = 2^24 d - 8 sum(q')
        const float qc = __builtin_fmaf(d[r], kTwo24 * kLog2e, -s8l);
        sc[r] = __builtin_fmaf((float)as_h2(sr[r]).x, qc, qa);
      }
      // Tokens past the end exist only in a split's last chunk (a uniform branch).
      if (cb.nt < kChunk) {
#pragma unroll
        for (int r = 0; r < 4; ++r)
          if (tb + r >= cb.nt) sc[r] = -INFINITY;
      }

      // ---- lazy running max (scores are relative to mref already) ---------------------
      const float mx = fmaxf(fmaxf(sc[0], sc[1]), fmaxf(sc[2], sc[3]));
      if (__any(m_run == -INFINITY || mx > kTau)) {
        // chunk max of head hq: its lanes differ in jb (col bits 2, 3) and kg
        // (lanes ^ 4 and ^ 8 by DPP rotations, ^ 16 and ^ 32 by permlane
        // swaps: no LDS round trips on the first chunk's path)
        const float cm = xor32_max(xor16_max(row16_mod4_max(mx)));
        const float mref = (m_run == -INFINITY) ? 0.f : m_run;
        const float m_new = fmaxf(m_run, mref + cm);
        // (a wave's first chunk: the sums and acc are still zero)
        if (!__all(m_run == -INFINITY)) {
          const float f = (m_run == -INFINITY) ? 0.f : fast_exp2(m_run - m_new);
          l_run *= f;
          w_run *= f;
          x_run *= f;
          // acc row 4kg + r holds head r (rows >= 4 repeat heads r, unused);
          // lane r of every quad holds head r's factor
          const float fr[4] = {dpp_f<kDppQuadBcast<0>>(f), dpp_f<kDppQuadBcast<1>>(f),
                               dpp_f<kDppQuadBcast<2>>(f), dpp_f<kDppQuadBcast<3>>(f)};
#pragma unroll
          for (int r = 0; r < 4; ++r)
#pragma unroll
            for (int nb = 0; nb < 8; ++nb) acc[nb][r] *= fr[r];
        }
        const float shift = ((m_new == -INFINITY) ? 0.f : m_new) - mref;
#pragma unroll
        for (int r = 0; r < 4; ++r) sc[r] -= shift;
        m_run = m_new;
      }

      // ---- weights: p (fp16), p*s_v and p*s_v/16 (fp16 products) -------------------------
      {
        const h2_t p01 = h2_t{(_Float16)fast_exp2(sc[0]), (_Float16)fast_exp2(sc[1])};
        const h2_t p23 = h2_t{(_Float16)fast_exp2(sc[2]), (_Float16)fast_exp2(sc[3])};
        const h2_t sv01 = as_h2(__builtin_amdgcn_perm(s4.y, s4.x, 0x07060302u));
        const h2_t sv23 = as_h2(__builtin_amdgcn_perm(s4.w, s4.z, 0x07060302u));
        const h2_t w01 = p01 * sv01, w23 = p23 * sv23;
        l_run = __builtin_amdgcn_fdot2(p01, ones, l_run, false);
        l_run = __builtin_amdgcn_fdot2(p23, ones, l_run, false);
        w_run = __builtin_amdgcn_fdot2(w01, ones, w_run, false);
        w_run = __builtin_amdgcn_fdot2(w23, ones, w_run, false);
        // to the V-product operand layout: (head hq, 4-token group 4 jb + kg)
        const int g4 = 4 * jb + kg;
        W.pw[0][hq][g4] = uint2{__builtin_bit_cast(uint32_t, p01), __builtin_bit_cast(uint32_t, p23)};
        W.pw[1][hq][g4] = uint2{__builtin_bit_cast(uint32_t, w01), __builtin_bit_cast(uint32_t, w23)};
        if constexpr (!kDenseV) {
          const h2_t x01 = w01 * sixteenth, x23 = w23 * sixteenth;
          x_run = __builtin_amdgcn_fdot2(x01, ones, x_run, false);
          x_run = __builtin_amdgcn_fdot2(x23, ones, x_run, false);
          W.pw[2][hq][g4] = uint2{__builtin_bit_cast(uint32_t, x01), __builtin_bit_cast(uint32_t, x23)};
        }
      }
      wave_lds_sync();

      // ---- P_g and code P.V, two 16-token tiles per K=32 product --------------------------
      // K index 8kg + e of the products below is token 16(2P) + 4kg + e (e < 4)
      // or 16(2P+1) + 4kg + e - 4 (e >= 4).  Operand rows are heads (col & 3:
      // rows >= 4 repeat heads 0..3 and are never read).
      const int hr = col & 3;
      f4_t pg = {0.f, 0.f, 0.f, 0.f};  // P_g^T: lane holds groups 4kg+r, head col
#pragma unroll
      for (int P = 0; P < 2; ++P) {
        const uint2 pa = W.pw[0][hr][8 * P + kg], pb = W.pw[0][hr][8 * P + 4 + kg];
        const uint2 wa = W.pw[1][hr][8 * P + kg], wb = W.pw[1][hr][8 * P + 4 + kg];
        const h8_t ap = h8_of(pa.x, pa.y, pb.x, pb.y);
        const h8_t aw = h8_of(wa.x, wa.y, wb.x, wb.y);
        // E^T: group col x these tokens (fp16 1.0 = 0x3c00); each run of 4
        // tokens lies in one V group (stride >= 4)
        pg = mfma32(h8_of(eop[P][0], eop[P][0], eop[P][1], eop[P][1]), ap, pg);
        const int i0 = 2 * P, i1 = 2 * P + 1;
        if constexpr (kDenseV) {
          // V codes, dense rows: B = 8 tokens x dim 8col + e.  Byte pairs of
          // a token pair's 24-bit groups (token r0 in the low half, r1 in the
          // high half): bytes 0-1 hold fields 0, 1, 2 at bits 0, 3, 6; bytes
          // 1-2 fields 3, 4, 5 at bits 1, 4, 7; byte 2 fields 6, 7 at bits 2,
          // 5.  A field u at bit pos of a half, ORed with the fp16 exponent of
          // 2^(10 - pos), is the fp16 value 2^(10 - pos) + u exactly.
          uint32_t q0[4], q1[4], q2[4];
#pragma unroll
          for (int u = 0; u < 2; ++u)
#pragma unroll
            for (int m = 0; m < 2; ++m) {
              const uint32_t xa = cb.vw[i0 + u][2 * m], xb = cb.vw[i0 + u][2 * m + 1];
              q0[2 * u + m] = __builtin_amdgcn_perm(xb, xa, 0x05040100u);
              q1[2 * u + m] = __builtin_amdgcn_perm(xb, xa, 0x06050201u);
              q2[2 * u + m] = __builtin_amdgcn_perm(xb, xa, 0x0c060c02u);
            }
          auto vop = [&](const uint32_t(&q)[4], uint32_t m, uint32_t mg) {
            return h8_of(and_or(q[0], m, mg), and_or(q[1], m, mg), and_or(q[2], m, mg),
                         and_or(q[3], m, mg));
          };
          acc[0] = mfma32(aw, vop(q0, 0x00070007u, mg3[0]), acc[0]);
          acc[1] = mfma32(aw, vop(q0, 0x00380038u, mg3[3]), acc[1]);
          acc[2] = mfma32(aw, vop(q0, 0x01C001C0u, mg3[6]), acc[2]);
          acc[3] = mfma32(aw, vop(q1, 0x000E000Eu, mg3[1]), acc[3]);
          acc[4] = mfma32(aw, vop(q1, 0x00700070u, mg3[4]), acc[4]);
          acc[5] = mfma32(aw, vop(q1, 0x03800380u, mg3[7]), acc[5]);
          acc[6] = mfma32(aw, vop(q2, 0x001C001Cu, mg3[2]), acc[6]);
          acc[7] = mfma32(aw, vop(q2, 0x00E000E0u, mg3[5]), acc[7]);
        } else {
        const uint2 xa = W.pw[2][hr][8 * P + kg], xb = W.pw[2][hr][8 * P + 4 + kg];
        const h8_t ax = h8_of(xa.x, xa.y, xb.x, xb.y);
        // V codes: B = 8 tokens x dim 8col + nb (nibble nb of word col)
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const uint32_t sel = (uint32_t)k | (0x0cu << 8) | ((uint32_t)(4 + k) << 16) | (0x0cu << 24);
          const uint32_t a01 = __builtin_amdgcn_perm(cb.vw[i0][1], cb.vw[i0][0], sel);
          const uint32_t a23 = __builtin_amdgcn_perm(cb.vw[i0][3], cb.vw[i0][2], sel);
          const uint32_t b01 = __builtin_amdgcn_perm(cb.vw[i1][1], cb.vw[i1][0], sel);
          const uint32_t b23 = __builtin_amdgcn_perm(cb.vw[i1][3], cb.vw[i1][2], sel);
          const h8_t blo = h8_of(and_or(a01, 0x000F000Fu, magic), and_or(a23, 0x000F000Fu, magic),
                                 and_or(b01, 0x000F000Fu, magic), and_or(b23, 0x000F000Fu, magic));
          const h8_t bhi = h8_of(and_or(a01, 0x00F000F0u, magic), and_or(a23, 0x00F000F0u, magic),
                                 and_or(b01, 0x00F000F0u, magic), and_or(b23, 0x00F000F0u, magic));
          acc[2 * k] = mfma32(aw, blo, acc[2 * k]);
          acc[2 * k + 1] = mfma32(ax, bhi, acc[2 * k + 1]);
        }
        }
      }

      // ---- anchor term: P_g as an fp16 hi/lo pair in one K=32 product -------------------
      // K index 8kg + e: group 4kg + e, hi part (e < 4) or lo part (e >= 4); the
      // anchor rows are duplicated in the B operand to match.
      {
        const h2_t ph01 = h2_t{(_Float16)pg[0], (_Float16)pg[1]};
        const h2_t ph23 = h2_t{(_Float16)pg[2], (_Float16)pg[3]};
        const h2_t pl01 = h2_t{(_Float16)(pg[0] - (float)ph01.x), (_Float16)(pg[1] - (float)ph01.y)};
        const h2_t pl23 = h2_t{(_Float16)(pg[2] - (float)ph23.x), (_Float16)(pg[3] - (float)ph23.y)};
        const h8_t pa = h8_t{ph01.x, ph01.y, ph23.x, ph23.y, pl01.x, pl01.y, pl23.x, pl23.y};
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const h4_t blo = rows_operand(va, k, false), bhi = rows_operand(va, k, true);
          acc[2 * k] = mfma32(pa, h8_t{blo[0], blo[1], blo[2], blo[3], blo[0], blo[1], blo[2], blo[3]},
                              acc[2 * k]);
          acc[2 * k + 1] = mfma32(pa, h8_t{bhi[0], bhi[1], bhi[2], bhi[3], bhi[0], bhi[1], bhi[2], bhi[3]},
                                  acc[2 * k + 1]);
        }
      }
    };

    // Software pipeline: the next chunk's loads are issued before the current
    // chunk is computed (two register buffers, unrolled by two).  Splits of at
    // most one chunk per wave (kOneChunk) have nothing to pipeline.
    if constexpr (kOneChunk) {
      if (has_work) compute(bufA, 0);
      phase_mark(a, 3);  // wave 0's chunk computed (issued)
    } else if (has_work) {
      // The wave's n >= 1 chunks c0l, c0l + kStep, ... below t1, in pairs and
      // one last single chunk, so that the loop has one exit, at its end.  (An
      // exit between the two halves joins the loop header with the first
      // half's loads in flight, and the header then waits for all of them
      // before it issues the next chunk's.)  The last pair's V anchor loads
      // are dead (offsets past the buffer, no memory access).
      constexpr int64_t kStep = (int64_t)kWaves * kChunk;
      int n = __builtin_amdgcn_readfirstlane((int)((t1 - c0l + kStep - 1) / kStep));
      for (; n > 1; n -= 2) {
        stage((int)(c0l + kStep), bufB);
        compute(bufA, 0);
        c0l += kStep;
        stage_va((int)c0l);
        stage((int)(c0l + kStep), bufA);
        compute(bufB, 1);
        c0l += kStep;
        stage_va((int)c0l);
      }
      if (n) compute(bufA, 0);
    }

    // ---- totals of head hq: its 16 lanes hold disjoint tokens ---------------------------
    // (the lanes of a row by DPP rotations, the 4 rows by shuffles)
    l_run = row16_mod4_sum(l_run);
    w_run = row16_mod4_sum(w_run);
    x_run = row16_mod4_sum(x_run);
#pragma unroll
    for (int x = 16; x < 64; x *= 2) {
      l_run += __shfl_xor(l_run, x, 64);
      w_run += __shfl_xor(w_run, x, 64);
      x_run += __shfl_xor(x_run, x, 64);
    }
    // lane r of every quad: head r
    const float sw[4] = {dpp_f<kDppQuadBcast<0>>(w_run), dpp_f<kDppQuadBcast<1>>(w_run),
                         dpp_f<kDppQuadBcast<2>>(w_run), dpp_f<kDppQuadBcast<3>>(w_run)};
    const float sx[4] = {dpp_f<kDppQuadBcast<0>>(x_run), dpp_f<kDppQuadBcast<1>>(x_run),
                         dpp_f<kDppQuadBcast<2>>(x_run), dpp_f<kDppQuadBcast<3>>(x_run)};
    // merge_finish_g4 reads (m, l) of head col from the lanes col < 4 of kg 0:
    // head col's score lanes of block 0.  Code columns: x = 1032 + c (even nb,
    // weight p s) or 1152 + 16c (odd nb, weight p s / 16).
    merge_finish_g4(a, lds.mg, b, h, gn, slot, live, m_run, l_run, [&](int nb, int r) {
      if constexpr (kDenseV) {
        // field u of dim 8col + nb entered as 2^(10 - pos) + u, code u - 4
        constexpr float kOff[8] = {1028.f, 132.f, 20.f, 516.f, 68.f, 12.f, 260.f, 36.f};
        return acc[nb][r] - kOff[nb] * sw[r];
      } else {
        const float corr = (nb & 1) ? 1024.f * sx[r] + 8.f * sw[r] : 1032.f * sw[r];
        return acc[nb][r] - corr;
      }
    });
    if constexpr (!kBalanced) return;
    __syncthreads();  // the next segment's merge reuses the merge area
  }
}

// ---------------------------------------------------------------------------
// Uncompressed fp16 flash decode (cq_fp16_decode_attn), head_dim 128, GQA
// groups of at most 4 q heads: the baseline the compressed path is measured
// against.  K, V: fp16 [B][H][cap][128].  Same grid plan, workgroup merge and
// split fold as decode_g4_kernel; each wave takes 64-token chunks.
//
// Scores: S = K q'^T with v_mfma_f32_16x16x32_f16, A = 16 K rows (token i of
// tile j) x 32 dims, B = q' (column c = head c % 4, so every quad of lanes
// holds the 4 heads).  K-step s covers dims 32 s .. 32 s + 31, lane group kg
// dims 32 s + 8 kg .. + 7: one load instruction reads 64 contiguous bytes of
// each of 16 rows (the next step the other half of their 128-byte lines, so
// these loads keep the default cache policy and the second half hits L2).
// P.V: A = p (rows = heads), B = V with column n of tile m = dim 8 n + m: lane
// (n, kg) loads 16 bytes (dims 8n .. 8n + 7) of 8 token rows per 32-token
// step (the 16 lanes of a row read it whole), and one byte permute per two
// tokens moves element m of two rows into one operand dword.
// ---------------------------------------------------------------------------
struct alignas(16) F16Lds {
  h8_t q[kG4][16];         // q' of head h, dims 8m .. 8m + 7 (heads >= G: 0)
  uint2 p[kWaves][kG4][4][4];  // fp16 p of (wave, head, tile, lane group kg): 4 tokens
  G4Merge mg;
};

__global__ __launch_bounds__(kThreadsMfma) void decode_fp16_g4_kernel(DecodeArgs a) {
  __shared__ F16Lds lds;
  prefetch_args();
  phase_mark(a, 0);  // workgroup started
  const int split = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int col = lane & 15, kg = lane >> 4, hq = col & 3;
  const int gn = a.G;
  const int64_t T = seq_len_of(a, b);
  const int64_t t0 = (int64_t)split * a.split_len, t1 = min(T, t0 + a.split_len);
  if (split_is_empty(split, t0, T)) return;
  const int64_t bh = (int64_t)b * a.H + h;
  const __amdgpu_buffer_rsrc_t rk =
      make_rsrc(a.kf[0] + bh * a.cap_kf[0] * kD, (uint32_t)(a.cap_kf[0] * kD * 2));
  const __amdgpu_buffer_rsrc_t rv =
      make_rsrc(a.kf[1] + bh * a.cap_kf[1] * kD, (uint32_t)(a.cap_kf[1] * kD * 2));

  uint4 q_raw = uint4{0u, 0u, 0u, 0u};
  if (tid < 64 && (tid >> 4) < gn)
    q_raw = *(const uint4 *)((const uint16_t *)a.q +
                             ((int64_t)b * a.nq + h * a.G + (tid >> 4)) * kD + 8 * (tid & 15));
  uint4 kr[4][4], vr[2][8];
  // chunk at c0 (rows past the buffer read 0; tokens past t1 are masked)
  auto load = [&](int64_t c0) {
    const uint32_t r0 = (uint32_t)c0;
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int st = 0; st < 4; ++st)
        kr[j][st] = bload128_cached(rk, (r0 + 16u * j + col) * 256u + 64u * st + 16u * kg);
#pragma unroll
    for (int st = 0; st < 2; ++st)
#pragma unroll
      for (int e = 0; e < 8; ++e)
        vr[st][e] = bload128(rv, (r0 + 32u * st + 8u * kg + e) * 256u + 16u * col);
  };
  int64_t c0 = t0 + (int64_t)wave * kChunk;
  load(c0);
  phase_mark(a, 1);  // first chunk's loads issued
  if (tid < 64) {
    h8_t v = {};
    if ((tid >> 4) < gn) v = __builtin_bit_cast(h8_t, q_raw) * (_Float16)a.scale;
    lds.q[tid >> 4][tid & 15] = v;
  }
  __syncthreads();
  phase_mark(a, 2);  // q table ready
  h8_t qb[4];
#pragma unroll
  for (int st = 0; st < 4; ++st) qb[st] = lds.q[hq][4 * st + kg];

  float m_run = -INFINITY, l_run = 0.f;
  f4_t acc[8];
#pragma unroll
  for (int nb = 0; nb < 8; ++nb) acc[nb] = f4_t{0.f, 0.f, 0.f, 0.f};
  const h2_t ones = {(_Float16)1.f, (_Float16)1.f};
  while (c0 < t1) {  // wave-uniform
    const int nt = (int)min((int64_t)kChunk, t1 - c0);
    f4_t S[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      S[j] = f4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int st = 0; st < 4; ++st) S[j] = mfma32(__builtin_bit_cast(h8_t, kr[j][st]), qb[st], S[j]);
    }
    // lane (col, kg): tokens 16 j + 4 kg + r of head hq, log2 units
    float sc[4][4];
    float mx = -INFINITY;
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        sc[j][r] = (16 * j + 4 * kg + r < nt) ? S[j][r] * kLog2e : -INFINITY;
        mx = max_nn(mx, sc[j][r]);
      }
    const float cm = xor32_max(xor16_max(mx));  // the chunk's max of head hq
    if (__any(m_run == -INFINITY || cm > m_run + kTau)) {
      const float m_new = fmaxf(m_run, cm);
      const float f = (m_run == -INFINITY) ? 0.f : fast_exp2(m_run - m_new);
      l_run *= f;
      const float fr[4] = {dpp_f<kDppQuadBcast<0>>(f), dpp_f<kDppQuadBcast<1>>(f),
                           dpp_f<kDppQuadBcast<2>>(f), dpp_f<kDppQuadBcast<3>>(f)};
#pragma unroll
      for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int nb = 0; nb < 8; ++nb) acc[nb][r] *= fr[r];
      m_run = m_new;
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const h2_t p01 = h2_t{(_Float16)fast_exp2(sc[j][0] - m_run), (_Float16)fast_exp2(sc[j][1] - m_run)};
      const h2_t p23 = h2_t{(_Float16)fast_exp2(sc[j][2] - m_run), (_Float16)fast_exp2(sc[j][3] - m_run)};
      l_run = __builtin_amdgcn_fdot2(p01, ones, l_run, false);
      l_run = __builtin_amdgcn_fdot2(p23, ones, l_run, false);
      if (col < kG4)
        lds.p[wave][col][j][kg] = uint2{__builtin_bit_cast(uint32_t, p01), __builtin_bit_cast(uint32_t, p23)};
    }
    wave_lds_sync();
    // P.V: step st covers tokens 32 st .. + 31; A row i (head i % 4), K index
    // 8 kg + e = token 32 st + 8 kg + e = tile 2 st + kg / 2, row 8 (kg & 1) + e
#pragma unroll
    for (int st = 0; st < 2; ++st) {
      const uint4 pa = *(const uint4 *)&lds.p[wave][hq][2 * st + (kg >> 1)][2 * (kg & 1)];
      const h8_t ap = __builtin_bit_cast(h8_t, pa);
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        uint32_t lo[4], hi[4];
#pragma unroll
        for (int e2 = 0; e2 < 4; ++e2) {
          const uint32_t w0 = (&vr[st][2 * e2].x)[m], w1 = (&vr[st][2 * e2 + 1].x)[m];
          lo[e2] = __builtin_amdgcn_perm(w1, w0, 0x05040100u);
          hi[e2] = __builtin_amdgcn_perm(w1, w0, 0x07060302u);
        }
        acc[2 * m] = mfma32(ap, h8_of(lo[0], lo[1], lo[2], lo[3]), acc[2 * m]);
        acc[2 * m + 1] = mfma32(ap, h8_of(hi[0], hi[1], hi[2], hi[3]), acc[2 * m + 1]);
      }
    }
    wave_lds_sync();  // this chunk's p reads before the next chunk's writes
    c0 += (int64_t)kWaves * kChunk;
    if (c0 < t1) load(c0);
  }
  phase_mark(a, 3);  // wave 0's chunks computed (issued)
  // head hq's weight sum: its lanes col, col + 16, col + 32, col + 48
  l_run = xor32_sum(xor16_sum(l_run));
  merge_finish_g4(a, lds.mg, b, h, gn, split, kGridLive, m_run, l_run,
                  [&](int nb, int r) { return acc[nb][r]; });
}

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------
bool g4_shape(const DecodeArgs &a) {
  const bool pow2 = ((a.stride[0] & (a.stride[0] - 1)) | (a.stride[1] & (a.stride[1] - 1))) == 0;
  return a.G <= kG4 && pow2 && a.stride[0] >= 4 && a.stride[1] >= 4;
}

bool g4_supported(const DecodeArgs &a) { return g4_shape(a) && mfma_supported(a); }

int64_t g4_resident() {
  return resident_workgroups(reinterpret_cast<const void *>(decode_g4_kernel<true>), kThreadsMfma,
                             kSlotG4);
}

// Uniform batches (one length bound, or one sequence) take the grid plan
// unless the balanced partition gives its busiest workgroup fewer units;
// per-sequence lengths always take the balanced partition.  Both plan one
// resident generation of workgroups.  Balanced: P workgroups per kv head
// (never more than the batch has units), and a sequence spans at most
// balanced_slots(P, max_T) of them, the partial slots per sequence.
int launch_decode_g4(DecodeArgs &a, void *workspace, size_t ws_bytes, hipStream_t stream) {
  a.chunk_heads = kG4;
  a.n_chunks = 1;
  const int64_t resident = g4_resident();
  const int64_t n_max = units_of(a.max_T);
  int64_t P = std::max((int64_t)1, resident / a.H);
  P = std::min(P, (int64_t)a.B * n_max);
  bool balanced = a.seq_lens && a.B > 1;
  if (!balanced) {
    const SplitPlan g = plan_splits((int64_t)a.B * a.H, a.max_T, resident);
    const int64_t grid_units = g.split_len / kUnit;
    const int64_t bal_units = ((int64_t)a.B * n_max + P - 1) / P;
    if (bal_units < grid_units && !split_tokens_override()) {
      balanced = true;
    } else {
      a.nsplit = g.nsplit;
      a.split_len = g.split_len;
    }
  }
  if (balanced) {
    // unit indices are 32-bit in the kernel
    if ((int64_t)a.B * n_max >= ((int64_t)1 << 31)) return CQ_ERR_UNSUPPORTED;
    a.nsplit = (int)balanced_slots(P, a.max_T);
    a.split_len = kUnit;
  }
  int st = setup_workspace(a, workspace, ws_bytes);
  if (st) return st;
  // Fold records: every split waits for the others, so the grid must be one
  // resident generation; a folder's lanes hold up to 64 splits.
  const int64_t slots = (int64_t)a.B * a.H * a.nsplit;
  if (!balanced && a.nsplit > 1 && a.nsplit <= 64 && slots <= kMaxRecSplits && slots <= resident)
    a.recs = records_of(workspace);
  const bool dense_v = a.fbits[1] == 3;  // (K rows are INT4: mfma_supported)
  if (balanced) {
    const dim3 grid((unsigned)P, (unsigned)a.H, 1u);
    if (dense_v) decode_g4_kernel<true, false, true><<<grid, dim3(kThreadsMfma), 0, stream>>>(a);
    else decode_g4_kernel<true><<<grid, dim3(kThreadsMfma), 0, stream>>>(a);
  } else {
    const dim3 grid((unsigned)a.nsplit, (unsigned)a.H, (unsigned)a.B);
    if (dense_v)
      decode_g4_kernel<false, false, true><<<grid, dim3(kThreadsMfma), 0, stream>>>(a);
    else if (a.split_len <= (int64_t)kWaves * kChunk)
      decode_g4_kernel<false, true><<<grid, dim3(kThreadsMfma), 0, stream>>>(a);
    else
      decode_g4_kernel<false><<<grid, dim3(kThreadsMfma), 0, stream>>>(a);
  }
  return hipGetLastError() == hipSuccess ? CQ_OK : CQ_ERR_LAUNCH;
}

bool fp16_g4_supported(const DecodeArgs &a) {
  return a.D == kD && a.G <= kG4 && a.q_dtype == CQ_F16 && a.max_T < (1 << 24) &&
         a.cap_kf[0] * kD * 2 < ((int64_t)1 << 31) && a.cap_kf[1] * kD * 2 < ((int64_t)1 << 31) &&
         (((uintptr_t)a.kf[0] | (uintptr_t)a.kf[1] | (uintptr_t)a.q) & 15u) == 0;
}

int64_t fp16_g4_resident() {
  return resident_workgroups(reinterpret_cast<const void *>(decode_fp16_g4_kernel), kThreadsMfma,
                             kSlotFp16G4);
}

// Grid plan of one resident generation, fold records when the split slots
// fit them (as launch_decode_g4's grid plan).
int launch_decode_fp16_g4(DecodeArgs &a, void *workspace, size_t ws_bytes, hipStream_t stream) {
  a.chunk_heads = kG4;
  a.n_chunks = 1;
  const int64_t resident = fp16_g4_resident();
  const SplitPlan g = plan_splits((int64_t)a.B * a.H, a.max_T, resident);
  a.nsplit = g.nsplit;
  a.split_len = g.split_len;
  int st = setup_workspace(a, workspace, ws_bytes);
  if (st) return st;
  const int64_t slots = (int64_t)a.B * a.H * a.nsplit;
  if (a.nsplit > 1 && a.nsplit <= 64 && slots <= kMaxRecSplits && slots <= resident)
    a.recs = records_of(workspace);
  const dim3 grid((unsigned)a.nsplit, (unsigned)a.H, (unsigned)a.B);
  decode_fp16_g4_kernel<<<grid, dim3(kThreadsMfma), 0, stream>>>(a);
  return hipGetLastError() == hipSuccess ? CQ_OK : CQ_ERR_LAUNCH;
}

}  // namespace cq
