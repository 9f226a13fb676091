// cq_decode_mfma.hip — gfx950 MFMA split-K decode over the ChronoQuant cache
// (head_dim 128, fp16 queries, strides >= 4, any GQA ratio in chunks of 16 q
// heads), and a plain fp16 MFMA flash decode used as the uncompressed baseline.
//
// Reference semantics: the fused Metal kernel (kernels.py:79-228) — scores
// q'.(a + c*s) with q' = fp16(q*fp16(scale)), softmax, sum_t p_t (a + c*s).
// The contraction is factored so that both products are MFMA tiles:
//   score_t = q'.a_g(t) + s_t * (q'.c_t)
//   out     = sum_g P_g a_g + sum_t (p_t s_t) c_t,   P_g = sum_{t in g} p_t
// * q'.c_t: A = 16 tokens x 32 code nibbles, B = q'^T, v_mfma_f32_16x16x32_f16.
//   A nibble n enters as the fp16 denormal n * 2^-24 (one AND per pair; the
//   gfx950 MFMA takes fp16 denormals exactly), so q'.n is exact up to fp32
//   summation and q'.c = 2^24 * raw - 8 * sum(q').  q'.a: the same with 16
//   K anchor rows as A, kept in a per-wave LDS table.
// * The score tile's output layout (lane = q head, 4 consecutive tokens) is
//   the A- and the B-operand layout of the MFMA K index, and two 16-token
//   tiles fill one K=32 product (gfx950 issues v_mfma_f32_16x16x32_f16 at the
//   cost of the 16x16x16 form, so every product here is K=32):
//   - (p*s) against the V codes, nibbles as fp16 1024+n (even dims) or
//     1024+16n (odd dims, weighted by p*s/16), the constants removed at the
//     end with sum(p s) and sum(p s / 16);
//   - P_g^T = E^T p^T with E the 0/1 token->group matrix, accumulated over a
//     64-token chunk, then P_g (an fp16 hi/lo pair in one K=32 operand)
//     against the V anchors.
//   Code and anchor terms share one fp32 accumulator tile per 16 dims.
// Softmax in the log2 domain with a lazy running max per 64-token chunk
// (rescale only when the chunk max exceeds it by more than 2^8), so the fp16
// weights stay <= 256.
//
// Memory: each wave owns 64-token chunks of its split.  Per chunk it issues
// every load (scales, K code rows, V code words, K and V anchor rows) before
// the first wait; code rows of I-frames and padding use offsets past the
// buffer, which buffer loads return as 0.  Workgroups are 8 waves, so a split
// is 512 tokens.
#include <hip/hip_runtime.h>
#include <math.h>

#include <algorithm>

#include "cq_mfma_common.h"

namespace cq {

// Per-wave LDS.  The token tables of two chunks are live at once (the one
// being computed and the one whose loads are in flight): index [buffer].
struct alignas(16) WaveScratch {
  int slot_k[kChunk], slot_v[kChunk];  // P-frame slot (-1: I-frame / padding), staging only
  int gkl[2][kChunk], gvl[2][kChunk];  // anchor index relative to the chunk's first
  uint32_t s16[2][kChunk];             // fp16 K scale | fp16 V scale << 16 (0: none)
  float qa[16][kHeads];                // q'.anchor_k by (local anchor, head)
};

// The registers one chunk's loads land in (the V anchor rows, used last, are
// single-buffered and reloaded right after their use).
struct ChunkBuf {
  uint4 ka[4];        // K anchor row gk_base + col, dims 32kg + 8kb .. +7
  uint4 kw[4];        // K code words 4kg..4kg+3 of token 16i + col
  uint32_t vw[4][4];  // V code word col of token 16i + 4kg + r
  int nt;             // valid tokens (0: nothing to compute)
};

union DecodeLds {
  WaveScratch w[kWaves];
  MergeScratch mg;
};

// ---------------------------------------------------------------------------
// compressed cache
// ---------------------------------------------------------------------------
// Pow2: both strides are powers of two, so token -> anchor / slot arithmetic
// is shifts and masks instead of the float-reciprocal division.
// kBalanced = false: grid plan, workgroup (split, column, sequence) takes
// tokens [split * split_len, +split_len) of one sequence.  kBalanced = true:
// the balanced partition of the batch's units (cq_plan.h) over the P
// workgroups of each (kv head, q-head chunk) column, one or more segments
// per workgroup, with the loop state in LDS exactly as in the GQA-4 kernel
// (cq_decode_g4.hip), including its two register-pressure remedies.
template <bool Pow2, bool kBalanced>
__global__ __launch_bounds__(kThreadsMfma) void decode_mfma_kernel(DecodeArgs a) {
  __shared__ DecodeLds lds;
  __shared__ int32_t s_units[kBalanced ? kMaxTableSeqs + 1 : 1];
  __shared__ int32_t s_loop[8];  // cursor unit [2], cursor sequence [2], end unit, P, n
  prefetch_args();
  const int h = blockIdx.y / a.n_chunks;
  const int chunk = blockIdx.y - h * a.n_chunks;
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
    const int tid = kBalanced ? thread_id() : (int)threadIdx.x;
    __builtin_assume(tid >= 0 && tid < kThreadsMfma);
    // (the wave index in a scalar register: the chunk loop's bounds derive
    // from it, so its branches are uniform)
    const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int col = lane & 15;  // q head (operand column) / 16-dim output column
    const int kg = lane >> 4;   // K group of the MFMA operands
    const int j0 = chunk * kHeads;
    const int gn = min(kHeads, a.G - j0);
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
      const int64_t u_next = segment_at(us, blockIdx.x, __builtin_amdgcn_readfirstlane(sl[5]), u, b,
                                        seq_len_of(a, b), sg);
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
    const int sk = a.stride[0], sv = a.stride[1];
    const float isk = a.inv_stride[0], isv = a.inv_stride[1];
    const int lsk = Pow2 ? __builtin_ctz(sk) : 0, lsv = Pow2 ? __builtin_ctz(sv) : 0;
    auto div_k = [&](int t) { return Pow2 ? t >> lsk : div_stride(t, sk, isk); };
    auto div_v = [&](int t) { return Pow2 ? t >> lsv : div_stride(t, sv, isv); };

    const __amdgpu_buffer_rsrc_t r_kfk =
        make_rsrc(a.kf[0] + bh * a.cap_kf[0] * kD, (uint32_t)(a.cap_kf[0] * kD * 2));
    const __amdgpu_buffer_rsrc_t r_kfv =
        make_rsrc(a.kf[1] + bh * a.cap_kf[1] * kD, (uint32_t)(a.cap_kf[1] * kD * 2));
    const __amdgpu_buffer_rsrc_t r_pkk =
        make_rsrc(a.pk[0] + bh * a.cap_pf[0] * 16, (uint32_t)(a.cap_pf[0] * 64));
    const __amdgpu_buffer_rsrc_t r_pkv =
        make_rsrc(a.pk[1] + bh * a.cap_pf[1] * 16, (uint32_t)(a.cap_pf[1] * 64));
    const __amdgpu_buffer_rsrc_t r_sck = make_rsrc(a.sc[0] + bh * a.cap_pf[0], (uint32_t)(a.cap_pf[0] * 2));
    const __amdgpu_buffer_rsrc_t r_scv = make_rsrc(a.sc[1] + bh * a.cap_pf[1], (uint32_t)(a.cap_pf[1] * 2));

    // raw q rows of head col, dims 32kg .. 32kg+31 (converted after the first
    // chunk's loads are issued, so the two round trips overlap)
    const bool qok = col < gn;
    uint4 qraw[4];
    {
      const uint16_t *qrow =
          (const uint16_t *)a.q + ((int64_t)b * a.nq + h * a.G + j0 + (qok ? col : 0)) * kD + 32 * kg;
#pragma unroll
      for (int kb = 0; kb < 4; ++kb) qraw[kb] = *(const uint4 *)(qrow + 8 * kb);
    }
    uint32_t magic;  // fp16 1024 in both halves, held in a VGPR for v_and_or_b32
    asm volatile("v_mov_b32 %0, 0x64006400" : "=v"(magic));

    float m_run = -INFINITY;  // per head col, log2 units
    float l_run = 0.f;        // sum of fp16 p over this lane's tokens
    float w_run = 0.f;        // sum of fp16 p*s_v
    float w16_run = 0.f;      // sum of fp16 p*s_v/16
    f4_t acc[8];
#pragma unroll
    for (int nb = 0; nb < 8; ++nb) acc[nb] = f4_t{0.f, 0.f, 0.f, 0.f};
    const h2_t ones = {(_Float16)1.f, (_Float16)1.f};
    const h2_t sixteenth = {(_Float16)0.0625f, (_Float16)0.0625f};

    WaveScratch &W = lds.w[wave];
    // Stage the chunk at c0 into cb and token-table buffer sl: token table to
    // LDS, then every load of the chunk.  A chunk past the end (nt = 0) gets
    // offsets past every buffer, so its loads return zeros without traffic.
    auto stage = [&](int c0, ChunkBuf &cb, int sl) {
      const int nt = (int)max((int64_t)0, min((int64_t)kChunk, t1 - c0));
      cb.nt = nt;
      const int gk_base = div_k(c0);
      const int gk_last = nt ? div_k(c0 + nt - 1) : gk_base;
      const int gv_base = div_v(c0);
      // anchor offsets stay below 2^30; buffers are below 2^31 bytes (mfma_supported)
      const uint32_t dead = nt ? 0u : 0x80000000u;
      // token phase: one token per lane; scale loads first
      uint32_t s16;
      {
        const bool valid = lane < nt;
        const int t = c0 + (valid ? lane : max(nt - 1, 0));
        const int gk = div_k(t), gv = div_v(t);
        const int slk = (valid && t != gk * sk) ? t - gk - 1 : -1;
        const int slv = (valid && t != gv * sv) ? t - gv - 1 : -1;
        // slot -1 reads past the buffer: 0 (no scale)
        const uint32_t sk16 = bload16(r_sck, (uint32_t)slk * 2u);
        const uint32_t sv16 = bload16(r_scv, (uint32_t)slv * 2u);
        W.slot_k[lane] = slk;
        W.slot_v[lane] = slv;
        W.gkl[sl][lane] = gk - gk_base;
        W.gvl[sl][lane] = gv - gv_base;
        s16 = sk16 | (sv16 << 16);
      }
      wave_lds_sync();
      {
        const uint32_t row = ((uint32_t)min(gk_base + col, gk_last) * 256u + 64u * kg) | dead;
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) cb.ka[kb] = bload128(r_kfk, row + 16u * kb);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int slot = W.slot_k[16 * i + col];
        cb.kw[i] = bload128(r_pkk, (uint32_t)slot * 64u + 16u * kg);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int4 sl4 = *(const int4 *)&W.slot_v[16 * i + 4 * kg];
        cb.vw[i][0] = bload32(r_pkv, (uint32_t)sl4.x * 64u + 4u * col);
        cb.vw[i][1] = bload32(r_pkv, (uint32_t)sl4.y * 64u + 4u * col);
        cb.vw[i][2] = bload32(r_pkv, (uint32_t)sl4.z * 64u + 4u * col);
        cb.vw[i][3] = bload32(r_pkv, (uint32_t)sl4.w * 64u + 4u * col);
      }
      W.s16[sl][lane] = s16;
    };
    // V anchor rows gv_base + 4kg + r of the chunk at c0, dims 8col .. 8col+7.
    // (balanced plan: the pipeline registers are zero-initialised; left
    // undefined on a segment without work, they would be carried from the
    // previous segment and stay live across the whole body)
    uint4 va[4];
    if constexpr (kBalanced) va[0] = va[1] = va[2] = va[3] = uint4{0u, 0u, 0u, 0u};
    auto stage_va = [&](int c0) {
      const int nt = (int)max((int64_t)0, min((int64_t)kChunk, t1 - c0));
      const int gv_base = div_v(c0);
      const int gv_last = nt ? div_v(c0 + nt - 1) : gv_base;
      const uint32_t dead = nt ? 0u : 0x80000000u;
#pragma unroll
      for (int r = 0; r < 4; ++r)
        va[r] = bload128(r_kfv, ((uint32_t)min(gv_base + 4 * kg + r, gv_last) * 256u + 16u * col) | dead);
    };

    // q'^T operand in the K order (dims 32kg + 8kb + {0,4,1,5,2,6,3,7}); columns
    // >= gn are zero.  s8 = 8 * sum_d q'_d of head col.
    h8_t qc[4];
    float s8 = 0.f;
    auto prep_q = [&]() {
      const _Float16 sc16 = qok ? (_Float16)a.scale : (_Float16)0.f;
      const float scb = qok ? bf16_round(a.scale) : 0.f;
      const bool bf = a.q_dtype == CQ_BF16;
      float qs = 0.f;
#pragma unroll
      for (int kb = 0; kb < 4; ++kb) {
        // fp16 q: fp16(q * fp16(scale)); bf16 q: bf16(q * bf16(scale)) as fp16
        const h8_t v = bf ? bf16x8_scaled_to_f16(qraw[kb], scb)
                          : __builtin_bit_cast(h8_t, qraw[kb]) * sc16;
        qc[kb] = h8_t{v[0], v[4], v[1], v[5], v[2], v[6], v[3], v[7]};
#pragma unroll
        for (int e = 0; e < 8; ++e) qs += (float)v[e];
      }
      s8 = 8.f * shfl_sum_kg(qs);
    };

    // Compute the chunk staged in cb / token-table buffer sl.
    auto compute = [&](ChunkBuf &cb, int sl) {
      // ---- q'.anchor table (anchor gk_base + 4kg + r, head col) ---------------------
      {
        f4_t d = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) d = mfma32(korder(cb.ka[kb]), qc[kb], d);
#pragma unroll
        for (int r = 0; r < 4; ++r) W.qa[4 * kg + r][col] = d[r];
      }
      wave_lds_sync();

      // ---- scores of the 4 tiles (tokens 16i + 4kg + r, head col) ----------------
      float sc[4][4];
      float mx = -INFINITY;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        f4_t d = {0.f, 0.f, 0.f, 0.f};
        d = mfma32(unpack_k(cb.kw[i].x), qc[0], d);
        d = mfma32(unpack_k(cb.kw[i].y), qc[1], d);
        d = mfma32(unpack_k(cb.kw[i].z), qc[2], d);
        d = mfma32(unpack_k(cb.kw[i].w), qc[3], d);
        const int tb = 16 * i + 4 * kg;
        const int4 g4 = *(const int4 *)&W.gkl[sl][tb];
        const uint4 s4 = *(const uint4 *)&W.s16[sl][tb];
        const int gr[4] = {g4.x, g4.y, g4.z, g4.w};
        const uint32_t sr[4] = {s4.x, s4.y, s4.z, s4.w};
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float qa = W.qa[gr[r]][col];
          const float qdotc = __builtin_fmaf(d[r], kTwo24, -s8);  // q'.c
          const float skr = (float)as_h2(sr[r]).x;
          sc[i][r] = __builtin_fmaf(skr, qdotc, qa) * kLog2e;
        }
      }
      // Tokens past the end exist only in a split's last chunk (a uniform
      // branch).  Columns of q heads >= gn are not masked: their q' is zero,
      // their scores finite, and their rows of acc / l are never read.
      if (cb.nt < kChunk) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int r = 0; r < 4; ++r)
            if (16 * i + 4 * kg + r >= cb.nt) sc[i][r] = -INFINITY;
      }
#pragma unroll
      for (int i = 0; i < 4; ++i)
        mx = fmaxf(mx, fmaxf(fmaxf(sc[i][0], sc[i][1]), fmaxf(sc[i][2], sc[i][3])));

      // ---- lazy running max for the chunk ------------------------------------------
      mx = shfl_max_kg(mx);
      if (__any(mx > m_run + kTau)) {
        const float m_new = fmaxf(m_run, mx);
        const float f = (m_run == -INFINITY) ? 0.f : fast_exp2(m_run - m_new);
        l_run *= f;
        w_run *= f;
        w16_run *= f;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float fr = __shfl(f, 4 * kg + r, 64);  // factor of head 4kg + r
#pragma unroll
          for (int nb = 0; nb < 8; ++nb) acc[nb][r] *= fr;
        }
        m_run = m_new;
      }
      const float mref = (m_run == -INFINITY) ? 0.f : m_run;  // masked heads: scores are -inf

      // ---- weights, P_g and code P.V, two 16-token tiles per K=32 product ------------
      // K index 8kg + e of the products below is token 16(2P) + 4kg + e (e < 4)
      // or 16(2P+1) + 4kg + e - 4 (e >= 4): the 4 tokens the score tile gave
      // this lane group in each of the two tiles.
      f4_t pg = {0.f, 0.f, 0.f, 0.f};  // P_g^T: lane holds groups 4kg+r, head col
#pragma unroll
      for (int P = 0; P < 2; ++P) {
        h2_t pp[2][2], ww[2][2], xx[2][2];
        uint32_t ee[2][2];
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          const int i = 2 * P + u;
          const int tb = 16 * i + 4 * kg;
          const uint4 s4 = *(const uint4 *)&W.s16[sl][tb];
          const int4 g4 = *(const int4 *)&W.gvl[sl][tb];
          // p (fp16), p*s_v and p*s_v/16 (fp16 products)
          const h2_t p01 = h2_t{(_Float16)fast_exp2(sc[i][0] - mref), (_Float16)fast_exp2(sc[i][1] - mref)};
          const h2_t p23 = h2_t{(_Float16)fast_exp2(sc[i][2] - mref), (_Float16)fast_exp2(sc[i][3] - mref)};
          const h2_t sv01 = as_h2(__builtin_amdgcn_perm(s4.y, s4.x, 0x07060302u));
          const h2_t sv23 = as_h2(__builtin_amdgcn_perm(s4.w, s4.z, 0x07060302u));
          const h2_t w01 = p01 * sv01, w23 = p23 * sv23;
          const h2_t x01 = w01 * sixteenth, x23 = w23 * sixteenth;
          l_run = __builtin_amdgcn_fdot2(p01, ones, l_run, false);
          l_run = __builtin_amdgcn_fdot2(p23, ones, l_run, false);
          w_run = __builtin_amdgcn_fdot2(w01, ones, w_run, false);
          w_run = __builtin_amdgcn_fdot2(w23, ones, w_run, false);
          w16_run = __builtin_amdgcn_fdot2(x01, ones, w16_run, false);
          w16_run = __builtin_amdgcn_fdot2(x23, ones, w16_run, false);
          pp[u][0] = p01, pp[u][1] = p23;
          ww[u][0] = w01, ww[u][1] = w23;
          xx[u][0] = x01, xx[u][1] = x23;
          // E^T: group col x these tokens (fp16 1.0 = 0x3c00)
          ee[u][0] = (g4.x == col ? 0x3c00u : 0u) | (g4.y == col ? 0x3c000000u : 0u);
          ee[u][1] = (g4.z == col ? 0x3c00u : 0u) | (g4.w == col ? 0x3c000000u : 0u);
        }
        const h8_t ap = h8_t{pp[0][0].x, pp[0][0].y, pp[0][1].x, pp[0][1].y,
                             pp[1][0].x, pp[1][0].y, pp[1][1].x, pp[1][1].y};
        const h8_t aw = h8_t{ww[0][0].x, ww[0][0].y, ww[0][1].x, ww[0][1].y,
                             ww[1][0].x, ww[1][0].y, ww[1][1].x, ww[1][1].y};
        const h8_t ax = h8_t{xx[0][0].x, xx[0][0].y, xx[0][1].x, xx[0][1].y,
                             xx[1][0].x, xx[1][0].y, xx[1][1].x, xx[1][1].y};
        pg = mfma32(h8_of(ee[0][0], ee[0][1], ee[1][0], ee[1][1]), ap, pg);
        // V codes: B = 8 tokens x dim 8col + nb (nibble nb of word col)
        const int i0 = 2 * P, i1 = 2 * P + 1;
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

      // ---- anchor term: P_g as an fp16 hi/lo pair in one K=32 product ---------------
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
    // chunk is computed (two register buffers, unrolled by two).  The wave's
    // n >= 1 chunks c0l, c0l + kStep, ... below t1 run in pairs and one last
    // single chunk, so that the loop has one exit, at its end (an exit between
    // the two halves joins the loop header with the first half's loads in
    // flight, and the header then waits for all of them).  The last pair's V
    // anchor loads are dead (offsets past the buffer, no memory access).
    int64_t c0l = t0 + (int64_t)wave * kChunk;
    if (c0l < t1) {
      constexpr int64_t kStep = (int64_t)kWaves * kChunk;
      ChunkBuf bufA, bufB;
      if constexpr (kBalanced) bufA = bufB = ChunkBuf{};
      stage((int)c0l, bufA, 0);
      stage_va((int)c0l);
      prep_q();
      int n = __builtin_amdgcn_readfirstlane((int)((t1 - c0l + kStep - 1) / kStep));
      for (; n > 1; n -= 2) {
        stage((int)(c0l + kStep), bufB, 1);
        compute(bufA, 0);
        c0l += kStep;
        stage_va((int)c0l);
        stage((int)(c0l + kStep), bufA, 0);
        compute(bufB, 1);
        c0l += kStep;
        stage_va((int)c0l);
      }
      if (n) compute(bufA, 0);
    }

    // ---- totals: the 4 lane groups of a column hold disjoint tokens ---------------
    l_run = shfl_sum_kg(l_run);
    w_run = shfl_sum_kg(w_run);
    w16_run = shfl_sum_kg(w16_run);
    float sw[4], sw16[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      sw[r] = __shfl(w_run, 4 * kg + r, 64);
      sw16[r] = __shfl(w16_run, 4 * kg + r, 64);
    }
    // code columns: x = 1032 + c (even nb, weight p s) or 1152 + 16c (odd nb,
    // weight p s / 16): subtract the constant parts
    merge_and_finish(a, lds.mg, b, h, chunk, j0, gn, slot, live, m_run, l_run,
                     [&](int nb, int r) {
      const float corr = (nb & 1) ? 1024.f * sw16[r] + 8.f * sw[r] : 1032.f * sw[r];
      return acc[nb][r] - corr;
    });
    if constexpr (!kBalanced) return;
    __syncthreads();  // the next segment's staging reuses the merge area
  }
}

// ---------------------------------------------------------------------------
// plain fp16 cache (the uncompressed flash-decode baseline): K, V [cap][128]
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(kThreadsMfma) void decode_plain_kernel(DecodeArgs a) {
  __shared__ DecodeLds lds;
  prefetch_args();
  const int split = blockIdx.x;
  const int h = blockIdx.y / a.n_chunks;
  const int chunk = blockIdx.y - h * a.n_chunks;
  const int b = blockIdx.z;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int col = lane & 15, kg = lane >> 4;
  const int j0 = chunk * kHeads;
  const int gn = min(kHeads, a.G - j0);
  const int64_t bh = (int64_t)b * a.H + h;
  const int64_t T = seq_len_of(a, b);
  const int64_t t0 = (int64_t)split * a.split_len;
  const int64_t t1 = min(T, t0 + a.split_len);
  if (split_is_empty(split, t0, T)) return;
  const __amdgpu_buffer_rsrc_t r_k =
      make_rsrc(a.kf[0] + bh * a.cap_kf[0] * kD, (uint32_t)(a.cap_kf[0] * kD * 2));
  const __amdgpu_buffer_rsrc_t r_v =
      make_rsrc(a.kf[1] + bh * a.cap_kf[1] * kD, (uint32_t)(a.cap_kf[1] * kD * 2));

  // q'^T in natural order: dims 32kb + 8kg + e
  h8_t qn[4];
  {
    const bool qok = col < gn;
    const _Float16 sc16 = qok ? (_Float16)a.scale : (_Float16)0.f;
    const uint16_t *qrow =
        (const uint16_t *)a.q + ((int64_t)b * a.nq + h * a.G + j0 + (qok ? col : 0)) * kD + 8 * kg;
    uint4 u[4];
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) u[kb] = *(const uint4 *)(qrow + 32 * kb);
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) qn[kb] = __builtin_bit_cast(h8_t, u[kb]) * sc16;
  }

  float m_run = -INFINITY, l_run = 0.f;
  f4_t acc[8];
#pragma unroll
  for (int nb = 0; nb < 8; ++nb) acc[nb] = f4_t{0.f, 0.f, 0.f, 0.f};
  const h2_t ones = {(_Float16)1.f, (_Float16)1.f};

  for (int64_t c0l = t0 + (int64_t)wave * kChunk; c0l < t1; c0l += kWaves * kChunk) {
    const int c0 = (int)c0l;
    const int nt = (int)min((int64_t)kChunk, t1 - c0l);
    // K rows 16i + col (dims 32kb + 8kg) and V rows 16i + 4kg + r (dims 8col)
    uint4 kr[4][4], vr[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t row = (uint32_t)min(c0 + 16 * i + col, c0 + nt - 1);
#pragma unroll
      for (int kb = 0; kb < 4; ++kb) kr[i][kb] = bload128(r_k, row * 256u + 64u * kb + 16u * kg);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const uint32_t row = (uint32_t)min(c0 + 16 * i + 4 * kg + r, c0 + nt - 1);
        vr[i][r] = bload128(r_v, row * 256u + 16u * col);
      }
    float sc[4][4];
    float mx = -INFINITY;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      f4_t d = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kb = 0; kb < 4; ++kb) d = mfma32(__builtin_bit_cast(h8_t, kr[i][kb]), qn[kb], d);
      const int tb = 16 * i + 4 * kg;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float pen = (tb + r < nt && col < gn) ? 0.f : -INFINITY;
        sc[i][r] = __builtin_fmaf(d[r], kLog2e, pen);
        mx = fmaxf(mx, sc[i][r]);
      }
    }
    mx = shfl_max_kg(mx);
    if (__any(mx > m_run + kTau)) {
      const float m_new = fmaxf(m_run, mx);
      const float f = (m_run == -INFINITY) ? 0.f : fast_exp2(m_run - m_new);
      l_run *= f;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float fr = __shfl(f, 4 * kg + r, 64);
#pragma unroll
        for (int nb = 0; nb < 8; ++nb) acc[nb][r] *= fr;
      }
      m_run = m_new;
    }
    const float mref = (m_run == -INFINITY) ? 0.f : m_run;
    // P.V with two 16-token tiles per K=32 product (K index 8kg + e: token
    // 16(2P) + 4kg + e for e < 4, 16(2P+1) + 4kg + e - 4 for e >= 4)
#pragma unroll
    for (int P = 0; P < 2; ++P) {
      h2_t pp[2][2];
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const int i = 2 * P + u;
        pp[u][0] = h2_t{(_Float16)fast_exp2(sc[i][0] - mref), (_Float16)fast_exp2(sc[i][1] - mref)};
        pp[u][1] = h2_t{(_Float16)fast_exp2(sc[i][2] - mref), (_Float16)fast_exp2(sc[i][3] - mref)};
        l_run = __builtin_amdgcn_fdot2(pp[u][0], ones, l_run, false);
        l_run = __builtin_amdgcn_fdot2(pp[u][1], ones, l_run, false);
      }
      const h8_t ap = h8_t{pp[0][0].x, pp[0][0].y, pp[0][1].x, pp[0][1].y,
                           pp[1][0].x, pp[1][0].y, pp[1][1].x, pp[1][1].y};
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const h4_t l0 = rows_operand(vr[2 * P], k, false), l1 = rows_operand(vr[2 * P + 1], k, false);
        const h4_t o0 = rows_operand(vr[2 * P], k, true), o1 = rows_operand(vr[2 * P + 1], k, true);
        acc[2 * k] = mfma32(ap, h8_t{l0[0], l0[1], l0[2], l0[3], l1[0], l1[1], l1[2], l1[3]}, acc[2 * k]);
        acc[2 * k + 1] =
            mfma32(ap, h8_t{o0[0], o0[1], o0[2], o0[3], o1[0], o1[1], o1[2], o1[3]}, acc[2 * k + 1]);
      }
    }
  }
  l_run = shfl_sum_kg(l_run);
  merge_and_finish(a, lds.mg, b, h, chunk, j0, gn, split, kGridLive, m_run, l_run,
                   [&](int nb, int r) { return acc[nb][r]; });
}

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------
static bool plain_mode(const DecodeArgs &a) { return a.stride[0] == 1 && a.stride[1] == 1; }

bool mfma_supported(const DecodeArgs &a) {
  if (a.D != kD) return false;
  // INT4 rows, or 3-bit dense V rows under the GQA-4 kernel's dense instance
  if (a.fbits[0] != 4 || (a.fbits[1] != 4 && !(a.fbits[1] == 3 && g4_shape(a))))
    return false;
  // compressed cache: fp16 or bf16 queries; fp16 baseline: fp16 queries
  if (a.q_dtype != CQ_F16 && !(a.q_dtype == CQ_BF16 && !plain_mode(a))) return false;
  if (a.max_T >= (1 << 24)) return false;
  // buffer resources address each (sequence, head) region with 32-bit offsets
  for (int i = 0; i < 2; ++i)
    if (a.cap_kf[i] * kD * 2 >= ((int64_t)1 << 31) || a.cap_pf[i] * 64 >= ((int64_t)1 << 31))
      return false;
  // one K and one V anchor tile per 64-token chunk
  if (!plain_mode(a) && (a.stride[0] < 4 || a.stride[1] < 4)) return false;
  const uintptr_t al = (uintptr_t)a.kf[0] | (uintptr_t)a.kf[1] | (uintptr_t)a.pk[0] |
                       (uintptr_t)a.pk[1] | (uintptr_t)a.q;
  return (al & 15u) == 0;
}

static int64_t resident_of(int slot) {
  const void *k =
      slot == kSlotPlain      ? reinterpret_cast<const void *>(decode_plain_kernel)
      : slot == kSlotMfmaPow2 ? reinterpret_cast<const void *>(decode_mfma_kernel<true, true>)
                              : reinterpret_cast<const void *>(decode_mfma_kernel<false, true>);
  return resident_workgroups(k, kThreadsMfma, slot);
}

int64_t mfma_max_resident() {
  return std::max(std::max(std::max(resident_of(kSlotPlain), g4_resident()), fp16_g4_resident()),
                  std::max(resident_of(kSlotMfmaPow2), resident_of(kSlotMfma)));
}

// The compressed cache takes the balanced partition for per-sequence lengths
// (B > 1) or when it gives the busiest workgroup fewer units than the grid
// plan, as in launch_decode_g4; the fp16 baseline always takes the grid plan.
int launch_decode_mfma(DecodeArgs &a, void *workspace, size_t ws_bytes, hipStream_t stream) {
  if (!plain_mode(a) && g4_supported(a)) return launch_decode_g4(a, workspace, ws_bytes, stream);
  const bool pow2 = ((a.stride[0] & (a.stride[0] - 1)) | (a.stride[1] & (a.stride[1] - 1))) == 0;
  const int slot = plain_mode(a) ? kSlotPlain : pow2 ? kSlotMfmaPow2 : kSlotMfma;
  const int64_t resident = resident_of(slot);
  a.chunk_heads = kHeads;
  a.n_chunks = (a.G + kHeads - 1) / kHeads;
  const int64_t cols = (int64_t)a.H * a.n_chunks;
  const int64_t n_max = units_of(a.max_T);
  int64_t P = std::min(std::max((int64_t)1, resident / cols), (int64_t)a.B * n_max);
  bool balanced = false;
  if (!plain_mode(a)) {
    const SplitPlan g = plan_splits((int64_t)a.B * cols, a.max_T, resident);
    const int64_t bal_units = ((int64_t)a.B * n_max + P - 1) / P;
    balanced = (a.seq_lens && a.B > 1) ||
               (bal_units < g.split_len / kUnit && !split_tokens_override());
    // unit indices are 32-bit in the kernel
    if (balanced && (int64_t)a.B * n_max >= ((int64_t)1 << 31)) balanced = false;
  }
  int st;
  if (balanced) {
    a.nsplit = (int)balanced_slots(P, a.max_T);
    a.split_len = kUnit;
    st = setup_workspace(a, workspace, ws_bytes);
  } else {
    st = prepare_launch(a, kHeads, resident, workspace, ws_bytes);
  }
  if (st) return st;
  const dim3 blk(kThreadsMfma);
  if (balanced) {
    const dim3 grid((unsigned)P, (unsigned)cols, 1u);
    if (pow2) decode_mfma_kernel<true, true><<<grid, blk, 0, stream>>>(a);
    else decode_mfma_kernel<false, true><<<grid, blk, 0, stream>>>(a);
  } else {
    const dim3 grid((unsigned)a.nsplit, (unsigned)cols, (unsigned)a.B);
    if (slot == kSlotPlain) decode_plain_kernel<<<grid, blk, 0, stream>>>(a);
    else if (pow2) decode_mfma_kernel<true, false><<<grid, blk, 0, stream>>>(a);
    else decode_mfma_kernel<false, false><<<grid, blk, 0, stream>>>(a);
  }
  return hipGetLastError() == hipSuccess ? CQ_OK : CQ_ERR_LAUNCH;
}

}  // namespace cq
