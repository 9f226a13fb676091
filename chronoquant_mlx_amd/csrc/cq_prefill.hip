// cq_prefill.hip — gfx950 chunked-prefill attention over the ChronoQuant cache
// (head_dim 128, fp16 or bf16 queries): the last n_q cached tokens of every sequence
// attend to the cache, causally or to all of it.
//
// Reference semantics: the reconstruct fallback of chronoquant_sdpa for
// q_len > 1 (attention.py:61-74 over cache.py:131-160): K and V rebuilt in
// fp16 as r = fp16(a + fp16(fp16(c) * s)), q' = fp16(q * fp16(scale)),
// scores rounded to fp16, causal mask q_idx >= k_idx (attention.py:12-16),
// softmax in fp32, fp16 weights against V, fp16 output.  Here the softmax is
// the online (flash) form, with the weights rounded to fp16 where they enter
// the P.V product.
//
// Workgroup = 16 waves = 256 query rows of one kv head: 256 / G positions x the
// G q heads of the group (row R: position p0 + R / G, head R % G), over one
// of nsplit contiguous pieces of its key range (split-K: without splits a
// chunk's grid is about one workgroup per CU, which leaves every load's
// latency exposed; splits give each CU several).  256 rows share each
// rebuilt block, so the rebuild costs a quarter of what it would for 64.
// Per 64-key block:
//   1. waves 0-7 rebuild the K block (row-major), waves 8-15 the V block
//      (transposed, dims x keys) in LDS with the reference's fp16 rounding;
//   2. each wave computes S^T = K . Q^T for its 16 rows (v_mfma_f32_16x16x32_f16,
//      4 key tiles x 4 K-steps), so a lane holds 16 scores of one row;
//   3. online softmax in the log2 domain (lazy rescale beyond 2^8);
//   4. O += P . V (8 dim tiles x 2 K-steps; two 16-key tiles per K=32 step).
// With several splits each workgroup writes its rows' unnormalised (m, l, o)
// to the workspace, and the last of a tile's splits to finish (a ticket on a
// per-(sequence, kv head, tile) counter) merges them by log-sum-exp, as the
// decode's split combine does.
#include <hip/hip_runtime.h>
#include <math.h>

#include <algorithm>

#include "cq_decode_common.h"

namespace cq {
namespace {

typedef _Float16 h2_t __attribute__((ext_vector_type(2)));
typedef _Float16 h4_t __attribute__((ext_vector_type(4)));
typedef _Float16 h8_t __attribute__((ext_vector_type(8)));
typedef float f4_t __attribute__((ext_vector_type(4)));
typedef int i4_t __attribute__((ext_vector_type(4)));

constexpr int kD = 128;
constexpr int kRows = 256;       // query rows per workgroup
constexpr int kKeys = 64;        // keys per block
constexpr int kThreads = 1024;   // 16 waves: 16 rows each
// K block row stride (fp16 elements): rows 72 dwords apart.  Measured on the
// c4 chunk against other paddings of the same block (136: 117.6-118.0 us,
// 144: 114.4-114.6, 152: 117.5-119.1, 160: 116.6-117.2, 168: 115.6-118.9).
constexpr int kKStride = kD + 16;
// V block row stride (fp16 elements).  Measured on the c4 chunk with the
// transpose-read P.V: 144: 104.6-105.1 us, 136: 106.4-106.7, 152:
// 106.4-107.0, 160: 108.6-109.0.
constexpr int kVStride = kD + 16;
constexpr float kTau = 8.f;

struct PrefillArgs {
  const uint16_t *kf[2];
  const uint32_t *pk[2];
  const uint16_t *sc[2];
  int64_t cap_kf[2], cap_pf[2];
  int stride[2];
  float inv_stride[2];
  int B, H, G, nq;
  int64_t n_q, T;
  int causal;
  float scale;
  const uint16_t *q;  // [B][nq][n_q][D] fp16 or bf16
  uint16_t *out;      // [B][nq][n_q][D], the dtype of q
  int nsplit, tiles;
  float *part_ml;      // [B][nq][n_q][nsplit][2]  (m in log2 units, l)
  float *part_acc;     // [B][nq][n_q][nsplit][D]  (real dim order)
  uint32_t *counters;  // [B][H][tiles]
};

// bf16 q' = bf16(q * bf16(scale)) (one rounding of the exact fp32 product),
// then fp16 for the MFMA operand (exact for |q'| in fp16's normal range).
__device__ __forceinline__ float bf16_round(float f) {
  uint32_t u = __float_as_uint(f);
  u += 0x7FFFu + ((u >> 16) & 1u);
  return __uint_as_float(u & 0xFFFF0000u);
}
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
  uint32_t u = __float_as_uint(f);
  u += 0x7FFFu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

__device__ __forceinline__ h2_t as_h2(uint32_t u) { return __builtin_bit_cast(h2_t, u); }
// Packed fp16 max of non-NaN pairs, without the canonicalising moves the
// compiler puts around v_pk_max_f16 in IEEE mode: the IEEE 754-2019 maximum,
// one v_pk_maximum3_f16 on gfx950.
__device__ __forceinline__ h2_t pk_max_nn(h2_t a, h2_t b) {
  return __builtin_elementwise_maximum(a, b);
}
__device__ __forceinline__ uint32_t as_u(h2_t h) { return __builtin_bit_cast(uint32_t, h); }
__device__ __forceinline__ h8_t h8_of(uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
  const h2_t x = as_h2(a), y = as_h2(b), z = as_h2(c), w = as_h2(d);
  return h8_t{x.x, x.y, y.x, y.y, z.x, z.y, w.x, w.y};
}
__device__ __forceinline__ f4_t mfma32(h8_t a, h8_t b, f4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ uint4 bload128(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  const i4_t v = __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 0);
  return uint4{(uint32_t)v[0], (uint32_t)v[1], (uint32_t)v[2], (uint32_t)v[3]};
}
__device__ __forceinline__ uint2 bload64(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  const __attribute__((ext_vector_type(2))) int v = __builtin_amdgcn_raw_buffer_load_b64(r, (int)off, 0, 0);
  return uint2{(uint32_t)v[0], (uint32_t)v[1]};
}
__device__ __forceinline__ uint32_t bload32(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(r, (int)off, 0, 0);
}
__device__ __forceinline__ uint32_t bload16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(r, (int)off, 0, 0);
}

// One code word (8 nibbles, dims 0..7 of a group) and the group's fp16
// anchor (a01, a23, a45, a67) -> the rebuilt fp16 values in dim order:
// fp16(a + fp16(fp16(n - 8) * s)).  The low and high nibbles of the bytes
// are interleaved into bytes n0 n1 n2 n3 / n4 n5 n6 n7, then a byte permute
// against the magic constant makes each nibble fp16 1024 + n; subtracting
// 1032 is exact.  Codes past the end of the cache read as 0 and the scale as
// 0, so c * s = -0 and an I-frame row is its anchor exactly.
__device__ __forceinline__ uint4 rebuild8(uint32_t cw, uint4 a, h2_t s2, uint32_t magic) {
  const uint32_t lo = cw & 0x0F0F0F0Fu, hi = (cw >> 4) & 0x0F0F0F0Fu;
  const uint32_t x0 = __builtin_amdgcn_perm(hi, lo, 0x05010400u);  // bytes n0 n1 n2 n3
  const uint32_t x1 = __builtin_amdgcn_perm(hi, lo, 0x07030602u);  // bytes n4 n5 n6 n7
  const h2_t bias = {(_Float16)-1032.f, (_Float16)-1032.f};
  const uint32_t sel_a = 0x07010500u, sel_b = 0x07030502u;  // bytes (0,1) / (2,3) of x
  const h2_t c01 = as_h2(__builtin_amdgcn_perm(magic, x0, sel_a)) + bias;
  const h2_t c23 = as_h2(__builtin_amdgcn_perm(magic, x0, sel_b)) + bias;
  const h2_t c45 = as_h2(__builtin_amdgcn_perm(magic, x1, sel_a)) + bias;
  const h2_t c67 = as_h2(__builtin_amdgcn_perm(magic, x1, sel_b)) + bias;
  return uint4{as_u(as_h2(a.x) + c01 * s2), as_u(as_h2(a.y) + c23 * s2),
               as_u(as_h2(a.z) + c45 * s2), as_u(as_h2(a.w) + c67 * s2)};
}

// LDS transpose read (gfx950 ds_read_b64_tr_b16): within each group of 16
// lanes, lane 4j + c addresses 4 fp16 (c: a 4-column slice of row j) and
// lane r of the group receives element r % 4 of lanes r / 4, r / 4 + 4,
// r / 4 + 8, r / 4 + 12 (checked on the device: rows j = 0..3 of the
// group's 4 x 16 tile come back as the 4 values of column r).
typedef short s4_t __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint2 lds_read_tr16(const uint16_t *p) {
  const s4_t v = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) s4_t *)(p));
  return __builtin_bit_cast(uint2, v);
}

// Two block buffers: block kb + 1 is rebuilt into one while block kb's
// products read the other, so each block needs one barrier.
struct alignas(16) PrefillLds {
  uint16_t k[2][kKeys][kKStride];  // K block, [key][dim]
  uint16_t v[2][kKeys][kVStride];  // V block, [key][dim]
};

// Split epilogue: this workgroup's rows' (m, l, o) go to the workspace with
// device-scope stores; the last of the tile's nsplit workgroups to take a
// ticket folds every row's partials by log-sum-exp, writes the output and
// resets the counter.  Row R of the tile is position p0 + R / G, head R % G;
// lane (col, kg) of wave w holds o of rows 16w + 4kg + r at dims 16dt + col,
// and m, l of row 16w + col.
template <bool Bf16>
__device__ __forceinline__ void split_epilogue(const PrefillArgs &a, int b, int h, int tile,
                                               int split, int64_t p0, float m_run, float l_run,
                                               const f4_t (&acc)[8]) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int col = lane & 15, kg = lane >> 4;
  const int G = a.G, ns = a.nsplit;
  const int64_t L = a.n_q;
  const int64_t rows = (int64_t)a.B * a.nq * L;  // global rows (host-bounded below 2^31 / (ns D 4))
  const __amdgpu_buffer_rsrc_t racc = make_rsrc(a.part_acc, (uint32_t)(rows * ns * kD * 4));
  const __amdgpu_buffer_rsrc_t rml = make_rsrc(a.part_ml, (uint32_t)(rows * ns * 8));
  auto grow = [&](int R) {  // global row of tile row R (valid position)
    return (((int64_t)b * a.nq + h * G + R % G) * L + p0 + R / G);
  };
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int R = 16 * wave + 4 * kg + r;
    if (p0 + R / G < L) {
      const uint32_t base = (uint32_t)((grow(R) * ns + split) * kD);
#pragma unroll
      for (int dt = 0; dt < 8; ++dt) {
        store_dev1(racc, 4u * (base + 16 * dt + col), acc[dt][r]);
      }
    }
  }
  {
    const int R = 16 * wave + col;
    if (kg == 0 && p0 + R / G < L)
      store_dev2(rml, (uint32_t)((grow(R) * ns + split) * 8), f2v_t{m_run, l_run});
  }
  __shared__ int s_last;
  __builtin_amdgcn_s_waitcnt(0);  // this thread's partial stores are complete
  __syncthreads();
  uint32_t *ctr = a.counters + ((int64_t)b * a.H + h) * a.tiles + tile;
  if (tid == 0) {
    const uint32_t prev = __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    s_last = (prev == (uint32_t)(ns - 1));
  }
  __syncthreads();
  if (!s_last) return;
  // fold: thread -> (row R, 4 real dims), all splits' loads issued before use
  for (int u = tid; u < kRows * (kD / 4); u += kThreads) {
    const int R = u / (kD / 4), d0 = 4 * (u % (kD / 4));
    if (p0 + R / G >= L) continue;
    const int64_t g = grow(R);
    float M = -INFINITY, Ls = 0.f, o0 = 0.f, o1 = 0.f, o2 = 0.f, o3 = 0.f;
    for (int s0 = 0; s0 < ns; s0 += 8) {
      f2v_t ml[8];
      f4v_t ov[8];
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const uint32_t sp = (uint32_t)(g * ns + min(s0 + k, ns - 1));
        ml[k] = load_dev2(rml, sp * 8u);
        ov[k] = load_dev4(racc, (sp * (uint32_t)kD + (uint32_t)d0) * 4u);
      }
      float mb = M;
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        if (s0 + k >= ns) ml[k].x = -INFINITY;
        mb = fmaxf(mb, ml[k].x);
      }
      const float mref = (mb == -INFINITY) ? 0.f : mb;
      const float f = (M == -INFINITY) ? 0.f : fast_exp2(M - mref);
      Ls *= f;
      o0 *= f;
      o1 *= f;
      o2 *= f;
      o3 *= f;
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const float w = (ml[k].x == -INFINITY) ? 0.f : fast_exp2(ml[k].x - mref);
        Ls += w * ml[k].y;
        o0 += w * ov[k].x;
        o1 += w * ov[k].y;
        o2 += w * ov[k].z;
        o3 += w * ov[k].w;
      }
      M = mb;
    }
    const float inv = Ls > 0.f ? 1.f / Ls : 0.f;
    uint16_t *orow = a.out + g * kD + d0;
    const float ov4[4] = {o0 * inv, o1 * inv, o2 * inv, o3 * inv};
    uint16_t hv[4];
#pragma unroll
    for (int c = 0; c < 4; ++c)
      hv[c] = Bf16 ? f32_to_bf16_bits(ov4[c]) : __builtin_bit_cast(uint16_t, (_Float16)ov4[c]);
    *(uint2 *)orow = uint2{(uint32_t)hv[0] | ((uint32_t)hv[1] << 16),
                           (uint32_t)hv[2] | ((uint32_t)hv[3] << 16)};
  }
  if (tid == 0) __hip_atomic_store(ctr, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Bf16: queries (and output) are bf16.  The reference then computes the
// scores in fp32 (bf16 x fp16 promotes), so they are not rounded to fp16.
// Pow2: both strides are powers of two (token -> anchor / slot by shifts).
// At most 128 VGPRs (4 waves per SIMD): the waves waiting on their block's
// loads overlap the others' products.  Keeping the next block's raw data in
// registers instead (a software prefetch) needs ~160 VGPRs and fewer waves,
// and measured slower (188 vs 167 us on the c4 chunk at 128 rows per
// workgroup).
template <bool Bf16, bool Pow2>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(4, 4)))
void prefill_mfma_kernel(PrefillArgs a) {
  __shared__ PrefillLds lds;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int col = lane & 15, kg = lane >> 4;
  const int h = blockIdx.y, b = blockIdx.z;
  const int split = (int)(blockIdx.x % (unsigned)a.nsplit);
  const int tile = (int)(blockIdx.x / (unsigned)a.nsplit);
  const int G = a.G, ppw = kRows / G;  // positions per workgroup
  const int64_t p0 = (int64_t)tile * ppw;
  const int64_t bh = (int64_t)b * a.H + h;
  const int T = (int)a.T;  // < 2^24 (host-checked)
  const int64_t L = a.n_q;
  const int qbase = T - (int)L;  // position of query 0

  // ---- Q fragment: row (16 wave + col), dims 32s + 8kg .. +7 of K-step s;
  // B operand of S^T = K . Q^T -------------------------------------------------
  const int my_row = 16 * wave + col;
  const int64_t my_pos = p0 + my_row / G;
  const int my_head = my_row % G;
  const bool my_valid = my_pos < L;
  h8_t qf[4];
  {
    const _Float16 sc16 = (_Float16)a.scale;
    const float scb = bf16_round(a.scale);
    const uint16_t *qrow = a.q + (((int64_t)b * a.nq + h * G + my_head) * L + (my_valid ? my_pos : 0)) * kD;
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const uint4 u = *(const uint4 *)(qrow + 32 * s + 8 * kg);  // dims 32s + 8kg .. +7
      h8_t v;
      if (Bf16) {
        const uint32_t w4[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          v[2 * i] = (_Float16)bf16_round(__uint_as_float(w4[i] << 16) * scb);
          v[2 * i + 1] = (_Float16)bf16_round(__uint_as_float(w4[i] & 0xFFFF0000u) * scb);
        }
      } else {
        v = __builtin_bit_cast(h8_t, u) * sc16;  // fp16(q * fp16(scale))
      }
      if (!my_valid) v = h8_t{};
      qf[s] = v;
    }
  }
  // causal limit of this lane's row (scores rows = lane col)
  const int lim = a.causal ? qbase + (int)my_pos : T - 1;
  // every key of a block at or below lim_all is visible to every row of the tile
  const int lim_all = a.causal ? qbase + (int)p0 : T - 1;

  float m_run = -INFINITY, l_run = 0.f;
  f4_t acc[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) acc[i] = f4_t{0.f, 0.f, 0.f, 0.f};

  const int64_t last_pos = min(p0 + ppw, L) - 1;
  const int key_end = a.causal ? qbase + (int)last_pos + 1 : T;  // keys [0, key_end)
  const int n_all = (key_end + kKeys - 1) / kKeys;
  // this split's blocks [kb_lo, kb_hi) of the tile's n_all (possibly none)
  const int kb_lo = split * n_all / a.nsplit, kb_hi = (split + 1) * n_all / a.nsplit;

  // Block staging: waves 0-7 load and rebuild the K block, waves 8-15 the V
  // block, so that each thread holds one component's raw data in registers.
  // Both blocks are row-major ([key][dim]); thread st (tid % 512) takes key
  // (st % 16) + 16 (st / 128), dims 16 ((st / 16) % 8) .. +15 (2 code
  // words): the lanes of one 16-byte LDS write phase are consecutive keys
  // (rows kKStride / 2 dwords apart).  The P.V product reads V's operand
  // columns with transpose reads.
  // the component is wave-uniform: keep it scalar, so that the buffer
  // resources below are too (per-lane resources put every load in a
  // compiler waterfall loop)
  const int c = __builtin_amdgcn_readfirstlane(tid < kThreads / 2 ? 0 : 1);
  const int st = tid & (kThreads / 2 - 1);
  const int stride = a.stride[c];
  const float istride = a.inv_stride[c];
  const int lstride = __builtin_ctz(stride), mstride = stride - 1;
  const __amdgpu_buffer_rsrc_t r_kf = make_rsrc(a.kf[c] + bh * a.cap_kf[c] * kD, (uint32_t)(a.cap_kf[c] * kD * 2));
  const __amdgpu_buffer_rsrc_t r_pk = make_rsrc(a.pk[c] + bh * a.cap_pf[c] * 16, (uint32_t)(a.cap_pf[c] * 64));
  const __amdgpu_buffer_rsrc_t r_sc = make_rsrc(a.sc[c] + bh * a.cap_pf[c], (uint32_t)(a.cap_pf[c] * 2));
  const int kkey = (st & 15) | ((st >> 7) << 4), ke = (st >> 4) & 7;
  uint32_t magic;  // fp16 1024 in both halves, an opaque VGPR for the byte permutes
  asm volatile("v_mov_b32 %0, 0x64006400" : "=v"(magic));
  uint32_t r_cw[2], r_s;  // code words 2ke, 2ke + 1 of key kkey, its scale
  uint4 r_an[2];          // its anchor row, dims 16 ke + 8j ..
  // token t -> anchor index g (-1 past the end) and P-frame slot (-1:
  // I-frame or past the end)
  auto locate = [&](int t, int &g, int &slot) {
    const bool in = t < T;
    if (Pow2) {
      g = t >> lstride;
      slot = (in && (t & mstride)) ? t - g - 1 : -1;
    } else {
      g = div_stride(t, stride, istride);
      slot = (in && t != g * stride) ? t - g - 1 : -1;
    }
    if (!in) g = -1;
  };
  // Staging offsets of key t = k0 + kkey: scale, code words, anchor row
  // (offsets past a buffer read zeros: slot -1 of an I-frame or past the
  // end, anchor -1 past the end).
  auto offsets_of = [&](int t, uint32_t &o_sc, uint32_t &o_cw, uint32_t &o_an) {
    int g, slot;
    locate(t, g, slot);
    o_an = g >= 0 ? (uint32_t)g * 256u + 32u * ke : 0x80000000u;
    o_sc = (uint32_t)slot * 2u;
    o_cw = (uint32_t)slot * 64u + 8u * ke;
  };
  // Blocks are staged in increasing order, 64 keys apart.  With a
  // power-of-two stride <= 64 a key's frame type is the same in every block
  // and its anchor and slot advance by fixed steps, so the offsets are kept
  // and stepped (one compare per block for the end of the cache) instead of
  // recomputed.
  const bool stepped = Pow2 && lstride <= 6;  // uniform
  const int g_step = 64 >> lstride;
  const bool pframe = (kkey & mstride) != 0;
  uint32_t s_sc = 0, s_cw = 0, s_an = 0;  // the next block's offsets (stepped)
  int s_t = 0;
  if (stepped && kb_lo < kb_hi) offsets_of(kb_lo * kKeys + kkey, s_sc, s_cw, s_an);
  s_t = kb_lo * kKeys + kkey;
  const uint32_t d_sc = pframe ? 2u * (uint32_t)(64 - g_step) : 0u;
  const uint32_t d_cw = pframe ? 64u * (uint32_t)(64 - g_step) : 0u;
  const uint32_t d_an = 256u * (uint32_t)g_step;
  auto load_block = [&](int k0) {
    uint32_t o_sc, o_cw, o_an;
    if (stepped) {
      const bool in = s_t < T;
      o_sc = in ? s_sc : 0x80000000u;
      o_cw = in ? s_cw : 0x80000000u;
      o_an = in ? s_an : 0x80000000u;
      s_t += kKeys;
      s_sc += d_sc;
      s_cw += d_cw;
      s_an += d_an;
    } else {
      offsets_of(k0 + kkey, o_sc, o_cw, o_an);
    }
    r_s = bload16(r_sc, o_sc);
    const uint2 cw = bload64(r_pk, o_cw);
    r_cw[0] = cw.x;
    r_cw[1] = cw.y;
#pragma unroll
    for (int j = 0; j < 2; ++j) r_an[j] = bload128(r_kf, o_an + 16u * j);
  };

  // ---- 1. rebuild the staged block: K (waves 0-7) or V (waves 8-15) into
  // LDS buffer `buf` --------------------------------------------------------------
  auto rebuild = [&](int buf) {
    const h2_t s2 = as_h2(r_s * 0x10001u);
    uint4 *dst = (uint4 *)(c == 0 ? &lds.k[buf][kkey][16 * ke] : &lds.v[buf][kkey][16 * ke]);
#pragma unroll
    for (int j = 0; j < 2; ++j) dst[j] = rebuild8(r_cw[j], r_an[j], s2, magic);
  };

  // Pipeline: while block kb's products read one LDS buffer, the waves
  // rebuild block kb + 1 (staged in registers during block kb - 1) into the
  // other and issue block kb + 2's loads; one barrier per block.
  if (kb_lo < kb_hi) {  // uniform
    load_block(kb_lo * kKeys);
    rebuild(0);
    if (kb_lo + 1 < kb_hi) load_block((kb_lo + 1) * kKeys);
  }
  __syncthreads();
  for (int kb = kb_lo; kb < kb_hi; ++kb) {
    const int k0 = kb * kKeys;
    const int cur = (kb - kb_lo) & 1;
    if (kb + 1 < kb_hi) {  // uniform
      rebuild(cur ^ 1);
      if (kb + 2 < kb_hi) load_block(k0 + 2 * kKeys);
    }

    // ---- 2. S^T = K . Q^T: lane (col = row, kg) gets keys 16t + 4kg + r ---------
    // Scores in natural units: the log2 scaling is folded into the
    // exponent's fma below, and the row max is scaled once (scaling by
    // log2 e > 0 keeps the max).  fp16 q: rounded to fp16 like the
    // fallback's fp16 matmul and kept packed (s2, two per register): the max
    // runs on the pairs and the exponent's fma reads an fp16 half directly.
    // bf16 q: fp32 (sc).
    float sc[4][4];
    h2_t s2[4][2];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      f4_t d = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const uint4 kv = *(const uint4 *)&lds.k[cur][16 * t + col][32 * s + 8 * kg];
        d = mfma32(__builtin_bit_cast(h8_t, kv), qf[s], d);
      }
#pragma unroll
      for (int r = 0; r < 4; r += 2) {
        if (Bf16) {
          sc[t][r] = d[r];
          sc[t][r + 1] = d[r + 1];
        } else {
          typedef float f2_t __attribute__((ext_vector_type(2)));
          s2[t][r >> 1] = __builtin_convertvector(f2_t{d[r], d[r + 1]}, h2_t);
        }
      }
    }
    // Keys past lim_all exist only in a tile's last blocks (a uniform branch).
    if (k0 + kKeys - 1 > lim_all) {
#pragma unroll
      for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int r = 0; r < 4; ++r)
          if (k0 + 16 * t + 4 * kg + r > lim) {
            if (Bf16)
              sc[t][r] = -INFINITY;
            else
              s2[t][r >> 1][r & 1] = (_Float16)-INFINITY;
          }
    }
    float mx;
    if (Bf16) {
      mx = -INFINITY;
#pragma unroll
      for (int t = 0; t < 4; ++t)
        mx = fmaxf(mx, fmaxf(fmaxf(sc[t][0], sc[t][1]), fmaxf(sc[t][2], sc[t][3])));
    } else {
      h2_t m2 = pk_max_nn(s2[0][0], s2[0][1]);
#pragma unroll
      for (int t = 1; t < 4; ++t) m2 = pk_max_nn(m2, pk_max_nn(s2[t][0], s2[t][1]));
      mx = max_nn((float)m2.x, (float)m2.y);
    }
    // ---- 3. online softmax (row max over the 4 lane groups of the column) -------
    mx = xor32_max(xor16_max(mx)) * kLog2e;  // log2 units, as m_run
    if (__any(mx > m_run + kTau)) {
      const float m_new = fmaxf(m_run, mx);
      const float f = (m_run == -INFINITY) ? 0.f : fast_exp2(m_run - m_new);
      l_run *= f;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float fr = __shfl(f, 4 * kg + r, 64);  // factor of row 4kg + r
#pragma unroll
        for (int i = 0; i < 8; ++i) acc[i][r] *= fr;
      }
      m_run = m_new;
    }
    const float mref = (m_run == -INFINITY) ? 0.f : m_run;
    const h2_t ones = {(_Float16)1.f, (_Float16)1.f};
    h2_t pp[4][2];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      // p = 2^(s log2 e - m) in one fma + exp; l sums the fp16 weights (the
      // values P.V uses) in fp32, two per v_dot2_f32_f16
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const float x0 = Bf16 ? sc[t][2 * u] : (float)s2[t][u].x;
        const float x1 = Bf16 ? sc[t][2 * u + 1] : (float)s2[t][u].y;
        pp[t][u] = h2_t{(_Float16)fast_exp2(__builtin_fmaf(x0, kLog2e, -mref)),
                        (_Float16)fast_exp2(__builtin_fmaf(x1, kLog2e, -mref))};
        l_run = __builtin_amdgcn_fdot2(pp[t][u], ones, l_run, false);
      }
    }
    // ---- 4. O += P . V: K index 8kg + e = key 16(2P) + 4kg + e (e < 4) or
    // 16(2P+1) + 4kg + e - 4.  B operand of dim tile dt: lane (n, kg) needs
    // V[those keys][16dt + n]; with the transpose read, lane 4j + c of
    // group kg addresses keys 32P + 4kg + j (+ 16), dims 16dt + 4c .. +3 --
#pragma unroll
    for (int P = 0; P < 2; ++P) {
      const h8_t ap = h8_of(as_u(pp[2 * P][0]), as_u(pp[2 * P][1]), as_u(pp[2 * P + 1][0]),
                            as_u(pp[2 * P + 1][1]));
      const uint16_t *vrow = &lds.v[cur][32 * P + 4 * kg + (col >> 2)][4 * (col & 3)];
#pragma unroll
      for (int dt = 0; dt < 8; ++dt) {
        const uint2 v0 = lds_read_tr16(vrow + 16 * dt);
        const uint2 v1 = lds_read_tr16(vrow + 16 * kVStride + 16 * dt);
        acc[dt] = mfma32(ap, h8_of(v0.x, v0.y, v1.x, v1.y), acc[dt]);
      }
    }
    __syncthreads();  // buffer cur is rebuilt next iteration
  }

  // ---- output: lane (col = dim 16dt + col, kg) holds rows 4kg + r ---------------
  l_run = xor32_sum(xor16_sum(l_run));
  if (a.nsplit > 1) {
    split_epilogue<Bf16>(a, b, h, tile, split, p0, m_run, l_run, acc);
    return;
  }
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int row = 16 * wave + 4 * kg + r;
    const int64_t pos = p0 + row / G;
    const int head = row % G;
    const float lr = __shfl(l_run, 4 * kg + r, 64);
    const float inv = lr > 0.f ? 1.f / lr : 0.f;
    if (pos < L) {
      uint16_t *orow = a.out + (((int64_t)b * a.nq + h * G + head) * L + pos) * kD;
#pragma unroll
      for (int dt = 0; dt < 8; ++dt) {
        orow[16 * dt + col] = Bf16 ? f32_to_bf16_bits(acc[dt][r] * inv)
                         : __builtin_bit_cast(uint16_t, (_Float16)(acc[dt][r] * inv));
      }
    }
  }
}

}  // namespace
}  // namespace cq

using namespace cq;

namespace cq {
namespace {

// Split plan: enough key splits that the grid fills one resident generation
// of workgroups (several per CU), at most kMaxPrefillSplits and no more than
// the longest tile has key blocks; 1 when the workspace bounds are exceeded.
constexpr int kMaxPrefillSplits = 16;

struct PrefillPlan {
  int tiles, nsplit;
  size_t ws_bytes;  // 0: no workspace needed
};

PrefillPlan prefill_plan(int64_t B, int64_t H, int64_t G, int64_t n_q, int64_t T) {
  PrefillPlan p;
  const int64_t ppw = kRows / G;
  p.tiles = (int)((n_q + ppw - 1) / ppw);
  const int64_t groups = (int64_t)p.tiles * H * B;
  const int64_t resident = resident_workgroups(
      reinterpret_cast<const void *>(prefill_mfma_kernel<false, true>), kThreads, kSlotPrefill);
  int64_t ns = (resident + groups - 1) / groups;
  ns = std::min<int64_t>(ns, kMaxPrefillSplits);
  ns = std::min<int64_t>(ns, (T + kKeys - 1) / kKeys);
  const int64_t rows = B * H * G * n_q;
  if (ns < 2 || B * H * p.tiles > kMaxCounters || rows * ns * kD * 4 >= ((int64_t)1 << 31)) ns = 1;
  p.nsplit = (int)ns;
  p.ws_bytes = ns > 1 ? kCounterRegion + round256((size_t)rows * ns * 8) +
                            round256((size_t)rows * ns * kD * 4)
                      : 0;
  return p;
}

}  // namespace
}  // namespace cq

using namespace cq;

extern "C" size_t cq_prefill_workspace_size(int32_t batch, int32_t n_kv_heads, int32_t n_q_heads,
                                            int64_t n_q, int64_t seq_len) {
  if (batch < 1 || n_kv_heads < 1 || n_q_heads < n_kv_heads || n_q_heads % n_kv_heads || n_q < 1)
    return 0;
  const int G = n_q_heads / n_kv_heads;
  if (G > kRows || kRows % G) return 0;
  return prefill_plan(batch, n_kv_heads, G, n_q, seq_len).ws_bytes;
}

extern "C" int cq_prefill_attn(const cq_cache_desc *cache, const void *q, int32_t q_dtype,
                               int32_t n_q_heads, int64_t n_q, float scale, int32_t causal,
                               int64_t seq_len, void *out, void *workspace,
                               size_t workspace_bytes, cq_stream_t stream) {
  int st = validate_cache(cache);
  if (st) return st;
  // dense residual rows: the reconstruct fallback serves them
  if (field_bits(cache->k) != 4 || field_bits(cache->v) != 4) return CQ_ERR_UNSUPPORTED;
  if (!q || !out) return CQ_ERR_ARG;
  if (q_dtype != CQ_F16 && q_dtype != CQ_BF16) return CQ_ERR_DTYPE;
  if (cache->head_dim != kD) return CQ_ERR_UNSUPPORTED;
  if (n_q_heads < 1 || n_q_heads % cache->n_kv_heads) return CQ_ERR_SHAPE;
  const int G = n_q_heads / cache->n_kv_heads;
  if (G > kRows || kRows % G) return CQ_ERR_UNSUPPORTED;
  if (n_q < 1 || seq_len < n_q || seq_len >= (1 << 24)) return CQ_ERR_SHAPE;
  if (((uintptr_t)q | (uintptr_t)out) & 15) return CQ_ERR_ALIGN;
  PrefillArgs a;
  const cq_component *cp[2] = {&cache->k, &cache->v};
  for (int i = 0; i < 2; ++i) {
    a.kf[i] = cp[i]->keyframes;
    a.pk[i] = cp[i]->packed;
    a.sc[i] = cp[i]->scales;
    a.cap_kf[i] = cp[i]->cap_keyframes;
    a.cap_pf[i] = cp[i]->cap_pframes;
    a.stride[i] = cp[i]->stride;
    a.inv_stride[i] = 1.0f / (float)cp[i]->stride;
    if (num_keyframes(seq_len, a.stride[i]) > a.cap_kf[i] ||
        num_pframes(seq_len, a.stride[i]) > a.cap_pf[i])
      return CQ_ERR_CAPACITY;
    // buffer resources address each (sequence, head) region with 32-bit offsets
    if (a.cap_kf[i] * kD * 2 >= ((int64_t)1 << 31) || a.cap_pf[i] * 64 >= ((int64_t)1 << 31))
      return CQ_ERR_UNSUPPORTED;
  }
  a.B = cache->batch;
  a.H = cache->n_kv_heads;
  a.G = G;
  a.nq = n_q_heads;
  a.n_q = n_q;
  a.T = seq_len;
  a.causal = causal ? 1 : 0;
  a.scale = scale;
  a.q = (const uint16_t *)q;
  a.out = (uint16_t *)out;
  const PrefillPlan plan = prefill_plan(a.B, a.H, G, n_q, seq_len);
  a.tiles = plan.tiles;
  a.nsplit = 1;
  a.part_ml = a.part_acc = nullptr;
  a.counters = nullptr;
  if (plan.nsplit > 1 && workspace) {  // no workspace: one split per tile
    if ((uintptr_t)workspace & 255) return CQ_ERR_ALIGN;
    if (workspace_bytes < plan.ws_bytes) return CQ_ERR_WORKSPACE;
    const int64_t rows = (int64_t)a.B * n_q_heads * n_q;
    char *w = (char *)workspace;
    a.counters = (uint32_t *)w;
    a.part_ml = (float *)(w + kCounterRegion);
    a.part_acc = (float *)(w + kCounterRegion + round256((size_t)rows * plan.nsplit * 8));
    a.nsplit = plan.nsplit;
  }
  const dim3 grid((unsigned)(a.tiles * a.nsplit), (unsigned)a.H, (unsigned)a.B);
  const bool pow2 = ((a.stride[0] & (a.stride[0] - 1)) | (a.stride[1] & (a.stride[1] - 1))) == 0;
  const dim3 blk(kThreads);
  const hipStream_t s = (hipStream_t)stream;
  if (q_dtype == CQ_BF16) {
    if (pow2) prefill_mfma_kernel<true, true><<<grid, blk, 0, s>>>(a);
    else prefill_mfma_kernel<true, false><<<grid, blk, 0, s>>>(a);
  } else {
    if (pow2) prefill_mfma_kernel<false, true><<<grid, blk, 0, s>>>(a);
    else prefill_mfma_kernel<false, false><<<grid, blk, 0, s>>>(a);
  }
  return hipGetLastError() == hipSuccess ? CQ_OK : CQ_ERR_LAUNCH;
}
