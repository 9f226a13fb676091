// cq_codec.hip — encode side of the ChronoQuant hot path on gfx950:
// residual quantisation (codec), INT4 packing, the fused append (I-frame or
// quantise+pack in place) and the fp16 reconstruction used by the fallback
// attention path.  A (token, kv head) row is encoded by one wavefront, or at
// head_dim 128 with 16-bit tokens by 16 lanes (four rows per wave); the row
// absmax is a DPP reduction; every floating-point op is rounded to the input
// dtype the way the reference's MLX arrays round it.
#include <hip/hip_runtime.h>
#include <math.h>

#include <algorithm>

#include "cq_device.h"

namespace cq {

// Per-lane slice of one row: dims [lane*E, lane*E + E), E in {1, 2, 4}.
constexpr int kMaxE = 4;

__host__ __device__ inline int dims_per_lane(int D) {
  return D <= 64 ? 1 : (D <= 128 ? 2 : 4);
}

// Residual quantisation of one row held by one wavefront.
// Follows ChronoQuantCodecMLX.quantize_delta (reference codec.py:23-65):
//   amax = max|d|; s = R(amax/(h-1)); dead zone: thr = R(amax*R(dz)),
//   d = |d| < thr ? 0 : d, s = R(max(amax',eps-guard)/(h-1));
//   code = clip(rint(R(d/s_safe)), -h, h-1); code = 0 if s < eps.
// R rounds to the dtype; eps = R(1e-10) (0 for fp16, so the guards never
// fire there).  A NaN quotient (0/0 for an all-zero fp16 row) gives code 0.
template <int DT>
__device__ __forceinline__ float codec_row(float (&d)[kMaxE], int E, int bits,
                                           float dz, int (&code)[kMaxE]) {
  using T = Dt<DT>;
  const int half = (1 << bits) >> 1;
  const float hm1 = (float)(half - 1);
  const float eps = T::round(1e-10f);
  float a = 0.f;
#pragma unroll
  for (int i = 0; i < kMaxE; ++i)
    if (i < E) a = fmaxf(a, fabsf(d[i]));
  const float amax = wave_max(a);
  float scale = T::round(amax / hm1);
  if (dz > 0.f) {
    const float thr = T::round(amax * T::round(dz));
    float a2 = 0.f;
#pragma unroll
    for (int i = 0; i < kMaxE; ++i) {
      if (i < E) {
        if (fabsf(d[i]) < thr) d[i] = 0.f;
        a2 = fmaxf(a2, fabsf(d[i]));
      }
    }
    const float amax_c = wave_max(a2);
    const float amax_safe = (amax_c < eps) ? amax : amax_c;
    scale = T::round(amax_safe / hm1);
  }
  const float scale_safe = (scale < eps) ? 1.0f : scale;
#pragma unroll
  for (int i = 0; i < kMaxE; ++i) {
    const float q = T::round(d[i] / scale_safe);
    int c;
    if (q != q) {
      c = 0;
    } else {
      float r = rintf(q);  // round half to even
      r = fminf(fmaxf(r, (float)(-half)), hm1);
      c = (int)r;
    }
    if (scale < eps) c = 0;
    code[i] = c;
  }
  return scale;
}

// Pack this lane's E nibbles into its part of word (lane*E)/8 and OR the
// 8/E lanes of that word together.  nibble = clip(code + 8, 0, 15); dims at
// or past D carry nibble 0 (reference kernels.py:40-43, MSL :15-21).
__device__ __forceinline__ uint32_t pack_lane(const int (&code)[kMaxE], int E,
                                              int lane, int D) {
  uint32_t part = 0;
#pragma unroll
  for (int i = 0; i < kMaxE; ++i) {
    if (i < E) {
      const int dim = lane * E + i;
      int u = code[i] + 8;
      u = u < 0 ? 0 : (u > 15 ? 15 : u);
      if (dim < D) part |= (uint32_t)u << (4 * (dim & 7));
    }
  }
  if (E == 1) return group_or<8>(part);
  if (E == 2) return group_or<4>(part);
  return group_or<2>(part);
}

// ---------------------------------------------------------------------------
// cq_quantize_delta: one wavefront per row
// ---------------------------------------------------------------------------
template <int DT>
__global__ __launch_bounds__(256) void quantize_delta_kernel(
    const void *__restrict__ delta, int64_t n_rows, int D, int bits, float dz,
    int8_t *__restrict__ codes, uint16_t *__restrict__ scales) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  if (row >= n_rows) return;  // wave-uniform
  const int E = dims_per_lane(D);
  float d[kMaxE];
  int code[kMaxE];
#pragma unroll
  for (int i = 0; i < kMaxE; ++i) {
    const int dim = lane * E + i;
    d[i] = (i < E && dim < D) ? Dt<DT>::load(delta, row * D + dim) : 0.f;
  }
  const float s = codec_row<DT>(d, E, bits, dz, code);
#pragma unroll
  for (int i = 0; i < kMaxE; ++i) {
    const int dim = lane * E + i;
    if (i < E && dim < D) codes[row * D + dim] = (int8_t)code[i];
  }
  if (lane == 0) scales[row] = f2h(s);
}

// ---------------------------------------------------------------------------
// cq_pack_int4 / cq_unpack_int4: one thread per word
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void pack_kernel(const int8_t *__restrict__ codes,
                                                   int64_t n_words, int D, int W,
                                                   uint32_t *__restrict__ packed) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n_words) return;
  const int64_t row = i / W;
  const int w = (int)(i - row * W);
  uint32_t word = 0;
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    const int dim = 8 * w + k;
    if (dim < D) {
      int u = (int)codes[row * D + dim] + 8;
      u = u < 0 ? 0 : (u > 15 ? 15 : u);
      word |= (uint32_t)u << (4 * k);
    }
  }
  packed[i] = word;
}

__global__ __launch_bounds__(256) void unpack_kernel(const uint32_t *__restrict__ packed,
                                                     int64_t n_words, int D, int W,
                                                     int8_t *__restrict__ codes) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n_words) return;
  const int64_t row = i / W;
  const int w = (int)(i - row * W);
  const uint32_t word = packed[i];
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    const int dim = 8 * w + k;
    if (dim < D) codes[row * D + dim] = (int8_t)((int)((word >> (4 * k)) & 0xfu) - 8);
  }
}

// ---------------------------------------------------------------------------
// cq_append, one wavefront per (component, b, new token s, kv head) row (any
// head_dim and dtype; head_dim 128 with 16-bit tokens takes
// append_row4_kernel below)
// ---------------------------------------------------------------------------
struct AppendArgs {
  cq_component comp[2];
  const void *x[2];
  int64_t xs[2][3];  // element strides b, h, s
  int B, H, D, W;
  int S;             // new tokens per sequence (2 B S H rows < 2^31, host-checked)
  int vec;           // 16-bit dtype, E = 2, unit element stride, even row starts:
                     // each lane's 2 elements are one aligned 32-bit load
  const int32_t *offsets;
  int64_t offset;
};

// n / d for 0 <= n < 2^31, d >= 1: a float estimate, then the remainder
// brought into [0, d) (the estimate is off by at most one below 2^24 and by
// a few units up to 2^31, so the loops run at most a handful of times).
__device__ __forceinline__ int div_pos(int n, int d) {
  int q = (int)((float)n / (float)d);
  int r = n - q * d;
  while (r < 0) { --q; r += d; }
  while (r >= d) { ++q; r -= d; }
  return q;
}

// The operands of one token row, held by a wave: this lane's E dims of the
// token (v) and of its fp16 anchor (an; unused for an I-frame), and where
// the row goes: component ci, row bh = b * H + h, position t, group g =
// t / stride.
struct TokenRow {
  float v[kMaxE], an[kMaxE];
  int64_t bh, t, g;
  int ci;
};

// This lane's dims of keyframe row g of bh (g clamped into the capacity: a
// token whose anchor lies past it is dropped by encode_token).  vec: D = 128,
// the lane's 2 elements are one 32-bit load.
__device__ __forceinline__ void load_cache_anchor(const cq_component &c, int64_t bh, int64_t g,
                                                  int lane, int D, bool vec,
                                                  float (&an)[kMaxE]) {
  const int E = dims_per_lane(D);
  const int64_t gg = g < 0 ? 0 : (g >= c.cap_keyframes ? c.cap_keyframes - 1 : g);
  const uint16_t *arow = c.keyframes + (bh * c.cap_keyframes + gg) * D;
  if (vec) {
    const uint32_t u = ((const uint32_t *)arow)[lane];
    an[0] = h2f((uint16_t)(u & 0xffffu));
    an[1] = h2f((uint16_t)(u >> 16));
#pragma unroll
    for (int i = 2; i < kMaxE; ++i) an[i] = 0.f;
  } else {
#pragma unroll
    for (int i = 0; i < kMaxE; ++i) {
      const int dim = lane * E + i;
      an[i] = (i < E && dim < D) ? h2f(arow[dim]) : 0.f;
    }
  }
}

// Word `lane` of a dense row (fb-bit fields, fb < 4) held by a wave whose
// lane l has the codes of dims l*E .. l*E + E - 1: lane l's fields form the
// E*fb stream bits from E*fb*l, and word w ORs the (at most 32/(E*fb) + 2)
// lanes whose bits meet [32w, 32w + 32).  Dims past D give 0 bits.  Called
// by the whole wave (the shuffles read every lane).
__device__ __forceinline__ uint32_t dense_row_word(const int (&code)[kMaxE], int E, int fb,
                                                   int lane, int D) {
  const int cb = E * fb;  // stream bits per lane
  uint32_t chunk = 0;
#pragma unroll
  for (int i = 0; i < kMaxE; ++i)
    if (i < E && lane * E + i < D) chunk |= code_field(code[i], fb) << (fb * i);
  const int j0 = (32 * lane) / cb;
  const int n = 32 / cb + 2;  // wave-uniform
  uint32_t word = 0;
  for (int k = 0; k < n; ++k) {
    const int j = j0 + k;
    const uint32_t cj = (uint32_t)__shfl((int)chunk, j & 63, 64);
    const int sh = cb * j - 32 * lane;
    if (j < 64 && sh < 32 && sh > -cb) word |= sh >= 0 ? cj << sh : cj >> (-sh);
  }
  return word;
}

// Encode one token row whose operands are loaded: the fp16 I-frame when t is
// a multiple of the stride (reference cache.py:103-105), else the residual
// against anchor g (cache.py:107-116: d = round(token - round(anchor))),
// quantised and packed into P-frame slot t - g - 1.  No loads: a wave can
// have the operands of several rows in flight before encoding any.  Rows
// past the capacities, and negative positions, are dropped (device
// positions: the host could not check them).
template <int DT>
__device__ __forceinline__ void encode_token(const cq_component &c, const TokenRow &r, int lane,
                                             int D, int W) {
  const int E = dims_per_lane(D);
  const int64_t bh = r.bh, t = r.t, g = r.g;
  if (t < 0) return;
  if (t - g * c.stride == 0) {
    if (g >= c.cap_keyframes) return;
    uint16_t *row = c.keyframes + (bh * c.cap_keyframes + g) * D;
#pragma unroll
    for (int i = 0; i < kMaxE; ++i) {
      const int dim = lane * E + i;
      if (i < E && dim < D) row[dim] = f2h(r.v[i]);
    }
    return;
  }
  const int64_t slot = t - g - 1;
  if (slot >= c.cap_pframes || g >= c.cap_keyframes) return;
  float d[kMaxE];
#pragma unroll
  for (int i = 0; i < kMaxE; ++i) d[i] = Dt<DT>::round(r.v[i] - Dt<DT>::round(r.an[i]));
  int code[kMaxE];
  const float sc = codec_row<DT>(d, E, c.delta_bits, c.dead_zone, code);
  const int fb = field_bits(c);
  if (fb == 4) {
    const uint32_t word = pack_lane(code, E, lane, D);
    const int wl = lane * E;
    if ((wl & 7) == 0 && (wl >> 3) < W)
      c.packed[(bh * c.cap_pframes + slot) * W + (wl >> 3)] = word;
  } else {
    const int rw = row_words_of(D, fb);
    const uint32_t word = dense_row_word(code, E, fb, lane, D);
    if (lane < rw) c.packed[(bh * c.cap_pframes + slot) * rw + lane] = word;
  }
  if (lane == 0) c.scales[bh * c.cap_pframes + slot] = f2h(sc);
}

// Load phase of one (component, b, new token s, kv head) row of cq_append.
// 32-bit index arithmetic (the host bounds 2 B S H); the row decomposition
// and t / stride are the only divisions, each a float estimate + fix-up.
// The anchor (fp16 I-frame of group g) comes from the new tokens when that
// I-frame is appended by this call (the same fp16 value the cache will
// hold), else from the cache, so the waves of one launch never depend on
// each other.
template <int DT>
__device__ __forceinline__ void load_append_row(const AppendArgs &a, int item, int per_comp,
                                                TokenRow &r) {
  const int lane = threadIdx.x & 63;
  const int ci = item >= per_comp ? 1 : 0;
  item -= ci * per_comp;
  const int bs = div_pos(item, a.H);
  const int h = item - bs * a.H;
  const int b = div_pos(bs, a.S);
  const int s = bs - b * a.S;

  const cq_component &c = a.comp[ci];
  const int D = a.D, E = dims_per_lane(D);
  const int64_t off = a.offsets ? (int64_t)a.offsets[b] : a.offset;
  const int64_t t = off + s;
  const int stride = c.stride;
  const int64_t g = (t >= 0 && t < 0x7fffffff) ? (int64_t)div_pos((int)t, stride)
                                               : (t < 0 ? -1 : t / stride);
  r.ci = ci;
  r.t = t;
  r.g = g;
  r.bh = (int64_t)b * a.H + h;
  const void *x = a.x[ci];
  const int64_t xrow = b * a.xs[ci][0] + h * a.xs[ci][1] + (int64_t)s * a.xs[ci][2];
  auto load_x = [&](int64_t row, float (&out)[kMaxE], bool to_f16) {
    if (a.vec) {  // one 32-bit load of this lane's 2 elements
      const uint32_t u = ((const uint32_t *)x)[(row >> 1) + lane];
      const float lo = DT == CQ_BF16 ? bf2f((uint16_t)(u & 0xffffu)) : h2f((uint16_t)(u & 0xffffu));
      const float hi = DT == CQ_BF16 ? bf2f((uint16_t)(u >> 16)) : h2f((uint16_t)(u >> 16));
      out[0] = to_f16 ? h2f(f2h(lo)) : lo;
      out[1] = to_f16 ? h2f(f2h(hi)) : hi;
#pragma unroll
      for (int i = 2; i < kMaxE; ++i) out[i] = 0.f;
    } else {
#pragma unroll
      for (int i = 0; i < kMaxE; ++i) {
        const int dim = lane * E + i;
        const float e = (i < E && dim < D) ? Dt<DT>::load(x, row + dim) : 0.f;
        out[i] = to_f16 ? h2f(f2h(e)) : e;
      }
    }
  };
  load_x(xrow, r.v, false);
  const int64_t ta = g * stride;
  if (t != ta && ta >= off)  // wave-uniform
    load_x(b * a.xs[ci][0] + h * a.xs[ci][1] + (ta - off) * a.xs[ci][2], r.an, true);
  else
    load_cache_anchor(c, r.bh, g, lane, D, a.vec != 0, r.an);
}

// Rows per wave and iteration: their loads are all issued before the first
// row is encoded.  (gfx9 counts loads and stores with one in-order counter,
// so a wave taking one row at a time waited for each row's stores before
// the next row's loads could be used: two round trips per row.)
constexpr int kAppendRowsPerWave = 1;

template <int DT>
__global__ __launch_bounds__(256) void append_kernel(AppendArgs a) {
  // Grid-stride over the rows: a bulk append has millions of rows, and one
  // short-lived workgroup per 4 rows left the GPU waiting on workgroup
  // launches (the host caps the grid).
  const int lane = threadIdx.x & 63;
  const int per_comp = a.B * a.S * a.H, total = 2 * per_comp;
  const int waves = (int)gridDim.x * (int)(blockDim.x >> 6);
  // the row indices are wave-uniform: keep them (and all index math) scalar
  const int first = __builtin_amdgcn_readfirstlane((int)blockIdx.x * (int)(blockDim.x >> 6) +
                                                   (int)(threadIdx.x >> 6));
  for (int base = first; base < total; base += kAppendRowsPerWave * waves) {
    TokenRow r[kAppendRowsPerWave];
#pragma unroll
    for (int j = 0; j < kAppendRowsPerWave; ++j)
      load_append_row<DT>(a, min(base + j * waves, total - 1), per_comp, r[j]);
#pragma unroll
    for (int j = 0; j < kAppendRowsPerWave; ++j)
      if (base + j * waves < total) encode_token<DT>(a.comp[r[j].ci], r[j], lane, a.D, a.W);
  }
}

// ---------------------------------------------------------------------------
// cq_append at head_dim 128 with 16-bit tokens: four rows per wave, one row
// per 16 lanes, lane j of a row holding dims 8j .. 8j+7 (one 16-byte load of
// the token and of its anchor, one packed word out).  The per-row work (the
// absmax reductions over 16 lanes, the scale, the index arithmetic) is done
// by the same instructions for four rows, where the one-row-per-wave kernel
// spent them on one (the bulk append was bound by VALU issue at ~270
// instructions per row).  Same arithmetic as codec_row / encode_token.
// ---------------------------------------------------------------------------
template <int DT>
__device__ __forceinline__ void unpack8_dt(uint4 u, bool f16, float (&f)[8]) {
  const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint16_t lo = (uint16_t)(w[i] & 0xffffu), hi = (uint16_t)(w[i] >> 16);
    f[2 * i] = (DT == CQ_BF16 && !f16) ? bf2f(lo) : h2f(lo);
    f[2 * i + 1] = (DT == CQ_BF16 && !f16) ? bf2f(hi) : h2f(hi);
  }
}

// codec_row over a 16-lane row, 8 dims per lane (D = 128).
template <int DT>
__device__ __forceinline__ float codec_row16(float (&d)[8], int bits, float dz, int (&code)[8]) {
  using T = Dt<DT>;
  const int half = (1 << bits) >> 1;
  const float hm1 = (float)(half - 1);
  const float eps = T::round(1e-10f);
  float m = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) m = fmaxf(m, fabsf(d[i]));
  const float amax = row16_max(m);
  float scale = T::round(amax / hm1);
  if (dz > 0.f) {  // uniform over the row's 16 lanes
    const float thr = T::round(amax * T::round(dz));
    float m2 = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      if (fabsf(d[i]) < thr) d[i] = 0.f;
      m2 = fmaxf(m2, fabsf(d[i]));
    }
    const float amax_c = row16_max(m2);
    const float amax_safe = (amax_c < eps) ? amax : amax_c;
    scale = T::round(amax_safe / hm1);
  }
  const float scale_safe = (scale < eps) ? 1.0f : scale;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const float q = T::round(d[i] / scale_safe);
    int c;
    if (q != q) {
      c = 0;
    } else {
      float r = rintf(q);  // round half to even
      r = fminf(fmaxf(r, (float)(-half)), hm1);
      c = (int)r;
    }
    if (scale < eps) c = 0;
    code[i] = c;
  }
  return scale;
}

template <int DT>
__global__ __launch_bounds__(256) void append_row4_kernel(AppendArgs a) {
  const int lane = threadIdx.x & 63, j = lane & 15;
  const int per_comp = a.B * a.S * a.H, total = 2 * per_comp;
  const int waves = (int)gridDim.x * (int)(blockDim.x >> 6);
  const int first = 4 * __builtin_amdgcn_readfirstlane((int)blockIdx.x * (int)(blockDim.x >> 6) +
                                                       (int)(threadIdx.x >> 6));
  for (int base = first; base < total; base += 4 * waves) {
    const int item0 = base + (lane >> 4);  // this lane's row
    const bool live = item0 < total;
    int item = live ? item0 : total - 1;
    const int ci = item >= per_comp ? 1 : 0;
    item -= ci * per_comp;
    const int bs = div_pos(item, a.H);
    const int h = item - bs * a.H;
    const int b = div_pos(bs, a.S);
    const int s = bs - b * a.S;
    // the row's component (rows of both can share a wave)
    uint16_t *const kf = ci ? a.comp[1].keyframes : a.comp[0].keyframes;
    uint32_t *const pk = ci ? a.comp[1].packed : a.comp[0].packed;
    uint16_t *const sc = ci ? a.comp[1].scales : a.comp[0].scales;
    const int64_t cap_kf = ci ? a.comp[1].cap_keyframes : a.comp[0].cap_keyframes;
    const int64_t cap_pf = ci ? a.comp[1].cap_pframes : a.comp[0].cap_pframes;
    const int stride = ci ? a.comp[1].stride : a.comp[0].stride;
    const int bits = ci ? a.comp[1].delta_bits : a.comp[0].delta_bits;
    const int fb = ci ? field_bits(a.comp[1]) : field_bits(a.comp[0]);
    const int rw = row_words_of(128, fb);
    const float dz = ci ? a.comp[1].dead_zone : a.comp[0].dead_zone;
    const uint16_t *x = (const uint16_t *)(ci ? a.x[1] : a.x[0]);
    const int64_t xs0 = ci ? a.xs[1][0] : a.xs[0][0], xs1 = ci ? a.xs[1][1] : a.xs[0][1],
                  xs2 = ci ? a.xs[1][2] : a.xs[0][2];

    const int64_t off = a.offsets ? (int64_t)a.offsets[b] : a.offset;
    const int64_t t = off + s;
    const int64_t g = (t >= 0 && t < 0x7fffffff) ? (int64_t)div_pos((int)t, stride)
                                                 : (t < 0 ? -1 : t / stride);
    const int64_t bh = (int64_t)b * a.H + h;
    const int64_t ta = g * stride;
    const bool iframe = t == ta;
    const bool an_in = !iframe && ta >= off;  // anchor appended by this call
    const int64_t gg = g < 0 ? 0 : (g >= cap_kf ? cap_kf - 1 : g);
    const uint4 *xp = (const uint4 *)(x + b * xs0 + h * xs1 + (int64_t)s * xs2 + 8 * j);
    const uint4 *ap = an_in ? (const uint4 *)(x + b * xs0 + h * xs1 + (ta - off) * xs2 + 8 * j)
                            : (const uint4 *)(kf + (bh * cap_kf + gg) * 128 + 8 * j);
    const uint4 xv = *xp, av = *ap;
    float v[8], an[8];
    unpack8_dt<DT>(xv, false, v);
    unpack8_dt<DT>(av, !an_in, an);
    if (an_in) {
#pragma unroll
      for (int i = 0; i < 8; ++i) an[i] = h2f(f2h(an[i]));  // the fp16 I-frame value
    }
    const bool ok = live && t >= 0 && g < cap_kf;
    if (iframe) {
      if (ok) {
        uint32_t w[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) w[i] = (uint32_t)f2h(v[2 * i]) | ((uint32_t)f2h(v[2 * i + 1]) << 16);
        *(uint4 *)(kf + (bh * cap_kf + g) * 128 + 8 * j) = uint4{w[0], w[1], w[2], w[3]};
      }
    } else {
      float d[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) d[i] = Dt<DT>::round(v[i] - Dt<DT>::round(an[i]));
      int code[8];
      const float scale = codec_row16<DT>(d, bits, dz, code);
      const int64_t slot = t - g - 1;
      // this lane's 8 fields (8 fb stream bits from 8 fb j); a dense row's
      // word j takes them from lanes j1 = 32j / 8fb and j1 + 1 of the row
      // (the row's 16 lanes share this branch)
      uint32_t chunk = 0;
#pragma unroll
      for (int i = 0; i < 8; ++i) chunk |= code_field(code[i], fb) << (fb * i);
      uint32_t word = chunk;
      if (fb != 4) {
        const int j1 = (32 * j) / (8 * fb), o = (32 * j) % (8 * fb);
        const uint32_t lo = (uint32_t)__shfl((int)chunk, (lane & 48) + min(j1, 15), 64);
        const uint32_t hi = (uint32_t)__shfl((int)chunk, (lane & 48) + min(j1 + 1, 15), 64);
        word = (lo >> o) | (hi << (8 * fb - o));
      }
      if (ok && slot < cap_pf) {
        if (j < rw) pk[(bh * cap_pf + slot) * rw + j] = word;
        if (j == 0) sc[bh * cap_pf + slot] = f2h(scale);
      }
    }
  }
}

// ---------------------------------------------------------------------------
// cq_qkv_rope_append: one decode token per sequence, from the fused QKV
// projection straight into the caches.  One wavefront per (b, head) over the
// nq query, nkv key and nkv value heads; lane j holds dims j and j + 64 (one
// rotary pair).  Query and key heads: RMSNorm (rounded to the dtype), then
// the rotary embedding at positions[b * pos_bstride], exactly as
// cq_qkv_norm_rope computes them; query rows go to q_out, key rows (rounded
// to the dtype, as that kernel's output is) and value rows are appended at
// cache position t = offsets[b] (or offset) as cq_append encodes them.  With
// one new token the anchor of a P-frame is always in the cache already.
// ---------------------------------------------------------------------------
struct RopeAppendArgs {
  cq_component comp[2];
  const void *qkv;  // [B][(nq + 2 nkv) * 128]
  const void *q_w, *k_w;
  void *q_out;                 // [B][nq][128]
  const float *cos_t, *sin_t;  // [max_pos][64]
  const int64_t *positions;
  int64_t pos_bstride, max_pos;
  const int32_t *offsets;
  int64_t offset;
  int32_t *lengths;  // optional: t + 1 per sequence
  int B, nq, nkv, W;
  float eps;
};

template <int DT>
__global__ __launch_bounds__(256) void rope_append_kernel(RopeAppendArgs a) {
  const int lane = threadIdx.x & 63;
  const int heads = a.nq + 2 * a.nkv;
  const int row = (int)blockIdx.x * 4 + (int)(threadIdx.x >> 6);
  if (row >= a.B * heads) return;  // wave-uniform
  const int b = div_pos(row, heads), h = row - b * heads;
  float x1 = Dt<DT>::load(a.qkv, (int64_t)row * 128 + lane);
  float x2 = Dt<DT>::load(a.qkv, (int64_t)row * 128 + lane + 64);
  const int64_t t = a.offsets ? (int64_t)a.offsets[b] : a.offset;
  if (a.lengths && h == 0 && lane == 0) a.lengths[b] = (int32_t)(t + 1);
  // key / value rows: the anchor row's load goes out with the token's
  const int ci = h >= a.nq + a.nkv ? 1 : 0;
  const int hk = h - a.nq - ci * a.nkv;
  TokenRow r;
  r.ci = ci;
  r.t = t;
  r.bh = (int64_t)b * a.nkv + hk;
  if (h >= a.nq) {
    const cq_component &c = a.comp[ci];
    r.g = (t >= 0 && t < 0x7fffffff) ? (int64_t)div_pos((int)t, c.stride)
                                     : (t < 0 ? -1 : t / c.stride);
    load_cache_anchor(c, r.bh, r.g, lane, 128, true, r.an);
  }
  if (h < a.nq + a.nkv) {
    const bool is_q = h < a.nq;
    const void *w = is_q ? a.q_w : a.k_w;
    if (w) {
      const float inv = 1.f / sqrtf(wave_sum(x1 * x1 + x2 * x2) / 128.f + a.eps);
      x1 = Dt<DT>::round(x1 * inv * Dt<DT>::load(w, lane));
      x2 = Dt<DT>::round(x2 * inv * Dt<DT>::load(w, lane + 64));
    }
    const int64_t pos = a.positions[(int64_t)b * a.pos_bstride];
    float c = __builtin_nanf(""), s = c;
    if (pos >= 0 && pos < a.max_pos) {
      c = a.cos_t[pos * 64 + lane];
      s = a.sin_t[pos * 64 + lane];
    }
    const float y1 = x1 * c - x2 * s, y2 = x2 * c + x1 * s;
    if (is_q) {
      const int64_t o = ((int64_t)b * a.nq + h) * 128;
      Dt<DT>::store(a.q_out, o + lane, y1);
      Dt<DT>::store(a.q_out, o + lane + 64, y2);
      return;
    }
    x1 = Dt<DT>::round(y1);
    x2 = Dt<DT>::round(y2);
  }
  // key or value row: to the codec's lane layout (lane holds dims 2 lane and
  // 2 lane + 1), from lanes 2 lane mod 64 and 2 lane + 1 mod 64 of the
  // first (lane < 32) or second half.  With one new token a P-frame's
  // anchor is always in the cache.
  const int s0 = (2 * lane) & 63;
  const float a0 = __shfl(x1, s0, 64), a1 = __shfl(x1, s0 + 1, 64);
  const float b0 = __shfl(x2, s0, 64), b1 = __shfl(x2, s0 + 1, 64);
  r.v[0] = lane < 32 ? a0 : b0;
  r.v[1] = lane < 32 ? a1 : b1;
  r.v[2] = r.v[3] = 0.f;
  encode_token<DT>(a.comp[ci], r, lane, 128, a.W);
}

// ---------------------------------------------------------------------------
// cq_reconstruct: one thread per (b, h, t, word) — reference cache.py:131-156
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void reconstruct_kernel(cq_component c, int B, int H,
                                                          int D, int W, int64_t T,
                                                          uint16_t *__restrict__ out) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t total = (int64_t)B * H * T * W;
  if (i >= total) return;
  const int w = (int)(i % W);
  const int64_t bht = i / W;
  const int64_t t = bht % T;
  const int64_t bh = bht / T;
  const int64_t g = t / c.stride;
  const bool is_p = (t - g * c.stride) != 0;
  const uint16_t *anc = c.keyframes + (bh * c.cap_keyframes + g) * D;
  uint16_t *o = out + bht * D;
  const int fb = field_bits(c), rw = row_words_of(D, fb);
  uint32_t fields = 0;  // the 8 fields of dims 8w .. 8w + 7
  float s = 0.f;
  if (is_p) {
    const int64_t slot = t - g - 1;
    fields = stream_bits(c.packed + (bh * c.cap_pframes + slot) * rw, rw, 8 * fb * w, 8 * fb);
    s = h2f(c.scales[bh * c.cap_pframes + slot]);
  }
  const uint32_t mask = (1u << fb) - 1u;
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    const int dim = 8 * w + k;
    if (dim >= D) break;
    float delta = 0.f;
    if (is_p) {
      const int code = (int)((fields >> (fb * k)) & mask) - (1 << (fb - 1));
      delta = h2f(f2h((float)code * s));
    }
    o[dim] = f2h(h2f(anc[dim]) + delta);  // fp16 add, cache.py:156
  }
}

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------
static int launch_status() {
  return hipGetLastError() == hipSuccess ? CQ_OK : CQ_ERR_LAUNCH;
}

static bool bits_ok(int bits) { return bits >= 2 && bits <= 4; }

constexpr int64_t kAppendGroups = 16384;

int validate_cache(const cq_cache_desc *c) {
  if (!c) return CQ_ERR_ARG;
  if (c->batch < 1 || c->n_kv_heads < 1) return CQ_ERR_SHAPE;
  if (c->head_dim < 1 || c->head_dim > kMaxHeadDim) return CQ_ERR_SHAPE;
  for (const cq_component *p : {&c->k, &c->v}) {
    if (!p->keyframes || !p->packed || !p->scales) return CQ_ERR_ARG;
    if (p->stride < 1 || !bits_ok(p->delta_bits)) return CQ_ERR_ARG;
    if (!(p->dead_zone >= 0.f)) return CQ_ERR_ARG;
    if (p->cap_keyframes < 1 || p->cap_pframes < 1) return CQ_ERR_CAPACITY;
    if (p->packing != CQ_PACK_INT4 && p->packing != CQ_PACK_DENSE) return CQ_ERR_ARG;
  }
  return CQ_OK;
}

int64_t num_keyframes(int64_t n, int stride) { return n <= 0 ? 0 : (n - 1) / stride + 1; }
int64_t num_pframes(int64_t n, int stride) { return n - num_keyframes(n, stride); }

}  // namespace cq

using namespace cq;

extern "C" {

const char *cq_status_string(int32_t status) {
  switch (status) {
    case CQ_OK: return "ok";
    case CQ_ERR_ARG: return "invalid argument (null pointer or bad scalar)";
    case CQ_ERR_SHAPE: return "shape out of range (head_dim must be 1..256, heads/batch >= 1)";
    case CQ_ERR_DTYPE: return "unsupported dtype";
    case CQ_ERR_ALIGN: return "pointer misaligned";
    case CQ_ERR_CAPACITY: return "cache capacity exceeded";
    case CQ_ERR_WORKSPACE: return "workspace missing or too small";
    case CQ_ERR_UNSUPPORTED: return "unsupported configuration";
    case CQ_ERR_LAUNCH: return "kernel launch failed";
    case CQ_ERR_SCRATCH:
      return "shape needs more split workspace than the static scratch holds "
             "(CQ_NOALLOC_SCRATCH_BYTES); use cq_decode_attn with a workspace";
    case CQ_ERR_TIMEOUT:
      return "a split wait of an earlier decode ran out of poll rounds and folded without "
             "every partial (its output is unreliable); the workspace has been cleared";
    default: return "unknown status";
  }
}

int cq_quantize_delta(const void *delta, int32_t dtype, int64_t n_rows, int32_t head_dim,
                      int32_t delta_bits, float dead_zone, int8_t *codes,
                      uint16_t *scales, cq_stream_t stream) {
  if (n_rows < 0) return CQ_ERR_ARG;
  if (head_dim < 1 || head_dim > kMaxHeadDim) return CQ_ERR_SHAPE;
  if (!bits_ok(delta_bits) || !(dead_zone >= 0.f)) return CQ_ERR_ARG;
  if (n_rows == 0) return CQ_OK;
  if (!delta || !codes || !scales) return CQ_ERR_ARG;
  const dim3 grid((unsigned)((n_rows + 3) / 4)), block(256);
  hipStream_t st = (hipStream_t)stream;
  switch (dtype) {
    case CQ_F16: quantize_delta_kernel<CQ_F16><<<grid, block, 0, st>>>(delta, n_rows, head_dim, delta_bits, dead_zone, codes, scales); break;
    case CQ_BF16: quantize_delta_kernel<CQ_BF16><<<grid, block, 0, st>>>(delta, n_rows, head_dim, delta_bits, dead_zone, codes, scales); break;
    case CQ_F32: quantize_delta_kernel<CQ_F32><<<grid, block, 0, st>>>(delta, n_rows, head_dim, delta_bits, dead_zone, codes, scales); break;
    default: return CQ_ERR_DTYPE;
  }
  return launch_status();
}

int cq_pack_int4(const int8_t *codes, int64_t n_rows, int32_t head_dim, uint32_t *packed,
                 cq_stream_t stream) {
  if (n_rows < 0 || head_dim < 1) return CQ_ERR_SHAPE;
  if (n_rows == 0) return CQ_OK;
  if (!codes || !packed) return CQ_ERR_ARG;
  const int W = (head_dim + 7) / 8;
  const int64_t n = n_rows * W;
  pack_kernel<<<dim3((unsigned)((n + 255) / 256)), dim3(256), 0, (hipStream_t)stream>>>(
      codes, n, head_dim, W, packed);
  return launch_status();
}

int cq_unpack_int4(const uint32_t *packed, int64_t n_rows, int32_t head_dim, int8_t *codes,
                   cq_stream_t stream) {
  if (n_rows < 0 || head_dim < 1) return CQ_ERR_SHAPE;
  if (n_rows == 0) return CQ_OK;
  if (!codes || !packed) return CQ_ERR_ARG;
  const int W = (head_dim + 7) / 8;
  const int64_t n = n_rows * W;
  unpack_kernel<<<dim3((unsigned)((n + 255) / 256)), dim3(256), 0, (hipStream_t)stream>>>(
      packed, n, head_dim, W, codes);
  return launch_status();
}

int cq_append(const cq_cache_desc *cache, const void *keys, const int64_t *key_strides,
              const void *values, const int64_t *value_strides, int32_t dtype,
              int64_t n_new, const int32_t *offsets, int64_t offset, cq_stream_t stream) {
  int st = validate_cache(cache);
  if (st) return st;
  if (n_new < 0 || offset < 0) return CQ_ERR_ARG;
  if (n_new == 0) return CQ_OK;
  if (!keys || !values || !key_strides || !value_strides) return CQ_ERR_ARG;
  if (!offsets) {  // host-side capacity check when positions are known here
    for (const cq_component *p : {&cache->k, &cache->v}) {
      if (num_keyframes(offset + n_new, p->stride) > p->cap_keyframes ||
          num_pframes(offset + n_new, p->stride) > p->cap_pframes)
        return CQ_ERR_CAPACITY;
    }
  }
  AppendArgs a;
  a.comp[0] = cache->k;
  a.comp[1] = cache->v;
  a.x[0] = keys;
  a.x[1] = values;
  for (int i = 0; i < 3; ++i) {
    a.xs[0][i] = key_strides[i];
    a.xs[1][i] = value_strides[i];
  }
  a.B = cache->batch;
  a.H = cache->n_kv_heads;
  a.D = cache->head_dim;
  a.W = (cache->head_dim + 7) / 8;
  const int64_t items = 2 * (int64_t)a.B * n_new * a.H;
  // 32-bit row indices in the kernel (base + 3 * grid waves stays below 2^31)
  if (items >= 0x7fffffff - (1 << 20)) return CQ_ERR_SHAPE;
  a.S = (int)n_new;
  // 16-bit dtype, D = 128 (2 elements per lane), unit element stride, even
  // row strides and 4-byte aligned bases: each lane loads its 2 elements at once
  a.vec = (dtype == CQ_F16 || dtype == CQ_BF16) && a.D == 128 &&
          key_strides[2] >= 0 && value_strides[2] >= 0 &&
          ((key_strides[0] | key_strides[1] | key_strides[2] | value_strides[0] |
            value_strides[1] | value_strides[2]) & 1) == 0 &&
          (((uintptr_t)keys | (uintptr_t)values) & 3) == 0;
  a.offsets = offsets;
  a.offset = offset;
  // at most kAppendGroups workgroups (8 resident generations of 4-wave
  // groups on 256 CUs); each wave then takes kAppendRowsPerWave rows at a
  // time, every (grid waves)-th row
  const int64_t per_group = 4 * kAppendRowsPerWave;
  const dim3 grid((unsigned)std::min<int64_t>((items + per_group - 1) / per_group, kAppendGroups)),
      block(256);
  hipStream_t s = (hipStream_t)stream;
  // head_dim 128, 16-bit tokens whose rows start 16-byte aligned, 16-byte
  // aligned keyframe rows: four rows per wave
  const bool row4 = (dtype == CQ_F16 || dtype == CQ_BF16) && a.D == 128 &&
                    ((key_strides[0] | key_strides[1] | key_strides[2] | value_strides[0] |
                      value_strides[1] | value_strides[2]) & 7) == 0 &&
                    key_strides[2] >= 0 && value_strides[2] >= 0 &&
                    (((uintptr_t)keys | (uintptr_t)values | (uintptr_t)cache->k.keyframes |
                      (uintptr_t)cache->v.keyframes) & 15) == 0;
  if (row4) {
    const dim3 g4((unsigned)std::min<int64_t>((items + 15) / 16, kAppendGroups));
    if (dtype == CQ_F16) append_row4_kernel<CQ_F16><<<g4, block, 0, s>>>(a);
    else append_row4_kernel<CQ_BF16><<<g4, block, 0, s>>>(a);
    return launch_status();
  }
  switch (dtype) {
    case CQ_F16: append_kernel<CQ_F16><<<grid, block, 0, s>>>(a); break;
    case CQ_BF16: append_kernel<CQ_BF16><<<grid, block, 0, s>>>(a); break;
    case CQ_F32: append_kernel<CQ_F32><<<grid, block, 0, s>>>(a); break;
    default: return CQ_ERR_DTYPE;
  }
  return launch_status();
}

int cq_qkv_rope_append(const cq_cache_desc *cache, const void *qkv, const void *q_w,
                       const void *k_w, void *q_out, const float *cos_t, const float *sin_t,
                       int64_t max_pos, const int64_t *positions, int64_t pos_bstride,
                       int32_t n_q_heads, float eps, int32_t dtype, const int32_t *offsets,
                       int64_t offset, int32_t *lengths, cq_stream_t stream) {
  int st = validate_cache(cache);
  if (st) return st;
  if (!qkv || !q_out || !cos_t || !sin_t || !positions) return CQ_ERR_ARG;
  if (offset < 0 || max_pos < 1 || pos_bstride < 0) return CQ_ERR_ARG;
  if (cache->head_dim != 128) return CQ_ERR_UNSUPPORTED;
  if (n_q_heads < 1) return CQ_ERR_SHAPE;
  if (dtype != CQ_F16 && dtype != CQ_BF16 && dtype != CQ_F32) return CQ_ERR_DTYPE;
  if (!offsets) {
    for (const cq_component *p : {&cache->k, &cache->v}) {
      if (num_keyframes(offset + 1, p->stride) > p->cap_keyframes ||
          num_pframes(offset + 1, p->stride) > p->cap_pframes)
        return CQ_ERR_CAPACITY;
    }
  }
  // the keyframe rows are read 4 bytes per lane
  if (((uintptr_t)cache->k.keyframes | (uintptr_t)cache->v.keyframes) & 3) return CQ_ERR_ALIGN;
  RopeAppendArgs a;
  a.comp[0] = cache->k;
  a.comp[1] = cache->v;
  a.qkv = qkv;
  a.q_w = q_w;
  a.k_w = k_w;
  a.q_out = q_out;
  a.cos_t = cos_t;
  a.sin_t = sin_t;
  a.positions = positions;
  a.pos_bstride = pos_bstride;
  a.max_pos = max_pos;
  a.offsets = offsets;
  a.offset = offset;
  a.lengths = lengths;
  a.B = cache->batch;
  a.nq = n_q_heads;
  a.nkv = cache->n_kv_heads;
  a.W = 16;
  a.eps = eps;
  const int64_t rows = (int64_t)a.B * (a.nq + 2 * a.nkv);
  if (rows >= 0x7fffffff - 4) return CQ_ERR_SHAPE;  // 32-bit row indices in the kernel
  const dim3 grid((unsigned)((rows + 3) / 4)), block(256);
  hipStream_t s = (hipStream_t)stream;
  switch (dtype) {
    case CQ_F16: rope_append_kernel<CQ_F16><<<grid, block, 0, s>>>(a); break;
    case CQ_BF16: rope_append_kernel<CQ_BF16><<<grid, block, 0, s>>>(a); break;
    default: rope_append_kernel<CQ_F32><<<grid, block, 0, s>>>(a); break;
  }
  return launch_status();
}

int cq_reconstruct(const cq_cache_desc *cache, int32_t component, int64_t seq_len,
                   uint16_t *out, cq_stream_t stream) {
  int st = validate_cache(cache);
  if (st) return st;
  if (component != CQ_KEYS && component != CQ_VALUES) return CQ_ERR_ARG;
  if (seq_len < 0) return CQ_ERR_ARG;
  if (seq_len == 0) return CQ_OK;
  if (!out) return CQ_ERR_ARG;
  const cq_component &c = component == CQ_KEYS ? cache->k : cache->v;
  if (num_keyframes(seq_len, c.stride) > c.cap_keyframes ||
      num_pframes(seq_len, c.stride) > c.cap_pframes)
    return CQ_ERR_CAPACITY;
  const int D = cache->head_dim, W = (D + 7) / 8;
  const int64_t total = (int64_t)cache->batch * cache->n_kv_heads * seq_len * W;
  reconstruct_kernel<<<dim3((unsigned)((total + 255) / 256)), dim3(256), 0,
                       (hipStream_t)stream>>>(c, cache->batch, cache->n_kv_heads, D, W,
                                              seq_len, out);
  return launch_status();
}

}  // extern "C"
