/*
 * cq_oracle.c — CPU restatement of the ChronoQuant hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the parity checker for the HIP
 * kernels in chronoquant_mlx_amd/csrc and the timed CPU baseline of bench.py.
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
 * load it; the product path never does.
 *
 * It restates, function by function, the reference implementation
 * (gauravsaini/chronoquant_mlx, MLX/Metal) with every floating-point
 * rounding point made explicit:
 *   cqo_quantize_delta        codec.py:23-65   (ChronoQuantCodecMLX.quantize_delta)
 *   cqo_pack_int4             kernels.py:34-54 + MSL kernels.py:9-22
 *   cqo_unpack_int4           kernels.py:57-61
 *   cqo_append_component      cache.py:87-129  (one sequence, H heads)
 *   cqo_reconstruct_component cache.py:131-156
 *   cqo_sdpa_fallback         attention.py:8-20 + 61-74 (reconstruct + dense SDPA)
 *   cqo_sdpa_fallback_mask    the same with a boolean array mask (attention.py:18-19)
 *   cqo_sdpa_fallback_bf16q   the same for bf16 queries (fp32 scores and weights)
 *   cqo_sdpa_fused            MSL kernels.py:79-228 (fp32 dequant, online softmax)
 *   cqo_sdpa_exact            textbook softmax attention in binary64 (closed form)
 * Arithmetic model: MLX evaluates fp16/bf16 elementwise ops with the result
 * rounded to the array dtype (round-to-nearest-even); Python scalars are weak
 * and take the array's dtype (so 1e-10 becomes fp16 0).  Each op below is
 * computed exactly or in binary32 and then rounded to the dtype; binary32 has
 * p = 24 >= 2*11 + 2, so double rounding through binary32 is innocuous for
 * + - * / in fp16 and bf16.
 *
 * Residual assumptions (not observable without MLX, which this environment
 * lacks): mx.round rounds half to even; a NaN code (0/0 when a row's residual
 * is all zero in fp16) converts to int8 0; fp16 matmuls in the fallback
 * accumulate exactly and round once (this oracle accumulates in binary64).
 *
 * Build: oracle/Makefile (gcc, -ffp-contract=off so no FMA contraction).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

enum { DT_F16 = 0, DT_BF16 = 1, DT_F32 = 2 };

/* ------------------------------------------------------------------------ */
/* IEEE binary16 and bfloat16, round to nearest even, written from the      */
/* format definitions.                                                       */
/* ------------------------------------------------------------------------ */

static inline uint32_t f32_bits(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  return u;
}
static inline float bits_f32(uint32_t u) {
  float f;
  memcpy(&f, &u, 4);
  return f;
}

float cqo_h2f(uint16_t h) {
  uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  uint32_t exp = (h >> 10) & 0x1fu;
  uint32_t man = h & 0x3ffu;
  if (exp == 0x1f) return bits_f32(sign | 0x7f800000u | (man << 13));
  if (exp == 0) {
    /* zero or subnormal: man * 2^-24, exact in binary32 */
    float v = (float)man * 5.9604644775390625e-08f;
    return sign ? -v : v;
  }
  return bits_f32(sign | ((exp + 112u) << 23) | (man << 13));
}

uint16_t cqo_f2h(float f) {
  uint32_t x = f32_bits(f);
  uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
  uint32_t ax = x & 0x7fffffffu;
  if (ax > 0x7f800000u) return sign | 0x7e00u | (uint16_t)((ax >> 13) & 0x3ffu);
  if (ax >= 0x477ff000u) return sign | 0x7c00u; /* >= 65520 rounds to inf */
  if (ax < 0x38800000u) {                       /* below 2^-14: subnormal */
    if (ax <= 0x33000000u) return sign;         /* <= 2^-25 rounds to 0 */
    uint32_t e = ax >> 23;
    uint32_t m = (ax & 0x7fffffu) | 0x800000u;
    uint32_t shift = 126u - e; /* units of 2^-24 */
    uint32_t n = m >> shift;
    uint32_t rem = m & ((1u << shift) - 1u);
    uint32_t half = 1u << (shift - 1u);
    if (rem > half || (rem == half && (n & 1u))) n++;
    return sign | (uint16_t)n;
  }
  uint32_t h = ((ax >> 23) - 112u) << 10 | ((ax & 0x7fffffu) >> 13);
  uint32_t rem = ax & 0x1fffu;
  if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
  return sign | (uint16_t)h;
}

float cqo_bf2f(uint16_t b) { return bits_f32((uint32_t)b << 16); }

uint16_t cqo_f2bf(float f) {
  uint32_t x = f32_bits(f);
  if ((x & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((x >> 16) | 0x40u);
  uint32_t lsb = (x >> 16) & 1u;
  x += 0x7fffu + lsb;
  return (uint16_t)(x >> 16);
}

/* round a binary32 value to the dtype and back */
static inline float rnd(int dt, float x) {
  if (dt == DT_F16) return cqo_h2f(cqo_f2h(x));
  if (dt == DT_BF16) return cqo_bf2f(cqo_f2bf(x));
  return x;
}

static inline float load_dt(int dt, const void *p, int64_t i) {
  if (dt == DT_F16) return cqo_h2f(((const uint16_t *)p)[i]);
  if (dt == DT_BF16) return cqo_bf2f(((const uint16_t *)p)[i]);
  return ((const float *)p)[i];
}

/* round half to even, written out (independent of the FP environment) */
static inline float rint_half_even(float x) {
  float fl = floorf(x);
  float diff = x - fl; /* exact for |x| < 2^23 */
  if (diff > 0.5f) return fl + 1.0f;
  if (diff < 0.5f) return fl;
  return (fmodf(fl, 2.0f) == 0.0f) ? fl : fl + 1.0f;
}

/* ------------------------------------------------------------------------ */
/* codec.py:23-65 — ChronoQuantCodecMLX.quantize_delta                       */
/* ------------------------------------------------------------------------ */
static void quantize_row(int dt, const float *delta_in, int D, int bits,
                         float dz, int8_t *codes, uint16_t *scale_out,
                         float *work) {
  const int half_levels = (1 << bits) / 2;        /* codec.py:14 */
  const float hm1 = (float)(half_levels - 1);     /* weak int -> dtype, exact */
  const float eps = rnd(dt, 1e-10f);              /* weak 1e-10 -> dtype */
  float amax = 0.0f;                              /* codec.py:32 */
  for (int d = 0; d < D; ++d) {
    float a = fabsf(delta_in[d]);
    if (a > amax) amax = a;
    work[d] = delta_in[d];
  }
  float scale = rnd(dt, amax / hm1); /* codec.py:33 */
  if (dz > 0.0f) {                   /* codec.py:36-45 */
    float thr = rnd(dt, amax * rnd(dt, dz));
    float amax_c = 0.0f;
    for (int d = 0; d < D; ++d) {
      if (fabsf(work[d]) < thr) work[d] = 0.0f;
      float a = fabsf(work[d]);
      if (a > amax_c) amax_c = a;
    }
    float amax_safe = (amax_c < eps) ? amax : amax_c;
    scale = rnd(dt, amax_safe / hm1);
  }
  float scale_safe = (scale < eps) ? 1.0f : scale; /* codec.py:48 */
  for (int d = 0; d < D; ++d) {
    float q = rnd(dt, work[d] / scale_safe); /* codec.py:50: dtype division */
    int c;
    if (isnan(q)) {
      c = 0; /* defined: NaN converts to code 0 */
    } else {
      float r = rint_half_even(q);
      if (r < (float)(-half_levels)) r = (float)(-half_levels); /* codec.py:51 */
      if (r > hm1) r = hm1;
      c = (int)r;
    }
    if (scale < eps) c = 0; /* codec.py:54 */
    codes[d] = (int8_t)c;
  }
  /* codec.py:65: scale.astype(float16) */
  *scale_out = cqo_f2h(scale);
}

/* delta: [n_rows][D] of dtype; codes int8 [n_rows][D]; scales fp16 [n_rows] */
void cqo_quantize_delta(int dt, const void *delta, int64_t n_rows, int D,
                        int bits, float dz, int8_t *codes, uint16_t *scales) {
  float *row = (float *)malloc(sizeof(float) * (size_t)D * 2);
  for (int64_t r = 0; r < n_rows; ++r) {
    for (int d = 0; d < D; ++d) row[d] = load_dt(dt, delta, r * D + d);
    quantize_row(dt, row, D, bits, dz, codes + r * D, scales + r, row + D);
  }
  free(row);
}

/* ------------------------------------------------------------------------ */
/* kernels.py:34-54 (+ MSL :9-22) and kernels.py:57-61                       */
/* ------------------------------------------------------------------------ */
static void pack_row(const int8_t *codes, int D, uint32_t *out) {
  int W = (D + 7) / 8;
  for (int w = 0; w < W; ++w) {
    uint32_t word = 0;
    for (int i = 0; i < 8; ++i) {
      int d = 8 * w + i;
      uint32_t nib = 0; /* pad nibble (kernels.py:41-43) */
      if (d < D) {
        int u = (int)codes[d] + 8;
        if (u < 0) u = 0;
        if (u > 15) u = 15;
        nib = (uint32_t)u;
      }
      word |= (nib & 0xfu) << (4 * i);
    }
    out[w] = word;
  }
}

void cqo_pack_int4(const int8_t *codes, int64_t n_rows, int D, uint32_t *packed) {
  int W = (D + 7) / 8;
  for (int64_t r = 0; r < n_rows; ++r) pack_row(codes + r * D, D, packed + r * W);
}

void cqo_unpack_int4(const uint32_t *packed, int64_t n_rows, int D, int8_t *codes) {
  int W = (D + 7) / 8;
  for (int64_t r = 0; r < n_rows; ++r)
    for (int d = 0; d < D; ++d)
      codes[r * D + d] =
          (int8_t)((int)((packed[r * W + d / 8] >> (4 * (d % 8))) & 0xfu) - 8);
}

/* ------------------------------------------------------------------------ */
/* cache.py:53-61 and 87-129 — one sequence, H heads                         */
/* ------------------------------------------------------------------------ */
int64_t cqo_num_keyframes(int64_t n, int stride) {
  return n <= 0 ? 0 : (n - 1) / stride + 1;
}
int64_t cqo_num_pframes(int64_t n, int stride) {
  return n - cqo_num_keyframes(n, stride);
}

/*
 * Component storage of one sequence:
 *   kf fp16 [H][cap_kf][D], pk uint32 [H][cap_pf][W], sc fp16 [H][cap_pf]
 * x: new tokens, element (h, s, d) at x[h*sh + s*ss + d] of dtype.
 * Returns 0, or -1 if a capacity would be exceeded.
 */
int cqo_append_component(int dt, const void *x, int64_t sh, int64_t ss,
                         int H, int D, int64_t S, int64_t offset, int stride,
                         int bits, float dz, uint16_t *kf, int64_t cap_kf,
                         uint32_t *pk, int64_t cap_pf, uint16_t *sc) {
  int W = (D + 7) / 8;
  if (cqo_num_keyframes(offset + S, stride) > cap_kf) return -1;
  if (cqo_num_pframes(offset + S, stride) > cap_pf) return -1;
  float *delta = (float *)malloc(sizeof(float) * (size_t)D * 2);
  int8_t *codes = (int8_t *)malloc((size_t)D);
  for (int64_t ls = 0; ls < S; ++ls) { /* cache.py:99 */
    int64_t t = offset + ls;
    for (int h = 0; h < H; ++h) {
      int64_t xb = h * sh + ls * ss;
      if (t % stride == 0) { /* cache.py:103-105: I-frame = fp16(token) */
        uint16_t *row = kf + ((int64_t)h * cap_kf + t / stride) * D;
        for (int d = 0; d < D; ++d) row[d] = cqo_f2h(load_dt(dt, x, xb + d));
        continue;
      }
      int64_t g = t / stride; /* cache.py:107-111 */
      const uint16_t *anc = kf + ((int64_t)h * cap_kf + g) * D;
      for (int d = 0; d < D; ++d) { /* cache.py:113: token - anchor.astype */
        float a = rnd(dt, cqo_h2f(anc[d]));
        delta[d] = rnd(dt, load_dt(dt, x, xb + d) - a);
      }
      int64_t slot = t - g - 1;
      uint16_t sv;
      quantize_row(dt, delta, D, bits, dz, codes, &sv, delta + D); /* :114 */
      pack_row(codes, D, pk + ((int64_t)h * cap_pf + slot) * W);   /* :115 */
      sc[(int64_t)h * cap_pf + slot] = sv;                         /* :116 */
    }
  }
  free(delta);
  free(codes);
  return 0;
}

/* cache.py:131-156: out fp16 [H][T][D] */
void cqo_reconstruct_component(int H, int D, int64_t T, int stride,
                               const uint16_t *kf, int64_t cap_kf,
                               const uint32_t *pk, int64_t cap_pf,
                               const uint16_t *sc, uint16_t *out) {
  int W = (D + 7) / 8;
  for (int h = 0; h < H; ++h)
    for (int64_t t = 0; t < T; ++t) {
      int64_t g = t / stride;
      const uint16_t *anc = kf + ((int64_t)h * cap_kf + g) * D;
      uint16_t *o = out + ((int64_t)h * T + t) * D;
      int is_p = (t % stride) != 0;
      int64_t slot = is_p ? t - g - 1 : 0;
      float s = is_p ? cqo_h2f(sc[(int64_t)h * cap_pf + slot]) : 0.0f;
      const uint32_t *row = pk + ((int64_t)h * cap_pf + slot) * W;
      for (int d = 0; d < D; ++d) {
        float delta = 0.0f; /* mx.where(is_pframe, delta, zeros) */
        if (is_p) {
          int c = (int)((row[d / 8] >> (4 * (d % 8))) & 0xfu) - 8;
          delta = cqo_h2f(cqo_f2h((float)c * s)); /* codec.py:73, fp16 mul */
        }
        o[d] = cqo_f2h(cqo_h2f(anc[d]) + delta); /* cache.py:156, fp16 add */
      }
    }
}

/* ------------------------------------------------------------------------ */
/* attention.py:8-20 + 61-74 — reconstruct fallback, fp16 queries           */
/* ------------------------------------------------------------------------ */
/*
 * q: fp16 [nq][Tq][D]; rk, rv: fp16 [H][T][D]; out fp16 [nq][Tq][D].
 * causal != 0 applies the "causal" string mask (attention.py:12-16); mask
 * (uint8 [Tq][T], may be NULL) is a boolean array mask (attention.py:18-19:
 * where(mask, scores, finfo(fp16).min)), applied after the causal one.
 */
void cqo_sdpa_fallback_mask(const uint16_t *q, const uint16_t *rk,
                            const uint16_t *rv, int nq, int H, int64_t Tq,
                            int64_t T, int D, float scale, int causal,
                            const uint8_t *mask, uint16_t *out) {
  int rep = nq / H; /* attention.py:50 */
  float scale_h = cqo_h2f(cqo_f2h(scale));
#pragma omp parallel
  {
    float *qs = (float *)malloc(sizeof(float) * D);
    float *sc = (float *)malloc(sizeof(float) * (size_t)T);
    double *acc = (double *)malloc(sizeof(double) * D);
#pragma omp for collapse(2) schedule(static)
    for (int j = 0; j < nq; ++j)
      for (int64_t i = 0; i < Tq; ++i) {
        int h = j / rep;
        const uint16_t *qr = q + ((int64_t)j * Tq + i) * D;
        for (int d = 0; d < D; ++d) /* attention.py:52 q_scaled, fp16 */
          qs[d] = cqo_h2f(cqo_f2h(cqo_h2f(qr[d]) * scale_h));
        float mx = -INFINITY;
        for (int64_t t = 0; t < T; ++t) { /* attention.py:57 scores, fp16 */
          const uint16_t *kr = rk + ((int64_t)h * T + t) * D;
          double s = 0.0;
          for (int d = 0; d < D; ++d) s += (double)qs[d] * (double)cqo_h2f(kr[d]);
          float sf = cqo_h2f(cqo_f2h((float)s));
          if (causal && (T - Tq + i) < t) sf = -65504.0f; /* finfo(fp16).min */
          if (mask && !mask[i * T + t]) sf = -65504.0f;
          sc[t] = sf;
          if (sf > mx) mx = sf;
        }
        double den = 0.0; /* softmax(precise=True): fp32 internals */
        for (int64_t t = 0; t < T; ++t) den += exp((double)sc[t] - (double)mx);
        for (int d = 0; d < D; ++d) acc[d] = 0.0;
        for (int64_t t = 0; t < T; ++t) {
          float w = cqo_h2f(cqo_f2h((float)(exp((double)sc[t] - (double)mx) / den)));
          const uint16_t *vr = rv + ((int64_t)h * T + t) * D;
          for (int d = 0; d < D; ++d) acc[d] += (double)w * (double)cqo_h2f(vr[d]);
        }
        uint16_t *o = out + ((int64_t)j * Tq + i) * D;
        for (int d = 0; d < D; ++d) o[d] = cqo_f2h((float)acc[d]);
      }
    free(qs);
    free(sc);
    free(acc);
  }
}

void cqo_sdpa_fallback(const uint16_t *q, const uint16_t *rk,
                       const uint16_t *rv, int nq, int H, int64_t Tq,
                       int64_t T, int D, float scale, int causal,
                       uint16_t *out) {
  cqo_sdpa_fallback_mask(q, rk, rv, nq, H, Tq, T, D, scale, causal, NULL, out);
}

/*
 * The same fallback for bf16 queries over the fp16 reconstruction.  MLX
 * promotes bf16 x fp16 to fp32, so (attention.py:61-74): q_scaled =
 * bf16(q * bf16(scale)) (:65, the weak scalar takes the array's dtype);
 * scores = q_scaled @ k^T in fp32 (:70); masked entries take
 * finfo(float32).min (:12-19); softmax(precise=True) in fp32 gives fp32
 * weights (:72); weights @ v in fp32 (:73); one rounding to bf16 (:74).
 * q: bf16 [nq][Tq][D]; out: bf16 [nq][Tq][D].
 */
void cqo_sdpa_fallback_bf16q(const uint16_t *q, const uint16_t *rk,
                             const uint16_t *rv, int nq, int H, int64_t Tq,
                             int64_t T, int D, float scale, int causal,
                             const uint8_t *mask, uint16_t *out) {
  int rep = nq / H;
  float scale_b = cqo_bf2f(cqo_f2bf(scale));
#pragma omp parallel
  {
    float *qs = (float *)malloc(sizeof(float) * D);
    float *sc = (float *)malloc(sizeof(float) * (size_t)T);
    double *acc = (double *)malloc(sizeof(double) * D);
#pragma omp for collapse(2) schedule(static)
    for (int j = 0; j < nq; ++j)
      for (int64_t i = 0; i < Tq; ++i) {
        int h = j / rep;
        const uint16_t *qr = q + ((int64_t)j * Tq + i) * D;
        for (int d = 0; d < D; ++d) qs[d] = cqo_bf2f(cqo_f2bf(cqo_bf2f(qr[d]) * scale_b));
        float mx = -INFINITY;
        for (int64_t t = 0; t < T; ++t) {
          const uint16_t *kr = rk + ((int64_t)h * T + t) * D;
          double s = 0.0;
          for (int d = 0; d < D; ++d) s += (double)qs[d] * (double)cqo_h2f(kr[d]);
          float sf = (float)s;
          if ((causal && (T - Tq + i) < t) || (mask && !mask[i * T + t]))
            sf = -3.4028234663852886e38f; /* finfo(float32).min */
          sc[t] = sf;
          if (sf > mx) mx = sf;
        }
        double den = 0.0;
        for (int64_t t = 0; t < T; ++t) den += exp((double)sc[t] - (double)mx);
        for (int d = 0; d < D; ++d) acc[d] = 0.0;
        for (int64_t t = 0; t < T; ++t) {
          float w = (float)(exp((double)sc[t] - (double)mx) / den);
          const uint16_t *vr = rv + ((int64_t)h * T + t) * D;
          for (int d = 0; d < D; ++d) acc[d] += (double)w * (double)cqo_h2f(vr[d]);
        }
        uint16_t *o = out + ((int64_t)j * Tq + i) * D;
        for (int d = 0; d < D; ++d) o[d] = cqo_f2bf((float)acc[d]);
      }
    free(qs);
    free(sc);
    free(acc);
  }
}

/* ------------------------------------------------------------------------ */
/* MSL kernels.py:79-228 semantics: k = fp32(a) + fp32(c)*fp32(s), q' =      */
/* fp32(fp16(q*scale)) (attention.py:46), output fp32.  Here the sums run in  */
/* binary64 so this is the fused kernel's math without its summation order.  */
/* ------------------------------------------------------------------------ */
/* absw (may be NULL): sum_t p_t |v_t| / sum_t p_t per output element, the
 * scale of a weighted sum's rounding error (a kernel whose weights carry
 * relative error u differs by at most u * absw). */
void cqo_sdpa_fused_absw(const uint16_t *q, int nq, int H, int D, int64_t T,
                         float scale, int stride_k, int stride_v,
                         const uint16_t *kf_k, int64_t cap_kf_k, const uint32_t *pk_k,
                         int64_t cap_pf_k, const uint16_t *sc_k,
                         const uint16_t *kf_v, int64_t cap_kf_v, const uint32_t *pk_v,
                         int64_t cap_pf_v, const uint16_t *sc_v, float *out, float *absw) {
  int rep = nq / H;
  int W = (D + 7) / 8;
  float scale_h = cqo_h2f(cqo_f2h(scale));
  /* q heads are independent: one per thread (same sums in the same order) */
#pragma omp parallel for schedule(dynamic, 1)
  for (int j = 0; j < nq; ++j) {
    int h = j / rep;
    double *sc = (double *)malloc(sizeof(double) * (size_t)T);
    double mx = -INFINITY;
    for (int64_t t = 0; t < T; ++t) {
      int64_t g = t / stride_k;
      int is_p = (t % stride_k) != 0;
      int64_t slot = is_p ? t - g - 1 : 0;
      float s = is_p ? cqo_h2f(sc_k[(int64_t)h * cap_pf_k + slot]) : 0.0f;
      double acc = 0.0;
      for (int d = 0; d < D; ++d) {
        float qd = cqo_h2f(cqo_f2h(cqo_h2f(q[(int64_t)j * D + d]) * scale_h));
        float kv = cqo_h2f(kf_k[((int64_t)h * cap_kf_k + g) * D + d]);
        if (is_p) {
          int c = (int)((pk_k[((int64_t)h * cap_pf_k + slot) * W + d / 8] >> (4 * (d % 8))) & 0xfu) - 8;
          kv = kv + (float)c * s;
        }
        acc += (double)qd * (double)kv;
      }
      sc[t] = acc;
      if (acc > mx) mx = acc;
    }
    double den = 0.0;
    double *o = (double *)calloc((size_t)D, sizeof(double));
    double *oa = (double *)calloc((size_t)D, sizeof(double));
    for (int64_t t = 0; t < T; ++t) {
      double p = exp(sc[t] - mx);
      den += p;
      int64_t g = t / stride_v;
      int is_p = (t % stride_v) != 0;
      int64_t slot = is_p ? t - g - 1 : 0;
      float s = is_p ? cqo_h2f(sc_v[(int64_t)h * cap_pf_v + slot]) : 0.0f;
      for (int d = 0; d < D; ++d) {
        float vv = cqo_h2f(kf_v[((int64_t)h * cap_kf_v + g) * D + d]);
        if (is_p) {
          int c = (int)((pk_v[((int64_t)h * cap_pf_v + slot) * W + d / 8] >> (4 * (d % 8))) & 0xfu) - 8;
          vv = vv + (float)c * s;
        }
        o[d] += p * (double)vv;
        oa[d] += p * fabs((double)vv);
      }
    }
    for (int d = 0; d < D; ++d) out[(int64_t)j * D + d] = (float)(den > 0 ? o[d] / den : 0.0);
    if (absw)
      for (int d = 0; d < D; ++d) absw[(int64_t)j * D + d] = (float)(den > 0 ? oa[d] / den : 0.0);
    free(o);
    free(oa);
    free(sc);
  }
}

void cqo_sdpa_fused(const uint16_t *q, int nq, int H, int D, int64_t T,
                    float scale, int stride_k, int stride_v,
                    const uint16_t *kf_k, int64_t cap_kf_k, const uint32_t *pk_k,
                    int64_t cap_pf_k, const uint16_t *sc_k,
                    const uint16_t *kf_v, int64_t cap_kf_v, const uint32_t *pk_v,
                    int64_t cap_pf_v, const uint16_t *sc_v, float *out) {
  cqo_sdpa_fused_absw(q, nq, H, D, T, scale, stride_k, stride_v, kf_k, cap_kf_k, pk_k,
                      cap_pf_k, sc_k, kf_v, cap_kf_v, pk_v, cap_pf_v, sc_v, out, NULL);
}

/* Textbook attention in binary64: out[j] = sum_t softmax(q'_j . k_t) v_t, */
/* q' = q*scale exactly (no fp16 rounding); k, v fp16 [H][T][D].            */
void cqo_sdpa_exact(const uint16_t *q, const uint16_t *k, const uint16_t *v,
                    int nq, int H, int64_t T, int D, double scale, double *out) {
  int rep = nq / H;
  double *sc = (double *)malloc(sizeof(double) * (size_t)T);
  for (int j = 0; j < nq; ++j) {
    int h = j / rep;
    double mx = -INFINITY;
    for (int64_t t = 0; t < T; ++t) {
      double s = 0.0;
      for (int d = 0; d < D; ++d)
        s += (double)cqo_h2f(q[(int64_t)j * D + d]) * scale *
             (double)cqo_h2f(k[((int64_t)h * T + t) * D + d]);
      sc[t] = s;
      if (s > mx) mx = s;
    }
    double den = 0.0;
    for (int64_t t = 0; t < T; ++t) den += exp(sc[t] - mx);
    for (int d = 0; d < D; ++d) {
      double a = 0.0;
      for (int64_t t = 0; t < T; ++t)
        a += exp(sc[t] - mx) * (double)cqo_h2f(v[((int64_t)h * T + t) * D + d]);
      out[(int64_t)j * D + d] = a / den;
    }
  }
  free(sc);
}

/* ------------------------------------------------------------------------ */
/* CPU baseline step (bench.py): the reference's per-layer decode work for  */
/* one sequence: reconstruct K and V (cache.py:131-160) then the dense      */
/* fallback SDPA (attention.py:61-74).  rk/rv/out are caller scratch.       */
/* ------------------------------------------------------------------------ */
int cqo_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}

void cqo_set_threads(int n) {
#ifdef _OPENMP
  if (n > 0) omp_set_num_threads(n);
#else
  (void)n;
#endif
}

void cqo_decode_step(const uint16_t *q, int nq, int H, int D, int64_t T,
                     float scale, int stride_k, int stride_v,
                     const uint16_t *kf_k, int64_t cap_kf_k, const uint32_t *pk_k,
                     int64_t cap_pf_k, const uint16_t *sc_k,
                     const uint16_t *kf_v, int64_t cap_kf_v, const uint32_t *pk_v,
                     int64_t cap_pf_v, const uint16_t *sc_v, uint16_t *rk,
                     uint16_t *rv, uint16_t *out) {
#pragma omp parallel for schedule(static)
  for (int h = 0; h < H; ++h) {
    cqo_reconstruct_component(1, D, T, stride_k, kf_k + (int64_t)h * cap_kf_k * D,
                              cap_kf_k, pk_k + (int64_t)h * cap_pf_k * ((D + 7) / 8),
                              cap_pf_k, sc_k + (int64_t)h * cap_pf_k,
                              rk + (int64_t)h * T * D);
    cqo_reconstruct_component(1, D, T, stride_v, kf_v + (int64_t)h * cap_kf_v * D,
                              cap_kf_v, pk_v + (int64_t)h * cap_pf_v * ((D + 7) / 8),
                              cap_pf_v, sc_v + (int64_t)h * cap_pf_v,
                              rv + (int64_t)h * T * D);
  }
  cqo_sdpa_fallback(q, rk, rv, nq, H, 1, T, D, scale, 0, out);
}

/* bulk conversions, exposed for the oracle's own tests */
void cqo_f32_to_f16_array(const float *in, int64_t n, uint16_t *out) {
  for (int64_t i = 0; i < n; ++i) out[i] = cqo_f2h(in[i]);
}
void cqo_f16_to_f32_array(const uint16_t *in, int64_t n, float *out) {
  for (int64_t i = 0; i < n; ++i) out[i] = cqo_h2f(in[i]);
}
void cqo_f32_to_bf16_array(const float *in, int64_t n, uint16_t *out) {
  for (int64_t i = 0; i < n; ++i) out[i] = cqo_f2bf(in[i]);
}
