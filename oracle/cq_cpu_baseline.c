/*
 * CPU baseline of the fused compressed decode, fp32 (TEST INFRASTRUCTURE:
 * used only by bench.py's cpu_baseline leg and by the tests that check it).
 *
 * cqb_fused_decode_f32 computes what the reference's fused operator
 * computes (kernels.py:79-228, called as kernels.py:248-279 from
 * attention.py:46-58): per query head j of kv head h = j / rep,
 *   k_t = fp32(keyframe[t / stride_k]) + fp32(code_t) * fp32(scale_t)
 *         (the keyframe alone when t % stride_k == 0),
 *   v_t likewise with stride_v,
 *   out_j = sum_t exp(q'_j . k_t - m) v_t / sum_t exp(q'_j . k_t - m),
 * with q' = fp32(fp16(q * fp16(scale))) (attention.py:46) and fp32
 * accumulation, as the reference's kernel does.  It is built for speed on
 * a host CPU rather than as a restatement of the reference's summation
 * order:
 *   - the keys of one kv head are split into chunks, one (head, chunk) task
 *     per OpenMP iteration, merged in chunk order at the end;
 *   - each K/V row is decoded once and used by all rep query heads of its
 *     kv head (GQA sharing);
 *   - within a chunk the softmax runs blockwise (32 keys: scores, block
 *     maximum, rescale, exponentials, weighted V sum), with AVX2/FMA/F16C
 *     over the head dimension and a polynomial exponential (cqb_exp8).
 * Its result agrees with cqo_sdpa_fused (binary64 sums) to fp32 rounding,
 * which the oracle's tests check.
 */
#include <immintrin.h>
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define CQB_BLOCK 32   /* keys per softmax block */
#define CQB_MAX_REP 16 /* query heads per kv head */
#define CQB_MAX_D 256

static inline float cqb_round_f16(float x) {
  return _cvtsh_ss(_cvtss_sh(x, _MM_FROUND_TO_NEAREST_INT));
}

/* One decoded row (D floats): keyframe row `anc` plus, for a P-frame, the
 * INT4 lanes of `pk` (word w holds dims 8w..8w+7, dim 8w+i in bits 4i..4i+3,
 * code = nibble - 8; kernels.py:56-77) times `s`. */
static inline void cqb_row(const uint16_t *anc, const uint32_t *pk, float s,
                           int is_p, int D, float *o) {
  const __m256i sh = _mm256_setr_epi32(0, 4, 8, 12, 16, 20, 24, 28);
  const __m256i m15 = _mm256_set1_epi32(15), m8 = _mm256_set1_epi32(8);
  const __m256 vs = _mm256_set1_ps(s);
  for (int w = 0; w < D / 8; ++w) {
    __m256 a = _mm256_cvtph_ps(_mm_loadu_si128((const __m128i *)(anc + 8 * w)));
    if (is_p) {
      __m256i c = _mm256_srlv_epi32(_mm256_set1_epi32((int)pk[w]), sh);
      c = _mm256_sub_epi32(_mm256_and_si256(c, m15), m8);
      a = _mm256_add_ps(a, _mm256_mul_ps(_mm256_cvtepi32_ps(c), vs));
    }
    _mm256_storeu_ps(o + 8 * w, a);
  }
}

static inline float cqb_hsum(__m256 v) {
  __m128 lo = _mm256_castps256_ps128(v), hi = _mm256_extractf128_ps(v, 1);
  lo = _mm_add_ps(lo, hi);
  lo = _mm_add_ps(lo, _mm_movehl_ps(lo, lo));
  lo = _mm_add_ss(lo, _mm_movehdup_ps(lo));
  return _mm_cvtss_f32(lo);
}

/* exp of 8 floats for x <= 0 (scores minus their running maximum):
 * Cody-Waite reduction x = n ln2 + r, |r| <= ln2/2, with ln2 split in a
 * short high part (exact products n * hi) and a low correction, then
 * e^r by its Taylor series to r^7 (truncation below 6e-9 relative, under
 * half an fp32 ulp) and 2^n built in the exponent field.  x below -87
 * (results below fp32's normal range) gives 0; -inf gives 0. */
static inline __m256 cqb_exp8(__m256 x) {
  const __m256 lo_lim = _mm256_set1_ps(-87.0f);
  __m256 under = _mm256_cmp_ps(x, lo_lim, _CMP_LT_OQ);
  x = _mm256_max_ps(x, lo_lim);
  x = _mm256_min_ps(x, _mm256_set1_ps(88.0f));
  __m256 n = _mm256_round_ps(_mm256_mul_ps(x, _mm256_set1_ps(1.44269504088896341f)),
                             _MM_FROUND_TO_NEAREST_INT | _MM_FROUND_NO_EXC);
  __m256 r = _mm256_fnmadd_ps(n, _mm256_set1_ps(0.693359375f), x);
  r = _mm256_fnmadd_ps(n, _mm256_set1_ps(-2.12194440e-4f), r);
  __m256 p = _mm256_set1_ps(1.0f / 5040.0f);
  p = _mm256_fmadd_ps(p, r, _mm256_set1_ps(1.0f / 720.0f));
  p = _mm256_fmadd_ps(p, r, _mm256_set1_ps(1.0f / 120.0f));
  p = _mm256_fmadd_ps(p, r, _mm256_set1_ps(1.0f / 24.0f));
  p = _mm256_fmadd_ps(p, r, _mm256_set1_ps(1.0f / 6.0f));
  p = _mm256_fmadd_ps(p, r, _mm256_set1_ps(0.5f));
  p = _mm256_fmadd_ps(p, r, _mm256_set1_ps(1.0f));
  p = _mm256_fmadd_ps(p, r, _mm256_set1_ps(1.0f));
  __m256i e = _mm256_slli_epi32(_mm256_add_epi32(_mm256_cvtps_epi32(n), _mm256_set1_epi32(127)), 23);
  p = _mm256_mul_ps(p, _mm256_castsi256_ps(e));
  return _mm256_andnot_ps(under, p);
}

/* Sum of each of 8 vectors, as one vector: lane k = sum of a[k]. */
static inline __m256 cqb_sum8x8(const __m256 *a) {
  __m256 t0 = _mm256_hadd_ps(a[0], a[1]), t1 = _mm256_hadd_ps(a[2], a[3]);
  __m256 t2 = _mm256_hadd_ps(a[4], a[5]), t3 = _mm256_hadd_ps(a[6], a[7]);
  __m256 u0 = _mm256_hadd_ps(t0, t1), u1 = _mm256_hadd_ps(t2, t3);
  return _mm256_add_ps(_mm256_permute2f128_ps(u0, u1, 0x20),
                       _mm256_permute2f128_ps(u0, u1, 0x31));
}

typedef struct {
  const uint16_t *kf;
  const uint32_t *pk;
  const uint16_t *sc;
  int64_t cap_kf, cap_pf;
  int stride;
} cqb_comp;

static inline void cqb_decode_row(const cqb_comp *c, int h, int D, int64_t t,
                                  float *o) {
  int64_t g = t / c->stride;
  int is_p = (t % c->stride) != 0;
  int64_t slot = is_p ? t - g - 1 : 0;
  float s = is_p ? _cvtsh_ss(c->sc[(int64_t)h * c->cap_pf + slot]) : 0.0f;
  cqb_row(c->kf + ((int64_t)h * c->cap_kf + g) * D,
          c->pk + ((int64_t)h * c->cap_pf + slot) * (D / 8), s, is_p, D, o);
}

/* acc[j][d0 .. d0 + 8 NR) = f[j] * acc + sum_i p[j][i] vb[i][d0 ..], for the
 * query heads j0 .. j0 + nj (nj <= 4), accumulators in registers. */
static inline __attribute__((always_inline)) void
cqb_pv_tile(float *acc, int D, int d0, int j0, int nj, int n, const float *vb,
            float p[][CQB_BLOCK], const float *f, const int NR) {
  __m256 a[4][4];
  for (int j = 0; j < nj; ++j)
    for (int r = 0; r < NR; ++r)
      a[j][r] = _mm256_mul_ps(_mm256_loadu_ps(acc + (size_t)(j0 + j) * D + d0 + 8 * r),
                              _mm256_set1_ps(f[j0 + j]));
  for (int i = 0; i < n; ++i) {
    __m256 v[4];
    for (int r = 0; r < NR; ++r) v[r] = _mm256_load_ps(vb + (size_t)i * D + d0 + 8 * r);
    for (int j = 0; j < nj; ++j) {
      __m256 pj = _mm256_set1_ps(p[j0 + j][i]);
      for (int r = 0; r < NR; ++r) a[j][r] = _mm256_fmadd_ps(pj, v[r], a[j][r]);
    }
  }
  for (int j = 0; j < nj; ++j)
    for (int r = 0; r < NR; ++r)
      _mm256_storeu_ps(acc + (size_t)(j0 + j) * D + d0 + 8 * r, a[j][r]);
}

/* One (kv head, key range) task: partial maximum m[j], sum l[j] and
 * unnormalised accumulator acc[j][D] for the rep query heads.  Per block
 * of keys: decode the K rows, the scores of 8 keys at a time per query
 * head, the block's maximum and exponentials, decode the V rows, then the
 * weighted V sums over register tiles of the head dimension. */
static void cqb_task(const float *qs, int rep, int D, int h, int64_t t0,
                     int64_t t1, const cqb_comp *K, const cqb_comp *V,
                     float *m, float *l, float *acc) {
  static __thread float kb[CQB_BLOCK * CQB_MAX_D] __attribute__((aligned(32)));
  static __thread float vb[CQB_BLOCK * CQB_MAX_D] __attribute__((aligned(32)));
  float sc[CQB_MAX_REP][CQB_BLOCK] __attribute__((aligned(32)));
  float f[CQB_MAX_REP];
  for (int j = 0; j < rep; ++j) {
    m[j] = -INFINITY;
    l[j] = 0.0f;
  }
  memset(acc, 0, sizeof(float) * (size_t)rep * D);
  for (int64_t b = t0; b < t1; b += CQB_BLOCK) {
    int n = (int)((t1 - b) < CQB_BLOCK ? (t1 - b) : CQB_BLOCK);
    int n8 = (n + 7) & ~7;
    for (int i = 0; i < n; ++i) cqb_decode_row(K, h, D, b + i, kb + (size_t)i * D);
    for (int i = n; i < n8; ++i) memset(kb + (size_t)i * D, 0, sizeof(float) * D);
    for (int j = 0; j < rep; ++j) {
      const float *qj = qs + (size_t)j * D;
      for (int i0 = 0; i0 < n8; i0 += 8) {
        __m256 a[8];
        for (int k = 0; k < 8; ++k) a[k] = _mm256_setzero_ps();
        for (int d = 0; d < D; d += 8) {
          __m256 qv = _mm256_loadu_ps(qj + d);
          for (int k = 0; k < 8; ++k)
            a[k] = _mm256_fmadd_ps(qv, _mm256_load_ps(kb + (size_t)(i0 + k) * D + d), a[k]);
        }
        _mm256_store_ps(&sc[j][i0], cqb_sum8x8(a));
      }
      for (int i = n; i < n8; ++i) sc[j][i] = -INFINITY; /* padding keys */
      __m256 mv = _mm256_set1_ps(m[j]);
      for (int i0 = 0; i0 < n8; i0 += 8) mv = _mm256_max_ps(mv, _mm256_load_ps(&sc[j][i0]));
      __m128 m4 = _mm_max_ps(_mm256_castps256_ps128(mv), _mm256_extractf128_ps(mv, 1));
      m4 = _mm_max_ps(m4, _mm_movehl_ps(m4, m4));
      m4 = _mm_max_ss(m4, _mm_movehdup_ps(m4));
      float bm = _mm_cvtss_f32(m4);
      __m256 bmv = _mm256_set1_ps(bm), sv = _mm256_setzero_ps();
      for (int i0 = 0; i0 < n8; i0 += 8) {
        __m256 e = cqb_exp8(_mm256_sub_ps(_mm256_load_ps(&sc[j][i0]), bmv));
        _mm256_store_ps(&sc[j][i0], e);
        sv = _mm256_add_ps(sv, e);
      }
      f[j] = _mm_cvtss_f32(_mm256_castps256_ps128(
          cqb_exp8(_mm256_set1_ps(m[j] - bm)))); /* 0 on the first block */
      l[j] = l[j] * f[j] + cqb_hsum(sv);
      m[j] = bm;
    }
    for (int i = 0; i < n; ++i) cqb_decode_row(V, h, D, b + i, vb + (size_t)i * D);
    for (int j0 = 0; j0 < rep; j0 += 4) {
      int nj = rep - j0 < 4 ? rep - j0 : 4;
      int d0 = 0;
      for (; d0 + 32 <= D; d0 += 32) cqb_pv_tile(acc, D, d0, j0, nj, n, vb, sc, f, 4);
      for (; d0 < D; d0 += 8) cqb_pv_tile(acc, D, d0, j0, nj, n, vb, sc, f, 1);
    }
  }
}

/*
 * q: fp16 [nq][D] (unscaled); out: fp32 [nq][D].  Component arrays as the
 * oracle stores them: keyframes fp16 [H][cap_kf][D], packed uint32
 * [H][cap_pf][D/8], scales fp16 [H][cap_pf].  n_chunks <= 0 picks the key
 * split from the thread count.  Returns 0, or -1 for a shape this
 * vectorised form does not take (D not a multiple of 8 or above 256, more
 * than 16 query heads per kv head, nq not a multiple of H).
 */
int cqb_fused_decode_f32(const uint16_t *q, int nq, int H, int D, int64_t T,
                         float scale, int stride_k, int stride_v,
                         const uint16_t *kf_k, int64_t cap_kf_k, const uint32_t *pk_k,
                         int64_t cap_pf_k, const uint16_t *sc_k,
                         const uint16_t *kf_v, int64_t cap_kf_v, const uint32_t *pk_v,
                         int64_t cap_pf_v, const uint16_t *sc_v, int n_chunks,
                         float *out) {
  if (H <= 0 || nq % H != 0 || D % 8 != 0 || D > CQB_MAX_D || nq / H > CQB_MAX_REP)
    return -1;
  int rep = nq / H;
  if (T <= 0) {
    memset(out, 0, sizeof(float) * (size_t)nq * D);
    return 0;
  }
  int threads = 1;
#ifdef _OPENMP
  threads = omp_get_max_threads();
#endif
  if (n_chunks <= 0) {
    int64_t by_len = (T + 255) / 256; /* at least 256 keys per task */
    int64_t want = (4 * (int64_t)threads + H - 1) / H;
    n_chunks = (int)(by_len < want ? by_len : want);
    if (n_chunks < 1) n_chunks = 1;
  }
  int64_t per = (T + n_chunks - 1) / n_chunks;
  per = (per + CQB_BLOCK - 1) / CQB_BLOCK * CQB_BLOCK;
  n_chunks = (int)((T + per - 1) / per);

  float scale_h = cqb_round_f16(scale);
  float *qs = (float *)malloc(sizeof(float) * (size_t)nq * D);
  size_t part = (size_t)rep * (D + 2); /* m[rep], l[rep], acc[rep][D] */
  float *parts = (float *)malloc(sizeof(float) * part * (size_t)H * n_chunks);
  for (int64_t i = 0; i < (int64_t)nq * D; ++i)
    qs[i] = cqb_round_f16(_cvtsh_ss(q[i]) * scale_h);
  cqb_comp K = {kf_k, pk_k, sc_k, cap_kf_k, cap_pf_k, stride_k};
  cqb_comp V = {kf_v, pk_v, sc_v, cap_kf_v, cap_pf_v, stride_v};

#pragma omp parallel for schedule(dynamic, 1)
  for (int task = 0; task < H * n_chunks; ++task) {
    int h = task / n_chunks, c = task % n_chunks;
    int64_t t0 = (int64_t)c * per, t1 = t0 + per < T ? t0 + per : T;
    float *pm = parts + part * (size_t)task;
    cqb_task(qs + (size_t)h * rep * D, rep, D, h, t0, t1, &K, &V, pm, pm + rep,
             pm + 2 * rep);
  }

  for (int h = 0; h < H; ++h)
    for (int j = 0; j < rep; ++j) {
      float M = -INFINITY, L = 0.0f;
      for (int c = 0; c < n_chunks; ++c) {
        float mc = parts[part * ((size_t)h * n_chunks + c) + j];
        M = mc > M ? mc : M;
      }
      float *o = out + ((size_t)h * rep + j) * D;
      for (int d = 0; d < D; ++d) o[d] = 0.0f;
      for (int c = 0; c < n_chunks; ++c) {
        const float *pm = parts + part * ((size_t)h * n_chunks + c);
        float f = expf(pm[j] - M);
        L += pm[rep + j] * f;
        const float *a = pm + 2 * rep + (size_t)j * D;
        for (int d = 0; d < D; ++d) o[d] += a[d] * f;
      }
      float inv = L > 0.0f ? 1.0f / L : 0.0f;
      for (int d = 0; d < D; ++d) o[d] *= inv;
    }
  free(parts);
  free(qs);
  return 0;
}
