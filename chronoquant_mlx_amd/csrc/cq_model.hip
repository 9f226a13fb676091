// cq_model.hip — fused elementwise kernels of the end-to-end decoder (the
// roles mlx's mx.fast.rms_norm / mx.fast.rope and the SwiGLU gate play in
// the mlx_lm models the reference's end-to-end runs drive): residual add +
// RMSNorm, per-head q/k RMSNorm + rotary embedding with the split of a fused
// QKV projection into the attention layout, and the SwiGLU gate.  Math in
// fp32, one rounding to the tensor dtype per stored value, as the unfused
// torch sequence rounds.
#include <hip/hip_runtime.h>
#include <math.h>

#include "cq_device.h"

namespace cq {
namespace {

constexpr int kNormThreads = 256;
constexpr int kNormMaxVec = 4;  // 16-byte vectors per thread: dim <= 8192 for 16-bit dtypes

template <int DT>
__device__ __forceinline__ void unpack8(const uint4 &u, float f[8]) {
  const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint16_t lo = (uint16_t)(w[i] & 0xffffu), hi = (uint16_t)(w[i] >> 16);
    f[2 * i] = DT == CQ_F16 ? h2f(lo) : bf2f(lo);
    f[2 * i + 1] = DT == CQ_F16 ? h2f(hi) : bf2f(hi);
  }
}

template <int DT>
__device__ __forceinline__ uint4 pack8(const float f[8]) {
  uint32_t w[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t lo = DT == CQ_F16 ? f2h(f[2 * i]) : f2bf(f[2 * i]);
    const uint32_t hi = DT == CQ_F16 ? f2h(f[2 * i + 1]) : f2bf(f[2 * i + 1]);
    w[i] = lo | (hi << 16);
  }
  return make_uint4(w[0], w[1], w[2], w[3]);
}

__device__ __forceinline__ float block_sum(float v, float *red) {
  v = wave_sum(v);
  const int wv = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) red[wv] = v;
  __syncthreads();
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < kNormThreads / 64; ++i) s += red[i];
  return s;
}

// One workgroup per row of a 16-bit dtype, dim % 8 == 0, dim <= 2048 * NV.
// h = res ? round(x + res) : x (written to h_out when res is given);
// y = h * rsqrt(mean(h^2) + eps) * w.
template <int DT, int NV>
__global__ __launch_bounds__(kNormThreads) void rms_norm_vec_kernel(
    const void *x, const void *res, const void *w, void *y, void *h_out, int dim, float eps) {
  __shared__ float red[kNormThreads / 64];
  const int nvec = dim >> 3;
  const int64_t base = (int64_t)blockIdx.x * nvec;
  float v[NV][8];
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int c = threadIdx.x + i * kNormThreads;
    if (c < nvec) {
      unpack8<DT>(((const uint4 *)x)[base + c], v[i]);
      if (res) {
        float r[8];
        unpack8<DT>(((const uint4 *)res)[base + c], r);
#pragma unroll
        for (int e = 0; e < 8; ++e) v[i][e] = Dt<DT>::round(v[i][e] + r[e]);
        ((uint4 *)h_out)[base + c] = pack8<DT>(v[i]);
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) ss += v[i][e] * v[i][e];
    }
  }
  const float inv = 1.f / sqrtf(block_sum(ss, red) / (float)dim + eps);
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int c = threadIdx.x + i * kNormThreads;
    if (c < nvec) {
      float g[8];
      unpack8<DT>(((const uint4 *)w)[c], g);
#pragma unroll
      for (int e = 0; e < 8; ++e) v[i][e] = v[i][e] * inv * g[e];
      ((uint4 *)y)[base + c] = pack8<DT>(v[i]);
    }
  }
}

// Any dtype and dim: one workgroup per row, strided scalar loops.
template <int DT>
__global__ __launch_bounds__(kNormThreads) void rms_norm_kernel(
    const void *x, const void *res, const void *w, void *y, void *h_out, int dim, float eps) {
  __shared__ float red[kNormThreads / 64];
  const int64_t base = (int64_t)blockIdx.x * dim;
  float ss = 0.f;
  for (int d = threadIdx.x; d < dim; d += kNormThreads) {
    float v = Dt<DT>::load(x, base + d);
    if (res) {
      v = Dt<DT>::round(v + Dt<DT>::load(res, base + d));
      Dt<DT>::store(h_out, base + d, v);
    }
    ss += v * v;
  }
  const float inv = 1.f / sqrtf(block_sum(ss, red) / (float)dim + eps);
  // h is re-read from h_out (this thread wrote it) when the residual is added
  const void *src = res ? h_out : x;
  for (int d = threadIdx.x; d < dim; d += kNormThreads)
    Dt<DT>::store(y, base + d, Dt<DT>::load(src, base + d) * inv * Dt<DT>::load(w, d));
}

struct QkvArgs {
  const void *qkv;  // [B][L][(nq + 2 nkv) * 128]
  const void *q_w, *k_w;
  void *q_out, *k_out, *v_out;  // [B][nq|nkv][L][128]
  const float *cos_t, *sin_t;   // [max_pos][64]
  const int64_t *positions;
  int64_t pos_bstride, max_pos, L;
  int B, nq, nkv;
  float eps;
};

// One wave per (b, l, head) over the nq query, nkv key and nkv value heads
// of a fused projection row; lane j holds dims j and j + 64 (one rotary
// pair).  Query and key heads: RMSNorm (rounded), then rotary embedding;
// value heads: copied.  A position outside [0, max_pos) yields NaN.
template <int DT>
__global__ __launch_bounds__(256) void qkv_norm_rope_kernel(QkvArgs a) {
  const int lane = threadIdx.x & 63;
  const int heads = a.nq + 2 * a.nkv;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= (int64_t)a.B * a.L * heads) return;  // wave-uniform
  const int h = (int)(row % heads);
  const int64_t bl = row / heads;
  const int64_t l = bl % a.L;
  const int b = (int)(bl / a.L);
  const int64_t xin = row * 128;
  float x1 = Dt<DT>::load(a.qkv, xin + lane), x2 = Dt<DT>::load(a.qkv, xin + lane + 64);
  if (h >= a.nq + a.nkv) {
    const int hv = h - a.nq - a.nkv;
    const int64_t o = (((int64_t)b * a.nkv + hv) * a.L + l) * 128;
    Dt<DT>::store(a.v_out, o + lane, x1);
    Dt<DT>::store(a.v_out, o + lane + 64, x2);
    return;
  }
  const bool is_q = h < a.nq;
  const void *w = is_q ? a.q_w : a.k_w;
  if (w) {
    const float inv = 1.f / sqrtf(wave_sum(x1 * x1 + x2 * x2) / 128.f + a.eps);
    x1 = Dt<DT>::round(x1 * inv * Dt<DT>::load(w, lane));
    x2 = Dt<DT>::round(x2 * inv * Dt<DT>::load(w, lane + 64));
  }
  const int64_t pos = a.positions[b * a.pos_bstride + l];
  float c = __builtin_nanf(""), s = c;
  if (pos >= 0 && pos < a.max_pos) {
    c = a.cos_t[pos * 64 + lane];
    s = a.sin_t[pos * 64 + lane];
  }
  const int hh = is_q ? h : h - a.nq;
  void *out = is_q ? a.q_out : a.k_out;
  const int64_t o = (((int64_t)b * (is_q ? a.nq : a.nkv) + hh) * a.L + l) * 128;
  Dt<DT>::store(out, o + lane, x1 * c - x2 * s);
  Dt<DT>::store(out, o + lane + 64, x2 * c + x1 * s);
}

// y = silu(gu[r][c]) * gu[r][n + c]; 8 columns per thread when n % 8 == 0.
template <int DT>
__global__ __launch_bounds__(256) void silu_mul_vec_kernel(const void *gu, void *y, int64_t rows,
                                                           int64_t n) {
  const int64_t nv = n >> 3;
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= rows * nv) return;
  const int64_t r = i / nv, c = i - r * nv;
  float g[8], u[8];
  unpack8<DT>(((const uint4 *)gu)[r * 2 * nv + c], g);
  unpack8<DT>(((const uint4 *)gu)[r * 2 * nv + nv + c], u);
#pragma unroll
  for (int e = 0; e < 8; ++e) g[e] = Dt<DT>::round(g[e] / (1.f + expf(-g[e]))) * u[e];
  ((uint4 *)y)[i] = pack8<DT>(g);
}

template <int DT>
__global__ __launch_bounds__(256) void silu_mul_kernel(const void *gu, void *y, int64_t rows,
                                                       int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= rows * n) return;
  const int64_t r = i / n, c = i - r * n;
  const float g = Dt<DT>::load(gu, r * 2 * n + c), u = Dt<DT>::load(gu, r * 2 * n + n + c);
  // silu rounded to the dtype first, as torch's silu(gate) * up computes it
  Dt<DT>::store(y, i, Dt<DT>::round(g / (1.f + expf(-g))) * u);
}

bool aligned16(const void *p) { return ((uintptr_t)p & 15u) == 0; }

template <int DT>
int launch_norm(const void *x, const void *res, const void *w, void *y, void *h_out, int64_t rows,
                int dim, float eps, hipStream_t s) {
  const dim3 grid((unsigned)rows);
  const bool vec = DT != CQ_F32 && dim % 8 == 0 && dim <= 2048 * kNormMaxVec && aligned16(x) &&
                   aligned16(w) && aligned16(y) && (!res || (aligned16(res) && aligned16(h_out)));
  if (vec && dim <= 2048)
    rms_norm_vec_kernel<DT, 1><<<grid, kNormThreads, 0, s>>>(x, res, w, y, h_out, dim, eps);
  else if (vec && dim <= 4096)
    rms_norm_vec_kernel<DT, 2><<<grid, kNormThreads, 0, s>>>(x, res, w, y, h_out, dim, eps);
  else if (vec)
    rms_norm_vec_kernel<DT, kNormMaxVec><<<grid, kNormThreads, 0, s>>>(x, res, w, y, h_out, dim,
                                                                       eps);
  else
    rms_norm_kernel<DT><<<grid, kNormThreads, 0, s>>>(x, res, w, y, h_out, dim, eps);
  return hipGetLastError() == hipSuccess ? CQ_OK : CQ_ERR_LAUNCH;
}

int norm_entry(const void *x, const void *res, const void *w, void *y, void *h_out, int64_t rows,
               int32_t dim, float eps, int32_t dtype, cq_stream_t stream) {
  if (!x || !w || !y || (res && !h_out)) return CQ_ERR_ARG;
  if (rows < 0 || rows > 0x7fffffff || dim < 1) return CQ_ERR_SHAPE;
  if (rows == 0) return CQ_OK;
  hipStream_t s = (hipStream_t)stream;
  if (dtype == CQ_F16) return launch_norm<CQ_F16>(x, res, w, y, h_out, rows, dim, eps, s);
  if (dtype == CQ_BF16) return launch_norm<CQ_BF16>(x, res, w, y, h_out, rows, dim, eps, s);
  if (dtype == CQ_F32) return launch_norm<CQ_F32>(x, res, w, y, h_out, rows, dim, eps, s);
  return CQ_ERR_DTYPE;
}

}  // namespace
}  // namespace cq

using namespace cq;

extern "C" int cq_rms_norm(const void *x, const void *w, void *y, int64_t rows, int32_t dim,
                           float eps, int32_t dtype, cq_stream_t stream) {
  return norm_entry(x, nullptr, w, y, nullptr, rows, dim, eps, dtype, stream);
}

extern "C" int cq_add_rms_norm(const void *x, const void *residual, const void *w, void *h_out,
                               void *y, int64_t rows, int32_t dim, float eps, int32_t dtype,
                               cq_stream_t stream) {
  if (!residual) return CQ_ERR_ARG;
  return norm_entry(x, residual, w, y, h_out, rows, dim, eps, dtype, stream);
}

extern "C" int cq_qkv_norm_rope(const void *qkv, const void *q_w, const void *k_w, void *q_out,
                                void *k_out, void *v_out, const float *cos_t, const float *sin_t,
                                int64_t max_pos, const int64_t *positions, int64_t pos_bstride,
                                int32_t batch, int64_t seq, int32_t n_q_heads, int32_t n_kv_heads,
                                int32_t head_dim, float eps, int32_t dtype, cq_stream_t stream) {
  if (!qkv || !q_out || !k_out || !v_out || !cos_t || !sin_t || !positions) return CQ_ERR_ARG;
  if (head_dim != 128) return CQ_ERR_UNSUPPORTED;
  if (batch < 1 || seq < 1 || n_q_heads < 1 || n_kv_heads < 1 || max_pos < 1)
    return CQ_ERR_SHAPE;
  const int64_t rows = (int64_t)batch * seq * (n_q_heads + 2 * n_kv_heads);
  if ((rows + 3) / 4 > 0x7fffffff) return CQ_ERR_SHAPE;
  QkvArgs a{qkv,    q_w,   k_w,       q_out,       k_out,   v_out, cos_t,     sin_t,
            positions, pos_bstride, max_pos, seq, batch, n_q_heads, n_kv_heads, eps};
  const dim3 grid((unsigned)((rows + 3) / 4));
  hipStream_t s = (hipStream_t)stream;
  if (dtype == CQ_F16) qkv_norm_rope_kernel<CQ_F16><<<grid, 256, 0, s>>>(a);
  else if (dtype == CQ_BF16) qkv_norm_rope_kernel<CQ_BF16><<<grid, 256, 0, s>>>(a);
  else if (dtype == CQ_F32) qkv_norm_rope_kernel<CQ_F32><<<grid, 256, 0, s>>>(a);
  else return CQ_ERR_DTYPE;
  return hipGetLastError() == hipSuccess ? CQ_OK : CQ_ERR_LAUNCH;
}

extern "C" int cq_silu_mul(const void *gu, void *y, int64_t rows, int64_t n, int32_t dtype,
                           cq_stream_t stream) {
  if (!gu || !y) return CQ_ERR_ARG;
  if (rows < 0 || n < 1) return CQ_ERR_SHAPE;
  if (rows == 0) return CQ_OK;
  const bool vec = dtype != CQ_F32 && n % 8 == 0 && aligned16(gu) && aligned16(y);
  const int64_t threads = vec ? rows * (n / 8) : rows * n;
  if ((threads + 255) / 256 > 0x7fffffff) return CQ_ERR_SHAPE;
  const dim3 grid((unsigned)((threads + 255) / 256));
  hipStream_t s = (hipStream_t)stream;
  if (dtype == CQ_F16) {
    if (vec) silu_mul_vec_kernel<CQ_F16><<<grid, 256, 0, s>>>(gu, y, rows, n);
    else silu_mul_kernel<CQ_F16><<<grid, 256, 0, s>>>(gu, y, rows, n);
  } else if (dtype == CQ_BF16) {
    if (vec) silu_mul_vec_kernel<CQ_BF16><<<grid, 256, 0, s>>>(gu, y, rows, n);
    else silu_mul_kernel<CQ_BF16><<<grid, 256, 0, s>>>(gu, y, rows, n);
  } else if (dtype == CQ_F32) {
    silu_mul_kernel<CQ_F32><<<grid, 256, 0, s>>>(gu, y, rows, n);
  } else {
    return CQ_ERR_DTYPE;
  }
  return hipGetLastError() == hipSuccess ? CQ_OK : CQ_ERR_LAUNCH;
}
