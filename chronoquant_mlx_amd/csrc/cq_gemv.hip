// cq_gemv.hip — y = W x for a single input row: the projections of one
// decode step of the end-to-end decoder (a torch Linear with M = 1), where
// the whole cost is streaming the weight matrix from HBM once.
//
// W [n][k] row-major (a Linear weight, out x in), x [k], y [n]; fp16 or bf16
// with fp32 accumulation (v_dot2c_f32_{f16,bf16}) and one rounding per
// output.  A workgroup of 4 waves owns 8 consecutive rows; the 4 waves take
// interleaved 512-element blocks of k (each lane 16 bytes of every row per
// block), so a wave has 8 row loads of 1 KB each in flight per block.  The
// lane partial sums fold with a DPP wave sum, the 4 waves' through LDS.
#include <hip/hip_runtime.h>

#include "cq_decode_common.h"

namespace cq {
namespace {

constexpr int kGemvThreads = 256;  // 4 waves
constexpr int kGemvWaves = kGemvThreads / 64;
constexpr int kGemvRows = 8;       // rows per workgroup
constexpr int kGemvBlk = 512;      // row elements one wave-wide 16-byte load covers
constexpr uint32_t kDead = 0x80000000u;  // an offset past every buffer: loads read 0
constexpr int kPolicyStreamGemv = 2;     // weights are read once: non-temporal

typedef __bf16 bf2_t __attribute__((ext_vector_type(2)));
typedef _Float16 hh2_t __attribute__((ext_vector_type(2)));

template <int DT>
__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
  if constexpr (DT == CQ_BF16)
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf2_t, a), __builtin_bit_cast(bf2_t, b),
                                           c, false);
  else
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(hh2_t, a), __builtin_bit_cast(hh2_t, b), c,
                                  false);
}

template <int DT>
__device__ __forceinline__ float dot8(uint4 w, uint4 x, float c) {
  c = dot2<DT>(w.x, x.x, c);
  c = dot2<DT>(w.y, x.y, c);
  c = dot2<DT>(w.z, x.z, c);
  return dot2<DT>(w.w, x.w, c);
}

template <int Policy>
__device__ __forceinline__ uint4 ld128(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  const __attribute__((ext_vector_type(4))) int v =
      __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, Policy);
  return uint4{(uint32_t)v[0], (uint32_t)v[1], (uint32_t)v[2], (uint32_t)v[3]};
}

// What the kernel multiplies W by (x is the row it is given):
//   kPlain: x itself.
//   kNorm:  RMSNorm of h = round(x + res) (res optional; the add_rms_norm
//           semantics): round(h * rsqrt(mean(h^2) + eps) * nw).  Every
//           workgroup recomputes the row's inverse norm and keeps h in LDS;
//           workgroup 0 writes h to h_out (the residual stream) when given.
//   kSilu:  x = [gate | up] of length 2k: round(round(silu(gate)) * up), the
//           SwiGLU gate, as cq_silu_mul computes it.
enum GemvMode { kPlain = 0, kNorm = 1, kSilu = 2 };
constexpr int kGemvMaxNormK = 8192;  // h cached in LDS (16 KB of 16-bit values)
constexpr unsigned kGemvPairMaxGroups = 1024;  // workgroups up to which kNorm takes kPair

struct GemvArgs {
  const uint16_t *w;
  const uint16_t *x;
  const uint16_t *res;  // kNorm: residual or null
  const uint16_t *nw;   // kNorm: norm weight [k]
  uint16_t *h_out;      // kNorm with res: round(x + res), written by workgroup 0
  uint16_t *y;
  int64_t n;
  int k;
  float eps;
};

template <int DT>
__device__ __forceinline__ void unpack8f(uint4 u, float f[8]) {
  const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[2 * i] = DT == CQ_BF16 ? bf2f((uint16_t)(w[i] & 0xffffu)) : h2f((uint16_t)(w[i] & 0xffffu));
    f[2 * i + 1] = DT == CQ_BF16 ? bf2f((uint16_t)(w[i] >> 16)) : h2f((uint16_t)(w[i] >> 16));
  }
}
template <int DT>
__device__ __forceinline__ uint4 pack8f(const float f[8]) {
  uint32_t w[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t lo = DT == CQ_BF16 ? f2bf(f[2 * i]) : f2h(f[2 * i]);
    const uint32_t hi = DT == CQ_BF16 ? f2bf(f[2 * i + 1]) : f2h(f[2 * i + 1]);
    w[i] = lo | (hi << 16);
  }
  return uint4{w[0], w[1], w[2], w[3]};
}
template <int DT>
__device__ __forceinline__ float round_dt(float v) {
  return DT == CQ_BF16 ? bf2f(f2bf(v)) : h2f(f2h(v));
}

// kPair: a wave takes its blocks two at a time, with both blocks' 16 row
// loads in flight before its first wait.  It pays where the whole grid is
// resident at once (a few workgroups per CU, as in the QKV projection):
// there the rows in flight per wave bound the rate.  With more workgroups
// than fit at once it is slower (fewer waves per SIMD at its register count).
template <int DT, int Mode, bool kPair = false>
__global__ __launch_bounds__(kGemvThreads) void gemv_kernel(GemvArgs a) {
  __shared__ float red[kGemvWaves][kGemvRows];
  __shared__ uint4 hs[Mode == kNorm ? kGemvMaxNormK / 8 : 1];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int k = a.k;
  const int64_t n0 = (int64_t)blockIdx.x * kGemvRows;
  const int rows = (int)min((int64_t)kGemvRows, a.n - n0);
  // this workgroup's rows (host: 8 rows of k 16-bit elements < 2^31 bytes)
  const __amdgpu_buffer_rsrc_t rw = make_rsrc(a.w + n0 * k, (uint32_t)rows * (uint32_t)k * 2u);
  const __amdgpu_buffer_rsrc_t rx =
      make_rsrc(a.x, (uint32_t)k * (Mode == kSilu ? 4u : 2u));
  float inv = 0.f;
  if constexpr (Mode == kNorm) {
    // h = round(x + res) into LDS, and the row's sum of squares
    const __amdgpu_buffer_rsrc_t rr = make_rsrc(a.res, a.res ? (uint32_t)k * 2u : 0u);
    float ss = 0.f;
    for (int sgm = threadIdx.x; 8 * sgm < k; sgm += kGemvThreads) {
      float h[8];
      unpack8f<DT>(ld128<0>(rx, (uint32_t)sgm * 16u), h);
      if (a.res) {
        float r8[8];
        unpack8f<DT>(ld128<0>(rr, (uint32_t)sgm * 16u), r8);
#pragma unroll
        for (int e = 0; e < 8; ++e) h[e] = round_dt<DT>(h[e] + r8[e]);
      }
      const uint4 hv = pack8f<DT>(h);
      hs[sgm] = hv;
      if (a.h_out && blockIdx.x == 0) ((uint4 *)a.h_out)[sgm] = hv;
#pragma unroll
      for (int e = 0; e < 8; ++e) ss += h[e] * h[e];
    }
    ss = wave_sum(ss);
    if (lane == 0) red[wave][0] = ss;
    __syncthreads();
    float tot = 0.f;
#pragma unroll
    for (int i = 0; i < kGemvWaves; ++i) tot += red[i][0];
    inv = 1.f / sqrtf(tot / (float)k + a.eps);
    __syncthreads();  // red is reused below
  }
  const __amdgpu_buffer_rsrc_t rn = make_rsrc(a.nw, Mode == kNorm ? (uint32_t)k * 2u : 0u);
  float acc[kGemvRows];
#pragma unroll
  for (int r = 0; r < kGemvRows; ++r) acc[r] = 0.f;
  if constexpr (kPair) {
    // both blocks' operands first, then their 16 weight rows; the blocks
    // are still summed in increasing order
    for (int blk = wave; blk * kGemvBlk < k; blk += 2 * kGemvWaves) {
      int e[2];
      bool in[2];
      uint4 op[2][2];  // kPlain: x; kNorm: the norm weight; kSilu: gate, up
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        e[u] = (blk + u * kGemvWaves) * kGemvBlk + 8 * lane;
        in[u] = e[u] < k;
        const uint32_t off = in[u] ? (uint32_t)e[u] * 2u : kDead;
        if constexpr (Mode == kNorm) {
          op[u][0] = ld128<0>(rn, off);
        } else {
          op[u][0] = ld128<0>(rx, off);
          if constexpr (Mode == kSilu)
            op[u][1] = ld128<0>(rx, in[u] ? (uint32_t)(k + e[u]) * 2u : kDead);
        }
      }
      uint4 wv[2][kGemvRows];
#pragma unroll
      for (int u = 0; u < 2; ++u)
#pragma unroll
        for (int r = 0; r < kGemvRows; ++r)
          wv[u][r] = ld128<kPolicyStreamGemv>(
              rw, (in[u] && r < rows) ? ((uint32_t)r * (uint32_t)k + (uint32_t)e[u]) * 2u : kDead);
      // (the scheduler would otherwise sink the second block's loads below
      // the first block's products to save registers)
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        uint4 xv;
        if constexpr (Mode == kPlain) {
          xv = op[u][0];
        } else if constexpr (Mode == kNorm) {
          float h[8], g[8];
          unpack8f<DT>(in[u] ? hs[e[u] >> 3] : uint4{0u, 0u, 0u, 0u}, h);
          unpack8f<DT>(op[u][0], g);
#pragma unroll
          for (int i = 0; i < 8; ++i) h[i] = h[i] * inv * g[i];
          xv = pack8f<DT>(h);
        } else {
          float g[8], up[8];
          unpack8f<DT>(op[u][0], g);
          unpack8f<DT>(op[u][1], up);
#pragma unroll
          for (int i = 0; i < 8; ++i) g[i] = round_dt<DT>(g[i] / (1.f + expf(-g[i]))) * up[i];
          xv = pack8f<DT>(g);
        }
#pragma unroll
        for (int r = 0; r < kGemvRows; ++r) acc[r] = dot8<DT>(wv[u][r], xv, acc[r]);
      }
    }
  } else {
#pragma unroll 2
  for (int blk = wave; blk * kGemvBlk < k; blk += kGemvWaves) {
    const int e = blk * kGemvBlk + 8 * lane;  // this lane's 8 elements of every row
    const bool in = e < k;                    // (k % 8 == 0: all 8 or none)
    uint4 wv[kGemvRows];
#pragma unroll
    for (int r = 0; r < kGemvRows; ++r)
      wv[r] = ld128<kPolicyStreamGemv>(
          rw, (in && r < rows) ? ((uint32_t)r * (uint32_t)k + (uint32_t)e) * 2u : kDead);
    uint4 xv;
    if constexpr (Mode == kPlain) {
      xv = ld128<0>(rx, in ? (uint32_t)e * 2u : kDead);
    } else if constexpr (Mode == kNorm) {
      float h[8], g[8];
      unpack8f<DT>(in ? hs[e >> 3] : uint4{0u, 0u, 0u, 0u}, h);
      unpack8f<DT>(ld128<0>(rn, in ? (uint32_t)e * 2u : kDead), g);
#pragma unroll
      for (int i = 0; i < 8; ++i) h[i] = h[i] * inv * g[i];
      xv = pack8f<DT>(h);
    } else {
      float g[8], u[8];
      unpack8f<DT>(ld128<0>(rx, in ? (uint32_t)e * 2u : kDead), g);
      unpack8f<DT>(ld128<0>(rx, in ? (uint32_t)(k + e) * 2u : kDead), u);
#pragma unroll
      for (int i = 0; i < 8; ++i) g[i] = round_dt<DT>(g[i] / (1.f + expf(-g[i]))) * u[i];
      xv = pack8f<DT>(g);
    }
#pragma unroll
    for (int r = 0; r < kGemvRows; ++r) acc[r] = dot8<DT>(wv[r], xv, acc[r]);
  }
  }
#pragma unroll
  for (int r = 0; r < kGemvRows; ++r) {
    const float sm = wave_sum(acc[r]);
    if (lane == 0) red[wave][r] = sm;
  }
  __syncthreads();
  if (threadIdx.x < (unsigned)rows) {
    float sm = 0.f;
#pragma unroll
    for (int i = 0; i < kGemvWaves; ++i) sm += red[i][threadIdx.x];
    a.y[n0 + threadIdx.x] = DT == CQ_BF16 ? f2bf(sm) : f2h(sm);
  }
}

template <int DT>
void launch_gemv(const GemvArgs &a, int mode, dim3 grid, hipStream_t s) {
  const dim3 blk(kGemvThreads);
  // the paired form where the grid is resident at once (a few workgroups
  // per CU on MI355X's 256 CUs): the QKV projection, not gate/up
  if (mode == kNorm && grid.x <= kGemvPairMaxGroups) gemv_kernel<DT, kNorm, true><<<grid, blk, 0, s>>>(a);
  else if (mode == kNorm) gemv_kernel<DT, kNorm><<<grid, blk, 0, s>>>(a);
  else if (mode == kSilu) gemv_kernel<DT, kSilu><<<grid, blk, 0, s>>>(a);
  else gemv_kernel<DT, kPlain><<<grid, blk, 0, s>>>(a);
}

int gemv_entry(const GemvArgs &a, int mode, int dtype, cq_stream_t stream) {
  if (!a.w || !a.x || !a.y) return CQ_ERR_ARG;
  if (a.n < 1 || a.k < 8 || a.k % 8) return CQ_ERR_SHAPE;
  if (dtype != CQ_F16 && dtype != CQ_BF16) return CQ_ERR_DTYPE;
  uintptr_t al = (uintptr_t)a.w | (uintptr_t)a.x;
  if (mode == kNorm) {
    if (!a.nw) return CQ_ERR_ARG;
    if (a.k > kGemvMaxNormK) return CQ_ERR_UNSUPPORTED;
    al |= (uintptr_t)a.nw | (uintptr_t)a.res | (uintptr_t)a.h_out;
  }
  if (al & 15) return CQ_ERR_ALIGN;
  if ((int64_t)kGemvRows * a.k * 2 >= ((int64_t)1 << 31)) return CQ_ERR_UNSUPPORTED;
  const int64_t groups = (a.n + kGemvRows - 1) / kGemvRows;
  if (groups > 0x7fffffff) return CQ_ERR_SHAPE;
  const dim3 grid((unsigned)groups);
  hipStream_t s = (hipStream_t)stream;
  if (dtype == CQ_BF16) launch_gemv<CQ_BF16>(a, mode, grid, s);
  else launch_gemv<CQ_F16>(a, mode, grid, s);
  return hipGetLastError() == hipSuccess ? CQ_OK : CQ_ERR_LAUNCH;
}

}  // namespace
}  // namespace cq

using namespace cq;

extern "C" int cq_gemv(const void *w, const void *x, void *y, int64_t n, int32_t k, int32_t dtype,
                       cq_stream_t stream) {
  GemvArgs a{(const uint16_t *)w, (const uint16_t *)x, nullptr, nullptr, nullptr,
             (uint16_t *)y, n, k, 0.f};
  return gemv_entry(a, kPlain, dtype, stream);
}

extern "C" int cq_gemv_rms_norm(const void *w, const void *x, const void *residual,
                                const void *norm_w, float eps, void *h_out, void *y, int64_t n,
                                int32_t k, int32_t dtype, cq_stream_t stream) {
  if (h_out && !residual) return CQ_ERR_ARG;
  GemvArgs a{(const uint16_t *)w, (const uint16_t *)x, (const uint16_t *)residual,
             (const uint16_t *)norm_w, (uint16_t *)h_out, (uint16_t *)y, n, k, eps};
  return gemv_entry(a, kNorm, dtype, stream);
}

extern "C" int cq_gemv_silu(const void *w, const void *gate_up, void *y, int64_t n, int32_t k,
                            int32_t dtype, cq_stream_t stream) {
  GemvArgs a{(const uint16_t *)w, (const uint16_t *)gate_up, nullptr, nullptr, nullptr,
             (uint16_t *)y, n, k, 0.f};
  return gemv_entry(a, kSilu, dtype, stream);
}
