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

template <int DT>
__global__ __launch_bounds__(kGemvThreads) void gemv_kernel(const uint16_t *w, const uint16_t *x,
                                                            uint16_t *y, int64_t n, int k) {
  __shared__ float red[kGemvWaves][kGemvRows];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t n0 = (int64_t)blockIdx.x * kGemvRows;
  const int rows = (int)min((int64_t)kGemvRows, n - n0);
  // this workgroup's rows (host: 8 rows of k 16-bit elements < 2^31 bytes)
  const __amdgpu_buffer_rsrc_t rw = make_rsrc(w + n0 * k, (uint32_t)rows * (uint32_t)k * 2u);
  const __amdgpu_buffer_rsrc_t rx = make_rsrc(x, (uint32_t)k * 2u);
  float acc[kGemvRows];
#pragma unroll
  for (int r = 0; r < kGemvRows; ++r) acc[r] = 0.f;
#pragma unroll 2
  for (int blk = wave; blk * kGemvBlk < k; blk += kGemvWaves) {
    const int e = blk * kGemvBlk + 8 * lane;  // this lane's 8 elements of every row
    const bool in = e < k;                    // (k % 8 == 0: all 8 or none)
    const uint4 xv = ld128<0>(rx, in ? (uint32_t)e * 2u : kDead);
    uint4 wv[kGemvRows];
#pragma unroll
    for (int r = 0; r < kGemvRows; ++r)
      wv[r] = ld128<kPolicyStreamGemv>(
          rw, (in && r < rows) ? ((uint32_t)r * (uint32_t)k + (uint32_t)e) * 2u : kDead);
#pragma unroll
    for (int r = 0; r < kGemvRows; ++r) acc[r] = dot8<DT>(wv[r], xv, acc[r]);
  }
#pragma unroll
  for (int r = 0; r < kGemvRows; ++r) {
    const float s = wave_sum(acc[r]);
    if (lane == 0) red[wave][r] = s;
  }
  __syncthreads();
  if (threadIdx.x < (unsigned)rows) {
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < kGemvWaves; ++i) s += red[i][threadIdx.x];
    y[n0 + threadIdx.x] = DT == CQ_BF16 ? f2bf(s) : f2h(s);
  }
}

}  // namespace
}  // namespace cq

using namespace cq;

extern "C" int cq_gemv(const void *w, const void *x, void *y, int64_t n, int32_t k, int32_t dtype,
                       cq_stream_t stream) {
  if (!w || !x || !y) return CQ_ERR_ARG;
  if (n < 1 || k < 8 || k % 8) return CQ_ERR_SHAPE;
  if (dtype != CQ_F16 && dtype != CQ_BF16) return CQ_ERR_DTYPE;
  if (((uintptr_t)w | (uintptr_t)x) & 15) return CQ_ERR_ALIGN;
  if ((int64_t)kGemvRows * k * 2 >= ((int64_t)1 << 31)) return CQ_ERR_UNSUPPORTED;
  const int64_t groups = (n + kGemvRows - 1) / kGemvRows;
  if (groups > 0x7fffffff) return CQ_ERR_SHAPE;
  const dim3 grid((unsigned)groups), blk(kGemvThreads);
  hipStream_t s = (hipStream_t)stream;
  if (dtype == CQ_BF16)
    gemv_kernel<CQ_BF16><<<grid, blk, 0, s>>>((const uint16_t *)w, (const uint16_t *)x,
                                              (uint16_t *)y, n, k);
  else
    gemv_kernel<CQ_F16><<<grid, blk, 0, s>>>((const uint16_t *)w, (const uint16_t *)x,
                                             (uint16_t *)y, n, k);
  return hipGetLastError() == hipSuccess ? CQ_OK : CQ_ERR_LAUNCH;
}
