// cq_decode_common.h — pieces shared by the decode kernels: argument block,
// split planning, workspace layout, and the per-workgroup epilogue (direct
// output, or split partial + last-workgroup log-sum-exp combine).
//
// Softmax state is kept in the log2 domain everywhere: scores are multiplied
// by log2(e) once and every exponential is exp2.
#pragma once

#include <hip/hip_runtime.h>

#include "cq_device.h"

namespace cq {

int validate_cache(const cq_cache_desc *c);
int64_t num_keyframes(int64_t n, int stride);
int64_t num_pframes(int64_t n, int stride);

constexpr int kMaxSplits = 1024;
constexpr int kThreadsMfma = 512;   // 8 waves per MFMA workgroup
constexpr int kSplitGranule = 512;  // tokens; one 64-token chunk per wave of an 8-wave group

struct DecodeArgs {
  // component 0 = keys, 1 = values
  const uint16_t *kf[2];
  const uint32_t *pk[2];
  const uint16_t *sc[2];
  int64_t cap_kf[2], cap_pf[2];
  int stride[2];
  float inv_stride[2];  // 1/stride rounded up a little (see div_stride)
  int B, H, D, W, G, nq, n_chunks, chunk_heads;
  const void *q;
  int q_dtype;
  float scale;
  const int32_t *seq_lens;
  int64_t seq_len;
  int64_t max_T;  // host-validated bound (capacities checked against it)
  void *out;
  int out_dtype;
  float *part_ml;      // [B][nq][nsplit][2]  (m in log2 units, l)
  float *part_acc;     // [B][nq][nsplit][D]
  uint32_t *counters;  // [B][H][n_chunks]
  int nsplit;
  int64_t split_len;
  int lpt_log2;  // portable kernel: lanes per token = 1 << lpt_log2 (>= W)
};

__device__ __forceinline__ int64_t seq_len_of(const DecodeArgs &a, int b) {
  return a.seq_lens ? min((int64_t)max(a.seq_lens[b], 0), a.max_T) : a.seq_len;
}

// t / s for 0 <= t < 2^24 and s >= 1: float estimate, then one correction
// each way (the estimate is off by at most one).
__device__ __forceinline__ int div_stride(int t, int s, float inv_s) {
  int g = (int)((float)t * inv_s);
  int r = t - g * s;
  if (r < 0) --g;
  else if (r >= s) ++g;
  return g;
}

// Split partials cross workgroups (and XCDs, whose L2s are not coherent with
// each other) without cache-wide fences: they are written with device-scope
// relaxed atomic stores (write-through to the device coherence point), each
// thread waits for its stores to complete (s_waitcnt vmcnt(0)), the workgroup
// syncs, and one thread bumps the counter with a device-scope atomic.  The
// workgroup that brings the counter to nsplit reads the partials back with
// device-scope atomic loads.  (__threadfence() would instead write back and
// invalidate the whole L2 in every workgroup.)
__device__ __forceinline__ void store_dev(float *p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float load_dev(const float *p) {
  return __hip_atomic_load(const_cast<float *>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Per-workgroup epilogue.  The workgroup's merged state for q heads
// j0 .. j0+gn-1 of kv head h is in LDS: wm[j] (running max, log2 units),
// wl[j] (sum of weights), wo[j*ostride + d] (unnormalised output).  With one
// split it writes the output; otherwise it writes a partial, and the last
// workgroup of (b, h, chunk) to finish merges all partials and resets the
// counter it used.  `scratch` (kCombineScratchFloats floats of LDS) may alias
// wm/wl/wo: it is written only after they have been consumed.  The merge
// issues its loads in batches before using them, so it costs about one
// memory round trip per phase plus the partial bytes.
constexpr int kCombineWeights = 4096;  // (m, l) pairs of a head batch: 2 x 2048
constexpr int kCombineScratchFloats = kCombineWeights + 16 + 16 * 256;

__device__ __forceinline__ void finish_workgroup(const DecodeArgs &a, int b, int h, int chunk,
                                                 int j0, int gn, int split, const float *wm,
                                                 const float *wl, const float *wo, int ostride,
                                                 float *scratch) {
  const int tid = threadIdx.x, nthr = blockDim.x;
  const bool direct = a.nsplit == 1;
  for (int e = tid; e < gn * a.D; e += nthr) {
    const int j = e / a.D, dim = e - j * a.D;
    const int64_t bq = (int64_t)b * a.nq + h * a.G + j0 + j;
    const float L = wl[j], O = wo[j * ostride + dim];
    if (direct) {
      store_any(a.out_dtype, a.out, bq * a.D + dim, L > 0.f ? O / L : 0.f);
    } else {
      store_dev(&a.part_acc[(bq * a.nsplit + split) * a.D + dim], O);
      if (dim == 0) {
        store_dev(&a.part_ml[(bq * a.nsplit + split) * 2 + 0], wm[j]);
        store_dev(&a.part_ml[(bq * a.nsplit + split) * 2 + 1], L);
      }
    }
  }
  if (direct) return;

  __shared__ int s_last;
  __builtin_amdgcn_s_waitcnt(0);  // this thread's partial stores are complete
  __syncthreads();
  uint32_t *ctr = a.counters + ((int64_t)b * a.H + h) * a.n_chunks + chunk;
  if (tid == 0) {
    const uint32_t prev =
        __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    s_last = (prev == (uint32_t)(a.nsplit - 1));
  }
  __syncthreads();
  if (!s_last) return;
  __builtin_amdgcn_s_waitcnt(0);

  // scratch: m -> weights [hb][nsplit] at the bottom, l [hb][nsplit] from
  // kCombineWeights/2, 1/L [16], outputs [hb][D]
  const int nsplit = a.nsplit;
  const int wave = tid >> 6, lane = tid & 63, nwaves = nthr >> 6;
  const int half = kCombineWeights / 2;
  const int hb_max = max(1, min(16, half / nsplit));
  float *s_wt = scratch;
  float *s_l = scratch + half;
  float *s_inv = scratch + kCombineWeights;
  float *s_out = s_inv + 16;
  const int64_t bq0 = (int64_t)b * a.nq + h * a.G + j0;
  const int nd4 = (a.D + 3) / 4;
  for (int jb = 0; jb < gn; jb += hb_max) {
    const int hb = min(hb_max, gn - jb);
    // (m, l) of every (head, split) of the batch, one load each
    for (int e = tid; e < hb * nsplit; e += nthr) {
      const int j = e / nsplit, sp = e - j * nsplit;
      const float *ml = a.part_ml + ((bq0 + jb + j) * nsplit + sp) * 2;
      s_wt[e] = load_dev(ml);
      s_l[e] = load_dev(ml + 1);
    }
    for (int e = tid; e < hb * a.D; e += nthr) s_out[e] = 0.f;
    __syncthreads();
    // one wave per head: max, weights, 1 / sum of weighted l
    for (int j = wave; j < hb; j += nwaves) {
      float mx = -INFINITY;
      for (int sp = lane; sp < nsplit; sp += 64) mx = fmaxf(mx, s_wt[j * nsplit + sp]);
      mx = wave_max(mx);
      float ls = 0.f;
      for (int sp = lane; sp < nsplit; sp += 64) {
        const float m = s_wt[j * nsplit + sp];
        const float w = (mx == -INFINITY || m == -INFINITY) ? 0.f : fast_exp2(m - mx);
        ls += w * s_l[j * nsplit + sp];
        s_wt[j * nsplit + sp] = w;
      }
      ls = wave_sum(ls);
      if (lane == 0) s_inv[j] = ls > 0.f ? 1.f / ls : 0.f;
    }
    __syncthreads();
    // weighted sum of the partial outputs: a thread takes (head, 4 dims) and a
    // slice of the splits; 8 splits' loads are in flight before they are used
    const int units = hb * nd4;
    const int slices = max(1, nthr / units);
    const int slice = tid / units;
    if (slice < slices) {
      for (int u = tid % units; u < units; u += nthr) {
        const int j = u / nd4, d0 = 4 * (u - j * nd4);
        const int nc = min(4, a.D - d0);
        const float *pa = a.part_acc + (bq0 + jb + j) * nsplit * a.D + d0;
        float o[4] = {0.f, 0.f, 0.f, 0.f};
        int sp = slice;
        for (; sp + 7 * slices < nsplit; sp += 8 * slices) {
          float v[8][4];
#pragma unroll
          for (int k = 0; k < 8; ++k)
#pragma unroll
            for (int c = 0; c < 4; ++c)
              v[k][c] = c < nc ? load_dev(pa + (int64_t)(sp + k * slices) * a.D + c) : 0.f;
#pragma unroll
          for (int k = 0; k < 8; ++k) {
            const float w = s_wt[j * nsplit + sp + k * slices];
#pragma unroll
            for (int c = 0; c < 4; ++c) o[c] += w * v[k][c];
          }
        }
        for (; sp < nsplit; sp += slices) {
          const float w = s_wt[j * nsplit + sp];
#pragma unroll
          for (int c = 0; c < 4; ++c)
            if (c < nc) o[c] += w * load_dev(pa + (int64_t)sp * a.D + c);
        }
#pragma unroll
        for (int c = 0; c < 4; ++c)
          if (c < nc) atomicAdd(&s_out[j * a.D + d0 + c], o[c]);
      }
    }
    __syncthreads();
    for (int e = tid; e < hb * a.D; e += nthr) {
      const int j = e / a.D, dim = e - j * a.D;
      store_any(a.out_dtype, a.out, (bq0 + jb + j) * a.D + dim, s_out[e] * s_inv[j]);
    }
    __syncthreads();
  }
  if (tid == 0) __hip_atomic_store(ctr, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ---------------------------------------------------------------------------
// host-side planning
// ---------------------------------------------------------------------------
struct SplitPlan {
  int nsplit;
  int64_t split_len;
};

// Splits of kSplitGranule-multiple length, sized so that the grid holds about
// two workgroups per CU (256 CUs) when the context allows, at most kMaxSplits.
inline SplitPlan plan_splits(int B, int H, int64_t max_T) {
  SplitPlan p;
  const int64_t groups = (int64_t)B * H;
  const int64_t target = 512;
  int64_t ns = (target + groups - 1) / groups;
  if (max_T <= 0) max_T = 1;
  int64_t len = (max_T + ns - 1) / ns;
  len = (len + kSplitGranule - 1) / kSplitGranule * kSplitGranule;
  ns = (max_T + len - 1) / len;
  if (ns > kMaxSplits) {
    len = (max_T + kMaxSplits - 1) / kMaxSplits;
    len = (len + kSplitGranule - 1) / kSplitGranule * kSplitGranule;
    ns = (max_T + len - 1) / len;
  }
  p.nsplit = (int)ns;
  p.split_len = len;
  return p;
}

// Workspace layout: a fixed 64 KiB counter region first (one uint32 per
// (sequence, kv head, q-head chunk); the kernels return every counter to zero),
// then the split partials, whose size varies with the split count.  Keeping
// the counters at a fixed place means calls of different shapes sharing one
// workspace never see each other's partials as counters.
constexpr size_t kCounterRegion = 64 << 10;
constexpr int64_t kMaxCounters = kCounterRegion / sizeof(uint32_t);

inline size_t round256(size_t x) { return (x + 255) / 256 * 256; }

inline size_t workspace_bytes_for(int B, int nq, int D, int nsplit) {
  const size_t ml = (size_t)B * nq * nsplit * 2 * sizeof(float);
  const size_t acc = (size_t)B * nq * nsplit * D * sizeof(float);
  return kCounterRegion + round256(ml) + round256(acc);
}

inline void carve_workspace(DecodeArgs &a, void *ws) {
  char *p = (char *)ws;
  a.counters = (uint32_t *)p;
  p += kCounterRegion;
  const size_t ml = (size_t)a.B * a.nq * a.nsplit * 2 * sizeof(float);
  a.part_ml = (float *)p;
  p += round256(ml);
  a.part_acc = (float *)p;
}

// Common launch preparation: split plan and workspace.  chunk_heads = q heads
// per workgroup of the kernel being launched.
inline int prepare_launch(DecodeArgs &a, int chunk_heads, void *workspace, size_t ws_bytes) {
  a.chunk_heads = chunk_heads;
  a.n_chunks = (a.G + chunk_heads - 1) / chunk_heads;
  const SplitPlan p = plan_splits(a.B, a.H, a.max_T);
  a.nsplit = p.nsplit;
  a.split_len = p.split_len;
  if (a.nsplit > 1) {
    if ((int64_t)a.B * a.H * a.n_chunks > kMaxCounters) return CQ_ERR_UNSUPPORTED;
    if (!workspace) return CQ_ERR_WORKSPACE;
    if (ws_bytes < workspace_bytes_for(a.B, a.nq, a.D, a.nsplit)) return CQ_ERR_WORKSPACE;
    carve_workspace(a, workspace);
  } else {
    a.part_ml = a.part_acc = nullptr;
    a.counters = nullptr;
  }
  return CQ_OK;
}

int launch_decode_mfma(DecodeArgs &a, void *workspace, size_t ws_bytes, hipStream_t stream);
bool mfma_supported(const DecodeArgs &a);

}  // namespace cq
