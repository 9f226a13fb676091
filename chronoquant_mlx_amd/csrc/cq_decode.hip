// cq_decode.hip — fused dequant + GQA attention for one query token per
// sequence over the ChronoQuant cache (split-K flash decode), and the
// uncompressed fp16 flash-decode baseline.
//
// Work split: grid (split, kv head x q-head chunk, sequence).  Each workgroup
// owns a contiguous token range of one (sequence, kv head) and all q heads of
// that GQA group, so every compressed byte is read once for the whole group.
// It writes an unnormalised partial (running max m, sum l, acc[D]) per q head;
// the last workgroup of each (sequence, kv head, chunk) — found with an
// atomic counter in the workspace — merges the partials with log-sum-exp and
// resets the counter, so the combine costs no extra launch.
#include <hip/hip_runtime.h>
#include <math.h>

#include "cq_device.h"

namespace cq {

int validate_cache(const cq_cache_desc *c);
int64_t num_keyframes(int64_t n, int stride);
int64_t num_pframes(int64_t n, int stride);

constexpr int kGenericGroup = 8;  // q heads per workgroup in the portable kernel
constexpr int kMaxSplits = 1024;

struct DecodeArgs {
  // component 0 = keys, 1 = values
  const uint16_t *kf[2];
  const uint32_t *pk[2];
  const uint16_t *sc[2];
  int64_t cap_kf[2], cap_pf[2];
  int stride[2];
  int B, H, D, W, G, nq, n_chunks;
  const void *q;
  int q_dtype;
  float scale;
  const int32_t *seq_lens;
  int64_t seq_len;
  int64_t max_T;  // host-validated bound (capacities checked against it)
  void *out;
  int out_dtype;
  float *part_ml;    // [B][nq][nsplit][2]
  float *part_acc;   // [B][nq][nsplit][D]
  uint32_t *counters;  // [B][H][n_chunks]
  int nsplit;
  int64_t split_len;
  int lpt_log2;  // lanes per token = 1 << lpt_log2 (>= W)
};

__device__ __forceinline__ float shfl_xor_f(float v, int m) { return __shfl_xor(v, m, 64); }

// Merge state (m, l, acc) with (mo, lo, acco); m = -inf marks "empty".
__device__ __forceinline__ void merge_weights(float m, float mo, float &wa, float &wb,
                                              float &mn) {
  mn = fmaxf(m, mo);
  if (mn == -INFINITY) {
    wa = 0.f;
    wb = 0.f;
  } else {
    wa = fast_exp2((m - mn) * kLog2e);
    wb = fast_exp2((mo - mn) * kLog2e);
  }
}

// Loads 8 dims [8w, 8w+8) of an fp16 row (dims >= D read as 0).
__device__ __forceinline__ void load_row8(const uint16_t *row, int w, int D, float (&x)[8]) {
  if (8 * w + 8 <= D && (D & 7) == 0) {
    const uint4 u = *(const uint4 *)(row + 8 * w);
    const uint32_t parts[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      x[2 * i] = h2f((uint16_t)(parts[i] & 0xffffu));
      x[2 * i + 1] = h2f((uint16_t)(parts[i] >> 16));
    }
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i) x[i] = (8 * w + i < D) ? h2f(row[8 * w + i]) : 0.f;
  }
}

// Token t of component ci, dims [8w, 8w+8): anchor + (code-8)*scale in fp32
// (the reference fused kernel's dequant, kernels.py:145-157, 167-178).
__device__ __forceinline__ void dequant8(const DecodeArgs &a, int ci, int64_t bh, int64_t t,
                                         int w, float (&x)[8]) {
  const int stride = a.stride[ci];
  const int64_t g = t / stride;
  load_row8(a.kf[ci] + (bh * a.cap_kf[ci] + g) * a.D, w, a.D, x);
  if (t - g * stride != 0) {
    const int64_t slot = t - g - 1;
    const uint32_t word = a.pk[ci][(bh * a.cap_pf[ci] + slot) * a.W + w];
    const float s = h2f(a.sc[ci][bh * a.cap_pf[ci] + slot]);
#pragma unroll
    for (int i = 0; i < 8; ++i) x[i] += (float)((int)((word >> (4 * i)) & 0xfu) - 8) * s;
  }
}

// Portable decode kernel: lanes per token = pow2 >= W words; each lane owns
// one 8-dim word of its token.  Exact per-token online softmax in fp32.
__global__ __launch_bounds__(256) void decode_generic_kernel(DecodeArgs a) {
  const int split = blockIdx.x;
  const int h = blockIdx.y / a.n_chunks;
  const int chunk = blockIdx.y - h * a.n_chunks;
  const int b = blockIdx.z;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int lpt = 1 << a.lpt_log2;
  const int tpw = 64 >> a.lpt_log2;
  const int w = lane & (lpt - 1);
  const int sub = lane >> a.lpt_log2;
  const int j0 = chunk * kGenericGroup;
  const int gn = min(kGenericGroup, a.G - j0);
  const int64_t bh = (int64_t)b * a.H + h;
  const int64_t T = a.seq_lens ? min((int64_t)max(a.seq_lens[b], 0), a.max_T) : a.seq_len;
  const int64_t t0 = (int64_t)split * a.split_len;
  const int64_t t1 = min(T, t0 + a.split_len);
  const bool wok = w < a.W;

  // q' = round_qdtype(q * round_qdtype(scale)) (attention.py:46)
  float qv[kGenericGroup][8];
  const float sc_r = round_any(a.q_dtype, a.scale);
#pragma unroll
  for (int j = 0; j < kGenericGroup; ++j) {
    const int qh = h * a.G + j0 + j;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int dim = 8 * w + i;
      float v = 0.f;
      if (j < gn && wok && dim < a.D)
        v = round_any(a.q_dtype, load_any(a.q_dtype, a.q, ((int64_t)b * a.nq + qh) * a.D + dim) * sc_r);
      qv[j][i] = v;
    }
  }

  float m[kGenericGroup], l[kGenericGroup], acc[kGenericGroup][8];
#pragma unroll
  for (int j = 0; j < kGenericGroup; ++j) {
    m[j] = -INFINITY;
    l[j] = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[j][i] = 0.f;
  }

  for (int64_t base = t0 + (int64_t)wave * tpw; base < t1; base += 4 * tpw) {
    const int64_t t = base + sub;
    const bool valid = t < t1;
    float k[8], v[8];
    if (valid && wok) {
      dequant8(a, 0, bh, t, w, k);
      dequant8(a, 1, bh, t, w, v);
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) k[i] = v[i] = 0.f;
    }
    float s[kGenericGroup];
#pragma unroll
    for (int j = 0; j < kGenericGroup; ++j) {
      float p = 0.f;
#pragma unroll
      for (int i = 0; i < 8; ++i) p += qv[j][i] * k[i];
      for (int o = 1; o < lpt; o <<= 1) p += shfl_xor_f(p, o);
      s[j] = p;
    }
    if (valid) {
#pragma unroll
      for (int j = 0; j < kGenericGroup; ++j) {
        const float mn = fmaxf(m[j], s[j]);
        const float f = fast_exp2((m[j] - mn) * kLog2e);
        const float p = fast_exp2((s[j] - mn) * kLog2e);
        m[j] = mn;
        l[j] = l[j] * f + p;
#pragma unroll
        for (int i = 0; i < 8; ++i) acc[j][i] = acc[j][i] * f + p * v[i];
      }
    }
  }

  // merge the token sub-groups of this wave (lanes with equal w)
  for (int o = lpt; o < 64; o <<= 1) {
#pragma unroll
    for (int j = 0; j < kGenericGroup; ++j) {
      const float mo = shfl_xor_f(m[j], o), lo = shfl_xor_f(l[j], o);
      float wa, wb, mn;
      merge_weights(m[j], mo, wa, wb, mn);
      m[j] = mn;
      l[j] = l[j] * wa + lo * wb;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float ao = shfl_xor_f(acc[j][i], o);
        acc[j][i] = acc[j][i] * wa + ao * wb;
      }
    }
  }

  // merge the 4 waves through LDS
  __shared__ float s_m[4][kGenericGroup], s_l[4][kGenericGroup];
  __shared__ float s_acc[4][kGenericGroup][kMaxHeadDim];
  __shared__ int s_last;
  if (sub == 0) {
#pragma unroll
    for (int j = 0; j < kGenericGroup; ++j) {
      if (w == 0) {
        s_m[wave][j] = m[j];
        s_l[wave][j] = l[j];
      }
#pragma unroll
      for (int i = 0; i < 8; ++i)
        if (wok && 8 * w + i < a.D) s_acc[wave][j][8 * w + i] = acc[j][i];
    }
  }
  __syncthreads();

  const bool direct = a.nsplit == 1;
  for (int e = tid; e < gn * a.D; e += 256) {
    const int j = e / a.D, dim = e - j * a.D;
    float M = -INFINITY;
    for (int wv = 0; wv < 4; ++wv) M = fmaxf(M, s_m[wv][j]);
    float L = 0.f, O = 0.f;
    if (M != -INFINITY) {
      for (int wv = 0; wv < 4; ++wv) {
        const float f = fast_exp2((s_m[wv][j] - M) * kLog2e);
        L += s_l[wv][j] * f;
        O += s_acc[wv][j][dim] * f;
      }
    }
    const int qh = h * a.G + j0 + j;
    const int64_t bq = (int64_t)b * a.nq + qh;
    if (direct) {
      store_any(a.out_dtype, a.out, bq * a.D + dim, L > 0.f ? O / L : 0.f);
    } else {
      a.part_acc[(bq * a.nsplit + split) * a.D + dim] = O;
      if (dim == 0) {
        a.part_ml[(bq * a.nsplit + split) * 2 + 0] = M;
        a.part_ml[(bq * a.nsplit + split) * 2 + 1] = L;
      }
    }
  }
  if (direct) return;

  // last workgroup of this (b, h, chunk) merges all splits
  __threadfence();
  __syncthreads();
  uint32_t *ctr = a.counters + ((int64_t)b * a.H + h) * a.n_chunks + chunk;
  if (tid == 0) {
    const uint32_t prev = __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_ACQ_REL,
                                                 __HIP_MEMORY_SCOPE_AGENT);
    s_last = (prev == (uint32_t)(a.nsplit - 1));
  }
  __syncthreads();
  if (!s_last) return;
  __threadfence();

  __shared__ float s_w[kMaxSplits];
  __shared__ float s_red[256];
  for (int j = 0; j < gn; ++j) {
    const int qh = h * a.G + j0 + j;
    const int64_t bq = (int64_t)b * a.nq + qh;
    const float *ml = a.part_ml + bq * a.nsplit * 2;
    float mx = -INFINITY;
    for (int sp = tid; sp < a.nsplit; sp += 256) mx = fmaxf(mx, ml[2 * sp]);
    s_red[tid] = mx;
    __syncthreads();
    for (int o = 128; o > 0; o >>= 1) {
      if (tid < o) s_red[tid] = fmaxf(s_red[tid], s_red[tid + o]);
      __syncthreads();
    }
    const float M = s_red[0];
    __syncthreads();
    float lsum = 0.f;
    for (int sp = tid; sp < a.nsplit; sp += 256) {
      const float f = (M == -INFINITY) ? 0.f : fast_exp2((ml[2 * sp] - M) * kLog2e);
      s_w[sp] = f;
      lsum += ml[2 * sp + 1] * f;
    }
    s_red[tid] = lsum;
    __syncthreads();
    for (int o = 128; o > 0; o >>= 1) {
      if (tid < o) s_red[tid] += s_red[tid + o];
      __syncthreads();
    }
    const float L = s_red[0];
    const float inv = L > 0.f ? 1.f / L : 0.f;
    for (int dim = tid; dim < a.D; dim += 256) {
      float O = 0.f;
      for (int sp = 0; sp < a.nsplit; ++sp)
        O += a.part_acc[(bq * a.nsplit + sp) * a.D + dim] * s_w[sp];
      store_any(a.out_dtype, a.out, bq * a.D + dim, O * inv);
    }
    __syncthreads();
  }
  if (tid == 0) __hip_atomic_store(ctr, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------
struct SplitPlan {
  int nsplit;
  int64_t split_len;
};

// Splits sized so that the grid holds ~2 workgroups per CU (256 CUs), each
// split a multiple of 64 tokens, at most kMaxSplits splits.
static SplitPlan plan_splits(int B, int H, int n_chunks, int64_t max_T) {
  SplitPlan p;
  const int64_t groups = (int64_t)B * H * n_chunks;
  const int64_t target = 512;
  int64_t ns = (target + groups - 1) / groups;
  if (max_T <= 0) max_T = 1;
  int64_t len = (max_T + ns - 1) / ns;
  len = ((len + 63) / 64) * 64;
  if (len < 64) len = 64;
  ns = (max_T + len - 1) / len;
  if (ns > kMaxSplits) {
    len = (max_T + kMaxSplits - 1) / kMaxSplits;
    len = ((len + 63) / 64) * 64;
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

static size_t round256(size_t x) { return (x + 255) / 256 * 256; }

static size_t workspace_bytes_for(int B, int H, int nq, int D, int n_chunks, int nsplit) {
  (void)H;
  (void)n_chunks;
  const size_t ml = (size_t)B * nq * nsplit * 2 * sizeof(float);
  const size_t acc = (size_t)B * nq * nsplit * D * sizeof(float);
  return kCounterRegion + round256(ml) + round256(acc);
}

static void carve_workspace(DecodeArgs &a, void *ws) {
  char *p = (char *)ws;
  a.counters = (uint32_t *)p;
  p += kCounterRegion;
  const size_t ml = (size_t)a.B * a.nq * a.nsplit * 2 * sizeof(float);
  a.part_ml = (float *)p;
  p += round256(ml);
  a.part_acc = (float *)p;
}

static int lpt_log2_for(int W) {
  int l = 0;
  while ((1 << l) < W) ++l;
  return l;
}

static int launch_generic(DecodeArgs &a, int64_t max_T, void *workspace, size_t ws_bytes,
                          hipStream_t stream) {
  a.n_chunks = (a.G + kGenericGroup - 1) / kGenericGroup;
  const SplitPlan p = plan_splits(a.B, a.H, a.n_chunks, max_T);
  a.nsplit = p.nsplit;
  a.split_len = p.split_len;
  a.lpt_log2 = lpt_log2_for(a.W);
  if (a.nsplit > 1) {
    if ((int64_t)a.B * a.H * a.n_chunks > kMaxCounters) return CQ_ERR_UNSUPPORTED;
    if (!workspace) return CQ_ERR_WORKSPACE;
    if (ws_bytes < workspace_bytes_for(a.B, a.H, a.nq, a.D, a.n_chunks, a.nsplit))
      return CQ_ERR_WORKSPACE;
    carve_workspace(a, workspace);
  } else {
    a.part_ml = a.part_acc = nullptr;
    a.counters = nullptr;
  }
  const dim3 grid((unsigned)a.nsplit, (unsigned)(a.H * a.n_chunks), (unsigned)a.B);
  decode_generic_kernel<<<grid, dim3(256), 0, stream>>>(a);
  return hipGetLastError() == hipSuccess ? CQ_OK : CQ_ERR_LAUNCH;
}

static int fill_decode_args(DecodeArgs &a, const cq_cache_desc *c, const void *q,
                            int q_dtype, int nq, float scale, const int32_t *seq_lens,
                            int64_t seq_len, int64_t max_T, void *out, int out_dtype) {
  if (!q || !out) return CQ_ERR_ARG;
  if (q_dtype < CQ_F16 || q_dtype > CQ_F32 || out_dtype < CQ_F16 || out_dtype > CQ_F32)
    return CQ_ERR_DTYPE;
  if (nq < 1 || nq % c->n_kv_heads != 0) return CQ_ERR_SHAPE;
  if (seq_len < 0 || max_T < 0) return CQ_ERR_ARG;
  if (!seq_lens) max_T = seq_len;
  const cq_component *cp[2] = {&c->k, &c->v};
  for (int i = 0; i < 2; ++i) {
    a.kf[i] = cp[i]->keyframes;
    a.pk[i] = cp[i]->packed;
    a.sc[i] = cp[i]->scales;
    a.cap_kf[i] = cp[i]->cap_keyframes;
    a.cap_pf[i] = cp[i]->cap_pframes;
    a.stride[i] = cp[i]->stride;
    if (num_keyframes(max_T, cp[i]->stride) > cp[i]->cap_keyframes ||
        num_pframes(max_T, cp[i]->stride) > cp[i]->cap_pframes)
      return CQ_ERR_CAPACITY;
  }
  a.B = c->batch;
  a.H = c->n_kv_heads;
  a.D = c->head_dim;
  a.W = (c->head_dim + 7) / 8;
  a.nq = nq;
  a.G = nq / c->n_kv_heads;
  a.q = q;
  a.q_dtype = q_dtype;
  a.scale = scale;
  a.seq_lens = seq_lens;
  a.seq_len = seq_len;
  a.max_T = max_T;
  a.out = out;
  a.out_dtype = out_dtype;
  return CQ_OK;
}

}  // namespace cq

using namespace cq;

extern "C" {

size_t cq_decode_workspace_size(int32_t batch, int32_t n_kv_heads, int32_t n_q_heads,
                                int32_t head_dim, int64_t max_seq_len) {
  if (batch < 1 || n_kv_heads < 1 || n_q_heads < 1 || head_dim < 1) return 0;
  const int G = n_q_heads / n_kv_heads;
  const int n_chunks = (G + kGenericGroup - 1) / kGenericGroup;
  const SplitPlan p = plan_splits(batch, n_kv_heads, n_chunks, max_seq_len);
  return workspace_bytes_for(batch, n_kv_heads, n_q_heads, head_dim, n_chunks, p.nsplit);
}

int cq_decode_attn_generic(const cq_cache_desc *cache, const void *q, int32_t q_dtype,
                           int32_t n_q_heads, float scale, const int32_t *seq_lens,
                           int64_t seq_len, int64_t max_seq_len, void *out,
                           int32_t out_dtype, void *workspace, size_t workspace_bytes,
                           cq_stream_t stream) {
  int st = validate_cache(cache);
  if (st) return st;
  DecodeArgs a;
  st = fill_decode_args(a, cache, q, q_dtype, n_q_heads, scale, seq_lens, seq_len,
                        max_seq_len, out, out_dtype);
  if (st) return st;
  const int64_t max_T = seq_lens ? max_seq_len : seq_len;
  return launch_generic(a, max_T, workspace, workspace_bytes, (hipStream_t)stream);
}

int cq_decode_attn(const cq_cache_desc *cache, const void *q, int32_t q_dtype,
                   int32_t n_q_heads, float scale, const int32_t *seq_lens,
                   int64_t seq_len, int64_t max_seq_len, void *out, int32_t out_dtype,
                   void *workspace, size_t workspace_bytes, cq_stream_t stream) {
  return cq_decode_attn_generic(cache, q, q_dtype, n_q_heads, scale, seq_lens, seq_len,
                                max_seq_len, out, out_dtype, workspace, workspace_bytes,
                                stream);
}

int cq_fp16_decode_attn(const uint16_t *k, const uint16_t *v, int64_t cap_tokens,
                        int32_t batch, int32_t n_kv_heads, int32_t head_dim, const void *q,
                        int32_t q_dtype, int32_t n_q_heads, float scale,
                        const int32_t *seq_lens, int64_t seq_len, int64_t max_seq_len,
                        void *out, int32_t out_dtype, void *workspace,
                        size_t workspace_bytes, cq_stream_t stream) {
  // A plain fp16 cache is a ChronoQuant component with stride 1 (every token
  // an I-frame); the P-frame arrays are never read.
  if (!k || !v) return CQ_ERR_ARG;
  cq_cache_desc c{};
  c.batch = batch;
  c.n_kv_heads = n_kv_heads;
  c.head_dim = head_dim;
  static uint32_t dummy_words;
  static uint16_t dummy_scales;
  for (cq_component *p : {&c.k, &c.v}) {
    p->packed = &dummy_words;
    p->scales = &dummy_scales;
    p->cap_keyframes = cap_tokens;
    p->cap_pframes = 1;
    p->stride = 1;
    p->delta_bits = 4;
    p->dead_zone = 0.f;
  }
  c.k.keyframes = const_cast<uint16_t *>(k);
  c.v.keyframes = const_cast<uint16_t *>(v);
  return cq_decode_attn_generic(&c, q, q_dtype, n_q_heads, scale, seq_lens, seq_len,
                                max_seq_len, out, out_dtype, workspace, workspace_bytes,
                                stream);
}

}  // extern "C"
