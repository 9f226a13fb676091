// cq_decode.hip — decode-attention entry points and the portable decode kernel.
//
// Work split (both kernels): grid (split, kv head x q-head chunk, sequence).
// Each workgroup owns a contiguous token range of one (sequence, kv head) and
// a chunk of the q heads of that GQA group, so every compressed byte is read
// once per chunk.  cq_decode_attn routes head_dim 128 with fp16 queries to the
// MFMA kernel (cq_decode_mfma.hip) and everything else to the portable kernel.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <math.h>
#include <stdlib.h>

#include <mutex>

#include "cq_decode_common.h"

namespace cq {

constexpr int kGenericGroup = 8;  // q heads per workgroup in the portable kernel

__device__ __forceinline__ float shfl_xor_f(float v, int m) { return __shfl_xor(v, m, 64); }

__device__ __forceinline__ void merge_weights(float m, float mo, float &wa, float &wb, float &mn) {
  mn = fmaxf(m, mo);
  if (mn == -INFINITY) {
    wa = 0.f;
    wb = 0.f;
  } else {
    wa = fast_exp2(m - mn);
    wb = fast_exp2(mo - mn);
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
    const int fb = a.fbits[ci], rw = row_words_of(a.D, fb);
    // the fields of dims 8w .. 8w + 7 (one word of an INT4 row)
    const uint32_t f8 = stream_bits(a.pk[ci] + (bh * a.cap_pf[ci] + slot) * rw, rw, 8 * fb * w, 8 * fb);
    const float s = h2f(a.sc[ci][bh * a.cap_pf[ci] + slot]);
    const uint32_t mask = (1u << fb) - 1u;
    const int bias = 1 << (fb - 1);
#pragma unroll
    for (int i = 0; i < 8; ++i) x[i] += (float)((int)((f8 >> (fb * i)) & mask) - bias) * s;
  }
}

// Portable decode kernel: lanes per token = pow2 >= W words; each lane owns
// one 8-dim word of its token.  Exact per-token online softmax in fp32.
__global__ __launch_bounds__(256) void decode_generic_kernel(DecodeArgs a) {
  prefetch_args();
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
  const int64_t T = seq_len_of(a, b);
  const int64_t t0 = (int64_t)split * a.split_len;
  const int64_t t1 = min(T, t0 + a.split_len);
  if (split_is_empty(split, t0, T)) return;
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
        v = round_any(a.q_dtype,
                      load_any(a.q_dtype, a.q, ((int64_t)b * a.nq + qh) * a.D + dim) * sc_r);
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
      s[j] = p * kLog2e;
    }
    if (valid) {
#pragma unroll
      for (int j = 0; j < kGenericGroup; ++j) {
        const float mn = fmaxf(m[j], s[j]);
        const float f = fast_exp2(m[j] - mn);
        const float p = fast_exp2(s[j] - mn);
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
  // the combine scratch aliases the wave accumulators once they are merged
  constexpr int kAccFloats = 4 * kGenericGroup * kMaxHeadDim;
  __shared__ float s_acc_raw[kAccFloats];
  float(*s_acc)[kGenericGroup][kMaxHeadDim] = (float(*)[kGenericGroup][kMaxHeadDim])s_acc_raw;
  __shared__ float w_m[kGenericGroup], w_l[kGenericGroup];
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
  if (tid < gn) {
    float M = -INFINITY;
    for (int wv = 0; wv < 4; ++wv) M = fmaxf(M, s_m[wv][tid]);
    float L = 0.f;
    if (M != -INFINITY)
      for (int wv = 0; wv < 4; ++wv) L += s_l[wv][tid] * fast_exp2(s_m[wv][tid] - M);
    w_m[tid] = M;
    w_l[tid] = L;
  }
  __syncthreads();
  for (int e = tid; e < gn * a.D; e += 256) {
    const int j = e / a.D, dim = e - j * a.D;
    const float M = w_m[j];
    float O = 0.f;
    if (M != -INFINITY)
      for (int wv = 0; wv < 4; ++wv) O += s_acc[wv][j][dim] * fast_exp2(s_m[wv][j] - M);
    s_acc[0][j][dim] = O;  // each (j, dim) is read and rewritten by one thread
  }
  __syncthreads();
  finish_workgroup(a, b, h, chunk, j0, gn, split, kGridLive, w_m, w_l, &s_acc[0][0][0],
                   kMaxHeadDim);
}

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------
static int lpt_log2_for(int W) {
  int l = 0;
  while ((1 << l) < W) ++l;
  return l;
}

static std::atomic<int> g_poll_rounds{kDefaultPollRounds};

int current_poll_rounds() { return g_poll_rounds.load(std::memory_order_relaxed); }

int64_t split_tokens_override() {
  static const int64_t v = [] {
    const char *e = getenv("CQ_DECODE_SPLIT_TOKENS");
    if (!e || !*e) return (int64_t)0;
    char *end = nullptr;
    const long long x = strtoll(e, &end, 10);
    // whole split granules only: every kernel's split plan assumes them
    return (end && *end == 0 && x > 0 && x % kSplitGranule == 0 && x <= (1 << 24))
               ? (int64_t)x
               : (int64_t)0;
  }();
  return v;
}

int64_t resident_workgroups(const void *kernel, int threads, int slot) {
  constexpr int kMaxDevices = 64;
  static std::atomic<int64_t> cache[kMaxDevices][kSlotCount];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) dev = 0;
  const bool cached = dev >= 0 && dev < kMaxDevices;
  if (cached) {
    const int64_t v = cache[dev][slot].load(std::memory_order_relaxed);
    if (v > 0) return v;
  }
  int cus = 0, per_cu = 0;
  const bool ok =
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess &&
      hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, threads, 0) == hipSuccess &&
      cus > 0 && per_cu > 0;
  (void)hipGetLastError();
  if (!ok) return 256;  // no device answer: plan for one MI355X generation
  const int64_t v = (int64_t)cus * per_cu;
  if (cached) cache[dev][slot].store(v, std::memory_order_relaxed);
  return v;
}

static int64_t generic_resident() {
  return resident_workgroups(reinterpret_cast<const void *>(decode_generic_kernel), 256,
                             kSlotGeneric);
}

int64_t decode_max_resident() { return std::max(generic_resident(), mfma_max_resident()); }

static int launch_generic(DecodeArgs &a, void *workspace, size_t ws_bytes, hipStream_t stream) {
  int st = prepare_launch(a, kGenericGroup, generic_resident(), workspace, ws_bytes);
  if (st) return st;
  a.lpt_log2 = (int16_t)lpt_log2_for(a.W);
  const dim3 grid((unsigned)a.nsplit, (unsigned)(a.H * a.n_chunks), (unsigned)a.B);
  decode_generic_kernel<<<grid, dim3(256), 0, stream>>>(a);
  return hipGetLastError() == hipSuccess ? CQ_OK : CQ_ERR_LAUNCH;
}

static int fill_decode_args(DecodeArgs &a, const cq_cache_desc *c, const void *q, int q_dtype,
                            int nq, float scale, const int32_t *seq_lens, int64_t seq_len,
                            int64_t max_T, void *out, int out_dtype) {
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
    a.inv_stride[i] = 1.0f / (float)cp[i]->stride;
    a.fbits[i] = (int8_t)field_bits(*cp[i]);
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

static int decode_entry(const cq_cache_desc *cache, const void *q, int32_t q_dtype,
                        int32_t n_q_heads, float scale, const int32_t *seq_lens, int64_t seq_len,
                        int64_t max_seq_len, void *out, int32_t out_dtype, void *workspace,
                        size_t workspace_bytes, cq_stream_t stream, bool allow_mfma) {
  int st = validate_cache(cache);
  if (st) return st;
  DecodeArgs a;
  st = fill_decode_args(a, cache, q, q_dtype, n_q_heads, scale, seq_lens, seq_len, max_seq_len,
                        out, out_dtype);
  if (st) return st;
  if (allow_mfma && mfma_supported(a))
    return launch_decode_mfma(a, workspace, workspace_bytes, (hipStream_t)stream);
  return launch_generic(a, workspace, workspace_bytes, (hipStream_t)stream);
}

// ---------------------------------------------------------------------------
// static scratch of cq_decode_attn_noalloc
// ---------------------------------------------------------------------------
// The split partials and counters of the allocation-free decode.  Each GPU
// that loads this code object holds its own zero-filled copy until the
// process ends; the decode kernels return the counters to zero after every
// call.  In host code `scratch` names a host-side stand-in, never the device
// copy: kernels receive the per-device address resolved below.
constexpr size_t kScratchBytes = CQ_NOALLOC_SCRATCH_BYTES;
__device__ __align__(256) unsigned char scratch[kScratchBytes];

constexpr int kMaxScratchDevices = 64;
static std::atomic<void *> g_scratch[kMaxScratchDevices];
static std::mutex g_scratch_mu;

// Device address of the current device's scratch, resolved once per device.
static int current_scratch(void **out) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) {
    (void)hipGetLastError();
    return CQ_ERR_LAUNCH;
  }
  if (dev < 0 || dev >= kMaxScratchDevices) return CQ_ERR_UNSUPPORTED;
  void *p = g_scratch[dev].load(std::memory_order_acquire);
  if (!p) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    p = g_scratch[dev].load(std::memory_order_relaxed);
    if (!p) {
      const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
      if (e != hipSuccess || !p) {
        (void)hipGetLastError();
        return CQ_ERR_LAUNCH;
      }
      g_scratch[dev].store(p, std::memory_order_release);
    }
  }
  *out = p;
  return CQ_OK;
}

}  // namespace cq

using namespace cq;

extern "C" {

size_t cq_decode_workspace_size(int32_t batch, int32_t n_kv_heads, int32_t n_q_heads,
                                int32_t head_dim, int64_t max_seq_len) {
  if (batch < 1 || n_kv_heads < 1 || n_q_heads < 1 || head_dim < 1) return 0;
  // enough for the grid plan of every decode kernel and for the balanced
  // plan of the MFMA kernels (at most resident / n_kv_heads workgroups per
  // column)
  const SplitPlan p = plan_splits((int64_t)batch * n_kv_heads, max_seq_len, decode_max_resident());
  const int64_t bal = balanced_slots(std::max((int64_t)1, decode_max_resident() / n_kv_heads),
                                     max_seq_len);
  return workspace_bytes_for(batch, n_q_heads, head_dim, (int)std::max((int64_t)p.nsplit, bal));
}

int cq_decode_attn_generic(const cq_cache_desc *cache, const void *q, int32_t q_dtype,
                           int32_t n_q_heads, float scale, const int32_t *seq_lens,
                           int64_t seq_len, int64_t max_seq_len, void *out, int32_t out_dtype,
                           void *workspace, size_t workspace_bytes, cq_stream_t stream) {
  return decode_entry(cache, q, q_dtype, n_q_heads, scale, seq_lens, seq_len, max_seq_len, out,
                      out_dtype, workspace, workspace_bytes, stream, false);
}

int cq_decode_attn(const cq_cache_desc *cache, const void *q, int32_t q_dtype,
                   int32_t n_q_heads, float scale, const int32_t *seq_lens, int64_t seq_len,
                   int64_t max_seq_len, void *out, int32_t out_dtype, void *workspace,
                   size_t workspace_bytes, cq_stream_t stream) {
  return decode_entry(cache, q, q_dtype, n_q_heads, scale, seq_lens, seq_len, max_seq_len, out,
                      out_dtype, workspace, workspace_bytes, stream, true);
}

int cq_decode_attn_noalloc(const cq_cache_desc *cache, const void *q, int32_t q_dtype,
                           int32_t n_q_heads, float scale, const int32_t *seq_lens,
                           int64_t seq_len, int64_t max_seq_len, void *out, int32_t out_dtype,
                           cq_stream_t stream) {
  int st = validate_cache(cache);
  if (st) return st;
  if (n_q_heads < 1 || seq_len < 0 || max_seq_len < 0) return CQ_ERR_ARG;
  // the bound every plan of this shape fits in (the size cq_decode_workspace_size
  // asks callers of cq_decode_attn for)
  const size_t need = cq_decode_workspace_size(cache->batch, cache->n_kv_heads, n_q_heads,
                                               cache->head_dim, seq_lens ? max_seq_len : seq_len);
  if (need > kScratchBytes) return CQ_ERR_SCRATCH;
  void *ws = nullptr;
  st = current_scratch(&ws);
  if (st) return st;
  return decode_entry(cache, q, q_dtype, n_q_heads, scale, seq_lens, seq_len, max_seq_len, out,
                      out_dtype, ws, kScratchBytes, stream, true);
}

int cq_decode_status(void *workspace, cq_stream_t stream) {
  if (!workspace) {
    const int st = current_scratch(&workspace);
    if (st) return st;
  }
  if ((uintptr_t)workspace & 255) return CQ_ERR_ALIGN;
  const hipStream_t s = (hipStream_t)stream;
  uint32_t word = 0;
  if (hipStreamSynchronize(s) != hipSuccess ||
      hipMemcpy(&word, (char *)workspace + kStatusOffset, sizeof(word), hipMemcpyDeviceToHost) !=
          hipSuccess) {
    (void)hipGetLastError();
    return CQ_ERR_LAUNCH;
  }
  if (word == 0) return CQ_OK;
  // every kernel of the stream has finished, so no late split store can land
  // after this clear
  if (hipMemsetAsync(workspace, 0, kCounterRegion, s) != hipSuccess ||
      hipStreamSynchronize(s) != hipSuccess) {
    (void)hipGetLastError();
    return CQ_ERR_LAUNCH;
  }
  return CQ_ERR_TIMEOUT;
}

int32_t cq_set_fold_poll_bound(int32_t rounds) {
  return g_poll_rounds.exchange(rounds < 1 ? kDefaultPollRounds : rounds,
                                std::memory_order_relaxed);
}

int cq_fp16_decode_attn(const uint16_t *k, const uint16_t *v, int64_t cap_tokens,
                        int32_t batch, int32_t n_kv_heads, int32_t head_dim, const void *q,
                        int32_t q_dtype, int32_t n_q_heads, float scale,
                        const int32_t *seq_lens, int64_t seq_len, int64_t max_seq_len,
                        void *out, int32_t out_dtype, void *workspace,
                        size_t workspace_bytes, cq_stream_t stream) {
  // A plain fp16 cache is a ChronoQuant component with stride 1: every token
  // is an I-frame, so only the anchor path runs and the P-frame arrays are
  // never dereferenced (they get the K/V pointers as placeholders).
  if (!k || !v) return CQ_ERR_ARG;
  cq_cache_desc c{};
  c.batch = batch;
  c.n_kv_heads = n_kv_heads;
  c.head_dim = head_dim;
  const uint16_t *src[2] = {k, v};
  cq_component *comp[2] = {&c.k, &c.v};
  for (int i = 0; i < 2; ++i) {
    comp[i]->keyframes = const_cast<uint16_t *>(src[i]);
    comp[i]->packed = (uint32_t *)const_cast<uint16_t *>(src[i]);
    comp[i]->scales = const_cast<uint16_t *>(src[i]);
    comp[i]->cap_keyframes = cap_tokens;
    comp[i]->cap_pframes = 1;
    comp[i]->stride = 1;
    comp[i]->delta_bits = 4;
    comp[i]->dead_zone = 0.f;
    comp[i]->packing = CQ_PACK_INT4;
  }
  int st = validate_cache(&c);
  if (st) return st;
  DecodeArgs a;
  st = fill_decode_args(a, &c, q, q_dtype, n_q_heads, scale, seq_lens, seq_len, max_seq_len, out,
                        out_dtype);
  if (st) return st;
  // the purpose-built fp16 kernel where it applies (head_dim 128, GQA <= 4,
  // fp16 queries), else the compressed-cache kernels over stride-1 components
  if (fp16_g4_supported(a))
    return launch_decode_fp16_g4(a, workspace, workspace_bytes, (hipStream_t)stream);
  return decode_entry(&c, q, q_dtype, n_q_heads, scale, seq_lens, seq_len, max_seq_len, out,
                      out_dtype, workspace, workspace_bytes, stream, true);
}

}  // extern "C"
