// cq_decode_common.h — pieces shared by the decode kernels: argument block,
// split planning, workspace layout, and the per-workgroup epilogue (direct
// output, or split partial + last-workgroup log-sum-exp combine).
//
// Softmax state is kept in the log2 domain everywhere: scores are multiplied
// by log2(e) once and every exponential is exp2.
#pragma once

#include <hip/hip_runtime.h>
#include <math.h>

#include "cq_device.h"
#include "cq_plan.h"

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
  uint32_t *flags;     // [B][H][nsplit] split-ready flags (GQA-4 kernel); null: tickets
  uint32_t *recs;      // [B][H][nsplit][64 units] fold records (GQA-4 grid plan); null: unused
  int nsplit;
  int64_t split_len;
  int16_t lpt_log2; // portable kernel: lanes per token = 1 << lpt_log2 (>= W)
  int8_t fbits[2];  // stored field bits per component: 4 (INT4 lanes) or the dense width
  int poll_rounds;  // bound of the split waits (fold records, split-ready flags)
  uint32_t *status; // sticky status word of the workspace (kStatus* bits)
};

// Kernel arguments are read through the scalar cache, which every dispatch
// starts cold.  The compiler places each argument's load at its first use, and
// first uses behind branches cost one dependent miss each before the first
// vector load can issue.  Touching every 64-byte line of the argument block at
// entry turns them into one round trip; later argument loads hit.
__device__ __forceinline__ void prefetch_args() {
  static_assert(sizeof(DecodeArgs) <= 256, "argument block spans more than four lines");
  const void *p = (const void *)__builtin_amdgcn_kernarg_segment_ptr();
  uint32_t d0, d1, d2, d3;
  asm volatile(
      "s_load_dword %0, %4, 0x0\n\t"
      "s_load_dword %1, %4, 0x40\n\t"
      "s_load_dword %2, %4, 0x80\n\t"
      "s_load_dword %3, %4, 0xc0\n\t"
      "s_waitcnt lgkmcnt(0)"
      : "=s"(d0), "=s"(d1), "=s"(d2), "=s"(d3)
      : "s"(p));
}

#ifdef CQ_PHASE_TIMES
// Diagnostic build only (libchronoquant_phases.so, built with
// -DCQ_PHASE_TIMES; see phase_times.py): thread 0 of every workgroup of a
// fold-record launch stores the device clock (s_memrealtime, 100 MHz, the
// same on every CU) at phase p into slot [linear workgroup][p] of the
// split-partial area, which such launches leave unused.
// (Wave 0 stores, every lane the same value: a branch on the thread index
// would make the compiler treat the block indices behind it as divergent
// and wrap the kernel's buffer loads in waterfall loops.)
__device__ __forceinline__ void phase_mark(const DecodeArgs &a, int p) {
  if (__builtin_amdgcn_readfirstlane(threadIdx.x >> 6) == 0 && a.recs && a.part_acc) {
    const uint32_t wg = blockIdx.x + gridDim.x * (blockIdx.y + gridDim.y * blockIdx.z);
    ((uint64_t *)a.part_acc)[wg * 8u + (uint32_t)p] = __builtin_amdgcn_s_memrealtime();
  }
}
#else
__device__ __forceinline__ void phase_mark(const DecodeArgs &, int) {}
#endif

__device__ __forceinline__ int64_t seq_len_of(const DecodeArgs &a, int b) {
  return a.seq_lens ? min((int64_t)max(a.seq_lens[b], 0), a.max_T) : a.seq_len;
}

// Grid plan (one split of split_len tokens per workgroup, grid x): a split
// past its sequence's end has nothing to do and takes no part in the combine;
// split 0 always takes part.  Called by a whole workgroup before any barrier.
__device__ __forceinline__ bool split_is_empty(int split, int64_t t0, int64_t T) {
  return split > 0 && t0 >= T;
}
// Grid plan: splits holding tokens of a sequence of length T (at least 1:
// split 0 answers an empty sequence).
__device__ __forceinline__ int grid_live(const DecodeArgs &a, int64_t T) {
  return (int)max((int64_t)1, min((int64_t)a.nsplit, (T + a.split_len - 1) / a.split_len));
}
constexpr int kGridLive = -1;  // finish_workgroup: live count from the grid plan

// Balanced plan (cq_plan.h): start[b] = first unit of sequence b, start[B] =
// total units, for per-sequence lengths.  Wave 0 scans 64 sequences at a
// time; the whole workgroup syncs once.
__device__ __forceinline__ void build_unit_table(const DecodeArgs &a, int32_t *start) {
  const int tid = threadIdx.x;
  if (tid < 64) {
    int32_t carry = 0;
    for (int b0 = 0; b0 < a.B; b0 += 64) {
      const int b = b0 + tid;
      int32_t n = b < a.B ? (int32_t)units_of(seq_len_of(a, b)) : 0;
#pragma unroll
      for (int d = 1; d < 64; d *= 2) {
        const int32_t y = __shfl_up(n, d, 64);
        if (tid >= d) n += y;
      }
      if (b < a.B) start[b + 1] = carry + n;
      carry += __shfl(n, 63, 64);
    }
    if (tid == 0) start[0] = 0;
  }
  __syncthreads();
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

// Buffer resource over [base, base + bytes): loads past the end return 0.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void *base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, (int)bytes,
                                           0x00020000);
}
// Vector forms of the device-scope accesses above: the same sc1 cache policy
// (cache-policy operand 16), 8 or 16 bytes per access.
constexpr int kPolicyDevice = 16;
typedef float f2v_t __attribute__((ext_vector_type(2)));
typedef float f4v_t __attribute__((ext_vector_type(4)));
typedef _Float16 h2v_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ f2v_t load_dev2(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(f2v_t, __builtin_amdgcn_raw_buffer_load_b64(r, (int)off, 0, kPolicyDevice));
}
__device__ __forceinline__ f4v_t load_dev4(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(f4v_t, __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, kPolicyDevice));
}
__device__ __forceinline__ float load_dev1(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, (int)off, 0, kPolicyDevice));
}
__device__ __forceinline__ void store_dev2(__amdgpu_buffer_rsrc_t r, uint32_t off, f2v_t v) {
  __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(
      __attribute__((ext_vector_type(2))) int, v), r, (int)off, 0, kPolicyDevice);
}
__device__ __forceinline__ void store_dev4(__amdgpu_buffer_rsrc_t r, uint32_t off, f4v_t v) {
  __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(
      __attribute__((ext_vector_type(4))) int, v), r, (int)off, 0, kPolicyDevice);
}
__device__ __forceinline__ void store_dev1(__amdgpu_buffer_rsrc_t r, uint32_t off, float v) {
  __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(int, v), r, (int)off, 0, kPolicyDevice);
}

constexpr int kCombineBatch = 8;  // splits whose loads are in flight together

// The last workgroup's fold of the nsplit partials of every (head, 4 dims).
// A unit's `slices` threads are adjacent lanes (slices a power of two <= 64),
// so the slices fold with xor shuffles: no LDS, no barrier.  The batch loop is
// fully unrolled and branch-free, so all of a batch's loads are in flight
// together (a branch inside it would make the compiler wait for each load).
template <bool Vec>
__device__ __forceinline__ void merge_partials(const DecodeArgs &a, __amdgpu_buffer_rsrc_t racc,
                                               __amdgpu_buffer_rsrc_t rml, int64_t bq0, int gn,
                                               int nsplit) {
  const int tid = threadIdx.x, nthr = blockDim.x;
  const int D = a.D, nd4 = (D + 3) / 4;
  const int units = gn * nd4;
  int slices = 1;
  while (slices * 2 <= nsplit && units * slices * 2 <= nthr && slices < 64) slices *= 2;
  const int rounds = (units * slices + nthr - 1) / nthr;
  for (int rd = 0; rd < rounds; ++rd) {
    const int t = rd * nthr + tid;
    const int u = t / slices, sl = t - u * slices;
    const bool live = u < units;  // whole slice groups are live together
    const int uu = live ? u : 0;
    const int j = uu / nd4, d0 = 4 * (uu - j * nd4);
    const uint32_t row0 = (uint32_t)((bq0 + j) * a.nsplit);  // rows hold a.nsplit slots
    float M = -INFINITY, L = 0.f;
    float o[4] = {0.f, 0.f, 0.f, 0.f};
    for (int sp0 = sl; sp0 < nsplit; sp0 += kCombineBatch * slices) {
      f2v_t ml[kCombineBatch];
      f4v_t ov[kCombineBatch];
#pragma unroll
      for (int k = 0; k < kCombineBatch; ++k) {
        // splits past the end re-read the last live split (written by this
        // call) and are masked below
        const uint32_t spo = row0 + (uint32_t)min(sp0 + k * slices, nsplit - 1);
        ml[k] = load_dev2(rml, spo * 8u);
        const uint32_t off = (spo * (uint32_t)D + (uint32_t)d0) * 4u;
        if constexpr (Vec) {
          ov[k] = load_dev4(racc, off);
        } else {
          // dims past D read the next row (or zeros past the buffer): unused
          ov[k] = f4v_t{load_dev1(racc, off), load_dev1(racc, off + 4u), load_dev1(racc, off + 8u),
                        load_dev1(racc, off + 12u)};
        }
      }
      float mb = M;
#pragma unroll
      for (int k = 0; k < kCombineBatch; ++k) {
        if (sp0 + k * slices >= nsplit) ml[k].x = -INFINITY;
        mb = fmaxf(mb, ml[k].x);
      }
      // no branch on mb: a branch would let the compiler sink the partial
      // loads below it, a second round trip.  mb = -inf (nothing yet) gives
      // zero factors and weights.
      const float mref = (mb == -INFINITY) ? 0.f : mb;
      const float f = (M == -INFINITY) ? 0.f : fast_exp2(M - mref);
      L *= f;
#pragma unroll
      for (int c = 0; c < 4; ++c) o[c] *= f;
#pragma unroll
      for (int k = 0; k < kCombineBatch; ++k) {
        const float w = (ml[k].x == -INFINITY) ? 0.f : fast_exp2(ml[k].x - mref);
        L += w * ml[k].y;
        o[0] += w * ov[k].x;
        o[1] += w * ov[k].y;
        o[2] += w * ov[k].z;
        o[3] += w * ov[k].w;
      }
      M = mb;
    }
    // fold the slices of the unit (adjacent lanes)
    float Mx = M;
    for (int x = 1; x < slices; x *= 2) Mx = fmaxf(Mx, __shfl_xor(Mx, x, 64));
    const float f = (M == -INFINITY) ? 0.f : fast_exp2(M - Mx);
    L *= f;
#pragma unroll
    for (int c = 0; c < 4; ++c) o[c] *= f;
    for (int x = 1; x < slices; x *= 2) {
      L += __shfl_xor(L, x, 64);
#pragma unroll
      for (int c = 0; c < 4; ++c) o[c] += __shfl_xor(o[c], x, 64);
    }
    if (live && sl == 0) {
      const float inv = L > 0.f ? 1.f / L : 0.f;
      const int64_t oi = (bq0 + j) * D + d0;
      if (Vec && a.out_dtype == CQ_F16) {
        const h2v_t lo = h2v_t{(_Float16)(o[0] * inv), (_Float16)(o[1] * inv)};
        const h2v_t hi = h2v_t{(_Float16)(o[2] * inv), (_Float16)(o[3] * inv)};
        *(uint2 *)((uint16_t *)a.out + oi) =
            uint2{__builtin_bit_cast(uint32_t, lo), __builtin_bit_cast(uint32_t, hi)};
      } else {
        for (int c = 0; c < 4 && d0 + c < D; ++c) store_any(a.out_dtype, a.out, oi + c, o[c] * inv);
      }
    }
  }
}

// Buffer resources over the split partials (32-bit offsets: the host bounds
// both arrays below 2^31 bytes).  Wave-uniform: per-lane resources would make
// the compiler serialise every access over the distinct resources.
__device__ __forceinline__ void partial_rsrcs(const DecodeArgs &a, __amdgpu_buffer_rsrc_t &racc,
                                              __amdgpu_buffer_rsrc_t &rml) {
  const uint32_t rows = (uint32_t)(a.B * a.nq * a.nsplit);
  racc = make_rsrc(a.part_acc, rows * (uint32_t)a.D * 4u);
  rml = make_rsrc(a.part_ml, rows * 8u);
}

// After a workgroup has issued its partial stores: wait for them and take a
// ticket on the (sequence, kv head, chunk) counter.  True (for the whole
// workgroup) in the last of the `live` workgroups, which then folds every
// partial and resets the counter (*ctr).
__device__ __forceinline__ bool split_ticket(const DecodeArgs &a, int b, int h, int chunk,
                                             int live, uint32_t *&ctr) {
  __shared__ int s_last;
  __builtin_amdgcn_s_waitcnt(0);  // this thread's partial stores are complete
  __syncthreads();
  ctr = a.counters + ((int64_t)b * a.H + h) * a.n_chunks + chunk;
  if (threadIdx.x == 0) {
    const uint32_t prev =
        __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    s_last = (prev == (uint32_t)(live - 1));
  }
  __syncthreads();
  return s_last;
}

__device__ __forceinline__ void reset_ticket(uint32_t *ctr) {
  if (threadIdx.x == 0) __hip_atomic_store(ctr, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// The split epilogue after a workgroup has issued its partial stores: the
// ticket, and in the last of the `live` workgroups the fold of every partial
// and the counter reset.  Called by the whole workgroup.
__device__ __forceinline__ void combine_tail(const DecodeArgs &a, int b, int h, int chunk, int gn,
                                             int live, bool vec, __amdgpu_buffer_rsrc_t racc,
                                             __amdgpu_buffer_rsrc_t rml, int64_t bq0) {
  uint32_t *ctr;
  if (!split_ticket(a, b, h, chunk, live, ctr)) return;
  // ---- last workgroup: fold the nsplit partials of every (head, 4 dims) ----
  if (vec) merge_partials<true>(a, racc, rml, bq0, gn, live);
  else merge_partials<false>(a, racc, rml, bq0, gn, live);
  reset_ticket(ctr);
}

// Per-workgroup epilogue.  The workgroup's merged state for q heads
// j0 .. j0+gn-1 of kv head h is in LDS: wm[j] (running max, log2 units),
// wl[j] (sum of weights), wo[j*ostride + d] (unnormalised output).  `live`
// workgroups share sequence b (kGridLive: the grid plan's splits holding
// tokens, derived here while the partial stores are in flight); this one
// holds partial slot `slot`.  With one live workgroup it writes the output;
// otherwise it writes its partial, and the last of the live workgroups of
// (b, h, chunk) to finish merges all partials and resets the counter it used.
//
// The merge costs one memory round trip: a thread owns (head, 4 dims) and a
// slice of the splits, issues every load of its splits ((m, l) pairs and
// 16-byte partial vectors) before using any, folds them with a running
// log-sum-exp, and the slices of a unit (adjacent lanes) are folded the same
// way with xor shuffles.

__device__ __forceinline__ void finish_workgroup(const DecodeArgs &a, int b, int h, int chunk,
                                                 int j0, int gn, int slot, int live,
                                                 const float *wm, const float *wl,
                                                 const float *wo, int ostride) {
  const int tid = threadIdx.x, nthr = blockDim.x;
  const int D = a.D, nd4 = (D + 3) / 4;
  const bool vec = (D & 3) == 0;  // 16-byte partial accesses
  const int64_t bq0 = (int64_t)b * a.nq + h * a.G + j0;
  if (live == kGridLive ? a.nsplit == 1 : live == 1) {
    for (int e = tid; e < gn * D; e += nthr) {
      const int j = e / D, dim = e - j * D;
      const float L = wl[j], O = wo[j * ostride + dim];
      store_any(a.out_dtype, a.out, (bq0 + j) * D + dim, L > 0.f ? O / L : 0.f);
    }
    return;
  }
  const int nsplit = a.nsplit;
  __amdgpu_buffer_rsrc_t racc, rml;
  partial_rsrcs(a, racc, rml);
  // partials: (m, l) and o of this split, 16 bytes per access
  for (int u = tid; u < gn * nd4; u += nthr) {
    const int j = u / nd4, d0 = 4 * (u - j * nd4);
    const uint32_t row = (uint32_t)((bq0 + j) * nsplit + slot);
    const uint32_t base = row * (uint32_t)D * 4u;
    const float *o = wo + j * ostride + d0;
    if (vec) {
      store_dev4(racc, base + 4u * d0, f4v_t{o[0], o[1], o[2], o[3]});
    } else {
      for (int c = 0; c < 4 && d0 + c < D; ++c) store_dev1(racc, base + 4u * (d0 + c), o[c]);
    }
    if (d0 == 0) store_dev2(rml, row * 8u, f2v_t{wm[j], wl[j]});
  }

  if (live == kGridLive) live = grid_live(a, seq_len_of(a, b));
  combine_tail(a, b, h, chunk, gn, live, vec, racc, rml, bq0);
}

// ---------------------------------------------------------------------------
// host-side planning
// ---------------------------------------------------------------------------
struct SplitPlan {
  int nsplit;
  int64_t split_len;
};

// Workgroups of `kernel` (launched with `threads` threads) that run at once on
// the current device: CUs x maximum active blocks per CU, cached per device
// under `slot` (one slot per decode kernel).
enum ResidentSlot {
  kSlotGeneric = 0, kSlotMfmaPow2, kSlotMfma, kSlotPlain, kSlotG4, kSlotPrefill, kSlotFp16G4,
  kSlotCount
};
int64_t resident_workgroups(const void *kernel, int threads, int slot);
int64_t mfma_max_resident();     // max over the MFMA-file kernels
int64_t decode_max_resident();   // max over every decode kernel

// Tokens per split forced by the environment variable CQ_DECODE_SPLIT_TOKENS
// (a positive multiple of kSplitGranule, read once per process; 0 when unset
// or invalid).  A tuning knob for split-count sweeps: every grid plan then uses
// splits of that length, and uniform batches keep the grid plan.
int64_t split_tokens_override();

// Splits of kSplitGranule-multiple length sized so that the whole grid
// (groups workgroups per split) is resident at once: one generation of
// workgroups, no tail of late starters.  At most kMaxSplits.
inline SplitPlan plan_splits(int64_t groups, int64_t max_T, int64_t target) {
  SplitPlan p;
  if (groups < 1) groups = 1;
  if (target < 1) target = 1;
  int64_t ns = max((int64_t)1, target / groups);
  if (max_T <= 0) max_T = 1;
  int64_t len = (max_T + ns - 1) / ns;
  len = (len + kSplitGranule - 1) / kSplitGranule * kSplitGranule;
  if (const int64_t forced = split_tokens_override()) len = forced;
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

// Workspace layout: a fixed region first, which the kernels return to zero
// after every call: 64 KiB of split tickets (one uint32 per (sequence, kv
// head, q-head chunk)), 192 KiB of split-ready flags (one uint32 per
// (sequence, kv head, split) of the GQA-4 kernel) and 1.5 MiB of fold records
// (the GQA-4 grid plan's split partials, zero until written); then the split
// partials of the other plans, whose size varies with the split count.
// Keeping the zero region at a fixed place means calls of different shapes
// (and the prefill) sharing one workspace never see each other's partials as
// counters, flags or records.
constexpr size_t kCounterBytes = 64 << 10;
constexpr size_t kFlagBytes = 192 << 10;
// Fold record: one (split, head, 8 dims) unit of a split partial, 12 words:
// m, l, 2 unused, then the 8 unnormalised outputs, each stored as its bit
// pattern + 1 so that a zero word means "not written yet".
constexpr int kRecWords = 12;
constexpr int kRecUnits = 64;  // 4 heads x 16 groups of 8 dims per (sequence, kv head, split)
constexpr int64_t kMaxRecSplits = 512;  // (sequence, kv head, split) triples
constexpr size_t kRecBytes = (size_t)kMaxRecSplits * kRecUnits * kRecWords * sizeof(uint32_t);
constexpr size_t kCounterRegion = kCounterBytes + kFlagBytes + kRecBytes;
constexpr int64_t kMaxCounters = kCounterBytes / sizeof(uint32_t);
// The last 256 bytes of the flag area hold the workspace's sticky status
// word: a split wait that ran out of poll rounds sets kStatusFoldTimeout
// there (its fold went ahead without the missing partials, and a late split
// may then have left its record or flag set in the zero region).
// cq_decode_status reads it and, when set, clears the whole zero region.
constexpr size_t kStatusOffset = kCounterBytes + kFlagBytes - 256;
constexpr int64_t kMaxFlags = (kFlagBytes - 256) / sizeof(uint32_t);
constexpr uint32_t kStatusFoldTimeout = 1u;
// Poll rounds of a split wait unless a test lowers them (cq_set_fold_poll_bound).
constexpr int kDefaultPollRounds = 1 << 20;
int current_poll_rounds();

inline size_t round256(size_t x) { return (x + 255) / 256 * 256; }

inline size_t workspace_bytes_for(int B, int nq, int D, int nsplit) {
  const size_t ml = (size_t)B * nq * nsplit * 2 * sizeof(float);
  const size_t acc = (size_t)B * nq * nsplit * D * sizeof(float);
  return kCounterRegion + round256(ml) + round256(acc);
}

inline void carve_workspace(DecodeArgs &a, void *ws) {
  char *p = (char *)ws;
  a.status = (uint32_t *)(p + kStatusOffset);
  a.poll_rounds = current_poll_rounds();
  a.counters = (uint32_t *)p;
  a.flags = (int64_t)a.B * a.H * a.nsplit <= kMaxFlags ? (uint32_t *)(p + kCounterBytes) : nullptr;
  a.recs = nullptr;  // the GQA-4 grid launcher opts in (records_of)
  p += kCounterRegion;
  const size_t ml = (size_t)a.B * a.nq * a.nsplit * 2 * sizeof(float);
  a.part_ml = (float *)p;
  p += round256(ml);
  a.part_acc = (float *)p;
}

// The fold-record region of a carved workspace.
inline uint32_t *records_of(void *ws) {
  return (uint32_t *)((char *)ws + kCounterBytes + kFlagBytes);
}

// Common launch preparation: split plan and workspace.  chunk_heads = q heads
// per workgroup of the kernel being launched; resident = its resident
// workgroup capacity.  The plan never has more splits than the one
// cq_decode_workspace_size sizes for (fewer groups per split there, and the
// largest capacity of any decode kernel).
// Workspace for a.nsplit partial slots per (sequence, q head) (none needed
// for one).
inline int setup_workspace(DecodeArgs &a, void *workspace, size_t ws_bytes) {
  if (a.nsplit > 1) {
    if ((int64_t)a.B * a.H * a.n_chunks > kMaxCounters) return CQ_ERR_UNSUPPORTED;
    // the split partials are addressed with 32-bit byte offsets
    if ((int64_t)a.B * a.nq * a.nsplit * a.D * 4 >= ((int64_t)1 << 31)) return CQ_ERR_UNSUPPORTED;
    if (!workspace) return CQ_ERR_WORKSPACE;
    if ((uintptr_t)workspace & 255) return CQ_ERR_ALIGN;
    if (ws_bytes < workspace_bytes_for(a.B, a.nq, a.D, a.nsplit)) return CQ_ERR_WORKSPACE;
    carve_workspace(a, workspace);
  } else {
    a.part_ml = a.part_acc = nullptr;
    a.counters = a.flags = a.recs = a.status = nullptr;
    a.poll_rounds = 0;
  }
  return CQ_OK;
}

// Grid-plan launch preparation: split plan and workspace.
inline int prepare_launch(DecodeArgs &a, int chunk_heads, int64_t resident, void *workspace,
                          size_t ws_bytes) {
  a.chunk_heads = chunk_heads;
  a.n_chunks = (a.G + chunk_heads - 1) / chunk_heads;
  const SplitPlan p = plan_splits((int64_t)a.B * a.H * a.n_chunks, a.max_T, resident);
  a.nsplit = p.nsplit;
  a.split_len = p.split_len;
  return setup_workspace(a, workspace, ws_bytes);
}

// Balanced-plan partial slots per sequence for P workgroups per column: a
// sequence spans at most min(P, units of the length bound) workgroups.
inline int64_t balanced_slots(int64_t P, int64_t max_T) {
  const int64_t n = units_of(max_T);
  return P < n ? P : n;
}

int launch_decode_mfma(DecodeArgs &a, void *workspace, size_t ws_bytes, hipStream_t stream);
bool mfma_supported(const DecodeArgs &a);
// GQA groups of at most 4 q heads (cq_decode_g4.hip): the shape conditions
// alone, and together with mfma_supported's
bool g4_shape(const DecodeArgs &a);
bool g4_supported(const DecodeArgs &a);
int64_t g4_resident();
int launch_decode_g4(DecodeArgs &a, void *workspace, size_t ws_bytes, hipStream_t stream);
// the uncompressed fp16 baseline at head_dim 128, GQA <= 4, fp16 queries
bool fp16_g4_supported(const DecodeArgs &a);
int64_t fp16_g4_resident();
int launch_decode_fp16_g4(DecodeArgs &a, void *workspace, size_t ws_bytes, hipStream_t stream);

}  // namespace cq
