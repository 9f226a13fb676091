// cq_plan.h — the balanced token partition of a decode batch over the
// workgroups of one (kv head, q-head chunk) column.
//
// Every sequence b is cut into units of kUnit tokens (one 64-token chunk per
// wave of an 8-wave workgroup).  The units of the batch are laid end to end,
// sequence b at [S_b, S_b + n_b), U units in all, and workgroup p of P takes
// units [floor(pU/P), floor((p+1)U/P)).  Every workgroup so gets the same
// number of tokens to within one unit, whatever the sequences' lengths.  A
// workgroup's range can end one sequence and start the next: each piece is a
// segment with its own partial slot, and the workgroups sharing a sequence
// combine their partials by log-sum-exp as the split-K combine does.
//
// n_b is either max(1, ceil(T_b / kUnit)) (the unit table, built from the
// per-sequence lengths; an empty sequence owns one unit so that it gets its
// zero output) or, for batches without per-sequence lengths or too many
// sequences for the table, the same n for every sequence, from the batch's
// length bound.  Units of sequence b past its end (only in the second form)
// are not processed and take no part in the combine.
//
// Plain C++ so that the host-side tests can check the enumeration.
#pragma once

#include <stdint.h>

#if defined(__HIPCC__)
#define CQ_HD __host__ __device__ __forceinline__
#else
#define CQ_HD inline
#endif

namespace cq {

constexpr int kUnit = 512;             // tokens per unit
constexpr int kMaxTableSeqs = 1024;    // sequences the unit table holds

CQ_HD int64_t units_of(int64_t T) {
  const int64_t n = (T + kUnit - 1) / kUnit;
  return n < 1 ? 1 : n;
}

// The workgroup whose range holds unit u (0 <= u < U): the largest p with
// floor(pU/P) <= u.
CQ_HD int64_t unit_owner(int64_t u, int64_t U, int64_t P) { return ((u + 1) * P - 1) / U; }

// First unit of workgroup p.
CQ_HD int64_t unit_begin(int64_t p, int64_t U, int64_t P) { return p * U / P; }

// One piece of a workgroup's range: tokens [t0, t1) of sequence b, written to
// partial slot `slot` of that sequence's `live` slots (live == 1: the whole
// sequence is in this segment and the workgroup writes the output itself).
struct Segment {
  int b;
  int slot, live;
  int64_t t0, t1;
};

// Layout of the unit space: the table (start[b] = S_b for b <= B, start[B] =
// U) or uniform n units per sequence.
struct UnitSpace {
  const int32_t *start;  // nullptr: uniform
  int64_t n;             // uniform: units per sequence
  int B;
  CQ_HD int64_t S(int b) const {
    if (!start) return (int64_t)b * n;
#if defined(__HIP_DEVICE_COMPILE__)
    // the table is in LDS and the same for every lane: keep the value scalar
    return (int64_t)__builtin_amdgcn_readfirstlane(start[b]);
#else
    return (int64_t)start[b];
#endif
  }
  CQ_HD int64_t total() const { return S(B); }
  // sequence holding unit u (0 <= u < U): the largest b with S_b <= u
  CQ_HD int seq_of(int64_t u) const {
    if (!start) return (int)(u / n);
    int lo = 0, hi = B - 1;
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (S(mid) <= u) lo = mid;
      else hi = mid - 1;
    }
    return lo;
  }
};

// The segment of workgroup p that starts at unit u (u inside p's range and
// inside sequence b = seq_of(u)); T = the sequence's length.  Returns the
// unit after the segment.  seg.live == 0: the segment lies past the
// sequence's end (nothing to do).
CQ_HD int64_t segment_at(const UnitSpace &us, int64_t p, int64_t P, int64_t u, int b, int64_t T,
                         Segment &seg) {
  const int64_t U = us.total();
  const int64_t u_end = unit_begin(p + 1, U, P);
  const int64_t S = us.S(b), E = us.S(b + 1);
  const int64_t ue = E < u_end ? E : u_end;
  // units of the sequence that hold tokens (the uniform form pads short ones)
  const int64_t e = units_of(T);
  const int64_t last = S + (e < E - S ? e : E - S) - 1;  // last unit with tokens
  const int64_t first_owner = unit_owner(S, U, P);
  seg.b = b;
  seg.t0 = (u - S) * kUnit;
  seg.t1 = (ue - S) * kUnit;
  if (seg.t1 > T) seg.t1 = T;
  if (u > last) {
    seg.live = 0;
    seg.slot = 0;
  } else {
    seg.live = (int)(unit_owner(last, U, P) - first_owner + 1);
    seg.slot = (int)(p - first_owner);
  }
  return ue;
}

// Uniform unit space (n units for each of B sequences) over P workgroups:
// true if every workgroup's range lies inside one sequence, so that each
// workgroup has exactly one segment.
CQ_HD bool uniform_single_segment(int64_t B, int64_t n, int64_t P) {
  const int64_t U = B * n;
  if (P > U) P = U;
  for (int64_t p = 0; p < P; ++p) {
    const int64_t u0 = unit_begin(p, U, P), u1 = unit_begin(p + 1, U, P);
    if (u0 / n != (u1 - 1) / n) return false;
  }
  return true;
}

}  // namespace cq
