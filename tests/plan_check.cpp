// Host-side check of the decode kernels' balanced token partition
// (chronoquant_mlx_amd/csrc/cq_plan.h): walks every workgroup's range the
// way the kernels do and checks that every token of every sequence is
// processed exactly once, that each sequence's live segments use partial
// slots 0 .. live-1 once each and agree on live, that a one-segment sequence
// is covered whole, and that slots stay inside the workspace's row capacity.
// Built and run by tests/test_plan.py; prints "ok <cases>" or the first
// failing case.
#include <stdio.h>
#include <stdlib.h>

#include <vector>

#include "../chronoquant_mlx_amd/csrc/cq_plan.h"

using namespace cq;

static uint64_t rng = 0x9e3779b97f4a7c15ull;
static uint64_t next() {
  rng ^= rng << 13;
  rng ^= rng >> 7;
  rng ^= rng << 17;
  return rng;
}

static int fail(const char *what, int B, int64_t P, int mode, int b) {
  printf("FAIL %s B=%d P=%lld mode=%d b=%d\n", what, B, (long long)P, mode, b);
  return 1;
}

// mode 0: unit table from the lengths; mode 1: uniform units from max_T
static int check(const std::vector<int64_t> &T, int64_t max_T, int64_t P_grid, int mode) {
  const int B = (int)T.size();
  std::vector<int32_t> start(B + 1, 0);
  for (int b = 0; b < B; ++b) start[b + 1] = start[b] + (int32_t)units_of(T[b]);
  UnitSpace us;
  us.start = mode == 0 ? start.data() : nullptr;
  us.n = units_of(max_T);
  us.B = B;
  const int64_t U = us.total();
  const int64_t P = P_grid < U ? P_grid : U;  // the kernels' P_eff
  const int64_t cap = (P_grid < units_of(max_T)) ? P_grid : units_of(max_T);
  const bool single = mode == 1 && uniform_single_segment(B, us.n, P_grid);
  std::vector<std::vector<int>> cover(B);
  for (int b = 0; b < B; ++b) cover[b].assign((size_t)T[b], 0);
  std::vector<std::vector<int>> slots(B);
  std::vector<int> live(B, -1), nseg(B, 0);
  for (int64_t p = 0; p < P; ++p) {
    const int64_t u0 = unit_begin(p, U, P), u1 = unit_begin(p + 1, U, P);
    if (u1 <= u0) return fail("empty workgroup", B, P_grid, mode, -1);
    int64_t u = u0;
    int b = us.seq_of(u0);
    int segs = 0;
    while (u < u1) {
      if (single && ++segs > 1) return fail("single-segment claim", B, P_grid, mode, b);
      if (b < 0 || b >= B) return fail("sequence out of range", B, P_grid, mode, b);
      if (us.S(b) > u || us.S(b + 1) <= u) return fail("seq_of", B, P_grid, mode, b);
      Segment s;
      const int64_t nu = segment_at(us, p, P, u, b, T[b], s);
      if (nu <= u) return fail("no progress", B, P_grid, mode, b);
      if (s.live > 0) {
        if (s.t0 < 0 || s.t1 < s.t0 || s.t1 > T[b]) return fail("token range", B, P_grid, mode, b);
        for (int64_t t = s.t0; t < s.t1; ++t) cover[b][(size_t)t]++;
        if (live[b] >= 0 && live[b] != s.live) return fail("live disagrees", B, P_grid, mode, b);
        live[b] = s.live;
        if (s.slot < 0 || s.slot >= s.live) return fail("slot range", B, P_grid, mode, b);
        if (s.live > 1 && s.slot >= cap) return fail("slot capacity", B, P_grid, mode, b);
        slots[b].push_back(s.slot);
        nseg[b]++;
        if (s.live == 1 && (s.t0 != 0 || s.t1 != T[b])) return fail("lone segment", B, P_grid, mode, b);
      } else if (s.t0 < T[b]) {
        return fail("dropped tokens", B, P_grid, mode, b);
      }
      u = nu;
      ++b;
    }
  }
  for (int b = 0; b < B; ++b) {
    for (int64_t t = 0; t < T[b]; ++t)
      if (cover[b][(size_t)t] != 1) return fail("coverage", B, P_grid, mode, b);
    if (live[b] < 1) return fail("no output", B, P_grid, mode, b);
    if (nseg[b] != live[b]) return fail("segment count", B, P_grid, mode, b);
    std::vector<int> seen(live[b], 0);
    for (int s : slots[b]) {
      if (seen[s]) return fail("slot twice", B, P_grid, mode, b);
      seen[s] = 1;
    }
  }
  return 0;
}

int main() {
  int cases = 0;
  // the benchmark shapes: c1, c2, and 32 ragged sequences of 1K..32K
  {
    if (check({16384}, 16384, 32, 1)) return 1;
    if (check(std::vector<int64_t>(8, 32768), 32768, 32, 1)) return 1;
    std::vector<int64_t> T;
    for (int b = 0; b < 32; ++b) T.push_back(1024 + (int64_t)(next() % 31745));
    for (int mode = 0; mode < 2; ++mode)
      if (check(T, 32768, 32, mode)) return 1;
    cases += 4;
  }
  for (int it = 0; it < 6000; ++it) {
    const int B = 1 + (int)(next() % (it % 4 == 0 ? 200 : 12));
    const int64_t max_T = (int64_t)(next() % (it % 3 == 0 ? 40000 : 3000));
    std::vector<int64_t> T(B);
    const int kind = (int)(next() % 4);
    for (int b = 0; b < B; ++b) {
      if (kind == 0) T[b] = max_T;                               // uniform
      else if (kind == 1) T[b] = max_T ? (int64_t)(next() % (max_T + 1)) : 0;  // ragged
      else if (kind == 2) T[b] = (next() % 3 == 0) ? 0 : max_T;  // empty sequences
      else T[b] = (int64_t)(next() % 4) * kUnit + (int64_t)(next() % 3) - 1;  // unit edges
      if (T[b] < 0) T[b] = 0;
      if (T[b] > max_T) T[b] = max_T;
    }
    const int64_t P = 1 + (int64_t)(next() % 300);
    for (int mode = 0; mode < 2; ++mode) {
      if (check(T, max_T, P, mode)) return 1;
      ++cases;
    }
  }
  printf("ok %d\n", cases);
  return 0;
}
