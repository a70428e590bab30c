// cgdr_schedule.h -- the load wave's wait rule and the packed-batch dispatch order, in plain
// C++ so host tests can check them.
//
// The load wave keeps D chunks of loads in flight (D = pipeline stages - 1).  At loop
// iteration c it first issues chunk c+D, then waits for chunk c+1 with s_waitcnt vmcnt(N),
// which returns once at most N of its VMEM instructions are outstanding; loads complete in
// issue order.  The instructions of chunk j form one group.  A group is full -- exactly
// PER_CHUNK instructions -- for every chunk but the last of the sequence, which may be partial
// (DMA instructions with no valid row are skipped), so it must never be among the groups a
// non-zero N leaves outstanding.
#pragma once

#include <stdint.h>

namespace cgdr {
namespace sched {

// Chunk groups issued after chunk c+1 that may stay outstanding when waiting for it at loop
// iteration c (after issuing chunk c+D), or 0 (wait for everything).  Outstanding after the
// wait point are groups c+2 .. min(c+D, NC-1); they are all full iff c+D < NC-1.
constexpr int loop_allowance(int c, int D, int NC) { return (D >= 2 && c + D < NC - 1) ? D - 1 : 0; }

// Same for the prologue's wait for chunk 0 with chunks 0 .. D-1 issued: groups 1 .. D-1 stay
// outstanding, all full iff D-1 < NC-1.
constexpr int prologue_allowance(int D, int NC) { return (D >= 2 && D < NC) ? D - 1 : 0; }

// Dispatch order of a packed variable-length batch (cu_seqlens given, H % nx == 0 for nx XCDs,
// so that n_tasks = N * H * nv is a multiple of nx and each XCD's range of dispatch indices
// holds q = n_tasks / nx of them).  Dispatch index d is read as (XCD block x, sequence rank r,
// head within the block, V-tile): block x gets heads [x * H/nx, (x+1) * H/nx) of every
// sequence, and within a block the rank varies slowest, so the longest sequences are
// dispatched first.
struct VarlenSlot {
  int rank, head, vtile;
};
constexpr VarlenSlot varlen_slot(int d, int n_tasks, int H, int nv, int nx) {
  const int hx = H / nx, q = n_tasks / nx;
  const int x = d / q, l = d - x * q;
  const int gi = l / nv;
  return VarlenSlot{gi / hx, x * hx + gi % hx, l % nv};
}

// Rank of sequence n among the N sequences of cu_seqlens by length: the number of sequences
// longer than it, or as long with a lower index.  The ranks of 0 .. N-1 are a permutation.
constexpr int seq_rank(const int64_t* cu, int N, int n) {
  const int64_t mine = cu[n + 1] - cu[n];
  int rank = 0;
  for (int m = 0; m < N; ++m) {
    const int64_t lm = cu[m + 1] - cu[m];
    rank += (lm > mine || (lm == mine && m < n)) ? 1 : 0;
  }
  return rank;
}

}  // namespace sched
}  // namespace cgdr
