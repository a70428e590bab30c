// cgdr_schedule.h -- the load wave's wait rule, in plain C++ so host tests can check it.
//
// The load wave keeps D chunks of loads in flight (D = pipeline stages - 1).  At loop
// iteration c it first issues chunk c+D, then waits for chunk c+1 with s_waitcnt vmcnt(N),
// which returns once at most N of its VMEM instructions are outstanding; loads complete in
// issue order.  The instructions of chunk j form one group.  A group is full -- exactly
// PER_CHUNK instructions -- for every chunk but the last of the sequence, which may be partial
// (DMA instructions with no valid row are skipped), so it must never be among the groups a
// non-zero N leaves outstanding.
#pragma once

namespace cgdr {
namespace sched {

// Chunk groups issued after chunk c+1 that may stay outstanding when waiting for it at loop
// iteration c (after issuing chunk c+D), or 0 (wait for everything).  Outstanding after the
// wait point are groups c+2 .. min(c+D, NC-1); they are all full iff c+D < NC-1.
constexpr int loop_allowance(int c, int D, int NC) { return (D >= 2 && c + D < NC - 1) ? D - 1 : 0; }

// Same for the prologue's wait for chunk 0 with chunks 0 .. D-1 issued: groups 1 .. D-1 stay
// outstanding, all full iff D-1 < NC-1.
constexpr int prologue_allowance(int D, int NC) { return (D >= 2 && D < NC) ? D - 1 : 0; }

}  // namespace sched
}  // namespace cgdr
