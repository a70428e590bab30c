// cgdr_schedule.h -- the load wave's wait rule, in plain C++ so host tests can check it.
//
// The load wave keeps D chunks of loads in flight (D = pipeline stages - 1).  Before the
// compute waves may use chunk c+1 it waits with s_waitcnt vmcnt(N), which returns once at
// most N of its VMEM instructions are outstanding; loads complete in issue order.  A full
// chunk issues exactly PER_CHUNK instructions.  The last chunk of a sequence may be partial
// and then issues fewer (DMA instructions with no valid row are skipped), so it must never be
// among the chunks a non-zero N leaves outstanding.
#pragma once

namespace cgdr {
namespace sched {

// Chunks issued after chunk c+1 that may stay outstanding when waiting for it at loop
// iteration c, or 0 (wait for everything).  In flight after the wait point are chunks
// c+2 .. min(c+D-1, NC-1); they are all full iff c+D-1 < NC-1.
constexpr int loop_allowance(int c, int D, int NC) { return (D >= 2 && c + D < NC) ? D - 2 : 0; }

// Same for the prologue's wait for chunk 0 with chunks 0 .. D-2 issued: chunks 1 .. D-2 stay
// outstanding, all full iff D-2 < NC-1.
constexpr int prologue_allowance(int D, int NC) { return (D >= 2 && D - 1 < NC) ? D - 2 : 0; }

}  // namespace sched
}  // namespace cgdr
