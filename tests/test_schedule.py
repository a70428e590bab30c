"""CPU check of the load wave's vmcnt wait rule (csrc/cgdr_schedule.h), compiled with g++.

The C++ driver replays the load wave's issue/wait sequence (chunk c+D issued, then chunk c+1
awaited) for every prefetch depth D, sequence length (in chunks) and instruction count of a
partial last chunk, with loads completing in issue order as late as each s_waitcnt vmcnt(N)
allows, and a 63-deep counter.  At every wait it checks that the awaited chunk has fully
landed.  The same driver with the rule that ignores a shorter last group must report a
violation.
"""

import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "cann-operator-challenge-august_amd", "csrc")

DRIVER = r'''
#include <cstdio>
#include <deque>
#include "cgdr_schedule.h"
using namespace cgdr::sched;

// The rule without the last-group exception (steady allowance whenever chunk c+D was issued).
static int loop_allow_naive(int c, int D, int NC) { return (D >= 2 && c + D < NC) ? D - 1 : 0; }
static int pro_allow_naive(int D, int NC) { return (D >= 2 && D <= NC) ? D - 1 : 0; }

struct Sim {
  std::deque<int> q;     // chunk id of each outstanding instruction, oldest first
  int per, last_count, NC;
  bool ok = true;
  void issue(int j) {
    int n = (j == NC - 1) ? last_count : per;
    for (int i = 0; i < n; ++i) { if (q.size() == 63) q.pop_front(); q.push_back(j); }
  }
  void wait(int N) { while ((int)q.size() > N) q.pop_front(); }
  void check(int j) { for (int x : q) if (x == j) ok = false; }
};

static bool run(int D, int NC, int per, int last_count, bool naive) {
  Sim s; s.per = per; s.last_count = last_count; s.NC = NC;
  const int steady = (D - 1) * per;
  for (int j = 0; j < D && j < NC; ++j) s.issue(j);
  int a = naive ? pro_allow_naive(D, NC) : prologue_allowance(D, NC);
  s.wait(a > 0 ? steady : 0); s.check(0);
  for (int c = 0; c < NC; ++c) {
    if (c + D < NC) s.issue(c + D);
    if (c + 1 < NC) {
      a = naive ? loop_allow_naive(c, D, NC) : loop_allowance(c, D, NC);
      s.wait(a > 0 ? steady : 0); s.check(c + 1);
    }
  }
  return s.ok;
}

int main() {
  int bad_new = 0, bad_naive = 0, cases = 0;
  for (int D = 1; D <= 4; ++D)
    for (int per : {19, 35, 37, 41, 67})
      for (int NC = 1; NC <= 12; ++NC)
        for (int last = 1; last <= per; ++last) {
          if ((D - 1) * per > 63) continue;   // excluded by the kernel's static_assert
          ++cases;
          bad_new += !run(D, NC, per, last, false);
          bad_naive += !run(D, NC, per, last, true);
        }
  printf("%d %d %d\n", cases, bad_new, bad_naive);
  return 0;
}
'''


def test_wait_rule_lands_every_awaited_chunk(tmp_path):
    src = tmp_path / "sched.cpp"
    src.write_text(DRIVER)
    exe = tmp_path / "sched"
    subprocess.run(["g++", "-std=c++17", "-O1", "-Wall", "-Werror", "-I", CSRC, str(src), "-o", str(exe)], check=True)
    cases, bad_new, bad_naive = map(int, subprocess.run([str(exe)], capture_output=True, text=True,
                                                      check=True).stdout.split())
    assert cases > 1000
    assert bad_new == 0
    assert bad_naive > 0, "the simulation must catch the rule without the last-group exception"


ORDER_DRIVER = r'''
#include <cstdio>
#include <cstdint>
#include <random>
#include <vector>
#include "cgdr_schedule.h"
using namespace cgdr::sched;

// rank without the tie-break by index (a planted mistake: equal lengths share a rank)
static int rank_no_tiebreak(const int64_t* cu, int N, int n) {
  int r = 0;
  for (int m = 0; m < N; ++m) r += (cu[m + 1] - cu[m]) > (cu[n + 1] - cu[n]);
  return r;
}

// The kernel's order_task on the host: the lane whose sequence has rank r (N <= 64), else r.
static int order(const std::vector<int64_t>& cu, int N, int H, int nv, int nx, int d, bool naive) {
  const VarlenSlot s = varlen_slot(d, N * H * nv, H, nv, nx);
  int n = s.rank;
  if (N <= 64) {
    n = -1;
    for (int m = 0; m < N; ++m) {
      const int rk = naive ? rank_no_tiebreak(cu.data(), N, m) : seq_rank(cu.data(), N, m);
      if (rk == s.rank) { n = m; break; }
    }
    if (n < 0) n = s.rank;   // the kernel's fallback when no lane matches
  }
  return (n * H + s.head) * nv + s.vtile;
}

int main() {
  std::mt19937 rng(7);
  int cases = 0, bad = 0, naive_bad = 0;
  for (int nx : {8, 4, 2, 1})
  for (int N : {1, 2, 3, 5, 16, 17, 63, 64, 65, 100})
    for (int H : {8, 16, 32, 64})
      for (int nv : {1, 2, 4, 8})
        for (int trial = 0; trial < 3; ++trial) {
          std::vector<int64_t> cu(N + 1, 0);
          for (int i = 0; i < N; ++i) {
            // trial 0: many ties (lengths from a few values, zeros included); else U[0, 9000)
            const int64_t L = trial == 0 ? 64 * (int64_t)(rng() % 3) : (int64_t)(rng() % 9000);
            cu[i + 1] = cu[i] + L;
          }
          const int T = N * H * nv, q = T / nx, hx = H / nx;
          std::vector<int> seen(T, 0), seen_naive(T, 0);
          bool ok = true, ok_naive = true;
          for (int d = 0; d < T; ++d) {
            const int t = order(cu, N, H, nv, nx, d, false), tn = order(cu, N, H, nv, nx, d, true);
            if (t < 0 || t >= T || seen[t]++) ok = false;
            if (tn < 0 || tn >= T || seen_naive[tn]++) ok_naive = false;
            if (!ok) break;
            const int x = d / q, head = (t / nv) % H, n = t / nv / H;
            if (head / hx != x) ok = false;   // the block's own heads
            if (d % q > 0 && N <= 64) {       // within a block: lengths never increase
              const int tp = order(cu, N, H, nv, nx, d - 1, false), np = tp / nv / H;
              if (cu[np + 1] - cu[np] < cu[n + 1] - cu[n]) ok = false;
            }
          }
          // every block gets the same work: hx heads x nv tiles of every sequence
          std::vector<int64_t> work(nx, 0);
          for (int d = 0; ok && d < T; ++d) {
            const int n = order(cu, N, H, nv, nx, d, false) / nv / H;
            work[d / q] += cu[n + 1] - cu[n];
          }
          for (int x = 1; ok && x < nx; ++x) if (work[x] != work[0]) ok = false;
          ++cases;
          bad += !ok;
          naive_bad += !ok_naive;
        }
  printf("%d %d %d\n", cases, bad, naive_bad);
  return 0;
}
'''


def test_varlen_dispatch_order_is_balanced_permutation(tmp_path):
    """The packed-batch dispatch order (cgdr_schedule.h varlen_slot / seq_rank, with the
    kernel's lane search) is a permutation of the tasks for N up to 100 sequences (ties and
    empty sequences included) and 8, 4, 2 or 1 XCDs; XCD block x holds heads
    [x H/nx, (x+1) H/nx) of every sequence, so every block gets the same work; and within a
    block lengths never increase (N <= 64).
    The rank without its tie-break must fail the permutation check on tied lengths."""
    src = tmp_path / "order.cpp"
    src.write_text(ORDER_DRIVER)
    exe = tmp_path / "order"
    subprocess.run(["g++", "-std=c++17", "-O1", "-Wall", "-Werror", "-I", CSRC, str(src), "-o", str(exe)], check=True)
    cases, bad, naive_bad = map(int, subprocess.run([str(exe)], capture_output=True, text=True,
                                                    check=True).stdout.split())
    assert cases == 4 * 10 * 4 * 4 * 3
    assert bad == 0
    assert naive_bad > 0, "the check must catch ranks without the tie-break"
