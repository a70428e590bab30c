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
