// cgdr_host.h -- host-side helpers shared by the operators of libcgdr_fwd_h: the
// per-thread error message behind cgdr_last_error() (the role of OP_LOGE in the
// reference's host code).
#pragma once

#include <atomic>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>

#include <hip/hip_runtime.h>

#include "../../include/cgdr_fwd_h.h"

namespace cgdr_host {

inline thread_local char last_error[512] = "";

inline cgdr_status fail(cgdr_status st, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(last_error, sizeof(last_error), fmt, ap);
  va_end(ap);
  return st;
}

// XCDs of the calling thread's current device, which the hardware deals workgroups to
// round-robin (8 on MI355X, the figure used when no device answers).  Queried once per device
// and kept: the count cannot change while the process runs.
inline int device_xcds() {
  static std::atomic<int> cache[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) {
    (void)hipGetLastError();
    return 8;
  }
  const bool cached = dev >= 0 && dev < 64;
  if (cached) {
    const int c = cache[dev].load(std::memory_order_relaxed);
    if (c > 0) return c;
  }
  int v = 0;
  const bool ok = hipDeviceGetAttribute(&v, hipDeviceAttributeNumberOfXccs, dev) == hipSuccess && v > 0;
  (void)hipGetLastError();
  if (!ok) return 8;
  if (cached) cache[dev].store(v, std::memory_order_relaxed);
  return v;
}

}  // namespace cgdr_host
