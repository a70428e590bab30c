// cgdr_host.h -- host-side helpers shared by the operators of libcgdr_fwd_h: the
// per-thread error message behind cgdr_last_error() (the role of OP_LOGE in the
// reference's host code).
#pragma once

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
// round-robin (8 on MI355X, the figure used when no device answers).
inline int device_xcds() {
  int dev = 0, v = 0;
  int n = 8;
  if (hipGetDevice(&dev) == hipSuccess &&
      hipDeviceGetAttribute(&v, hipDeviceAttributeNumberOfXccs, dev) == hipSuccess && v > 0)
    n = v;
  (void)hipGetLastError();
  return n;
}

}  // namespace cgdr_host
