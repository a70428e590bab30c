// cgdr_host.h -- host-side helpers shared by the operators of libcgdr_fwd_h: the
// per-thread error message behind cgdr_last_error() (the role of OP_LOGE in the
// reference's host code) and environment overrides used by tests and benchmarks.
#pragma once

#include <cstdarg>
#include <cstdio>
#include <cstdlib>

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

inline int env_int(const char* name, int dflt) {
  const char* s = getenv(name);
  if (s == nullptr || *s == 0) return dflt;
  return atoi(s);
}

}  // namespace cgdr_host
