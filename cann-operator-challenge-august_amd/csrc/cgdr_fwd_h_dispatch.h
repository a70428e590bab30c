// cgdr_fwd_h_dispatch.h -- launch plan of the FwdH operator and the kernel dispatch for one key
// dimension.  The kernel instantiations of each key dimension live in a translation unit of
// their own (cgdr_fwd_h_k32.hip ... cgdr_fwd_h_k256.hip, one explicit instantiation of
// launch_kd each), so the library builds in parallel; cgdr_fwd_h.hip holds the C ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

#include "cgdr_kernels.h"

namespace cgdr_fwd {

struct Plan {
  int kernel;        // 0 bf16 pipeline, 1 fp32, 2 bf16 with the contest numerics (two passes)
  int helpers;       // bf16: one L2-prefetch workgroup per task
  int ncw;           // 16-column blocks (Vt = 16 * ncw)
  int rs;            // compute waves per 16-column block (bf16: 2 = state rows split; fp32: 1, 2, 4)
  int nlw;           // load waves (bf16 pipeline)
  int stages;        // LDS ring depth (bf16 pipeline)
  int threads;
  int64_t tasks;
  int cus;           // compute units and XCDs the plan was made for
  int xcds;
};

template <int KD, int NCW, int NLW, int STAGES, int NUM, int RS>
hipError_t launch_bf16(const cgdr::FwdHParams& p, int64_t tasks, hipStream_t stream) {
  using L = cgdr::Bf16Layout<KD, NCW, NLW, STAGES, RS>;
  const unsigned grid = (unsigned)(p.helpers ? 2 * tasks : tasks);
  hipLaunchKernelGGL((cgdr::cgdr_fwd_h_bf16_kernel<KD, NCW, NLW, STAGES, NUM, RS>), dim3(grid),
                     dim3(L::THREADS), 0, stream, p);
  return hipGetLastError();
}

template <int KD, int NCW, int RSF = 1>
hipError_t launch_f32(const cgdr::FwdHParams& p, int64_t tasks, hipStream_t stream) {
  using L = cgdr::F32Layout<KD, NCW, RSF>;
  hipLaunchKernelGGL((cgdr::cgdr_fwd_h_f32_kernel<KD, NCW, RSF>), dim3((unsigned)tasks), dim3(L::THREADS), 0, stream,
                     p);
  return hipGetLastError();
}

// fp32: the row split RSF the plan picked (instantiated where it fits, see f32_config_ok)
template <int KD, int NCW>
hipError_t dispatch_f32(const cgdr::FwdHParams& p, const Plan& pl, hipStream_t s) {
  if constexpr (cgdr::f32_config_ok<KD, NCW, 4>())
    if (pl.rs == 4) return launch_f32<KD, NCW, 4>(p, pl.tasks, s);
  if constexpr (cgdr::f32_config_ok<KD, NCW, 2>())
    if (pl.rs == 2) return launch_f32<KD, NCW, 2>(p, pl.tasks, s);
  return launch_f32<KD, NCW, 1>(p, pl.tasks, s);
}

// NUM: the kernel's numerics mode (0 default, 1 contest fast pass, 2 contest full pass).
// Configurations that do not fit (LDS, vmcnt range, waves) are not instantiated; the plan never
// selects them.
template <int KD, int NCW, int NLW, int NUM, int RS>
hipError_t dispatch_bf16_stages(const cgdr::FwdHParams& p, const Plan& pl, hipStream_t s) {
  if constexpr (cgdr::bf16_config_ok<KD, NCW, NLW, 4, RS>())
    if (pl.stages == 4) return launch_bf16<KD, NCW, NLW, 4, NUM, RS>(p, pl.tasks, s);
  if constexpr (cgdr::bf16_config_ok<KD, NCW, NLW, 3, RS>())
    if (pl.stages == 3) return launch_bf16<KD, NCW, NLW, 3, NUM, RS>(p, pl.tasks, s);
  if constexpr (cgdr::bf16_config_ok<KD, NCW, NLW, 2, RS>())
    return launch_bf16<KD, NCW, NLW, 2, NUM, RS>(p, pl.tasks, s);
  return hipErrorInvalidConfiguration;
}

template <int KD, int NCW, int NUM, int RS>
hipError_t dispatch_bf16_nlw(const cgdr::FwdHParams& p, const Plan& pl, hipStream_t s) {
  if (pl.nlw == 1) return dispatch_bf16_stages<KD, NCW, 1, NUM, RS>(p, pl, s);
  if constexpr (NUM == 0)
    if (pl.nlw == 4) return dispatch_bf16_stages<KD, NCW, 4, NUM, RS>(p, pl, s);
  return dispatch_bf16_stages<KD, NCW, 2, NUM, RS>(p, pl, s);
}

template <int KD, int NUM>
hipError_t dispatch_bf16(const cgdr::FwdHParams& p, const Plan& pl, hipStream_t s) {
  if constexpr (KD == 256) {
    return dispatch_bf16_nlw<KD, 1, NUM, 1>(p, pl, s);
  } else {
    if constexpr (KD >= 64) {
      if (pl.rs == 2) {
        if (pl.ncw == 2) return dispatch_bf16_nlw<KD, 2, NUM, 2>(p, pl, s);
        return dispatch_bf16_nlw<KD, 1, NUM, 2>(p, pl, s);
      }
    }
    if (pl.ncw == 2) return dispatch_bf16_nlw<KD, 2, NUM, 1>(p, pl, s);
    if (pl.ncw == 4) return dispatch_bf16_nlw<KD, 4, NUM, 1>(p, pl, s);
    return dispatch_bf16_nlw<KD, 1, NUM, 1>(p, pl, s);
  }
}

// Contest numerics: the fast pass (plain fp16 roundings) flags every (sequence, head) where a
// saturating cast or nan_to_num could have changed a value; the full pass then recomputes just
// those heads with the casts (its workgroups for unflagged heads return at once), without
// helper workgroups, whose progress counters the fast pass has used up.
template <int KD>
hipError_t dispatch_contest(const cgdr::FwdHParams& p, const Plan& pl, hipStream_t s) {
  hipError_t e = dispatch_bf16<KD, 1>(p, pl, s);
  if (e != hipSuccess) return e;
  cgdr::FwdHParams q = p;
  q.helpers = 0;
  q.progress = nullptr;
  return dispatch_bf16<KD, 2>(q, pl, s);
}

// The kernels of a plan for key dimension KD (explicitly instantiated once per KD).
template <int KD>
hipError_t launch_kd(const cgdr::FwdHParams& p, const Plan& pl, hipStream_t s) {
  if (pl.kernel == 0) return dispatch_bf16<KD, 0>(p, pl, s);
  if (pl.kernel == 2) return dispatch_contest<KD>(p, pl, s);
  if (pl.ncw == 2) return dispatch_f32<KD, 2>(p, pl, s);
  if (pl.ncw == 4) return dispatch_f32<KD, 4>(p, pl, s);
  return dispatch_f32<KD, 1>(p, pl, s);
}

extern template hipError_t launch_kd<32>(const cgdr::FwdHParams&, const Plan&, hipStream_t);
extern template hipError_t launch_kd<64>(const cgdr::FwdHParams&, const Plan&, hipStream_t);
extern template hipError_t launch_kd<128>(const cgdr::FwdHParams&, const Plan&, hipStream_t);
extern template hipError_t launch_kd<256>(const cgdr::FwdHParams&, const Plan&, hipStream_t);

}  // namespace cgdr_fwd
