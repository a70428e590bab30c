// cgdr_fwd_h_k32.hip -- the FwdH kernel instantiations for key dimension 32 (see
// cgdr_fwd_h_dispatch.h; one translation unit per key dimension keeps the build parallel).
#include "cgdr_fwd_h_dispatch.h"

template hipError_t cgdr_fwd::launch_kd<32>(const cgdr::FwdHParams&, const cgdr_fwd::Plan&, hipStream_t);
