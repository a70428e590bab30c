// cgdr_fwd_h_k64.hip -- the FwdH kernel instantiations for key dimension 64 (see
// cgdr_fwd_h_dispatch.h; one translation unit per key dimension keeps the build parallel).
#include "cgdr_fwd_h_dispatch.h"

template hipError_t cgdr_fwd::launch_kd<64>(const cgdr::FwdHParams&, const cgdr_fwd::Plan&, hipStream_t);
