// cgdr_fwd_h_k256.hip -- the FwdH kernel instantiations for key dimension 256 (see
// cgdr_fwd_h_dispatch.h; one translation unit per key dimension keeps the build parallel).
#include "cgdr_fwd_h_dispatch.h"

template hipError_t cgdr_fwd::launch_kd<256>(const cgdr::FwdHParams&, const cgdr_fwd::Plan&, hipStream_t);
