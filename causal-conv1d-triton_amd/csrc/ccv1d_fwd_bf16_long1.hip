// Instantiations of the vectorised fwd kernels for x of type __bf16 (widths 17..24, one channel per
// lane, with and without silu and seq_idx).
#define CCV1D_DEFINE_FAST_LAUNCHERS
#include "ccv1d_launch.h"

namespace ccv1d {
template hipError_t launch_fwd_fast_long1_t<__bf16>(const FwdParams& p, hipStream_t s);
}  // namespace ccv1d
