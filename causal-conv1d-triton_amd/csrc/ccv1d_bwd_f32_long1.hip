// Instantiations of the vectorised bwd kernels for x of type float (widths 17..24, one channel per
// lane, with and without silu and seq_idx).
#define CCV1D_DEFINE_FAST_LAUNCHERS
#include "ccv1d_launch.h"

namespace ccv1d {
template hipError_t launch_bwd_fast_long1_t<float>(const BwdParams& p, hipStream_t s);
}  // namespace ccv1d
