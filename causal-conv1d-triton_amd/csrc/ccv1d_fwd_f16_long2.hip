// Instantiations of the vectorised fwd kernels for x of type _Float16 (widths 25..32, one channel per
// lane, with and without silu and seq_idx).
#define CCV1D_DEFINE_FAST_LAUNCHERS
#include "ccv1d_launch.h"

namespace ccv1d {
template hipError_t launch_fwd_fast_long2_t<_Float16>(const FwdParams& p, hipStream_t s);
}  // namespace ccv1d
