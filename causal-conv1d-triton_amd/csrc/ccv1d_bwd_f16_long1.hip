// Instantiations of the vectorised bwd kernels for x of type _Float16 (widths 17..24, one channel per
// lane, with and without silu and seq_idx).
#define CCV1D_DEFINE_FAST_LAUNCHERS
#include "ccv1d_launch.h"

namespace ccv1d {
template hipError_t launch_bwd_fast_long1_t<_Float16>(const BwdParams& p, hipStream_t s);
}  // namespace ccv1d
