// Launchers of the scalar (any width / any alignment) kernels, the partial-sum reduction and the
// fill kernel.
#include <atomic>

#include "ccv1d_generic.h"
#include "ccv1d_launch.h"

namespace ccv1d {

static_assert(kMaxGenericW <= kGenericRingW, "the ring backward covers every generic width");
static_assert(generic_ring_bytes(kGenericRingW, 4) <= 160 * 1024, "LDS of one gfx950 CU");

// Dynamic LDS above the default 64 KiB per workgroup must be allowed per kernel first. Each ring
// kernel is allowed the most any width takes (generic_ring_bytes(kGenericRingW, ...), at most the
// 160 KiB of a gfx950 CU) once per device, on its first launch there that needs more than 64 KiB:
// later launches, including those recorded into a captured graph, make no runtime call for it.
// `done` is the kernel's own set of devices (bit d for device d < 64; others set it every launch).
static hipError_t allow_lds(const void* kernel, size_t bytes, size_t max_bytes,
                            std::atomic<uint64_t>& done) {
  if (bytes <= 65536) return hipSuccess;
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  const uint64_t bit = dev < 64 ? uint64_t(1) << dev : 0;
  if (bit && (done.load(std::memory_order_acquire) & bit)) return hipSuccess;
  e = hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize, (int)max_bytes);
  if (e == hipSuccess && bit) done.fetch_or(bit, std::memory_order_acq_rel);
  return e;
}

template <typename TX>
hipError_t launch_fwd_generic_t(const FwdParams& p, hipStream_t s) {
  const dim3 grid((unsigned)((int64_t)p.B * p.tl.nT), (unsigned)((p.D + 63) / 64));
  if (p.W <= kGenericRingW) {
    static std::atomic<uint64_t> lds_allowed{0};
    const void* k = reinterpret_cast<const void*>(&fwd_generic_ring_kernel<TX>);
    const size_t shmem = generic_ring_bytes(p.W, 2);
    const hipError_t e = allow_lds(k, shmem, generic_ring_bytes(kGenericRingW, 2), lds_allowed);
    if (e != hipSuccess) return e;
    return launch(k, grid, dim3(64), shmem, s, &p);
  }
  return launch(reinterpret_cast<const void*>(&fwd_generic_kernel<TX>), grid, dim3(64), 0, s, &p);
}

// Widths up to kMaxGenericW (<= kGenericRingW); wider ones take launch_bwd_wide_t.
template <typename TX>
hipError_t launch_bwd_generic_t(const BwdParams& p, hipStream_t s) {
  const dim3 grid((unsigned)((int64_t)p.B * p.tl.nT), (unsigned)((p.D + 63) / 64));
  static std::atomic<uint64_t> lds_allowed{0};
  const void* k = reinterpret_cast<const void*>(&bwd_generic_ring_kernel<TX>);
  const size_t shmem = generic_ring_bytes(p.W, 4);
  const hipError_t e = allow_lds(k, shmem, generic_ring_bytes(kGenericRingW, 4), lds_allowed);
  if (e != hipSuccess) return e;
  return launch(k, grid, dim3(64), shmem, s, &p);
}

template <typename TX>
hipError_t launch_bwd_wide_t(const BwdParams& p, float* G, hipStream_t s) {
  const dim3 grid((unsigned)((int64_t)p.B * p.tl.nT), (unsigned)((p.D + 63) / 64));
  BwdParams pc = p;
  void* args[] = {&pc, &G};
  hipError_t e = hipLaunchKernel(reinterpret_cast<const void*>(&bwd_g_kernel<TX>), grid, dim3(64),
                                 args, 0, s);
  if (e != hipSuccess) return e;
  return launch_args(reinterpret_cast<const void*>(&bwd_wide_kernel<TX>), grid, dim3(64), 0, s,
                     args);
}

template hipError_t launch_fwd_generic_t<float>(const FwdParams&, hipStream_t);
template hipError_t launch_fwd_generic_t<_Float16>(const FwdParams&, hipStream_t);
template hipError_t launch_fwd_generic_t<__bf16>(const FwdParams&, hipStream_t);
template hipError_t launch_fwd_generic_t<double>(const FwdParams&, hipStream_t);
template hipError_t launch_bwd_generic_t<float>(const BwdParams&, hipStream_t);
template hipError_t launch_bwd_generic_t<_Float16>(const BwdParams&, hipStream_t);
template hipError_t launch_bwd_generic_t<__bf16>(const BwdParams&, hipStream_t);
template hipError_t launch_bwd_generic_t<double>(const BwdParams&, hipStream_t);
template hipError_t launch_bwd_wide_t<float>(const BwdParams&, float*, hipStream_t);
template hipError_t launch_bwd_wide_t<_Float16>(const BwdParams&, float*, hipStream_t);
template hipError_t launch_bwd_wide_t<__bf16>(const BwdParams&, float*, hipStream_t);
template hipError_t launch_bwd_wide_t<double>(const BwdParams&, float*, hipStream_t);

hipError_t launch_reduce(const ReduceParams& p, hipStream_t s) {
  const int64_t n = (int64_t)(p.W + (p.has_bias ? 1 : 0)) * p.D;
  const dim3 grid((unsigned)((n + 63) / 64));
  return launch(reinterpret_cast<const void*>(&reduce_partials_kernel<kReduceNW>), grid,
                dim3(kReduceNW * 64), 0, s, &p);
}

hipError_t launch_fill(void* dst, int dst_dt, const void* src, int src_dt, int64_t n, hipStream_t s) {
  if (n <= 0) return hipSuccess;
  int64_t blocks = (n + 255) / 256;
  if (blocks > 4096) blocks = 4096;
  void* args[] = {&dst, &dst_dt, &src, &src_dt, &n};
  return hipLaunchKernel(reinterpret_cast<const void*>(&fill_kernel), dim3((unsigned)blocks), dim3(256),
                         args, 0, s);
}

}  // namespace ccv1d
