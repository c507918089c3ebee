// Launch helpers: compile-time configuration of the kernels and the dispatch from runtime
// (width, activation, seq_idx, channels per lane) to template instantiations. Each pass, x dtype and
// width range has its instantiations in a translation unit of its own
// (ccv1d_{fwd,bwd}_<dtype>[_wide].hip), so they compile in parallel.
#pragma once

#include <hip/hip_ext.h>

#include "ccv1d_device.h"

namespace ccv1d {

// Shape of the vectorised kernels per x dtype: CPL channels per lane, NW waves per workgroup, R rows
// per pipelined batch, and the cache policy of the row loads and stores (RowBuf). Chosen by
// measuring whole training steps (forward then backward over rotating input sets, bf16,
// B=4 T=8192 D=1024 W=4) on MI355X, where each pass runs right after the other; a pass timed alone
// favours different choices, because each pass's policies decide what the other finds in the
// Infinity Cache. The forward keeps x cacheable, so that the backward that follows finds it in the
// Infinity Cache, and writes out through the L2 at device scope (sc1), which leaves little dirty
// data for the L2 write-back at the end of the kernel; the backward reads x and dout non-temporally
// (their last use) and stores dx non-temporally at device scope. 16-byte rows (fp32) keep the plain
// and non-temporal stores their global-store path supports.
//
// The forward's out stores are non-temporal instead (OST_STREAM, chosen by the host per call,
// FwdParams::out_nt) when no backward follows (inference) and the pass streams more than 64 MiB,
// or when x and out together exceed half the Infinity Cache, so that x would not stay resident
// for the backward anyway; such inference passes also load x non-temporally (FwdParams::x_nt;
// forward alone at B=4 T=8192 D=1024 over 512 MiB of rotating inputs 28.7 -> 27.6 us, neutral at
// T=32768). Measured on
// B=4 D=1024 W=4 bf16, the forward alone at T=8192 29.6 -> 23.3-24.7 us and the fwd+bwd step at
// T=32768 245-250 -> 227-231 us, while the T=8192 step, whose 64 MiB x stays cached, is 2.7-4 us
// faster with sc1 stores.
template <typename TX> struct FwdCfg {
  static constexpr int CPL = 4;
  // Small grids: 2 channels per lane, twice the waves (chosen by the host per shape).
  static constexpr int CPL_SMALL = 2;
  static constexpr int NW = 8;
  static constexpr int R = 4;
  static constexpr int XLD = kCachePlain;
  static constexpr int OST = sizeof(TX) == 2 ? kCacheSC1 : kCachePlain;
  static constexpr int OST_STREAM = kCacheNT;
  // Inference passes that stream (FwdParams::x_nt): x is read once, with no backward to find it.
  static constexpr int XLD_STREAM = kCacheNT;
};
template <typename TX> struct BwdCfg {
  static constexpr int CPL = 4;
  // Widths kBwdWideW..kBwdLongW-1 keep 2 channels per lane: 4 would need about 150-190 VGPRs (the
  // weights, the x and g windows and the dweight sums are all per channel), one workgroup per CU;
  // with 2 the kernel holds 4 waves per SIMD (B=4 T=16384 D=4096 W=7 with seq_idx: 657 -> 582 us
  // per step; at W=4 the benchmark shape is 2.5 us faster with 4 channels).
  static constexpr int CPL_WIDE = 2;
  static constexpr int NW = 8;
  static constexpr int R = 4;
  static constexpr int XLD = kCacheNT;
  static constexpr int YLD = kCacheNT;
  static constexpr int DXST = sizeof(TX) == 2 ? kCacheSC1NT : kCacheNT;
  // dx rows that straddle 128-byte lines (BwdParams::dx_nt; widths below kUnitWideW): plain
  // non-temporal stores. Configuration 3 writing dx into the in_proj gradient (pitch 10576
  // channels), column-fastest order: 247 -> 233 us.
  static constexpr int DXST_STREAM = kCacheNT;
};
constexpr int kMaxFastW = 32;    // widths 2..kMaxFastW have register-window kernels
// The forward takes 2 channels per lane from width 7: with 4, widths 7 and 8 need 118-132 VGPRs
// (4 waves per SIMD at most), with 2 they need about 70 and the short-tile grids of mid-size shapes
// gain the most (forward alone at W=8: B=32 T=1024 D=2048 73.9 -> 54.3 us, B=4 T=1024 D=8192 37.7
// -> 31.2; fwd+bwd step at B=4 T=8192 D=1024: W=7 68.8 -> 67.6 us, W=8 71.4 -> 69.9). At widths 5
// and 6 the 4-channel forward was faster at B=4 T=8192 D=1024 (forward alone 28.4 against 29.7 us
// at W=5, 28.8 against 29.6 at W=6) and on large grids with 32-row tiles (B=8 T=4096 D=4096 W=6
// 98.9 against 105.0 us), so they keep 4 there (fwd_shape in ccv1d_api.hip still gives 16-bit x 2
// channels on the grids where 4 would take 16-row tiles).
constexpr int kFwdWideW = 7;     // first width whose forward always uses FwdCfg::CPL_SMALL
constexpr int kBwdWideW = 6;     // first width whose backward uses BwdCfg::CPL_WIDE
// One channel per lane (kCplLong) from width kFwdLongW in the forward and from kBwdLongW in the
// backward. From width 17 the weights, the windows and the dweight sums of W taps per channel fit
// the registers of 2 waves per SIMD only with one channel (backward at width 32: 187-189 VGPRs,
// no spills). The backward takes one channel from width 11 already: 80-112 VGPRs at widths 11-16
// (4-6 waves per SIMD, against 2 with two channels). Measured (bf16, B=4 T=8192 D=1024, bias +
// silu, fwd+bwd step, 2 against 1 channel in the backward): W=11 84.0 -> 80.7 us, W=12 86.0 ->
// 82.2, W=14 94.8 -> 90.5, W=16 103.1 -> 97.5; at W=9 and 10 one channel was 2.5 us slower. The
// forward alone with one channel: 0.3-0.7 us faster at widths 9-12, as much slower at 13-16,
// hence 2 channels up to 16.
constexpr int kFwdLongW = 17;
constexpr int kBwdLongW = 11;
constexpr int kCplLong = 1;
constexpr int kMaxGenericW = 128;  // LDS rings of the generic backward (x, g, weights, dweight
                                   // sums: 4 * W * 64 * 4 bytes + the rows' ids, 128.5 KiB at 128);
                                   // wider backwards keep g in the workspace (bwd_g/bwd_wide)
constexpr int kReduceNW = 16;    // waves per reduction workgroup
constexpr int kGenericL = 64;    // rows per tile of the generic kernels

// Timing events of the calling thread (ccv1d_time_main_kernel). `pending` holds a request for the
// thread's next entry-point call, which takes it; the call sets `armed` right before its main kernel
// and clears it after, and launch() gives an armed pair to that one launch.
struct KernelEvents {
  hipEvent_t start = nullptr, stop = nullptr;
  bool pending = false, armed = false;
};
inline KernelEvents& kernel_events() {
  static thread_local KernelEvents e;
  return e;
}

inline hipError_t launch_args(const void* kernel, dim3 grid, dim3 block, size_t shmem,
                              hipStream_t s, void** args) {
  KernelEvents& ev = kernel_events();
  if (ev.armed) {
    // HIP sets both events from the dispatch's own start and end timestamps.
    ev.armed = false;
    return hipExtLaunchKernel(kernel, grid, block, args, shmem, s, ev.start, ev.stop, 0);
  }
  return hipLaunchKernel(kernel, grid, block, args, shmem, s);
}

inline hipError_t launch(const void* kernel, dim3 grid, dim3 block, size_t shmem, hipStream_t s,
                         const void* params) {
  void* args[] = {const_cast<void*>(params)};
  return launch_args(kernel, grid, block, shmem, s, args);
}

// The vectorised kernels are instantiated in translation units of their own per pass, dtype and
// width range, so the build compiles them in parallel: widths 2..8 (ccv1d_{fwd,bwd}_<dtype>.hip),
// 9..16 (_wide.hip), 17..24 (_long1.hip) and 25..32 (_long2.hip). First widths of the last three:
constexpr int kUnitWideW = 9, kUnitLong1W = 17, kUnitLong2W = 25;
template <typename TX>
hipError_t launch_fwd_fast_narrow_t(const FwdParams& p, hipStream_t s);
template <typename TX>
hipError_t launch_fwd_fast_wide_t(const FwdParams& p, hipStream_t s);
template <typename TX>
hipError_t launch_fwd_fast_long1_t(const FwdParams& p, hipStream_t s);
template <typename TX>
hipError_t launch_fwd_fast_long2_t(const FwdParams& p, hipStream_t s);
template <typename TX>
hipError_t launch_bwd_fast_narrow_t(const BwdParams& p, hipStream_t s);
template <typename TX>
hipError_t launch_bwd_fast_wide_t(const BwdParams& p, hipStream_t s);
template <typename TX>
hipError_t launch_bwd_fast_long1_t(const BwdParams& p, hipStream_t s);
template <typename TX>
hipError_t launch_bwd_fast_long2_t(const BwdParams& p, hipStream_t s);
template <typename TX>
inline hipError_t launch_fwd_fast_t(const FwdParams& p, hipStream_t s) {
  if (p.W < kUnitWideW) return launch_fwd_fast_narrow_t<TX>(p, s);
  if (p.W < kUnitLong1W) return launch_fwd_fast_wide_t<TX>(p, s);
  return p.W < kUnitLong2W ? launch_fwd_fast_long1_t<TX>(p, s) : launch_fwd_fast_long2_t<TX>(p, s);
}
template <typename TX>
inline hipError_t launch_bwd_fast_t(const BwdParams& p, hipStream_t s) {
  if (p.W < kUnitWideW) return launch_bwd_fast_narrow_t<TX>(p, s);
  if (p.W < kUnitLong1W) return launch_bwd_fast_wide_t<TX>(p, s);
  return p.W < kUnitLong2W ? launch_bwd_fast_long1_t<TX>(p, s) : launch_bwd_fast_long2_t<TX>(p, s);
}
template <typename TX>
hipError_t launch_fwd_generic_t(const FwdParams& p, hipStream_t s);
template <typename TX>
hipError_t launch_bwd_generic_t(const BwdParams& p, hipStream_t s);
// Backward above kMaxGenericW: g to the fp32 buffer G of (batch, seqlen, dim) floats, then dx and
// the partial rows from it (the second is the main kernel for ccv1d_time_main_kernel).
template <typename TX>
hipError_t launch_bwd_wide_t(const BwdParams& p, float* G, hipStream_t s);
hipError_t launch_reduce(const ReduceParams& p, hipStream_t s);
hipError_t launch_fill(void* dst, int dst_dt, const void* src, int src_dt, int64_t n, hipStream_t s);

}  // namespace ccv1d

#ifdef CCV1D_DEFINE_FAST_LAUNCHERS
#include "ccv1d_fast.h"

namespace ccv1d {

template <typename TX, int W, bool SILU, bool SEQ, int CPL, int XLD, int OST>
static hipError_t fwd_one_st(const FwdParams& p, hipStream_t s) {
  using C = FwdCfg<TX>;
  return launch(reinterpret_cast<const void*>(
                    &fwd_fast_kernel<TX, W, SILU, SEQ, CPL, C::NW, C::R, XLD, OST>),
                dim3(p.tl.nBlk), dim3(C::NW * 64), 0, s, &p);
}

// The cache policies the host chose for this call (FwdParams::out_nt, x_nt; x_nt implies out_nt).
template <typename TX, int W, bool SILU, bool SEQ, int CPL>
static hipError_t fwd_one(const FwdParams& p, hipStream_t s) {
  using C = FwdCfg<TX>;
  if (p.x_nt) return fwd_one_st<TX, W, SILU, SEQ, CPL, C::XLD_STREAM, C::OST_STREAM>(p, s);
  if (p.out_nt) return fwd_one_st<TX, W, SILU, SEQ, CPL, C::XLD, C::OST_STREAM>(p, s);
  return fwd_one_st<TX, W, SILU, SEQ, CPL, C::XLD, C::OST>(p, s);
}

// The channels per lane the host's tiling chose (Tiling::vec): CPL or CPL_SMALL below kFwdWideW,
// CPL_SMALL from it, kCplLong from kFwdLongW. Any other value is rejected.
template <typename TX, int W, bool SILU, bool SEQ>
static hipError_t fwd_vec(const FwdParams& p, hipStream_t s) {
  using C = FwdCfg<TX>;
  if constexpr (W >= kFwdLongW) {
    if (p.tl.vec == kCplLong) return fwd_one<TX, W, SILU, SEQ, kCplLong>(p, s);
  } else {
    if (p.tl.vec == C::CPL_SMALL) return fwd_one<TX, W, SILU, SEQ, C::CPL_SMALL>(p, s);
    if constexpr (W < kFwdWideW) {
      if (p.tl.vec == C::CPL) return fwd_one<TX, W, SILU, SEQ, C::CPL>(p, s);
    }
  }
  return hipErrorInvalidValue;
}

// The backward's batch depth: C::R rows where the register budget holds it, else 2 rows, which
// keeps the other instances from spilling. C::R fits at widths <= 4 with rows of at most 8 bytes
// (4 waves per SIMD), and with 2 channels of 16-bit x per lane (4-byte rows: 83-104 VGPRs at widths
// 5-8) except with seq_idx from width 5, whose kernel also holds the sequence ids. Measured (fwd+bwd
// step, bf16, R = 4 against 2): B=4 T=8192 D=1024 W=6 -1.2 %, W=7 -2.8 %, W=8 -2.5 %; B=8 T=4096
// D=5376 W=8 -0.4 %; with seq_idx (B=4 T=16384 D=4096 W=7) +1 %, hence 2 there. Width 5 with 4
// channels and 4 rows spills. With one channel per lane, width 20 takes 2 rows: 128 VGPRs, 4 waves
// per SIMD, against 134 and 3 waves with 4 rows (step B=4 T=8192 D=1024 133.5 -> 117.1 us, B=8
// T=4096 D=4096 489 -> 438); at the other widths from 17, 2 rows were 0-6 % slower (no change of
// occupancy, or none that paid: W=21 137.5 -> 144, W=24 147 -> 154).
template <typename TX, int W, bool SEQ, int CPL>
constexpr int bwd_rows() {
  using C = BwdCfg<TX>;
  if (CPL == 1 && W == 20) return 2;
  if (W <= 4 && CPL * (int)sizeof(TX) <= 8) return C::R;
  if (!SEQ && CPL * (int)sizeof(TX) <= 4) return C::R;
  return 2;
}

template <typename TX, int W, bool SILU, bool SEQ, int CPL, int DXST>
static hipError_t bwd_one_st(const BwdParams& p, hipStream_t s) {
  using C = BwdCfg<TX>;
  return launch(reinterpret_cast<const void*>(
                    &bwd_fast_kernel<TX, W, SILU, SEQ, CPL, C::NW, bwd_rows<TX, W, SEQ, CPL>(),
                                     C::XLD, C::YLD, DXST>),
                dim3(p.tl.nBlk), dim3(C::NW * 64), 0, s, &p);
}

// The dx store policy the host chose for this call (BwdParams::dx_nt), below kUnitWideW.
template <typename TX, int W, bool SILU, bool SEQ, int CPL>
static hipError_t bwd_one(const BwdParams& p, hipStream_t s) {
  using C = BwdCfg<TX>;
  if constexpr (W < kUnitWideW && C::DXST_STREAM != C::DXST) {
    if (p.dx_nt) return bwd_one_st<TX, W, SILU, SEQ, CPL, C::DXST_STREAM>(p, s);
  }
  return bwd_one_st<TX, W, SILU, SEQ, CPL, C::DXST>(p, s);
}

// The channels per lane the host's tiling chose (Tiling::vec): CPL_WIDE from kBwdWideW up; below
// it CPL or CPL_WIDE; kCplLong from kBwdLongW. Any other value is rejected.
template <typename TX, int W, bool SILU, bool SEQ>
static hipError_t bwd_vec(const BwdParams& p, hipStream_t s) {
  using C = BwdCfg<TX>;
  if constexpr (W >= kBwdLongW) {
    if (p.tl.vec == kCplLong) return bwd_one<TX, W, SILU, SEQ, kCplLong>(p, s);
  } else {
    if (p.tl.vec == C::CPL_WIDE) return bwd_one<TX, W, SILU, SEQ, C::CPL_WIDE>(p, s);
    if constexpr (W < kBwdWideW) {
      if (p.tl.vec == C::CPL) return bwd_one<TX, W, SILU, SEQ, C::CPL>(p, s);
    }
  }
  return hipErrorInvalidValue;
}

template <typename TX, int W>
static hipError_t fwd_w(const FwdParams& p, hipStream_t s) {
  const bool seq = p.seq != nullptr;
  if (p.silu) return seq ? fwd_vec<TX, W, true, true>(p, s) : fwd_vec<TX, W, true, false>(p, s);
  return seq ? fwd_vec<TX, W, false, true>(p, s) : fwd_vec<TX, W, false, false>(p, s);
}

template <typename TX, int W>
static hipError_t bwd_w(const BwdParams& p, hipStream_t s) {
  const bool seq = p.seq != nullptr;
  if (p.silu) return seq ? bwd_vec<TX, W, true, true>(p, s) : bwd_vec<TX, W, true, false>(p, s);
  return seq ? bwd_vec<TX, W, false, true>(p, s) : bwd_vec<TX, W, false, false>(p, s);
}

template <typename TX>
hipError_t launch_fwd_fast_narrow_t(const FwdParams& p, hipStream_t s) {
  switch (p.W) {
    case 2: return fwd_w<TX, 2>(p, s);
    case 3: return fwd_w<TX, 3>(p, s);
    case 4: return fwd_w<TX, 4>(p, s);
    case 5: return fwd_w<TX, 5>(p, s);
    case 6: return fwd_w<TX, 6>(p, s);
    case 7: return fwd_w<TX, 7>(p, s);
    case 8: return fwd_w<TX, 8>(p, s);
    default: return hipErrorInvalidValue;
  }
}

template <typename TX>
hipError_t launch_fwd_fast_wide_t(const FwdParams& p, hipStream_t s) {
  switch (p.W) {
    case 9: return fwd_w<TX, 9>(p, s);
    case 10: return fwd_w<TX, 10>(p, s);
    case 11: return fwd_w<TX, 11>(p, s);
    case 12: return fwd_w<TX, 12>(p, s);
    case 13: return fwd_w<TX, 13>(p, s);
    case 14: return fwd_w<TX, 14>(p, s);
    case 15: return fwd_w<TX, 15>(p, s);
    case 16: return fwd_w<TX, 16>(p, s);
    default: return hipErrorInvalidValue;
  }
}

template <typename TX>
hipError_t launch_bwd_fast_narrow_t(const BwdParams& p, hipStream_t s) {
  switch (p.W) {
    case 2: return bwd_w<TX, 2>(p, s);
    case 3: return bwd_w<TX, 3>(p, s);
    case 4: return bwd_w<TX, 4>(p, s);
    case 5: return bwd_w<TX, 5>(p, s);
    case 6: return bwd_w<TX, 6>(p, s);
    case 7: return bwd_w<TX, 7>(p, s);
    case 8: return bwd_w<TX, 8>(p, s);
    default: return hipErrorInvalidValue;
  }
}

template <typename TX>
hipError_t launch_bwd_fast_wide_t(const BwdParams& p, hipStream_t s) {
  switch (p.W) {
    case 9: return bwd_w<TX, 9>(p, s);
    case 10: return bwd_w<TX, 10>(p, s);
    case 11: return bwd_w<TX, 11>(p, s);
    case 12: return bwd_w<TX, 12>(p, s);
    case 13: return bwd_w<TX, 13>(p, s);
    case 14: return bwd_w<TX, 14>(p, s);
    case 15: return bwd_w<TX, 15>(p, s);
    case 16: return bwd_w<TX, 16>(p, s);
    default: return hipErrorInvalidValue;
  }
}

template <typename TX>
hipError_t launch_fwd_fast_long1_t(const FwdParams& p, hipStream_t s) {
  switch (p.W) {
    case 17: return fwd_w<TX, 17>(p, s);
    case 18: return fwd_w<TX, 18>(p, s);
    case 19: return fwd_w<TX, 19>(p, s);
    case 20: return fwd_w<TX, 20>(p, s);
    case 21: return fwd_w<TX, 21>(p, s);
    case 22: return fwd_w<TX, 22>(p, s);
    case 23: return fwd_w<TX, 23>(p, s);
    case 24: return fwd_w<TX, 24>(p, s);
    default: return hipErrorInvalidValue;
  }
}

template <typename TX>
hipError_t launch_fwd_fast_long2_t(const FwdParams& p, hipStream_t s) {
  switch (p.W) {
    case 25: return fwd_w<TX, 25>(p, s);
    case 26: return fwd_w<TX, 26>(p, s);
    case 27: return fwd_w<TX, 27>(p, s);
    case 28: return fwd_w<TX, 28>(p, s);
    case 29: return fwd_w<TX, 29>(p, s);
    case 30: return fwd_w<TX, 30>(p, s);
    case 31: return fwd_w<TX, 31>(p, s);
    case 32: return fwd_w<TX, 32>(p, s);
    default: return hipErrorInvalidValue;
  }
}

template <typename TX>
hipError_t launch_bwd_fast_long1_t(const BwdParams& p, hipStream_t s) {
  switch (p.W) {
    case 17: return bwd_w<TX, 17>(p, s);
    case 18: return bwd_w<TX, 18>(p, s);
    case 19: return bwd_w<TX, 19>(p, s);
    case 20: return bwd_w<TX, 20>(p, s);
    case 21: return bwd_w<TX, 21>(p, s);
    case 22: return bwd_w<TX, 22>(p, s);
    case 23: return bwd_w<TX, 23>(p, s);
    case 24: return bwd_w<TX, 24>(p, s);
    default: return hipErrorInvalidValue;
  }
}

template <typename TX>
hipError_t launch_bwd_fast_long2_t(const BwdParams& p, hipStream_t s) {
  switch (p.W) {
    case 25: return bwd_w<TX, 25>(p, s);
    case 26: return bwd_w<TX, 26>(p, s);
    case 27: return bwd_w<TX, 27>(p, s);
    case 28: return bwd_w<TX, 28>(p, s);
    case 29: return bwd_w<TX, 29>(p, s);
    case 30: return bwd_w<TX, 30>(p, s);
    case 31: return bwd_w<TX, 31>(p, s);
    case 32: return bwd_w<TX, 32>(p, s);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace ccv1d
#endif
