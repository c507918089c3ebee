// C ABI of libccv1d.so (declared in include/ccv1d.h): argument validation, the empty-input paths,
// the choice between the vectorised and the generic kernels, time tiling, and launches on the
// caller's stream. This is the host launcher layer of the reference (`_fwd`, `_bwd`, `_chunking`;
// causal_conv1d.py:377-541) moved into native code.
#include <atomic>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <mutex>
#include <string>

#include "ccv1d.h"
#include "ccv1d_launch.h"

using namespace ccv1d;

namespace {

thread_local std::string g_last_error;

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

int hip_fail(hipError_t e, const char* what) {
  return fail(CCV1D_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

bool valid_dt(int dt) { return dt >= CCV1D_F32 && dt <= CCV1D_F64; }

int esize(int dt) { return dt == CCV1D_F64 ? 8 : dt == CCV1D_F32 ? 4 : 2; }

// Bytes from the first element of a (B, T, D) array with unit channel stride to one past its last.
int64_t span_bytes(int64_t B, int64_t T, int64_t D, int64_t s_b, int64_t s_t, int es) {
  return ((B - 1) * s_b + (T - 1) * s_t + D) * es;
}

// Whether the byte ranges [a, a + na) and [b, b + nb) share a byte.
bool ranges_meet(const void* a, int64_t na, const void* b, int64_t nb) {
  const uintptr_t pa = reinterpret_cast<uintptr_t>(a), pb = reinterpret_cast<uintptr_t>(b);
  return pa < pb + static_cast<uintptr_t>(nb) && pb < pa + static_cast<uintptr_t>(na);
}

// Channels per lane and waves per workgroup of the vectorised kernels for an x dtype.
struct FastShape {
  int cpl, nw;
};

template <template <typename> class Cfg>
FastShape shape_of(int x_dt) {
  switch (x_dt) {
    case CCV1D_BF16: return {Cfg<__bf16>::CPL, Cfg<__bf16>::NW};
    case CCV1D_F16: return {Cfg<_Float16>::CPL, Cfg<_Float16>::NW};
    default: return {Cfg<float>::CPL, Cfg<float>::NW};
  }
}

// Longest tile of the vectorised kernels (defaults and overrides alike). With seq_idx a wave reads the
// ids of its tile and both halos (L + 2 (W - 1) rows) up front into one RowIds.
// Every tile is at least min_tile_rows(W) long (defaults and overrides), longer than the window
// (W - 1), so only the first tile of a row has a window outside x.
constexpr int kMaxTileRows = 64;
// Longest tile without seq_idx for the backward with one channel per lane and the forward from
// kFwdTileRows128W (see bwd_tiling_for, fwd_tiling_for); with seq_idx a tile and both halos must fit
// one RowIds, which keeps kMaxTileRows.
constexpr int kMaxTileRowsLong = 128;
constexpr int kFwdTileRows128W = 24;
constexpr int kMinTileRows = 8;
static_assert(kMaxTileRows + 2 * (kMaxFastW - 1) <= kRowIds, "tile and halos must fit one RowIds");
static_assert(kMaxFastW <= kMaxTileRows, "the longest tile must be longer than every window");

// Shortest tile for width W: the shortest power of two from kMinTileRows up that is longer than the
// window of W - 1 rows (8 rows up to width 8, 16 up to 16, 32 up to 32).
int min_tile_rows(int64_t W) {
  int L = kMinTileRows;
  while (L < W) L *= 2;
  return L;
}

// Row tiling overrides for tuning sweeps: CCV1D_FWD_ROWS / CCV1D_BWD_ROWS (rows per tile of the
// vectorised kernels; a power of two in [8, kMaxTileRows], ignored for widths whose shortest tile
// is longer). They change the backward's partial-row count and hence the dweight/dbias summation
// order, so they exist only in a library built with -DCCV1D_TUNING (make EXTRA_HIPFLAGS=
// -DCCV1D_TUNING); the shipped library ignores the environment and its tiling depends on the
// shape alone.
struct Tune {
  int fwd_rows = 0;
  int bwd_rows = 0;
  int fwd_out_nt = -1;  // CCV1D_FWD_OUT_NT: 0 / 1 forces the forward's out-store policy
  int fwd_x_nt = -1;    // CCV1D_FWD_X_NT: 1 forces non-temporal x loads (and out stores)
};

const Tune& tune() {
#ifdef CCV1D_TUNING
  static const Tune t = [] {
    Tune v;
    auto rd = [](const char* name) {
      const char* e = std::getenv(name);
      if (!e) return 0;
      const int r = std::atoi(e);
      return (r >= kMinTileRows && r <= kMaxTileRows && (r & (r - 1)) == 0) ? r : 0;
    };
    v.fwd_rows = rd("CCV1D_FWD_ROWS");
    v.bwd_rows = rd("CCV1D_BWD_ROWS");
    if (const char* e = std::getenv("CCV1D_FWD_OUT_NT")) v.fwd_out_nt = std::atoi(e) != 0;
    if (const char* e = std::getenv("CCV1D_FWD_X_NT")) v.fwd_x_nt = std::atoi(e) != 0;
    return v;
  }();
#else
  static const Tune t{};
#endif
  return t;
}

// Bytes of x plus out above which the forward's out rows are stored non-temporally even when a
// backward follows: half the 256 MiB Infinity Cache. Below it x stays cached for the backward, and
// device-scope stores of out are faster (B=4 T=8192 D=1024 bf16, 128 MiB: step 60.2 us against
// 62.8-64.2 with non-temporal stores); above it the cache cannot hold x until the backward reads it
// and non-temporal stores win (T=32768, 512 MiB: 245-250 -> 227-231 us).
constexpr int64_t kFwdCachedBytes = int64_t(128) << 20;

// For inference (no backward follows) the threshold is lower: non-temporal out stores, with x also
// loaded non-temporally, pay once the pass streams more than 64 MiB (B=4 D=1024 bf16, forward
// alone over 512 MiB of rotating x: T=8192 28.7 -> 27.4-27.6 us, T=32768 108-109 -> 105.7-106.8
// us), while small calls are faster with the default policies (T=512: 4.24 against 4.76 us;
// chunks of B=16 T=256 D=2048: 9.17 against 9.92 us per call).
constexpr int64_t kFwdInferenceCachedBytes = int64_t(64) << 20;

// Whether the forward stores out non-temporally, by the bytes of x and out: above
// kFwdInferenceCachedBytes for inference, above kFwdCachedBytes when a backward follows.
bool fwd_out_streams(bool inference, int64_t B, int64_t T, int64_t D, int x_dt) {
  if (tune().fwd_out_nt >= 0) return tune().fwd_out_nt != 0;
  const int64_t bytes = 2 * B * T * D * esize(x_dt);
  return bytes > (inference ? kFwdInferenceCachedBytes : kFwdCachedBytes);
}

// Workgroups along time, per batch row and wave column, below which the tiles are shortened (down
// to the shortest tile). With fewer, every dispatch wave of the grid covers few rows of many
// columns: measured at B=8 T=4096 D=4096 (8 workgroups per column with 64-row tiles) the step took
// 293 us against 243 us with 32-row tiles; at B=4 T=8192 D=4096 (16 per column) 64 rows stay
// better (248 vs 251 us). That holds for the backward with 4 channels per lane and the forward below
// kFwdLongTileW. The backward with 2 or 1 channels per lane (widths from 6, and small grids) and the
// forward from kFwdLongTileW (its window of W - 1 halo rows is re-read per tile) take the longest
// tile the wave target allows, however few workgroups that leaves along time (the rule is not
// applied). Measured on one box, bf16, bias + silu, the rule's tiles against 64-row tiles:
//   fwd+bwd step: B=8 T=4096 D=4096 W=6 251 -> 238 us, W=9 292 -> 270, W=16 426 -> 382, W=24 701
//   -> 580; B=8 T=4096 D=5376 W=7 357 -> 335, W=20 775 -> 653; B=32 T=1024 D=2048 W=6 145 -> 137,
//   W=16 226 -> 201; B=8 T=1024 D=4096 W=8 94 -> 78; B=64 T=512 D=2048 W=12 184 -> 166; (W=4, 4
//   channels: B=8 T=4096 D=4096 227 against 243 with 64 rows, the benchmark shape 60.4 against
//   62.5);
//   forward alone: B=8 T=4096 D=4096 W=12 113 -> 104 us, W=16 131 -> 112, W=24 169 -> 151;
//   B=16 T=2048 D=2048 W=16 83 -> 62; B=64 T=512 D=2048 W=16 83 -> 59 (W=4-9 mixed: B=8 T=4096
//   D=4096 W=4 99 against 133 with 64 rows, W=9 108 against 113).
constexpr int64_t kMinTimeWorkgroups = 16;
constexpr int kFwdLongTileW = 12;

// Waves the vectorised kernels' tilings aim for (16 per CU).
constexpr int64_t kTargetWaves = 4096;

// Tiling of the vectorised kernels: the longest tile (fewest halo re-reads) that still gives the
// grid `target_waves` waves, every column `min_time_wg` workgroups along time and at least `nw`
// tiles along time (a workgroup's waves take consecutive tiles, so fewer would leave some of its
// waves without one: B=64 T=512 D=2048 W=24 fwd+bwd 283 us with 64-row tiles, 329 with 128, whose
// 4 tiles fill half of each workgroup), a function of the shape alone so that results, including
// the dweight summation order, do not depend on the device.
Tiling fast_tiling(int64_t B, int64_t T, int64_t D, int vec, int nw, int lmin, int lmax,
                   int64_t target_waves, int override_rows,
                   int64_t min_time_wg = kMinTimeWorkgroups) {
  Tiling t{};
  const int64_t G = D / vec;
  t.nGW = (int32_t)cdiv(G, 64);
  int L = lmax;
  if (override_rows > 0) {
    L = override_rows;
  } else {
    while (L > lmin && (B * cdiv(T, L) * t.nGW < target_waves ||
                        cdiv(cdiv(T, L), nw) < min_time_wg || cdiv(T, L) < nw))
      L >>= 1;
  }
  t.L = L;
  t.nT = (int32_t)cdiv(T, L);
  t.nTB = (int32_t)cdiv(t.nT, nw);
  t.nBlk = (int32_t)(B * t.nGW * t.nTB);
  t.vec = vec;
  return t;
}

// Workgroups below which the forward halves its shortest tile once more (16 -> 8 rows): small
// grids are bound by how many CUs they reach, not by the extra halo reads (measured: B=4 T=512
// D=1024 forward 7.0 -> 5.3 us; B=4 T=2048, whose 16-row grid has 256 workgroups, stays at 16).
constexpr int64_t kFwdSmallGrid = 256;

// The forward from width kFwdTileRows128W without seq_idx takes tiles of up to kMaxTileRowsLong
// rows (its window of W - 1 halo rows is re-read per tile). Measured (forward alone, bf16, 64
// against 128 rows): B=4 T=8192 D=1024 W=24 40.4 -> 39.8 us, W=32 48.5 -> 46.8; B=8 T=4096 D=4096
// W=24 153.5 -> 146.6, W=32 181.9 -> 169.5; B=4 T=1024 D=8192 W=32 49.4 -> 47.2; at widths 17-20
// mixed (B=16 T=2048 D=2048 W=17 63.7 against 69.7 with 128 rows).
Tiling fwd_tiling_for(int64_t B, int64_t T, int64_t D, int64_t W, int cpl, int nw, bool seq) {
  const int lmin = min_tile_rows(W);
  const int over = tune().fwd_rows >= lmin ? tune().fwd_rows : 0;
  const int64_t min_time_wg = W >= kFwdLongTileW ? 1 : kMinTimeWorkgroups;
  const int lmax = W >= kFwdTileRows128W && !seq ? kMaxTileRowsLong : kMaxTileRows;
  Tiling t = fast_tiling(B, T, D, cpl, nw, lmin > 16 ? lmin : 16, lmax, kTargetWaves, over,
                         min_time_wg);
  if (over == 0 && t.L == 16 && lmin < 16 && t.nBlk < kFwdSmallGrid)
    t = fast_tiling(B, T, D, cpl, nw, lmin, lmin, kTargetWaves, lmin);
  return t;
}

int fwd_cpl_small(int x_dt) {
  switch (x_dt) {
    case CCV1D_BF16: return FwdCfg<__bf16>::CPL_SMALL;
    case CCV1D_F16: return FwdCfg<_Float16>::CPL_SMALL;
    default: return FwdCfg<float>::CPL_SMALL;
  }
}

// Channels per lane and waves per workgroup of the vectorised forward for a shape: CPL, or
// CPL_SMALL when the CPL grid falls short of kTargetWaves waves even with its shortest tiles (or
// dim is not a multiple of CPL). Measured (forward alone, bf16, W=4, 2 against 4 channels): B=4
// D=1024 T=512 5.23 -> 4.68 us, T=2048 8.47 -> 8.11; B=16 D=2048 chunks of T=256 9.36 -> 9.04 us
// per call, decode steps 2.56 -> 2.53. Grids that reach the target keep 4 channels (benchmark shape
// 29.5 against 31.8 us; B=2 T=8192 D=1024 13.3 against 14.0). fp32 x follows the same rule in both
// passes (fwd+bwd step, B=4 D=1024 W=4: T=512 19.1 -> 16.8 us, T=2048 39.9 -> 37.7). 16-bit x
// also takes CPL_SMALL where the CPL grid reaches the target only with tiles shorter than
// kFwdShortTile rows: each workgroup then spends much of its short life on its start (halo, taps,
// first batch), which twice the resident workgroups hide. Measured (bf16, widths 2-6, 2 against 4
// channels, 16-row tiles in both): forward alone 3-27 % faster on 9 of 10 mid-size shapes (B=32
// T=1024 D=2048 W=4 65.5 -> 50.3 us, B=8 T=1024 D=4096 W=4 31.7 -> 28.0), up to 5 % slower on the
// tenth (B=16 T=512 D=4096), and the fwd+bwd step 1-11 % faster on all ten; fp32 x (16- against
// 8-byte rows) was mixed (-15 % to +6 %) and keeps 4. From width kFwdWideW up the forward always
// takes CPL_SMALL (its weights and window are per channel), from kFwdLongW up kCplLong.
constexpr int kFwdShortTile = 32;

FastShape fwd_shape(int x_dt, int64_t B, int64_t T, int64_t D, int64_t W) {
  FastShape sh = shape_of<FwdCfg>(x_dt);
  if (W >= kFwdLongW) {
    sh.cpl = kCplLong;
  } else if (W >= kFwdWideW) {
    sh.cpl = fwd_cpl_small(x_dt);
  } else if (x_dt != CCV1D_F64 && B > 0 && T > 0 && D > 0) {
    const Tiling t = fwd_tiling_for(B, T, D, W, sh.cpl, sh.nw, false);
    if (D % sh.cpl || B * t.nT * t.nGW < kTargetWaves || (esize(x_dt) == 2 && t.L < kFwdShortTile))
      sh.cpl = fwd_cpl_small(x_dt);
  }
  return sh;
}

Tiling fwd_fast_tiling(int64_t B, int64_t T, int64_t D, int64_t W, int x_dt, bool seq) {
  const FastShape sh = fwd_shape(x_dt, B, T, D, W);
  return fwd_tiling_for(B, T, D, W, sh.cpl, sh.nw, seq);
}

// Workgroups below which the backward halves its tiles (down to kMinTileRows): a grid with fewer
// workgroups than CUs is bound by the latency of one wave's walk through its tile, not by
// bandwidth. Measured at B=4 D=1024 W=4 (fwd+bwd step): T=512 24.6 -> 16.2 us (32 -> 8 rows, 32 ->
// 128 workgroups), T=2048 28.4 -> 24.2 us (32 -> 16 rows, 128 -> 256 workgroups); the benchmark
// shape (512 workgroups) keeps 32 rows.
constexpr int64_t kBwdSmallGrid = 256;

// The backward with one channel per lane (kCplLong) and no seq_idx takes tiles of up to
// kMaxTileRowsLong rows: halving the tiles' count halves the work each tile spends outside the
// pipelined loop (its halo rows, the g rows handed between waves, the partial dweight row), which
// grows with the width. Measured (fwd+bwd step, bf16, B=4 T=8192 D=1024, 64 against 128 rows in the
// backward): W=12 83.1 -> 80.7 us, W=16 97.9 -> 93.4, W=20 117.1 -> 114.1, W=24 149.6 -> 133.3,
// W=32 190.5 -> 166.5.

// Below kBwdWideW, where the backward takes 2 channels per lane because the 4-channel grid is
// small, 16-bit x also halves 32-row tiles to 16 while the grid has fewer than
// kBwdNarrowSmallGrid workgroups (fewer than kTargetWaves waves), and no further. Measured
// (fwd+bwd step, bias + silu, 32 against 16 rows, same box): bf16 W=4 B=4 T=2048 D=1024 20.8 ->
// 20.45 us (weight only 20.4 -> 19.6), B=1 T=4096 D=2048 21.4 -> 20.8, B=16 T=256 D=2048 21.2 ->
// 20.5; W=2 and W=3 0.6-0.9 us faster on those shapes, W=5 0.75 faster on two and even on the
// third; fp16 W=4 B=4 T=2048 D=1024 21.4 -> 21.2 (weight only 20.7 -> 20.0). Not taken: fp32 x
// (B=4 T=2048 D=1024 weight only 36.4 -> 36.8), halving 16-row tiles to 8 on such grids (0.1-0.3
// us slower at B=4 T=1024 D=1024 and B=2 T=2048 D=1024), 16-row tiles at W=8 (0.0-0.8 us slower)
// and, with one channel per lane, at W=16 (0.0-0.3 us slower).
constexpr int64_t kBwdNarrowSmallGrid = 512;
constexpr int kBwdNarrowShortRows = 16;

Tiling bwd_tiling_for(int64_t B, int64_t T, int64_t D, int64_t W, int x_dt, int cpl, int nw,
                      bool seq) {
  const int lmin = min_tile_rows(W);
  const int over = tune().bwd_rows >= lmin ? tune().bwd_rows : 0;
  const int64_t min_time_wg = cpl >= 4 ? kMinTimeWorkgroups : 1;
  const int lmax = cpl == kCplLong && !seq ? kMaxTileRowsLong : kMaxTileRows;
  Tiling t = fast_tiling(B, T, D, cpl, nw, 32, lmax, kTargetWaves, over, min_time_wg);
  while (over == 0 && t.nBlk < kBwdSmallGrid && t.L > lmin)
    t = fast_tiling(B, T, D, cpl, nw, t.L / 2, t.L / 2, kTargetWaves, t.L / 2);
  if (over == 0 && esize(x_dt) == 2 && W < kBwdWideW && cpl < 4 &&
      t.L == 2 * kBwdNarrowShortRows && t.nBlk < kBwdNarrowSmallGrid && kBwdNarrowShortRows >= lmin)
    t = fast_tiling(B, T, D, cpl, nw, kBwdNarrowShortRows, kBwdNarrowShortRows, kTargetWaves,
                    kBwdNarrowShortRows);
  return t;
}

// The vectorised backward at widths under kBwdWideW takes 2 channels per lane instead of 4 when
// the 4-channel grid is small: fewer than kTargetWaves waves, or tiles shortened below
// kBwdNarrowMinRows rows to reach them. 2 channels per lane doubles the waves while keeping the
// tiles longer. Measured (fwd+bwd step, bf16, 2 against 4 channels): B=4 D=1024 W=4 T=512 16.2 ->
// 13.8 us, T=2048 24.1 -> 22.5, T=4096 39.9 -> 37.2; B=2 T=8192 D=1024 38.8 -> 36.8; W=2 T=512
// 15.2 -> 13.8; W=3 T=2048 23.3 -> 22.1; W=5 T=2048 25.1 -> 22.9. Grids that reach the target with
// 32- or 64-row tiles keep 4 channels (B=4 D=1024 T=32768: 250 against 256-258 us; B=1 T=8192
// D=4096: 61.0 against 61.5; the benchmark shape: a tie at 32 rows, 62.3 us when 2 channels pick
// 64-row tiles).
constexpr int kBwdNarrowMinRows = 32;

int cpl_wide(int x_dt) {
  switch (x_dt) {
    case CCV1D_BF16: return BwdCfg<__bf16>::CPL_WIDE;
    case CCV1D_F16: return BwdCfg<_Float16>::CPL_WIDE;
    default: return BwdCfg<float>::CPL_WIDE;
  }
}

// Channels per lane and waves per workgroup of the vectorised backward for a shape: CPL_WIDE from
// kBwdWideW up (register budget), and below it when the 4-channel grid is small (above) or dim is
// not a multiple of 4; CPL otherwise; kCplLong from kBwdLongW up.
FastShape bwd_shape(int x_dt, int64_t B, int64_t T, int64_t D, int64_t W) {
  FastShape sh = shape_of<BwdCfg>(x_dt);
  if (W >= kBwdLongW) {
    sh.cpl = kCplLong;
  } else if (W >= kBwdWideW) {
    sh.cpl = cpl_wide(x_dt);
  } else if (x_dt != CCV1D_F64 && B > 0 && T > 0 && D > 0) {
    const Tiling t = bwd_tiling_for(B, T, D, W, x_dt, sh.cpl, sh.nw, false);
    if (D % sh.cpl || t.L < kBwdNarrowMinRows || B * t.nT * t.nGW < kTargetWaves)
      sh.cpl = cpl_wide(x_dt);
  }
  return sh;
}

Tiling bwd_fast_tiling(int64_t B, int64_t T, int64_t D, int64_t W, int x_dt, bool seq) {
  const FastShape sh = bwd_shape(x_dt, B, T, D, W);
  return bwd_tiling_for(B, T, D, W, x_dt, sh.cpl, sh.nw, seq);
}

// Workspace of the backward: the fp32 partial rows of dweight/dbias, (rows, W + 1, D) floats, and
// for widths above kMaxGenericW after them, 256-byte aligned, the fp32 g buffer (B, T, D).
size_t partial_bytes(int64_t rows, int64_t W, int64_t D) {
  return (size_t)(rows * (W + 1) * D * (int64_t)sizeof(float));
}
size_t g_buffer_bytes(int64_t B, int64_t T, int64_t D) {
  return (size_t)(B * T * D * (int64_t)sizeof(float));
}
size_t g_buffer_offset(size_t partials) { return (partials + 255) & ~(size_t)255; }

Tiling generic_tiling(int64_t T) {
  Tiling t{};
  t.L = kGenericL;
  t.nT = (int32_t)cdiv(T, kGenericL);
  return t;
}

// Restores the calling thread's current device on scope exit.
struct DeviceGuard {
  int prev = -1;
  bool changed = false;
  hipError_t err = hipSuccess;
  explicit DeviceGuard(int dev) {
    err = hipGetDevice(&prev);
    if (err == hipSuccess && prev != dev) {
      err = hipSetDevice(dev);
      changed = err == hipSuccess;
    }
  }
  ~DeviceGuard() {
    if (changed) (void)hipSetDevice(prev);
  }
};

int check_common(const void* x, int64_t s_xb, int64_t s_xt, int x_dt, const void* w, int w_dt,
                 const void* bias, int b_dt, const void* init, int i_dt, int64_t B, int64_t T,
                 int64_t D, int64_t W) {
  if (B < 0 || T < 0 || D < 0) return fail(CCV1D_ERR_INVALID, "negative shape (%lld, %lld, %lld)",
                                           (long long)B, (long long)T, (long long)D);
  if (W < 2) return fail(CCV1D_ERR_INVALID, "width must be >= 2 (got %lld)", (long long)W);
  if (!valid_dt(x_dt) || !valid_dt(w_dt) || (bias && !valid_dt(b_dt)) || (init && !valid_dt(i_dt)))
    return fail(CCV1D_ERR_INVALID, "bad dtype code");
  if (s_xb < 0 || s_xt < 0) return fail(CCV1D_ERR_INVALID, "negative stride");
  if (D > 0 && !w) return fail(CCV1D_ERR_INVALID, "weight is null");
  if (B * T * D > 0 && !x) return fail(CCV1D_ERR_INVALID, "x is null");
  if (D > 0 && (T + W) * (s_xt > D ? s_xt : D) >= (int64_t(1) << 31))
    return fail(CCV1D_ERR_INVALID, "(seqlen + width) * max(x time stride, dim) must be < 2^31");
  if (B >= (int64_t(1) << 31) || D >= (int64_t(1) << 31))
    return fail(CCV1D_ERR_INVALID, "batch and dim must be < 2^31");
  return CCV1D_OK;
}

// The vectorised kernels read and write rows of `cpl` channels per lane: dim a multiple of cpl, the
// base and the strides aligned to the access width, and every byte offset inside one batch slab
// below 2^32 (they address rows through 32-bit buffer offsets).
bool rows_ok(int x_dt, int cpl, int64_t T, int64_t D, const void* p, int64_t s_b, int64_t s_t) {
  const int64_t esz = esize(x_dt);
  if (D % cpl || s_b % cpl || s_t % cpl) return false;
  if (reinterpret_cast<uintptr_t>(p) % (uintptr_t)(cpl * esz)) return false;
  return ((T - 1) * s_t + D) * esz < (int64_t(1) << 32);
}

bool aligned_to(const void* p, int64_t bytes) {
  return (reinterpret_cast<uintptr_t>(p) % (uintptr_t)bytes) == 0;
}

// A channel slice of a wider channels-last tensor (strides other than the contiguous (T * D, D))
// whose rows do not all start on a 128-byte line: each row's first and last lines, and the lines
// where neighbouring wave columns meet, are shared with other columns (TileCoord's col_fast).
bool straddling_slice(const void* p, int64_t s_b, int64_t s_t, int64_t B, int64_t T, int64_t D,
                      int es) {
  if ((s_t == D || T == 1) && (s_b == T * D || B == 1)) return false;
  const bool aligned = aligned_to(p, 128) && (T == 1 || (s_t * es) % 128 == 0) &&
                       (B == 1 || (s_b * es) % 128 == 0);
  return !aligned;
}

uint32_t slab_bytes(int x_dt, int64_t T, int64_t D, int64_t s_t) {
  return (uint32_t)(((T - 1) * s_t + D) * esize(x_dt));
}

bool fast_dtype(int x_dt, int64_t W) { return W <= kMaxFastW && x_dt != CCV1D_F64; }

// Takes the calling thread's timing request (ccv1d_time_main_kernel), so that it applies to this
// entry-point call only, whatever the call does.
bool take_timing_request() {
  KernelEvents& ev = kernel_events();
  const bool on = ev.pending;
  ev.pending = false;
  ev.armed = false;
  return on;
}

// Hands a taken timing request to the main kernel's launch for the lifetime of this object (one
// launch takes it; it is cleared on scope exit in case the launch was not reached).
struct TimedLaunch {
  explicit TimedLaunch(bool on) { kernel_events().armed = on; }
  ~TimedLaunch() { kernel_events().armed = false; }
};

}  // namespace

extern "C" {

int ccv1d_abi_version(void) { return CCV1D_ABI_VERSION; }

const char* ccv1d_last_error(void) { return g_last_error.c_str(); }

int ccv1d_time_main_kernel(void* start_event, void* stop_event) {
  g_last_error.clear();
  if ((start_event == nullptr) != (stop_event == nullptr))
    return fail(CCV1D_ERR_INVALID, "give both timing events or neither");
  KernelEvents& ev = kernel_events();
  ev.start = static_cast<hipEvent_t>(start_event);
  ev.stop = static_cast<hipEvent_t>(stop_event);
  ev.pending = start_event != nullptr;
  ev.armed = false;
  return CCV1D_OK;
}

}  // extern "C"

namespace {

// ccv1d_fwd and ccv1d_fwd_inference: the same validation, tiling and kernels; `inference` selects
// non-temporal out stores (fwd_out_streams).
int fwd_entry(const void* x, int64_t x_stride_b, int64_t x_stride_t, int x_dtype,
              const void* weight, int weight_dtype, const void* bias, int bias_dtype,
              const int32_t* seq_idx, const void* initial_states, int init_dtype, void* out,
              void* final_states, int64_t batch, int64_t seqlen, int64_t dim, int64_t width,
              int silu, int device, void* stream, bool inference) {
  g_last_error.clear();
  const bool timed = take_timing_request();
  const int64_t B = batch, T = seqlen, D = dim, W = width, P = W - 1;
  int rc = check_common(x, x_stride_b, x_stride_t, x_dtype, weight, weight_dtype, bias, bias_dtype,
                        initial_states, init_dtype, B, T, D, W);
  if (rc) return rc;
  if (seq_idx && final_states)
    return fail(CCV1D_ERR_INVALID, "cannot return final states if seq_idx is given");
  if (B * T * D > 0 && !out) return fail(CCV1D_ERR_INVALID, "out is null");
  // out is written while other tiles still read their halo rows of x: no in-place forward.
  if (B * T * D > 0 &&
      ranges_meet(out, span_bytes(B, T, D, T * D, D, esize(x_dtype)), x,
                  span_bytes(B, T, D, x_stride_b, x_stride_t, esize(x_dtype))))
    return fail(CCV1D_ERR_INVALID, "out must not overlap x");
  if (B * D == 0) return CCV1D_OK;
  const int fcpl = fwd_shape(x_dtype, B, T, D, W).cpl;
  const bool fast = T > 0 && fast_dtype(x_dtype, W) &&
                    rows_ok(x_dtype, fcpl, T, D, x, x_stride_b, x_stride_t) &&
                    rows_ok(x_dtype, fcpl, T, D, out, T * D, D) &&
                    (!final_states || aligned_to(final_states, fcpl * esize(x_dtype)));
  Tiling tl{};
  if (T > 0) {
    if (fast) {
      tl = fwd_fast_tiling(B, T, D, W, x_dtype, seq_idx != nullptr);
      tl.col_fast = W <= kColFastMaxW &&
                    straddling_slice(x, x_stride_b, x_stride_t, B, T, D, esize(x_dtype));
    } else {
      tl = generic_tiling(T);
      if (B * tl.nT >= (int64_t(1) << 31) || cdiv(D, 64) > 65535)
        return fail(CCV1D_ERR_UNSUPPORTED, "shape too large for the generic kernel");
    }
  }
  DeviceGuard guard(device);
  if (guard.err != hipSuccess) return hip_fail(guard.err, "hipSetDevice");
  hipStream_t s = static_cast<hipStream_t>(stream);

  if (T == 0) {
    // With no rows, the final states are the initial states (causal_conv1d.py:437-444).
    if (final_states) {
      const hipError_t e = launch_fill(final_states, x_dtype, initial_states, init_dtype, B * P * D, s);
      if (e != hipSuccess) return hip_fail(e, "fill launch");
    }
    return CCV1D_OK;
  }

  FwdParams p{};
  p.x = x;
  p.w = weight;
  p.bias = bias;
  p.seq = seq_idx;
  p.init = initial_states;
  p.out = out;
  p.fin = final_states;
  p.s_xb = x_stride_b;
  p.s_xt = (int32_t)x_stride_t;
  p.B = (int32_t)B;
  p.T = (int32_t)T;
  p.D = (int32_t)D;
  p.W = (int32_t)W;
  p.w_dt = weight_dtype;
  p.b_dt = bias_dtype;
  p.i_dt = init_dtype;
  p.has_bias = bias != nullptr;
  p.has_init = initial_states != nullptr;
  p.has_final = final_states != nullptr;
  p.silu = silu != 0;
  p.out_nt = fwd_out_streams(inference, B, T, D, x_dtype);
  p.x_nt = tune().fwd_x_nt >= 0 ? tune().fwd_x_nt != 0 : inference && p.out_nt;
  if (fast) {
    p.x_bytes = slab_bytes(x_dtype, T, D, x_stride_t);
    p.o_bytes = slab_bytes(x_dtype, T, D, D);
  }

  p.tl = tl;
  hipError_t e;
  {
    const TimedLaunch timing(timed);
    if (fast) {
      switch (x_dtype) {
        case CCV1D_BF16: e = launch_fwd_fast_t<__bf16>(p, s); break;
        case CCV1D_F16: e = launch_fwd_fast_t<_Float16>(p, s); break;
        default: e = launch_fwd_fast_t<float>(p, s); break;
      }
    } else {
      switch (x_dtype) {
        case CCV1D_BF16: e = launch_fwd_generic_t<__bf16>(p, s); break;
        case CCV1D_F16: e = launch_fwd_generic_t<_Float16>(p, s); break;
        case CCV1D_F32: e = launch_fwd_generic_t<float>(p, s); break;
        default: e = launch_fwd_generic_t<double>(p, s); break;
      }
    }
  }
  if (e != hipSuccess) return hip_fail(e, "forward launch");
  return CCV1D_OK;
}

}  // namespace

extern "C" {

int ccv1d_fwd(const void* x, int64_t x_stride_b, int64_t x_stride_t, int x_dtype,
              const void* weight, int weight_dtype, const void* bias, int bias_dtype,
              const int32_t* seq_idx, const void* initial_states, int init_dtype, void* out,
              void* final_states, int64_t batch, int64_t seqlen, int64_t dim, int64_t width,
              int silu, int device, void* stream) {
  return fwd_entry(x, x_stride_b, x_stride_t, x_dtype, weight, weight_dtype, bias, bias_dtype,
                   seq_idx, initial_states, init_dtype, out, final_states, batch, seqlen, dim,
                   width, silu, device, stream, false);
}

int ccv1d_fwd_inference(const void* x, int64_t x_stride_b, int64_t x_stride_t, int x_dtype,
                        const void* weight, int weight_dtype, const void* bias, int bias_dtype,
                        const int32_t* seq_idx, const void* initial_states, int init_dtype,
                        void* out, void* final_states, int64_t batch, int64_t seqlen, int64_t dim,
                        int64_t width, int silu, int device, void* stream) {
  return fwd_entry(x, x_stride_b, x_stride_t, x_dtype, weight, weight_dtype, bias, bias_dtype,
                   seq_idx, initial_states, init_dtype, out, final_states, batch, seqlen, dim,
                   width, silu, device, stream, true);
}

size_t ccv1d_bwd_workspace_bytes(int64_t batch, int64_t seqlen, int64_t dim, int64_t width,
                                 int x_dtype) {
  const int64_t B = batch, T = seqlen, D = dim, W = width;
  if (B <= 0 || T <= 0 || D <= 0 || W < 2 || !valid_dt(x_dtype)) return 0;
  int64_t rows = B * generic_tiling(T).nT;
  if (W <= kMaxFastW && x_dtype != CCV1D_F64) {
    // With seq_idx the tiles are never longer, so its tiling has at least as many partial rows.
    const int64_t fr = B * bwd_fast_tiling(B, T, D, W, x_dtype, true).nTB;
    if (fr > rows) rows = fr;
  }
  size_t n = partial_bytes(rows, W, D);
  if (W > kMaxGenericW) n = g_buffer_offset(n) + g_buffer_bytes(B, T, D);
  return n;
}

}  // extern "C"

namespace {

// Scratch of the allocation-free backward (ccv1d_bwd_noalloc): its fp32 partial rows live here
// instead of in a caller workspace. The name is a host-side stand-in; the device address comes
// from hipGetSymbolAddress (scratch_on_current_device), once per device, and only that address is
// ever given to kernels. Every device the library runs on holds its own copy until the process
// ends.
static __device__ __align__(256) unsigned char scratch[CCV1D_NOALLOC_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;
std::atomic<void*> g_scratch_addr[kMaxDevices];
std::mutex g_scratch_mu;

// Device address of `scratch` on `device`, which must be the current device. Resolved at the
// first call on each device and kept.
int scratch_on_current_device(int device, void** addr) {
  if (device < 0 || device >= kMaxDevices)
    return fail(CCV1D_ERR_INVALID, "device %d outside the %d devices the scratch table covers",
                device, kMaxDevices);
  void* a = g_scratch_addr[device].load(std::memory_order_acquire);
  if (!a) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    a = g_scratch_addr[device].load(std::memory_order_relaxed);
    if (!a) {
      const hipError_t e = hipGetSymbolAddress(&a, HIP_SYMBOL(scratch));
      if (e != hipSuccess) return hip_fail(e, "hipGetSymbolAddress(scratch)");
      if (!a) return fail(CCV1D_ERR_HIP, "hipGetSymbolAddress(scratch) returned no address");
      g_scratch_addr[device].store(a, std::memory_order_release);
    }
  }
  *addr = a;
  return CCV1D_OK;
}

// A validated backward request: the kernel parameters, the path, the tiling and the workspace it
// needs, with everything but the workspace address filled in. Planning makes no HIP call, so a
// request is refused (status and message) before anything touches a device.
struct BwdPlan {
  BwdParams p{};
  ReduceParams r{};
  bool skip = false;   // dim == 0: nothing to do
  bool empty = false;  // batch == 0 or seqlen == 0: the fill path
  bool fast = false;
  bool wide = false;   // generic path above kMaxGenericW: g goes through the workspace
  int x_dt = 0;
  size_t g_off = 0;    // byte offset of the g buffer in the workspace (wide)
  size_t need = 0;     // workspace bytes the launches use
};

// Kernels, tiling and workspace of a backward with these rows (B, T, D > 0): the vectorised
// kernels when the x dtype, the width and the alignment of every row of x, dout and dx (and of
// dfinal_states) allow them, else the generic ones.
struct BwdPath {
  bool fast = false;
  bool wide = false;   // generic path above kMaxGenericW: g goes through the workspace
  Tiling tl{};
  int64_t rows = 0;    // partial rows of dweight/dbias
  size_t g_off = 0;    // byte offset of the g buffer in the workspace (wide)
  size_t need = 0;     // workspace bytes
};

BwdPath bwd_path(const void* x, int64_t x_stride_b, int64_t x_stride_t, int x_dtype, bool seq,
                 const void* dout, int64_t dout_stride_b, int64_t dout_stride_t,
                 const void* dfinal_states, const void* dx, int64_t dx_stride_b,
                 int64_t dx_stride_t, bool ws_aligned, int64_t B, int64_t T, int64_t D,
                 int64_t W) {
  BwdPath r;
  const int bcpl = bwd_shape(x_dtype, B, T, D, W).cpl;
  r.fast = fast_dtype(x_dtype, W) && rows_ok(x_dtype, bcpl, T, D, x, x_stride_b, x_stride_t) &&
           rows_ok(x_dtype, bcpl, T, D, dout, dout_stride_b, dout_stride_t) &&
           rows_ok(x_dtype, bcpl, T, D, dx, dx_stride_b, dx_stride_t) &&
           (!dfinal_states || aligned_to(dfinal_states, bcpl * esize(x_dtype))) && ws_aligned;
  if (r.fast) {
    r.tl = bwd_fast_tiling(B, T, D, W, x_dtype, seq);
    r.rows = B * r.tl.nTB;
  } else {
    r.tl = generic_tiling(T);
    r.rows = B * r.tl.nT;
    r.wide = W > kMaxGenericW;
  }
  r.need = partial_bytes(r.rows, W, D);
  if (r.wide) {
    r.g_off = g_buffer_offset(r.need);
    r.need = r.g_off + g_buffer_bytes(B, T, D);
  }
  return r;
}

// `ws_aligned`: the workspace the call will use is 16-byte aligned (the vectorised backward stores
// partial rows with 16-byte accesses).
// dx_stride_b / dx_stride_t: strides of dx in elements (T * D and D for a contiguous dx).
int plan_bwd(const void* x, int64_t x_stride_b, int64_t x_stride_t, int x_dtype,
             const void* weight, int weight_dtype, const void* bias, int bias_dtype,
             const int32_t* seq_idx, const void* initial_states, int init_dtype,
             const void* dout, int64_t dout_stride_b, int64_t dout_stride_t,
             const void* dfinal_states, void* dx, int64_t dx_stride_b, int64_t dx_stride_t,
             void* dinitial_states, void* dweight, void* dbias, bool ws_aligned, int64_t batch,
             int64_t seqlen, int64_t dim, int64_t width, int silu, BwdPlan& pl) {
  const int64_t B = batch, T = seqlen, D = dim, W = width;
  int rc = check_common(x, x_stride_b, x_stride_t, x_dtype, weight, weight_dtype, bias, bias_dtype,
                        initial_states, init_dtype, B, T, D, W);
  if (rc) return rc;
  if (dout_stride_b < 0 || dout_stride_t < 0) return fail(CCV1D_ERR_INVALID, "negative stride");
  if (D > 0 && (T + W) * (dout_stride_t > D ? dout_stride_t : D) >= (int64_t(1) << 31))
    return fail(CCV1D_ERR_INVALID, "(seqlen + width) * max(dout time stride, dim) must be < 2^31");
  // dx rows of one batch element must not overlap each other or the next element's.
  if (B * T * D > 0) {
    if ((T > 1 && dx_stride_t < D) || (B > 1 && dx_stride_b < (T - 1) * dx_stride_t + D))
      return fail(CCV1D_ERR_INVALID, "dx strides (%lld, %lld) overlap rows of (%lld, %lld, %lld)",
                  (long long)dx_stride_b, (long long)dx_stride_t, (long long)B, (long long)T,
                  (long long)D);
    if ((T + W) * (dx_stride_t > D ? dx_stride_t : D) >= (int64_t(1) << 31))
      return fail(CCV1D_ERR_INVALID, "(seqlen + width) * max(dx time stride, dim) must be < 2^31");
  }
  if (B * T * D > 0 && (!dout || !dx)) return fail(CCV1D_ERR_INVALID, "dout or dx is null");
  // dx is written while the other tiles still read x and dout (halo rows): it must not share
  // memory with either, e.g. dx = x for an in-place update.
  if (B * T * D > 0) {
    const int es = esize(x_dtype);
    const int64_t ndx = span_bytes(B, T, D, dx_stride_b, dx_stride_t, es);
    if (ranges_meet(dx, ndx, x, span_bytes(B, T, D, x_stride_b, x_stride_t, es)) ||
        ranges_meet(dx, ndx, dout, span_bytes(B, T, D, dout_stride_b, dout_stride_t, es)))
      return fail(CCV1D_ERR_INVALID, "dx must not overlap x or dout");
  }
  if (D > 0 && !dweight) return fail(CCV1D_ERR_INVALID, "dweight is null");
  if ((bias != nullptr) != (dbias != nullptr))
    return fail(CCV1D_ERR_INVALID, "dbias must be given exactly when bias is");
  if (dinitial_states && !initial_states)
    return fail(CCV1D_ERR_INVALID, "dinitial_states requires initial_states");
  if (seq_idx && dfinal_states)
    return fail(CCV1D_ERR_INVALID, "cannot take final-state gradients if seq_idx is given");
  pl.x_dt = x_dtype;
  pl.skip = D == 0;
  pl.empty = B == 0 || T == 0;

  BwdParams& p = pl.p;
  p.x = x;
  p.w = weight;
  p.bias = bias;
  p.seq = seq_idx;
  p.init = initial_states;
  p.dy = dout;
  p.dfin = dfinal_states;
  p.dx = dx;
  p.dinit = dinitial_states;
  p.s_xb = x_stride_b;
  p.s_yb = dout_stride_b;
  p.s_dxb = dx_stride_b;
  p.s_xt = (int32_t)x_stride_t;
  p.s_yt = (int32_t)dout_stride_t;
  p.s_dxt = (int32_t)dx_stride_t;
  p.B = (int32_t)B;
  p.T = (int32_t)T;
  p.D = (int32_t)D;
  p.W = (int32_t)W;
  p.w_dt = weight_dtype;
  p.b_dt = bias_dtype;
  p.i_dt = init_dtype;
  p.has_bias = bias != nullptr;
  p.has_init = initial_states != nullptr;
  p.has_dfinal = dfinal_states != nullptr;
  p.need_dinit = dinitial_states != nullptr;
  p.silu = silu != 0;
  ReduceParams& r = pl.r;
  r.dw = dweight;
  r.db = dbias;
  r.D = (int32_t)D;
  r.W = (int32_t)W;
  r.w_dt = weight_dtype;
  r.b_dt = bias_dtype;
  r.has_bias = bias != nullptr;
  if (pl.skip || pl.empty) return CCV1D_OK;

  const BwdPath path = bwd_path(x, x_stride_b, x_stride_t, x_dtype, seq_idx != nullptr, dout,
                                dout_stride_b, dout_stride_t, dfinal_states, dx, dx_stride_b,
                                dx_stride_t, ws_aligned, B, T, D, W);
  pl.fast = path.fast;
  pl.wide = path.wide;
  p.tl = path.tl;
  if (pl.fast) {
    p.x_bytes = slab_bytes(x_dtype, T, D, x_stride_t);
    p.y_bytes = slab_bytes(x_dtype, T, D, dout_stride_t);
    p.o_bytes = slab_bytes(x_dtype, T, D, dx_stride_t);
    const int es = esize(x_dtype);
    const bool dx_straddles = straddling_slice(dx, dx_stride_b, dx_stride_t, B, T, D, es);
    p.tl.col_fast = W <= kColFastMaxW &&
                    (dx_straddles || straddling_slice(x, x_stride_b, x_stride_t, B, T, D, es) ||
                     straddling_slice(dout, dout_stride_b, dout_stride_t, B, T, D, es));
    p.dx_nt = dx_straddles;
  } else if (path.rows >= (int64_t(1) << 31) || cdiv(D, 64) > 65535) {
    return fail(CCV1D_ERR_UNSUPPORTED, "shape too large for the generic kernel");
  }
  r.Pn = (int32_t)path.rows;
  pl.g_off = path.g_off;
  pl.need = path.need;
  return CCV1D_OK;
}

// Launches a planned backward with `workspace` (at least pl.need bytes) on `stream`: the main
// kernel then the reduction, or the fills of the empty path.
int run_bwd(BwdPlan& pl, void* workspace, int device, void* stream, bool timed) {
  if (pl.skip) return CCV1D_OK;
  DeviceGuard guard(device);
  if (guard.err != hipSuccess) return hip_fail(guard.err, "hipSetDevice");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const BwdParams& p = pl.p;

  if (pl.empty) {
    // No outputs: dweight = dbias = 0, and the initial-state gradient is the final-state gradient
    // (causal_conv1d.py:480-489).
    const int64_t P = p.W - 1;
    hipError_t e = launch_fill(pl.r.dw, p.w_dt, nullptr, 0, (int64_t)p.D * p.W, s);
    if (e == hipSuccess && pl.r.db) e = launch_fill(pl.r.db, p.b_dt, nullptr, 0, p.D, s);
    if (e == hipSuccess && p.dinit)
      e = launch_fill(p.dinit, p.i_dt, p.dfin, pl.x_dt, (int64_t)p.B * P * p.D, s);
    if (e != hipSuccess) return hip_fail(e, "fill launch");
    return CCV1D_OK;
  }

  pl.p.part = static_cast<float*>(workspace);
  pl.r.part = pl.p.part;
  hipError_t e;
  {
    const TimedLaunch timing(timed);
    if (pl.fast) {
      switch (pl.x_dt) {
        case CCV1D_BF16: e = launch_bwd_fast_t<__bf16>(p, s); break;
        case CCV1D_F16: e = launch_bwd_fast_t<_Float16>(p, s); break;
        default: e = launch_bwd_fast_t<float>(p, s); break;
      }
    } else if (pl.wide) {
      float* G = reinterpret_cast<float*>(static_cast<char*>(workspace) + pl.g_off);
      switch (pl.x_dt) {
        case CCV1D_BF16: e = launch_bwd_wide_t<__bf16>(p, G, s); break;
        case CCV1D_F16: e = launch_bwd_wide_t<_Float16>(p, G, s); break;
        case CCV1D_F32: e = launch_bwd_wide_t<float>(p, G, s); break;
        default: e = launch_bwd_wide_t<double>(p, G, s); break;
      }
    } else {
      switch (pl.x_dt) {
        case CCV1D_BF16: e = launch_bwd_generic_t<__bf16>(p, s); break;
        case CCV1D_F16: e = launch_bwd_generic_t<_Float16>(p, s); break;
        case CCV1D_F32: e = launch_bwd_generic_t<float>(p, s); break;
        default: e = launch_bwd_generic_t<double>(p, s); break;
      }
    }
  }
  if (e != hipSuccess) return hip_fail(e, "backward launch");
  e = launch_reduce(pl.r, s);
  if (e != hipSuccess) return hip_fail(e, "reduce launch");
  return CCV1D_OK;
}

}  // namespace

extern "C" {

size_t ccv1d_bwd_workspace_bytes_for(const void* x, int64_t x_stride_b, int64_t x_stride_t,
                                     int x_dtype, const int32_t* seq_idx, const void* dout,
                                     int64_t dout_stride_b, int64_t dout_stride_t,
                                     const void* dfinal_states, const void* dx, int64_t batch,
                                     int64_t seqlen, int64_t dim, int64_t width) {
  const int64_t B = batch, T = seqlen, D = dim, W = width;
  if (B <= 0 || T <= 0 || D <= 0 || W < 2 || !valid_dt(x_dtype)) return 0;
  if (x_stride_b < 0 || x_stride_t < 0 || dout_stride_b < 0 || dout_stride_t < 0) return 0;
  return bwd_path(x, x_stride_b, x_stride_t, x_dtype, seq_idx != nullptr, dout, dout_stride_b,
                  dout_stride_t, dfinal_states, dx, T * D, D, true, B, T, D, W)
      .need;
}

int ccv1d_bwd(const void* x, int64_t x_stride_b, int64_t x_stride_t, int x_dtype,
              const void* weight, int weight_dtype, const void* bias, int bias_dtype,
              const int32_t* seq_idx, const void* initial_states, int init_dtype,
              const void* dout, int64_t dout_stride_b, int64_t dout_stride_t,
              const void* dfinal_states, void* dx, void* dinitial_states, void* dweight,
              void* dbias, void* workspace, size_t workspace_bytes, int64_t batch, int64_t seqlen,
              int64_t dim, int64_t width, int silu, int device, void* stream) {
  g_last_error.clear();
  const bool timed = take_timing_request();
  BwdPlan pl;
  int rc = plan_bwd(x, x_stride_b, x_stride_t, x_dtype, weight, weight_dtype, bias, bias_dtype,
                    seq_idx, initial_states, init_dtype, dout, dout_stride_b, dout_stride_t,
                    dfinal_states, dx, seqlen * dim, dim, dinitial_states, dweight, dbias,
                    aligned_to(workspace, 16), batch, seqlen, dim, width, silu, pl);
  if (rc) return rc;
  if (pl.need > 0 && (!workspace || workspace_bytes < pl.need))
    return fail(CCV1D_ERR_WORKSPACE, "workspace of %zu bytes given, %zu needed", workspace_bytes,
                pl.need);
  return run_bwd(pl, workspace, device, stream, timed);
}

int ccv1d_bwd_dx_strided(const void* x, int64_t x_stride_b, int64_t x_stride_t, int x_dtype,
                         const void* weight, int weight_dtype, const void* bias, int bias_dtype,
                         const int32_t* seq_idx, const void* initial_states, int init_dtype,
                         const void* dout, int64_t dout_stride_b, int64_t dout_stride_t,
                         const void* dfinal_states, void* dx, int64_t dx_stride_b,
                         int64_t dx_stride_t, void* dinitial_states, void* dweight, void* dbias,
                         void* workspace, size_t workspace_bytes, int64_t batch, int64_t seqlen,
                         int64_t dim, int64_t width, int silu, int device, void* stream) {
  g_last_error.clear();
  const bool timed = take_timing_request();
  if (dx_stride_b < 0 || dx_stride_t < 0) return fail(CCV1D_ERR_INVALID, "negative dx stride");
  BwdPlan pl;
  int rc = plan_bwd(x, x_stride_b, x_stride_t, x_dtype, weight, weight_dtype, bias, bias_dtype,
                    seq_idx, initial_states, init_dtype, dout, dout_stride_b, dout_stride_t,
                    dfinal_states, dx, dx_stride_b, dx_stride_t, dinitial_states, dweight, dbias,
                    aligned_to(workspace, 16), batch, seqlen, dim, width, silu, pl);
  if (rc) return rc;
  if (pl.need > 0 && (!workspace || workspace_bytes < pl.need))
    return fail(CCV1D_ERR_WORKSPACE, "workspace of %zu bytes given, %zu needed", workspace_bytes,
                pl.need);
  return run_bwd(pl, workspace, device, stream, timed);
}

int ccv1d_bwd_noalloc(const void* x, int64_t x_stride_b, int64_t x_stride_t, int x_dtype,
                      const void* weight, int weight_dtype, const void* bias, int bias_dtype,
                      const int32_t* seq_idx, const void* initial_states, int init_dtype,
                      const void* dout, int64_t dout_stride_b, int64_t dout_stride_t,
                      const void* dfinal_states, void* dx, void* dinitial_states, void* dweight,
                      void* dbias, int64_t batch, int64_t seqlen, int64_t dim, int64_t width,
                      int silu, int device, void* stream) {
  g_last_error.clear();
  const bool timed = take_timing_request();
  BwdPlan pl;
  // The scratch is 256-byte aligned, as the vectorised backward's partial rows require.
  int rc = plan_bwd(x, x_stride_b, x_stride_t, x_dtype, weight, weight_dtype, bias, bias_dtype,
                    seq_idx, initial_states, init_dtype, dout, dout_stride_b, dout_stride_t,
                    dfinal_states, dx, seqlen * dim, dim, dinitial_states, dweight, dbias, true,
                    batch, seqlen, dim, width, silu, pl);
  if (rc) return rc;
  if (pl.need > (size_t)CCV1D_NOALLOC_SCRATCH_BYTES)
    return fail(CCV1D_ERR_WORKSPACE,
                "ccv1d_bwd_noalloc: this shape needs %zu bytes of partial sums and the built-in "
                "scratch holds %zu; call ccv1d_bwd with a workspace instead",
                pl.need, (size_t)CCV1D_NOALLOC_SCRATCH_BYTES);
  if (pl.skip) return CCV1D_OK;
  void* ws = nullptr;
  {
    DeviceGuard guard(device);
    if (guard.err != hipSuccess) return hip_fail(guard.err, "hipSetDevice");
    rc = scratch_on_current_device(device, &ws);
    if (rc) return rc;
  }
  return run_bwd(pl, ws, device, stream, timed);
}

}  // extern "C"
