// Vectorised forward and backward kernels for compile-time widths (2..kMaxFastW = 32) and
// channels-last x whose rows are aligned to the 2-, 4-, 8- or 16-byte access of CPL channels.
//
// Work decomposition (both passes): a lane owns CPL consecutive channels, a wave owns 64 such
// channel vectors over a tile of L consecutive rows, and a workgroup holds NW waves on consecutive
// tiles of the same channel range. Each wave walks its tile in time (the forward's odd tiles from
// the end) with a window of width - 1 rows in registers, so a row of x is loaded once per tile plus
// a (width - 1)-row halo that the
// neighbouring tile of the same workgroup (same CU) or of the same XCD (xcd_remap) has just read.
// Rows are processed in batches of R: the loads of batch k + 1 are issued before batch k is
// computed, so every wave keeps up to 2R rows of reads in flight while its ALUs work.
#pragma once

#include "ccv1d_device.h"

namespace ccv1d {

// Weights (D, W) and bias (D) for channels c0 .. c0 + CPL - 1, in fp32. Without a bias the bias
// registers hold -0.0, which leaves every z unchanged when added (x + (-0.0) == x bit for bit, also
// for x = +0.0 and -0.0), so the kernels add it unconditionally instead of selecting per element.
template <int W, int CPL>
__device__ __forceinline__ void load_taps(const void* w, int w_dt, const void* bias, int b_dt,
                                          bool has_bias, int c0, float (&wv)[W][CPL],
                                          float (&bv)[CPL]) {
  float flat[W * CPL];
  ld_vec_any<W * CPL>(w, (int64_t)c0 * W, w_dt, flat);
#pragma unroll
  for (int i = 0; i < CPL; ++i)
#pragma unroll
    for (int k = 0; k < W; ++k) wv[k][i] = flat[i * W + k];
  if (has_bias) {
    ld_vec_any<CPL>(bias, c0, b_dt, bv);
  } else {
#pragma unroll
    for (int i = 0; i < CPL; ++i) bv[i] = -0.0f;
  }
}

// Pre-activation of one row (causal_conv1d.py:129-138). In the reference's order:
//   z = w[P] * x[t]; z = fma(w[k], x[t-P+k], z) for k = 0..P-1 (masked by sequence equality);
//   z += bias (-0.0 without one); with ZERO_PAD, z = 0 on padding rows (sequence id < 0).
// With BIAS_FIRST the bias enters the first term instead, z = fma(w[P], x[t], bias), which saves
// the final add (a different rounding order: used where silu follows, whose results are held to
// tolerance; without an activation the forward keeps the reference's order bit for bit).
// xw holds rows t-P .. t-1, sw their sequence ids; xc is row t and st its sequence id.
template <int W, int CPL, bool SEQ, bool ZERO_PAD, bool BIAS_FIRST = false>
__device__ __forceinline__ void conv_row(const float (&wv)[W][CPL], const float (&bv)[CPL],
                                         const float (&xw)[W - 1][CPL],
                                         const int32_t (&sw)[W - 1], const float (&xc)[CPL],
                                         int32_t st, float (&z)[CPL]) {
  constexpr int P = W - 1;
#pragma unroll
  for (int i = 0; i < CPL; ++i) z[i] = BIAS_FIRST ? fmaf(wv[P][i], xc[i], bv[i]) : wv[P][i] * xc[i];
#pragma unroll
  for (int k = 0; k < P; ++k) {
    const bool m = !SEQ || sw[k] == st;
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
      const float f = fmaf(wv[k][i], xw[k][i], z[i]);
      z[i] = m ? f : z[i];
    }
  }
  if (!BIAS_FIRST) {
#pragma unroll
    for (int i = 0; i < CPL; ++i) z[i] += bv[i];
  }
  if (SEQ && ZERO_PAD && st < 0) {
#pragma unroll
    for (int i = 0; i < CPL; ++i) z[i] = 0.0f;
  }
}

template <int P, int CPL>
__device__ __forceinline__ void shift_in(float (&win)[P][CPL], const float (&v)[CPL]) {
#pragma unroll
  for (int k = 0; k + 1 < P; ++k)
#pragma unroll
    for (int i = 0; i < CPL; ++i) win[k][i] = win[k + 1][i];
#pragma unroll
  for (int i = 0; i < CPL; ++i) win[P - 1][i] = v[i];
}

template <int P>
__device__ __forceinline__ void shift_in(int32_t (&win)[P], int32_t v) {
#pragma unroll
  for (int k = 0; k + 1 < P; ++k) win[k] = win[k + 1];
  win[P - 1] = v;
}

// Workgroup -> (batch row, wave column, workgroup along time), with neighbouring time tiles kept
// on one XCD. The remapping works on chunks of kXcdChunk consecutive workgroup ids: a grid larger
// than what the device holds at once runs in waves of workgroups dispatched in id order, and within
// a chunk the logical blocks stay one contiguous range of the tensor (whole rows of a few batch
// rows), while a remap over the whole grid would spread every dispatch wave over all batch rows and
// half the channels. Measured on MI355X: at B=4 T=8192 D=4096 the step takes 246 us with chunks
// of 512 against 334 us with one remap over the grid; grids of at most 512 workgroups (the
// B=4 T=8192 D=1024 benchmark) are mapped as before.
//
// With Tiling::col_fast the wave columns of one range of rows are consecutive instead: where rows
// are not aligned to the 128-byte line (x a channel slice of a wider tensor, dx written into one),
// the lines at the column boundaries are shared by two columns, and with this order both columns
// touch them on the same XCD at about the same time. Measured at Mamba-2's in_proj slice (B=8
// T=4096 D=5376, row pitch 10576 channels, configuration 3): fwd+bwd 327 -> 320 us, backward with
// dx written into the in_proj gradient 256 -> 247 us (233 with non-temporal dx stores, see
// BwdCfg); on aligned rows the time-fastest order is faster (benchmark step 59.7 against 62.6 us,
// 11 of 13 mid-size shapes).
// Kernels of widths above kColFastMaxW (COL_FAST false) always take the time-fastest order: the
// branch cost the widest backward kernels up to 400 SGPR spills (W=32 step +4 us), and the slices
// it serves are measured at width 4.
constexpr int kXcdChunk = 512;
template <bool COL_FAST>
struct TileCoord {
  int b, gw, tb;
  __device__ __forceinline__ TileCoord(const Tiling& tl) {
    const int chunk = blockIdx.x / kXcdChunk;
    const int first = chunk * kXcdChunk;
    const int blk = first + xcd_remap(blockIdx.x - first, min(kXcdChunk, tl.nBlk - first));
    if (COL_FAST && tl.col_fast) {
      gw = blk % tl.nGW;
      const int rest = blk / tl.nGW;
      tb = rest % tl.nTB;
      b = rest / tl.nTB;
    } else {
      tb = blk % tl.nTB;
      const int rest = blk / tl.nTB;
      gw = rest % tl.nGW;
      b = rest / tl.nGW;
    }
  }
};

// Sequence ids of rows r0 .. r0 + 127 of concat(initial_states, x) (kRowIds rows), row r0 + j in
// lane j of `lo` (j < 64) or lane j - 64 of `hi`, read with two vector loads issued together. A tile
// and both its halos span at most 64 + 2 * 31 rows, so one RowIds serves every row a tile touches:
// at() gives the id of a row to the whole wave (v_readlane) without a load of its own, and no load
// of ids then sits in the tile's pipelined loop, where its wait would also cover the loads and
// stores issued before it.
static_assert(kRowIds == 128, "RowIds holds two 64-lane vectors");
struct RowIds {
  int32_t lo = 0, hi = 0;
  int r0 = 0;
  RowIds() = default;
  __device__ __forceinline__ RowIds(const int32_t* sb, int first, int T, bool has_init) : r0(first) {
    const int lane = threadIdx.x & 63;
    lo = seq_at(sb, r0 + lane, T, has_init);
    hi = seq_at(sb, r0 + 64 + lane, T, has_init);
  }
  // Id of row `row`, r0 <= row < r0 + kRowIds, row wave-uniform.
  __device__ __forceinline__ int32_t at(int row) const {
    const int j = row - r0;
    const int32_t a = __builtin_amdgcn_readlane(lo, j & 63);
    const int32_t b = __builtin_amdgcn_readlane(hi, j & 63);
    return j < 64 ? a : b;
  }
  // True when rows r0 .. r1-1 (r0 < r1 <= r0 + kRowIds) all carry the id of row r0. The wave votes
  // need every lane of the wave active (as in the two tests below).
  __device__ __forceinline__ bool one_id(int r1) const {
    const int lane = threadIdx.x & 63;
    const int32_t id0 = __builtin_amdgcn_readlane(lo, 0);
    bool ok = __all((r0 + lane < r1 ? lo : id0) == id0);
    ok = __all((r0 + 64 + lane < r1 ? hi : id0) == id0) && ok;
    return ok;
  }
  // One id and it is not padding (>= 0). Every sequence mask of such a tile is 1 and no row of it
  // is zeroed, so the tile can run the kernels' seq_idx-free code, which then gives bit-identical
  // results.
  __device__ __forceinline__ bool one_segment(int r1) const {
    return one_id(r1) && __builtin_amdgcn_readlane(lo, 0) >= 0;
  }
  // One id and it is padding (< 0): every mask is 1 and every row is zeroed (see bwd_tile's PAD).
  __device__ __forceinline__ bool one_padding_run(int r1) const {
    return one_id(r1) && __builtin_amdgcn_readlane(lo, 0) < 0;
  }
  // True when every row of [a, b) (r0 <= a, b <= r0 + kRowIds) carries a negative id.
  __device__ __forceinline__ bool all_padding(int a, int b) const {
    const int lane = threadIdx.x & 63;
    const int ra = r0 + lane, rb = r0 + 64 + lane;
    bool ok = __all(ra < a || ra >= b || lo < 0);
    ok = __all(rb < a || rb >= b || hi < 0) && ok;
    return ok;
  }
};

// =============================================================================================
// Forward: out = act(conv(x)) and final_states (causal_conv1d.py:44-164).
// =============================================================================================

template <typename TX, int W, bool SILU, bool SEQ, int CPL>
struct FwdLane {
  using IO = VecIO<TX, CPL>;
  using raw = typename IO::raw;
  static constexpr int P = W - 1;
  float wv[W][CPL];
  float bv[CPL];
  float xw[P][CPL];  // rows t-P .. t-1
  int32_t sw[P];     // their sequence ids

  // Output row t from its raw input row and sequence id.
  __device__ __forceinline__ raw row(const raw xr, int32_t st) {
    float xc[CPL], z[CPL];
    IO::unpack(xr, xc);
    conv_row<W, CPL, SEQ, true, SILU>(wv, bv, xw, sw, xc, st, z);
    if (SILU) {
#pragma unroll
      for (int i = 0; i < CPL; ++i) z[i] = z[i] * sigmoid_f(z[i]);
    }
    shift_in(xw, xc);
    if (SEQ) shift_in(sw, st);
    return IO::pack(z);
  }
};

// The same arithmetic for a walk towards earlier rows: xv holds rows t-P .. t of the output row t.
template <typename TX, int W, bool SILU, bool SEQ, int CPL>
struct FwdLaneRev {
  using IO = VecIO<TX, CPL>;
  using raw = typename IO::raw;
  static constexpr int P = W - 1;
  float wv[W][CPL];
  float bv[CPL];
  float xv[P + 1][CPL];  // rows t-P .. t
  int32_t sv[P + 1];     // their sequence ids

  // Output row t, then the window moves down one row: `xr` (row t-P-1, sequence id `st`) enters.
  __device__ __forceinline__ raw row(const raw xr, int32_t st) {
    float z[CPL];
    conv_row<W, CPL, SEQ, true, SILU>(wv, bv, reinterpret_cast<const float(&)[P][CPL]>(xv),
                                reinterpret_cast<const int32_t(&)[P]>(sv), xv[P], sv[P], z);
    if (SILU) {
#pragma unroll
      for (int i = 0; i < CPL; ++i) z[i] = z[i] * sigmoid_f(z[i]);
    }
#pragma unroll
    for (int k = P; k > 0; --k) {
#pragma unroll
      for (int i = 0; i < CPL; ++i) xv[k][i] = xv[k - 1][i];
      if (SEQ) sv[k] = sv[k - 1];
    }
    IO::unpack(xr, xv[0]);
    if (SEQ) sv[0] = st;
    return IO::pack(z);
  }
};

// One tile walked forward (rows t0 .. t1-1). Its halo rows, the first batch and the taps are requested
// together; then a ping-pong over two register batches keeps batch k + 1 in flight while batch k is
// computed. Rows past the tile end are clamped to its last row: a duplicate read keeps the number of
// loads in flight independent of the tile length, so the compiler's wait counts stay exact.
// Double batches (2R rows) per pass of a pipelined row loop: the fewest that make a pass longer
// than the window of P rows, so each window value live at the loop's back edge was produced in the
// pass and no register moves are needed there. Kernels of 2-row batches keep one (the seq_idx
// kernels were slower with more: configuration 5 at W=7 511 -> 523 us; the 4-channel backward at
// width 5 spilled).
template <bool SEQ, int R, int P>
constexpr int pass_batches() {
  return (!SEQ && R == 4) ? P / (2 * R) + 1 : 1;
}

template <typename TX, int W, bool SILU, bool SEQ, int CPL, int R, int XLD, int OST, bool DRAIN>
__device__ __forceinline__ void fwd_tile_forward(const FwdParams& p, const RowBuf<TX, CPL, XLD>& X,
                                                 const RowBuf<TX, CPL, kCachePlain, OST>& O,
                                                 const RowIds& ids, int c0, int t0, int t1,
                                                 int64_t init_off, TX* fin) {
  using IO = VecIO<TX, CPL>;
  using raw = typename IO::raw;
  constexpr int P = W - 1;
  const int D = p.D;
  const bool halo_in_x = t0 >= P;
  raw hr[P];
  if (halo_in_x) {
#pragma unroll
    for (int k = 0; k < P; ++k) hr[k] = X.ld(t0 - P + k);
  }
  raw A[R], B[R];
  int32_t sA[R], sB[R];
  auto load = [&](raw (&buf)[R], int32_t (&sq)[R], int t) {
#pragma unroll
    for (int r = 0; r < R; ++r) buf[r] = X.ld(min(t + r, t1 - 1));
#pragma unroll
    for (int r = 0; r < R; ++r) sq[r] = SEQ ? ids.at(min(t + r, t1 - 1)) : 0;
  };
  load(A, sA, t0);

  FwdLane<TX, W, SILU, SEQ, CPL> s;
  load_taps<W, CPL>(p.w, p.w_dt, p.bias, p.b_dt, p.has_bias, c0, s.wv, s.bv);
  // Every tile is at least min_tile_rows(W) > P rows long (the host's tiling, min_tile_rows in
  // ccv1d_api.hip), so a tile starts at row 0 or at a row >= P: a window not in x is the first
  // tile's, the P initial-state rows (or zeros).
  if (halo_in_x) {
#pragma unroll
    for (int k = 0; k < P; ++k) IO::unpack(hr[k], s.xw[k]);
  } else if (p.has_init) {
    ld_rows_any<P, CPL>(p.init, init_off, D, p.i_dt, s.xw);
  } else {
#pragma unroll
    for (int k = 0; k < P; ++k)
#pragma unroll
      for (int i = 0; i < CPL; ++i) s.xw[k][i] = 0.0f;
  }
#pragma unroll
  for (int k = 0; k < P; ++k) s.sw[k] = SEQ ? ids.at(t0 - P + k) : 0;

  auto compute = [&](const raw (&buf)[R], const int32_t (&sq)[R], int t) {
#pragma unroll
    for (int r = 0; r < R; ++r) O.st(t + r, s.row(buf[r], sq[r]));
  };
  int t = t0;
  // DRAIN: wait here for every request in flight (halo, first batch, taps). The compiler's wait at
  // the loop head merges this entry, where the first batch is the newest request, with the loop's
  // back edge, and without this wait it waits there for everything, the previous iteration's
  // stores included, every 2R rows; after it, the head waits only for the batch it needs.
  if (DRAIN) __builtin_amdgcn_s_waitcnt(0);
  // Passes of U double batches, so the window needs no register moves at the loop's back edge
  // (pass_batches; forward alone at B=4 T=8192 D=1024: W=12 30.2 -> 29.9 us, W=16 32.8 -> 32.2,
  // W=24 39.1 -> 37.9, W=32 45.7 -> 44.2).
  constexpr int U = pass_batches<SEQ, R, P>();
  if constexpr (U > 1) {
    for (; t + 2 * R * U <= t1; t += 2 * R * U) {
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int tu = t + 2 * R * u;
        load(B, sB, tu + R);
        compute(A, sA, tu);
        load(A, sA, tu + 2 * R);
        compute(B, sB, tu + R);
      }
    }
  }
  for (; t + 2 * R <= t1; t += 2 * R) {
    load(B, sB, t + R);
    compute(A, sA, t);
    load(A, sA, t + 2 * R);
    compute(B, sB, t + R);
  }
  if (t + R <= t1) {
    compute(A, sA, t);
    t += R;
  }
  for (; t < t1; ++t) O.st(t, s.row(X.ld(t), SEQ ? ids.at(t) : 0));
  // final_states of the tile ending at T: the window now holds rows T-P .. T-1 of
  // concat(initial_states, x) in fp32, exact copies of x.dtype values or converted initial states.
  if (fin) {
#pragma unroll
    for (int k = 0; k < P; ++k) IO::st(fin + (int64_t)k * D, IO::pack(s.xw[k]));
  }
}

// One tile walked backward (outputs t1-1 down to t0), for tiles with t0 >= min_tile_rows(W) > P,
// whose rows all lie in x. The window starts as rows t1-1-P .. t1-1; output t then takes in row t-P-1. Rows below
// t0-P are clamped to t0-P, for the same reason as the clamp of the forward walk.
template <typename TX, int W, bool SILU, bool SEQ, int CPL, int R, int XLD, int OST, bool DRAIN>
__device__ __forceinline__ void fwd_tile_reverse(const FwdParams& p, const RowBuf<TX, CPL, XLD>& X,
                                                 const RowBuf<TX, CPL, kCachePlain, OST>& O,
                                                 const RowIds& ids, int c0, int t0, int t1,
                                                 TX* fin) {
  using IO = VecIO<TX, CPL>;
  using raw = typename IO::raw;
  constexpr int P = W - 1;
  const int lo = t0 - P;
  raw wr[P + 1];
#pragma unroll
  for (int k = 0; k <= P; ++k) wr[k] = X.ld(t1 - 1 - P + k);
  // final_states of the tile ending at T: rows T-P .. T-1, all in x here, are wr[1..P].
  if (fin) {
#pragma unroll
    for (int k = 0; k < P; ++k) IO::st(fin + (int64_t)k * p.D, wr[k + 1]);
  }
  raw A[R], B[R];
  int32_t sA[R], sB[R];
  auto load = [&](raw (&buf)[R], int32_t (&sq)[R], int row) {
#pragma unroll
    for (int r = 0; r < R; ++r) buf[r] = X.ld(max(row - r, lo));
#pragma unroll
    for (int r = 0; r < R; ++r) sq[r] = SEQ ? ids.at(max(row - r, lo)) : 0;
  };
  load(A, sA, t1 - 2 - P);

  FwdLaneRev<TX, W, SILU, SEQ, CPL> s;
  load_taps<W, CPL>(p.w, p.w_dt, p.bias, p.b_dt, p.has_bias, c0, s.wv, s.bv);
#pragma unroll
  for (int k = 0; k <= P; ++k) {
    IO::unpack(wr[k], s.xv[k]);
    s.sv[k] = SEQ ? ids.at(t1 - 1 - P + k) : 0;
  }

  auto compute = [&](const raw (&buf)[R], const int32_t (&sq)[R], int t) {
#pragma unroll
    for (int r = 0; r < R; ++r) O.st(t - r, s.row(buf[r], sq[r]));
  };
  int t = t1 - 1;  // next output row
  if (DRAIN) __builtin_amdgcn_s_waitcnt(0);  // as in fwd_tile_forward
  constexpr int U = pass_batches<SEQ, R, P>();  // as in fwd_tile_forward
  if constexpr (U > 1) {
    for (; t - 2 * R * U + 1 >= t0; t -= 2 * R * U) {
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int tu = t - 2 * R * u;
        load(B, sB, tu - R - P - 1);
        compute(A, sA, tu);
        load(A, sA, tu - 2 * R - P - 1);
        compute(B, sB, tu - R);
      }
    }
  }
  for (; t - 2 * R + 1 >= t0; t -= 2 * R) {
    load(B, sB, t - R - P - 1);
    compute(A, sA, t);
    load(A, sA, t - 2 * R - P - 1);
    compute(B, sB, t - R);
  }
  if (t - R + 1 >= t0) {
    compute(A, sA, t);
    t -= R;
  }
  for (; t >= t0; --t) {
    const int row = max(t - P - 1, lo);
    O.st(t, s.row(X.ld(row), SEQ ? ids.at(row) : 0));
  }
}

// Even tiles walk forward and odd tiles backward. A tile's last P rows are the next tile's halo:
// with alternating directions both tiles read those rows at about the same time (both at their
// start, or both at their end), so the second read finds them in L2 instead of memory.
//
// 16-bit instances without seq_idx are compiled for 4 waves per SIMD (at most 128 VGPRs): width 16
// (2 channels per lane) needs 134 otherwise, which leaves one 8-wave workgroup per CU (B=4 T=8192
// D=1024 forward 42.2 -> 34.9 us; 2 VGPRs spill), as did width 8 when it took 4 channels per lane.
// The other widths already fit; the seq_idx and fp32 instances would spill more, so they keep the
// default bound.
template <typename TX, int W, bool SEQ>
constexpr int fwd_waves_per_simd() {
  return (sizeof(TX) == 2 && !SEQ) ? 4 : 2;
}

template <typename TX, int W, bool SILU, bool SEQ, int CPL, int NW, int R, int XLD, int OST>
__global__ __launch_bounds__(NW * 64, (fwd_waves_per_simd<TX, W, SEQ>())) void fwd_fast_kernel(
    const FwdParams p) {
  using IO = VecIO<TX, CPL>;
  constexpr int P = W - 1;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const TileCoord<(W <= kColFastMaxW)> tc(p.tl);
  const int tile = tc.tb * NW + wave;
  if (tile >= p.tl.nT) return;
  const int T = p.T, D = p.D;
  const int t0 = tile * p.tl.L;
  const int t1 = min(t0 + p.tl.L, T);
  // Ids of rows t0-P .. t0-P+127, which cover the tile and its halo (SEQ). A tile inside one segment
  // runs the seq_idx-free code (decided before any lane leaves).
  const RowIds ids = SEQ ? RowIds(p.seq + (int64_t)tc.b * T, t0 - P, T, p.has_init) : RowIds();
  const bool masked = SEQ && !ids.one_segment(t1);
  // A tile of padding rows only: z = 0 on every row, so every output is silu(0) = +0 (or +0 without
  // an activation), whatever x holds.
  const bool pad = masked && ids.all_padding(t0, t1);
  const int grp = tc.gw * 64 + lane;
  if (grp >= p.D / CPL) return;
  const int c0 = grp * CPL;

  const RowBuf<TX, CPL, XLD> X(static_cast<const TX*>(p.x) + (int64_t)tc.b * p.s_xb, p.x_bytes, c0,
                               p.s_xt);
  const RowBuf<TX, CPL, kCachePlain, OST> O(static_cast<const TX*>(p.out) + (int64_t)tc.b * T * D,
                                            p.o_bytes, c0, D);
  const int64_t init_off = (int64_t)tc.b * P * D + c0;
  // final_states (causal_conv1d.py:153-164) come from the registers of the tile ending at T.
  TX* const fin = (p.has_final && t1 == T) ? static_cast<TX*>(p.fin) + init_off : nullptr;

  if (SEQ && pad) {
    float zero[CPL];
#pragma unroll
    for (int i = 0; i < CPL; ++i) zero[i] = 0.0f;
    const typename IO::raw zr = IO::pack(zero);
    for (int t = t0; t < t1; ++t) O.st(t, zr);
    return;
  }

  // The wait before the pipelined loop (DRAIN, see fwd_tile_forward) in kernels without seq_idx:
  // B=4 D=1024 forward alone T=512 4.15 -> 4.03 us, 256-token chunks 9.40 -> 9.23, decode 2.60 ->
  // 2.49; benchmark step 60.9 -> 60.5 us. The seq_idx kernels are 0.7 % slower with it
  // (configuration 5), and keep the compiler's placement.
  constexpr bool DRAIN = !SEQ;
  if (masked) {
    if (tile & 1)
      fwd_tile_reverse<TX, W, SILU, SEQ, CPL, R, XLD, OST, DRAIN>(p, X, O, ids, c0, t0, t1, fin);
    else
      fwd_tile_forward<TX, W, SILU, SEQ, CPL, R, XLD, OST, DRAIN>(p, X, O, ids, c0, t0, t1,
                                                                  init_off, fin);
  } else {
    if (tile & 1)
      fwd_tile_reverse<TX, W, SILU, false, CPL, R, XLD, OST, DRAIN>(p, X, O, ids, c0, t0, t1, fin);
    else
      fwd_tile_forward<TX, W, SILU, false, CPL, R, XLD, OST, DRAIN>(p, X, O, ids, c0, t0, t1,
                                                                    init_off, fin);
  }
}

// =============================================================================================
// Backward (causal_conv1d.py:167-341).
//
// Per row t (forward walk): recompute z exactly as the forward does, g = dout * silu'(z) (zero on
// padding rows), accumulate dweight/dbias over the tile's own rows, and complete
//   dx[t-P] = w[P] g[t-P] + sum_{j=1..P} m_j w[P-j] g[t-P+j]     (+ dfinal where it applies)
// whose last term needs the current row. The tile runs P rows past its end (right halo) so its
// last P dx rows are complete; those halo rows add nothing to dweight. Tile 0 also emits rows
// -P..-1 (the initial-state gradient). The first P rows of a tile (where those initial-state rows
// and the rows of the previous tile come out) and the rows past T (where dfinal enters) are handled
// outside the pipelined loop, whose every step therefore ends in one plain dx store.
// dweight/dbias sums are combined across the workgroup's waves in LDS in wave order and written as
// one fp32 partial row per workgroup.
// =============================================================================================

// Keeps each value in a VGPR as it is (an empty asm with a read-write register operand): the
// compiler can no longer fold the instruction that produced it into its users.
template <int N>
__device__ __forceinline__ void pin_vgprs(float (&f)[N]) {
#pragma unroll
  for (int i = 0; i < N; ++i) asm("" : "+v"(f[i]));
}

// PAD: every row the lane sees is padding of one sequence id, so g = 0 on every row and every mask
// is 1: the arithmetic of the masked code on such rows, without dout or the activation.
template <typename TX, int W, bool SILU, bool SEQ, int CPL, bool PAD = false>
struct BwdLane {
  using IO = VecIO<TX, CPL>;
  using raw = typename IO::raw;
  static constexpr int P = W - 1;
  float wv[W][CPL];
  float bv[CPL];
  float xw[P][CPL];   // x rows t-P .. t-1
  float gw[P][CPL];   // g rows t-P .. t-1
  int32_t sw[P];      // sequence ids of rows t-P .. t-1
  float dw[W][CPL];
  float db[CPL];
  int own_end;

  // dx of row t - P, given g of row t (gt) and its sequence id (st).
  __device__ __forceinline__ void dx_row(const float (&gt)[CPL], int32_t st, bool with_last,
                                         float (&dx)[CPL]) const {
#pragma unroll
    for (int i = 0; i < CPL; ++i) dx[i] = wv[P][i] * gw[0][i];
#pragma unroll
    for (int j = 1; j < P; ++j) {
      const bool m = !SEQ || sw[j] == sw[0];
#pragma unroll
      for (int i = 0; i < CPL; ++i) {
        const float f = fmaf(wv[P - j][i], gw[j][i], dx[i]);
        dx[i] = m ? f : dx[i];
      }
    }
    if (with_last) {
      const bool m = !SEQ || st == sw[0];
#pragma unroll
      for (int i = 0; i < CPL; ++i) {
        const float f = fmaf(wv[0][i], gt[i], dx[i]);
        dx[i] = m ? f : dx[i];
      }
    }
  }

  // One row t = tt: g, dweight/dbias (own rows), and dx of row tt - P in `dx`; shifts the windows.
  __device__ __forceinline__ void step(int tt, const raw xr, const raw yr, int32_t st,
                                       float (&dx)[CPL]) {
    float xc[CPL], g[CPL];
    IO::unpack(xr, xc);
    if (PAD) {
#pragma unroll
      for (int i = 0; i < CPL; ++i) g[i] = 0.0f;
    } else {
      IO::unpack(yr, g);
    }
    if constexpr (__is_same(TX, _Float16) && CPL * sizeof(TX) == 4) {
      // fp16 rows of 2 channels: the converted values are pinned to registers as they are, so
      // the compiler neither folds the conversions into mixed-precision multiply-adds nor reuses
      // registers in a way that makes each pipelined batch wait for the previous batch's dx
      // stores (its loop head drained the memory counter to the stores). fp16 fwd+bwd, B=4 D=1024
      // W=4: weight only T=512 13.7 -> 12.5 us, T=2048 22.35 -> 21.2; bias + silu 0.05-0.2 us.
      pin_vgprs(xc);
      if (!PAD) pin_vgprs(g);
    }
    if (SILU && !PAD) {
      // wv and bv hold -log2(e) times the weights and bias: y = -log2(e) * z, and g is the
      // scaled gradient -ln2 * dout * silu'(z) (dsilu_scaled).
      float y[CPL];
      conv_row<W, CPL, SEQ, false, true>(wv, bv, xw, sw, xc, st, y);
#pragma unroll
      for (int i = 0; i < CPL; ++i) g[i] = dsilu_scaled(g[i], y[i]);
    }
    if (SEQ && st < 0) {
#pragma unroll
      for (int i = 0; i < CPL; ++i) g[i] = 0.0f;
    }
    if (tt < own_end) {
#pragma unroll
      for (int k = 0; k < P; ++k) {
        const bool m = !SEQ || sw[k] == st;
#pragma unroll
        for (int i = 0; i < CPL; ++i) {
          const float f = fmaf(g[i], xw[k][i], dw[k][i]);
          dw[k][i] = m ? f : dw[k][i];
        }
      }
#pragma unroll
      for (int i = 0; i < CPL; ++i) {
        dw[P][i] = fmaf(g[i], xc[i], dw[P][i]);
        db[i] += g[i];
      }
    }
    dx_row(g, st, true, dx);
    shift_in(xw, xc);
    shift_in(gw, g);
    if (SEQ) shift_in(sw, st);
  }
};

// Barrier for data exchanged through LDS only: waits for this wave's LDS operations, not for its
// global loads, so prefetches stay in flight across it.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Waves per SIMD the backward's register budget is sized for: 4 (at most 128 VGPRs) up to width 4
// and at width 5 with rows of at most 8 bytes (there the fp16 instance with seq_idx spills 16
// bytes per lane); otherwise 2 (at most 256), within which the instances' own allocation sets the
// occupancy (4-6 waves at widths 11-20 with one channel per lane, 2-3 from 21).
template <typename TX, int W, int CPL>
constexpr int bwd_waves_per_simd() {
  return (W <= 4 || (W == 5 && CPL * (int)sizeof(TX) <= 8)) ? 4 : 2;
}

// LDS of the backward: first the g values of every wave's first P rows (the right halo of the wave
// before it), later the dweight/dbias sums of every wave (at most 8 x 33 x 64 floats, 66 KiB, at
// width 32, whose kernels run one workgroup per CU; 40 KiB at width 4 with 4 channels per lane).
template <int W, int CPL, int NW>
constexpr int bwd_lds_floats() {
  constexpr int halo = NW * (W - 1) * 64 * CPL;
  constexpr int red = NW * (W + 1) * 64 * CPL;
  return halo > red ? halo : red;
}

// One wave's tile of the backward (the whole kernel but the choice of SEQ and PAD, see
// bwd_fast_kernel). PAD (with SEQ false): a tile inside one run of padding, which reads no dout.
template <typename TX, int W, bool SILU, bool SEQ, int CPL, int NW, int R, int XLD, int YLD, int DXST,
          bool PAD = false>
__device__ __forceinline__ void bwd_tile(const BwdParams& p, float* lds, const RowIds& ids) {
  using IO = VecIO<TX, CPL>;
  using raw = typename IO::raw;
  constexpr int P = W - 1;
  constexpr int COLS = 64 * CPL;

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const TileCoord<(W <= kColFastMaxW)> tc(p.tl);
  const int tile = tc.tb * NW + wave;
  const int G = p.D / CPL;
  const int grp = tc.gw * 64 + lane;
  const int c0 = grp * CPL;
  const int T = p.T, D = p.D;
  const bool active = tile < p.tl.nT && grp < G;
  const bool has_init = p.has_init;
  const int t0 = tile * p.tl.L;
  const int own_end = min(t0 + p.tl.L, T);
  // The next tile's first P rows of g come from its wave through LDS when it is in this workgroup;
  // otherwise this wave computes them itself (the right halo).
  const bool succ_here = wave < NW - 1 && tile + 1 < p.tl.nT;
  const int t_end = succ_here ? own_end : min(own_end + P, T);
  const int t_main = min(t0 + P, t_end);
  const int emit_lo = (tile == 0 && p.need_dinit) ? -P : t0;
  const int64_t state_off = (int64_t)tc.b * P * D + c0;
  // Sequence ids (SEQ): `ids` holds rows t0-P .. t0-P+127, which cover the tile and both halos.
  const TX* dfb = p.has_dfinal ? static_cast<const TX*>(p.dfin) + state_off : nullptr;
  const RowBuf<TX, CPL, XLD> X(static_cast<const TX*>(p.x) + (int64_t)tc.b * p.s_xb, p.x_bytes, c0, p.s_xt);
  const RowBuf<TX, CPL, YLD> Y(static_cast<const TX*>(p.dy) + (int64_t)tc.b * p.s_yb, p.y_bytes, c0, p.s_yt);
  const RowBuf<TX, CPL, kCachePlain, DXST> DX(static_cast<const TX*>(p.dx) + (int64_t)tc.b * p.s_dxb, p.o_bytes, c0, p.s_dxt);

  BwdLane<TX, W, SILU, SEQ, CPL, PAD> s;
  s.own_end = own_end;
#pragma unroll
  for (int k = 0; k < W; ++k)
#pragma unroll
    for (int i = 0; i < CPL; ++i) s.dw[k][i] = 0.0f;
#pragma unroll
  for (int i = 0; i < CPL; ++i) s.db[i] = 0.0f;

  // dx of `row` (or its initial-state gradient when row < 0), plus dfinal where it applies.
  auto emit_any = [&](int row, float (&dx)[CPL]) {
    if (row < emit_lo) return;
    if (dfb) {
      const int f = row - (T - P);
      if (f >= 0 && f < P) {
        float d[CPL];
        IO::unpack(IO::ld(dfb + f * D), d);
#pragma unroll
        for (int i = 0; i < CPL; ++i) dx[i] += d[i];
      }
    }
    if (row >= 0) DX.st(row, IO::pack(dx));
    else st_vec_any<CPL>(p.dinit, state_off + (int64_t)(row + P) * D, p.i_dt, dx);
  };

  raw Ax[R], Ay[R], Bx[R], By[R];
  auto load = [&](raw (&bx)[R], raw (&by)[R], int t) {
    // Rows past the end are clamped to the last row: a duplicate read keeps the number of loads in
    // flight fixed, so the compiler's wait counts stay exact.
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int row = min(t + r, t_end - 1);
      bx[r] = X.ld(row);
      by[r] = PAD ? raw{} : Y.ld(row);
    }
  };

  float* halo_out = lds + wave * P * COLS + lane * CPL;
  // The last NS rows of a wave whose pipelined rows number NS modulo R after its whole batches:
  // every wave with its successor in the workgroup, since tiles are a power of two >= 2R rows long
  // and the first P rows are peeled. Where a lane's rows are at most 4 bytes they are loaded with
  // the tile's first requests, so the tile's end does not wait for a load of its own: B=4 D=1024
  // fwd+bwd T=512 12.62 -> 12.31 us, T=2048 21.2 -> 20.9, B=4 T=8192 W=6 and 8 -0.3 to -0.5 us.
  // The 4-channel kernels keep the plain loads (benchmark step +0.12 us with them, 2 VGPRs per
  // row next to the 128 of 4 waves per SIMD), and so do widths from 9 (widths 10 and 19 went past
  // 128 VGPRs with them).
  constexpr int NS =
      (W <= 8 && CPL * sizeof(TX) <= 4) ? ((2 * R - P % (2 * R)) % (2 * R)) % R : 0;
  raw Sx[NS > 0 ? NS : 1], Sy[NS > 0 ? NS : 1];
  if (active) {
    // The halo rows, the tile's first P rows, the first pipelined batch and the taps are all
    // requested before anything waits on memory (rows past t_end are clamped to the last row).
    const bool halo_in_x = t0 >= P;
    raw hr[P], px[P], py[P];
    // Up to width 8 the rows a neighbouring wave reads again are loaded with the plain policy
    // (x's and dout's other loads are non-temporal, the first to be evicted), so they are still in
    // the L2 when it comes: the halo rows are also the last P rows of the previous tile, read at
    // the end of its walk, and the first wave's first P rows are the right halo of the previous
    // workgroup's last wave. Step B=4 T=8192 D=1024 bf16: W=4 60.6 -> 59.9 us (halo rows) -> 59.75
    // (first rows; plain first rows in every wave, which no other wave reads: 60.2), W=8 unchanged;
    // from W=9 the W-1 cached rows per tile cost more than they save (W=9 +0.5 us, W=32 +4 us).
    constexpr int HALO_LD = W <= 8 ? kCachePlain : XLD;
    constexpr int FIRST_YLD = W <= 8 ? kCachePlain : YLD;
    if (halo_in_x) {
#pragma unroll
      for (int k = 0; k < P; ++k) hr[k] = X.template ld<HALO_LD>(t0 - P + k);
    }
#pragma unroll
    for (int q = 0; q < P; ++q) {
      const int row = min(t0 + q, t_end - 1);
      if (W <= 8 && wave == 0) {
        px[q] = X.template ld<HALO_LD>(row);
        py[q] = PAD ? raw{} : Y.template ld<FIRST_YLD>(row);
      } else {
        px[q] = X.ld(row);
        py[q] = PAD ? raw{} : Y.ld(row);
      }
    }
    load(Ax, Ay, t_main);
    if constexpr (NS > 0) {
#pragma unroll
      for (int r = 0; r < NS; ++r) {
        const int row = max(t_end - NS + r, t0);
        Sx[r] = X.ld(row);
        Sy[r] = PAD ? raw{} : Y.ld(row);
      }
    }
    load_taps<W, CPL>(p.w, p.w_dt, p.bias, p.b_dt, p.has_bias, c0, s.wv, s.bv);
    if (SILU && !PAD) {
      // silu' in the base-2 domain (dsilu_scaled): weights and bias times -log2(e).
#pragma unroll
      for (int i = 0; i < CPL; ++i) {
#pragma unroll
        for (int k = 0; k < W; ++k) s.wv[k][i] *= kNegLog2e;
        s.bv[i] *= kNegLog2e;
      }
    }
    // Every tile is at least min_tile_rows(W) > P rows long (the host's tiling, min_tile_rows in
    // ccv1d_api.hip), so a tile starts at row 0 or at a row >= P: a window not in x is the first
    // tile's, the P initial-state rows (or zeros).
    if (halo_in_x) {
#pragma unroll
      for (int k = 0; k < P; ++k) IO::unpack(hr[k], s.xw[k]);
    } else if (has_init) {
      ld_rows_any<P, CPL>(p.init, state_off, D, p.i_dt, s.xw);
    } else {
#pragma unroll
      for (int k = 0; k < P; ++k)
#pragma unroll
        for (int i = 0; i < CPL; ++i) s.xw[k][i] = 0.0f;
    }
#pragma unroll
    for (int k = 0; k < P; ++k) {
      s.sw[k] = SEQ ? ids.at(t0 - P + k) : 0;
#pragma unroll
      for (int i = 0; i < CPL; ++i) s.gw[k][i] = 0.0f;
    }
    // The tile's first P rows: their dx rows belong to the previous tile (or are initial-state
    // rows), and their g values are the previous tile's right halo.
#pragma unroll
    for (int q = 0; q < P; ++q) {
      const int t = t0 + q;
      if (t < t_main) {
        float dx[CPL];
        s.step(t, px[q], py[q], SEQ ? ids.at(t) : 0, dx);
        emit_any(t - P, dx);
      }
#pragma unroll
      for (int i = 0; i < CPL; ++i) halo_out[q * COLS + i] = t < t_main ? s.gw[P - 1][i] : 0.0f;
    }
  }
  lds_barrier();

  if (active) {
    // Steady state: every step stores dx of row t - P, with t0 <= t - P < T - P.
    auto compute = [&](const raw (&bx)[R], const raw (&by)[R], int t) {
#pragma unroll
      for (int r = 0; r < R; ++r) {
        float dx[CPL];
        s.step(t + r, bx[r], by[r], SEQ ? ids.at(t + r) : 0, dx);
        DX.st(t + r - P, IO::pack(dx));
      }
    };
    int t = t_main;
    // Passes of U double batches (pass_batches). With 2RU > P rows per pass, every window value
    // live at the loop's back edge was produced in the pass, so the windows need no register moves
    // there (the 8-row pass at width 16 moved 30 registers per pass; 16-row passes: B=4 T=8192
    // D=1024 step W=9 71.4 -> 70.6 us, W=12 80.3 -> 79.4, W=16 92.9 -> 91.9; 24-row passes with
    // the forward's: W=24 128.5 -> 126.1). From width 25 the backward keeps 8-row passes (32-row
    // passes lost at W=32 what the forward's gained).
    constexpr int U = P < 6 * R ? pass_batches<SEQ, R, P>() : 1;
    if constexpr (U > 1) {
      for (; t + 2 * R * U <= t_end; t += 2 * R * U) {
#pragma unroll
        for (int u = 0; u < U; ++u) {
          const int tu = t + 2 * R * u;
          load(Bx, By, tu + R);
          compute(Ax, Ay, tu);
          load(Ax, Ay, tu + 2 * R);
          compute(Bx, By, tu + R);
        }
      }
    }
    for (; t + 2 * R <= t_end; t += 2 * R) {
      load(Bx, By, t + R);
      compute(Ax, Ay, t);
      load(Ax, Ay, t + 2 * R);
      compute(Bx, By, t + R);
    }
    if (t + R <= t_end) {
      compute(Ax, Ay, t);
      t += R;
    }
    if (NS > 0 && t_end - t == NS) {
#pragma unroll
      for (int r = 0; r < NS; ++r) {
        float dx[CPL];
        s.step(t + r, Sx[r], Sy[r], SEQ ? ids.at(t + r) : 0, dx);
        emit_any(t + r - P, dx);
      }
      t = t_end;
    }
    for (; t < t_end; ++t) {
      float dx[CPL];
      s.step(t, X.ld(t), PAD ? raw{} : Y.ld(t), SEQ ? ids.at(t) : 0, dx);
      emit_any(t - P, dx);
    }

    if (succ_here) {
      // The last P dx rows, from the next wave's g of rows own_end .. own_end + P - 1.
      const float* halo_in = lds + (wave + 1) * P * COLS + lane * CPL;
      if constexpr (W <= 8) {
        // All P rows are read from LDS before the first is used (read one by one, between the
        // stores of the rows before, each waited a round trip of its own), and their dx rows,
        // own_end - P .. own_end - 1, all lie in x (the tile is longer than P), so they skip the
        // initial-state branches. From width 9 the rows stay read one by one: the P x CPL registers
        // (and the changed schedule) took widths 19 and 20 past 128 VGPRs.
        float gh[P][CPL];
#pragma unroll
        for (int q = 0; q < P; ++q)
#pragma unroll
          for (int i = 0; i < CPL; ++i) gh[q][i] = halo_in[q * COLS + i];
#pragma unroll
        for (int q = 0; q < P; ++q) {
          const int tt = own_end + q;
          float dx[CPL];
          const int32_t st = SEQ ? ids.at(tt) : 0;
          s.dx_row(gh[q], st, true, dx);
          const int row = tt - P;
          if (dfb) {
            const int f = row - (T - P);
            if (f >= 0) {
              float d[CPL];
              IO::unpack(IO::ld(dfb + f * D), d);
#pragma unroll
              for (int i = 0; i < CPL; ++i) dx[i] += d[i];
            }
          }
          DX.st(row, IO::pack(dx));
          shift_in(s.gw, gh[q]);
          if (SEQ) shift_in(s.sw, st);
        }
      } else {
#pragma unroll
        for (int q = 0; q < P; ++q) {
          const int tt = own_end + q;
          float g[CPL], dx[CPL];
#pragma unroll
          for (int i = 0; i < CPL; ++i) g[i] = halo_in[q * COLS + i];
          const int32_t st = SEQ ? ids.at(tt) : 0;
          s.dx_row(g, st, true, dx);
          emit_any(tt - P, dx);
          shift_in(s.gw, g);
          if (SEQ) shift_in(s.sw, st);
        }
      }
    } else if (t_end == T) {
      // Rows past the end of the sequence have g = 0 and sequence id -1.
      float zero[CPL];
#pragma unroll
      for (int i = 0; i < CPL; ++i) zero[i] = 0.0f;
#pragma unroll
      for (int q = 0; q < P; ++q) {
        const int row = T + q - P;
        if (row < own_end) {
          float dx[CPL];
          s.dx_row(zero, -1, false, dx);
          emit_any(row, dx);
        }
        shift_in(s.gw, zero);
        if (SEQ) shift_in(s.sw, -1);
      }
    }
  }

  if (SILU && !PAD) {
    // The sums were accumulated from g~ = -ln2 * g (dsilu_scaled).
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
#pragma unroll
      for (int k = 0; k < W; ++k) s.dw[k][i] *= kNegLog2e;
      s.db[i] *= kNegLog2e;
    }
  }

  // Workgroup sum of dweight/dbias, then one partial row of W + 1 rows (dbias last). Every wave puts
  // its sums in LDS (the halo area is reused, after every wave has read its neighbour's halo), and
  // wave v sums rows v, v + NW, ... over the NW waves in wave order 0, 1, ..., NW-1 and stores
  // them. A row's reads are requested 4 waves at a time, so the workgroup's end waits two LDS round
  // trips where wave 0 alone, adding one wave's rows at a time, waited NW - 1 (all NW at once took
  // some instances past their register budget: width 5 with 4 channels per lane spilled, widths 19
  // and 20 went past 128 VGPRs).
  const int n_rows = p.has_bias ? W + 1 : W;
  if constexpr (NW > 1) {
    lds_barrier();
    float* dst = lds + wave * (W + 1) * COLS + lane * CPL;
#pragma unroll
    for (int k = 0; k < W; ++k)
#pragma unroll
      for (int i = 0; i < CPL; ++i) dst[k * COLS + i] = s.dw[k][i];
#pragma unroll
    for (int i = 0; i < CPL; ++i) dst[W * COLS + i] = s.db[i];
    lds_barrier();
    if (grp < G) {
      float* pp = p.part + ((int64_t)tc.b * p.tl.nTB + tc.tb) * (W + 1) * D + c0;
#pragma unroll 1
      for (int k = wave; k < n_rows; k += NW) {
        constexpr int VG = NW < 4 ? NW : 4;  // waves' rows read together
        static_assert(NW % VG == 0, "the groups of reads cover the workgroup's waves");
        float acc[CPL];
#pragma unroll
        for (int v0 = 0; v0 < NW; v0 += VG) {
          float c[VG][CPL];
#pragma unroll
          for (int v = 0; v < VG; ++v)
#pragma unroll
            for (int i = 0; i < CPL; ++i)
              c[v][i] = lds[((v0 + v) * (W + 1) + k) * COLS + lane * CPL + i];
#pragma unroll
          for (int v = 0; v < VG; ++v)
#pragma unroll
            for (int i = 0; i < CPL; ++i) acc[i] = (v0 + v == 0) ? c[v][i] : acc[i] + c[v][i];
        }
#pragma unroll
        for (int i = 0; i < CPL; ++i) pp[k * D + i] = acc[i];
      }
    }
  } else if (grp < G) {
    float* pp = p.part + ((int64_t)tc.b * p.tl.nTB + tc.tb) * (W + 1) * D + c0;
#pragma unroll
    for (int k = 0; k < W; ++k)
#pragma unroll
      for (int i = 0; i < CPL; ++i) pp[k * D + i] = s.dw[k][i];
    if (p.has_bias) {
#pragma unroll
      for (int i = 0; i < CPL; ++i) pp[W * D + i] = s.db[i];
    }
  }
}

// A wave whose tile (its rows and both halos, t0-P .. own_end+P-1) lies inside one non-padding
// segment runs the seq_idx-free instantiation of bwd_tile; one whose tile and halos, rows past T
// included (id -1), lie inside one run of padding runs the PAD instantiation (g = 0 on every row:
// no dout reads, no activation); the others run the masked one. All three have the same LDS
// barriers, so the waves of one workgroup may take different ones. The host keeps tiles short
// enough (L + 2 (W - 1) <= kRowIds) for one RowIds to cover a tile and its halos.
template <typename TX, int W, bool SILU, bool SEQ, int CPL, int NW, int R, int XLD, int YLD, int DXST>
__global__ __launch_bounds__(NW * 64, (bwd_waves_per_simd<TX, W, CPL>())) void bwd_fast_kernel(
    const BwdParams p) {
  __shared__ float lds[bwd_lds_floats<W, CPL, NW>()];
  if constexpr (SEQ) {
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const TileCoord<(W <= kColFastMaxW)> tc(p.tl);
    const int tile = tc.tb * NW + wave;
    const int t0 = tile * p.tl.L;
    const int r1 = min(t0 + p.tl.L + W - 1, p.T);
    const RowIds ids(p.seq + (int64_t)tc.b * p.T, t0 - (W - 1), p.T, p.has_init);
    // Evaluated on every path (its result is unused past the last tile), so that both id vectors
    // have arrived before either instantiation starts and no wait for them is left to its loop.
    const bool one = ids.one_segment(r1);
    const bool pad = ids.one_padding_run(t0 + p.tl.L + W - 1);
    if (tile < p.tl.nT && one) {
      bwd_tile<TX, W, SILU, false, CPL, NW, R, XLD, YLD, DXST>(p, lds, ids);
      return;
    }
    if (tile < p.tl.nT && pad) {
      bwd_tile<TX, W, false, false, CPL, NW, R, XLD, YLD, DXST, true>(p, lds, ids);
      return;
    }
    bwd_tile<TX, W, SILU, SEQ, CPL, NW, R, XLD, YLD, DXST>(p, lds, ids);
  } else {
    bwd_tile<TX, W, SILU, false, CPL, NW, R, XLD, YLD, DXST>(p, lds, RowIds());
  }
}

}  // namespace ccv1d
