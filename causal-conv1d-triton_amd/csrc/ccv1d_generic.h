// Scalar kernels for what the vectorised path does not cover: widths above kMaxFastW (32), channel
// counts that are not a multiple of the channels per lane, rows not aligned to the vector access,
// and fp64 x. One lane
// owns one channel of one tile; the lanes of a wave cover 64 consecutive channels, so every row
// access is still coalesced. Also: the deterministic partial-sum reduction and the small fill/copy
// kernel used by the empty-sequence paths.
#pragma once

#include "ccv1d_device.h"

namespace ccv1d {

template <typename TX>
struct GenRow {
  const TX* xb;        // x[b, 0, c]
  int s_xt;
  const void* initb;   // initial_states[b, 0, c] (byte-offset pointer), or null
  int i_dt, P, D;
  // Row `row` (>= -P) of concat(initial_states, x) in fp32 (causal_conv1d.py:28-41).
  __device__ __forceinline__ float operator()(int row) const {
    if (row >= 0) return static_cast<float>(xb[row * s_xt]);
    if (initb) return ld_any(initb, (int64_t)(row + P) * D, i_dt);
    return 0.0f;
  }
};

__device__ __forceinline__ int dt_size(int dt) { return dt == DT_F64 ? 8 : dt == DT_F32 ? 4 : 2; }

// Pre-activation of row t (same operation order as conv_row).
template <typename TX>
__device__ __forceinline__ float gen_conv(const GenRow<TX>& xx, const void* w, int w_dt, int c,
                                          int W, const int32_t* sb, int T, bool has_init, int t,
                                          int32_t st) {
  const int P = W - 1;
  const int64_t wo = (int64_t)c * W;
  float z = ld_any(w, wo + P, w_dt) * xx(t);
  for (int k = 0; k < P; ++k) {
    const int r = t - P + k;
    if (sb && seq_at(sb, r, T, has_init) != st) continue;
    z = fmaf(ld_any(w, wo + k, w_dt), xx(r), z);
  }
  return z;
}

template <typename TX>
__global__ __launch_bounds__(64) void fwd_generic_kernel(const FwdParams p) {
  const int c = blockIdx.y * 64 + threadIdx.x;
  if (c >= p.D) return;
  const int tile = blockIdx.x % p.tl.nT;
  const int b = blockIdx.x / p.tl.nT;
  const int T = p.T, D = p.D, W = p.W, P = W - 1;
  const bool has_init = p.has_init;
  const int t0 = tile * p.tl.L;
  const int t1 = min(t0 + p.tl.L, T);
  GenRow<TX> xx;
  xx.xb = static_cast<const TX*>(p.x) + (int64_t)b * p.s_xb + c;
  xx.s_xt = p.s_xt;
  xx.initb = has_init ? static_cast<const char*>(p.init) + ((int64_t)b * P * D + c) * dt_size(p.i_dt)
                      : nullptr;
  xx.i_dt = p.i_dt;
  xx.P = P;
  xx.D = D;
  const int32_t* sb = p.seq ? p.seq + (int64_t)b * T : nullptr;
  const float bias = p.has_bias ? ld_any(p.bias, c, p.b_dt) : 0.0f;
  TX* ob = static_cast<TX*>(p.out) + (int64_t)b * T * D + c;
  const bool silu = p.silu;
  for (int t = t0; t < t1; ++t) {
    const int32_t st = sb ? sb[t] : 0;
    float z = gen_conv(xx, p.w, p.w_dt, c, W, sb, T, has_init, t, st);
    if (p.has_bias) z += bias;
    if (sb && st < 0) z = 0.0f;
    if (silu) z = z * sigmoid_f(z);
    ob[t * D] = to_store<TX>(z);
  }
  if (p.has_final && t1 == T) {
    TX* fb = static_cast<TX*>(p.fin) + (int64_t)b * P * D + c;
    for (int q = 0; q < P; ++q) fb[q * D] = to_store<TX>(xx(T - P + q));
  }
}

// Widths up to kGenericRingW: the forward and backward below keep the weights and the window of
// the last W rows in LDS (one column per lane), so each row of x is read from memory once and each
// weight once per tile, instead of once per tap. The arithmetic, its order and the results are
// those of the kernels above and below them.
constexpr int kGenericRingW = 128;

// LDS of the ring kernels, in bytes: NARR float arrays [W][64], plus the rows' sequence ids.
__host__ __device__ constexpr size_t generic_ring_bytes(int W, int narr) {
  return ((size_t)narr * W * 64 + W) * sizeof(float);
}

// Row slot of the ring: rows t0-P, t0-P+1, ... take slots 0, 1, ..., W-1, 0, ...
__device__ __forceinline__ int ring_next(int s, int W) { return s + 1 == W ? 0 : s + 1; }

template <typename TX>
__global__ __launch_bounds__(64) void fwd_generic_ring_kernel(const FwdParams p) {
  extern __shared__ float lds[];
  const int lane = threadIdx.x;
  const int c = blockIdx.y * 64 + lane;
  if (c >= p.D) return;
  const int tile = blockIdx.x % p.tl.nT;
  const int b = blockIdx.x / p.tl.nT;
  const int T = p.T, D = p.D, W = p.W, P = W - 1;
  const bool has_init = p.has_init;
  const int t0 = tile * p.tl.L;
  const int t1 = min(t0 + p.tl.L, T);
  GenRow<TX> xx;
  xx.xb = static_cast<const TX*>(p.x) + (int64_t)b * p.s_xb + c;
  xx.s_xt = p.s_xt;
  xx.initb = has_init ? static_cast<const char*>(p.init) + ((int64_t)b * P * D + c) * dt_size(p.i_dt)
                      : nullptr;
  xx.i_dt = p.i_dt;
  xx.P = P;
  xx.D = D;
  const int32_t* sb = p.seq ? p.seq + (int64_t)b * T : nullptr;
  float* wl = lds;                                    // weights [W][64]
  float* xr = lds + W * 64;                           // x rows [W][64], ring
  int32_t* sr = reinterpret_cast<int32_t*>(lds + 2 * W * 64);  // their sequence ids [W]
  for (int k = 0; k < W; ++k) wl[k * 64 + lane] = ld_any(p.w, (int64_t)c * W + k, p.w_dt);
  for (int q = 0; q < P; ++q) {
    xr[q * 64 + lane] = xx(t0 - P + q);
    if (sb) sr[q] = seq_at(sb, t0 - P + q, T, has_init);
  }
  const float bias = p.has_bias ? ld_any(p.bias, c, p.b_dt) : 0.0f;
  TX* ob = static_cast<TX*>(p.out) + (int64_t)b * T * D + c;
  int slot = P;  // slot of row t0
  constexpr int RB = 8;
  for (int tb = t0; tb < t1; tb += RB) {
    // The batch's rows are requested together (rows past t1 repeat the last one).
    float xa[RB];
    int32_t sa[RB];
#pragma unroll
    for (int i = 0; i < RB; ++i) {
      const int t = min(tb + i, t1 - 1);
      xa[i] = xx(t);
      sa[i] = sb ? sb[t] : 0;
    }
#pragma unroll
    for (int i = 0; i < RB; ++i) {
      const int t = tb + i;
      if (t >= t1) break;
      const int32_t st = sa[i];
      xr[slot * 64 + lane] = xa[i];
      if (sb) sr[slot] = st;
      // gen_conv's order: w[P] x[t], then taps k = 0 .. P-1 (rows t-P+k, slots slot+1+k mod W).
      float z = wl[P * 64 + lane] * xa[i];
      int s = ring_next(slot, W);
      for (int k = 0; k < P; ++k) {
        if (!sb || sr[s] == st) z = fmaf(wl[k * 64 + lane], xr[s * 64 + lane], z);
        s = ring_next(s, W);
      }
      if (p.has_bias) z += bias;
      if (sb && st < 0) z = 0.0f;
      if (p.silu) z = z * sigmoid_f(z);
      ob[(int64_t)t * D] = to_store<TX>(z);
      slot = ring_next(slot, W);
    }
  }
  if (p.has_final && t1 == T) {
    TX* fb = static_cast<TX*>(p.fin) + (int64_t)b * P * D + c;
    for (int q = 0; q < P; ++q) fb[q * D] = to_store<TX>(xx(T - P + q));
  }
}

// Backward, one lane per channel, widths up to kGenericRingW. The last W rows of x and of g (the
// gradient of the pre-activation) live in LDS rings that share their row slots, beside the weights
// and the dweight sums (each a [W][64] array, one column per lane) and the rows' sequence ids; so
// the width is a runtime value and each row of x and dout is read from memory once. Same row
// semantics and summation structure as bwd_fast_kernel; partial row = b * nT + tile.
template <typename TX>
__global__ __launch_bounds__(64) void bwd_generic_ring_kernel(const BwdParams p) {
  extern __shared__ float lds[];
  const int lane = threadIdx.x;
  const int c = blockIdx.y * 64 + lane;
  if (c >= p.D) return;
  const int tile = blockIdx.x % p.tl.nT;
  const int b = blockIdx.x / p.tl.nT;
  const int T = p.T, D = p.D, W = p.W, P = W - 1;
  const bool has_init = p.has_init;
  const bool silu = p.silu;
  const bool need_dinit = p.need_dinit;
  float* wl = lds;                                    // weights [W][64]
  float* xr = lds + W * 64;                           // x rows [W][64], ring
  float* gr = lds + 2 * W * 64;                       // g rows [W][64], same slots
  float* dwl = lds + 3 * W * 64;                      // dweight sums [W][64]
  int32_t* sr = reinterpret_cast<int32_t*>(lds + 4 * W * 64);  // the rows' sequence ids [W]
  const int64_t wo = (int64_t)c * W;
  for (int k = 0; k < W; ++k) {
    wl[k * 64 + lane] = ld_any(p.w, wo + k, p.w_dt);
    dwl[k * 64 + lane] = 0.0f;
    gr[k * 64 + lane] = 0.0f;
  }
  float db = 0.0f;

  GenRow<TX> xx;
  xx.xb = static_cast<const TX*>(p.x) + (int64_t)b * p.s_xb + c;
  xx.s_xt = p.s_xt;
  const int isz = dt_size(p.i_dt);
  xx.initb = has_init ? static_cast<const char*>(p.init) + ((int64_t)b * P * D + c) * isz : nullptr;
  xx.i_dt = p.i_dt;
  xx.P = P;
  xx.D = D;
  const TX* yb = static_cast<const TX*>(p.dy) + (int64_t)b * p.s_yb + c;
  TX* dxb = static_cast<TX*>(p.dx) + (int64_t)b * p.s_dxb + c;
  void* dinitb = need_dinit ? static_cast<char*>(p.dinit) + ((int64_t)b * P * D + c) * isz : nullptr;
  const TX* dfb = p.has_dfinal ? static_cast<const TX*>(p.dfin) + (int64_t)b * P * D + c : nullptr;
  const int32_t* sb = p.seq ? p.seq + (int64_t)b * T : nullptr;
  const float bias = p.has_bias ? ld_any(p.bias, c, p.b_dt) : 0.0f;

  const int t0 = tile * p.tl.L;
  const int own_end = min(t0 + p.tl.L, T);
  const int t_end = min(own_end + P, T);
  const int emit_lo = (tile == 0 && need_dinit) ? -P : t0;
  for (int q = 0; q < P; ++q) {
    xr[q * 64 + lane] = xx(t0 - P + q);
    if (sb) sr[q] = seq_at(sb, t0 - P + q, T, has_init);
  }

  // dx of `row` (slot `s0`; rows row .. row + P in the ring), plus dfinal; stores dx or dinit.
  auto emit = [&](int row, int s0) {
    const int32_t q0 = sb ? sr[s0] : 0;
    float dx = wl[P * 64 + lane] * gr[s0 * 64 + lane];
    int s = ring_next(s0, W);
    for (int j = 1; j <= P; ++j) {
      if (!sb || sr[s] == q0) dx = fmaf(wl[(P - j) * 64 + lane], gr[s * 64 + lane], dx);
      s = ring_next(s, W);
    }
    if (dfb) {
      const int f = row - (T - P);
      if (f >= 0 && f < P) dx += static_cast<float>(dfb[f * D]);
    }
    if (row >= 0) dxb[(int64_t)row * p.s_dxt] = to_store<TX>(dx);
    else st_any(dinitb, (int64_t)(row + P) * D, p.i_dt, dx);
  };

  int slot = P;  // slot of row tt
  constexpr int RB = 8;
  for (int tb = t0; tb < t_end; tb += RB) {
    float xa[RB], ya[RB];
    int32_t sa[RB];
#pragma unroll
    for (int i = 0; i < RB; ++i) {
      const int t = min(tb + i, t_end - 1);
      xa[i] = xx(t);
      ya[i] = static_cast<float>(yb[(int64_t)t * p.s_yt]);
      sa[i] = sb ? sb[t] : 0;
    }
#pragma unroll
    for (int i = 0; i < RB; ++i) {
      const int tt = tb + i;
      if (tt >= t_end) break;
      const int32_t st = sa[i];
      xr[slot * 64 + lane] = xa[i];
      if (sb) sr[slot] = st;
      float g = ya[i];
      if (silu) {
        float z = wl[P * 64 + lane] * xa[i];
        int s = ring_next(slot, W);
        for (int k = 0; k < P; ++k) {
          if (!sb || sr[s] == st) z = fmaf(wl[k * 64 + lane], xr[s * 64 + lane], z);
          s = ring_next(s, W);
        }
        if (p.has_bias) z += bias;
        g = dsilu_times(g, z);
      }
      if (sb && st < 0) g = 0.0f;
      gr[slot * 64 + lane] = g;
      if (tt < own_end) {
        int s = ring_next(slot, W);
        for (int k = 0; k < P; ++k) {
          if (!sb || sr[s] == st) dwl[k * 64 + lane] = fmaf(g, xr[s * 64 + lane], dwl[k * 64 + lane]);
          s = ring_next(s, W);
        }
        dwl[P * 64 + lane] = fmaf(g, xa[i], dwl[P * 64 + lane]);
        db += g;
      }
      // Row tt - P sits in the slot after tt's.
      if (tt - P >= emit_lo) emit(tt - P, ring_next(slot, W));
      slot = ring_next(slot, W);
    }
  }
  if (t_end == T) {
    // Rows past the end: g = 0 and sequence id -1.
    for (int q = 0; q < P; ++q) {
      gr[slot * 64 + lane] = 0.0f;
      if (sb) sr[slot] = -1;
      const int row = T + q - P;
      if (row >= emit_lo && row < own_end) emit(row, ring_next(slot, W));
      slot = ring_next(slot, W);
    }
  }

  float* pp = p.part + ((int64_t)b * p.tl.nT + tile) * (W + 1) * D + c;
  for (int k = 0; k < W; ++k) pp[(int64_t)k * D] = dwl[k * 64 + lane];
  if (p.has_bias) pp[(int64_t)W * D] = db;
}

// Backward for widths whose g ring would not fit LDS (above kMaxGenericW): the gradient g of the
// pre-activation goes to a fp32 buffer G (batch, seqlen, dim) in the workspace, and a second kernel
// forms dx and the dweight/dbias partial rows from it, so no on-chip storage grows with the width.
// Same row semantics, summation orders and partial-row layout as bwd_generic_ring_kernel.

// G[b, t, c] = dout * silu'(z) (or dout), 0 on padding rows (causal_conv1d.py:274-288).
template <typename TX>
__global__ __launch_bounds__(64) void bwd_g_kernel(const BwdParams p, float* G) {
  const int c = blockIdx.y * 64 + threadIdx.x;
  if (c >= p.D) return;
  const int tile = blockIdx.x % p.tl.nT;
  const int b = blockIdx.x / p.tl.nT;
  const int T = p.T, D = p.D, W = p.W, P = W - 1;
  const bool has_init = p.has_init;
  GenRow<TX> xx;
  xx.xb = static_cast<const TX*>(p.x) + (int64_t)b * p.s_xb + c;
  xx.s_xt = p.s_xt;
  xx.initb = has_init
                 ? static_cast<const char*>(p.init) + ((int64_t)b * P * D + c) * dt_size(p.i_dt)
                 : nullptr;
  xx.i_dt = p.i_dt;
  xx.P = P;
  xx.D = D;
  const TX* yb = static_cast<const TX*>(p.dy) + (int64_t)b * p.s_yb + c;
  const int32_t* sb = p.seq ? p.seq + (int64_t)b * T : nullptr;
  const float bias = p.has_bias ? ld_any(p.bias, c, p.b_dt) : 0.0f;
  float* gb = G + (int64_t)b * T * D + c;
  const int t0 = tile * p.tl.L;
  const int t1 = min(t0 + p.tl.L, T);
  for (int t = t0; t < t1; ++t) {
    const int32_t st = sb ? sb[t] : 0;
    float g = static_cast<float>(yb[(int64_t)t * p.s_yt]);
    if (p.silu) {
      float z = gen_conv(xx, p.w, p.w_dt, c, W, sb, T, has_init, t, st);
      if (p.has_bias) z += bias;
      g = dsilu_times(g, z);
    }
    if (sb && st < 0) g = 0.0f;
    gb[(int64_t)t * D] = g;
  }
}

// dx (and the initial-state gradient) of the tile's rows from G, and the tile's dweight/dbias
// partial row (row b * nT + tile of `part`). dweight is accumulated KB taps at a time: each block
// walks the tile's rows once, so g is read W / KB times per row instead of W times.
template <typename TX, int KB = 8>
__global__ __launch_bounds__(64) void bwd_wide_kernel(const BwdParams p, const float* G) {
  const int c = blockIdx.y * 64 + threadIdx.x;
  if (c >= p.D) return;
  const int tile = blockIdx.x % p.tl.nT;
  const int b = blockIdx.x / p.tl.nT;
  const int T = p.T, D = p.D, W = p.W, P = W - 1;
  const bool has_init = p.has_init;
  GenRow<TX> xx;
  xx.xb = static_cast<const TX*>(p.x) + (int64_t)b * p.s_xb + c;
  xx.s_xt = p.s_xt;
  const int isz = dt_size(p.i_dt);
  xx.initb = has_init ? static_cast<const char*>(p.init) + ((int64_t)b * P * D + c) * isz : nullptr;
  xx.i_dt = p.i_dt;
  xx.P = P;
  xx.D = D;
  TX* dxb = static_cast<TX*>(p.dx) + (int64_t)b * p.s_dxb + c;
  void* dinitb =
      p.need_dinit ? static_cast<char*>(p.dinit) + ((int64_t)b * P * D + c) * isz : nullptr;
  const TX* dfb = p.has_dfinal ? static_cast<const TX*>(p.dfin) + (int64_t)b * P * D + c : nullptr;
  const int32_t* sb = p.seq ? p.seq + (int64_t)b * T : nullptr;
  const float* gb = G + (int64_t)b * T * D + c;
  const int64_t wo = (int64_t)c * W;
  // g of row `row` of concat(initial_states, x): 0 outside [0, T).
  auto g_at = [&](int row) { return (row >= 0 && row < T) ? gb[(int64_t)row * D] : 0.0f; };

  const int t0 = tile * p.tl.L;
  const int own_end = min(t0 + p.tl.L, T);
  const int emit_lo = (tile == 0 && p.need_dinit) ? -P : t0;
  // dx[row] = w[P] g[row] + sum_{j=1..P} m_j w[P-j] g[row+j] (+ dfinal), causal_conv1d.py:290-311.
  for (int row = emit_lo; row < own_end; ++row) {
    const int32_t s0 = sb ? seq_at(sb, row, T, has_init) : 0;
    float dx = ld_any(p.w, wo + P, p.w_dt) * g_at(row);
    for (int j = 1; j <= P; ++j) {
      if (sb && seq_at(sb, row + j, T, has_init) != s0) continue;
      dx = fmaf(ld_any(p.w, wo + P - j, p.w_dt), g_at(row + j), dx);
    }
    if (dfb) {
      const int f = row - (T - P);
      if (f >= 0 && f < P) dx += static_cast<float>(dfb[(int64_t)f * D]);
    }
    if (row >= 0) dxb[(int64_t)row * p.s_dxt] = to_store<TX>(dx);
    else st_any(dinitb, (int64_t)(row + P) * D, p.i_dt, dx);
  }

  // dweight[c, k] over the tile's own rows, ascending t for every k (causal_conv1d.py:313-321).
  float* pp = p.part + ((int64_t)b * p.tl.nT + tile) * (W + 1) * D + c;
  for (int kb = 0; kb < W; kb += KB) {
    float acc[KB];
#pragma unroll
    for (int j = 0; j < KB; ++j) acc[j] = 0.0f;
    for (int t = t0; t < own_end; ++t) {
      const float g = gb[(int64_t)t * D];
      const int32_t st = sb ? sb[t] : 0;
#pragma unroll
      for (int j = 0; j < KB; ++j) {
        const int k = kb + j;
        if (k >= W) break;
        const int r = t - P + k;
        if (k < P && sb && seq_at(sb, r, T, has_init) != st) continue;
        acc[j] = fmaf(g, xx(r), acc[j]);
      }
    }
#pragma unroll
    for (int j = 0; j < KB; ++j)
      if (kb + j < W) pp[(int64_t)(kb + j) * D] = acc[j];
  }
  if (p.has_bias) {
    float db = 0.0f;
    for (int t = t0; t < own_end; ++t) db += gb[(int64_t)t * D];
    pp[(int64_t)W * D] = db;
  }
}

// dweight[d, k] = sum_p part[p, k, d] and dbias[d] = sum_p part[p, W, d] (causal_conv1d.py:344-374),
// in an order fixed by Pn alone: wave w of NWR adds rows w, w + NWR, ... in ascending order, then the
// NWR wave sums are added in wave order.
template <int NWR>
__global__ __launch_bounds__(NWR * 64) void reduce_partials_kernel(const ReduceParams p) {
  __shared__ float red[NWR][64];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int K = p.W + (p.has_bias ? 1 : 0);
  const int64_t N = (int64_t)K * p.D;
  const int64_t n = (int64_t)blockIdx.x * 64 + lane;
  const int64_t rs = (int64_t)(p.W + 1) * p.D;
  float acc = 0.0f;
  if (n < N) {
    const float* src = p.part + n;
    int q = wave;
    // All loads of a group of 8 rows are issued before the first add.
    for (; q + 7 * NWR < p.Pn; q += 8 * NWR) {
      float v[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) v[u] = src[(int64_t)(q + u * NWR) * rs];
#pragma unroll
      for (int u = 0; u < 8; ++u) acc += v[u];
    }
    // The wave's last 0-7 rows, also all requested before the first add (a loop of load-then-add
    // waited one memory round trip per row: 2 of them at B=4 T=512 D=1024, 32 partial rows). The
    // adds keep the row order and skip the rows past Pn.
    if (q < p.Pn) {
      float v[8];
#pragma unroll
      for (int u = 0; u < 8; ++u)
        if (q + u * NWR < p.Pn) v[u] = src[(int64_t)(q + u * NWR) * rs];
#pragma unroll
      for (int u = 0; u < 8; ++u)
        if (q + u * NWR < p.Pn) acc += v[u];
    }
  }
  red[wave][lane] = acc;
  __syncthreads();
  if (wave == 0 && n < N) {
    float s = red[0][lane];
#pragma unroll
    for (int w = 1; w < NWR; ++w) s += red[w][lane];
    const int k = (int)(n / p.D);
    const int d = (int)(n % p.D);
    if (k < p.W) st_any(p.dw, (int64_t)d * p.W + k, p.w_dt, s);
    else st_any(p.db, d, p.b_dt, s);
  }
}

// dst[i] = src[i] converted between element types, or 0 when src is null (used instead of
// hipMemsetAsync so the paths stay valid inside captured graphs).
__global__ __launch_bounds__(256) void fill_kernel(void* dst, int dst_dt, const void* src, int src_dt,
                                                   int64_t n) {
  const bool same = src && src_dt == dst_dt;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) {
    if (same && dst_dt == DT_F64) static_cast<double*>(dst)[i] = static_cast<const double*>(src)[i];
    else st_any(dst, i, dst_dt, src ? ld_any(src, i, src_dt) : 0.0f);
  }
}

}  // namespace ccv1d
