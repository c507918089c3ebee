// Vectorised forward and backward kernels for compile-time widths (2..8), channels-last x whose
// rows are 16-byte aligned.
//
// Work decomposition (both passes): a lane owns VEC = 16 / sizeof(x) consecutive channels, a wave
// owns 64 such channel vectors (1 KiB of one row) over a tile of L consecutive rows, and a workgroup
// holds NW waves on consecutive tiles of the same channel range. Each wave walks forward in time and
// keeps the previous width - 1 rows in registers, so every row of x is loaded once per tile plus a
// (width - 1)-row halo that the neighbouring tile of the same workgroup (same CU) or of the same XCD
// (see xcd_remap) has just loaded.
#pragma once

#include "ccv1d_device.h"

namespace ccv1d {

// Row `row` (>= -P) of concat(initial_states, x) for this lane's VEC channels, in fp32
// (causal_conv1d.py:28-41). xb points at x[b, 0, c0], initb at initial_states[b, 0, c0].
template <typename TX, int VEC, int P>
__device__ __forceinline__ void load_row(const TX* xb, int s_xt, const void* initb, int i_dt,
                                         bool has_init, int D, int row, float (&f)[VEC]) {
  if (row >= 0) {
    Vec16<TX>::unpack(ld16(xb + row * s_xt), f);
  } else if (has_init) {
#pragma unroll
    for (int i = 0; i < VEC; ++i) f[i] = ld_any(initb, (int64_t)(row + P) * D + i, i_dt);
  } else {
#pragma unroll
    for (int i = 0; i < VEC; ++i) f[i] = 0.0f;
  }
}

// Weights (D, W) and bias (D) for channels c0 .. c0 + VEC - 1, in fp32.
template <int W, int VEC>
__device__ __forceinline__ void load_taps(const void* w, int w_dt, const void* bias, int b_dt,
                                          bool has_bias, int c0, float (&wv)[W][VEC],
                                          float (&bv)[VEC]) {
  if (w_dt == DT_F32) {
    const float* wp = static_cast<const float*>(w) + (int64_t)c0 * W;
#pragma unroll
    for (int i = 0; i < VEC; ++i)
#pragma unroll
      for (int k = 0; k < W; ++k) wv[k][i] = wp[i * W + k];
  } else {
#pragma unroll
    for (int i = 0; i < VEC; ++i)
#pragma unroll
      for (int k = 0; k < W; ++k) wv[k][i] = ld_any(w, (int64_t)(c0 + i) * W + k, w_dt);
  }
#pragma unroll
  for (int i = 0; i < VEC; ++i) bv[i] = has_bias ? ld_any(bias, c0 + i, b_dt) : 0.0f;
}

// Pre-activation of one row (causal_conv1d.py:129-138), in the reference's order:
//   z = w[P] * x[t]; z = fma(w[k], x[t-P+k], z) for k = 0..P-1 (masked by sequence equality);
//   z += bias; with ZERO_PAD, z = 0 on padding rows (sequence id < 0).
// xw holds rows t-P .. t-1, sw their sequence ids; xc is row t and st its sequence id.
template <int W, int VEC, bool SEQ, bool ZERO_PAD>
__device__ __forceinline__ void conv_row(const float (&wv)[W][VEC], const float (&bv)[VEC],
                                         bool has_bias, const float (&xw)[W - 1][VEC],
                                         const int32_t (&sw)[W - 1], const float (&xc)[VEC],
                                         int32_t st, float (&z)[VEC]) {
  constexpr int P = W - 1;
#pragma unroll
  for (int i = 0; i < VEC; ++i) z[i] = wv[P][i] * xc[i];
#pragma unroll
  for (int k = 0; k < P; ++k) {
    const bool m = !SEQ || sw[k] == st;
#pragma unroll
    for (int i = 0; i < VEC; ++i) {
      const float f = fmaf(wv[k][i], xw[k][i], z[i]);
      z[i] = m ? f : z[i];
    }
  }
  if (has_bias) {
#pragma unroll
    for (int i = 0; i < VEC; ++i) z[i] += bv[i];
  }
  if (SEQ && ZERO_PAD && st < 0) {
#pragma unroll
    for (int i = 0; i < VEC; ++i) z[i] = 0.0f;
  }
}

template <int P, int VEC>
__device__ __forceinline__ void shift_in(float (&win)[P][VEC], const float (&v)[VEC]) {
#pragma unroll
  for (int k = 0; k + 1 < P; ++k)
#pragma unroll
    for (int i = 0; i < VEC; ++i) win[k][i] = win[k + 1][i];
#pragma unroll
  for (int i = 0; i < VEC; ++i) win[P - 1][i] = v[i];
}

template <int P>
__device__ __forceinline__ void shift_in(int32_t (&win)[P], int32_t v) {
#pragma unroll
  for (int k = 0; k + 1 < P; ++k) win[k] = win[k + 1];
  win[P - 1] = v;
}

// =============================================================================================
// Forward: out = act(conv(x)) and final_states (causal_conv1d.py:44-164).
// =============================================================================================

template <typename TX, int W, bool SILU, bool SEQ>
struct FwdLane {
  static constexpr int VEC = Vec16<TX>::VEC;
  static constexpr int P = W - 1;
  float wv[W][VEC];
  float bv[VEC];
  float xw[P][VEC];   // rows t-P .. t-1
  int32_t sw[P];      // their sequence ids

  // One output row t from its input row xc (already unpacked) and sequence id st.
  __device__ __forceinline__ void step(bool has_bias, const float (&xc)[VEC], int32_t st, TX* orow) {
    float z[VEC];
    conv_row<W, VEC, SEQ, true>(wv, bv, has_bias, xw, sw, xc, st, z);
    if (SILU) {
#pragma unroll
      for (int i = 0; i < VEC; ++i) z[i] = z[i] * sigmoid_f(z[i]);
    }
    st16(orow, Vec16<TX>::pack(z));
    shift_in(xw, xc);
    if (SEQ) shift_in(sw, st);
  }
};

template <typename TX, int W, bool SILU, bool SEQ, int NW, int R>
__global__ __launch_bounds__(NW * 64) void fwd_fast_kernel(const FwdParams p) {
  using V = Vec16<TX>;
  constexpr int VEC = V::VEC;
  constexpr int P = W - 1;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int blk = xcd_remap(blockIdx.x, p.tl.nBlk);
  const int tb = blk % p.tl.nTB;
  const int rest = blk / p.tl.nTB;
  const int gw = rest % p.tl.nGW;
  const int b = rest / p.tl.nGW;
  const int tile = tb * NW + wave;
  if (tile >= p.tl.nT) return;
  const int grp = gw * 64 + lane;
  if (grp >= p.D / VEC) return;
  const int c0 = grp * VEC;
  const int T = p.T, D = p.D, s_xt = p.s_xt;
  const int t0 = tile * p.tl.L;
  const int t1 = min(t0 + p.tl.L, T);
  const bool has_bias = p.has_bias, has_init = p.has_init;

  const TX* xb = static_cast<const TX*>(p.x) + (int64_t)b * p.s_xb + c0;
  TX* ob = static_cast<TX*>(p.out) + (int64_t)b * T * D + c0;
  const int32_t* sb = SEQ ? p.seq + (int64_t)b * T : nullptr;
  const void* initb = nullptr;
  if (has_init) initb = static_cast<const char*>(p.init) +
                        ((int64_t)b * P * D + c0) * (p.i_dt == DT_F64 ? 8 : p.i_dt == DT_F32 ? 4 : 2);

  FwdLane<TX, W, SILU, SEQ> s;
  load_taps<W, VEC>(p.w, p.w_dt, p.bias, p.b_dt, has_bias, c0, s.wv, s.bv);
#pragma unroll
  for (int k = 0; k < P; ++k) {
    const int row = t0 - P + k;
    load_row<TX, VEC, P>(xb, s_xt, initb, p.i_dt, has_init, D, row, s.xw[k]);
    s.sw[k] = SEQ ? seq_at(sb, row, T, has_init) : 0;
  }

  int t = t0;
  // Full batches: the R row loads are issued together, ahead of the first use.
  for (; t + R <= t1; t += R) {
    uint4 raw[R];
    int32_t sr[R];
#pragma unroll
    for (int r = 0; r < R; ++r) raw[r] = ld16(xb + (t + r) * s_xt);
#pragma unroll
    for (int r = 0; r < R; ++r) sr[r] = SEQ ? sb[t + r] : 0;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      float xc[VEC];
      V::unpack(raw[r], xc);
      s.step(has_bias, xc, sr[r], ob + (t + r) * D);
    }
  }
  for (; t < t1; ++t) {
    float xc[VEC];
    V::unpack(ld16(xb + t * s_xt), xc);
    s.step(has_bias, xc, SEQ ? sb[t] : 0, ob + t * D);
  }

  // final_states = rows T-P .. T-1 of concat(initial_states, x) (causal_conv1d.py:153-164).
  if (p.has_final && t1 == T) {
    TX* fb = static_cast<TX*>(p.fin) + (int64_t)b * P * D + c0;
#pragma unroll
    for (int q = 0; q < P; ++q) {
      float f[VEC];
      load_row<TX, VEC, P>(xb, s_xt, initb, p.i_dt, has_init, D, T - P + q, f);
      st16(fb + q * D, V::pack(f));
    }
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
// -P..-1 (the initial-state gradient). dweight/dbias sums are combined across the workgroup's
// waves in LDS in wave order, and written as one fp32 partial row per workgroup.
// =============================================================================================

template <typename TX, int W, bool SILU, bool SEQ>
struct BwdLane {
  static constexpr int VEC = Vec16<TX>::VEC;
  static constexpr int P = W - 1;
  float wv[W][VEC];
  float bv[VEC];
  float xw[P][VEC];   // x rows t-P .. t-1
  float gw[P][VEC];   // g rows t-P .. t-1
  int32_t sw[P];      // sequence ids of rows t-P .. t-1
  float dw[W][VEC];
  float db[VEC];

  // dx of row `row` = t - P given g of row t (gt) and its sequence id (st), then the dfinal term.
  __device__ __forceinline__ void dx_row(const float (&gt)[VEC], int32_t st, float (&dx)[VEC]) {
#pragma unroll
    for (int i = 0; i < VEC; ++i) dx[i] = wv[P][i] * gw[0][i];
#pragma unroll
    for (int j = 1; j < P; ++j) {
      const bool m = !SEQ || sw[j] == sw[0];
#pragma unroll
      for (int i = 0; i < VEC; ++i) {
        const float f = fmaf(wv[P - j][i], gw[j][i], dx[i]);
        dx[i] = m ? f : dx[i];
      }
    }
    const bool m = !SEQ || st == sw[0];
#pragma unroll
    for (int i = 0; i < VEC; ++i) {
      const float f = fmaf(wv[0][i], gt[i], dx[i]);
      dx[i] = m ? f : dx[i];
    }
  }
};

template <typename TX, int W, bool SILU, bool SEQ, int NW, int R>
__global__ __launch_bounds__(NW * 64) void bwd_fast_kernel(const BwdParams p) {
  using V = Vec16<TX>;
  constexpr int VEC = V::VEC;
  constexpr int P = W - 1;
  __shared__ float red[(NW > 1 ? NW - 1 : 1) * (W + 1) * 64 * VEC];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int blk = xcd_remap(blockIdx.x, p.tl.nBlk);
  const int tb = blk % p.tl.nTB;
  const int rest = blk / p.tl.nTB;
  const int gwc = rest % p.tl.nGW;
  const int b = rest / p.tl.nGW;
  const int tile = tb * NW + wave;
  const int G = p.D / VEC;
  const int grp = gwc * 64 + lane;
  const int c0 = grp * VEC;
  const int T = p.T, D = p.D;
  const bool has_bias = p.has_bias;

  BwdLane<TX, W, SILU, SEQ> s;
#pragma unroll
  for (int k = 0; k < W; ++k)
#pragma unroll
    for (int i = 0; i < VEC; ++i) s.dw[k][i] = 0.0f;
#pragma unroll
  for (int i = 0; i < VEC; ++i) s.db[i] = 0.0f;

  if (tile < p.tl.nT && grp < G) {
    const int s_xt = p.s_xt, s_yt = p.s_yt;
    const bool has_init = p.has_init;
    const int t0 = tile * p.tl.L;
    const int own_end = min(t0 + p.tl.L, T);
    const int t_end = min(own_end + P, T);
    const int emit_lo = (tile == 0 && p.need_dinit) ? -P : t0;

    const TX* xb = static_cast<const TX*>(p.x) + (int64_t)b * p.s_xb + c0;
    const TX* yb = static_cast<const TX*>(p.dy) + (int64_t)b * p.s_yb + c0;
    TX* dxb = static_cast<TX*>(p.dx) + (int64_t)b * T * D + c0;
    const int32_t* sb = SEQ ? p.seq + (int64_t)b * T : nullptr;
    const int isz = p.i_dt == DT_F64 ? 8 : p.i_dt == DT_F32 ? 4 : 2;
    const void* initb = has_init
        ? static_cast<const void*>(static_cast<const char*>(p.init) + ((int64_t)b * P * D + c0) * isz)
        : nullptr;
    void* dinitb = p.need_dinit
        ? static_cast<void*>(static_cast<char*>(p.dinit) + ((int64_t)b * P * D + c0) * isz)
        : nullptr;
    const TX* dfb = p.has_dfinal ? static_cast<const TX*>(p.dfin) + (int64_t)b * P * D + c0 : nullptr;

    load_taps<W, VEC>(p.w, p.w_dt, p.bias, p.b_dt, has_bias, c0, s.wv, s.bv);
#pragma unroll
    for (int k = 0; k < P; ++k) {
      const int row = t0 - P + k;
      load_row<TX, VEC, P>(xb, s_xt, initb, p.i_dt, has_init, D, row, s.xw[k]);
      s.sw[k] = SEQ ? seq_at(sb, row, T, has_init) : 0;
#pragma unroll
      for (int i = 0; i < VEC; ++i) s.gw[k][i] = 0.0f;
    }

    // Stores dx of `row` (or its initial-state gradient when row < 0), adding dfinal first.
    auto emit = [&](int row, float (&dx)[VEC]) {
      if (dfb) {
        const int f = row - (T - P);
        if (f >= 0 && f < P) {
          float d[VEC];
          V::unpack(ld16(dfb + f * D), d);
#pragma unroll
          for (int i = 0; i < VEC; ++i) dx[i] += d[i];
        }
      }
      if (row >= 0) {
        st16(dxb + row * D, V::pack(dx));
      } else {
#pragma unroll
        for (int i = 0; i < VEC; ++i) st_any(dinitb, (int64_t)(row + P) * D + i, p.i_dt, dx[i]);
      }
    };

    auto step = [&](int tt, const float (&xc)[VEC], const float (&yc)[VEC], int32_t st) {
      float g[VEC];
      if (SILU) {
        float z[VEC];
        conv_row<W, VEC, SEQ, false>(s.wv, s.bv, has_bias, s.xw, s.sw, xc, st, z);
#pragma unroll
        for (int i = 0; i < VEC; ++i) g[i] = dsilu_times(yc[i], z[i]);
      } else {
#pragma unroll
        for (int i = 0; i < VEC; ++i) g[i] = yc[i];
      }
      if (SEQ && st < 0) {
#pragma unroll
        for (int i = 0; i < VEC; ++i) g[i] = 0.0f;
      }
      if (tt < own_end) {
#pragma unroll
        for (int k = 0; k < P; ++k) {
          const bool m = !SEQ || s.sw[k] == st;
#pragma unroll
          for (int i = 0; i < VEC; ++i) {
            const float f = fmaf(g[i], s.xw[k][i], s.dw[k][i]);
            s.dw[k][i] = m ? f : s.dw[k][i];
          }
        }
#pragma unroll
        for (int i = 0; i < VEC; ++i) {
          s.dw[P][i] = fmaf(g[i], xc[i], s.dw[P][i]);
          s.db[i] += g[i];
        }
      }
      const int row = tt - P;
      if (row >= emit_lo) {
        float dx[VEC];
        s.dx_row(g, st, dx);
        emit(row, dx);
      }
      shift_in(s.xw, xc);
      shift_in(s.gw, g);
      if (SEQ) shift_in(s.sw, st);
    };

    int t = t0;
    for (; t + R <= t_end; t += R) {
      uint4 rx[R], ry[R];
      int32_t sr[R];
#pragma unroll
      for (int r = 0; r < R; ++r) {
        rx[r] = ld16(xb + (t + r) * s_xt);
        ry[r] = ld16(yb + (t + r) * s_yt);
      }
#pragma unroll
      for (int r = 0; r < R; ++r) sr[r] = SEQ ? sb[t + r] : 0;
#pragma unroll
      for (int r = 0; r < R; ++r) {
        float xc[VEC], yc[VEC];
        V::unpack(rx[r], xc);
        V::unpack(ry[r], yc);
        step(t + r, xc, yc, sr[r]);
      }
    }
    for (; t < t_end; ++t) {
      float xc[VEC], yc[VEC];
      V::unpack(ld16(xb + t * s_xt), xc);
      V::unpack(ld16(yb + t * s_yt), yc);
      step(t, xc, yc, SEQ ? sb[t] : 0);
    }

    // Rows past the end of the sequence have g = 0 and sequence id -1; they complete the last P
    // dx rows when the tile reaches T.
    if (t_end == T) {
      float zero[VEC];
#pragma unroll
      for (int i = 0; i < VEC; ++i) zero[i] = 0.0f;
#pragma unroll
      for (int q = 0; q < P; ++q) {
        const int row = T + q - P;
        if (row >= emit_lo && row < own_end) {
          float dx[VEC];
#pragma unroll
          for (int i = 0; i < VEC; ++i) dx[i] = s.wv[P][i] * s.gw[0][i];
#pragma unroll
          for (int j = 1; j < P; ++j) {
            const bool m = !SEQ || s.sw[j] == s.sw[0];
#pragma unroll
            for (int i = 0; i < VEC; ++i) {
              const float f = fmaf(s.wv[P - j][i], s.gw[j][i], dx[i]);
              dx[i] = m ? f : dx[i];
            }
          }
          emit(row, dx);
        }
        shift_in(s.gw, zero);
        if (SEQ) shift_in(s.sw, -1);
      }
    }
  }

  // Workgroup sum of dweight/dbias in wave order 0, 1, ..., NW-1, then one partial row.
  constexpr int COLS = 64 * VEC;
  if (NW > 1) {
    if (wave > 0) {
      float* dst = red + (wave - 1) * (W + 1) * COLS + lane * VEC;
#pragma unroll
      for (int k = 0; k < W; ++k)
#pragma unroll
        for (int i = 0; i < VEC; ++i) dst[k * COLS + i] = s.dw[k][i];
#pragma unroll
      for (int i = 0; i < VEC; ++i) dst[W * COLS + i] = s.db[i];
    }
    __syncthreads();
  }
  if (wave == 0 && grp < G) {
#pragma unroll 1
    for (int wv = 1; wv < NW; ++wv) {
      const float* src = red + (wv - 1) * (W + 1) * COLS + lane * VEC;
#pragma unroll
      for (int k = 0; k < W; ++k)
#pragma unroll
        for (int i = 0; i < VEC; ++i) s.dw[k][i] += src[k * COLS + i];
#pragma unroll
      for (int i = 0; i < VEC; ++i) s.db[i] += src[W * COLS + i];
    }
    float* pp = p.part + ((int64_t)b * p.tl.nTB + tb) * (W + 1) * D + c0;
#pragma unroll
    for (int k = 0; k < W; ++k)
#pragma unroll
      for (int i = 0; i < VEC; i += 4)
        *reinterpret_cast<float4*>(pp + k * D + i) =
            make_float4(s.dw[k][i], s.dw[k][i + 1], s.dw[k][i + 2], s.dw[k][i + 3]);
    if (has_bias) {
#pragma unroll
      for (int i = 0; i < VEC; i += 4)
        *reinterpret_cast<float4*>(pp + W * D + i) =
            make_float4(s.db[i], s.db[i + 1], s.db[i + 2], s.db[i + 3]);
    }
  }
}

}  // namespace ccv1d
