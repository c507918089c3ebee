/*
 * ccv1d_oracle.c - CPU restatement of the reference's causal depthwise conv1d, forward and backward.
 *
 * TEST INFRASTRUCTURE ONLY. This file is the checker the GPU kernels are compared against. Only
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it, and never as the
 * thing measured or shipped: the product path (libccv1d.so) does not link, load or call it.
 *
 * Reference: jxiong21029/causal-conv1d-triton, causal_conv1d_triton/causal_conv1d.py. Each function
 * cites the lines it restates. The reference holds no golden vectors or known-answer tests; this
 * restatement is pinned instead by the checks in tests/test_oracle.py (closed-form grouped conv1d and
 * its autograd in float64, hand-derived known answers in tests/golden/, brute force on tiny inputs,
 * textbook special cases and bit-exact invariants), and tests/test_oracle_mutations.py shows that
 * each plausible mistake planted through ccv1d_oracle_set_mutation() fails at least one of them.
 *
 * Layout: every array is contiguous and fp32 (inputs already decoded from their storage type).
 *   x (B, T, D), weight (D, W), bias (D), seq (B, T) int32, init (B, P, D), P = W - 1.
 * Outputs are the fp32 values before the final cast to the output dtype, except dweight/dbias,
 * which are summed in double (the reference sums fp32 partials in an SM-count-dependent order,
 * causal_conv1d.py:337-374; the double sum is the value all such orders approximate).
 *
 * Build: oracle/Makefile (gcc -O2 -ffp-contract=off, so that the only fused multiply-adds are the
 * explicit fmaf() calls, matching the FMA contraction Triton applies to `z += w * x`).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>

static int g_mutation = 0;

/* Plants a deliberate mistake (test use only; 0 = none). See the MUT_* uses below. */
void ccv1d_oracle_set_mutation(int m) { g_mutation = m; }

enum {
  MUT_DROP_TAP0 = 1,      /* forward drops the oldest tap (k = 0) */
  MUT_TAP_INDEX = 2,      /* forward reads x[t-P+k+1] instead of x[t-P+k] for k < P */
  MUT_DSILU_SIGN = 3,     /* silu' uses (1 + s) instead of (1 - s) */
  MUT_W_TRANSPOSED = 4,   /* weight read as (W, D) instead of (D, W) */
  MUT_DX_UNFLIPPED = 5,   /* dx uses w[j] instead of w[P - j] */
  MUT_NO_SEQ_MASK_DX = 6, /* dx ignores sequence boundaries */
  MUT_FINAL_SHIFT = 7,    /* final_states taken one row early */
  MUT_NO_DFINAL = 8,      /* dfinal not added into dx / dinit */
  MUT_PAD_NOT_ZERO = 9,   /* forward does not zero padding rows */
  MUT_INIT_SEQ = 10       /* initial-state rows get sequence id -1 even with initial states */
};

static int P_of(int64_t W) { return (int)(W - 1); }

/* Row t of concat(initial_states, x) (causal_conv1d.py:28-41). */
static float xx_at(const float* xb, const float* ib, int64_t T, int64_t D, int P, int64_t t,
                   int64_t d) {
  if (t >= 0 && t < T) return xb[t * D + d];
  if (t < 0 && t >= -P && ib) return ib[(t + P) * D + d];
  return 0.0f;
}

/* Sequence id of row t (causal_conv1d.py:17-25). */
static int32_t seq_at(const int32_t* sb, int64_t T, int has_init, int64_t t) {
  if (t >= T) return -1;
  if (t < 0) return (has_init && g_mutation != MUT_INIT_SEQ) ? sb[0] : -1;
  return sb[t];
}

static float w_at(const float* w, int64_t D, int64_t W, int64_t d, int64_t k) {
  if (g_mutation == MUT_W_TRANSPOSED) return w[k * D + d];
  return w[d * W + k];
}

/* sigmoid as tl.sigmoid defines it: 1 / (1 + exp(-x)) (Triton language/standard.py). */
static float sigmoid_ref(float z) { return 1.0f / (1.0f + expf(-z)); }

/* Pre-activation z[b, t, d] including bias, without the padding zero (causal_conv1d.py:129-136 and
 * the backward recompute :277-284). With seq_idx the masked taps are skipped. */
static float conv_z(const float* xb, const float* ib, const int32_t* sb, const float* w,
                    const float* bias, int64_t T, int64_t D, int64_t W, int64_t t, int64_t d) {
  const int P = P_of(W);
  const int has_init = ib != NULL;
  const int32_t st = sb ? seq_at(sb, T, has_init, t) : 0;
  float z = w_at(w, D, W, d, P) * xx_at(xb, ib, T, D, P, t, d);
  for (int k = 0; k < P; ++k) {
    if (g_mutation == MUT_DROP_TAP0 && k == 0) continue;
    const int64_t r = (g_mutation == MUT_TAP_INDEX) ? t - P + k + 1 : t - P + k;
    if (sb && seq_at(sb, T, has_init, r) != st) continue;
    z = fmaf(w_at(w, D, W, d, k), xx_at(xb, ib, T, D, P, r, d), z);
  }
  if (bias) z += bias[d];
  return z;
}

/* Forward (causal_conv1d.py:44-164): out = act(z) with z = 0 on padding rows; final_states =
 * rows T-P .. T-1 of concat(initial_states, x). out and final_states may be NULL. */
void ccv1d_oracle_fwd(const float* x, const float* w, const float* bias, const int32_t* seq,
                      const float* init, float* out, float* final_states, int64_t B, int64_t T,
                      int64_t D, int64_t W, int silu) {
  const int P = P_of(W);
  for (int64_t b = 0; b < B; ++b) {
    const float* xb = x + b * T * D;
    const float* ib = init ? init + b * P * D : NULL;
    const int32_t* sb = seq ? seq + b * T : NULL;
    if (out) {
      for (int64_t t = 0; t < T; ++t) {
        const int32_t st = sb ? sb[t] : 0;
        for (int64_t d = 0; d < D; ++d) {
          float z = conv_z(xb, ib, sb, w, bias, T, D, W, t, d);
          if (sb && st < 0 && g_mutation != MUT_PAD_NOT_ZERO) z = 0.0f;
          if (silu) z = z * sigmoid_ref(z);
          out[(b * T + t) * D + d] = z;
        }
      }
    }
    if (final_states) {
      const int64_t shift = (g_mutation == MUT_FINAL_SHIFT) ? 1 : 0;
      for (int p = 0; p < P; ++p)
        for (int64_t d = 0; d < D; ++d)
          final_states[(b * P + p) * D + d] = xx_at(xb, ib, T, D, P, T - P + p - shift, d);
    }
  }
}

/* Backward (causal_conv1d.py:167-374).
 *   g[t]  = dout[t] * silu'(z[t]) (just dout[t] without silu), 0 on padding rows and outside [0, T)
 *   dx[r] = w[P] g[r] + sum_{j=1..P} [s(r+j) == s(r)] w[P-j] g[r+j]  (+ dfinal[r - (T-P)])
 *           for r in [-P, T); rows r < 0 are the initial-state gradient (stored when dinit != NULL)
 *   dweight[d, k] = sum_{b, t} g[t] * xx[t-P+k] * [s(t-P+k) == s(t)],  dbias[d] = sum_{b, t} g[t]
 * dx (B, T, D) and dinit (B, P, D) are fp32; dweight (D, W) and dbias (D) are double.
 * dfinal, dinit, bias/dbias may be NULL. Returns 0, or -1 if scratch memory cannot be allocated. */
int ccv1d_oracle_bwd(const float* x, const float* w, const float* bias, const int32_t* seq,
                     const float* init, const float* dout, const float* dfinal, float* dx,
                     float* dinit, double* dweight, double* dbias, int64_t B, int64_t T, int64_t D,
                     int64_t W, int silu) {
  const int P = P_of(W);
  float* g = (float*)malloc(sizeof(float) * (size_t)(T > 0 ? T : 1) * (size_t)(D > 0 ? D : 1));
  if (!g) return -1;
  for (int64_t i = 0; i < D * W; ++i) dweight[i] = 0.0;
  if (dbias)
    for (int64_t d = 0; d < D; ++d) dbias[d] = 0.0;
  for (int64_t b = 0; b < B; ++b) {
    const float* xb = x + b * T * D;
    const float* ib = init ? init + b * P * D : NULL;
    const int32_t* sb = seq ? seq + b * T : NULL;
    const int has_init = ib != NULL;
    const float* yb = dout + b * T * D;
    /* g (causal_conv1d.py:274-288) */
    for (int64_t t = 0; t < T; ++t) {
      const int32_t st = sb ? sb[t] : 0;
      for (int64_t d = 0; d < D; ++d) {
        float gv = yb[t * D + d];
        if (silu) {
          const float z = conv_z(xb, ib, sb, w, bias, T, D, W, t, d);
          const float s = sigmoid_ref(z);
          const float oms = (g_mutation == MUT_DSILU_SIGN) ? 1.0f + s : 1.0f - s;
          gv = gv * s * fmaf(z, oms, 1.0f);
        }
        if (sb && st < 0) gv = 0.0f;
        g[t * D + d] = gv;
      }
    }
    /* dx and dinit (causal_conv1d.py:290-311) */
    for (int64_t r = -P; r < T; ++r) {
      if (r < 0 && !dinit) continue;
      const int32_t sr = sb ? seq_at(sb, T, has_init, r) : 0;
      for (int64_t d = 0; d < D; ++d) {
        const float g0 = (r >= 0) ? g[r * D + d] : 0.0f;
        float v = w_at(w, D, W, d, P) * g0;
        for (int j = 1; j <= P; ++j) {
          const int64_t tj = r + j;
          const float gj = (tj >= 0 && tj < T) ? g[tj * D + d] : 0.0f;
          if (sb && g_mutation != MUT_NO_SEQ_MASK_DX && seq_at(sb, T, has_init, tj) != sr) continue;
          const int64_t k = (g_mutation == MUT_DX_UNFLIPPED) ? j : P - j;
          v = fmaf(w_at(w, D, W, d, k), gj, v);
        }
        if (dfinal && g_mutation != MUT_NO_DFINAL) {
          const int64_t f = r - (T - P);
          if (f >= 0 && f < P) v += dfinal[(b * P + f) * D + d];
        }
        if (r >= 0) dx[(b * T + r) * D + d] = v;
        else dinit[(b * P + r + P) * D + d] = v;
      }
    }
    /* dweight and dbias (causal_conv1d.py:313-321, 344-374) */
    for (int64_t t = 0; t < T; ++t) {
      const int32_t st = sb ? sb[t] : 0;
      for (int64_t d = 0; d < D; ++d) {
        const double gv = g[t * D + d];
        for (int k = 0; k < W; ++k) {
          const int64_t r = t - P + k;
          if (sb && k < P && seq_at(sb, T, has_init, r) != st) continue;
          dweight[d * W + k] += gv * (double)xx_at(xb, ib, T, D, P, r, d);
        }
        if (dbias) dbias[d] += gv;
      }
    }
  }
  free(g);
  return 0;
}
