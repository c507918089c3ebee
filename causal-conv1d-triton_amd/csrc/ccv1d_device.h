// Device-side building blocks shared by the gfx950 kernels: parameter blocks, element conversion,
// 16-byte channel-vector pack/unpack, the fp32 tap sum and the silu epilogue.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace ccv1d {

enum : int { DT_F32 = 0, DT_F16 = 1, DT_BF16 = 2, DT_F64 = 3 };

// ---------------------------------------------------------------------------------------------
// Parameter blocks (passed by value in the kernel argument segment).
// ---------------------------------------------------------------------------------------------

// Time tiling of the vectorised kernels. A wave owns `L` consecutive rows ("a tile") of 64 channel
// vectors ("a wave column"); a workgroup holds NW waves on consecutive tiles of one wave column.
struct Tiling {
  int32_t L;     // rows per tile
  int32_t nT;    // tiles per batch row: ceil(T / L)
  int32_t nGW;   // wave columns: ceil(D / VEC / 64)
  int32_t nTB;   // workgroups along time per batch row: ceil(nT / NW)
  int32_t nBlk;  // workgroups in the grid: B * nGW * nTB
};

struct FwdParams {
  const void* x;
  const void* w;
  const void* bias;
  const int32_t* seq;
  const void* init;
  void* out;
  void* fin;
  int64_t s_xb;  // batch stride of x (elements)
  int32_t s_xt;  // time stride of x (elements)
  int32_t B, T, D, W;
  int32_t w_dt, b_dt, i_dt;
  int32_t has_bias, has_init, has_final, silu;
  Tiling tl;
};

struct BwdParams {
  const void* x;
  const void* w;
  const void* bias;
  const int32_t* seq;
  const void* init;
  const void* dy;
  const void* dfin;
  void* dx;
  void* dinit;
  float* part;   // (Pn, W + 1, D) fp32 partial sums; row W holds dbias
  int64_t s_xb, s_yb;
  int32_t s_xt, s_yt;
  int32_t B, T, D, W;
  int32_t w_dt, b_dt, i_dt;
  int32_t has_bias, has_init, has_dfinal, need_dinit, silu;
  Tiling tl;
};

struct ReduceParams {
  const float* part;
  void* dw;
  void* db;
  int32_t Pn;    // partial rows
  int32_t D, W;
  int32_t w_dt, b_dt, has_bias;
};

// ---------------------------------------------------------------------------------------------
// Scalar conversions for the side tensors (weight, bias, states) whose dtype is a runtime code.
// ---------------------------------------------------------------------------------------------

__device__ __forceinline__ float ld_any(const void* p, int64_t i, int dt) {
  switch (dt) {
    case DT_F32: return static_cast<const float*>(p)[i];
    case DT_F16: return static_cast<float>(static_cast<const _Float16*>(p)[i]);
    case DT_BF16: return static_cast<float>(static_cast<const __bf16*>(p)[i]);
    default: return static_cast<float>(static_cast<const double*>(p)[i]);
  }
}

__device__ __forceinline__ void st_any(void* p, int64_t i, int dt, float v) {
  switch (dt) {
    case DT_F32: static_cast<float*>(p)[i] = v; break;
    case DT_F16: static_cast<_Float16*>(p)[i] = static_cast<_Float16>(v); break;
    case DT_BF16: static_cast<__bf16*>(p)[i] = static_cast<__bf16>(v); break;
    default: static_cast<double*>(p)[i] = static_cast<double>(v); break;
  }
}

// ---------------------------------------------------------------------------------------------
// 16-byte channel vectors of the x dtype. One lane moves VEC consecutive channels of one row with a
// single 128-bit load or store; a wave therefore covers 64 * VEC channels (1 KiB) per instruction.
// ---------------------------------------------------------------------------------------------

typedef float f2v __attribute__((ext_vector_type(2)));
typedef __bf16 bf2v __attribute__((ext_vector_type(2)));
typedef _Float16 h2v __attribute__((ext_vector_type(2)));

template <typename TX> struct Vec16;

template <> struct Vec16<__bf16> {
  static constexpr int VEC = 8;
  __device__ static __forceinline__ void unpack(const uint4 v, float (&f)[8]) {
    const uint32_t u[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      f[2 * j] = __uint_as_float(u[j] << 16);
      f[2 * j + 1] = __uint_as_float(u[j] & 0xffff0000u);
    }
  }
  __device__ static __forceinline__ uint4 pack(const float (&f)[8]) {
    uint32_t u[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      // Round-to-nearest-even, one v_cvt_pk_bf16_f32 per channel pair.
      u[j] = __builtin_bit_cast(uint32_t, __builtin_convertvector((f2v){f[2 * j], f[2 * j + 1]}, bf2v));
    }
    return make_uint4(u[0], u[1], u[2], u[3]);
  }
};

template <> struct Vec16<_Float16> {
  static constexpr int VEC = 8;
  __device__ static __forceinline__ void unpack(const uint4 v, float (&f)[8]) {
    const uint32_t u[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const f2v p = __builtin_convertvector(__builtin_bit_cast(h2v, u[j]), f2v);
      f[2 * j] = p.x;
      f[2 * j + 1] = p.y;
    }
  }
  __device__ static __forceinline__ uint4 pack(const float (&f)[8]) {
    uint32_t u[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      u[j] = __builtin_bit_cast(uint32_t, __builtin_convertvector((f2v){f[2 * j], f[2 * j + 1]}, h2v));
    }
    return make_uint4(u[0], u[1], u[2], u[3]);
  }
};

template <> struct Vec16<float> {
  static constexpr int VEC = 4;
  __device__ static __forceinline__ void unpack(const uint4 v, float (&f)[4]) {
    f[0] = __uint_as_float(v.x);
    f[1] = __uint_as_float(v.y);
    f[2] = __uint_as_float(v.z);
    f[3] = __uint_as_float(v.w);
  }
  __device__ static __forceinline__ uint4 pack(const float (&f)[4]) {
    return make_uint4(__float_as_uint(f[0]), __float_as_uint(f[1]), __float_as_uint(f[2]),
                      __float_as_uint(f[3]));
  }
};

template <typename TX> __device__ __forceinline__ uint4 ld16(const TX* p) {
  return *reinterpret_cast<const uint4*>(p);
}
template <typename TX> __device__ __forceinline__ void st16(TX* p, uint4 v) {
  *reinterpret_cast<uint4*>(p) = v;
}

// ---------------------------------------------------------------------------------------------
// Arithmetic shared by forward and backward, so the backward's recomputed pre-activation is
// bit-identical to the forward's.
// ---------------------------------------------------------------------------------------------

// sigmoid(z) = 1 / (1 + exp(-z)) with the hardware exp2 and reciprocal (v_exp_f32, v_rcp_f32; about
// 1 ulp each). exp(-z) overflows to +inf for z < -88.7, giving exactly 0; it underflows to 0 for
// large z, giving exactly 1.
__device__ __forceinline__ float sigmoid_f(float z) {
  return __builtin_amdgcn_rcpf(1.0f + __expf(-z));
}

// silu'(z) = s * (1 + z * (1 - s)), s = sigmoid(z), evaluated in the reference's operation order
// (causal_conv1d.py:285-286): dz * s * (1 + z * (1 - s)).
__device__ __forceinline__ float dsilu_times(float dy, float z) {
  const float s = sigmoid_f(z);
  return dy * s * fmaf(z, 1.0f - s, 1.0f);
}

// Sequence id of row t of concat(initial_states, x) (causal_conv1d.py:17-25): rows t < 0 belong to
// seq_idx[b, 0] when there are initial states and are -1 otherwise; rows t >= T are -1.
__device__ __forceinline__ int32_t seq_at(const int32_t* seqb, int t, int T, bool has_init) {
  if (t >= T) return -1;
  if (t < 0) return has_init ? seqb[0] : -1;
  return seqb[t];
}

// Maps the hardware workgroup id to a logical one so that each of the 8 XCDs (which receive
// workgroups round-robin) runs one contiguous range of logical workgroups. Neighbouring time tiles,
// whose halo rows overlap, then share one XCD's L2.
__device__ __forceinline__ int xcd_remap(int bid, int n) {
  const int q = n >> 3, r = n & 7;
  const int x = bid & 7, j = bid >> 3;
  return x * q + (x < r ? x : r) + j;
}

}  // namespace ccv1d
