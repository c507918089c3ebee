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
  int32_t vec;   // channels per lane the tiling was made for (0 for the generic kernels)
  // Workgroup order: 0 = time fastest (a wave column's consecutive time tiles are consecutive
  // workgroups), 1 = wave column fastest (the columns of one range of rows are), for rows that are
  // not aligned to the 128-byte line, whose lines straddle neighbouring columns (TileCoord).
  int32_t col_fast;
};
// Widest kernels that follow Tiling::col_fast (wider ones always run time fastest).
constexpr int kColFastMaxW = 8;

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
  int32_t out_nt, x_nt;       // host side: non-temporal out stores / x loads for this call
  uint32_t x_bytes, o_bytes;  // per-batch byte extents of x and out (vectorised kernels)
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
  int64_t s_xb, s_yb, s_dxb;
  int32_t s_xt, s_yt, s_dxt;  // s_dxb, s_dxt: strides of dx (T * D and D when contiguous)
  int32_t B, T, D, W;
  int32_t w_dt, b_dt, i_dt;
  int32_t has_bias, has_init, has_dfinal, need_dinit, silu;
  uint32_t x_bytes, y_bytes, o_bytes;  // per-batch byte extents of x, dout and dx (vectorised)
  Tiling tl;
  // Host side: dx rows straddle 128-byte lines, stored non-temporally (BwdCfg). Kept after tl: in
  // front of it the widest kernels' kernel-argument loads left them 20-400 more SGPR spills.
  int32_t dx_nt;
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

// An fp32 result converted to the type T it is stored in, rounded from its fp32 value as the
// reference's stores round it. For 16-bit T the value first passes through an empty asm: without
// it the compiler may fold the conversion into the fma that produced the value (v_fma_mixlo_f16
// rounds the exact a * b + c to fp16 once), which differs from rounding the fp32 result in about
// one value in 10^5.
template <typename T>
__device__ __forceinline__ T to_store(float v) {
  if constexpr (sizeof(T) == 2) asm("" : "+v"(v));
  return static_cast<T>(v);
}

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
    case DT_F16: static_cast<_Float16*>(p)[i] = to_store<_Float16>(v); break;
    case DT_BF16: static_cast<__bf16*>(p)[i] = to_store<__bf16>(v); break;
    default: static_cast<double*>(p)[i] = static_cast<double>(v); break;
  }
}

// ---------------------------------------------------------------------------------------------
// Channel vectors of the x dtype. One lane moves CPL consecutive channels of one row with a single
// 2-, 4-, 8- or 16-byte load or store, so a wave covers 64 * CPL channels (128 B to 1 KiB) per
// instruction.
// ---------------------------------------------------------------------------------------------

typedef float f2v __attribute__((ext_vector_type(2)));
typedef __bf16 bf2v __attribute__((ext_vector_type(2)));
typedef _Float16 h2v __attribute__((ext_vector_type(2)));
typedef uint32_t u32x1 __attribute__((ext_vector_type(1)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

template <int BYTES> struct RawOf;
template <> struct RawOf<2> { using type = uint16_t; };
template <> struct RawOf<4> { using type = u32x1; };
template <> struct RawOf<8> { using type = u32x2; };
template <> struct RawOf<16> { using type = u32x4; };

template <typename TX, int CPL>
struct VecIO {
  static constexpr int BYTES = CPL * (int)sizeof(TX);
  static constexpr int WORDS = BYTES / 4;
  using raw = typename RawOf<BYTES>::type;

  __device__ static __forceinline__ raw ld(const TX* p) { return *reinterpret_cast<const raw*>(p); }
  __device__ static __forceinline__ void st(TX* p, raw v) { *reinterpret_cast<raw*>(p) = v; }
  // Non-temporal store: streamed output that no later work in the kernel reads.
  __device__ static __forceinline__ void st_nt(TX* p, raw v) {
    __builtin_nontemporal_store(v, reinterpret_cast<raw*>(p));
  }

  __device__ static __forceinline__ void unpack(const raw v, float (&f)[CPL]) {
    if constexpr (BYTES == 2) {  // one 16-bit channel
      if constexpr (__is_same(TX, __bf16)) f[0] = __uint_as_float((uint32_t)v << 16);
      else f[0] = static_cast<float>(__builtin_bit_cast(_Float16, v));
    } else {
#pragma unroll
      for (int j = 0; j < WORDS; ++j) {
        const uint32_t u = v[j];
        if constexpr (sizeof(TX) == 4) {
          f[j] = __uint_as_float(u);
        } else if constexpr (__is_same(TX, __bf16)) {
          f[2 * j] = __uint_as_float(u << 16);
          f[2 * j + 1] = __uint_as_float(u & 0xffff0000u);
        } else {
          const f2v q = __builtin_convertvector(__builtin_bit_cast(h2v, u), f2v);
          f[2 * j] = q.x;
          f[2 * j + 1] = q.y;
        }
      }
    }
  }

  // Round-to-nearest-even; one v_cvt_pk_{bf16,f16}_f32 per channel pair.
  __device__ static __forceinline__ raw pack(const float (&f)[CPL]) {
    if constexpr (BYTES == 2) {
      return __builtin_bit_cast(raw, to_store<TX>(f[0]));
    } else {
      raw v;
#pragma unroll
      for (int j = 0; j < WORDS; ++j) {
        if constexpr (sizeof(TX) == 4) {
          v[j] = __float_as_uint(f[j]);
        } else if constexpr (__is_same(TX, __bf16)) {
          v[j] = __builtin_bit_cast(uint32_t,
                                    __builtin_convertvector((f2v){f[2 * j], f[2 * j + 1]}, bf2v));
        } else {
          v[j] = __builtin_bit_cast(uint32_t,
                                    __builtin_convertvector((f2v){f[2 * j], f[2 * j + 1]}, h2v));
        }
      }
      return v;
    }
  }
};

// Rows of one batch slab of a channels-last tensor. Loads go through a buffer resource: the row
// offset is a uniform (scalar) byte offset and the lane's channel offset a 32-bit vector offset, so a
// row load costs no vector address arithmetic. The host guarantees every byte offset used here is
// below 2^32 and below `extent`, the resource's size.
//
// Stores of 8 bytes use the same resource. 16-byte stores use a global store instead: after a
// buffer_store_dwordx4 whose offset is in an SGPR the compiler does not keep the data VGPRs intact
// for the wait state a store of more than 8 bytes needs before a VALU may overwrite them, and on
// gfx950 such stores were measured to write values of the following instructions. The compiler does
// enforce that wait state after global stores.
//
// LD and ST are the cache-policy bits of the row loads and stores: the `aux` operand of the buffer
// intrinsics, on gfx950 1 = sc0, 2 = nt (non-temporal), 16 = sc1 (device scope: the store is written
// through the L2 instead of staying there dirty until the end of the kernel). 16-byte stores, which
// go through a global store, support the plain and the non-temporal policy only.
constexpr int kCachePlain = 0;
constexpr int kCacheNT = 2;
constexpr int kCacheSC1 = 16;
constexpr int kCacheSC1NT = kCacheSC1 | kCacheNT;
template <typename TX, int CPL, int LD = kCachePlain, int ST = kCachePlain>
struct RowBuf {
  using IO = VecIO<TX, CPL>;
  using raw = typename IO::raw;
  static_assert(IO::BYTES != 16 || ST == kCachePlain || ST == kCacheNT,
                "16-byte row stores support the plain and non-temporal policies only");
  __amdgpu_buffer_rsrc_t rs;
  const TX* base;      // row 0, channel 0 of the slab
  uint32_t lane_off;   // byte offset of this lane's first channel
  uint32_t row_bytes;  // time stride in bytes

  __device__ __forceinline__ RowBuf(const TX* slab, uint32_t extent, int c0, int stride_t) {
    rs = __builtin_amdgcn_make_buffer_rsrc(const_cast<TX*>(slab), 0, (int)extent, 0x00020000);
    base = slab;
    lane_off = (uint32_t)c0 * (uint32_t)sizeof(TX);
    row_bytes = (uint32_t)stride_t * (uint32_t)sizeof(TX);
  }
  // A row with the buffer's load policy, or with POL for rows that are read again soon (see
  // bwd_tile's halo).
  template <int POL = LD>
  __device__ __forceinline__ raw ld(int row) const {
    if constexpr (IO::BYTES == 16)
      return __builtin_bit_cast(raw, __builtin_amdgcn_raw_buffer_load_b128(rs, lane_off, (uint32_t)row * row_bytes, POL));
    else if constexpr (IO::BYTES == 8)
      return __builtin_bit_cast(raw, __builtin_amdgcn_raw_buffer_load_b64(rs, lane_off, (uint32_t)row * row_bytes, POL));
    else if constexpr (IO::BYTES == 4)
      return __builtin_bit_cast(raw, __builtin_amdgcn_raw_buffer_load_b32(rs, lane_off, (uint32_t)row * row_bytes, POL));
    else
      return __builtin_bit_cast(raw, __builtin_amdgcn_raw_buffer_load_b16(rs, lane_off, (uint32_t)row * row_bytes, POL));
  }
  __device__ __forceinline__ void st(int row, raw v) const {
    if constexpr (IO::BYTES == 16) {
      TX* p = reinterpret_cast<TX*>(const_cast<char*>(reinterpret_cast<const char*>(base)) +
                                    (uint64_t)((uint32_t)row * row_bytes + lane_off));
      if (ST == kCacheNT) IO::st_nt(p, v);
      else IO::st(p, v);
    } else if constexpr (IO::BYTES == 8) {
      __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u32x2, v), rs, lane_off,
                                            (uint32_t)row * row_bytes, ST);
    } else if constexpr (IO::BYTES == 4) {
      __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, v), rs, lane_off,
                                            (uint32_t)row * row_bytes, ST);
    } else {
      __builtin_amdgcn_raw_buffer_store_b16(v, rs, lane_off, (uint32_t)row * row_bytes, ST);
    }
  }
};

// N consecutive elements of a side tensor whose dtype is a runtime code, converted to fp32. The
// dtype switch is taken once for the whole vector so the N loads issue together.
template <int N>
__device__ __forceinline__ void ld_vec_any(const void* p, int64_t off, int dt, float (&f)[N]) {
  switch (dt) {
    case DT_F32: {
      const float* q = static_cast<const float*>(p) + off;
#pragma unroll
      for (int i = 0; i < N; ++i) f[i] = q[i];
    } break;
    case DT_F16: {
      const _Float16* q = static_cast<const _Float16*>(p) + off;
#pragma unroll
      for (int i = 0; i < N; ++i) f[i] = static_cast<float>(q[i]);
    } break;
    case DT_BF16: {
      const __bf16* q = static_cast<const __bf16*>(p) + off;
#pragma unroll
      for (int i = 0; i < N; ++i) f[i] = static_cast<float>(q[i]);
    } break;
    default: {
      const double* q = static_cast<const double*>(p) + off;
#pragma unroll
      for (int i = 0; i < N; ++i) f[i] = static_cast<float>(q[i]);
    } break;
  }
}

// M rows of N consecutive elements, `stride` elements apart, converted to fp32. One dtype switch
// for all rows, so the M * N loads issue before any of them is waited for.
template <int M, int N>
__device__ __forceinline__ void ld_rows_any(const void* p, int64_t off, int64_t stride, int dt,
                                            float (&f)[M][N]) {
  switch (dt) {
    case DT_F32: {
      const float* q = static_cast<const float*>(p) + off;
#pragma unroll
      for (int m = 0; m < M; ++m)
#pragma unroll
        for (int i = 0; i < N; ++i) f[m][i] = q[m * stride + i];
    } break;
    case DT_F16: {
      const _Float16* q = static_cast<const _Float16*>(p) + off;
#pragma unroll
      for (int m = 0; m < M; ++m)
#pragma unroll
        for (int i = 0; i < N; ++i) f[m][i] = static_cast<float>(q[m * stride + i]);
    } break;
    case DT_BF16: {
      const __bf16* q = static_cast<const __bf16*>(p) + off;
#pragma unroll
      for (int m = 0; m < M; ++m)
#pragma unroll
        for (int i = 0; i < N; ++i) f[m][i] = static_cast<float>(q[m * stride + i]);
    } break;
    default: {
      const double* q = static_cast<const double*>(p) + off;
#pragma unroll
      for (int m = 0; m < M; ++m)
#pragma unroll
        for (int i = 0; i < N; ++i) f[m][i] = static_cast<float>(q[m * stride + i]);
    } break;
  }
}

template <int N>
__device__ __forceinline__ void st_vec_any(void* p, int64_t off, int dt, const float (&f)[N]) {
  switch (dt) {
    case DT_F32: {
      float* q = static_cast<float*>(p) + off;
#pragma unroll
      for (int i = 0; i < N; ++i) q[i] = f[i];
    } break;
    case DT_F16: {
      _Float16* q = static_cast<_Float16*>(p) + off;
#pragma unroll
      for (int i = 0; i < N; ++i) q[i] = to_store<_Float16>(f[i]);
    } break;
    case DT_BF16: {
      __bf16* q = static_cast<__bf16*>(p) + off;
#pragma unroll
      for (int i = 0; i < N; ++i) q[i] = to_store<__bf16>(f[i]);
    } break;
    default: {
      double* q = static_cast<double*>(p) + off;
#pragma unroll
      for (int i = 0; i < N; ++i) q[i] = static_cast<double>(f[i]);
    } break;
  }
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

// The vectorised backward evaluates silu' in the base-2 domain. Its weights and bias are
// pre-multiplied by -log2(e), so the tap chain yields y = -log2(e) * z, the argument of exp2
// itself, and no per-element multiply forms it. With e = 2^y = exp(-z) and s = 1 / (1 + e):
//   silu'(z) = s * (1 + z * (1 - s)),  z = -ln2 * y
//   -ln2 * silu'(z) = s * fma(y, ln2^2 * (1 - s), -ln2)
// so g~ = dy * s * fma(y, fma(s, -ln2^2, ln2^2), -ln2) = -ln2 * g costs the same four operations
// as g. dx = sum_j (-log2(e) w) * (-ln2 g) = sum_j w * g needs no correction (log2(e) * ln2 = 1);
// the dweight/dbias sums, accumulated from g~, are multiplied by -log2(e) once per tile.
constexpr float kNegLog2e = -1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
constexpr float kLn2Sq = 0.4804530139182014f;

// g~ = -ln2 * dy * silu'(z) from y = -log2(e) * z (see above). Non-finite inputs propagate as in
// the unscaled form: z = +-inf gives 0 * inf = NaN where the reference's expression does.
__device__ __forceinline__ float dsilu_scaled(float dy, float y) {
  const float s = __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(y));
  const float u = fmaf(y, fmaf(s, -kLn2Sq, kLn2Sq), -kLn2);
  return (dy * s) * u;
}

// Rows whose sequence ids a wave of the vectorised kernels reads up front (RowIds): its tile and both
// halos must fit.
constexpr int kRowIds = 128;

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
