/*
 * ccv1d.h - C ABI of the MI355X (gfx950) causal depthwise conv1d library (libccv1d.so).
 *
 * The operation, over channels-last x of shape (batch, seqlen, dim), with P = width - 1:
 *
 *   xx[b, t, d]  = x[b, t, d]                 for 0 <= t < seqlen
 *                = initial_states[b, t+P, d]  for -P <= t < 0 (zero when there are no initial states)
 *   z[b, t, d]   = weight[d, P] * xx[t] + sum_{k<P} m_k * weight[d, k] * xx[t-P+k]   (fp32)
 *                  (+ bias[d]); with seq_idx, z = 0 where seq_idx[b, t] < 0
 *   out[b, t, d] = silu(z) if silu else z, rounded to the x dtype
 *
 * where m_k = (seq[t-P+k] == seq[t]) with seq_idx and 1 otherwise; rows t < 0 carry the sequence id of
 * seq_idx[b, 0] when initial states are given and -1 otherwise.
 *
 * Conventions shared by every entry point:
 *  - All tensor pointers are device pointers on `device`. The caller owns every buffer; the library
 *    never allocates device memory.
 *  - Work is enqueued asynchronously on `stream` (a hipStream_t; NULL = the legacy default stream of
 *    `device`). The calling thread's current device is restored before returning.
 *  - x and dout may have arbitrary batch and time strides (in elements) but a unit channel stride.
 *    Every other tensor is contiguous: weight (dim, width), bias (dim), seq_idx (batch, seqlen) int32,
 *    initial/final states and their gradients (batch, width - 1, dim), out and dx (batch, seqlen, dim).
 *  - Offsets inside one batch element are 32-bit: (seqlen + width) * max(x_stride_t, dim) and the same
 *    for dout must be below 2^31.
 *  - Return value: CCV1D_OK (0) or an error code; ccv1d_last_error() then describes the failure.
 *  - Reentrant and thread-safe; the only global state is the error string and the timing request of
 *    ccv1d_time_main_kernel (both thread-local). The library reads nothing from the environment:
 *    its tiling, and with it every summation order, is a function of the shape alone.
 */
#ifndef CCV1D_H
#define CCV1D_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define CCV1D_ABI_VERSION 1

/* Element types. x, out, final_states, dout, dfinal_states and dx may be F32, F16 or BF16 (F64 is
 * accepted on the generic path). weight, bias and initial_states may each have any of the four types;
 * they are converted to fp32 on load, and their gradients are stored in their own type. */
enum ccv1d_dtype { CCV1D_F32 = 0, CCV1D_F16 = 1, CCV1D_BF16 = 2, CCV1D_F64 = 3 };

enum ccv1d_status {
  CCV1D_OK = 0,
  CCV1D_ERR_INVALID = 1,     /* bad argument: null pointer, negative size, width < 2, bad dtype code */
  CCV1D_ERR_UNSUPPORTED = 2, /* valid request outside what the kernels implement (a grid beyond the
                                generic kernels' limits: batch * ceil(seqlen / 64) >= 2^31, or more
                                than 65535 * 64 channels on rows that need them) */
  CCV1D_ERR_WORKSPACE = 3,   /* workspace missing or smaller than ccv1d_bwd_workspace_bytes() */
  CCV1D_ERR_HIP = 4          /* a HIP runtime call or kernel launch failed */
};

/* Version of this ABI (CCV1D_ABI_VERSION of the built library). */
int ccv1d_abi_version(void);

/* Description of the last error raised on the calling thread ("" if none). */
const char* ccv1d_last_error(void);

/* Measurement aid; it has no counterpart in the reference, whose passes are timed from Python
 * around whole launches. Asks the calling thread's next ccv1d_fwd or ccv1d_bwd call to launch its
 * main kernel (the convolution kernel of the pass; not the dweight/dbias reduction or a fill)
 * through hipExtLaunchKernel with these two events, which HIP sets from that dispatch's own start
 * and end timestamps: once the kernel has completed, hipEventElapsedTime(start_event, stop_event)
 * is its execution time, without the marker packets of hipEventRecord around it. The events are
 * hipEvent_t handles with timing enabled, created by the caller. The request applies to the next
 * call only, whatever that call does; a call that launches no main kernel (empty input, an error)
 * leaves the events as they were. Not meant for stream capture. Two NULLs cancel a pending request;
 * exactly one NULL is CCV1D_ERR_INVALID. */
int ccv1d_time_main_kernel(void* start_event, void* stop_event);

/* Forward pass. Replaces the host launcher `_fwd` of the reference
 * (causal_conv1d_triton/causal_conv1d.py:433-472) together with the `_fwd_kernel` it launches
 * (causal_conv1d.py:44-164) and the empty-input path (causal_conv1d.py:437-444).
 *
 *  x                 (batch, seqlen, dim), strides (x_stride_b, x_stride_t, 1), type x_dtype
 *  weight            (dim, width), type weight_dtype
 *  bias              (dim,) or NULL, type bias_dtype
 *  seq_idx           (batch, seqlen) int32 or NULL
 *  initial_states    (batch, width - 1, dim) or NULL, type init_dtype
 *  out               (batch, seqlen, dim), type x_dtype; must not overlap x (no in-place
 *                    forward: CCV1D_ERR_INVALID)
 *  final_states      (batch, width - 1, dim) or NULL, type x_dtype: the last width - 1 rows of
 *                    concat(initial_states, x), i.e. the state for continuing the sequence. Must be
 *                    NULL when seq_idx is given (causal_conv1d.py:607-608).
 *  silu              0: no activation; 1: out = z * sigmoid(z)
 */
int ccv1d_fwd(const void* x, int64_t x_stride_b, int64_t x_stride_t, int x_dtype,
              const void* weight, int weight_dtype,
              const void* bias, int bias_dtype,
              const int32_t* seq_idx,
              const void* initial_states, int init_dtype,
              void* out, void* final_states,
              int64_t batch, int64_t seqlen, int64_t dim, int64_t width,
              int silu, int device, void* stream);

/* Forward for inference: the arguments, results and kernels of ccv1d_fwd, for a call after which no
 * backward reads x (no autograd). When x and out exceed 64 MiB it stores out non-temporally, which
 * suits a pass whose input is not read again soon (ccv1d_fwd does so only above 128 MiB, half the
 * 256 MiB Infinity Cache, and otherwise keeps both cacheable for the backward): forward alone at
 * B=4 T=8192 D=1024 bf16, 29.6 -> about 24 us. The reference has one forward for both uses
 * (causal_conv1d.py:433-472); results are bit-identical to ccv1d_fwd's. */
int ccv1d_fwd_inference(const void* x, int64_t x_stride_b, int64_t x_stride_t, int x_dtype,
                        const void* weight, int weight_dtype,
                        const void* bias, int bias_dtype,
                        const int32_t* seq_idx,
                        const void* initial_states, int init_dtype,
                        void* out, void* final_states,
                        int64_t batch, int64_t seqlen, int64_t dim, int64_t width,
                        int silu, int device, void* stream);

/* Bytes of device workspace ccv1d_bwd needs for this shape: fp32 partial sums of dweight/dbias (the
 * reference allocates the same kind of buffer at causal_conv1d.py:493) and, for widths above 128,
 * an fp32 buffer of batch * seqlen * dim values for the gradient of the pre-activation. An upper
 * bound over every path the shape can take; 0 for empty shapes. */
size_t ccv1d_bwd_workspace_bytes(int64_t batch, int64_t seqlen, int64_t dim, int64_t width,
                                 int x_dtype);

/* Bytes of device workspace ccv1d_bwd needs for these very tensors: the path its planner picks for
 * the alignment of x, dout, dfinal_states (may be NULL) and a contiguous dx (batch, seqlen, dim),
 * and a workspace aligned to 16 bytes (every torch allocation is). Never more than
 * ccv1d_bwd_workspace_bytes(batch, seqlen, dim, width, x_dtype), and often much less: that bound
 * covers the generic kernels' tiling (one partial row per 64 rows), which aligned rows never take.
 * Like the reference's partials allocation (causal_conv1d.py:493), sized from the launch it serves.
 * 0 for empty or invalid shapes. */
size_t ccv1d_bwd_workspace_bytes_for(const void* x, int64_t x_stride_b, int64_t x_stride_t,
                                     int x_dtype, const int32_t* seq_idx, const void* dout,
                                     int64_t dout_stride_b, int64_t dout_stride_t,
                                     const void* dfinal_states, const void* dx, int64_t batch,
                                     int64_t seqlen, int64_t dim, int64_t width);

/* Backward pass. Replaces the host launcher `_bwd` of the reference (causal_conv1d.py:475-541)
 * together with `_bwd_kernel` (causal_conv1d.py:167-341), `_reduce_partials_kernel`
 * (causal_conv1d.py:344-374) and the empty-input path (causal_conv1d.py:480-489).
 *
 *  x, weight, bias, seq_idx, initial_states, silu: as passed to ccv1d_fwd
 *  dout              (batch, seqlen, dim), strides (dout_stride_b, dout_stride_t, 1), type x_dtype
 *  dfinal_states     (batch, width - 1, dim) or NULL, type x_dtype: gradient of final_states
 *  dx                (batch, seqlen, dim), type x_dtype (always written)
 *  dinitial_states   (batch, width - 1, dim) or NULL, type init_dtype; written when non-NULL, which
 *                    requires initial_states
 *  dweight           (dim, width), type weight_dtype (always written)
 *  dbias             (dim,), type bias_dtype; required iff bias is non-NULL
 *  workspace         device buffer of at least ccv1d_bwd_workspace_bytes() bytes (256-byte aligned);
 *                    may be NULL when that size is 0
 *
 * dweight and dbias are deterministic: the summation order depends only on the shape.
 */
int ccv1d_bwd(const void* x, int64_t x_stride_b, int64_t x_stride_t, int x_dtype,
              const void* weight, int weight_dtype,
              const void* bias, int bias_dtype,
              const int32_t* seq_idx,
              const void* initial_states, int init_dtype,
              const void* dout, int64_t dout_stride_b, int64_t dout_stride_t,
              const void* dfinal_states,
              void* dx, void* dinitial_states, void* dweight, void* dbias,
              void* workspace, size_t workspace_bytes,
              int64_t batch, int64_t seqlen, int64_t dim, int64_t width,
              int silu, int device, void* stream);

/* Backward that writes dx with caller-given strides, for callers that fuse the convolution with
 * the projection before it (the Mamba-2 in_proj epilogue): dx goes straight into its slice of the
 * gradient of the projection's output, e.g. channels [c0, c0 + dim) of a (batch, seqlen, width_all)
 * buffer, so no later copy assembles that gradient (which would read and write dx once more). The
 * reference has no counterpart (its dx is always a new contiguous tensor, causal_conv1d.py:478);
 * the CUDA causal-conv1d package's backward takes its dx buffer the same way.
 * Arguments and results are those of ccv1d_bwd, plus dx's strides in elements (unit channel
 * stride): dx_stride_t >= dim, dx_stride_b >= (seqlen - 1) * dx_stride_t + dim, and
 * (seqlen + width) * max(dx_stride_t, dim) < 2^31. Elements of the buffer outside dx's rows and
 * channels are left untouched. dx must not overlap x or dout (checked on the address ranges from
 * each one's first to its last element; CCV1D_ERR_INVALID), in this entry point and in
 * ccv1d_bwd. */
int ccv1d_bwd_dx_strided(const void* x, int64_t x_stride_b, int64_t x_stride_t, int x_dtype,
                         const void* weight, int weight_dtype,
                         const void* bias, int bias_dtype,
                         const int32_t* seq_idx,
                         const void* initial_states, int init_dtype,
                         const void* dout, int64_t dout_stride_b, int64_t dout_stride_t,
                         const void* dfinal_states,
                         void* dx, int64_t dx_stride_b, int64_t dx_stride_t,
                         void* dinitial_states, void* dweight, void* dbias,
                         void* workspace, size_t workspace_bytes,
                         int64_t batch, int64_t seqlen, int64_t dim, int64_t width,
                         int silu, int device, void* stream);

/* Allocation-free backward. It has no counterpart in the reference: it is for callers that cannot
 * allocate device memory or pass a workspace (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc). Arguments and results are those of ccv1d_bwd without the
 * workspace: the fp32 partial sums of dweight/dbias go to a scratch array built into the library,
 * CCV1D_NOALLOC_SCRATCH_BYTES bytes on every device it runs on, held until the process ends. The
 * call allocates nothing.
 *  - Shapes whose partial sums need more (ccv1d_bwd_workspace_bytes() gives an upper bound) are
 *    refused with CCV1D_ERR_WORKSPACE before anything is launched.
 *  - Calls that overlap on one device share its scratch and race: the caller orders them (one
 *    stream, or events between streams). The scratch keeps the last call's contents; each call
 *    writes every partial sum before reading it, so nothing needs clearing.
 *  - The first call on a device resolves the scratch's device address (hipGetSymbolAddress); make
 *    it outside stream capture. */
#define CCV1D_NOALLOC_SCRATCH_BYTES (32u << 20)

int ccv1d_bwd_noalloc(const void* x, int64_t x_stride_b, int64_t x_stride_t, int x_dtype,
                      const void* weight, int weight_dtype,
                      const void* bias, int bias_dtype,
                      const int32_t* seq_idx,
                      const void* initial_states, int init_dtype,
                      const void* dout, int64_t dout_stride_b, int64_t dout_stride_t,
                      const void* dfinal_states,
                      void* dx, void* dinitial_states, void* dweight, void* dbias,
                      int64_t batch, int64_t seqlen, int64_t dim, int64_t width,
                      int silu, int device, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* CCV1D_H */
