"""Causal depthwise conv1d over channels-last inputs for AMD Instinct MI355X (gfx950), with forward
and backward. Per channel d, output row t is a dot product of the filter weight[d, 0:W] with input
rows t-W+1 .. t (the last filter tap meets row t), plus bias[d], through an optional silu; rows
before 0 come from `initial_states`, the W-1 rows that precede x[:, 0] (zeros without them).
x is (batch, seqlen, dim), the states (batch, width - 1, dim). Any width >= 2; fp32, fp16 and
bf16 inputs; fp32 arithmetic.

This module is the Python side of the drop-in: it keeps the public function, autograd wiring,
argument checks, canonicalisation and output allocation of the reference
(causal_conv1d_triton/causal_conv1d.py:377-639), and hands every launch to the hand-written HIP
kernels of libccv1d.so through its C ABI (include/ccv1d.h). There is no other compute path.
"""

import torch
from torch import Tensor

from . import _ffi


def _check_inputs(x, weight, bias, seq_idx, initial_states):
    """The reference's argument assertions (causal_conv1d.py:397-408), plus one it leaves to its
    Triton launcher: every optional tensor must sit on x's GPU, since the library receives raw
    device addresses and a host tensor's address would reach a kernel. Each shape is read once and
    devices are compared by index (x is on a GPU), which keeps the checks to about 1 us per call, a
    tenth of an eager decode step."""
    xs = x.shape
    assert len(xs) == 3, "x must be (batch, seqlen, dim)"
    B, T, D = xs
    ws = weight.shape
    assert len(ws) == 2 and ws[0] == D, "weight must be (dim, width)"
    W = ws[1]
    assert W >= 2, "width must be >= 2"
    assert x.is_cuda, "x must be on a GPU"
    dev = x.get_device()
    assert weight.get_device() == dev, "weight must be on the device of x"
    if bias is not None:
        assert bias.shape == (D,), "bias must be (dim,)"
        assert bias.get_device() == dev, "bias must be on the device of x"
    if initial_states is not None:
        assert initial_states.shape == (B, W - 1, D), "initial_states must be (batch, width - 1, dim)"
        assert initial_states.get_device() == dev, "initial_states must be on the device of x"
    if seq_idx is not None:
        assert seq_idx.shape == (B, T), "seq_idx must be (batch, seqlen)"
        assert seq_idx.get_device() == dev, "seq_idx must be on the device of x"
    # The library indexes the elements of one batch row, halo included, with 32-bit signed offsets
    # (the C ABI refuses larger rows; its vectorised kernels also need the byte offsets below 2^32
    # and otherwise take the generic ones).
    st = x.stride(1)
    assert (T + W) * (st if st > D else D) < 2**31, "seqlen * dim too large for 32-bit offsets"


def _check_grads(x, width, dout, dfinal_states):
    """The backward's incoming gradients must sit on x's device (the reference's launcher refuses
    host tensors; here their addresses would reach a kernel) and have the shapes of out and of the
    final states: the library reads batch * seqlen * dim elements of dout and batch * (width - 1)
    * dim of dfinal_states, so a smaller tensor would be read past its end."""
    dev = x.get_device()
    assert dout.get_device() == dev, "the gradient of out must be on the device of x"
    assert dout.shape == x.shape, "the gradient of out must have the shape of x"
    if dfinal_states is not None:
        assert dfinal_states.get_device() == dev, (
            "the gradient of final_states must be on the device of x")
        B, _, D = x.shape
        assert dfinal_states.shape == (B, width - 1, D), (
            "the gradient of final_states must be (batch, width - 1, dim)")


def _channels_contiguous(t: Tensor) -> Tensor:
    """Copies only when the channel stride is not 1 (causal_conv1d.py:411-412)."""
    return t if t.stride(-1) == 1 else t.contiguous()


def _fwd(x, weight, bias, seq_idx, initial_states, final_states, silu, inference=False):
    """Allocates `out` and runs the forward kernel (reference `_fwd`, causal_conv1d.py:433-472).
    T == 0 is handled inside the library (final_states = initial_states or zeros). `inference`:
    no backward follows (the library then streams out past the caches)."""
    if not inference and _ffi._torch_native is not None:
        # Allocation and launch in one native call (None for tensor subclasses).
        out = _ffi._torch_native.fwd_train(x, weight, bias, seq_idx, initial_states, final_states,
                                           silu)
        if out is not None:
            return out
    B, T, D = x.shape
    out = torch.empty(B, T, D, device=x.device, dtype=x.dtype)
    _ffi.fwd(x, weight, bias, seq_idx, initial_states, out, final_states, silu, inference)
    return out


def _bwd(x, weight, bias, seq_idx, initial_states, dout, dfinal_states, need_dinit, silu):
    """Allocates the gradients and the fp32 partial-sum workspace and runs the backward kernels
    (reference `_bwd`, causal_conv1d.py:475-541). dweight and dbias are always computed; the
    empty-input cases (dweight = dbias = 0, dinit = dfinal) are handled inside the library."""
    if _ffi._torch_native is not None:
        # The same checks, allocations and launch in one native call (None for tensor subclasses).
        res = _ffi._torch_native.bwd(x, weight, bias, seq_idx, initial_states, dout, dfinal_states,
                                     need_dinit, silu)
        if res is not None:
            return res
    B, T, D = x.shape
    W = weight.shape[1]
    _check_grads(x, W, dout, dfinal_states)
    dx = torch.empty(B, T, D, device=x.device, dtype=x.dtype)
    dinit = torch.empty_like(initial_states) if need_dinit else None
    dweight = torch.empty_like(weight)
    dbias = torch.empty_like(bias) if bias is not None else None
    nbytes = _ffi.bwd_workspace_bytes_for(x, seq_idx, dout, dfinal_states, dx, W)
    workspace = torch.empty(nbytes, device=x.device, dtype=torch.uint8) if nbytes else None
    _ffi.bwd(x, weight, bias, seq_idx, initial_states, dout, dfinal_states, dx, dinit, dweight,
             dbias, workspace, silu)
    return dx, dweight, dbias, dinit


# ---------------------------------------------------------------------------------------------
# The two passes as torch.library custom operators, so that torch.compile traces
# causal_conv1d_fn without a graph break (the reference keeps its host code dynamo-friendly,
# causal_conv1d.py:386-394). The fake implementations give output shapes and dtypes; autograd is
# registered on the forward operator. Absent optional outputs are returned as empty tensors.
# ---------------------------------------------------------------------------------------------


@torch.library.custom_op("causal_conv1d_amd::fwd", mutates_args=(), device_types="cuda")
def _fwd_op(
    x: Tensor,
    weight: Tensor,
    bias: Tensor | None,
    seq_idx: Tensor | None,
    initial_states: Tensor | None,
    return_final_states: bool,
    silu: bool,
) -> tuple[Tensor, Tensor]:
    B, T, D = x.shape
    if return_final_states:
        final_states = torch.empty(B, weight.shape[1] - 1, D, device=x.device, dtype=x.dtype)
    else:
        final_states = x.new_empty(0)
    out = _fwd(x, weight, bias, seq_idx, initial_states,
               final_states if return_final_states else None, silu)
    return out, final_states


@_fwd_op.register_fake
def _fwd_fake(x, weight, bias, seq_idx, initial_states, return_final_states, silu):
    B, T, D = x.shape
    out = x.new_empty(B, T, D)
    final_states = x.new_empty(B, weight.shape[1] - 1, D) if return_final_states else x.new_empty(0)
    return out, final_states


@torch.library.custom_op("causal_conv1d_amd::bwd", mutates_args=(), device_types="cuda")
def _bwd_op(
    x: Tensor,
    weight: Tensor,
    bias: Tensor | None,
    seq_idx: Tensor | None,
    initial_states: Tensor | None,
    dout: Tensor,
    dfinal_states: Tensor | None,
    need_dinit: bool,
    silu: bool,
) -> tuple[Tensor, Tensor, Tensor, Tensor]:
    dx, dweight, dbias, dinit = _bwd(x, weight, bias, seq_idx, initial_states, dout,
                                     dfinal_states, need_dinit, silu)
    return (dx, dweight, dbias if dbias is not None else x.new_empty(0),
            dinit if dinit is not None else x.new_empty(0))


@_bwd_op.register_fake
def _bwd_fake(x, weight, bias, seq_idx, initial_states, dout, dfinal_states, need_dinit, silu):
    B, T, D = x.shape
    dbias = bias.new_empty(bias.shape) if bias is not None else x.new_empty(0)
    dinit = initial_states.new_empty(initial_states.shape) if need_dinit else x.new_empty(0)
    return x.new_empty(B, T, D), weight.new_empty(weight.shape), dbias, dinit


def _fwd_op_setup_context(ctx, inputs, output):
    x, weight, bias, seq_idx, initial_states, return_final_states, silu = inputs
    ctx.save_for_backward(x, weight, bias, seq_idx, initial_states)
    ctx.silu = silu
    ctx.return_final_states = return_final_states


def _fwd_op_backward(ctx, dout, dfinal_states):
    x, weight, bias, seq_idx, initial_states = ctx.saved_tensors
    need_dinit = initial_states is not None and ctx.needs_input_grad[4]
    if not ctx.return_final_states or dfinal_states is None:
        dfinal_states = None
    else:
        dfinal_states = dfinal_states.contiguous()
    dx, dweight, dbias, dinit = _bwd_op(x, weight, bias, seq_idx, initial_states,
                                        _channels_contiguous(dout), dfinal_states, need_dinit,
                                        ctx.silu)
    return (dx, dweight, dbias if bias is not None else None, None,
            dinit if need_dinit else None, None, None)


_fwd_op.register_autograd(_fwd_op_backward, setup_context=_fwd_op_setup_context)


def _new_final_states(x, width):
    """Uninitialised (batch, width - 1, dim) buffer of x's dtype for the forward to fill."""
    return torch.empty(x.shape[0], width - 1, x.shape[2], device=x.device, dtype=x.dtype)


class _CausalConv1dFn(torch.autograd.Function):
    """Eager autograd node (the reference's wiring, causal_conv1d.py:544-576). Only the inputs
    are kept for the backward, never `out`: the backward kernel recomputes the pre-activation it
    needs for silu, which costs arithmetic instead of a stored activation tensor."""

    @staticmethod
    def forward(ctx, x, weight, bias, seq_idx, initial_states, return_final_states, silu):
        final_states = _new_final_states(x, weight.shape[1]) if return_final_states else None
        out = _fwd(x, weight, bias, seq_idx, initial_states, final_states, silu)
        ctx.save_for_backward(x, weight, bias, seq_idx, initial_states)
        ctx.silu = silu
        ctx.return_final_states = return_final_states
        if return_final_states:
            return out, final_states
        return out

    @staticmethod
    def backward(ctx, dout, *rest):
        x, weight, bias, seq_idx, initial_states = ctx.saved_tensors
        # The final states' gradient exists only when they were returned (and autograd may still
        # hand over None when they did not reach the loss).
        dfinal = rest[0] if ctx.return_final_states and rest else None
        if dfinal is not None:
            dfinal = dfinal.contiguous()
        want_dinit = initial_states is not None and ctx.needs_input_grad[4]
        dx, dweight, dbias, dinit = _bwd(x, weight, bias, seq_idx, initial_states,
                                         _channels_contiguous(dout), dfinal, want_dinit, ctx.silu)
        # One gradient per forward input: x, weight, bias, seq_idx, initial_states and the two
        # flags.
        return dx, dweight, dbias, None, dinit, None, None


def _silu_flag(activation) -> bool:
    """True for silu (also spelled swish), False for no activation; anything else is refused as
    the reference refuses it (causal_conv1d.py:605-606)."""
    if activation is None:
        return False
    if activation == "silu" or activation == "swish":
        return True
    raise NotImplementedError("activation must be None, silu, or swish")


def causal_conv1d_fn(
    x: Tensor,
    weight: Tensor,
    bias: Tensor | None = None,
    seq_idx: Tensor | None = None,
    initial_states: Tensor | None = None,
    return_final_states: bool = False,
    final_states_out: Tensor | None = None,
    activation: str | None = None,
) -> Tensor | tuple[Tensor, Tensor]:
    """Depthwise causal convolution along time, with autograd (interface of the reference's
    causal_conv1d.py:579-639).

    Each channel d of x has its own filter weight[d, :] of length W; output row t sees input rows
    t-W+1 .. t, and rows before the start come from `initial_states` (zeros when it is None):

        out[b, t, d] = act(bias[d] + sum_{k<W} weight[d, k] * xx[b, t - W + 1 + k, d])
        xx = cat(initial_states, x) along time

    Arguments:
      x: (batch, seqlen, dim) on a GPU, bf16/fp16/fp32 (or fp64, on the scalar kernels), unit
         stride along dim (other strides, zero included, are free; a tensor without one is
         copied first).
      weight: (dim, width) with width >= 2, any float dtype; dweight comes back in that dtype.
      bias: optional (dim,).
      seq_idx: optional (batch, seqlen) integer ids marking packed sequences: a tap only reaches
         rows with the same id as the output row, and rows with a negative id are padding, whose
         outputs (and input gradients) are zero. initial_states are treated as rows of
         seq_idx[:, 0]'s sequence. Not allowed together with return_final_states.
      initial_states: optional (batch, width - 1, dim), the width - 1 rows that precede x[:, 0].
      return_final_states: also return the last width - 1 rows of cat(initial_states, x), which
         are the initial_states of a following chunk; gradients flow through them.
      final_states_out: optional (batch, width - 1, dim) tensor that receives a copy of the final
         states and is returned in their place; needs return_final_states=True.
      activation: None, or "silu" (same as "swish").

    Returns `out` (batch, seqlen, dim) in x's dtype, or `(out, final_states)`. All arithmetic is
    fp32; the kernels are the HIP kernels of libccv1d.so, with no other compute path.
    """
    silu = _silu_flag(activation)
    if seq_idx is not None:
        assert not return_final_states, "cannot return final states if seq_idx is not None"
    if final_states_out is not None:
        assert return_final_states, "final_states_out requires return_final_states=True"
    compiling = torch.compiler.is_compiling()
    if _ffi._torch_native is not None and not compiling:
        # Inference on plain tensors: checks, canonicalisation, allocation and the launch in one
        # native call (decode steps are host-bound). None: autograd must record the call, or an
        # argument is a tensor subclass; both continue below.
        res = _ffi._torch_native.fwd(x, weight, bias, seq_idx, initial_states,
                                     return_final_states, silu)
        if res is not None:
            if final_states_out is None:
                return res
            return res[0], final_states_out.copy_(res[1])
    _check_inputs(x, weight, bias, seq_idx, initial_states)
    x = _channels_contiguous(x)
    weight = weight.contiguous()
    if bias is not None:
        bias = bias.contiguous()
    if seq_idx is not None:
        seq_idx = seq_idx.to(torch.int32).contiguous()
    if initial_states is not None:
        initial_states = initial_states.contiguous()

    final_states = None
    if compiling:
        # Traced by torch.compile: the registered operators carry the passes and their autograd.
        out, final_states = _fwd_op(x, weight, bias, seq_idx, initial_states,
                                    return_final_states, silu)
    elif torch.is_grad_enabled() and (x.requires_grad or weight.requires_grad
                                      or (bias is not None and bias.requires_grad)
                                      or (initial_states is not None
                                          and initial_states.requires_grad)):
        res = _CausalConv1dFn.apply(x, weight, bias, seq_idx, initial_states,
                                    return_final_states, silu)
        out, final_states = res if return_final_states else (res, None)
    else:
        # Inference: no autograd node, the forward kernel writes straight into fresh buffers.
        if return_final_states:
            final_states = _new_final_states(x, weight.shape[1])
        out = _fwd(x, weight, bias, seq_idx, initial_states, final_states, silu, inference=True)

    if not return_final_states:
        return out
    if final_states_out is not None:
        final_states = final_states_out.copy_(final_states)
    return out, final_states
