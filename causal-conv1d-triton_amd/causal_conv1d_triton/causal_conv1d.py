"""Causal depthwise conv1d over channels-last inputs for AMD Instinct MI355X (gfx950), with forward
and backward:

    out[b, t, d] = act(bias[d] + sum_k weight[d, k] * x[b, t - (W - 1) + k, d])

where positions t < 0 read `initial_states` (or zero). x is (batch, seqlen, dim) and the states are
(batch, width - 1, dim): the states are literally the inputs preceding x[:, 0]. Any width >= 2 and
fp32/fp16/bf16 inputs are supported; accumulation is fp32.

This module is the Python side of the drop-in: it keeps the public function, autograd wiring,
argument checks, canonicalisation and output allocation of the reference
(causal_conv1d_triton/causal_conv1d.py:377-639), and hands every launch to the hand-written HIP
kernels of libccv1d.so through its C ABI (include/ccv1d.h). There is no other compute path.
"""

import torch
from torch import Tensor

from . import _ffi


def _check_inputs(x, weight, bias, seq_idx, initial_states):
    """Same assertions as the reference's _check_inputs (causal_conv1d.py:397-408). Each shape is
    read once and devices are compared by index (x is on a GPU), which keeps the checks to about
    1 us per call, a tenth of an eager decode step."""
    xs = x.shape
    assert len(xs) == 3, "x must be (batch, seqlen, dim)"
    B, T, D = xs
    ws = weight.shape
    assert len(ws) == 2 and ws[0] == D, "weight must be (dim, width)"
    W = ws[1]
    assert W >= 2, "width must be >= 2"
    assert x.is_cuda and weight.get_device() == x.get_device()
    assert bias is None or bias.shape == (D,)
    assert initial_states is None or initial_states.shape == (B, W - 1, D)
    assert seq_idx is None or seq_idx.shape == (B, T)
    # Offsets within one batch element are computed in int32.
    st = x.stride(1)
    assert (T + W) * (st if st > D else D) < 2**31


def _channels_contiguous(t: Tensor) -> Tensor:
    """Copies only when the channel stride is not 1 (causal_conv1d.py:411-412)."""
    return t if t.stride(-1) == 1 else t.contiguous()


def _fwd(x, weight, bias, seq_idx, initial_states, final_states, silu):
    """Allocates `out` and runs the forward kernel (reference `_fwd`, causal_conv1d.py:433-472).
    T == 0 is handled inside the library (final_states = initial_states or zeros)."""
    B, T, D = x.shape
    out = torch.empty(B, T, D, device=x.device, dtype=x.dtype)
    _ffi.fwd(x, weight, bias, seq_idx, initial_states, out, final_states, silu)
    return out


def _bwd(x, weight, bias, seq_idx, initial_states, dout, dfinal_states, need_dinit, silu):
    """Allocates the gradients and the fp32 partial-sum workspace and runs the backward kernels
    (reference `_bwd`, causal_conv1d.py:475-541). dweight and dbias are always computed; the
    empty-input cases (dweight = dbias = 0, dinit = dfinal) are handled inside the library."""
    B, T, D = x.shape
    W = weight.shape[1]
    dx = torch.empty(B, T, D, device=x.device, dtype=x.dtype)
    dinit = torch.empty_like(initial_states) if need_dinit else None
    dweight = torch.empty_like(weight)
    dbias = torch.empty_like(bias) if bias is not None else None
    nbytes = _ffi.bwd_workspace_bytes(B, T, D, W, x.dtype)
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


class _CausalConv1dFn(torch.autograd.Function):
    """Autograd wiring of the reference (causal_conv1d.py:544-576): saves the inputs (not the
    output) and recomputes the pre-activation in backward."""

    @staticmethod
    def forward(ctx, x, weight, bias, seq_idx, initial_states, return_final_states, silu):
        final_states = None
        if return_final_states:
            final_states = torch.empty(
                x.shape[0], weight.shape[1] - 1, x.shape[2], device=x.device, dtype=x.dtype
            )
        out = _fwd(x, weight, bias, seq_idx, initial_states, final_states, silu)
        ctx.save_for_backward(x, weight, bias, seq_idx, initial_states)
        ctx.silu = silu
        ctx.return_final_states = return_final_states
        return (out, final_states) if return_final_states else out

    @staticmethod
    def backward(ctx, dout, *args):
        x, weight, bias, seq_idx, initial_states = ctx.saved_tensors
        dfinal_states = args[0] if ctx.return_final_states else None
        if dfinal_states is not None:
            dfinal_states = dfinal_states.contiguous()
        need_dinit = initial_states is not None and ctx.needs_input_grad[4]
        dx, dweight, dbias, dinit = _bwd(
            x,
            weight,
            bias,
            seq_idx,
            initial_states,
            _channels_contiguous(dout),
            dfinal_states,
            need_dinit,
            ctx.silu,
        )
        return dx, dweight, dbias, None, dinit, None, None


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
    """Causal depthwise conv1d over channels-last inputs (reference causal_conv1d.py:579-639).

    x: (batch, seqlen, dim); must be contiguous along dim
    weight: (dim, width), width >= 2
    bias: (dim,)
    seq_idx: (batch, seqlen) integer sequence ids for packed sequences. Positions with negative ids
        are considered padding, and give zero outputs. Can be combined with initial_states, which
        count as part of seq_idx[:, 0]'s sequence, but cannot be combined with return_final_states
    initial_states: (batch, width - 1, dim), the inputs preceding x[:, 0]
    return_final_states: also return the last width - 1 rows of concat(initial_states, x), i.e. the
        initial_states for continuing the sequence; supports grad
    final_states_out: optional (batch, width - 1, dim) buffer to copy the final states into
    activation: None, "silu", or "swish"

    Returns out of shape (batch, seqlen, dim) and dtype x.dtype, or (out, final_states).
    """
    if activation not in (None, "silu", "swish"):
        raise NotImplementedError("activation must be None, silu, or swish")
    if seq_idx is not None:
        assert not return_final_states, "cannot return final states if seq_idx is not None"
    if final_states_out is not None:
        assert return_final_states, "final_states_out requires return_final_states=True"
    _check_inputs(x, weight, bias, seq_idx, initial_states)

    x = _channels_contiguous(x)
    weight = weight.contiguous()
    bias = bias.contiguous() if bias is not None else None
    seq_idx = seq_idx.to(torch.int32).contiguous() if seq_idx is not None else None
    initial_states = initial_states.contiguous() if initial_states is not None else None
    silu = activation is not None

    needs_grad = torch.is_grad_enabled() and any(
        t is not None and t.requires_grad for t in (x, weight, bias, initial_states)
    )
    if torch.compiler.is_compiling():
        # Under torch.compile the passes go through the registered custom operators.
        out, final_states = _fwd_op(x, weight, bias, seq_idx, initial_states, return_final_states,
                                    silu)
        result = (out, final_states) if return_final_states else out
    elif needs_grad:
        result = _CausalConv1dFn.apply(
            x, weight, bias, seq_idx, initial_states, return_final_states, silu
        )
    else:
        final_states = None
        if return_final_states:
            final_states = torch.empty(
                x.shape[0], weight.shape[1] - 1, x.shape[2], device=x.device, dtype=x.dtype
            )
        out = _fwd(x, weight, bias, seq_idx, initial_states, final_states, silu)
        result = (out, final_states) if return_final_states else out

    if final_states_out is not None:
        out, final_states = result
        result = out, final_states_out.copy_(final_states)
    return result
