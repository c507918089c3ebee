"""Backward for callers that fuse the convolution with the projection in front of it.

In a Mamba-2 layer the convolution's input xBC is a channel slice of the in_proj output zxbcdt,
(batch, seqlen, d_in_proj). Through autograd the gradient of that slice comes back as a new
contiguous tensor, and assembling the gradient of zxbcdt (the split's backward concatenates the
slices' gradients) reads and writes it once more: at Mamba-2 2.7B's shape (batch 8, seqlen 4096,
5376 channels, bf16) 704 MB per training step on top of the convolution's own 1.76 GB.
`causal_conv1d_bwd` writes dx straight into a caller-given strided buffer instead, for example
channels [c0, c0 + dim) of a preallocated gradient of zxbcdt, as custom autograd functions of
fused Mamba layers do with the CUDA causal-conv1d package's backward. The reference has no such
entry point: its dx is always a new contiguous tensor (causal_conv1d.py:478). The kernels are
those of causal_conv1d_fn's backward (libccv1d.so, ccv1d_bwd_dx_strided); only dx's addressing
differs.
"""

import torch
from torch import Tensor

from . import _ffi
from .causal_conv1d import _channels_contiguous, _check_grads, _check_inputs, _silu_flag


def causal_conv1d_bwd(
    x: Tensor,
    weight: Tensor,
    bias: Tensor | None,
    dout: Tensor,
    seq_idx: Tensor | None = None,
    initial_states: Tensor | None = None,
    dfinal_states: Tensor | None = None,
    dx: Tensor | None = None,
    return_dinitial_states: bool = False,
    activation: str | None = None,
) -> tuple[Tensor, Tensor, Tensor | None, Tensor | None]:
    """Gradients of causal_conv1d_fn(x, weight, bias, seq_idx, initial_states, activation=...)
    for the upstream gradient `dout` (and `dfinal_states` of the final states, when the forward
    returned them).

    dx: optional output buffer of shape (batch, seqlen, dim) and x's dtype with a unit channel
        stride and non-overlapping rows, e.g. zxbcdt_grad[..., c0:c0 + dim]; elements of the
        underlying storage outside it are left untouched. A new contiguous tensor when None.

    Returns (dx, dweight, dbias, dinitial_states): dbias is None without a bias, and
    dinitial_states is None unless return_dinitial_states (which needs initial_states).
    """
    silu = _silu_flag(activation)
    _check_inputs(x, weight, bias, seq_idx, initial_states)
    if seq_idx is not None:
        assert dfinal_states is None, "cannot take final-state gradients if seq_idx is not None"
    if return_dinitial_states:
        assert initial_states is not None, "return_dinitial_states requires initial_states"
    x = _channels_contiguous(x)
    dout = _channels_contiguous(dout)
    weight = weight.contiguous()
    bias = bias.contiguous() if bias is not None else None
    seq_idx = seq_idx.to(torch.int32).contiguous() if seq_idx is not None else None
    initial_states = initial_states.contiguous() if initial_states is not None else None
    dfinal_states = dfinal_states.contiguous() if dfinal_states is not None else None
    B, T, D = x.shape
    W = weight.shape[1]
    _check_grads(x, W, dout, dfinal_states)
    if dx is None:
        dx = torch.empty(B, T, D, device=x.device, dtype=x.dtype)
    else:
        assert dx.shape == x.shape, "dx must have the shape of x"
        assert dx.dtype == x.dtype, "dx must have the dtype of x"
        assert dx.get_device() == x.get_device(), "dx must be on the device of x"
        assert dx.stride(-1) == 1, "dx must have a unit channel stride"
    dinit = torch.empty_like(initial_states) if return_dinitial_states else None
    dweight = torch.empty_like(weight)
    dbias = torch.empty_like(bias) if bias is not None else None
    nbytes = _ffi.bwd_workspace_bytes(B, T, D, W, x.dtype)
    workspace = torch.empty(nbytes, device=x.device, dtype=torch.uint8) if nbytes else None
    _ffi.bwd_dx_strided(x, weight, bias, seq_idx, initial_states, dout, dfinal_states, dx, dinit,
                        dweight, dbias, workspace, silu)
    return dx, dweight, dbias, dinit
