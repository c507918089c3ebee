"""The reference's math as a PyTorch CPU grouped conv1d, fp32: the CPU baseline of the benchmark.

TEST INFRASTRUCTURE ONLY: imported by bench.py's cpu_baseline leg (and tests/), never by the product
package. The reference has no CPU path of its own (causal_conv1d.py:403 asserts x.is_cuda); its
README states the operation as a depthwise causal conv1d (README.md:7), which is what this computes:
left-pad the time axis by width-1 zeros, F.conv1d with groups=dim, add bias, silu; the backward is
torch autograd of that graph.

Inputs are laid out (batch, dim, seqlen) contiguous fp32 (the layout F.conv1d reads), prepared by the
caller outside any timed region.
"""

import torch
import torch.nn.functional as F


def prepare(x_btd, w, bias, dy_btd):
    """fp32 (B, D, T) contiguous copies of x and dy; fp32 weight (D, 1, W) and bias, with grads."""
    x = x_btd.detach().float().transpose(1, 2).contiguous().requires_grad_(True)
    dy = dy_btd.detach().float().transpose(1, 2).contiguous()
    wt = w.detach().float()[:, None, :].clone().requires_grad_(True)
    b = None if bias is None else bias.detach().float().clone().requires_grad_(True)
    return x, wt, b, dy


def fwd(x, wt, b, silu):
    """out (B, D, T) = act(conv1d(pad_left(x, W-1), wt, b, groups=D))."""
    z = F.conv1d(F.pad(x, (wt.shape[-1] - 1, 0)), wt, b, groups=x.shape[1])
    return F.silu(z) if silu else z


def fwd_bwd(x, wt, b, dy, silu):
    """One forward and the gradients of x, weight and bias for the upstream gradient dy."""
    out = fwd(x, wt, b, silu)
    inputs = (x, wt) if b is None else (x, wt, b)
    return out, torch.autograd.grad(out, inputs, dy)
