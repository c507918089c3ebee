"""torch.compile and torch.library: under torch.compile, causal_conv1d_fn goes through the custom
operators causal_conv1d_amd::fwd / ::bwd. They run the same kernels as the eager path, so the compiled
function must give the same bits (outputs and every gradient), trace without a graph break, and the
operators must pass torch.library.opcheck (schema, fake implementation, autograd registration,
AOT dispatch)."""

import pytest
import torch

from causal_conv1d_triton import causal_conv1d_fn

pytestmark = pytest.mark.gpu

DEV = "cuda"


def _inputs(seed, B=2, T=300, D=96, W=4, init=False, seq=False):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(B, T, D, generator=g).to(torch.bfloat16)
    w = torch.randn(D, W, generator=g) / 2
    b = torch.randn(D, generator=g)
    s0 = torch.randn(B, W - 1, D, generator=g).to(torch.bfloat16) if init else None
    dy = torch.randn(B, T, D, generator=g).to(torch.bfloat16)
    sq = None
    if seq:
        sq = torch.zeros(B, T, dtype=torch.int32)
        sq[:, T // 3:] = 1
        sq[:, -T // 10:] = -1
    return x, w, b, s0, dy, sq


def _run(fn, x, w, b, s0, dy, sq, final):
    leaves = [t.to(DEV).detach().requires_grad_(True) for t in (x, w, b)]
    init = None if s0 is None else s0.to(DEV).detach().requires_grad_(True)
    seq = None if sq is None else sq.to(DEV)
    res = fn(*leaves, init, seq)
    out, fin = res if final else (res, None)
    loss = (out.float() * dy.to(DEV).float()).sum()
    if fin is not None:
        loss = loss + fin.float().sum()
    loss.backward()
    grads = [t.grad for t in leaves] + ([] if init is None else [init.grad])
    torch.cuda.synchronize()
    return [out] + ([] if fin is None else [fin]) + grads


@pytest.mark.parametrize("variant", ["bias_silu", "init_final", "seq"])
def test_compiled_matches_eager_bit_for_bit(variant):
    init = variant == "init_final"
    final = variant == "init_final"
    seq = variant == "seq"

    def f(x, w, b, s0, sq):
        return causal_conv1d_fn(x, w, b, seq_idx=sq, initial_states=s0, return_final_states=final,
                                activation="silu")

    torch._dynamo.reset()
    compiled = torch.compile(f, backend="aot_eager", fullgraph=True)
    args = _inputs(7, init=init, seq=seq)
    eager = _run(f, *args, final)
    comp = _run(compiled, *args, final)
    assert len(eager) == len(comp)
    for i, (a, c) in enumerate(zip(eager, comp)):
        assert torch.equal(a, c), f"tensor {i} of {variant} differs between eager and compiled"


def test_opcheck_forward_and_backward_operators():
    x, w, b, s0, dy, _ = _inputs(3, T=130, D=64, init=True)
    x, w, b, s0, dy = (t.to(DEV) for t in (x, w, b, s0, dy))
    fwd = torch.ops.causal_conv1d_amd.fwd.default
    bwd = torch.ops.causal_conv1d_amd.bwd.default
    torch.library.opcheck(fwd, (x.requires_grad_(), w.requires_grad_(), b, None, s0, True, True))
    torch.library.opcheck(fwd, (x.detach(), w.detach(), None, None, None, False, False))
    torch.library.opcheck(bwd, (x.detach(), w.detach(), b, None, s0, dy, None, True, True))
