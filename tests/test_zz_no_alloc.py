"""The allocation-free backward (ccv1d_bwd_noalloc) against the backward with a caller workspace
(ccv1d_bwd), both called through the C ABI: same kernels, tiling and summation order, so every
output must be bit-identical. Calls follow each other on one device with no clearing of the
built-in scratch in between, larger shapes before smaller ones, so a result that read partial sums
left by an earlier call would differ. One case is also checked against the CPU oracle on a channel
subset (bf16 outputs atol/rtol 1e-2, fp32 dweight/dbias rtol 1e-3). The refusal of shapes whose
partial sums exceed the scratch is host code, tested without a GPU in test_abi.py."""

import math

import pytest
import torch

import ccv1d_oracle as oracle
from causal_conv1d_triton import _ffi

pytestmark = pytest.mark.gpu

DEV = "cuda"


def _inputs(seed, B, T, D, W, xdt=torch.bfloat16, bias=True, init=False, seq=None):
    g = torch.Generator().manual_seed(seed)
    t = {
        "x": torch.randn(B, T, D, generator=g).to(xdt),
        "w": torch.randn(D, W, generator=g) / math.sqrt(W),
        "b": torch.randn(D, generator=g) if bias else None,
        "init": torch.randn(B, W - 1, D, generator=g).to(xdt) if init else None,
        "dy": torch.randn(B, T, D, generator=g).to(xdt),
        "seq": seq,
    }
    return {k: (None if v is None else v.to(DEV)) for k, v in t.items()}


def _outputs(t):
    x, w, b, init = t["x"], t["w"], t["b"], t["init"]
    return {"dx": torch.empty_like(x), "dw": torch.empty_like(w),
            "db": None if b is None else torch.empty_like(b),
            "dinit": None if init is None else torch.empty_like(init)}


def _with_workspace(t, silu=True):
    o = _outputs(t)
    B, T, D = t["x"].shape
    n = _ffi.bwd_workspace_bytes(B, T, D, t["w"].shape[1], t["x"].dtype)
    ws = torch.empty(n, dtype=torch.uint8, device=DEV) if n else None
    _ffi.bwd(t["x"], t["w"], t["b"], t["seq"], t["init"], t["dy"], None, o["dx"], o["dinit"],
             o["dw"], o["db"], ws, silu)
    return o


def _no_alloc(t, silu=True):
    o = _outputs(t)
    _ffi.bwd_noalloc(t["x"], t["w"], t["b"], t["seq"], t["init"], t["dy"], None, o["dx"],
                     o["dinit"], o["dw"], o["db"], silu)
    return o


def _same(a, b, what):
    for k in a:
        if a[k] is None:
            assert b[k] is None, (what, k)
        else:
            assert torch.equal(a[k], b[k]), (what, k)


def _seq(B, T, seed):
    g = torch.Generator().manual_seed(seed)
    s = torch.empty(B, T, dtype=torch.int32)
    for b in range(B):
        t, sid = 0, 0
        while t < T:
            n = int(torch.randint(20, 300, (1,), generator=g))
            s[b, t:t + n] = sid if sid % 5 else -1
            t, sid = t + n, sid + 1
    return s


# Larger requests first: each later call finds the scratch holding a larger earlier call's sums.
CASES = [
    ("benchmark shape", dict(B=4, T=8192, D=1024, W=4, init=True)),
    ("smaller, fast kernels", dict(B=2, T=700, D=256, W=4, init=True)),
    ("width 200: g in the scratch", dict(B=2, T=300, D=100, W=200, init=True)),
    ("generic kernels (width 20)", dict(B=2, T=333, D=100, W=20, init=True)),
    ("seq_idx, width 7", dict(B=2, T=1500, D=512, W=7, seq=True)),
    ("fp32 x, no bias", dict(B=1, T=64, D=64, W=3, xdt=torch.float32, bias=False)),
]


def test_no_alloc_matches_workspace_backward_in_sequence():
    """Two or more calls in a row, each smaller than the one before: bit-identical to ccv1d_bwd."""
    for i, (name, kw) in enumerate(CASES):
        kw = dict(kw)
        seq = _seq(kw["B"], kw["T"], i).to(DEV) if kw.pop("seq", False) else None
        t = _inputs(100 + i, seq=seq, **kw)
        ref = _with_workspace(t)
        got = _no_alloc(t)
        torch.cuda.synchronize()
        _same(ref, got, name)


def test_no_alloc_against_oracle():
    """A second, smaller call after the benchmark shape, checked against the oracle."""
    big = _inputs(7, 4, 8192, 1024, 4)
    _no_alloc(big)
    B, T, D, W = 2, 257, 256, 4
    t = _inputs(8, B, T, D, W, init=True)
    got = _no_alloc(t)
    torch.cuda.synchronize()
    cols = torch.tensor([0, 1, 100, 255])
    f = lambda a: None if a is None else a.index_select(-1, cols.to(DEV)).float().cpu().numpy()  # noqa: E731
    rdx, rdinit, rdw, rdb = oracle.bwd(f(t["x"]), t["w"][cols.to(DEV)].cpu().numpy(), f(t["dy"]),
                                       t["b"][cols.to(DEV)].cpu().numpy(), None, f(t["init"]),
                                       None, need_dinit=True, silu=True)
    pick = lambda a: a.index_select(-1, cols.to(DEV)).float().cpu()  # noqa: E731
    torch.testing.assert_close(pick(got["dx"]), torch.from_numpy(rdx), rtol=1e-2, atol=1e-2)
    torch.testing.assert_close(pick(got["dinit"]), torch.from_numpy(rdinit), rtol=1e-2, atol=1e-2)
    # fp32 sums against the oracle's float64 ones: rtol 1e-3, with an absolute floor of 1e-5 of
    # the entries' rms for sums that cancel to near zero (as in the parity tests)
    for key, ref in (("dw", rdw), ("db", rdb)):
        ref = torch.from_numpy(ref)
        floor = 1e-5 * ref.pow(2).mean().sqrt().item() + 1e-7
        torch.testing.assert_close(got[key][cols.to(DEV)].double().cpu(), ref, rtol=1e-3,
                                   atol=floor)
