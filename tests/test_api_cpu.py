"""The Python boundary without a GPU: import surface, signature and the reference's error behaviour
(causal_conv1d.py:397-408, :605-610), which all fire before any kernel launch."""

import inspect

import pytest
import torch

import causal_conv1d_triton
from causal_conv1d_triton import causal_conv1d_fn


def test_import_surface():
    # causal_conv1d_triton/__init__.py:1-3 of the reference
    assert causal_conv1d_triton.__all__ == ["causal_conv1d_fn"]


def test_signature_matches_reference():
    # causal_conv1d.py:579-588 of the reference
    sig = inspect.signature(causal_conv1d_fn)
    assert list(sig.parameters) == ["x", "weight", "bias", "seq_idx", "initial_states",
                                    "return_final_states", "final_states_out", "activation"]
    defaults = {k: v.default for k, v in sig.parameters.items()}
    assert defaults["bias"] is None and defaults["seq_idx"] is None
    assert defaults["initial_states"] is None and defaults["final_states_out"] is None
    assert defaults["return_final_states"] is False and defaults["activation"] is None


def _t(B=2, T=8, D=4, W=4):
    return torch.randn(B, T, D), torch.randn(D, W)


def test_bad_activation():
    x, w = _t()
    with pytest.raises(NotImplementedError):
        causal_conv1d_fn(x, w, activation="relu")


def test_seq_idx_with_final_states():
    x, w = _t()
    with pytest.raises(AssertionError, match="final states"):
        causal_conv1d_fn(x, w, seq_idx=torch.zeros(2, 8, dtype=torch.int32),
                         return_final_states=True)


def test_final_states_out_requires_return():
    x, w = _t()
    with pytest.raises(AssertionError, match="return_final_states"):
        causal_conv1d_fn(x, w, final_states_out=torch.empty(2, 3, 4))


def test_cpu_tensors_rejected():
    x, w = _t()
    with pytest.raises(AssertionError):
        causal_conv1d_fn(x, w)


@pytest.mark.parametrize("case", ["x2d", "w_dim", "w1", "bias", "init", "seq"])
def test_shape_checks(case):
    x, w = _t()
    kw = {}
    if case == "x2d":
        x = x[0]
    elif case == "w_dim":
        w = torch.randn(5, 4)
    elif case == "w1":
        w = torch.randn(4, 1)
    elif case == "bias":
        kw["bias"] = torch.randn(5)
    elif case == "init":
        kw["initial_states"] = torch.randn(2, 2, 4)
    elif case == "seq":
        kw["seq_idx"] = torch.zeros(2, 7, dtype=torch.int32)
    with pytest.raises(AssertionError):
        causal_conv1d_fn(x, w, **kw)


def test_ffi_refuses_unsupported_dtype():
    from causal_conv1d_triton import _ffi

    with pytest.raises(TypeError):
        _ffi._code(torch.zeros(1, dtype=torch.int32))


@pytest.mark.parametrize("bias", [False, True])
@pytest.mark.parametrize("init", [False, True])
@pytest.mark.parametrize("final", [False, True])
def test_custom_op_fake_shapes(bias, init, final):
    """The torch.library operators (used under torch.compile) report the shapes and dtypes of the
    tensors the kernels write, checked with fake CUDA tensors (no device needed)."""
    from torch._subclasses.fake_tensor import FakeTensorMode

    B, T, D, W = 2, 33, 24, 4
    with FakeTensorMode():
        x = torch.empty(B, T, D, device="cuda", dtype=torch.bfloat16)
        w = torch.empty(D, W, device="cuda", dtype=torch.float32)
        b = torch.empty(D, device="cuda", dtype=torch.float16) if bias else None
        s0 = torch.empty(B, W - 1, D, device="cuda", dtype=torch.float32) if init else None
        out, fin = torch.ops.causal_conv1d_amd.fwd(x, w, b, None, s0, final, True)
        assert out.shape == (B, T, D) and out.dtype == x.dtype and out.device == x.device
        assert fin.shape == ((B, W - 1, D) if final else (0,))
        dfin = torch.empty(B, W - 1, D, device="cuda", dtype=x.dtype) if final else None
        dx, dw, db, di = torch.ops.causal_conv1d_amd.bwd(x, w, b, None, s0, out, dfin, init, True)
        assert dx.shape == x.shape and dx.dtype == x.dtype
        assert dw.shape == w.shape and dw.dtype == w.dtype
        assert db.shape == ((D,) if bias else (0,)) and (not bias or db.dtype == b.dtype)
        assert di.shape == ((B, W - 1, D) if init else (0,)) and (not init or di.dtype == s0.dtype)


@pytest.mark.parametrize("which", ["weight", "bias", "initial_states", "seq_idx"])
def test_host_tensors_rejected_before_launch(which):
    """Every optional tensor must be on x's GPU: the library takes raw device addresses, so a host
    tensor is refused with an AssertionError (as the reference refuses a host weight,
    causal_conv1d.py:403) before anything is launched. Fake CUDA tensors stand in for the GPU, and
    the tensor under test is a real host tensor."""
    from torch._subclasses.fake_tensor import FakeTensorMode

    B, T, D, W = 2, 16, 8, 4
    host = {
        "weight": torch.randn(D, W),
        "bias": torch.randn(D),
        "initial_states": torch.randn(B, W - 1, D),
        "seq_idx": torch.zeros(B, T, dtype=torch.int32),
    }[which]
    with FakeTensorMode(allow_non_fake_inputs=True):
        x = torch.empty(B, T, D, device="cuda", dtype=torch.bfloat16)
        kw = {"weight": torch.empty(D, W, device="cuda")}
        kw[which] = host
        with pytest.raises(AssertionError, match="device of x"):
            causal_conv1d_fn(x, **kw)


@pytest.mark.parametrize("which", ["dout", "dfinal_states"])
def test_host_gradients_rejected_before_launch(which):
    """The backward entry refuses incoming gradients that are not on x's device."""
    from torch._subclasses.fake_tensor import FakeTensorMode

    from causal_conv1d_triton.causal_conv1d import _bwd

    B, T, D, W = 2, 16, 8, 4
    with FakeTensorMode(allow_non_fake_inputs=True):
        x = torch.empty(B, T, D, device="cuda", dtype=torch.bfloat16)
        w = torch.empty(D, W, device="cuda")
        dout = torch.empty(B, T, D, device="cuda", dtype=torch.bfloat16)
        dfin = torch.empty(B, W - 1, D, device="cuda", dtype=torch.bfloat16)
        if which == "dout":
            dout = torch.randn(B, T, D).to(torch.bfloat16)
        else:
            dfin = torch.randn(B, W - 1, D).to(torch.bfloat16)
        with pytest.raises(AssertionError, match="device of x"):
            _bwd(x, w, None, None, None, dout, dfin, False, True)


@pytest.mark.parametrize("which,shape", [
    ("dout", (2, 15, 8)), ("dfinal_states", (3, 8)), ("dfinal_states", (2, 3, 7)),
    ("dfinal_states", (2, 2, 8)),
])
def test_misshaped_gradients_rejected_before_launch(which, shape):
    """The backward entries refuse incoming gradients smaller (or otherwise shaped) than out and the
    final states: the library would read batch * seqlen * dim and batch * (width - 1) * dim
    elements from them. Checked before any launch, in causal_conv1d_bwd (fused.py) and in the
    autograd node's backward."""
    from torch._subclasses.fake_tensor import FakeTensorMode

    from causal_conv1d_triton.causal_conv1d import _bwd
    from causal_conv1d_triton.fused import causal_conv1d_bwd

    B, T, D, W = 2, 16, 8, 4
    with FakeTensorMode():
        x = torch.empty(B, T, D, device="cuda", dtype=torch.bfloat16)
        w = torch.empty(D, W, device="cuda")
        dout = torch.empty(B, T, D, device="cuda", dtype=torch.bfloat16)
        dfin = torch.empty(B, W - 1, D, device="cuda", dtype=torch.bfloat16)
        bad = torch.empty(shape, device="cuda", dtype=torch.bfloat16)
        if which == "dout":
            dout = bad
        else:
            dfin = bad
        with pytest.raises(AssertionError, match="shape|width - 1"):
            causal_conv1d_bwd(x, w, None, dout, dfinal_states=dfin, activation="silu")
        with pytest.raises(AssertionError, match="shape|width - 1"):
            _bwd(x, w, None, None, None, dout, dfin, False, True)
