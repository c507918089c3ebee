"""Binding of libccv1d.so, the C ABI declared in include/ccv1d.h.

The library is the only compute path: if it is missing or fails to load, every call raises. It must be
loaded after `import torch` so that it binds to the HIP runtime torch has already loaded (same
soname), which makes torch's streams and device pointers valid arguments.

The two launch entry points go through the package's CPython extension `_ccv1d_native`
(csrc/ccv1d_pyext.c) when it is built, which links the same libccv1d.so and converts the arguments
at a fraction of ctypes' per-call cost; otherwise, and for everything else, through ctypes. Both
call the same C functions with the same arguments.
"""

import ctypes
import os

import torch

_LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libccv1d.so")

DTYPE_CODES = {torch.float32: 0, torch.float16: 1, torch.bfloat16: 2, torch.float64: 3}

_c_i64 = ctypes.c_int64
_c_int = ctypes.c_int
_c_ptr = ctypes.c_void_p

_lib = None

try:
    from . import _ccv1d_native as _native
except ImportError:  # not built: the ctypes binding serves every call
    _native = None


class CCV1DError(RuntimeError):
    """A libccv1d call returned an error status."""


# The inference forward over torch tensors in one native call (csrc/ccv1d_torch.cpp), when built.
try:
    from . import _ccv1d_torch as _torch_native
except ImportError:  # not built: causal_conv1d_fn makes the call from Python
    _torch_native = None
else:
    _torch_native.set_error_type(CCV1DError)


def library_path() -> str:
    return _LIB_PATH


def load() -> ctypes.CDLL:
    """Loads libccv1d.so once and declares the signatures of its exports."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(_LIB_PATH):
        raise RuntimeError(
            f"{_LIB_PATH} is not built; run `make -C causal-conv1d-triton_amd` "
            "(or __graft_entry__.build()) first"
        )
    lib = ctypes.CDLL(_LIB_PATH)
    lib.ccv1d_abi_version.restype = _c_int
    lib.ccv1d_abi_version.argtypes = []
    lib.ccv1d_last_error.restype = ctypes.c_char_p
    lib.ccv1d_last_error.argtypes = []
    lib.ccv1d_fwd.restype = _c_int
    lib.ccv1d_fwd.argtypes = [
        _c_ptr, _c_i64, _c_i64, _c_int,  # x, strides, dtype
        _c_ptr, _c_int,  # weight
        _c_ptr, _c_int,  # bias
        _c_ptr,  # seq_idx
        _c_ptr, _c_int,  # initial_states
        _c_ptr, _c_ptr,  # out, final_states
        _c_i64, _c_i64, _c_i64, _c_i64,  # batch, seqlen, dim, width
        _c_int, _c_int, _c_ptr,  # silu, device, stream
    ]
    lib.ccv1d_fwd_inference.restype = _c_int
    lib.ccv1d_fwd_inference.argtypes = lib.ccv1d_fwd.argtypes
    lib.ccv1d_bwd_dx_strided.restype = _c_int
    lib.ccv1d_time_main_kernel.restype = _c_int
    lib.ccv1d_time_main_kernel.argtypes = [_c_ptr, _c_ptr]
    lib.ccv1d_bwd_workspace_bytes.restype = ctypes.c_size_t
    lib.ccv1d_bwd_workspace_bytes.argtypes = [_c_i64, _c_i64, _c_i64, _c_i64, _c_int]
    lib.ccv1d_bwd_workspace_bytes_for.restype = ctypes.c_size_t
    lib.ccv1d_bwd_workspace_bytes_for.argtypes = [
        _c_ptr, _c_i64, _c_i64, _c_int,  # x, strides, dtype
        _c_ptr,  # seq_idx
        _c_ptr, _c_i64, _c_i64,  # dout, strides
        _c_ptr, _c_ptr,  # dfinal_states, dx
        _c_i64, _c_i64, _c_i64, _c_i64,  # batch, seqlen, dim, width
    ]
    lib.ccv1d_bwd.restype = _c_int
    lib.ccv1d_bwd.argtypes = [
        _c_ptr, _c_i64, _c_i64, _c_int,  # x
        _c_ptr, _c_int,  # weight
        _c_ptr, _c_int,  # bias
        _c_ptr,  # seq_idx
        _c_ptr, _c_int,  # initial_states
        _c_ptr, _c_i64, _c_i64,  # dout, strides
        _c_ptr,  # dfinal_states
        _c_ptr, _c_ptr, _c_ptr, _c_ptr,  # dx, dinitial_states, dweight, dbias
        _c_ptr, ctypes.c_size_t,  # workspace, bytes
        _c_i64, _c_i64, _c_i64, _c_i64,  # batch, seqlen, dim, width
        _c_int, _c_int, _c_ptr,  # silu, device, stream
    ]
    lib.ccv1d_bwd_dx_strided.argtypes = (lib.ccv1d_bwd.argtypes[:16]   # x .. dx
                                         + [_c_i64, _c_i64]             # dx strides
                                         + lib.ccv1d_bwd.argtypes[16:])  # dinit .. stream
    lib.ccv1d_bwd_noalloc.restype = _c_int
    lib.ccv1d_bwd_noalloc.argtypes = (lib.ccv1d_bwd.argtypes[:19]   # x .. dbias, as ccv1d_bwd
                                      + lib.ccv1d_bwd.argtypes[21:])  # batch .. stream
    _lib = lib
    return lib


def _code(t: torch.Tensor) -> int:
    try:
        return DTYPE_CODES[t.dtype]
    except KeyError:
        raise TypeError(f"unsupported dtype {t.dtype}") from None


def _ptr(t):
    return None if t is None else t.data_ptr()


def _check(rc: int, lib) -> None:
    if rc != 0:
        raise CCV1DError(f"libccv1d error {rc}: {lib.ccv1d_last_error().decode()}")


# torch's current stream on a device, as a raw hipStream_t. The private getter returns the handle
# without building a torch.cuda.Stream object (0.07 us per call against 1.8 us for
# torch.cuda.current_stream(device).cuda_stream on MI355X hosts); the public route is kept for
# torch builds without it.
_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def _stream(index: int) -> int:
    if _raw_stream is not None:
        return _raw_stream(index)
    return torch.cuda.current_stream(index).cuda_stream


def fwd(x, weight, bias, seq_idx, initial_states, out, final_states, silu: bool,
        inference: bool = False) -> None:
    """ccv1d_fwd, or with `inference` ccv1d_fwd_inference (the same kernels with the store policy
    of a forward that no backward follows)."""
    B, T, D = x.shape
    W = weight.shape[1]
    dev = x.get_device()
    args = (
        x.data_ptr(), x.stride(0), x.stride(1), _code(x),
        weight.data_ptr(), _code(weight),
        _ptr(bias), 0 if bias is None else _code(bias),
        _ptr(seq_idx),
        _ptr(initial_states), 0 if initial_states is None else _code(initial_states),
        out.data_ptr(), _ptr(final_states),
        B, T, D, W,
        int(silu), dev, _stream(dev),
    )
    if inference:
        rc = load().ccv1d_fwd_inference(*args)
    elif _native is not None:
        rc = _native.fwd(*args)
    else:
        rc = (_lib if _lib is not None else load()).ccv1d_fwd(*args)
    if rc:
        _check(rc, load())


def time_main_kernel(start, stop) -> None:
    """Asks the calling thread's next fwd or bwd call to time its main kernel with two
    torch.cuda.Event(enable_timing=True): afterwards start.elapsed_time(stop) is that kernel's own
    execution time (ccv1d_time_main_kernel in include/ccv1d.h). torch creates an event's HIP handle
    at its first record, so each event must have been recorded once before."""
    if not (start.cuda_event and stop.cuda_event):
        raise ValueError("record each event once before using it for kernel timing")
    lib = load()
    _check(lib.ccv1d_time_main_kernel(start.cuda_event, stop.cuda_event), lib)


def bwd_workspace_bytes(B: int, T: int, D: int, W: int, x_dtype: torch.dtype) -> int:
    """Upper bound of the backward's workspace over every path a shape can take."""
    return load().ccv1d_bwd_workspace_bytes(B, T, D, W, DTYPE_CODES.get(x_dtype, 0))


def bwd_workspace_bytes_for(x, seq_idx, dout, dfinal_states, dx, W: int) -> int:
    """Workspace of the path ccv1d_bwd takes for these tensors (dx contiguous)."""
    B, T, D = x.shape
    return load().ccv1d_bwd_workspace_bytes_for(
        x.data_ptr(), x.stride(0), x.stride(1), _code(x), _ptr(seq_idx),
        dout.data_ptr(), dout.stride(0), dout.stride(1), _ptr(dfinal_states), dx.data_ptr(),
        B, T, D, W)


def _bwd_args(x, weight, bias, seq_idx, initial_states, dout, dfinal_states, dx, dinit, dweight,
              dbias, silu):
    """Arguments of ccv1d_bwd before and after its (workspace, workspace_bytes) pair."""
    B, T, D = x.shape
    W = weight.shape[1]
    dev = x.get_device()
    if dout.dtype != x.dtype:
        raise TypeError(f"dout dtype {dout.dtype} differs from x dtype {x.dtype}")
    if dfinal_states is not None and dfinal_states.dtype != x.dtype:
        raise TypeError(f"dfinal_states dtype {dfinal_states.dtype} differs from x dtype {x.dtype}")
    head = (
        x.data_ptr(), x.stride(0), x.stride(1), _code(x),
        weight.data_ptr(), _code(weight),
        _ptr(bias), 0 if bias is None else _code(bias),
        _ptr(seq_idx),
        _ptr(initial_states), 0 if initial_states is None else _code(initial_states),
        dout.data_ptr(), dout.stride(0), dout.stride(1),
        _ptr(dfinal_states),
        dx.data_ptr(), _ptr(dinit), dweight.data_ptr(), _ptr(dbias),
    )
    return head, (B, T, D, W, int(silu), dev, _stream(dev))


def bwd_dx_strided(x, weight, bias, seq_idx, initial_states, dout, dfinal_states, dx, dinit,
                   dweight, dbias, workspace, silu: bool) -> None:
    """ccv1d_bwd_dx_strided through ctypes: the backward writing dx with dx's own strides."""
    head, tail = _bwd_args(x, weight, bias, seq_idx, initial_states, dout, dfinal_states, dx, dinit,
                           dweight, dbias, silu)
    # head ends with dx, dinit, dweight, dbias: dx's strides go right after dx
    args = (head[:16] + (dx.stride(0), dx.stride(1)) + head[16:]
            + (_ptr(workspace), 0 if workspace is None else workspace.numel()) + tail)
    lib = load()
    _check(lib.ccv1d_bwd_dx_strided(*args), lib)


def bwd_noalloc(x, weight, bias, seq_idx, initial_states, dout, dfinal_states, dx, dinit, dweight,
                dbias, silu: bool) -> None:
    """ccv1d_bwd_noalloc through ctypes: the backward with the library's built-in scratch instead
    of a workspace (for callers that cannot allocate)."""
    head, tail = _bwd_args(x, weight, bias, seq_idx, initial_states, dout, dfinal_states, dx, dinit,
                           dweight, dbias, silu)
    lib = load()
    _check(lib.ccv1d_bwd_noalloc(*head, *tail), lib)


def bwd(x, weight, bias, seq_idx, initial_states, dout, dfinal_states, dx, dinit, dweight, dbias,
        workspace, silu: bool) -> None:
    head, tail = _bwd_args(x, weight, bias, seq_idx, initial_states, dout, dfinal_states, dx, dinit,
                           dweight, dbias, silu)
    args = head + (_ptr(workspace), 0 if workspace is None else workspace.numel()) + tail
    if _native is not None:
        rc = _native.bwd(*args)
    else:
        rc = (_lib if _lib is not None else load()).ccv1d_bwd(*args)
    if rc:
        _check(rc, load())
