"""The C-ABI library without a GPU: it loads next to torch's HIP runtime, exports every entry point
include/ccv1d.h declares, and rejects invalid requests with the documented status codes before any
HIP call is made."""

import ctypes
import os
import re

import pytest

import torch  # noqa: F401  (the library binds to torch's HIP runtime)
from causal_conv1d_triton import _ffi

_HDR = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include",
                    "ccv1d.h")


def _header():
    with open(_HDR) as f:
        return f.read()


def _declared():
    return sorted(set(re.findall(r"^\s*(?:int|size_t|const char\*)\s+(ccv1d_\w+)\(", _header(),
                                 flags=re.M)))


def test_header_declares_the_entry_points():
    assert _declared() == ["ccv1d_abi_version", "ccv1d_bwd", "ccv1d_bwd_dx_strided",
                           "ccv1d_bwd_noalloc", "ccv1d_bwd_workspace_bytes",
                           "ccv1d_bwd_workspace_bytes_for", "ccv1d_fwd",
                           "ccv1d_fwd_inference", "ccv1d_last_error", "ccv1d_time_main_kernel"]


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(_ffi.library_path())
    for name in _declared():
        assert hasattr(lib, name), name


def test_abi_version_matches_header():
    v = int(re.search(r"#define CCV1D_ABI_VERSION (\d+)", _header()).group(1))
    assert _ffi.load().ccv1d_abi_version() == v


def test_workspace_bytes():
    lib = _ffi.load()
    assert lib.ccv1d_bwd_workspace_bytes(0, 10, 8, 4, 2) == 0
    assert lib.ccv1d_bwd_workspace_bytes(1, 0, 8, 4, 2) == 0
    assert lib.ccv1d_bwd_workspace_bytes(1, 10, 8, 1, 2) == 0
    n = lib.ccv1d_bwd_workspace_bytes(4, 8192, 1024, 4, 2)
    # never less than the generic kernel's one fp32 partial row of (width + 1) * dim floats per
    # 64-row tile
    assert n >= 4 * (8192 // 64) * 5 * 1024 * 4
    # whole fp32 partial rows of (width + 1) * dim floats
    assert n % (5 * 1024 * 4) == 0


def test_workspace_bytes_of_wide_widths():
    """Above width 128 the backward's workspace holds the partial rows (one per 64-row tile, W + 1
    rows of dim floats) and, 256-byte aligned after them, one fp32 g value per element."""
    lib = _ffi.load()
    for B, T, D, W in ((2, 300, 100, 129), (4, 8192, 1024, 200), (1, 1, 8, 257)):
        part = B * -(-T // 64) * (W + 1) * D * 4
        want = (part + 255) // 256 * 256 + B * T * D * 4
        assert lib.ccv1d_bwd_workspace_bytes(B, T, D, W, 2) == want


def _ws_for(lib, x=1 << 20, sxb=None, sxt=None, xdt=2, seq=None, dy=1 << 24, dfin=None,
            dx=1 << 28, B=4, T=8192, D=1024, W=4):
    sxt = D if sxt is None else sxt
    sxb = T * sxt if sxb is None else sxb
    return lib.ccv1d_bwd_workspace_bytes_for(x, sxb, sxt, xdt, seq, dy, sxb, sxt, dfin, dx, B, T, D,
                                             W)


def test_workspace_bytes_for_the_call():
    """The workspace of the path a call takes (its pointers' alignment and strides decide it): the
    vectorised backward's partial rows for aligned rows, the generic kernels' bound otherwise; never
    more than the shape-only upper bound. No pointer is dereferenced."""
    lib = _ffi.load()
    bound = lib.ccv1d_bwd_workspace_bytes(4, 8192, 1024, 4, 2)
    fast = _ws_for(lib)
    # the benchmark shape: 4 batch rows x 32 workgroups along time, (W + 1) x dim fp32 each
    assert fast == 4 * 32 * 5 * 1024 * 4
    assert fast < bound
    # x misaligned by one element: the generic kernels, one partial row per 64-row tile
    assert _ws_for(lib, x=(1 << 20) + 2) == 4 * (8192 // 64) * 5 * 1024 * 4 <= bound
    # a time stride that is not a multiple of the channel vector: generic as well
    assert _ws_for(lib, sxt=1027, sxb=8192 * 1027) == 4 * 128 * 5 * 1024 * 4
    # width above 128: partial rows plus the fp32 g buffer, as the shape-only bound says
    assert _ws_for(lib, B=2, T=300, D=100, W=129) == lib.ccv1d_bwd_workspace_bytes(2, 300, 100, 129, 2)
    # empty and invalid shapes
    assert _ws_for(lib, B=0) == 0 and _ws_for(lib, T=0) == 0 and _ws_for(lib, W=1) == 0
    assert _ws_for(lib, xdt=9) == 0
    # random shapes: never above the bound
    import random
    rnd = random.Random(0)
    for _ in range(200):
        B, T, D, W = rnd.randint(1, 8), rnd.randint(1, 5000), rnd.randint(1, 3000), rnd.randint(2, 40)
        xdt = rnd.choice([0, 1, 2, 3])
        n = _ws_for(lib, B=B, T=T, D=D, W=W, xdt=xdt, x=(1 << 20) + rnd.choice([0, 2, 16]),
                    seq=rnd.choice([None, 1 << 30]))
        assert 0 < n <= lib.ccv1d_bwd_workspace_bytes(B, T, D, W, xdt), (B, T, D, W, xdt)


def test_small_grid_backward_tiles():
    """The vectorised backward writes one partial row ((W + 1) x dim fp32) per batch row and
    workgroup of 8 tiles along time, so its workspace shows the tiling. At B=4 D=1024 the 4-channel
    grid is small and the backward takes 2 channels per lane: at T=2048 W=4 its 32-row tiles leave
    256 workgroups, and 16-bit x halves them to 16 rows (16 workgroups along time per batch row)
    while fp32 x keeps 32 (8), as does 16-bit x from width 6; at T=512 the tiles shrink to 8 rows
    for fewer than 256 workgroups, whatever the dtype."""
    lib = _ffi.load()
    row = 5 * 1024 * 4
    assert _ws_for(lib, T=2048, xdt=2) == 4 * 16 * row   # bf16
    assert _ws_for(lib, T=2048, xdt=1) == 4 * 16 * row   # fp16
    assert _ws_for(lib, T=2048, xdt=0) == 4 * 8 * row    # fp32
    assert _ws_for(lib, T=2048, W=8) == 4 * 8 * 9 * 1024 * 4
    assert _ws_for(lib, T=512, xdt=2) == 4 * 8 * row
    assert _ws_for(lib, T=512, xdt=0) == 4 * 8 * row
    # never above the shape-only bound the default backward allocates
    for xdt in (0, 1, 2):
        assert _ws_for(lib, T=2048, xdt=xdt) <= lib.ccv1d_bwd_workspace_bytes(4, 2048, 1024, 4, xdt)


def _fwd(lib, **kw):
    a = dict(x=1 << 20, sxb=0, sxt=8, xdt=2, w=1 << 21, wdt=0, b=None, bdt=0, seq=None, init=None,
             idt=0, out=1 << 22, fin=None, B=1, T=4, D=8, W=4, silu=1, dev=0, stream=None)
    a.update(kw)
    return lib.ccv1d_fwd(a["x"], a["sxb"], a["sxt"], a["xdt"], a["w"], a["wdt"], a["b"], a["bdt"],
                         a["seq"], a["init"], a["idt"], a["out"], a["fin"], a["B"], a["T"], a["D"],
                         a["W"], a["silu"], a["dev"], a["stream"])


@pytest.mark.parametrize("kw,msg", [
    (dict(W=1), "width"),
    (dict(B=-1), "negative"),
    (dict(xdt=7), "dtype"),
    (dict(x=None), "x is null"),
    (dict(w=None), "weight is null"),
    (dict(out=None), "out is null"),
    (dict(seq=1 << 23, fin=1 << 24), "final states"),
    (dict(T=1 << 28, D=16, sxt=16), "2^31"),
    (dict(out=1 << 20), "overlap"),                # an in-place forward
    (dict(out=(1 << 20) + 2 * 8 * 3), "overlap"),  # out starts at x's last row
])
def test_fwd_rejects_invalid_arguments(kw, msg):
    lib = _ffi.load()
    assert _fwd(lib, **kw) == 1
    assert msg in lib.ccv1d_last_error().decode()


def test_fwd_empty_batch_is_a_no_op():
    lib = _ffi.load()
    assert _fwd(lib, B=0, x=None, out=None) == 0
    assert lib.ccv1d_last_error().decode() == ""


def _bwd(lib, **kw):
    a = dict(x=1 << 20, xdt=2, w=1 << 21, b=None, init=None, dy=1 << 22, dfin=None, dx=1 << 23,
             dinit=None, dw=1 << 24, db=None, ws=None, wsb=0, B=1, T=4, D=8, W=4, seq=None)
    a.update(kw)
    return lib.ccv1d_bwd(a["x"], 0, 8, a["xdt"], a["w"], 0, a["b"], 0, a["seq"], a["init"], 0,
                         a["dy"], 0, 8, a["dfin"], a["dx"], a["dinit"], a["dw"], a["db"], a["ws"],
                         a["wsb"], a["B"], a["T"], a["D"], a["W"], 1, 0, None)


@pytest.mark.parametrize("kw,code,msg", [
    (dict(db=1 << 25), 1, "dbias"),
    (dict(b=1 << 25), 1, "dbias"),
    (dict(dinit=1 << 25), 1, "initial_states"),
    (dict(dy=None), 1, "dout or dx"),
    (dict(dw=None), 1, "dweight"),
    (dict(seq=1 << 25, dfin=1 << 26), 1, "seq_idx"),
    (dict(ws=None, wsb=0), 3, "workspace"),
    (dict(ws=1 << 27, wsb=16), 3, "workspace"),
    # widths above 128 also keep g in the workspace: one partial row is not enough
    (dict(W=200, ws=1 << 27, wsb=201 * 8 * 4), 3, "workspace"),
])
def test_bwd_rejects_invalid_arguments(kw, code, msg):
    # every case fails validation, so no HIP call is reached
    lib = _ffi.load()
    assert _bwd(lib, **kw) == code
    assert msg in lib.ccv1d_last_error().decode()


def _bwd_noalloc(lib, **kw):
    # stand-in addresses (never dereferenced) far enough apart for the largest shape below
    a = dict(x=1 << 36, xdt=2, w=1 << 21, b=None, init=None, dy=1 << 38, dfin=None, dx=1 << 40,
             dinit=None, dw=1 << 24, db=None, B=1, T=4, D=8, W=4, seq=None)
    a.update(kw)
    return lib.ccv1d_bwd_noalloc(a["x"], 0, 8 if a["D"] == 8 else a["D"], a["xdt"], a["w"], 0,
                                 a["b"], 0, a["seq"], a["init"], 0, a["dy"], 0,
                                 8 if a["D"] == 8 else a["D"], a["dfin"], a["dx"], a["dinit"],
                                 a["dw"], a["db"], a["B"], a["T"], a["D"], a["W"], 1, 0, None)


def _noalloc_limit():
    m = re.search(r"#define CCV1D_NOALLOC_SCRATCH_BYTES \((\d+)u << (\d+)\)", _header())
    return int(m.group(1)) << int(m.group(2))


@pytest.mark.parametrize("kw,code,msg", [
    (dict(db=1 << 25), 1, "dbias"),
    (dict(dinit=1 << 25), 1, "initial_states"),
    (dict(dy=None), 1, "dout or dx"),
    (dict(W=1), 1, "width"),
    # partial sums beyond the built-in scratch: B * (T / 64 rows) partial rows of 5 * D floats
    (dict(B=64, T=65536, D=4096), 3, "scratch"),
])
def test_bwd_noalloc_rejects_before_any_hip_call(kw, code, msg):
    """The allocation-free backward validates and sizes the request before it touches a device
    (here there is none): bad arguments and shapes whose partial sums exceed its scratch are
    refused with the documented codes."""
    lib = _ffi.load()
    assert _bwd_noalloc(lib, **kw) == code
    assert msg in lib.ccv1d_last_error().decode()


def test_bwd_noalloc_limit_matches_workspace_sizing():
    """The scratch limit of the header bounds the shapes the allocation-free backward accepts: the
    benchmark shape fits, and the refused shape above needs more than the limit."""
    lib = _ffi.load()
    limit = _noalloc_limit()
    assert limit == 32 << 20
    assert lib.ccv1d_bwd_workspace_bytes(4, 8192, 1024, 4, 2) <= limit
    assert lib.ccv1d_bwd_workspace_bytes(64, 65536, 4096, 4, 2) > limit


def _bwd_strided(lib, dxsb, dxst, **kw):
    a = dict(x=1 << 20, w=1 << 21, dy=1 << 22, dx=1 << 23, dw=1 << 24, B=2, T=4, D=8, W=4)
    a.update(kw)
    return lib.ccv1d_bwd_dx_strided(a["x"], 32, 8, 2, a["w"], 0, None, 0, None, None, 0, a["dy"],
                                    32, 8, None, a["dx"], dxsb, dxst, None, a["dw"], None, None, 0,
                                    a["B"], a["T"], a["D"], a["W"], 1, 0, None)


@pytest.mark.parametrize("dxsb,dxst,msg", [
    (32, 4, "overlap"),     # time stride below dim: rows overlap
    (16, 8, "overlap"),     # batch stride below (T - 1) * stride + dim
    (-1, 8, "negative"),
    (1 << 40, 1 << 28, "2^31"),
])
def test_bwd_dx_strided_rejects_overlapping_or_huge_strides(dxsb, dxst, msg):
    """Strides of dx that would make rows overlap, or in-batch offsets beyond 32 bits, are
    refused before any HIP call."""
    lib = _ffi.load()
    assert _bwd_strided(lib, dxsb, dxst) == 1
    assert msg in lib.ccv1d_last_error().decode()


@pytest.mark.parametrize("dx,dxsb,dxst", [
    (1 << 20, 32, 8),             # dx = x: an in-place update
    (1 << 22, 32, 8),             # dx = dout
    ((1 << 20) + 2 * 31, 32, 8),  # dx starts at x's last element
    ((1 << 22) - 2 * 3, 32, 8),   # dx's last row reaches into dout's first
])
def test_bwd_rejects_dx_overlapping_inputs(dx, dxsb, dxst):
    """dx is written while other tiles still read x and dout: address ranges that meet are
    refused before any HIP call (bf16: 2 bytes per element; x and dout span 32 elements)."""
    lib = _ffi.load()
    assert _bwd_strided(lib, dxsb, dxst, dx=dx) == 1
    assert "overlap x or dout" in lib.ccv1d_last_error().decode()
    assert _bwd(lib, dx=1 << 20) == 1
    assert "overlap x or dout" in lib.ccv1d_last_error().decode()


def test_timing_request_needs_both_events_or_neither():
    lib = _ffi.load()
    assert lib.ccv1d_time_main_kernel(1 << 20, None) == 1
    assert "both timing events" in lib.ccv1d_last_error().decode()
    assert lib.ccv1d_time_main_kernel(None, 1 << 20) == 1
    assert lib.ccv1d_time_main_kernel(None, None) == 0
    assert lib.ccv1d_last_error().decode() == ""
    # A request (here with stand-in handles that must never reach HIP) is taken by the next call,
    # which fails validation and so launches nothing; the cancel after it leaves nothing pending.
    assert lib.ccv1d_time_main_kernel(1 << 20, 1 << 21) == 0
    assert _fwd(lib, W=1) == 1
    assert lib.ccv1d_time_main_kernel(None, None) == 0


def test_timing_helper_needs_created_events():
    class Unrecorded:
        cuda_event = 0
    with pytest.raises(ValueError, match="record each event"):
        _ffi.time_main_kernel(Unrecorded(), Unrecorded())


# The package's CPython binding of the two launch entry points (csrc/ccv1d_pyext.c): same C
# functions, same arguments, same status codes, and one library instance shared with ctypes (so
# ccv1d_last_error reads the error of a call made through either).

def _native():
    assert _ffi._native is not None, "the CPython binding is built with the library (make)"
    return _ffi._native


def test_native_binding_matches_the_library():
    nat = _native()
    assert nat.abi_version() == _ffi.load().ccv1d_abi_version()
    libs = {line.split()[-1] for line in open("/proc/self/maps") if "libccv1d" in line}
    assert libs == {os.path.realpath(_ffi.library_path())}


@pytest.mark.parametrize("kw,msg", [
    (dict(W=1), "width"),
    (dict(xdt=7), "dtype"),
    (dict(out=None), "out is null"),
    (dict(seq=1 << 23, fin=1 << 24), "final states"),
])
def test_native_fwd_rejects_invalid_arguments(kw, msg):
    lib = _ffi.load()
    assert _fwd(_NativeAsLib(), **kw) == 1
    assert msg in lib.ccv1d_last_error().decode()


@pytest.mark.parametrize("kw,code,msg", [
    (dict(db=1 << 25), 1, "dbias"),
    (dict(ws=None, wsb=0), 3, "workspace"),
    (dict(W=200, ws=1 << 27, wsb=201 * 8 * 4), 3, "workspace"),
])
def test_native_bwd_rejects_invalid_arguments(kw, code, msg):
    lib = _ffi.load()
    assert _bwd(_NativeAsLib(), **kw) == code
    assert msg in lib.ccv1d_last_error().decode()


def test_native_binding_checks_its_arguments():
    nat = _native()
    with pytest.raises(TypeError):
        nat.fwd(1, 2, 3)
    with pytest.raises(TypeError):
        nat.bwd()
    args = [1 << 20, 0, 8, 2, 1 << 21, 0, None, 0, None, None, 0, 1 << 22, None, 1, 4, 8, 4, 1, 0,
            None]
    with pytest.raises(TypeError):
        nat.fwd(*(args[:3] + ["2"] + args[4:]))
    with pytest.raises(OverflowError):
        nat.fwd(*(args[:3] + [1 << 40] + args[4:]))


class _NativeAsLib:
    """Exposes the CPython binding under the C names, for the argument builders above."""

    def ccv1d_fwd(self, *a):
        return _native().fwd(*a)

    def ccv1d_bwd(self, *a):
        return _native().bwd(*a)
