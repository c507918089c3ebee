"""GPU parity: the HIP kernels (through causal_conv1d_fn -> libccv1d.so) against the C oracle on
identical seeded inputs, plus the invariants that must hold bit for bit.

Tolerances (from the build's north star):
  * bf16/fp16 out, dx, dinit: |gpu - ref| <= 1e-2 + 1e-2 |ref|, ref = the oracle's fp32 value. The
    kernels evaluate every output in the oracle's operation order, so without an activation the
    results are also required to be bit-identical to the oracle rounded to the output dtype, and
    with silu all but 1% of them, plus one, must be (the exp/reciprocal implementations and the
    place of the bias in the sum differ by fp32 ulps, which flips about 1e-4 of the roundings; the
    one extra value keeps a sample of a few values from failing on a single flip).
  * fp32 out, dx, dinit: |gpu - ref| <= 1e-5 + 1e-5 |ref|.
  * dweight, dbias (fp32): |gpu - ref| <= 1e-3 |ref| + 1e-5 rms(ref), ref summed in double. The
    absolute term covers entries near zero, where the rounding of any fp32 accumulation over the
    rows (here and in the reference alike) is not small relative to the entry itself; over this
    suite the largest deviation is 2.6e-6 rms(ref), and 1e-5 |ref| on entries above 0.1 rms(ref).
    In a bf16/fp16 parameter dtype the result is rounded, so rtol 1e-2 replaces 1e-3.
  * Bit-exact: padding positions give out == 0 and dx == 0, final_states == the last width-1 rows
    of concat(initial_states, x), chunked forward == full forward, repeated backward gives the same
    dweight/dbias bits.
BASELINE configurations 2-5 run at full size; the oracle (single-threaded C) checks a subset of
channels there, which is exact because channels never interact in a depthwise convolution.
"""

import math
import os

import numpy as np
import pytest
import torch

import ccv1d_oracle as oracle
from causal_conv1d_triton import causal_conv1d_fn

pytestmark = pytest.mark.gpu

DEV = "cuda"


def _gen(seed):
    return torch.Generator().manual_seed(seed)


def make_inputs(seed, B, T, D, W, xdt=torch.bfloat16, wdt=torch.float32, bias=True, init=False,
                idt=None, seq=None, wdist="normal"):
    g = _gen(seed)
    inp = {"B": B, "T": T, "D": D, "W": W}
    inp["x"] = torch.randn(B, T, D, generator=g).to(xdt)
    if wdist == "uniform":
        inp["w"] = (torch.rand(D, W, generator=g) - 0.5).to(wdt)
        inp["b"] = ((torch.rand(D, generator=g) - 0.5) * 0.2).to(wdt) if bias else None
    else:
        inp["w"] = (torch.randn(D, W, generator=g) / math.sqrt(W)).to(wdt)
        inp["b"] = torch.randn(D, generator=g).to(wdt) if bias else None
    inp["init"] = torch.randn(B, W - 1, D, generator=g).to(idt or xdt) if init else None
    inp["dy"] = torch.randn(B, T, D, generator=g).to(xdt)
    inp["dfinal"] = torch.randn(B, W - 1, D, generator=g).to(xdt)
    inp["seq"] = seq
    return inp


def varlen_seq(seed, B, T, lo=64, hi=4096, pad_frac=0.05):
    """Consecutive segments with lengths ~U[lo, hi] and ids 0, 1, 2, ...; last pad_frac is -1."""
    g = _gen(seed)
    s = torch.empty(B, T, dtype=torch.int32)
    for b in range(B):
        t, sid = 0, 0
        while t < T:
            n = int(torch.randint(lo, hi + 1, (1,), generator=g))
            s[b, t:t + n] = sid
            t += n
            sid += 1
        s[b, T - int(pad_frac * T):] = -1
    return s


def _np32(t):
    return None if t is None else t.float().numpy()


def _sub(t, cols, dim=-1):
    return None if t is None else t.index_select(dim, cols)


def oracle_ref(inp, silu, cols=None, final=False, dfinal=False, need_dinit=False, bwd=True):
    """Oracle outputs (fp32 numpy; dweight/dbias float64) for all channels or the subset `cols`."""
    x, w, b, init, dy, df = inp["x"], inp["w"], inp["b"], inp["init"], inp["dy"], inp["dfinal"]
    if cols is not None:
        x, dy = _sub(x, cols), _sub(dy, cols)
        init, df = _sub(init, cols), _sub(df, cols)
        w, b = _sub(w, cols, 0), _sub(b, cols, 0)
    seq = None if inp["seq"] is None else inp["seq"].numpy()
    r = {}
    r["out"], r["final"] = oracle.fwd(_np32(x), _np32(w), _np32(b), seq, _np32(init), silu=silu,
                                      final=final)
    if bwd:
        r["dx"], r["dinit"], r["dw"], r["db"] = oracle.bwd(
            _np32(x), _np32(w), _np32(dy), _np32(b), seq, _np32(init),
            _np32(df) if dfinal else None, need_dinit=need_dinit, silu=silu)
    return r


def run_gpu(inp, activation, return_final=False, dfinal=False, init_grad=False, bwd=True,
            x_override=None):
    x = (x_override if x_override is not None else inp["x"].to(DEV)).detach().requires_grad_(bwd)
    w = inp["w"].to(DEV).requires_grad_(bwd)
    b = inp["b"].to(DEV).requires_grad_(bwd) if inp["b"] is not None else None
    init = inp["init"].to(DEV).requires_grad_(init_grad) if inp["init"] is not None else None
    seq = inp["seq"].to(DEV) if inp["seq"] is not None else None
    res = causal_conv1d_fn(x, w, b, seq_idx=seq, initial_states=init,
                           return_final_states=return_final, activation=activation)
    out, fin = res if return_final else (res, None)
    r = {"out": out.detach().cpu(), "final": None if fin is None else fin.detach().cpu()}
    if bwd:
        loss = (out.float() * inp["dy"].to(DEV).float()).sum()
        if return_final and dfinal:
            loss = loss + (fin.float() * inp["dfinal"].to(DEV).float()).sum()
        loss.backward()
        r["dx"] = x.grad.cpu()
        r["dw"] = w.grad.cpu()
        r["db"] = None if b is None else b.grad.cpu()
        r["dinit"] = None if init is None or not init_grad else init.grad.cpu()
    torch.cuda.synchronize()
    return r


def check_lowp(gpu, ref32, exact, what):
    """bf16/fp16/fp32 values vs the oracle's fp32 values (see the module docstring)."""
    ref = torch.from_numpy(np.ascontiguousarray(ref32))
    if gpu.dtype == torch.float32:
        torch.testing.assert_close(gpu, ref, rtol=1e-5, atol=1e-5, msg=what)
        return
    if gpu.dtype == torch.float64:
        torch.testing.assert_close(gpu, ref.double(), rtol=1e-5, atol=1e-5, msg=what)
        return
    torch.testing.assert_close(gpu.float(), ref, rtol=1e-2, atol=1e-2, msg=what)
    same = (gpu == ref.to(gpu.dtype)) | (gpu.isnan() & ref.to(gpu.dtype).isnan())
    differ = same.numel() - int(same.sum())
    if exact:
        assert differ == 0, f"{what}: {differ} of {same.numel()} values differ from the oracle's rounding"
    else:
        assert differ <= 0.01 * same.numel() + 1, \
            f"{what}: {differ} of {same.numel()} values differ from the oracle's rounding"


def check_sum(gpu, ref64, what):
    ref = torch.from_numpy(np.ascontiguousarray(ref64))
    tol = 1e-3 if gpu.dtype in (torch.float32, torch.float64) else 1e-2
    rms = ref.pow(2).mean().sqrt().item() if ref.numel() else 0.0
    torch.testing.assert_close(gpu.double(), ref, rtol=tol, atol=1e-5 * rms + 1e-7, msg=what)


def compare(gpu, ref, silu, cols=None):
    pick = (lambda t: t) if cols is None else (lambda t: None if t is None else _sub(t, cols))
    exact = not silu
    check_lowp(pick(gpu["out"]), ref["out"], exact, "out")
    if gpu.get("final") is not None and ref.get("final") is not None:
        # final states are rows of cat(initial_states, x) stored in x's dtype: rows taken from
        # initial states of another dtype are rounded on the way (causal_conv1d.py:156-164)
        fin = pick(gpu["final"])
        assert torch.equal(fin, torch.from_numpy(ref["final"]).to(fin.dtype)), "final"
    if "dx" in gpu and "dx" in ref:
        check_lowp(pick(gpu["dx"]), ref["dx"], exact, "dx")
        w_sub = gpu["dw"] if cols is None else _sub(gpu["dw"], cols, 0)
        check_sum(w_sub, ref["dw"], "dweight")
        if gpu["db"] is not None:
            b_sub = gpu["db"] if cols is None else _sub(gpu["db"], cols, 0)
            check_sum(b_sub, ref["db"], "dbias")
        if gpu.get("dinit") is not None:
            check_lowp(pick(gpu["dinit"]), ref["dinit"], exact, "dinit")


def test_native_library_is_loaded():
    inp = make_inputs(0, 1, 16, 64, 4)
    run_gpu(inp, "silu")
    with open("/proc/self/maps") as f:
        maps = f.read()
    assert "libccv1d.so" in maps


def test_readme_example():
    """x (2,1024,512) bf16 ~N(0,1), weight (512,4) fp32 ~N(0,1), bias (512)
    fp32 ~N(0,1), silu, out.sum().backward(); seed 0."""
    g = _gen(0)
    x = torch.randn(2, 1024, 512, generator=g).to(torch.bfloat16)
    w = torch.randn(512, 4, generator=g)
    b = torch.randn(512, generator=g)
    inp = {"x": x, "w": w, "b": b, "init": None, "seq": None, "dfinal": None,
           "dy": torch.ones(2, 1024, 512, dtype=torch.bfloat16)}
    gpu = run_gpu(inp, "silu")
    compare(gpu, oracle_ref(inp, True), True)


@pytest.mark.parametrize("W", [2, 3, 4, 5, 6, 7, 8, 9, 10, 12, 15, 16, 17, 20, 24, 25, 31, 32])
@pytest.mark.parametrize("act", [None, "silu"])
def test_widths_and_lengths(W, act):
    """Widths of the register-window kernels (2-32; one channel per lane from 17), at lengths around
    the window (T = P - 1, P, P + 1) and beyond, with state handoff both ways."""
    P = W - 1
    for T in sorted({1, max(1, P - 1), P, P + 1, 17, 1000}):
        for D in (8, 1024):
            inp = make_inputs(1000 * W + T + D, 2, T, D, W, bias=act is not None, init=T % 2 == 1)
            gpu = run_gpu(inp, act, return_final=True, dfinal=True, init_grad=True)
            ref = oracle_ref(inp, act is not None, final=True, dfinal=True,
                             need_dinit=inp["init"] is not None)
            compare(gpu, ref, act is not None)


@pytest.mark.parametrize("D", [1, 7, 1000, 5376])
def test_channel_counts(D):
    inp = make_inputs(D, 2, 300, D, 4, init=True)
    gpu = run_gpu(inp, "silu", return_final=True, dfinal=True, init_grad=True)
    compare(gpu, oracle_ref(inp, True, final=True, dfinal=True, need_dinit=True), True)


@pytest.mark.parametrize("W", [6, 8])
@pytest.mark.parametrize("D", [1002, 260])
@pytest.mark.parametrize("xdt", [torch.bfloat16, torch.float32])
def test_wide_widths_channel_counts(W, D, xdt):
    """Widths from 6 keep 2 channels per lane in the backward: D = 1002 (not a multiple of 4, so
    the forward takes the generic kernel while the backward stays vectorised) and D = 260 (a last
    wave column that is mostly empty)."""
    inp = make_inputs(W * 10 + D, 3, 333, D, W, xdt=xdt, init=True)
    gpu = run_gpu(inp, "silu", return_final=True, dfinal=True, init_grad=True)
    compare(gpu, oracle_ref(inp, True, final=True, dfinal=True, need_dinit=True), True)


@pytest.mark.parametrize("xdt", [torch.float32, torch.float16, torch.bfloat16, torch.float64])
@pytest.mark.parametrize("wdt", [torch.float32, torch.bfloat16, torch.float16])
def test_dtypes(xdt, wdt):
    """Every x dtype against every weight/bias dtype, with initial states in a third dtype (fp32
    for fp32 weights, the other 16-bit type for 16-bit weights), so the conversions on load and
    the stores of dweight, dbias and the initial-state gradient in their own dtype all run; widths
    4 (vectorised kernels and, with a dim that is not a multiple of 4, the generic ones), 12 and 20
    (one channel per lane). Without the activation out, dx and dinit must be bit-identical to the
    oracle's fp32 values rounded once to their dtype."""
    idt = {torch.float32: torch.float32, torch.bfloat16: torch.float16,
           torch.float16: torch.bfloat16}[wdt]
    for W, D in ((4, 256), (4, 250), (12, 250), (20, 250)):
        for act in ("silu", None):
            inp = make_inputs(7 + W, 2, 257, D, W, xdt=xdt, wdt=wdt, init=True, idt=idt)
            gpu = run_gpu(inp, act, return_final=True, dfinal=True, init_grad=True)
            assert gpu["out"].dtype == xdt and gpu["dx"].dtype == xdt
            assert gpu["dw"].dtype == wdt and gpu["db"].dtype == wdt and gpu["dinit"].dtype == idt
            compare(gpu, oracle_ref(inp, act is not None, final=True, dfinal=True, need_dinit=True),
                    act is not None)


@pytest.mark.parametrize("layout", ["time_stride", "aligned_slice", "misaligned_slice"])
def test_strided_x_and_dout(layout):
    B, T, D, W = 2, 500, 256, 4
    inp = make_inputs(11, B, T, D, W, init=True)
    if layout == "time_stride":
        big = torch.zeros(B, 2 * T, D, dtype=torch.bfloat16)
        big[:, ::2] = inp["x"]
        xg = big.to(DEV)[:, ::2]
    else:
        off = 64 if layout == "aligned_slice" else 3
        big = torch.zeros(B, T, D + 72, dtype=torch.bfloat16)
        big[..., off:off + D] = inp["x"]
        xg = big.to(DEV)[..., off:off + D]
    assert xg.stride(-1) == 1 and not xg.is_contiguous()
    x = xg.detach().requires_grad_(True)
    w = inp["w"].to(DEV).requires_grad_(True)
    b = inp["b"].to(DEV).requires_grad_(True)
    init = inp["init"].to(DEV).requires_grad_(True)
    out = causal_conv1d_fn(x, w, b, initial_states=init, activation="silu")
    dyb = torch.zeros(B, 2 * T, D, dtype=torch.bfloat16, device=DEV)
    dyb[:, ::2] = inp["dy"].to(DEV)
    out.backward(dyb[:, ::2])
    gpu = {"out": out.detach().cpu(), "dx": x.grad.cpu(), "dw": w.grad.cpu(), "db": b.grad.cpu(),
           "dinit": init.grad.cpu()}
    compare(gpu, oracle_ref(inp, True, need_dinit=True), True)


@pytest.mark.parametrize("W", [2, 4, 7, 20, 32])
@pytest.mark.parametrize("init", [False, True])
def test_seq_idx(W, init):
    B, T, D = 3, 2000, 512
    seq = varlen_seq(W, B, T, lo=16, hi=400, pad_frac=0.05)
    seq[1, 100:140] = -7           # negative ids other than -1 are padding too
    seq[2, 300:350] = 0            # a later segment reusing an earlier id still connects
    inp = make_inputs(W + 10 * init, B, T, D, W, init=init, seq=seq)
    gpu = run_gpu(inp, "silu", init_grad=init)
    ref = oracle_ref(inp, True, need_dinit=init)
    compare(gpu, ref, True)
    pad = seq < 0
    assert torch.all(gpu["out"][pad] == 0) and torch.all(gpu["dx"][pad] == 0)


@pytest.mark.parametrize("W", [4, 7, 24])
def test_seq_idx_long_segments(W):
    """Long segments with few boundaries: most tiles lie inside one segment (and run the seq-free
    code), the others carry a boundary or padding; both kinds must match the oracle, and padding
    positions stay exactly zero."""
    B, T, D = 2, 4096, 512
    seq = varlen_seq(40 + W, B, T, lo=300, hi=1500, pad_frac=0.03)
    inp = make_inputs(50 + W, B, T, D, W, init=True, seq=seq)
    gpu = run_gpu(inp, "silu", init_grad=True)
    compare(gpu, oracle_ref(inp, True, need_dinit=True), True)
    pad = seq < 0
    assert torch.all(gpu["out"][pad] == 0) and torch.all(gpu["dx"][pad] == 0)


@pytest.mark.parametrize("W", [4, 7, 32])
def test_seq_idx_padding_runs(W):
    """Runs of padding long enough to hold whole tiles, which take the padding path (forward: zero
    stores; backward: g = 0, no dout reads): at the start of a row (with initial states, whose rows
    then belong to the padding), in the middle with id -3, and at the end with id -2 (rows past T
    count as id -1, so the tiles whose halo reaches T stay on the masked path); a run of
    alternating -1/-2 is not one run and stays masked. A non-finite x inside a padding run
    reaches dweight as NaN (0 * inf), as in the reference."""
    B, T, D = 3, 3000, 512
    seq = varlen_seq(60 + W, B, T, lo=100, hi=700, pad_frac=0.0)
    seq[0, :600] = -1
    seq[0, -300:] = -1
    seq[1, 1000:1800] = -3
    seq[1, -500:] = -2
    seq[2, 2000:2400] = torch.tensor([-1, -1, -1, -1, -1, -2, -2, -2, -2, -2]).repeat(40)
    inp = make_inputs(70 + W, B, T, D, W, init=True, seq=seq)
    gpu = run_gpu(inp, "silu", init_grad=True)
    compare(gpu, oracle_ref(inp, True, need_dinit=True), True)
    pad = seq < 0
    assert torch.all(gpu["out"][pad] == 0) and torch.all(gpu["dx"][pad] == 0)
    assert torch.all(gpu["dinit"][0] == 0)  # row 0 starts in padding: no gradient reaches init

    inp["x"][1, 1400, 7] = float("inf")  # inside the -3 run
    inp["x"][0, 100, 9] = float("nan")   # inside the leading run
    gpu = run_gpu(inp, "silu", init_grad=True)
    ref = oracle_ref(inp, True, need_dinit=True)
    assert torch.equal(gpu["dw"].isnan(), torch.from_numpy(ref["dw"]).isnan())
    assert gpu["dw"][7].isnan().any() and gpu["dw"][9].isnan().any()
    assert torch.all(gpu["out"][pad] == 0) and torch.all(gpu["dx"][pad] == 0)
    fin = ~gpu["dw"].isnan()
    check_sum(gpu["dw"][fin], ref["dw"][fin.numpy()], "dw outside the NaN channels")


@pytest.mark.parametrize("W", [4, 7])
def test_seq_idx_int64_and_all_equal(W):
    B, T, D = 2, 300, 128
    inp = make_inputs(3, B, T, D, W, init=True)
    base = run_gpu(inp, "silu", init_grad=True)
    inp_eq = dict(inp, seq=torch.full((B, T), 5, dtype=torch.int64))
    same = run_gpu(inp_eq, "silu", init_grad=True)
    assert torch.equal(base["out"], same["out"]) and torch.equal(base["dx"], same["dx"])
    assert torch.equal(base["dinit"], same["dinit"])


def test_state_handoff_bit_exact():
    B, T, D, W = 3, 1000, 512, 4
    inp = make_inputs(5, B, T, D, W, init=True)
    x = inp["x"].to(DEV)
    w, b, init = inp["w"].to(DEV), inp["b"].to(DEV), inp["init"].to(DEV)
    with torch.no_grad():
        full, fin = causal_conv1d_fn(x, w, b, initial_states=init, return_final_states=True,
                                     activation="silu")
        xx = torch.cat([init, x], dim=1)
        assert torch.equal(fin, xx[:, T:])
        state, outs = init, []
        for lo, hi in ((0, 1), (1, 3), (3, 400), (400, 999), (999, 1000)):
            o, state = causal_conv1d_fn(x[:, lo:hi], w, b, initial_states=state,
                                        return_final_states=True, activation="silu")
            outs.append(o)
        assert torch.equal(torch.cat(outs, dim=1), full)
        assert torch.equal(state, fin)
        buf = torch.empty_like(fin)
        o2, f2 = causal_conv1d_fn(x, w, b, initial_states=init, return_final_states=True,
                                  final_states_out=buf, activation="swish")
        assert f2 is buf and torch.equal(buf, fin) and torch.equal(o2, full)


@pytest.mark.parametrize("W", [2, 4, 8])
@pytest.mark.parametrize("idt", [None, torch.bfloat16, torch.float32])
def test_final_states_from_either_tile_walk(W, idt):
    """final_states are written from the registers of the tile that ends at T, which walks forward
    in time (even tiles) or backward (odd tiles). At D=1024 these lengths end on an even and on an
    odd tile for each tile length the forward uses (8, 16, 32 and 64 rows), with no initial
    states, bf16 ones and fp32 ones. Bit-exact: final == cat(initial_states, x)[:, T:], and two
    chunks with the state handed over give the full pass."""
    P, D = W - 1, 1024
    g = torch.Generator(device=DEV).manual_seed(W)
    w = torch.randn(D, W, generator=g, device=DEV)
    for B, T in ((1, 16), (1, 24), (8, 904), (8, 920), (8, 4072), (2, 16392), (8, 8136),
                 (4, 16392)):
        x = torch.randn(B, T, D, generator=g, device=DEV).to(torch.bfloat16)
        init = None if idt is None else torch.randn(B, P, D, generator=g, device=DEV).to(idt)
        with torch.no_grad():
            out, fin = causal_conv1d_fn(x, w, initial_states=init, return_final_states=True,
                                        activation="silu")
            assert torch.equal(fin, x[:, T - P:]), (W, B, T)
            cut = T // 2 + 1
            o1, s1 = causal_conv1d_fn(x[:, :cut], w, initial_states=init, return_final_states=True,
                                      activation="silu")
            assert torch.equal(s1, x[:, cut - P:cut]), (W, B, T)
            o2, s2 = causal_conv1d_fn(x[:, cut:], w, initial_states=s1, return_final_states=True,
                                      activation="silu")
            assert torch.equal(s2, fin), (W, B, T)
            assert torch.equal(torch.cat([o1, o2], dim=1), out), (W, B, T)


def test_both_bindings_give_identical_results():
    """The CPython binding and the ctypes binding call the same C functions: identical outputs
    and gradients, bit for bit."""
    from causal_conv1d_triton import _ffi
    inp = make_inputs(21, 2, 300, 512, 4, init=True)
    native = _ffi._native
    assert native is not None
    try:
        a = run_gpu(inp, "silu", return_final=True, dfinal=True, init_grad=True)
        _ffi._native = None
        b = run_gpu(inp, "silu", return_final=True, dfinal=True, init_grad=True)
    finally:
        _ffi._native = native
    for k in a:
        if a[k] is not None:
            assert torch.equal(a[k], b[k]), k


@pytest.mark.parametrize("case", ["plain", "states", "seq", "fp32_no_bias", "strided_dout", "w20"])
def test_native_training_passes_match_python_path(case):
    """The autograd node's two passes go through the native calls of _ccv1d_torch (fwd_train,
    bwd: allocation and launch in one call); the same passes made from Python through the ctypes
    binding give identical outputs and gradients, bit for bit."""
    from causal_conv1d_triton import _ffi

    assert _ffi._torch_native is not None
    B, T, D, W = 3, 300, 256, 20 if case == "w20" else 4
    xdt = torch.float32 if case == "fp32_no_bias" else torch.bfloat16
    inp = make_inputs(91, B, T, D, W, xdt=xdt, bias=case != "fp32_no_bias",
                      init=case in ("states", "seq"),
                      seq=varlen_seq(10, B, T, lo=20, hi=90) if case == "seq" else None)
    final = case == "states"

    def run():
        x = inp["x"].to(DEV).requires_grad_(True)
        w = inp["w"].to(DEV).requires_grad_(True)
        b = None if inp["b"] is None else inp["b"].to(DEV).requires_grad_(True)
        init = None if inp["init"] is None else inp["init"].to(DEV).requires_grad_(True)
        seq = None if inp["seq"] is None else inp["seq"].to(DEV)
        res = causal_conv1d_fn(x, w, b, seq_idx=seq, initial_states=init,
                               return_final_states=final, activation="silu")
        out, fin = res if final else (res, None)
        dy = inp["dy"].to(DEV)
        if case == "strided_dout":
            big = torch.zeros(B, T, D + 8, dtype=dy.dtype, device=DEV)
            big[..., 4:4 + D] = dy
            dy = big[..., 4:4 + D]
        outs, grads_out = [out], [dy]
        if final:
            outs.append(fin)
            grads_out.append(inp["dfinal"].to(DEV))
        wrt = [t for t in (x, w, b, init) if t is not None]
        grads = torch.autograd.grad(outs, wrt, grads_out)
        return [out.detach()] + ([fin.detach()] if final else []) + list(grads)

    got = run()
    native, _ffi._native = _ffi._native, None
    torch_native, _ffi._torch_native = _ffi._torch_native, None
    try:
        want = run()
    finally:
        _ffi._native = native
        _ffi._torch_native = torch_native
    torch.cuda.synchronize()
    assert len(got) == len(want)
    for g, wnt in zip(got, want):
        assert g.dtype == wnt.dtype and torch.equal(g, wnt)


@pytest.mark.parametrize("W", [4, 12, 24])
@pytest.mark.parametrize("axis", ["time", "batch"])
def test_zero_stride_inputs_and_gradients(W, axis):
    """Expanded views (stride 0 along time or batch, unit channel stride) are read in place: x
    broadcast over one axis, and the gradient of out as autograd hands it over for a sum over that
    axis. Outputs and gradients equal those of the materialised copies bit for bit, through the
    native passes and through the ctypes path."""
    from causal_conv1d_triton import _ffi

    B, T, D = 3, 200, 96
    g = _gen(400 + W)
    shape = (B, 1, D) if axis == "time" else (1, T, D)
    x_small = torch.randn(*shape, generator=g).to(torch.bfloat16).to(DEV)
    r_small = torch.randn(*shape, generator=g).to(torch.bfloat16).to(DEV)
    w = (torch.randn(D, W, generator=g) / math.sqrt(W)).to(DEV)
    b = torch.randn(D, generator=g).to(DEV)
    x_exp = x_small.expand(B, T, D)
    dy_exp = r_small.expand(B, T, D)
    assert x_exp.stride(1 if axis == "time" else 0) == 0 and x_exp.stride(2) == 1
    assert dy_exp.stride(1 if axis == "time" else 0) == 0

    def run(x, dy):
        x = x.detach().requires_grad_(True)
        wr, br = w.detach().requires_grad_(True), b.detach().requires_grad_(True)
        out = causal_conv1d_fn(x, wr, br, activation="silu")
        grads = torch.autograd.grad(out, (x, wr, br), dy)
        return [out.detach()] + list(grads)

    want = run(x_exp.contiguous(), dy_exp.contiguous())
    got = run(x_exp, dy_exp)
    native, _ffi._native = _ffi._native, None
    torch_native, _ffi._torch_native = _ffi._torch_native, None
    try:
        got_py = run(x_exp, dy_exp)
    finally:
        _ffi._native = native
        _ffi._torch_native = torch_native
    torch.cuda.synchronize()
    for name, gv, pv, wv in zip(("out", "dx", "dweight", "dbias"), got, got_py, want):
        assert torch.equal(gv, wv), name
        assert torch.equal(pv, wv), name


def test_native_backward_refuses_foreign_gradients():
    """The native backward refuses a gradient of out on another device (a host address would
    reach a kernel) or of another dtype than x, before any launch."""
    from causal_conv1d_triton import causal_conv1d as cc

    inp = make_inputs(92, 2, 64, 128, 4)
    x, w, b = inp["x"].to(DEV), inp["w"].to(DEV), inp["b"].to(DEV)
    with pytest.raises(AssertionError, match="gradient of out must be on the device of x"):
        cc._bwd(x, w, b, None, None, inp["dy"], None, False, True)
    with pytest.raises(TypeError):
        cc._bwd(x, w, b, None, None, inp["dy"].to(DEV).float(), None, False, True)


@pytest.mark.parametrize("case", ["plain", "states", "seq_int64", "strided", "final_out",
                                  "generic", "empty"])
def test_native_inference_forward_matches_python_path(case):
    """Inference calls (no autograd) go through one native call (_ccv1d_torch: checks,
    canonicalisation, allocation, launch). The same call made from Python (the ctypes binding
    of the same C ABI) gives identical results, bit for bit."""
    from causal_conv1d_triton import _ffi
    from causal_conv1d_triton.causal_conv1d import _fwd

    assert _ffi._torch_native is not None
    B, T, D, W = 3, 257, 256, 4
    if case == "generic":
        W = 20
    if case == "empty":
        T = 0
    inp = make_inputs(90, B, T, D, W, init=case in ("states", "final_out", "empty"),
                      seq=varlen_seq(9, B, T, lo=20, hi=90) if case == "seq_int64" else None)
    x = inp["x"].to(DEV)
    if case == "strided":
        big = torch.zeros(B, T, D + 64, dtype=x.dtype, device=DEV)
        big[..., 32:32 + D] = x
        x = big[..., 32:32 + D]
    w, b = inp["w"].to(DEV), inp["b"].to(DEV)
    init = None if inp["init"] is None else inp["init"].to(DEV)
    seq = None if inp["seq"] is None else inp["seq"].to(DEV).long()
    final = seq is None
    buf = torch.empty(B, W - 1, D, dtype=x.dtype, device=DEV) if case == "final_out" else None
    with torch.no_grad():
        got = causal_conv1d_fn(x, w, b, seq_idx=seq, initial_states=init,
                               return_final_states=final, final_states_out=buf,
                               activation="silu")
        fin = torch.empty(B, W - 1, D, dtype=x.dtype, device=DEV) if final else None
        native, _ffi._native = _ffi._native, None
        torch_native, _ffi._torch_native = _ffi._torch_native, None
        try:
            want = _fwd(x, w, b, None if seq is None else seq.int(), init, fin, True)
        finally:
            _ffi._native = native
            _ffi._torch_native = torch_native
    torch.cuda.synchronize()
    if final:
        assert torch.equal(got[0], want) and torch.equal(got[1], fin)
        if buf is not None:
            assert got[1] is buf
    else:
        assert torch.equal(got, want)


@pytest.mark.parametrize("W,xdt", [(4, torch.bfloat16), (12, torch.bfloat16), (4, torch.float64)])
def test_kernel_timing_events(W, xdt):
    """ccv1d_time_main_kernel (fast and generic kernels): the timed launch gives bit-identical
    results, sets both events to a positive kernel time inside the interval of events recorded
    around the call, and covers one call only (an untimed call after it leaves the events as they
    were)."""
    from causal_conv1d_triton import _ffi

    B, T, D = 2, 700, 256
    inp = make_inputs(22, B, T, D, W, xdt=xdt)
    x, w, b, dy = (inp[k].to(DEV) for k in ("x", "w", "b", "dy"))
    ws = torch.empty(_ffi.bwd_workspace_bytes(B, T, D, W, xdt), dtype=torch.uint8, device=DEV)

    def fwd():
        out = torch.empty_like(x)
        _ffi.fwd(x, w, b, None, None, out, None, True)
        return out

    def bwd():
        dx, dw, db = torch.empty_like(x), torch.empty_like(w), torch.empty_like(b)
        _ffi.bwd(x, w, b, None, None, dy, None, dx, None, dw, db, ws, True)
        return dx, dw, db

    want_out, want_grads = fwd(), bwd()
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(6)]
    for e in ev:
        e.record()  # creates the HIP events
    ev[4].record()
    _ffi.time_main_kernel(ev[0], ev[1])
    out = fwd()
    ev[5].record()
    _ffi.time_main_kernel(ev[2], ev[3])
    grads = bwd()
    torch.cuda.synchronize()
    assert torch.equal(out, want_out)
    for got, want in zip(grads, want_grads):
        assert torch.equal(got, want)
    t_fwd, t_bwd = ev[0].elapsed_time(ev[1]), ev[2].elapsed_time(ev[3])
    assert 0 < t_fwd <= ev[4].elapsed_time(ev[5])
    assert 0 < t_bwd
    fwd()
    bwd()
    torch.cuda.synchronize()
    assert ev[0].elapsed_time(ev[1]) == t_fwd and ev[2].elapsed_time(ev[3]) == t_bwd


def _random_seq(g, B, T):
    """Segments of random lengths with ids that mostly increase, sometimes repeat an earlier id or
    go negative (padding runs with ids -1 or -2), so that tiles of every kind occur: inside one
    segment, across boundaries, inside one padding run, and across mixed padding."""
    s = torch.empty(B, T, dtype=torch.int32)
    for b in range(B):
        t, sid = 0, 0
        while t < T:
            n = int(torch.randint(1, max(2, T // 3), (1,), generator=g))
            u = float(torch.rand(1, generator=g))
            s[b, t:t + n] = -1 if u < 0.2 else (-2 if u < 0.25 else (max(sid - 1, 0) if u < 0.3
                                                                       else sid))
            t, sid = t + n, sid + 1
    return s


@pytest.mark.parametrize("case", range(96))
def test_random_cases(case):
    """Random shapes, widths, dtypes and options (bias, activation, initial states, seq_idx with
    padding runs, final states with their gradient) against the oracle."""
    g = _gen(1000 + case)
    pick = lambda opts: opts[int(torch.randint(0, len(opts), (1,), generator=g))]  # noqa: E731
    B = pick([1, 2, 3, 4])
    T = pick([1, 2, 5, 9, 17, 64, 100, 333, 700])
    D = pick([8, 64, 100, 256, 264, 1000, 1024])
    W = pick([2, 3, 4, 5, 6, 7, 8, 9, 11, 12, 13, 16, 17, 20, 24, 25, 32, 33])
    xdt = pick([torch.bfloat16, torch.bfloat16, torch.float16, torch.float32])
    wdt = pick([torch.float32, torch.float32, torch.bfloat16, torch.float16])
    idt = pick([None, torch.float32, torch.bfloat16, torch.float16])
    bias, silu, init = pick([True, False]), pick([True, False]), pick([True, False])
    seq = _random_seq(g, B, T) if pick([True, False]) else None
    final = seq is None and pick([True, False])
    inp = make_inputs(2000 + case, B, T, D, W, xdt=xdt, wdt=wdt, bias=bias, init=init, idt=idt,
                      seq=seq)
    act = "silu" if silu else None
    gpu = run_gpu(inp, act, return_final=final, dfinal=final, init_grad=init)
    ref = oracle_ref(inp, silu, final=final, dfinal=final, need_dinit=init)
    compare(gpu, ref, silu)
    if seq is not None:
        pad = seq < 0
        assert torch.all(gpu["out"][pad] == 0) and torch.all(gpu["dx"][pad] == 0), case


def test_deterministic_weight_grads():
    inp = make_inputs(9, 4, 4096, 1024, 4)
    a = run_gpu(inp, "silu")
    b = run_gpu(inp, "silu")
    assert torch.equal(a["dw"], b["dw"]) and torch.equal(a["db"], b["db"])
    assert torch.equal(a["dx"], b["dx"])


def test_init_without_grad_and_no_grad_inputs():
    inp = make_inputs(4, 2, 100, 64, 4, init=True)
    gpu = run_gpu(inp, "silu", init_grad=False)
    assert gpu["dinit"] is None
    compare(gpu, oracle_ref(inp, True), True)
    with torch.no_grad():
        out = causal_conv1d_fn(inp["x"].to(DEV), inp["w"].to(DEV), inp["b"].to(DEV),
                               initial_states=inp["init"].to(DEV), activation="silu")
    check_lowp(out.cpu(), oracle_ref(inp, True, bwd=False)["out"], False, "no-grad out")


@pytest.mark.parametrize("shape", [(2, 0, 64), (0, 10, 64), (2, 10, 0)])
def test_empty_inputs(shape):
    B, T, D = shape
    W = 4
    inp = make_inputs(1, B, T, D, W, init=True)
    x = inp["x"].to(DEV).requires_grad_(True)
    w = inp["w"].to(DEV).requires_grad_(True)
    b = inp["b"].to(DEV).requires_grad_(True)
    init = inp["init"].to(DEV).requires_grad_(True)
    out, fin = causal_conv1d_fn(x, w, b, initial_states=init, return_final_states=True,
                                activation="silu")
    assert out.shape == (B, T, D)
    assert torch.equal(fin, init.detach())  # with T == 0 the final states are the initial states
    dfin = inp["dfinal"].to(DEV)
    (out.float().sum() + (fin.float() * dfin.float()).sum()).backward()
    assert torch.equal(w.grad, torch.zeros_like(w)) and torch.equal(b.grad, torch.zeros_like(b))
    if T == 0:
        assert torch.equal(init.grad, dfin.to(init.dtype))


@pytest.mark.parametrize("W,xdt", [(3, torch.float16), (4, torch.bfloat16), (6, torch.bfloat16)])
def test_forward_channel_choices_agree(W, xdt):
    """The forward's channels per lane and tile length depend on the shape: (2, 8192, 2048) runs
    4 channels per lane on 32-row tiles, its first 1024 rows alone (a small grid) 2 channels, and
    16 copies of those rows 2 channels on the 16-row tiles the 4-channel tiling would take. Each
    output row depends only on rows up to it, so all three give the same first 1024 rows bit for
    bit (silu and bias included), and those match the oracle on a channel subset."""
    B, T, D, T0 = 2, 8192, 2048, 1024
    inp = make_inputs(60 + W, B, T, D, W, xdt=xdt)
    x, w, b = inp["x"].to(DEV), inp["w"].to(DEV), inp["b"].to(DEV)
    with torch.no_grad():
        long = causal_conv1d_fn(x, w, b, activation="silu")[:, :T0]
        prefix = causal_conv1d_fn(x[:, :T0].contiguous(), w, b, activation="silu")
        stacked = causal_conv1d_fn(x[:, :T0].repeat(8, 1, 1), w, b, activation="silu")
    torch.cuda.synchronize()
    assert torch.equal(long, prefix)
    assert torch.equal(stacked, prefix.repeat(8, 1, 1))
    cols = _cols(D, 8, W)
    sub = {"x": inp["x"][:, :T0], "w": inp["w"], "b": inp["b"], "init": None,
           "dy": inp["dy"][:, :T0], "dfinal": inp["dfinal"], "seq": None}
    ref = oracle_ref(sub, True, cols=cols, bwd=False)
    check_lowp(_sub(prefix.cpu(), cols), ref["out"], False, "out")


@pytest.mark.parametrize("case", ["cached", "seq_states", "streamed"])
def test_forward_cache_policies_leave_results_unchanged(case):
    """The forward picks its load/store cache policies and, for streaming inference calls, its
    workgroup walk per call (inference or training, and the bytes of x and out against the
    Infinity Cache); none of it touches the arithmetic. A training forward and an inference forward
    of the same inputs give identical outputs bit for bit, on both sides of the thresholds (64 MiB
    for inference, 128 MiB for training), and a channel subset matches the oracle."""
    B, T, D, W = {"cached": (4, 8192, 1024, 4), "seq_states": (2, 16384, 2048, 4),
                  "streamed": (4, 16384, 1024, 7)}[case]
    seq = varlen_seq(17, B, T, lo=64, hi=4096) if case == "seq_states" else None
    inp = make_inputs(41, B, T, D, W, init=case == "seq_states", seq=seq)
    x, w, b = inp["x"].to(DEV), inp["w"].to(DEV), inp["b"].to(DEV)
    init = None if inp["init"] is None else inp["init"].to(DEV)
    sq = None if seq is None else seq.to(DEV)
    final = seq is None
    xg = x.clone().requires_grad_(True)
    trained = causal_conv1d_fn(xg, w, b, seq_idx=sq, initial_states=init,
                               return_final_states=final, activation="silu")
    with torch.no_grad():
        inferred = causal_conv1d_fn(x, w, b, seq_idx=sq, initial_states=init,
                                    return_final_states=final, activation="silu")
    torch.cuda.synchronize()
    if final:
        assert torch.equal(trained[0].detach(), inferred[0])
        assert torch.equal(trained[1].detach(), inferred[1])
        out = inferred[0]
    else:
        assert torch.equal(trained.detach(), inferred)
        out = inferred
    cols = _cols(D, 6, 43)
    ref = oracle_ref(inp, True, cols=cols, bwd=False)
    check_lowp(_sub(out.cpu(), cols), ref["out"], False, "out")


@pytest.mark.parametrize("W,xdt", [(33, torch.bfloat16), (33, torch.float32), (64, torch.bfloat16),
                                   (64, torch.float32), (100, torch.bfloat16), (100, torch.float32),
                                   (128, torch.bfloat16), (128, torch.float32), (20, torch.float64)])
def test_generic_ring_widths(W, xdt):
    """Widths 33-128 (and fp64 x from width 2) run the generic kernels with their weights and row
    windows in LDS; from width 64 the backward's LDS exceeds the default 64 KiB and the launcher
    raises the kernel's limit. Against the oracle around the window length, with initial and final
    states and their gradients, and with seq_idx."""
    D = 72
    for T in (1, W - 1, W + 1, 300):
        init = T % 2 == 1
        inp = make_inputs(3 * W + T, 2, T, D, W, xdt=xdt, init=init)
        gpu = run_gpu(inp, "silu", return_final=True, dfinal=True, init_grad=init)
        ref = oracle_ref(inp, True, final=True, dfinal=True, need_dinit=init)
        compare(gpu, ref, True)
    seq = varlen_seq(W, 2, 400, lo=20, hi=150, pad_frac=0.1)
    inp = make_inputs(5 * W, 2, 400, D, W, xdt=xdt, init=True, seq=seq)
    gpu = run_gpu(inp, "silu", init_grad=True)
    compare(gpu, oracle_ref(inp, True, need_dinit=True), True)
    assert torch.all(gpu["out"][seq < 0] == 0) and torch.all(gpu["dx"][seq < 0] == 0)


@pytest.mark.parametrize("W", [17, 32])
@pytest.mark.parametrize("xdt", [torch.bfloat16, torch.float16, torch.float32])
def test_long_widths_dtypes_and_offsets(W, xdt):
    """Widths 17-32 take one channel per lane, so any channel count and any channel offset of x
    (rows aligned to one element only) run the register-window kernels: dims 72 (with a bias) and
    1000 (without), with and without the activation (without it bit-identical to the oracle:
    16-bit results rounded once from their fp32 values), and x, dout a slice at an odd
    channel offset of a wider tensor; with states and their gradients."""
    for D, T, bias in ((72, 300, True), (1000, 700, False)):
        for act in ("silu", None):
            inp = make_inputs(11 * W + D, 2, T, D, W, xdt=xdt, bias=bias, init=True)
            gpu = run_gpu(inp, act, return_final=True, dfinal=True, init_grad=True)
            compare(gpu, oracle_ref(inp, act is not None, final=True, dfinal=True, need_dinit=True),
                    act is not None)
    B, T, D, off = 2, 500, 200, 3
    inp = make_inputs(13 * W, B, T, D, W, xdt=xdt, init=True)
    big = torch.zeros(B, T, D + 9, dtype=xdt)
    big[..., off:off + D] = inp["x"]
    x = big.to(DEV)[..., off:off + D].detach().requires_grad_(True)
    dyb = torch.zeros(B, T, D + 5, dtype=xdt)
    dyb[..., 1:1 + D] = inp["dy"]
    w = inp["w"].to(DEV).requires_grad_(True)
    b = inp["b"].to(DEV).requires_grad_(True)
    init = inp["init"].to(DEV).requires_grad_(True)
    out = causal_conv1d_fn(x, w, b, initial_states=init, activation="silu")
    out.backward(dyb.to(DEV)[..., 1:1 + D])
    gpu = {"out": out.detach().cpu(), "dx": x.grad.cpu(), "dw": w.grad.cpu(), "db": b.grad.cpu(),
           "dinit": init.grad.cpu()}
    compare(gpu, oracle_ref(inp, True, need_dinit=True), True)


@pytest.mark.parametrize("W", [129, 200, 257])
@pytest.mark.parametrize("D", [8, 100])
def test_widths_above_128(W, D):
    """Any width >= 2 (reference README.md:40): above 128 the forward runs the generic kernel and
    the backward keeps g in the workspace (bwd_g_kernel, bwd_wide_kernel). Against the oracle at
    lengths around the window, with initial and final states and their gradients."""
    for T in (1, W - 1, W + 1, 300):
        init = T % 2 == 1
        inp = make_inputs(7 * W + T + D, 2, T, D, W, init=init)
        gpu = run_gpu(inp, "silu", return_final=True, dfinal=True, init_grad=init)
        ref = oracle_ref(inp, True, final=True, dfinal=True, need_dinit=init)
        compare(gpu, ref, True)


@pytest.mark.parametrize("xdt", [torch.float32, torch.float16])
@pytest.mark.parametrize("act", [None, "silu"])
def test_width_200_seq_idx(xdt, act):
    """Width 200 with packed sequences (padding runs, a repeated id) and initial states, in fp32
    and fp16, with and without the activation."""
    B, T, D, W = 2, 700, 64, 200
    seq = varlen_seq(200, B, T, lo=40, hi=300, pad_frac=0.1)
    seq[1, 50:90] = -3
    inp = make_inputs(201, B, T, D, W, xdt=xdt, init=True, seq=seq, bias=act is not None)
    gpu = run_gpu(inp, act, init_grad=True)
    compare(gpu, oracle_ref(inp, act is not None, need_dinit=True), act is not None)
    pad = seq < 0
    assert torch.all(gpu["out"][pad] == 0) and torch.all(gpu["dx"][pad] == 0)


# ------------------------------------------------------------------------------------------------
# BASELINE configurations at full size.
# ------------------------------------------------------------------------------------------------

def _cols(D, n, seed):
    g = _gen(seed)
    idx = torch.randperm(D, generator=g)[:n]
    return torch.cat([idx, torch.tensor([0, D - 1])]).unique()


@pytest.mark.parametrize("B,T,D,W,xdt,seq", [
    (16, 512, 4096, 6, torch.bfloat16, False),   # one workgroup per column along time (64 rows)
    (32, 1024, 2048, 12, torch.bfloat16, True),  # one channel per lane, seq_idx tiles of all kinds
    (24, 1024, 3072, 16, torch.float16, False),
    (6, 2048, 4096, 20, torch.bfloat16, False),  # width 20: 2-row batches
    (8, 1024, 4096, 24, torch.float32, True),
    (4, 1024, 8192, 32, torch.bfloat16, False),  # 128-row tiles in both passes
    (8, 2048, 4096, 28, torch.float16, False),
])
def test_mid_size_long_tiles(B, T, D, W, xdt, seq):
    """Shapes where the backward (2 or 1 channels per lane) and the forward from width 12 take
    64-row tiles however few workgroups that leaves along time, and where, without seq_idx, the
    backward with one channel per lane takes 128-row tiles (widths 16, 20, 28 and 32 here) and the
    forward from width 24 too (28 and 32): a channel subset against the oracle, with initial
    states and their gradient, and final states and theirs where seq_idx allows them."""
    s = varlen_seq(B + W, B, T, lo=64, hi=1024, pad_frac=0.05) if seq else None
    inp = make_inputs(B * 100 + W, B, T, D, W, xdt=xdt, init=True, seq=s)
    gpu = run_gpu(inp, "silu", return_final=not seq, dfinal=not seq, init_grad=True)
    cols = _cols(D, 24, W)
    ref = oracle_ref(inp, True, cols=cols, final=not seq, dfinal=not seq, need_dinit=True)
    compare(gpu, ref, True, cols=cols)
    if seq:
        assert torch.all(gpu["out"][s < 0] == 0) and torch.all(gpu["dx"][s < 0] == 0)


@pytest.mark.parametrize("T", [512, 2048, 8192, 32768])
@pytest.mark.parametrize("variant", ["weight_only", "bias_silu"])
def test_config2_readme_sweep(T, variant):
    """B=4, D=1024, W=4, bf16 x, fp32 weight ~N(0, 1/4); weight only, or bias ~N(0,1) + silu."""
    bias = variant == "bias_silu"
    inp = make_inputs(T, 4, T, 1024, 4, bias=bias)
    act = "silu" if bias else None
    gpu = run_gpu(inp, act)
    cols = _cols(1024, 30, T)
    compare(gpu, oracle_ref(inp, bias, cols=cols), bias, cols=cols)


@pytest.mark.parametrize("B,T,D,W,xdt", [
    (2, 8192, 1024, 4, torch.bfloat16),  # forward 4 channels per lane, backward 2 (small grid)
    (4, 4096, 1024, 5, torch.float16),   # the same split at width 5 (backward with 4-row batches)
    (4, 2048, 1002, 4, torch.bfloat16),  # dim not a multiple of 4: both passes 2 channels per lane
    (1, 512, 262, 5, torch.float16),     # the same on a small grid at width 5
    (8, 1024, 4096, 4, torch.bfloat16),  # 16-row forward tiles: 2 channels in the forward, 4 back
    (8, 1024, 2048, 6, torch.float16),   # the same at width 6 (2 channels in both passes)
    (8, 1024, 2048, 4, torch.float32),   # fp32 keeps 4 channels on 16-row forward tiles
    (4, 8192, 1024, 6, torch.bfloat16),  # width 6: the widest 4-channel forward, 2-channel backward
    (4, 8192, 1024, 7, torch.float16),   # width 7: both passes 2 channels per lane
    (4, 8192, 1024, 8, torch.bfloat16),  # width 8: the same, 4-row backward batches
])
def test_channels_per_lane_choices(B, T, D, W, xdt):
    """Shapes on either side of the host's choice of 4 or 2 channels per lane in each pass, with
    initial states, final states and their gradients, against the oracle on a channel subset."""
    inp = make_inputs(B * T + D + W, B, T, D, W, xdt=xdt, init=True)
    gpu = run_gpu(inp, "silu", return_final=True, dfinal=True, init_grad=True)
    cols = _cols(D, 40, B * T)
    ref = oracle_ref(inp, True, cols=cols, final=True, dfinal=True, need_dinit=True)
    compare(gpu, ref, True, cols=cols)


@pytest.mark.parametrize("W,xdt", [(9, torch.bfloat16), (12, torch.bfloat16), (16, torch.bfloat16),
                                   (16, torch.float16), (17, torch.bfloat16), (20, torch.bfloat16),
                                   (24, torch.float16), (25, torch.bfloat16), (32, torch.bfloat16)])
def test_row_passes_longer_than_the_window(W, xdt):
    """From width 9 the pipelined row loops run passes of 2-4 double batches (16-32 rows, longer
    than the window) before the 8-row passes and the single rows of a tile's end. At B=4 T=8189
    D=1024 the grid reaches the tilings' wave target with their longest tiles (64 rows in the
    2-channel forward, 128 in the one-channel passes), so every pass kind runs, and the ragged
    last tile ends in a different place; against the oracle on a channel subset, without the
    activation bit-identical."""
    B, T, D = 4, 8189, 1024
    cols = _cols(D, 24, 31 * W)
    for act in ("silu", None):
        inp = make_inputs(17 * W + (act is None), B, T, D, W, xdt=xdt, init=True)
        gpu = run_gpu(inp, act, return_final=True, dfinal=True, init_grad=True)
        ref = oracle_ref(inp, act is not None, cols=cols, final=True, dfinal=True, need_dinit=True)
        compare(gpu, ref, act is not None, cols=cols)


@pytest.mark.parametrize("B,T,D,W,xdt,seq", [
    (4, 2048, 1024, 4, torch.bfloat16, False),
    (4, 2048, 1024, 2, torch.float16, False),
    (1, 4096, 2048, 3, torch.bfloat16, False),
    (16, 256, 2048, 5, torch.float16, False),
    (4, 2047, 1024, 4, torch.bfloat16, True),    # seq_idx, ragged last tile
    (4, 2048, 1024, 4, torch.float32, False),    # fp32 keeps 32-row tiles
])
def test_small_grid_backward_short_tiles(B, T, D, W, xdt, seq):
    """Grids whose 2-channel backward falls short of the wave target with 32-row tiles take 16-row
    tiles for 16-bit x at widths 2-5 (twice the partial dweight rows per column); against the
    oracle on a channel subset, with initial and final states and their gradients, and with
    seq_idx."""
    s = varlen_seq(60 + W, B, T, lo=40, hi=700, pad_frac=0.04) if seq else None
    inp = make_inputs(B + T + W, B, T, D, W, xdt=xdt, init=True, seq=s)
    gpu = run_gpu(inp, "silu", return_final=not seq, dfinal=not seq, init_grad=True)
    cols = _cols(D, 32, T + W)
    ref = oracle_ref(inp, True, cols=cols, final=not seq, dfinal=not seq, need_dinit=True)
    compare(gpu, ref, True, cols=cols)


def test_config3_mamba2_xbc():
    """B=8, T=4096, D=5376, W=4; x a channel slice of an in_proj output (time stride 10576)."""
    B, T, D, W = 8, 4096, 5376, 4
    inp = make_inputs(3, B, T, D, W, wdist="uniform")
    big = torch.empty(B, T, 10576, dtype=torch.bfloat16, device=DEV)
    big[..., 5120:5120 + D] = inp["x"].to(DEV)
    gpu = run_gpu(inp, "silu", x_override=big[..., 5120:5120 + D])
    cols = _cols(D, 24, 3)
    compare(gpu, oracle_ref(inp, True, cols=cols), True, cols=cols)


def test_config4_streaming_chunks_and_decode():
    """B=16, D=2048, W=4, T=8192 as 32 chunks of 256 with state handoff, and 64 decode steps of
    T=1: both bit-identical to one full-length pass."""
    B, T, D, W = 16, 8192, 2048, 4
    inp = make_inputs(4, B, T, D, W)
    x, w, b = inp["x"].to(DEV), inp["w"].to(DEV), inp["b"].to(DEV)
    with torch.no_grad():
        full, fin = causal_conv1d_fn(x, w, b, return_final_states=True, activation="silu")
        state, outs = None, []
        for c in range(32):
            o, state = causal_conv1d_fn(x[:, c * 256:(c + 1) * 256], w, b, initial_states=state,
                                        return_final_states=True, activation="silu")
            outs.append(o)
        assert torch.equal(torch.cat(outs, dim=1), full)
        assert torch.equal(state, fin)
        state = None
        for t in range(64):
            o, state = causal_conv1d_fn(x[:, t:t + 1], w, b, initial_states=state,
                                        return_final_states=True, activation="silu")
            assert torch.equal(o, full[:, t:t + 1]), t
    cols = _cols(D, 16, 4)
    ref = oracle_ref(inp, True, cols=cols, final=True, bwd=False)
    check_lowp(_sub(full.cpu(), cols), ref["out"], False, "full out")
    assert torch.equal(_sub(fin.cpu(), cols).float(), torch.from_numpy(ref["final"]))


def test_config4_chunked_training_matches_full():
    """Gradients through the state handoff: two chunks vs one pass (tolerance only, since the
    state gradient is rounded to bf16 between the chunks)."""
    B, T, D, W = 4, 1024, 512, 4
    inp = make_inputs(8, B, T, D, W)
    x = inp["x"].to(DEV).requires_grad_(True)
    w = inp["w"].to(DEV).requires_grad_(True)
    b = inp["b"].to(DEV).requires_grad_(True)
    dy = inp["dy"].to(DEV)
    out = causal_conv1d_fn(x, w, b, activation="silu")
    (out.float() * dy.float()).sum().backward()
    g_full = [t.grad.clone() for t in (x, w, b)]
    for t in (x, w, b):
        t.grad = None
    o1, s1 = causal_conv1d_fn(x[:, :400], w, b, return_final_states=True, activation="silu")
    o2 = causal_conv1d_fn(x[:, 400:], w, b, initial_states=s1, activation="silu")
    assert torch.equal(torch.cat([o1, o2], dim=1), out)
    (torch.cat([o1, o2], dim=1).float() * dy.float()).sum().backward()
    torch.testing.assert_close(x.grad.float(), g_full[0].float(), rtol=1e-2, atol=1e-2)
    torch.testing.assert_close(w.grad, g_full[1], rtol=1e-3, atol=1e-2)
    torch.testing.assert_close(b.grad, g_full[2], rtol=1e-3, atol=1e-2)


@pytest.mark.parametrize("W", [4, 7])
def test_config5_varlen_seq_idx(W):
    """B=4, T=16384, D=4096; segments ~U[64,4096] with ids 0,1,2,... and the last 5% padding (-1);
    initial_states bf16 belong to segment 0; bias + silu, forward + backward."""
    B, T, D = 4, 16384, 4096
    seq = varlen_seq(50 + W, B, T)
    inp = make_inputs(W, B, T, D, W, init=True, seq=seq)
    gpu = run_gpu(inp, "silu", init_grad=True)
    pad = seq < 0
    assert torch.all(gpu["out"][pad] == 0) and torch.all(gpu["dx"][pad] == 0)
    cols = _cols(D, 12, W)
    compare(gpu, oracle_ref(inp, True, cols=cols, need_dinit=True), True, cols=cols)


def test_maximum_in_batch_offset():
    """(T + W) * D just below 2^31: the largest sequence the 32-bit in-batch offsets allow."""
    D, W = 2048, 4
    T = (2**31 - 1) // D - W
    g = torch.Generator(DEV).manual_seed(12)
    x = torch.randn(1, T, D, generator=g, device=DEV, dtype=torch.bfloat16)
    w = torch.randn(D, W, generator=g, device=DEV) / 2
    with torch.no_grad():
        out, fin = causal_conv1d_fn(x, w, return_final_states=True)
    cols = torch.tensor([0, 1, 777, D - 1])
    xs = _sub(x, cols.to(DEV)).cpu()
    ws = _sub(w, cols.to(DEV), 0).cpu()
    del x
    ref, rfin = oracle.fwd(_np32(xs), _np32(ws), final=True)
    check_lowp(_sub(out.cpu(), cols), ref, True, "out")
    assert torch.equal(_sub(fin.cpu(), cols).float(), torch.from_numpy(rfin))


# ------------------------------------------------------------------------------------------------
# Workspaces and graphs reused across calls.
# ------------------------------------------------------------------------------------------------

def _bwd_direct(inp, workspace):
    from causal_conv1d_triton import _ffi

    x, w, b = inp["x"].to(DEV), inp["w"].to(DEV), inp["b"].to(DEV)
    dy = inp["dy"].to(DEV)
    dx, dw, db = torch.empty_like(x), torch.empty_like(w), torch.empty_like(b)
    _ffi.bwd(x, w, b, None, None, dy, None, dx, None, dw, db, workspace, True)
    torch.cuda.synchronize()
    return {"dx": dx.cpu(), "dw": dw.cpu(), "db": db.cpu()}


def test_reused_workspace_with_arbitrary_contents():
    """A reused workspace may hold anything (here an int64 arange). Results must not depend on its
    contents and must match the oracle, call after call."""
    from causal_conv1d_triton import _ffi

    B, T, D, W = 4, 2048, 1024, 4
    inp = make_inputs(21, B, T, D, W)
    n = _ffi.bwd_workspace_bytes(B, T, D, W, torch.bfloat16)
    ws = torch.arange((n + 7) // 8, dtype=torch.int64, device=DEV).view(torch.uint8)[:n]
    ref = oracle_ref(inp, True)
    first = _bwd_direct(inp, ws)
    for _ in range(3):
        again = _bwd_direct(inp, ws)
        assert torch.equal(again["dw"], first["dw"]) and torch.equal(again["db"], first["db"])
    check_sum(first["dw"], ref["dw"], "dweight")
    check_sum(first["db"], ref["db"], "dbias")
    check_lowp(first["dx"], ref["dx"], False, "dx")


def _direct_bwd_call(x, w, b, dy, ws, silu=True, stream=None):
    from causal_conv1d_triton import _ffi

    dx, dw = torch.empty_like(x), torch.empty_like(w)
    db = None if b is None else torch.empty_like(b)
    with torch.cuda.stream(stream or torch.cuda.current_stream()):
        _ffi.bwd(x, w, b, None, None, dy, None, dx, None, dw, db, ws, silu)
    return dx, dw, db


@pytest.mark.parametrize("B,T,D,W,bias", [
    (4, 2048, 1024, 4, True),
    (4, 8192, 1024, 4, True),    # 128 partial rows per wave column: the reduction kernel
    (2, 4096, 2048, 4, False),   # no bias: W value rows per channel
    (3, 777, 1000, 3, True),     # last wave column partly outside dim (1000 = 3 * 256 + 232)
    (1, 17, 256, 8, True),       # one partial row per wave column
    (2, 1024, 4096, 4, True),
])
def test_dweight_repeatable_with_garbage_workspace(B, T, D, W, bias):
    """dweight/dbias are bit-identical over repeated calls whose workspace starts with different
    contents each time (random bytes), and match the oracle."""
    from causal_conv1d_triton import _ffi

    inp = make_inputs(5 + W, B, T, D, W, bias=bias)
    x, w, dy = inp["x"].to(DEV), inp["w"].to(DEV), inp["dy"].to(DEV)
    b = inp["b"].to(DEV) if bias else None
    n = _ffi.bwd_workspace_bytes(B, T, D, W, torch.bfloat16)
    g = torch.Generator(device=DEV).manual_seed(7)
    results = []
    for _ in range(6):
        ws = torch.randint(0, 256, (n,), dtype=torch.uint8, device=DEV, generator=g)
        _, dw, db = _direct_bwd_call(x, w, b, dy, ws)
        torch.cuda.synchronize()
        results.append((dw.cpu(), None if db is None else db.cpu()))
    for dw, db in results[1:]:
        assert torch.equal(dw, results[0][0])
        assert db is None or torch.equal(db, results[0][1])
    ref = oracle_ref(inp, True)
    check_sum(results[0][0], ref["dw"], "dweight")
    if bias:
        check_sum(results[0][1], ref["db"], "dbias")


@pytest.mark.parametrize("B,T,D,W,bias", [
    (4, 512, 1024, 4, True),     # 32 partial rows per wave column (fewer than the 16 row sets x 8)
    (4, 2048, 1024, 4, True),
    (3, 777, 1000, 3, True),     # a wave column partly outside dim
    (2, 300, 96, 7, False),      # no bias, 2 channels per lane
    (1, 17, 256, 8, True),       # one partial row
    (4, 8192, 1024, 4, True),    # 128 rows
    (2, 8192, 2048, 4, False),
])
def test_reduction_order_matches_partial_rows(B, T, D, W, bias):
    """dweight/dbias equal, bit for bit, the fp32 sums of the partial rows the backward leaves at
    the start of its workspace ((rows, W + 1, dim) floats), added in the order reduce_partials_kernel
    documents: 16 interleaved row sets (set j holds rows j, j + 16, ...) each summed in row order
    from zero, then the set sums added in set order. A row missed or read before its writer
    finished would change the bits."""
    from causal_conv1d_triton import _ffi

    inp = make_inputs(90 + W, B, T, D, W, bias=bias)
    x, w, dy = inp["x"].to(DEV), inp["w"].to(DEV), inp["dy"].to(DEV)
    b = inp["b"].to(DEV) if bias else None
    n = _ffi.bwd_workspace_bytes(B, T, D, W, torch.bfloat16)
    ws = torch.randint(0, 256, (n,), dtype=torch.uint8, device=DEV,
                       generator=torch.Generator(device=DEV).manual_seed(3))
    _, dw, db = _direct_bwd_call(x, w, b, dy, ws)
    torch.cuda.synchronize()
    rows = _ffi.bwd_workspace_bytes_for(x, None, dy, None, torch.empty_like(x), W)
    rows //= (W + 1) * D * 4
    part = ws[:rows * (W + 1) * D * 4].view(torch.float32).view(rows, W + 1, D).cpu()
    sets = []
    for j in range(16):
        a = torch.zeros(W + 1, D)
        for r in range(j, rows, 16):
            a = a + part[r]
        sets.append(a)
    acc = sets[0]
    for a in sets[1:]:
        acc = acc + a
    assert torch.equal(dw.cpu(), acc[:W].t().contiguous())
    if bias:
        assert torch.equal(db.cpu(), acc[W])
    check_sum(dw.cpu(), oracle_ref(inp, True)["dw"], "dweight")


def test_back_to_back_calls_share_one_workspace():
    """Many backward calls queued on one stream with one workspace and no synchronisation in
    between; every call must give the same bits."""
    from causal_conv1d_triton import _ffi

    B, T, D, W = 4, 1024, 1024, 4
    inp = make_inputs(61, B, T, D, W)
    x, w, b, dy = (inp[k].to(DEV) for k in ("x", "w", "b", "dy"))
    ws = torch.zeros(_ffi.bwd_workspace_bytes(B, T, D, W, torch.bfloat16), dtype=torch.uint8,
                     device=DEV)
    outs = [_direct_bwd_call(x, w, b, dy, ws) for _ in range(40)]
    torch.cuda.synchronize()
    for dx, dw, db in outs[1:]:
        assert torch.equal(dx, outs[0][0]) and torch.equal(dw, outs[0][1])
        assert torch.equal(db, outs[0][2])


def test_concurrent_streams():
    """Backward calls on two streams at once, each with its own workspace, give the results of the
    same calls made one at a time."""
    from causal_conv1d_triton import _ffi

    B, T, D, W = 2, 4096, 1024, 4
    a = make_inputs(71, B, T, D, W)
    c = make_inputs(72, B, T, D, W)
    ta = [a[k].to(DEV) for k in ("x", "w", "b", "dy")]
    tc = [c[k].to(DEV) for k in ("x", "w", "b", "dy")]
    n = _ffi.bwd_workspace_bytes(B, T, D, W, torch.bfloat16)
    wsa = torch.empty(n, dtype=torch.uint8, device=DEV)
    wsc = torch.empty(n, dtype=torch.uint8, device=DEV)
    ref_a = [t.clone() for t in _direct_bwd_call(*ta, wsa)]
    ref_c = [t.clone() for t in _direct_bwd_call(*tc, wsc)]
    torch.cuda.synchronize()
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    s1.wait_stream(torch.cuda.current_stream())
    s2.wait_stream(torch.cuda.current_stream())
    got_a, got_c = [], []
    for _ in range(8):
        got_a.append(_direct_bwd_call(*ta, wsa, stream=s1))
        got_c.append(_direct_bwd_call(*tc, wsc, stream=s2))
    torch.cuda.synchronize()
    for ga, gc in zip(got_a, got_c):
        for u, v in zip(ga, ref_a):
            assert torch.equal(u, v)
        for u, v in zip(gc, ref_c):
            assert torch.equal(u, v)


@pytest.mark.parametrize("B,T,D,W", [(2, 4096, 1024, 4), (4, 512, 1024, 4), (2, 700, 96, 64),
                                     (2, 700, 96, 128)])
def test_graph_replays_match_eager(B, T, D, W):
    """fwd+bwd captured in a HIP graph and replayed several times, with the program's own eager work
    and synchronisations in between; every replay must equal the eager result bit for bit. Widths
    64 and 128 run the generic ring kernels, whose LDS above 64 KiB is allowed once per device on
    their first launch, so the captured launches make no runtime call for it."""
    inp = make_inputs(33, B, T, D, W, init=True)
    x = inp["x"].to(DEV).requires_grad_(True)
    w = inp["w"].to(DEV).requires_grad_(True)
    b = inp["b"].to(DEV).requires_grad_(True)
    init = inp["init"].to(DEV).requires_grad_(True)
    dy = inp["dy"].to(DEV)

    def step():
        out = causal_conv1d_fn(x, w, b, initial_states=init, activation="silu")
        return (out,) + torch.autograd.grad(out, (x, w, b, init), dy)

    eager = [t.detach().clone() for t in step()]
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        step()
    torch.cuda.current_stream().wait_stream(side)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        outs = step()
    for rep in range(4):
        g.replay()
        torch.cuda.synchronize()
        for a, e in zip(outs, eager):
            assert torch.equal(a, e), f"replay {rep}"
        # eager work between replays, including another backward on a fresh workspace
        other = step()
        torch.cuda.synchronize()
        assert torch.equal(other[2], eager[2])


# ------------------------------------------------------------------------------------------------
# Backward into a strided dx (fusion with the in_proj epilogue: dx lands in its slice of the
# projection output's gradient).
# ------------------------------------------------------------------------------------------------

@pytest.mark.parametrize("case", ["aligned", "odd_offset", "generic_width", "wide_width", "seq_idx",
                                  "states", "straddling"])
def test_backward_into_strided_dx(case):
    """causal_conv1d_bwd writes dx into channels [c0, c0 + dim) of a wider buffer: the same bits
    as the contiguous backward, and every other element of the buffer untouched. At an odd channel
    offset dx's rows are not aligned for the vectorised kernels, so the generic kernels run; their
    rounding differs from the vectorised ones', and that case is held to the tolerances."""
    from causal_conv1d_triton.causal_conv1d import _bwd
    from causal_conv1d_triton.fused import causal_conv1d_bwd

    B, T, D, W, c0, wide = 2, 700, 512, 4, 512, 1536
    if case == "odd_offset":
        c0 = 3                       # rows misaligned for the vectorised kernels: generic path
    if case == "straddling":
        # a 3104-byte pitch: rows start 0, 32, 64 or 96 bytes into a 128-byte line, so the
        # backward takes the column-fastest workgroup order and non-temporal dx stores
        wide = 1552
    if case == "generic_width":
        W = 20
    if case == "wide_width":
        W, T, D = 200, 300, 64
    seq = varlen_seq(31, B, T, lo=30, hi=200) if case == "seq_idx" else None
    init = case == "states"
    inp = make_inputs(77, B, T, D, W, init=init, seq=seq)
    x, w, b, dy = (inp[k].to(DEV) for k in ("x", "w", "b", "dy"))
    s0 = inp["init"].to(DEV) if init else None
    sq = None if seq is None else seq.to(DEV)
    dfin = inp["dfinal"].to(DEV) if case == "states" else None
    buf = torch.full((B, T, wide), 7.0, dtype=x.dtype, device=DEV)
    view = buf[..., c0:c0 + D]
    dx, dw, db, dinit = causal_conv1d_bwd(x, w, b, dy, seq_idx=sq, initial_states=s0,
                                          dfinal_states=dfin, dx=view,
                                          return_dinitial_states=init, activation="silu")
    want = _bwd(x, w, b, sq, s0, dy, dfin, init, True)
    torch.cuda.synchronize()
    assert dx.data_ptr() == view.data_ptr()
    if case == "odd_offset":
        torch.testing.assert_close(view.float(), want[0].float(), rtol=1e-2, atol=1e-2)
        # The generic kernels sum dweight/dbias over other tiles: fp32 rounding apart.
        for got, ref in ((dw, want[1]), (db, want[2])):
            rms = ref.double().pow(2).mean().sqrt().item()
            torch.testing.assert_close(got, ref, rtol=1e-3, atol=1e-5 * rms + 1e-7)
    else:
        assert torch.equal(view, want[0]), case
        assert torch.equal(dw, want[1]) and torch.equal(db, want[2]), case
    if init:
        assert torch.equal(dinit, want[3])
    outside = torch.ones(wide, dtype=torch.bool)
    outside[c0:c0 + D] = False
    assert torch.all(buf[..., outside.to(DEV)] == 7.0), "elements outside dx were written"
    ref = oracle_ref(inp, True, dfinal=dfin is not None, need_dinit=init)
    check_lowp(dx.cpu(), ref["dx"], False, "dx")
    check_sum(dw.cpu(), ref["dw"], "dweight")


@pytest.mark.parametrize("W", [4, 7])
def test_straddling_slices_match_contiguous(W):
    """x and the upstream gradient as channel slices of wider tensors whose rows straddle 128-byte
    lines (a pitch of 1552 channels, like Mamba-2's in_proj output) take the column-fastest
    workgroup order in both passes; every result is bit-identical to the same call on contiguous
    copies."""
    B, T, D, c0, wide = 2, 600, 512, 512, 1552
    inp = make_inputs(44, B, T, D, W, init=True)
    x, w, b, dy, s0 = (inp[k].to(DEV) for k in ("x", "w", "b", "dy", "init"))

    def run(xv, dyv):
        xv = xv.detach().requires_grad_(True)
        wv, bv, sv = (t.clone().requires_grad_(True) for t in (w, b, s0))
        out = causal_conv1d_fn(xv, wv, bv, initial_states=sv, activation="silu")
        grads = torch.autograd.grad(out, (xv, wv, bv, sv), dyv)
        return (out,) + grads

    bx = torch.zeros(B, T, wide, dtype=x.dtype, device=DEV)
    by = torch.zeros(B, T, wide, dtype=x.dtype, device=DEV)
    bx[..., c0:c0 + D] = x
    by[..., c0:c0 + D] = dy
    got = run(bx[..., c0:c0 + D], by[..., c0:c0 + D])
    want = run(x, dy)
    for g, e in zip(got, want):
        assert torch.equal(g, e)
