#!/usr/bin/env python3
"""Benchmark of the hot path: forward + backward of causal_conv1d_fn on one MI355X.

Workload (BASELINE.json metric): x (4, 8192, 1024) bf16 ~N(0,1), weight (1024, 4) fp32 ~N(0, 1/4),
bias (1024) fp32 ~N(0,1), activation silu, upstream gradient (4, 8192, 1024) bf16 ~N(0,1). One step =
out = causal_conv1d_fn(x, w, b, activation="silu") followed by the gradients of x, w and b
(torch.autograd.grad, so nothing is accumulated). Input sets rotate (4 sets of x and dy, 512 MiB, twice
the 256 MiB Infinity Cache) so every step reads its inputs from HBM. Up to 64 steps, the input sets in
rotation, are captured into one HIP graph and replayed, which removes Python launch overhead and
nearly all graph-launch gaps from the device timeline. The time of each pass inside the step comes from
events between the passes of eager steps that make the same launches, and the time of each pass's
main kernel (the roofline entry: the backward kernel) from events HIP sets to those kernels' own
dispatch start and end in other eager steps.
Every timed region follows at least --warmup steps and at least 50 ms of untimed replays, so it
measures the device's steady state rather than its clock ramp after idle.

Prints one JSON line. `value` is the step's algorithmic HBM bytes (read x, write out; read x, read dy,
write dx; plus weights and bias) divided by the measured step time, in GB/s.
"""

import argparse
import json
import math
import os
import sys
import time

import torch

_ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(_ROOT, "causal-conv1d-triton_amd"))

METRIC = "fwd+bwd latency (us) and achieved HBM GB/s vs peak, bf16 B=4 T=8192 D=1024 W=4"
PEAK_GBS = 8000.0  # MI355X HBM3E, public spec


def alg_bytes(B, T, D, W, ex=2, ew=4, eb=4):
    """Algorithmic HBM bytes of one forward and one backward pass (weights and bias read once per
    pass; the backward also writes dweight and dbias). The backward's fp32 partial-sum workspace is
    excluded: it is implementation traffic, reported by the rocprof counters."""
    n = B * T * D
    fwd = n * (ex + ex) + D * W * ew + D * eb
    bwd = n * (ex + ex + ex) + 2 * D * W * ew + 2 * D * eb
    return fwd, bwd


def bwd_kernel_alg_bytes(B, T, D, W, ex=2, ew=4, eb=4):
    """Algorithmic bytes of the backward pass's main kernel: x and dout read, dx written, weights
    and bias read. dweight and dbias are written by the reduction that follows it."""
    return B * T * D * (ex + ex + ex) + D * W * ew + D * eb


def _capture(fn, warm_stream):
    """Warms fn up on a side stream (as torch requires before capture) and captures it."""
    warm_stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(warm_stream):
        for _ in range(2):
            fn()
    torch.cuda.current_stream().wait_stream(warm_stream)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        fn()
    return g


# Calls per captured graph of the --configs, --widths and --shapes measurements.
CONFIG_GRAPH_CALLS = 32

# Steps per captured graph of the headline measurement (main()).
GRAPH_STEPS = 64

# Minimum untimed device work before each timed region. MI355X raises its clocks over roughly the
# first 10-15 ms of sustained work after any idle period of ~10 ms or more; a warm-up shorter than
# that measures the ramp instead of the steady state.
MIN_WARMUP_MS = 50.0


def _warm(graph, min_replays, min_ms=MIN_WARMUP_MS):
    """Replays `graph` at least `min_replays` times and for at least `min_ms` of wall time, without
    leaving the device idle in between. Returns the number of replays."""
    n, t0 = 0, time.perf_counter()
    while n < min_replays or (time.perf_counter() - t0) * 1e3 < min_ms:
        for _ in range(8):
            graph.replay()
        n += 8
        torch.cuda.synchronize()
    return n


_SPIN_CYCLES_PER_MS = None


def _spin_cycles_per_ms():
    """Cycles of torch's bounded spin kernel (torch.cuda._sleep) per millisecond on this device,
    measured once."""
    global _SPIN_CYCLES_PER_MS
    if _SPIN_CYCLES_PER_MS is None:
        s0, s1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda._sleep(1 << 16)  # first launch outside the measurement
        s0.record()
        torch.cuda._sleep(1 << 20)
        s1.record()
        torch.cuda.synchronize()
        _SPIN_CYCLES_PER_MS = (1 << 20) / max(s0.elapsed_time(s1), 1e-3)
    return _SPIN_CYCLES_PER_MS


# Device time queued ahead of a timed region: a replayed graph reaches the device only after the
# host has launched it (tens of microseconds for the first one), so a timed region that starts on an
# idle device would count that host latency as device time, about 1.5 us per step when only 20
# steps are timed. A bounded spin kernel keeps the device busy while the host queues the start
# event and the replays; the start event then executes right before the first replay.
LEAD_MS = 0.5


def _time_graphs(seq):
    """Device time of replaying the graphs in `seq` in order: events around the whole sequence,
    queued behind LEAD_MS of spin so the device never waits for the host inside the region."""
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    torch.cuda._sleep(int(_spin_cycles_per_ms() * LEAD_MS))
    start.record()
    for g in seq:
        g.replay()
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end)


def passes_in_step(sets, w, b, steps):
    """Mean device time of the forward and of the backward pass inside fwd+bwd steps, of the step,
    and of each pass's main kernel. The steps run eagerly through the launches causal_conv1d_fn and
    its autograd backward make (_fwd, then _bwd: the same kernels on the same stream). On some steps
    HIP events are recorded on the launch stream before the forward, between the passes and after
    the backward (pass times); on other steps no event packet is queued, and the library is asked
    (ccv1d_time_main_kernel) to launch the forward and the backward kernel with events that HIP sets
    from those dispatches' own start and end timestamps (kernel times, the same quantity a
    rocprofv3 kernel trace records). All measured steps are queued behind a bounded spin kernel
    (torch.cuda._sleep) that keeps the device busy while the host enqueues them, so the device then
    runs them back to back without waiting for the host and each interval is device time only.
    Returns {"fwd": ms, "bwd": ms, "step": ms, "fwd_kernel": ms, "bwd_kernel": ms}."""
    from causal_conv1d_triton import _ffi
    from causal_conv1d_triton.causal_conv1d import _bwd, _fwd

    n = len(sets)
    wd, bd = w.detach(), b.detach()

    def step(i, ev=None, kev=None):
        x, dy = sets[i % n]
        if ev:
            ev[0].record()
        if kev:
            _ffi.time_main_kernel(kev[0], kev[1])
        _fwd(x.detach(), wd, bd, None, None, None, True)
        if ev:
            ev[1].record()
        if kev:
            _ffi.time_main_kernel(kev[2], kev[3])
        r = _bwd(x.detach(), wd, bd, None, None, dy, None, False, True)
        if ev:
            ev[2].record()
        return r

    cycles_per_ms = _spin_cycles_per_ms()
    # host time to enqueue one step, measured on the warm-up steps
    k, t0 = 0, time.perf_counter()
    while k < 2 * n or (time.perf_counter() - t0) * 1e3 < MIN_WARMUP_MS:
        step(k)
        k += 1
        if k % 32 == 0:
            torch.cuda.synchronize()
    torch.cuda.synchronize()
    host_ms = (time.perf_counter() - t0) * 1e3 / k
    # Events on every EVERY-th step only: an event between two launches costs the device time of
    # its own, which the other steps then do not pay.
    every = 4
    steps = max(steps, 2 * every)
    evs = {i: [torch.cuda.Event(enable_timing=True) for _ in range(3)]
           for i in range(steps) if i % every == every - 1}
    kevs = {i: [torch.cuda.Event(enable_timing=True) for _ in range(4)]
            for i in range(steps) if i % every == every // 2 - 1}
    for kev in kevs.values():
        for e in kev:
            e.record()  # torch creates the HIP event at its first record
    first, last = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    # queue some warm steps, then the spin, then the measured steps, so the device is busy and warm
    for i in range(16):
        step(i)
    torch.cuda._sleep(int(cycles_per_ms * (2 * host_ms * steps + 5)))
    skip = 4 * every  # steps right after the spin, while clocks ramp up again
    for i in range(steps + skip):
        if i == skip:
            first.record()
        step(i, evs.get(i - skip), kevs.get(i - skip))
    last.record()
    torch.cuda.synchronize()
    use = list(evs.values())
    fwd = sum(e[0].elapsed_time(e[1]) for e in use) / len(use)
    bwd = sum(e[1].elapsed_time(e[2]) for e in use) / len(use)
    kuse = list(kevs.values())
    fwd_k = sum(e[0].elapsed_time(e[1]) for e in kuse) / len(kuse)
    bwd_k = sum(e[2].elapsed_time(e[3]) for e in kuse) / len(kuse)
    step_ms = first.elapsed_time(last) / steps
    return {"fwd": fwd, "bwd": bwd, "step": step_ms, "fwd_kernel": fwd_k, "bwd_kernel": bwd_k}


def calibrate_copy(dev, mib=256, reps=3):
    """Plain elementwise kernels of known traffic, run so that a rocprofv3 --pmc pass over this
    process also records FETCH_SIZE / WRITE_SIZE for kernels whose true HBM bytes are known: a fill
    (writes mib MiB) and a negation (reads mib MiB, writes mib MiB; larger than the 256 MB Infinity
    Cache, so its reads miss). The ratio of counter to true bytes scales the conv kernels' counters."""
    src = torch.empty(mib << 18, dtype=torch.float32, device=dev).fill_(1.0)
    dst = torch.empty_like(src)
    for _ in range(reps):
        torch.neg(src, out=dst)
    torch.cuda.synchronize()


def traffic_from_profiles():
    """HBM bytes per launch of the backward pass, derived from committed rocprofv3 counter runs
    (profiles/traffic.json; written from FETCH_SIZE and WRITE_SIZE passes scaled by a plain copy of
    known size). None when absent."""
    path = os.path.join(_ROOT, "profiles", "traffic.json")
    if not os.path.exists(path):
        return None
    with open(path) as f:
        return json.load(f)


def _timed_reps(fn, seconds, max_reps=1000):
    fn()  # first call outside the timed loop (allocator and thread-pool start-up)
    reps, t0 = 0, time.perf_counter()
    while True:
        fn()
        reps += 1
        el = time.perf_counter() - t0
        if el >= seconds or reps >= max_reps:
            return reps, el


def cpu_baseline(seconds):
    """The reference math on the GPU box's host cores, in the metric's unit (algorithmic GB/s).

    Main figure: a PyTorch CPU grouped conv1d in fp32 (oracle/torch_cpu.py), forward + autograd
    backward of the full workload (B=4 T=8192 D=1024 W=4, bias + silu) on all host threads, repeated
    for about `seconds` seconds; inputs are cast and transposed before the timed loop. Beside it, the
    single-threaded C oracle (oracle/ccv1d_oracle.c) on one batch row for about seconds / 2."""
    sys.path.insert(0, os.path.join(_ROOT, "oracle"))
    import numpy as np

    import ccv1d_oracle
    import torch_cpu

    torch.set_num_threads(os.cpu_count() or 1)
    B, T, D, W = 4, 8192, 1024, 4
    g = torch.Generator().manual_seed(0)
    xb = torch.randn(B, T, D, generator=g).to(torch.bfloat16)
    w = torch.randn(D, W, generator=g) / 2
    b = torch.randn(D, generator=g)
    dyb = torch.randn(B, T, D, generator=g).to(torch.bfloat16)
    x, wt, bb, dy = torch_cpu.prepare(xb, w, b, dyb)
    reps, el = _timed_reps(lambda: torch_cpu.fwd_bwd(x, wt, bb, dy, True), seconds)
    fwd_b, bwd_b = alg_bytes(B, T, D, W)
    out = {
        "value": round((fwd_b + bwd_b) * reps / el / 1e9, 3),
        "unit": "GB/s",
        "cores": torch.get_num_threads(),
        "kind": "port",
        "sample": f"oracle/torch_cpu.py (torch F.conv1d groups=D, fp32, autograd) fwd+bwd of the "
                  f"full workload, {reps} reps in {el:.1f} s, ms_per_step={el / reps * 1e3:.1f}",
        "host_cpus": os.cpu_count(),
    }
    B1 = 1
    rng = np.random.default_rng(0)
    x1 = rng.standard_normal((B1, T, D), dtype=np.float32)
    w1 = (rng.standard_normal((D, W), dtype=np.float32) / 2).astype(np.float32)
    b1 = rng.standard_normal(D, dtype=np.float32)
    dy1 = rng.standard_normal((B1, T, D), dtype=np.float32)

    def c_step():
        ccv1d_oracle.fwd(x1, w1, b1, silu=True)
        ccv1d_oracle.bwd(x1, w1, dy1, b1, silu=True)

    reps1, el1 = _timed_reps(c_step, seconds / 2)
    fb1, bb1 = alg_bytes(B1, T, D, W)
    out["c_oracle"] = {
        "value": round((fb1 + bb1) * reps1 / el1 / 1e9, 3), "unit": "GB/s", "cores": 1,
        "sample": f"oracle/ccv1d_oracle.c fwd+bwd, B=1 T=8192 D=1024 W=4 bias+silu (1/4 of the "
                  f"workload), {reps1} reps in {el1:.1f} s"}
    return out


def _alg_bytes_general(B, T, D, W, bias, init=False, seq=False, final=False, ex=2, ew=4, eb=4,
                       ei=2):
    """Algorithmic HBM bytes of a forward and of a backward pass with the optional tensors: weights
    and bias read once per pass, dweight/dbias written once; initial states read (and their gradient
    written), final states written, seq_idx read in each pass."""
    n = B * T * D
    st = B * (W - 1) * D
    fwd = n * 2 * ex + D * W * ew + (D * eb if bias else 0) + (st * ei if init else 0)
    fwd += (st * ex if final else 0) + (B * T * 4 if seq else 0)
    bwd = n * 3 * ex + 2 * D * W * ew + (2 * D * eb if bias else 0)
    bwd += (2 * st * ei if init else 0) + (B * T * 4 if seq else 0)
    return fwd, bwd


def run_configs(dev, widths=False, only=None, shapes=False, x_dtype=torch.bfloat16):
    """One JSON line per BASELINE configuration 2-5 (the reference's README sweep, the Mamba-2 xBC
    shape, chunked streaming and decode with state handoff, packed varlen seq_idx): device time per
    call from replayed graphs after the usual warm-up, plus, for the latency-bound streaming and
    decode calls, the host-inclusive eager time per call. With `widths`, instead: the benchmark
    shape (bf16, bias + silu) at every width the vectorised kernels cover, forward alone and
    forward + backward (widths 2-8, 9, 12, 16, 17, 20, 24 and 32). With `shapes`, instead: the
    same two passes over mid-size shapes (many batch rows or short sequences, where the tiling's
    choice of tile length matters) at widths 2-9, 12, 16 and 24.

    `only` (a set of strings, e.g. {"2:512", "5:7"} or, with `widths`, {"8"}) restricts the run to
    the named configurations (N, or N:T for configuration 2's lengths, N:W for configuration 5's
    widths) or widths, so that a profiler run covers one workload. `x_dtype` is the dtype of x and of
    the upstream gradient in configuration 2 (bf16 by default, as BASELINE.json states it); the
    other configurations keep bf16."""
    def want(cfg, sub=None):
        return not only or str(cfg) in only or (sub is not None and f"{cfg}:{sub}" in only)

    from causal_conv1d_triton import causal_conv1d_fn

    side = torch.cuda.Stream()
    gen = torch.Generator(device=dev).manual_seed(0)

    def emit(name, shape, us, fb, bb, kind, extra=None):
        line = {"config": name, "shape": shape, "pass": kind, "latency_us": round(us, 2)}
        nbytes = fb if kind == "fwd" else bb if kind == "bwd" else fb + bb
        if nbytes:
            line["gbs"] = round(nbytes / (us * 1e-6) / 1e9, 1)
            line["frac_of_peak"] = round(nbytes / (us * 1e-6) / 1e9 / PEAK_GBS, 4)
        if extra:
            line.update(extra)
        print(json.dumps(line), flush=True)

    def timed(graph_calls):
        # graph_calls: (graph, calls per replay); device time per call in us
        graph, per_replay = graph_calls
        _warm(graph, 2)
        reps = 20
        return _time_graphs([graph] * reps) / (reps * per_replay) * 1e3

    def looped(one_pass, n):
        # One graph that runs one_pass (n calls over the input sets) enough times to hold about
        # CONFIG_GRAPH_CALLS calls, so the idle gap between two graph replays (the next graph's
        # launch, about 3.6 us) weighs little on the time per call. Returns (graph, calls).
        rounds = max(1, CONFIG_GRAPH_CALLS // n)
        return _capture(lambda: [one_pass() for _ in range(rounds)], side), rounds * n

    def steps(sets, w, b, act, init=None, seq=None, xs=None):
        res = []

        def one_pass():
            for i, (x, dy) in enumerate(sets):
                xi = x if xs is None else xs[i]
                out = causal_conv1d_fn(xi, w, b, seq_idx=seq, initial_states=init, activation=act)
                grads = [t for t in (xi, w, b, init) if t is not None and t.requires_grad]
                res.append(torch.autograd.grad(out, grads, dy))
                del res[:-len(sets)]  # the last pass's gradients stay allocated
        gc = looped(one_pass, len(sets))
        res.clear()
        return gc

    def fwds(sets, w, b, act, op=None):
        # Forward alone, as inference calls it: causal_conv1d_fn with autograd off. With `op`
        # (a one-argument function of x), that function instead, under the same rotation.
        res = []

        def one_pass():
            with torch.no_grad():
                for x, _ in sets:
                    res.append(causal_conv1d_fn(x, w, b, activation=act) if op is None else op(x))
                    del res[:-len(sets)]
        gc = looped(one_pass, len(sets))
        res.clear()
        return gc

    if widths:
        B, T, D = 4, 8192, 1024
        sets = [(torch.randn(B, T, D, generator=gen, device=dev).to(torch.bfloat16)
                 .requires_grad_(True),
                 torch.randn(B, T, D, generator=gen, device=dev).to(torch.bfloat16))
                for _ in range(4)]
        b = torch.randn(D, generator=gen, device=dev).requires_grad_(True)
        for W in (2, 3, 4, 5, 6, 7, 8, 9, 12, 16, 17, 20, 24, 32):
            if only and str(W) not in only:
                continue
            w = (torch.randn(D, W, generator=gen, device=dev) / math.sqrt(W)).requires_grad_(True)
            fb, bb = _alg_bytes_general(B, T, D, W, True)
            shape = f"B={B} T={T} D={D} W={W} bias_silu"
            emit("widths", shape, timed(fwds(sets, w, b, "silu")), fb, bb, "fwd")
            emit("widths", shape, timed(steps(sets, w, b, "silu")), fb, bb, "fwd+bwd")
        return

    if shapes:
        for B, T, D in ((16, 2048, 2048), (32, 1024, 2048), (8, 1024, 4096), (64, 512, 2048),
                        (8, 4096, 4096), (2, 8192, 2048), (16, 512, 4096), (48, 1024, 1024),
                        (24, 1024, 3072), (4, 1024, 8192), (12, 2048, 2560), (6, 2048, 4096),
                        (8, 4096, 3072)):
            nsets = max(2, min(4, (512 << 20) // (B * T * D * 2)))
            sets = [(torch.randn(B, T, D, generator=gen, device=dev).to(torch.bfloat16)
                     .requires_grad_(True),
                     torch.randn(B, T, D, generator=gen, device=dev).to(torch.bfloat16))
                    for _ in range(nsets)]
            b = torch.randn(D, generator=gen, device=dev).requires_grad_(True)
            for W in (2, 3, 4, 5, 6, 7, 8, 9, 12, 16, 24):
                if only and str(W) not in only:
                    continue
                w = (torch.randn(D, W, generator=gen, device=dev) / math.sqrt(W)).requires_grad_(True)
                fb, bb = _alg_bytes_general(B, T, D, W, True)
                shape = f"B={B} T={T} D={D} W={W} bias_silu"
                emit("shapes", shape, timed(fwds(sets, w, b, "silu")), fb, bb, "fwd")
                emit("shapes", shape, timed(steps(sets, w, b, "silu")), fb, bb, "fwd+bwd")
            del sets
        return

    dt_tag = "" if x_dtype == torch.bfloat16 else " " + str(x_dtype).replace("torch.", "")
    # Configuration 2: README shape sweep, B=4 D=1024 W=4, weight only or bias + silu.
    for T in (512, 2048, 8192, 32768):
        if not want(2, T):
            continue
        B, D, W = 4, 1024, 4
        ex = torch.tensor([], dtype=x_dtype).element_size()
        nsets = max(2, min(8, (512 << 20) // (2 * B * T * D * ex)))
        nfwd = max(2, min(16, (512 << 20) // (B * T * D * ex)))
        sets = [(torch.randn(B, T, D, generator=gen, device=dev).to(x_dtype)
                 .requires_grad_(True),
                 torch.randn(B, T, D, generator=gen, device=dev).to(x_dtype))
                for _ in range(nsets)]
        w = (torch.randn(D, W, generator=gen, device=dev) / 2).requires_grad_(True)
        for variant in ("weight_only", "bias_silu"):
            bias = variant == "bias_silu"
            b = torch.randn(D, generator=gen, device=dev).requires_grad_(True) if bias else None
            act = "silu" if bias else None
            fb, bb = _alg_bytes_general(B, T, D, W, bias, ex=ex)
            shape = f"B={B} T={T} D={D} W={W} {variant}{dt_tag}"
            # forward alone over at least 512 MiB of x, twice the Infinity Cache
            fsets = sets + [(torch.randn(B, T, D, generator=gen, device=dev).to(x_dtype),
                             None) for _ in range(max(0, nfwd - nsets))]
            emit("2", shape, timed(fwds(fsets, w, b, act)), fb, bb, "fwd")
            if bias:
                # The copy ceiling of the forward alone: torch's clone of the same x under the same
                # rotation (reads and writes the forward's activation bytes, nothing else).
                emit("2", f"B={B} T={T} D={D}{dt_tag} torch clone of x", timed(fwds(fsets, w, b, act,
                     op=torch.clone)), 2 * B * T * D * ex, 0, "fwd", {"reference": "copy"})
            del fsets
            emit("2", shape, timed(steps(sets, w, b, act)), fb, bb, "fwd+bwd")
        del sets
    if want(3):
        run_config3(dev, gen, emit, timed, steps, looped)
    if want(4):
        run_config4(dev, gen, emit, timed, side)
    if any(want(5, W) for W in (4, 7)):
        run_config5(dev, gen, emit, timed, steps, [W for W in (4, 7) if want(5, W)])


def run_config3(dev, gen, emit, timed, steps, looped):
    """Configuration 3: Mamba-2 2.7B xBC, x a channel slice of an in_proj output."""
    B, T, D, W = 8, 4096, 5376, 4
    bigs = [torch.randn(B, T, 10576, generator=gen, device=dev).to(torch.bfloat16) for _ in range(2)]
    xs = [bg[..., 5120:5120 + D].detach().requires_grad_(True) for bg in bigs]
    sets = [(x, torch.randn(B, T, D, generator=gen, device=dev).to(torch.bfloat16)) for x in xs]
    w = (torch.rand(D, W, generator=gen, device=dev) - 0.5).requires_grad_(True)
    b = ((torch.rand(D, generator=gen, device=dev) - 0.5) * 0.2).requires_grad_(True)
    fb, bb = _alg_bytes_general(B, T, D, W, True)
    emit("3", f"B={B} T={T} D={D} W={W} x=slice(in_proj, stride 10576)",
         timed(steps(sets, w, b, "silu", xs=xs)), fb, bb, "fwd+bwd")
    # The backward's dx into the gradient of the in_proj output: written in place through the
    # strided-dx entry point, against a contiguous dx copied into its slice afterwards (what
    # assembling that gradient from the slices' gradients costs).
    from causal_conv1d_triton.causal_conv1d import _bwd
    from causal_conv1d_triton.fused import causal_conv1d_bwd

    grads = [torch.empty(B, T, 10576, dtype=torch.bfloat16, device=dev) for _ in range(2)]
    wd, bd = w.detach(), b.detach()

    def copied():
        for (x, dy), gz in zip(sets, grads):
            dx = _bwd(x.detach(), wd, bd, None, None, dy, None, False, True)[0]
            gz[..., 5120:5120 + D].copy_(dx)

    def in_place():
        for (x, dy), gz in zip(sets, grads):
            causal_conv1d_bwd(x.detach(), wd, bd, dy, dx=gz[..., 5120:5120 + D], activation="silu")

    saved = 2 * B * T * D * 2
    emit("3", f"B={B} T={T} D={D} W={W} backward, dx copied into the in_proj gradient", 
         timed(looped(copied, 2)), 0, bb + saved, "bwd",
         {"alg_bytes": bb + saved})
    emit("3", f"B={B} T={T} D={D} W={W} backward, dx written into the in_proj gradient",
         timed(looped(in_place, 2)), 0, bb, "bwd",
         {"alg_bytes": bb, "bytes_saved_per_step": saved})
    del grads

    # The same backward with a contiguous dx (no copy), and in place into a gradient whose rows
    # are padded to 10624 channels (a pitch of 21248 bytes, a multiple of the 128-byte line,
    # where Mamba's 10576 channels leave rows 32 bytes past one).
    def contiguous():
        for x, dy in sets:
            _bwd(x.detach(), wd, bd, None, None, dy, None, False, True)

    emit("3", f"B={B} T={T} D={D} W={W} backward, contiguous dx", timed(looped(contiguous, 2)),
         0, bb, "bwd", {"alg_bytes": bb})
    padded = [torch.empty(B, T, 10624, dtype=torch.bfloat16, device=dev) for _ in range(2)]

    def in_place_padded():
        for (x, dy), gz in zip(sets, padded):
            causal_conv1d_bwd(x.detach(), wd, bd, dy, dx=gz[..., 5120:5120 + D], activation="silu")

    emit("3", f"B={B} T={T} D={D} W={W} backward, dx written into a gradient of 10624 channels",
         timed(looped(in_place_padded, 2)), 0, bb, "bwd", {"alg_bytes": bb})
    del bigs, xs, sets, padded


def run_config4(dev, gen, emit, timed, side):
    """Configuration 4: streaming, B=16 D=2048 W=4, T=8192 as 32 chunks of 256 with state
    handoff, and decode steps of T=1."""
    from causal_conv1d_triton import causal_conv1d_fn

    B, T, D, W = 16, 8192, 2048, 4
    x = torch.randn(B, T, D, generator=gen, device=dev).to(torch.bfloat16)
    w = torch.randn(D, W, generator=gen, device=dev) / 2
    b = torch.randn(D, generator=gen, device=dev)
    for name, chunk, n in (("chunk", 256, 32), ("decode", 1, 64)):
        def stream_fn():
            state = None
            for c in range(n):
                _, state = causal_conv1d_fn(x[:, c * chunk:(c + 1) * chunk], w, b,
                                            initial_states=state, return_final_states=True,
                                            activation="silu")
        with torch.no_grad():
            g = _capture(stream_fn, side)
            dev_us = timed((g, n))
            for _ in range(3):
                stream_fn()
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            reps = 20
            for _ in range(reps):
                stream_fn()
            torch.cuda.synchronize()
            host_us = (time.perf_counter() - t0) * 1e6 / (reps * n)
        fb, _ = _alg_bytes_general(B, chunk, D, W, True, init=True, final=True)
        emit("4", f"B={B} D={D} W={W} {name} T={chunk} x{n}, state handoff", dev_us, fb, 0, "fwd",
             {"eager_us_per_call": round(host_us, 2)})
    del x


def run_config5(dev, gen, emit, timed, steps, widths):
    """Configuration 5: packed varlen seq_idx, B=4 T=16384 D=4096, W in {4, 7}, initial
    states."""
    B, T, D = 4, 16384, 4096
    seq = torch.empty(B, T, dtype=torch.int32)
    gs = torch.Generator().manual_seed(5)
    for bb_ in range(B):
        t, sid = 0, 0
        while t < T:
            n = int(torch.randint(64, 4097, (1,), generator=gs))
            seq[bb_, t:t + n] = sid
            t, sid = t + n, sid + 1
        seq[bb_, T - int(0.05 * T):] = -1
    seq = seq.to(dev)
    for W in widths:
        sets = [(torch.randn(B, T, D, generator=gen, device=dev).to(torch.bfloat16)
                 .requires_grad_(True),
                 torch.randn(B, T, D, generator=gen, device=dev).to(torch.bfloat16))
                for _ in range(2)]
        w = (torch.randn(D, W, generator=gen, device=dev) / math.sqrt(W)).requires_grad_(True)
        b = torch.randn(D, generator=gen, device=dev).requires_grad_(True)
        init = torch.randn(B, W - 1, D, generator=gen, device=dev).to(torch.bfloat16)
        init.requires_grad_(True)
        fb, bb = _alg_bytes_general(B, T, D, W, True, init=True, seq=True)
        emit("5", f"B={B} T={T} D={D} W={W} seq_idx varlen, initial_states",
             timed(steps(sets, w, b, "silu", init=init, seq=seq)), fb, bb, "fwd+bwd")
        del sets


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=1000)
    ap.add_argument("--warmup", type=int, default=200)
    ap.add_argument("--sets", type=int, default=4)
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--isolated", action="store_true",
                    help="also time each pass alone (graphs of one pass per input set)")
    ap.add_argument("--configs", action="store_true",
                    help="instead of the headline line, one JSON line per BASELINE configuration 2-5")
    ap.add_argument("--widths", action="store_true",
                    help="instead of the headline line, the benchmark shape at widths 2-32")
    ap.add_argument("--shapes", action="store_true",
                    help="instead of the headline line, mid-size shapes at widths 2-24")
    ap.add_argument("--only", default="",
                    help="with --configs, --widths or --shapes: comma-separated workloads to run "
                         "(e.g. 2:512,5:7 or, with --widths or --shapes, widths such as 8)")
    ap.add_argument("--x-dtype", choices=("bf16", "fp16", "fp32"), default="bf16",
                    help="with --configs: dtype of x and the upstream gradient in configuration 2")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="also run plain copies of known size (for rocprofv3 --pmc scaling)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py: this build measures one GPU; the op needs no collective (batch or "
              "channel shards run the same kernels independently). Run with --gpus 1.",
              file=sys.stderr)
        sys.exit(2)

    from causal_conv1d_triton import causal_conv1d_fn
    from causal_conv1d_triton.causal_conv1d import _bwd, _fwd

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    if args.configs or args.widths or args.shapes:
        run_configs(dev, widths=args.widths, shapes=args.shapes,
                    x_dtype={"bf16": torch.bfloat16, "fp16": torch.float16,
                             "fp32": torch.float32}[args.x_dtype],
                    only={t for t in args.only.split(",") if t} or None)
        return
    B, T, D, W = 4, 8192, 1024, 4
    gen = torch.Generator(device=dev).manual_seed(0)
    w = (torch.randn(D, W, generator=gen, device=dev) / 2).requires_grad_(True)
    b = torch.randn(D, generator=gen, device=dev).requires_grad_(True)
    sets = []
    for _ in range(args.sets):
        x = torch.randn(B, T, D, generator=gen, device=dev).to(torch.bfloat16).requires_grad_(True)
        dy = torch.randn(B, T, D, generator=gen, device=dev).to(torch.bfloat16)
        sets.append((x, dy))
    torch.cuda.synchronize()
    if args.calibrate_copy:
        calibrate_copy(dev)

    def step(i):
        x, dy = sets[i]
        out = causal_conv1d_fn(x, w, b, activation="silu")
        return torch.autograd.grad(out, (x, w, b), dy)

    # The timed steps are replays of one graph of up to GRAPH_STEPS steps (the input sets in
    # rotation), plus one graph for the remainder, so exactly args.steps steps are timed. Between
    # two graph replays the device idles for the launch of the next one, about 3.6 us (same box:
    # 59.9 us per step with 4 steps per graph, 59.0 with 16, 58.75 with 64): a cost of the harness,
    # not of the op, which inside a model's graph runs between other kernels. The outputs of the
    # last len(sets) steps stay allocated, so the steps rotate over len(sets) + 1 sets of output
    # buffers, as when each graph held one step per input set.
    side = torch.cuda.Stream()
    results = []

    def run(n):
        keep = []
        for i in range(n):
            keep.append(step(i % args.sets))
            if len(keep) > args.sets:
                keep.pop(0)
        results[:] = keep

    g_steps = min(args.steps, GRAPH_STEPS)
    main_graph = _capture(lambda: run(g_steps), side)
    rem = args.steps % g_steps
    seq = [main_graph] * (args.steps // g_steps)
    if rem:
        seq.append(_capture(lambda: run(rem), side))
    results.clear()
    warm_steps = _warm(main_graph, -(-args.warmup // g_steps)) * g_steps
    ms_step = _time_graphs(seq) / args.steps

    # Per-pass device time inside the step (events between the passes of eager steps).
    ms_pass = passes_in_step(sets, w, b, args.steps)
    ms_fwd, ms_bwd = ms_pass["fwd"], ms_pass["bwd"]

    isolated = None
    if args.isolated:
        # Each pass captured on its own and replayed back to back (the other pass does not run, so
        # neither finds the other's data in the Infinity Cache).
        fwd_graph = _capture(lambda: [_fwd(x.detach(), w.detach(), b.detach(), None, None, None,
                                           True) for x, _ in sets], side)
        bwd_graph = _capture(lambda: [_bwd(x.detach(), w.detach(), b.detach(), None, None, dy,
                                           None, False, True) for x, dy in sets], side)
        reps = max(1, args.steps // args.sets)
        _warm(fwd_graph, 2)
        iso_fwd = _time_graphs([fwd_graph] * reps) / (reps * args.sets)
        _warm(bwd_graph, 2)
        iso_bwd = _time_graphs([bwd_graph] * reps) / (reps * args.sets)
        isolated = {"fwd": round(iso_fwd * 1e3, 2), "bwd": round(iso_bwd * 1e3, 2)}

    fwd_b, bwd_b = alg_bytes(B, T, D, W)
    bk_b = bwd_kernel_alg_bytes(B, T, D, W)
    gbs = (fwd_b + bwd_b) / (ms_step * 1e-3) / 1e9
    bwd_gbs = bwd_b / (ms_bwd * 1e-3) / 1e9
    ms_bk = ms_pass["bwd_kernel"]
    bk_gbs = bk_b / (ms_bk * 1e-3) / 1e9
    tr = traffic_from_profiles()
    bk_traffic = None
    if tr is not None:
        k = tr["per_kernel_bytes"]["bwd_fast_kernel"]
        bk_traffic = k["read"] + k["write"]
    line = {
        "metric": METRIC,
        "value": round(gbs, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "warmup_steps_run": warm_steps,
        "ms_per_step": round(ms_step, 5),
        "latency_us": round(ms_step * 1e3, 2),
        "frac_of_peak": round(gbs / PEAK_GBS, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {
            "workload": "causal_conv1d_fn fwd+bwd, bias+silu (BASELINE configs[1] at T=8192)",
            "batch": B, "seqlen": T, "dim": D, "width": W,
            "x_dtype": "bf16", "weight_dtype": "fp32", "input_sets": args.sets,
            "timing": f"hip graphs of {min(args.steps, GRAPH_STEPS)} steps (the input sets in "
                      "rotation), replayed; events around the timed replays",
        },
        "passes_in_step_us": {"fwd": round(ms_fwd * 1e3, 2), "bwd": round(ms_bwd * 1e3, 2)},
        "passes_in_step_gbs": {"fwd": round(fwd_b / (ms_fwd * 1e-3) / 1e9, 1),
                               "bwd": round(bwd_gbs, 1)},
        "kernels_in_step_us": {"fwd_fast_kernel": round(ms_pass["fwd_kernel"] * 1e3, 2),
                               "bwd_fast_kernel": round(ms_bk * 1e3, 2)},
        "eager_step_us": round(ms_pass["step"] * 1e3, 2),
        "passes_isolated_us": isolated,
        "roofline": {
            "kernel": "bwd_fast_kernel (the backward pass's main kernel; reduce_partials_kernel "
                      "then sums its partials into dweight/dbias)",
            "measured": "events set by HIP from the kernel dispatch's own start and end timestamps "
                        "(ccv1d_time_main_kernel, hipExtLaunchKernel) on every 4th of "
                        f"{args.steps} eager fwd+bwd steps queued back to back (mean)",
            "launch_us": round(ms_bk * 1e3, 2),
            "bound": "hbm",
            "achieved": round(bk_gbs, 1),
            "peak": PEAK_GBS,
            "unit": "GB/s",
            "frac": round(bk_gbs / PEAK_GBS, 4),
            "traffic": bk_traffic,
            "traffic_source": None if tr is None else tr["source"],
            "alg_bytes": bk_b,
            "pass": {"launches": "bwd_fast_kernel + reduce_partials_kernel",
                     "us": round(ms_bwd * 1e3, 2), "alg_bytes": bwd_b,
                     "achieved": round(bwd_gbs, 1), "frac": round(bwd_gbs / PEAK_GBS, 4),
                     "traffic": None if tr is None else tr["bwd_pass_bytes"]},
        },
        "cpu_baseline": None if args.no_cpu_baseline else cpu_baseline(args.cpu_seconds),
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
