"""Register and scratch budgets of the built kernels, read from the library's own gfx950 code objects.

The vectorised tilings aim for 4096 waves (kTargetWaves in ccv1d_api.hip: 4 per SIMD on 256 CUs),
so a kernel that holds fewer than 4 waves per SIMD runs such a grid in two rounds: a change that
adds registers without changing any result can cost a step several microseconds (a tail variant
of the 2-channel backward took W=8 from 100 to 147 VGPRs, 3 waves per SIMD, step +4.6 us). These
tests read the AMDGPU metadata (VGPRs, spills, scratch bytes per lane) of every kernel of the
objects under causal-conv1d-triton_amd/_build, built here from this repository's sources, and
check:

* no kernel uses scratch memory (register spills), except the listed instances, whose few spilled
  registers are stored and reloaded once per wave outside the row loops;
* with 16-bit x and no seq_idx, every fwd_fast_kernel and every bwd_fast_kernel up to width 20
  fits 4 waves per SIMD (at most 128 VGPRs of the 512 a SIMD gives each lane); from width 21 the
  one-channel backward holds 3 or 2 by design (its dweight sums and windows of W taps);
* with fp32 x and no seq_idx, the forward at every width and the backward up to width 4 fit
  4 waves per SIMD.

The objects are built by `make -C causal-conv1d-triton_amd` (or `__graft_entry__.build()`); the
tests skip when they or the LLVM tools of the ROCm install are absent.
"""

import glob
import os
import re
import subprocess

import pytest

_ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
_BUILD = os.path.join(_ROOT, "causal-conv1d-triton_amd", "_build")
_LLVM = "/opt/rocm/llvm/bin"
_TARGET = "hipv4-amdgcn-amd-amdhsa--gfx950"

# (pass, x dtype code in the mangled name, width, seq_idx, channels per lane) -> max scratch bytes
# per lane. Measured on this build: one spilled pair of registers outside the row loops.
SCRATCH_ALLOWED = {
    ("fwd", "DF16b", 16, False, 2): 12,  # forward W=16, 2 channels: 128 VGPRs (4 waves per SIMD)
    ("bwd", "DF16_", 5, True, 4): 8,     # fp16 backward W=5 with seq_idx, 4 channels, 2-row batches
}

_FAST = re.compile(r"_ZN5ccv1d15(fwd|bwd)_fast_kernelI(DF16b|DF16_|f)Li(\d+)ELb([01])ELb([01])"
                   r"ELi(\d+)ELi(\d+)ELi(\d+)E")


def _tools_ok():
    return all(os.path.exists(os.path.join(_LLVM, t))
               for t in ("llvm-objcopy", "clang-offload-bundler", "llvm-readelf"))


def _kernels(tmp):
    """(object file, metadata dict) for every kernel of every built object."""
    objs = [o for o in sorted(glob.glob(os.path.join(_BUILD, "ccv1d_*.o")))
            if not os.path.basename(o).startswith("asan")]
    out = []
    for o in objs:
        fb = os.path.join(tmp, "fatbin.bin")
        co = os.path.join(tmp, "gfx950.co")
        r = subprocess.run([os.path.join(_LLVM, "llvm-objcopy"), "--dump-section",
                            f".hip_fatbin={fb}", o, os.devnull], capture_output=True)
        if r.returncode:
            continue  # a host-only object (the C ABI layer)
        subprocess.run([os.path.join(_LLVM, "clang-offload-bundler"), "--unbundle", "--type=o",
                        f"--input={fb}", f"--targets={_TARGET}", f"--output={co}"], check=True)
        notes = subprocess.run([os.path.join(_LLVM, "llvm-readelf"), "--notes", co],
                               capture_output=True, text=True, check=True).stdout
        for blk in notes.split("  - .agpr_count")[1:]:
            d = {}
            for k in ("name", "private_segment_fixed_size", "vgpr_count", "vgpr_spill_count"):
                m = re.search(r"\." + k + r":\s+(\S+)", blk)
                d[k] = m.group(1) if m else None
            out.append((os.path.basename(o), d))
    return out


@pytest.fixture(scope="module")
def kernels(tmp_path_factory):
    if not _tools_ok():
        pytest.skip("LLVM tools of the ROCm install not found")
    if not glob.glob(os.path.join(_BUILD, "ccv1d_*.o")):
        pytest.skip("library not built (make -C causal-conv1d-triton_amd)")
    ks = _kernels(str(tmp_path_factory.mktemp("codeobj")))
    if not ks:
        pytest.skip("no gfx950 code objects in the built objects")
    return ks


def _key(name):
    m = _FAST.match(name)
    if not m:
        return None
    kind, dt, w, _silu, seq, cpl, _nw, _r = m.groups()
    return kind, dt, int(w), seq == "1", int(cpl)


def _waves_per_simd(vgprs):
    # gfx950: 512 VGPRs per SIMD lane for wave64, allocated in granules of 8.
    return 512 // ((vgprs + 7) // 8 * 8)


def test_every_fast_instance_is_present(kernels):
    keys = {_key(d["name"]) for _, d in kernels} - {None}
    for kind in ("fwd", "bwd"):
        for dt in ("DF16b", "DF16_", "f"):
            widths = {k[2] for k in keys if k[0] == kind and k[1] == dt}
            assert widths == set(range(2, 33)), (kind, dt, sorted(widths))


def test_no_scratch_outside_the_listed_instances(kernels):
    bad = []
    for obj, d in kernels:
        scratch = int(d["private_segment_fixed_size"])
        if scratch == 0:
            continue
        k = _key(d["name"])
        allowed = SCRATCH_ALLOWED.get(k, 0) if k else 0
        if scratch > allowed:
            bad.append((obj, d["name"], scratch, d["vgpr_count"]))
    assert not bad, f"kernels using scratch (register spills): {bad}"


@pytest.mark.parametrize("dt", ["DF16b", "DF16_"])
def test_16bit_kernels_hold_four_waves_per_simd(kernels, dt):
    bad = []
    for _, d in kernels:
        k = _key(d["name"])
        if not k or k[1] != dt or k[3]:
            continue
        kind, _, w, _, cpl = k
        if kind == "bwd" and w > 20:
            continue
        v = int(d["vgpr_count"])
        if _waves_per_simd(v) < 4:
            bad.append((d["name"], v))
    assert not bad, f"below 4 waves per SIMD: {bad}"


def test_fp32_kernels_hold_four_waves_per_simd(kernels):
    bad = []
    for _, d in kernels:
        k = _key(d["name"])
        if not k or k[1] != "f" or k[3]:
            continue
        kind, _, w, _, _ = k
        if kind == "bwd" and w > 4:
            continue
        v = int(d["vgpr_count"])
        if _waves_per_simd(v) < 4:
            bad.append((d["name"], v))
    assert not bad, f"below 4 waves per SIMD: {bad}"


def test_waves_per_simd_formula():
    assert _waves_per_simd(128) == 4
    assert _waves_per_simd(129) == 3
    assert _waves_per_simd(100) == 4
    assert _waves_per_simd(96) == 5
    assert _waves_per_simd(147) == 3
    assert _waves_per_simd(64) == 8
