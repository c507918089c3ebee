"""Pins the C oracle (oracle/ccv1d_oracle.c) before it is trusted as the GPU checker: float64
closed forms (grouped F.conv1d and its autograd), the shifted-sum form with sequence masks,
per-element brute force, committed known-answer vectors, textbook special cases and bit-exact
invariants (state handoff, padding, seq special cases). CPU only."""

import pytest

import pins

WIDTHS = [2, 3, 4, 5, 7, 9]


def _lengths(W):
    P = W - 1
    return sorted({1, max(1, P - 1), P, P + 1, 17, 120})


@pytest.mark.parametrize("W", WIDTHS)
@pytest.mark.parametrize("variant", ["plain", "bias_silu", "init_bias_silu", "init_dfinal_noact"])
def test_fwd_bwd_vs_closed_form(W, variant):
    for T in _lengths(W):
        c = pins.make_case(
            seed=100 * W + T, B=2, T=T, D=7, W=W,
            bias=variant != "plain",
            init="init" in variant,
            dfinal="dfinal" in variant,
            silu="silu" in variant,
        )
        ok, det = pins.check_fwd_closed_form(c)
        assert ok, f"T={T}: {det}"
        ok, det = pins.check_bwd_autograd(c)
        assert ok, f"T={T}: {det}"


@pytest.mark.parametrize("W", [2, 4, 7])
@pytest.mark.parametrize("seq", ["segments", "padded"])
@pytest.mark.parametrize("init", [False, True])
def test_seq_vs_shifted_form(W, seq, init):
    for T in (1, W, 33, 200):
        c = pins.make_case(seed=7 * W + T, B=3, T=T, D=5, W=W, init=init, seq=seq, silu=True)
        ok, det = pins.check_fwd_shifted(c)
        assert ok, f"T={T}: {det}"
        ok, det = pins.check_bwd_autograd(c)
        assert ok, f"T={T}: {det}"


@pytest.mark.parametrize("W", [2, 3, 4, 6])
@pytest.mark.parametrize("seq", [None, "padded"])
@pytest.mark.parametrize("silu", [False, True])
def test_brute_force_tiny(W, seq, silu):
    for T in (1, W - 1, W + 2, 9):
        T = max(T, 1)
        c = pins.make_case(seed=31 * W + T, B=2, T=T, D=3, W=W, init=True, seq=seq,
                           dfinal=seq is None, silu=silu)
        ok, det = pins.check_brute(c)
        assert ok, f"T={T}: {det}"


@pytest.mark.parametrize("k", pins.kat_cases(), ids=lambda k: k["name"])
def test_known_answers(k):
    ok, det = pins.check_kat(k)
    assert ok, det


@pytest.mark.parametrize("W", [2, 4, 5])
@pytest.mark.parametrize("silu", [False, True])
def test_seq_special_cases(W, silu):
    c = pins.make_case(seed=W, B=2, T=50, D=6, W=W, init=True, silu=silu)
    ok, det = pins.check_seq_special(c)
    assert ok, det


@pytest.mark.parametrize("W", [2, 4, 9])
@pytest.mark.parametrize("init", [False, True])
def test_state_handoff(W, init):
    for T, split in ((40, 17), (40, 1), (W - 1, 1), (2 * W, W)):
        if split >= T:
            continue
        c = pins.make_case(seed=T + W, B=2, T=T, D=5, W=W, init=init, silu=True)
        ok, det = pins.check_state_handoff(c, split)
        assert ok, f"T={T} split={split}: {det}"


@pytest.mark.parametrize("W", [2, 4, 7])
def test_textbook_without_activation(W):
    c = pins.make_case(seed=W, B=3, T=64, D=9, W=W, init=True, dfinal=True, silu=False)
    ok, det = pins.check_textbook_no_act(c)
    assert ok, det


@pytest.mark.parametrize("silu", [False, True])
@pytest.mark.parametrize("bias", [False, True])
def test_torch_cpu_baseline_matches_oracle(silu, bias):
    """The benchmark's CPU baseline (oracle/torch_cpu.py, fp32 grouped conv1d + autograd) computes
    the same forward and gradients as the C oracle."""
    import numpy as np

    import torch_cpu

    c = pins.make_case(seed=11, B=2, T=75, D=9, W=4, bias=bias, silu=silu)
    x, wt, b, dy = torch_cpu.prepare(c["x"], c["w"], c["b"], c["dout"])
    out, grads = torch_cpu.fwd_bwd(x, wt, b, dy, silu)
    ref_out, _ = pins.oracle_fwd(c)
    dx, _, dw, db = pins.oracle_bwd(c)
    np.testing.assert_allclose(out.detach().transpose(1, 2).numpy(), ref_out, rtol=1e-5, atol=1e-5)
    np.testing.assert_allclose(grads[0].transpose(1, 2).numpy(), dx, rtol=1e-5, atol=1e-5)
    np.testing.assert_allclose(grads[1][:, 0, :].numpy(), dw, rtol=1e-5, atol=1e-4)
    if bias:
        np.testing.assert_allclose(grads[2].numpy(), db, rtol=1e-5, atol=1e-4)


@pytest.mark.parametrize("W", [129, 200, 257])
def test_wide_widths_vs_closed_form(W):
    """Widths above 128 (the reference allows any width >= 2, README.md:40): the oracle against the
    float64 grouped F.conv1d closed form and its autograd, at lengths around the window."""
    for T in (1, W - 1, W + 1, 300):
        c = pins.make_case(seed=W + T, B=2, T=T, D=3, W=W, init=True, dfinal=True, silu=True)
        ok, det = pins.check_fwd_closed_form(c)
        assert ok, f"T={T}: {det}"
        ok, det = pins.check_bwd_autograd(c)
        assert ok, f"T={T}: {det}"


@pytest.mark.parametrize("init", [False, True])
def test_wide_width_seq_vs_shifted_form(init):
    """seq_idx at width 200 against the shifted-sum form with sequence masks."""
    W = 200
    for T in (W - 1, 450):
        c = pins.make_case(seed=T, B=2, T=T, D=3, W=W, init=init, seq="padded", silu=True)
        ok, det = pins.check_fwd_shifted(c)
        assert ok, f"T={T}: {det}"
        ok, det = pins.check_bwd_autograd(c)
        assert ok, f"T={T}: {det}"
