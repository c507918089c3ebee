"""Shows that the pinning checks in tests/pins.py bite: each plausible mistake planted in the oracle
(a dropped term, a wrong index, a wrong sign, a transposed operand, a missing mask, a state
off by one row, a missing gradient term) makes at least one check fail, while the unmodified oracle
passes them all. The mistakes are planted in the CPU oracle only."""

import pytest

import ccv1d_oracle as oracle
import pins

MUTATIONS = {
    1: "drop oldest tap",
    2: "tap index off by one",
    3: "silu derivative sign",
    4: "weight transposed",
    5: "dx kernel not flipped",
    6: "dx ignores sequence boundaries",
    7: "final states one row early",
    8: "dfinal dropped",
    9: "padding not zeroed",
    10: "initial-state rows lose their sequence id",
}


def _all_checks():
    results = []
    c = pins.make_case(seed=5, B=2, T=24, D=5, W=4, init=True, dfinal=True, silu=True)
    results.append(pins.check_fwd_closed_form(c)[0])
    results.append(pins.check_bwd_autograd(c)[0])
    results.append(pins.check_state_handoff(c, 9)[0])
    cs = pins.make_case(seed=6, B=2, T=30, D=5, W=4, init=True, seq="padded", silu=True)
    results.append(pins.check_fwd_shifted(cs)[0])
    results.append(pins.check_bwd_autograd(cs)[0])
    results.append(pins.check_seq_special(cs)[0])
    ct = pins.make_case(seed=7, B=1, T=6, D=2, W=3, init=True, seq="padded", silu=True)
    results.append(pins.check_brute(ct)[0])
    for k in pins.kat_cases():
        results.append(pins.check_kat(k)[0])
    return results


@pytest.fixture(autouse=True)
def _restore():
    yield
    oracle.set_mutation(0)


def test_unmodified_oracle_passes_every_check():
    oracle.set_mutation(0)
    assert all(_all_checks())


@pytest.mark.parametrize("m", sorted(MUTATIONS), ids=lambda m: MUTATIONS[m])
def test_planted_mistake_is_caught(m):
    oracle.set_mutation(m)
    assert not all(_all_checks()), f"mutation {m} ({MUTATIONS[m]}) passed every check"
