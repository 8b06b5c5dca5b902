"""The oracle against the reference's own kernels.

tests/golden/kda_ref_fixtures.npz holds what the reference's chunked path
(/root/reference/src/kda_bt16/kernels.py, kda_bt16_debug: K1 and K2) computes
on nine small cases, run by Triton's CPU interpreter (the script beside the
fixture says how).  That interpreter rounds fp32 -> bf16 by truncation where
GPUs and NPUs round to nearest even, so the oracle is compared in its
truncating mode (``bf16_rounding("rtz")``): same rounding points, the
interpreter's rounding function.

Bars (per case; measured on the correct oracle: intermediates at most 0.32%
of elements off by at most 4 bf16 ulps, o at most 1.1% of elements not
bit-equal, ht within 2.2e-3 of max|ht|; the differences come from fp32
exp/sigmoid/summation order flipping a truncation):

* g (fp32 log2 gate cumsum): |diff| <= 1e-6 * max|g|;
* Aqk, A_inv, w, u: at most 1% of elements differ, by at most 4 bf16 ulps;
* o: at most 2% of elements differ from the reference's bits;
* ht: |diff| <= 5e-3 * max|ht|.

Mutation test: leaving out any one of the oracle's bf16 rounding points
(kernels.py:108-113, 153, 169-176, 261-291) breaks these bars on at least one
case, so each of them is pinned by the reference's own output.  The one point
not tested that way is the final rounding of o, which the bf16 output
dtype fixes.
"""

from __future__ import annotations

import pytest
import torch

from kda_oracle import ROUNDING_POINTS, bf16_rounding, chunked_reference, planted_mistake
from kda_testlib import load_ref_fixture, ref_fixture_cases, ulp_diff

CASES = ref_fixture_cases()


def _oracle(c) -> dict:
    o, ht, inter = chunked_reference(
        c["q"], c["k"], c["v"], c["g"], c["beta"], c["scale"], A_log=c["A_log"],
        dt_bias=c["dt_bias"], lower_bound=c["lower_bound"], initial_state=c["h0"],
        state_v_first=c["state_v_first"], use_gate=c["use_gate"], use_l2norm=c["use_l2norm"],
        use_beta_sigmoid=c["use_beta_sigmoid"])
    return dict(o=o, ht=ht, **inter)


def _violations(c, got) -> list[str]:
    """The bars this result breaks (empty when it meets them all)."""
    ref = c["ref"]
    bad = []
    dg = (got["g"] - ref["g"]).abs().max() / ref["g"].abs().max().clamp_min(1e-30)
    if dg > 1e-6:
        bad.append(f"g {dg:.2e}")
    for key in ("Aqk", "A_inv", "w", "u"):
        d = ulp_diff(got[key], ref[key])
        frac = (d > 0).float().mean().item()
        if frac > 0.01 or d.max().item() > 4:
            bad.append(f"{key} {frac:.4f} of elements off, max {d.max().item()} ulp")
    d = ulp_diff(got["o"], ref["o"])
    frac = (d > 0).float().mean().item()
    if frac > 0.02:
        bad.append(f"o {frac:.4f} of elements off")
    dh = (got["ht"] - ref["ht"]).abs().max() / ref["ht"].abs().max()
    if dh > 5e-3:
        bad.append(f"ht {dh:.2e}")
    return bad


@pytest.mark.parametrize("name", CASES)
def test_oracle_matches_reference_kernels(name):
    c = load_ref_fixture(name)
    with bf16_rounding("rtz"):
        got = _oracle(c)
    assert not _violations(c, got), f"{name}: {_violations(c, got)}"


def test_fixtures_cover_the_reference_flags():
    flags = {n: load_ref_fixture(n) for n in CASES}
    assert any(c["h0"] is not None for c in flags.values())
    assert any(not c["state_v_first"] for c in flags.values())
    assert any(not c["use_gate"] for c in flags.values())
    assert any(not c["use_l2norm"] and not c["use_beta_sigmoid"] for c in flags.values())
    assert any(c["lower_bound"] <= -10 for c in flags.values())
    Ts = {c["q"].shape[1] for c in flags.values()}
    assert 1 in Ts and 16 in Ts and any(t % 16 for t in Ts if t > 16)


@pytest.mark.parametrize("point", [p for p in ROUNDING_POINTS if p != "o"])
def test_each_rounding_point_is_pinned(point):
    """A planted mistake -- one rounding point left out -- must break the
    bars on at least one case."""
    broken = {}
    for name in CASES:
        c = load_ref_fixture(name)
        with bf16_rounding("rtz"), planted_mistake(point):
            bad = _violations(c, _oracle(c))
        if bad:
            broken[name] = bad
    assert broken, f"leaving out the rounding of {point} went unnoticed"


def test_rounding_modes():
    """bf16 keeps 7 fraction bits: near 1.0 one ulp is 2^-7."""
    from kda_oracle import _bf

    u = 2.0 ** -7
    x = torch.tensor([1 + u + u / 4, -(1 + u + u / 4), 1 + u / 2, 1 + 3 * u / 2])
    with bf16_rounding("rtz"):
        assert _bf(x).tolist() == [1 + u, -(1 + u), 1.0, 1 + u]
    # nearest, ties to the even neighbour
    assert _bf(x).tolist() == [1 + u, -(1 + u), 1.0, 1 + 2 * u]
