"""Pins of the grading rules in oracle/metrics.py (CPU).

``band`` restates megabench/harness/correctness.py:64-85 and ``integers_match`` the integer
rule of correctness.py:503-521. The checks here follow the reference's own tests of those
rules (megabench/tests/test_precision.py:131-187): the band accepts an alternative BF16
schedule of the same graph and the oracle rounded once to BF16, and rejects a x1.05 scale,
a one-element spike and NaN; an integer output may follow the BF16 reference or the oracle,
element by element, and nothing else.

Beside those, hand-computed vectors whose verdict follows from the rule's two inequalities,
each chosen so that a plausible mistake in ``band`` flips it: the reference and the oracle
swapped, the peak (max-abs) term dropped, the noise factor lost, the BF16 tolerance not
applied, the tolerance applied without regard to the reference's dtype.
"""

from __future__ import annotations

import dataclasses

import pytest
import torch

from oracle import layer, metrics
from vibe_megakernel_amd import cases as C
from vibe_megakernel_amd import workloads

BF16_STEP = 2.0 ** -7  # bf16 spacing in [1, 2)


def _vectors(n, ref_err, got_err):
    """exact fp32 ones; want = bf16(1 + ref_err); got = bf16(1 + got_err) (all exact in bf16)."""
    exact = torch.ones(n, dtype=torch.float32)
    want = torch.full((n,), 1.0 + ref_err, dtype=torch.bfloat16)
    got = torch.full((n,), 1.0 + got_err, dtype=torch.bfloat16)
    assert float(want[0]) == 1.0 + ref_err and float(got[0]) == 1.0 + got_err
    return want, got, exact


# -- closed forms -------------------------------------------------------------------------


def test_band_values_and_verdicts_follow_the_two_inequalities():
    # Uniform errors: relative L2 = max-abs = the per-element error (exact is all ones).
    d = BF16_STEP
    want, got, exact = _vectors(64, d, 3 * d)
    r = metrics.band(want, got, exact)
    assert r["relative_error"] == pytest.approx(3 * d, rel=1e-12)
    assert r["reference_relative_error"] == pytest.approx(d, rel=1e-12)
    assert r["max_abs_error"] == pytest.approx(3 * d, rel=1e-12)
    assert r["reference_max_abs_error"] == pytest.approx(d, rel=1e-12)
    # 3d = 0.0234375 <= 2d + 0.008 = 0.023625 on both terms: pass.
    assert r["pass"]
    # 4d = 0.03125 > 0.023625: fail.
    assert not metrics.band(*_vectors(64, d, 4 * d))["pass"]


def test_band_rejects_what_only_the_peak_term_sees():
    # One spike of 0.5 among 10000 elements: relative L2 ~0.0093 passes its bound
    # (2 * 0.0078 + 0.008), max-abs 0.5078 does not.
    d = BF16_STEP
    want, got, exact = _vectors(10000, d, d)
    got = got.clone()
    got[1234] = 1.0 + d + 0.5
    r = metrics.band(want, got, exact)
    assert r["relative_error"] <= 2 * r["reference_relative_error"] + 0.008
    assert not r["pass"]


def test_band_noise_factor_and_tolerance():
    d = 2.0 ** -4
    # got error 1.5d against a reference error d: within 2d (noise_factor 2), not within d + 0.008.
    want, got, exact = _vectors(32, d, 1.5 * d)
    assert metrics.band(want, got, exact)["pass"]
    assert not metrics.band(want, got, exact, noise_factor=1.0)["pass"]
    # A candidate error of 2d + 0.006 (fp32 candidate values) is within 2d + bf16_rtol, a
    # tolerance the rule grants only when the reference is bf16; rtol applies otherwise.
    exact = torch.ones(32, dtype=torch.float32)
    want_bf = torch.full((32,), 1.0 + d, dtype=torch.bfloat16)
    got = torch.full((32,), 1.0 + 2 * d + 0.006, dtype=torch.float32)
    assert metrics.band(want_bf, got, exact)["pass"]
    assert not metrics.band(want_bf.float(), got, exact)["pass"]      # fp32 reference: rtol 0
    assert metrics.band(want_bf.float(), got, exact, rtol=0.008)["pass"]
    assert not metrics.band(want_bf, got, exact, bf16_rtol=0.0)["pass"]


def test_band_rejects_non_finite_values():
    d = BF16_STEP
    want, got, exact = _vectors(16, d, d)
    assert metrics.band(want, got, exact)["pass"]
    for bad in (float("nan"), float("inf")):
        g = got.clone()
        g[3] = bad
        assert not metrics.band(want, g, exact)["pass"]
    assert not metrics.band(want, got * float("nan"), exact)["pass"]


# -- planted mistakes in the rule itself --------------------------------------------------


def _band_swapped(want, got, exact, **kw):
    return metrics.band(exact, got, want, **kw)


def _band_no_peak(want, got, exact, **kw):
    r = metrics.band(want, got, exact, **kw)
    return {**r, "pass": r["relative_error"] <= 2.0 * r["reference_relative_error"] + 0.008}


def _band_no_noise_factor(want, got, exact, **kw):
    return metrics.band(want, got, exact, noise_factor=1.0)


def test_planted_mistakes_in_band_are_caught():
    d = 2.0 ** -4
    # A candidate 2.5x as far from the oracle as the reference, and beyond the tolerance:
    # the rule fails it; with the reference and the oracle swapped it would pass.
    want, got, exact = _vectors(32, d, 2.5 * d)
    assert not metrics.band(want, got, exact)["pass"]
    assert _band_swapped(want, got, exact)["pass"]
    # The spike of test_band_rejects_what_only_the_peak_term_sees passes without the peak term.
    want, got, exact = _vectors(10000, BF16_STEP, BF16_STEP)
    got = got.clone()
    got[7] = 1.5 + BF16_STEP
    assert not metrics.band(want, got, exact)["pass"]
    assert _band_no_peak(want, got, exact)["pass"]
    # A candidate 1.5x as far as the reference passes the rule, not with the factor lost.
    want, got, exact = _vectors(32, d, 1.5 * d)
    assert metrics.band(want, got, exact)["pass"]
    assert not _band_no_noise_factor(want, got, exact)["pass"]


# -- the reference's acceptance and rejection cases, on the MoE layer ------------------------


@pytest.fixture(scope="module")
def tiny():
    case = C.case("moe-fp8-tiny-t4")
    out = []
    for seed in (3, 5, 7):
        values = workloads.make_inputs(case, seed, "cpu")
        want, exact = layer.reference(case, values), layer.oracle(case, values)
        out.append((case, values, want, exact))
    return out


def test_band_accepts_an_alternative_bf16_schedule(tiny):
    # test_precision.py:131-149: another BF16 schedule of the same graph differs in bits and
    # passes the band; so does the oracle's own output rounded once to bf16. The alternative
    # here is the reference's other SwiGLU rounding, silu rounded to bf16 before the product
    # (frontier.py:338 against :337): it changes most elements of y by an ulp or two.
    for case, values, want, exact in tiny:
        alt = layer.reference(dataclasses.replace(case, swiglu="bf16"), values)
        assert int((alt["y"] != want["y"]).sum()) > want["y"].numel() // 2
        assert metrics.band(want["y"], alt["y"], exact["y"])["pass"]
        assert metrics.band(want["y"], exact["y"].to(torch.bfloat16), exact["y"])["pass"]
        assert metrics.integers_match(alt["expert_ids"], want["expert_ids"], exact["expert_ids"])["pass"]


def test_band_rejects_errors_beyond_bf16_noise(tiny):
    # test_precision.py:151-167: scaled output, one corrupted element, non-finite.
    case, values, want, exact = tiny[0]
    y = want["y"]
    spike = y.clone()
    spike[0, 5] += float(y.float().abs().max())
    for label, bad in (("scaled", (y.float() * 1.05).to(torch.bfloat16)), ("one corrupted element", spike),
                       ("non-finite", y * float("nan"))):
        assert not metrics.band(y, bad, exact["y"])["pass"], label


def test_integer_outputs_follow_reference_or_oracle():
    # test_precision.py:169-187: each element may equal the reference or the oracle.
    routes = torch.tensor([[0, 1], [2, 3], [1, 0]])
    exact, want = routes, routes.clone()
    want[0, 1] = 2
    changed = routes.clone()
    changed[0, 1] = 2   # follows the reference
    changed[2, 1] = 0   # follows the oracle (unchanged)
    r = metrics.integers_match(changed, want, exact)
    assert r["pass"] and r["unmatched_elements"] == 0 and r["mismatched_elements"] == 0
    changed[1, 1] = 0   # follows neither
    r = metrics.integers_match(changed, want, exact)
    assert not r["pass"] and r["unmatched_elements"] == 1
    # A mix per element is allowed: reference at one element, oracle at another.
    mixed = want.clone()
    mixed[0, 1] = 1
    assert metrics.integers_match(mixed, want, exact)["pass"]
    # Planted mistake: requiring equality with the reference only rejects an oracle match.
    assert not torch.equal(mixed, want)
