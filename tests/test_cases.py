"""The case table, the byte/flop accounting and the seeded input generators (CPU only)."""

from __future__ import annotations

import json
import math
from pathlib import Path

import pytest
import torch

from oracle import formats
from vibe_megakernel_amd import cases as C
from vibe_megakernel_amd import workloads

BASELINE = json.loads((Path(__file__).resolve().parent.parent / "BASELINE.json").read_text())


def test_the_five_configs_are_the_baseline_configs():
    assert len(C.CASES) == len(BASELINE["configs"]) == 5
    want = [  # (T, H, E, K, I, shared, router) as each config line states them
        (4, 1024, 8, 2, 512, 0, "softmax"),
        (16, 4096, 8, 2, 14336, 0, "softmax"),
        (32, 2048, 128, 8, 768, 0, "softmax"),
        (64, 7168, 256, 8, 2048, 1, "sigmoid"),
        (128, 7168, 384, 8, 2048, 1, "sigmoid"),
    ]
    for c, text, w in zip(C.CASES, BASELINE["configs"], want):
        assert (c.tokens, c.hidden, c.experts, c.topk, c.intermediate, c.shared_experts, c.router) == w
        assert f"{c.tokens} tokens" in text and f"hidden {c.hidden}" in text
        assert c.power_of_two is False and c.weight_std == 0.02 and c.router_std == 0.02
    ds = C.case(C.HEADLINE)
    assert (ds.groups, ds.top_groups, ds.routed_scaling, ds.bias) == (8, 4, 2.5, "normal")
    kimi = C.case("moe-fp8-kimi-k2-t128")
    assert kimi.bias == "zipf" and kimi.zipf_s == 1.1
    assert all(c.max_gpu_launches == 1 for c in C.CASES)


def test_launch_budgets_against_the_reference_catalog():
    """Every fp8 form (layer, block, epilogue variant) and the serial MXFP4 form fit the
    reference's default budget of one launch per call (megabench/cases.py:32); the EP share
    declares more (dispatch, permute, experts, a NaN check, combine, with the exchanges
    between them) and is listed here so the difference stays explicit."""
    over = {c.id: c.max_gpu_launches for c in C.CASES + C.BLOCK_CASES + C.VARIANT_CASES + C.MX_CASES + C.EP_CASES
            if c.max_gpu_launches > C.REFERENCE_LAUNCH_BUDGET}
    assert over == {"megamoe-layer-deepseek-v4-pro-ep8-t512": 6}
    assert C.REFERENCE_LAUNCH_BUDGET == 1


@pytest.mark.parametrize("cid,eu,gb", [
    ("moe-fp8-tiny-t4", 5.47, 0.0087),
    ("moe-fp8-mixtral-t16", 7.92, 1.396),
    ("moe-fp8-qwen3-30b-a3b-t32", 111.8, 0.529),
    ("moe-fp8-deepseek-v3-t64", 222.4, 9.852),
    ("moe-fp8-kimi-k2-t128", 358.1, 15.83),
])
def test_algorithmic_bytes_and_expected_hits(cid, eu, gb):
    c = C.case(cid)
    assert C.expected_hit_experts(c) == pytest.approx(eu, rel=2e-3)
    hit = C.expected_hit_experts(c)
    lo, hi = C.algorithmic_bytes(c, math.floor(hit)), C.algorithmic_bytes(c, math.ceil(hit))
    interp = lo + (hi - lo) * (hit - math.floor(hit))
    assert interp / 1e9 == pytest.approx(gb, rel=6e-3)  # the table quotes 2-4 significant digits


def test_bytes_formula_terms():
    c = C.case(C.HEADLINE)
    H, I, E, T, K = c.hidden, c.intermediate, c.experts, c.tokens, c.topk
    per_expert = 3 * I * H + 4 * 3 * (I // 128) * (H // 128)
    assert C.algorithmic_bytes(c, 1) - C.algorithmic_bytes(c, 0) == per_expert
    assert C.algorithmic_bytes(c, 0) == per_expert + 4 * E * H + 4 * E + 4 * T * H + 12 * T * K
    assert C.algorithmic_flops(c) == 2 * T * E * H + 2 * T * K * 3 * I * H + 2 * T * 3 * I * H


def test_development_geometry_keeps_the_routing_rule():
    for c in C.CASES:
        d = C.development(c)
        assert d.router == c.router and d.bias == c.bias and d.routed_scaling == c.routed_scaling
        assert d.hidden == 256 and d.intermediate == 256 and d.experts <= 16
        assert d.experts % d.groups == 0 and d.topk <= d.experts
    with pytest.raises(ValueError):
        C.development(C.case(C.HEADLINE), experts=10)


def test_case_round_trip_and_validation():
    for c in C.CASES:
        assert C.Case.from_dict(c.to_dict()) == c
        assert C.Case.from_dict({**c.to_dict(), "execution": {"rank": 0}}) == c
    bad = C.case(C.HEADLINE).to_dict()
    for change in (dict(router="relu"), dict(bias="zipf", router="softmax"), dict(noise_factor=0.5)):
        with pytest.raises(ValueError):
            C.Case.from_dict({**bad, **change})


def test_seeds_are_stable_and_independent():
    assert workloads.seed_for(7301, "x") == workloads.seed_for(7301, "x")
    assert workloads.seed_for(7301, "x") != workloads.seed_for(7302, "x")
    assert workloads.seed_for(7301, "x") != workloads.seed_for(7301, "router")
    assert 0 <= workloads.seed_for(1, "gate:0") < 2 ** 63


def test_inputs_have_the_reference_layout_and_quantization_rule():
    c = C.case("moe-fp8-tiny-t4")
    v = workloads.make_inputs(c, 104729, "cpu")
    assert set(v) == set(workloads.input_names(c))
    T, H, E, I = c.tokens, c.hidden, c.experts, c.intermediate
    assert v["x"].dtype == torch.bfloat16 and tuple(v["x"].shape) == (T, H)
    assert v["router"].dtype == torch.float32 and tuple(v["router"].shape) == (E, H)
    assert v["gate"].dtype == torch.float8_e4m3fn and tuple(v["gate"].shape) == (E, I, H)
    assert tuple(v["gate_scale"].shape) == (E, I // 128, H // 128)
    assert tuple(v["down"].shape) == (E, H, I) and tuple(v["down_scale"].shape) == (E, H // 128, I // 128)
    again = workloads.make_inputs(c, 104729, "cpu")
    for k in v:
        assert torch.equal(v[k].view(torch.uint8) if v[k].dtype == torch.float8_e4m3fn else v[k],
                           again[k].view(torch.uint8) if again[k].dtype == torch.float8_e4m3fn else again[k])
    # Each stored block is exactly the packing of its own dequantized values.
    w = formats.unpack_weight(v["up"][3], v["up_scale"][3])
    q, s = formats.pack_weight(w)
    assert torch.equal(s, v["up_scale"][3])
    assert torch.equal(q.view(torch.uint8), v["up"][3].view(torch.uint8))
    assert 0.015 < float(w.std()) < 0.025 and 0.9 < float(v["x"].float().std()) < 1.1


def test_router_bias_profiles():
    ds, kimi = C.case(C.HEADLINE), C.case("moe-fp8-kimi-k2-t128")
    b = workloads.router_bias(ds, 3, "cpu")
    assert b.shape == (256,) and 0.07 < float(b.std()) < 0.13
    z = workloads.router_bias(kimi, 3, "cpu")
    ranked = z.sort(descending=True).values
    want = kimi.zipf_c * torch.arange(1, 385, dtype=torch.float64).pow(-kimi.zipf_s)
    torch.testing.assert_close(ranked.double(), want, rtol=1e-6, atol=0)
    assert workloads.router_bias(C.case("moe-fp8-tiny-t4"), 3, "cpu") is None
