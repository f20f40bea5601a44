"""Pins of the MXFP4-form oracle (oracle/mx.py, CPU), independent of the formulas it restates:

* E2M1: every code decoded from its sign / exponent / mantissa fields against the format's
  value table (quantization.py:9-10); every midpoint of the grid rounds to the even code;
  values on the grid and all-zero blocks round-trip exactly; the E8M0 scale exponent is the
  smallest that fits the block (amax / 2^e <= 6 < amax / 2^(e-1)), clamped at 2^-126;
* the input generator's packer (a per-binade half-to-even formulation) equals the oracle's
  (an argmin over the grid) on random and edge inputs;
* E8M0 activation exponents: equal to DeepGEMM's ceil-to-UE8M0 rule on the rows and edge
  values of megabench/tests/test_megamoe.py:56-65, and the round-trip error bound there;
* the widened layer against transformers' DeepseekV4Experts (the check of
  test_megamoe.py:128-148), and planted mistakes it must catch.
"""

from __future__ import annotations

import json
from pathlib import Path

import pytest
import torch

from oracle import mx
from vibe_megakernel_amd import cases as C
from vibe_megakernel_amd import workloads

GOLDEN = json.loads((Path(__file__).parent / "golden" / "known_answers.json").read_text())
FP4_TABLE = (0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0, -0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0)


def test_e2m1_codes_decode_from_their_fields():
    for code, want in enumerate(FP4_TABLE):
        got = mx.e2m1_value(code)
        assert got == want and (str(got)[0] == "-") == (str(want)[0] == "-"), code


def test_mxfp4_rounding_ties_to_even_and_round_trips():
    # One block with amax 6 (scale 2^0), holding every grid point and every midpoint.
    grid = [0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0]
    mids = [0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0]
    want_mid = [0.0, 1.0, 1.0, 2.0, 2.0, 4.0, 4.0]  # the even code of each pair
    row = grid + [-g for g in grid] + mids + [-m for m in mids] + [6.0, -6.0]
    x = torch.tensor(row, dtype=torch.float32)[None]
    packed, scales = mx.pack_mxfp4(x)
    assert scales.tolist() == [[127]]
    back = mx.unpack_mxfp4(packed, scales)[0].tolist()
    assert back[:16] == grid + [-g for g in grid]
    assert back[16:23] == want_mid and back[23:30] == [-m for m in want_mid]
    # Zero blocks: exponent clamped at -126, payload zero.
    p0, s0 = mx.pack_mxfp4(torch.zeros((2, 64)))
    assert (s0 == 1).all() and (p0 == 0).all()


def test_mxfp4_scale_is_the_smallest_that_fits():
    g = torch.Generator().manual_seed(1)
    x = torch.randn((64, 256), generator=g) * torch.logspace(-20, 20, 64)[:, None]
    _, s = mx.pack_mxfp4(x)
    amax = x.unflatten(-1, (-1, 32)).abs().amax(-1).double()
    e = s.double() - 127
    assert (amax / 2.0 ** e <= 6.0).all()
    assert (amax / 2.0 ** (e - 1) > 6.0).all()


def test_generator_packer_equals_oracle_packer():
    g = torch.Generator().manual_seed(2)
    x = torch.randn((48, 512), generator=g) * torch.logspace(-8, 8, 48)[:, None]
    x[0, :30] = torch.tensor([0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0, -0.25, -0.75, -1.25, -1.75, -2.5, -3.5, -5.0,
                              6.0, -6.0, 0.0, -0.0, 4.0, 3.0, 2.0, 1.5, 1.0, 0.5, 4.5, 5.5, 2.25, 2.75, 3.25, 3.75])
    pa, sa = workloads.pack_mxfp4(x)
    pb, sb = mx.pack_mxfp4(x)
    assert torch.equal(pa, pb) and torch.equal(sa, sb)
    qa, ea = workloads.pack_e4m3_e8m0(x)
    qb, eb = mx.pack_activation_e8m0(x)
    assert torch.equal(qa.view(torch.uint8), qb.view(torch.uint8)) and torch.equal(ea, eb)


def _ceil_to_ue8m0(maximum: torch.Tensor) -> torch.Tensor:
    """DeepGEMM per_token_cast_to_fp8's scale: the exponent of clamp(amax, 1e-4) / 448,
    rounded up (megabench/tests/test_megamoe.py:40-44)."""
    bits = (maximum.clamp_min(1e-4) / 448.0).view(torch.int32)
    exponent = ((bits >> 23) & 0xFF) + (bits & 0x7FFFFF).bool().int()
    return exponent.clamp(1, 254).to(torch.uint8)


def test_e8m0_activation_exponent_matches_deepgemm_rule_and_bound():
    g = torch.Generator().manual_seed(3)
    value = torch.randn((64, 256), generator=g) * torch.logspace(-6, 3, 64)[:, None]
    edges = torch.tensor(GOLDEN["fp8_edge_values"]["values"])
    value[:len(edges), 0] = edges
    payload, scales = mx.pack_activation_e8m0(value)
    maximum = value.unflatten(-1, (-1, 32)).abs().amax(-1)
    assert torch.equal(scales, _ceil_to_ue8m0(maximum))
    restored = mx.unpack_activation_e8m0(payload, scales)
    assert torch.isfinite(restored).all()
    scale = torch.exp2(scales.float() - 127).repeat_interleave(32, -1)
    assert ((restored - value).abs() <= value.abs() * 2 ** -4 + scale * 2 ** -10).all()


def _tiny(tokens=12):
    return C.development(C.case("moe-mxfp4-deepseek-v4-pro-t64"), tokens=tokens, experts=8, topk=4)


def _expected_with_transformers(case, values):
    from transformers.models.deepseek_v4.configuration_deepseek_v4 import DeepseekV4Config
    from transformers.models.deepseek_v4.modeling_deepseek_v4 import DeepseekV4Experts

    config = DeepseekV4Config(num_local_experts=case.experts, n_routed_experts=case.experts,
                              hidden_size=case.hidden, intermediate_size=case.intermediate,
                              moe_intermediate_size=case.intermediate, swiglu_limit=case.swiglu_limit,
                              hidden_act="silu")
    module = DeepseekV4Experts(config)
    with torch.no_grad():
        module.gate_up_proj.copy_(mx.unpack_mxfp4(values["l1_blocks"], values["l1_scales"]))
        module.down_proj.copy_(mx.unpack_mxfp4(values["l2_blocks"], values["l2_scales"]))
        x = mx.unpack_activation_e8m0(values["x"], values["x_scales"])
        return module(x, values["topk_idx"], values["topk_weights"]), module, x


@pytest.mark.parametrize("seed", [1, 2])
def test_widened_layer_matches_transformers_deepseek_v4_experts(seed):
    case = _tiny()
    values = workloads.make_inputs(case, seed, "cpu")
    expected, module, x = _expected_with_transformers(case, values)
    # The clamp is exercised by the generator's gain.
    assert int(((x @ module.gate_up_proj[0].T).abs() > case.swiglu_limit).sum()) > 0
    exact = mx.oracle(case, values)["y"]
    torch.testing.assert_close(exact, expected, rtol=1e-5, atol=1e-5 * float(expected.abs().max()))
    served = mx.reference(case, values)["y"].double()
    assert float((served - expected.double()).norm() / expected.double().norm()) < 0.05


def test_planted_mistakes_are_caught():
    case = _tiny()
    values = workloads.make_inputs(case, 3, "cpu")
    expected, _, _ = _expected_with_transformers(case, values)

    def off(v):
        y = mx.oracle(case, v)["y"]
        return float((y - expected).norm() / expected.norm()) > 1e-3

    I = case.intermediate
    swapped = dict(values, l1_blocks=torch.cat([values["l1_blocks"][:, I:], values["l1_blocks"][:, :I]], 1),
                   l1_scales=torch.cat([values["l1_scales"][:, I:], values["l1_scales"][:, :I]], 1))
    nibbles = dict(values, l2_blocks=((values["l2_blocks"] & 15) << 4) | (values["l2_blocks"] >> 4))
    unweighted = dict(values, topk_weights=torch.ones_like(values["topk_weights"]))
    shifted = dict(values, x_scales=values["x_scales"] + 1)
    for name, v in (("gate/up swapped", swapped), ("nibble order", nibbles), ("weights dropped", unweighted),
                    ("x scale", shifted)):
        assert off(v), name
    unclamped = C.Case.from_dict({**case.to_dict(), "swiglu_limit": 1e9})
    assert float((mx.oracle(unclamped, values)["y"] - expected).norm() / expected.norm()) > 1e-3
