"""Pins of the block-form oracle (CPU): oracle.layer.rms_norm, the restatement of
megabench/tasks/common.py:13-21 (RMSNorm, gamma applied in fp32 before the one bf16 rounding
for DeepSeek, to the rounded activation otherwise), and oracle.layer.block, the decoder
block of megabench/tasks/frontier.py:335-354 (rms -> layer -> residual add).

Independent pins of rms_norm: torch's own ``F.rms_norm`` (the fp32-gamma form) and
transformers' ``DeepseekV3RMSNorm`` (the bf16-gamma form), both of which take the mean of
squares in fp32 in their own order, so a bf16 output may differ by one ulp where the
exact and the fp32 mean round apart; closed forms (zero rows, constant rows, power-of-two
scale invariance at eps = 0); and planted mistakes (no eps, sum for mean, gamma dropped,
gamma applied on the wrong side of the rounding) that these checks must catch.
"""

from __future__ import annotations

import pytest
import torch
import torch.nn.functional as F

from oracle import layer
from vibe_megakernel_amd import cases as C
from vibe_megakernel_amd import workloads


def _rows(seed: int, T: int, H: int, scale: float = 1.0):
    g = torch.Generator().manual_seed(seed)
    x = (torch.randn((T, H), generator=g) * scale).to(torch.bfloat16)
    w = (torch.randn((H,), generator=g) * 0.1 + 1.0).to(torch.bfloat16)
    return x, w


def _ulps(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    return (a.view(torch.int16).int() - b.view(torch.int16).int()).abs()


def _close_to(got: torch.Tensor, want: torch.Tensor) -> bool:
    d = _ulps(got, want)
    return bool(d.max() <= 1 and (d > 0).float().mean() < 2e-3)


@pytest.mark.parametrize("shape", [(8, 7168), (16, 2048), (5, 1024)])
def test_fp32_gamma_form_matches_torch_rms_norm(shape):
    x, w = _rows(1, *shape)
    got = layer.rms_norm(x, w, 1e-6, True)
    want = F.rms_norm(x.float(), (shape[1],), w.float(), 1e-6).to(torch.bfloat16)
    assert _close_to(got, want)


@pytest.mark.parametrize("shape", [(8, 7168), (16, 2048)])
def test_bf16_gamma_form_matches_transformers_deepseek_rmsnorm(shape):
    from transformers.models.deepseek_v3.modeling_deepseek_v3 import DeepseekV3RMSNorm

    x, w = _rows(2, *shape)
    norm = DeepseekV3RMSNorm(shape[1], eps=1e-5)
    with torch.no_grad():
        norm.weight.copy_(w.float())
    norm = norm.to(torch.bfloat16)
    with torch.no_grad():
        want = norm(x)
    assert want.dtype == torch.bfloat16
    assert _close_to(layer.rms_norm(x, w, 1e-5, False), want)


def test_closed_forms():
    H = 1024
    _, w = _rows(3, 1, H)
    zero = torch.zeros((1, H), dtype=torch.bfloat16)
    for fp32w in (True, False):
        assert torch.equal(layer.rms_norm(zero, w, 1e-6, fp32w), zero)
        # A constant row of 0.5 with eps = 0: mean 0.25, r = 2, n = 1 exactly, out = gamma.
        half = torch.full((1, H), 0.5, dtype=torch.bfloat16)
        assert torch.equal(layer.rms_norm(half, w, 0.0, fp32w)[0], w)
        # Scaling a row by a power of two leaves its normalization unchanged at eps = 0.
        x, _ = _rows(4, 3, H)
        base = layer.rms_norm(x, w, 0.0, fp32w)
        for k in (-6, 3):
            assert torch.equal(layer.rms_norm((x.float() * 2.0 ** k).to(torch.bfloat16), w, 0.0, fp32w), base)


def test_planted_mistakes_are_caught():
    H = 2048
    x, w = _rows(5, 8, H, scale=1e-3)  # small rows: the mean of squares (~1e-6) is comparable to eps
    eps = 1e-5
    want = F.rms_norm(x.float(), (H,), w.float(), eps).to(torch.bfloat16)
    assert _close_to(layer.rms_norm(x, w, eps, True), want)
    xf = x.float()
    no_eps = (xf * torch.rsqrt(xf.square().mean(-1, keepdim=True)) * w.float()).to(torch.bfloat16)
    sum_for_mean = (xf * torch.rsqrt(xf.square().sum(-1, keepdim=True) + eps) * w.float()).to(torch.bfloat16)
    no_gamma = layer.rms_norm(x, torch.ones_like(w), eps, True)
    assert not _close_to(no_eps, want)
    assert not _close_to(sum_for_mean, want)
    assert not _close_to(no_gamma, want)
    # The two gamma forms differ (rounding before or after the gamma): each matches only its own pin.
    xs, ws = _rows(6, 16, H)
    fp32_form = F.rms_norm(xs.float(), (H,), ws.float(), eps).to(torch.bfloat16)
    assert _close_to(layer.rms_norm(xs, ws, eps, True), fp32_form)
    assert (_ulps(layer.rms_norm(xs, ws, eps, False), fp32_form) > 0).float().mean() > 0.05


def test_block_composition():
    case = C.development(C.case(C.HEADLINE + "-block"), tokens=6)
    values = workloads.make_inputs(case, 17, "cpu")
    out = layer.block_reference(case, values)
    xn = layer.rms_norm(values["x"], values["ln2"], case.norm_eps, True)
    inner = layer.reference(case, dict(values, x=xn))
    assert torch.equal(out["expert_ids"], inner["expert_ids"])
    assert torch.equal(out["y"], (values["x"].float() + inner["y"].float()).to(torch.bfloat16))
    # Without the block steps the block is the layer.
    plain = C.development(C.case(C.HEADLINE), tokens=6)
    pv = workloads.make_inputs(plain, 17, "cpu")
    assert torch.equal(layer.block_reference(plain, pv)["y"], layer.reference(plain, pv)["y"])
    # The widened block keeps fp32 and drops every bf16 rounding, the norm's included.
    wide = layer.block_oracle(case, values)
    assert wide["y"].dtype == torch.float32
    assert torch.allclose(wide["y"], out["y"].float(), rtol=0.05, atol=0.05)
