"""GPU parity of the epilogue variants, through the C ABI.

* GLM-5.3-Flash's MoE (glm53.py:263-274, SwiGLU in bf16 with the clamp at 10,
  glm53.py:174-175) via megamoe_forward_ex: the layer bars of tests/test_gpu_layer.py (ids
  bit-exact, weights, y max-rel/cosine against the BF16 schedule, the band rule against the
  FP32 oracle) on development geometries, one with weights large enough that the clamp acts,
  and on three tokens of the full shape; megamoe_forward_ex with the default epilogue equal
  to megamoe_forward bit for bit.
* GPT-OSS's combine (gptoss.py:112-124) via megamoe_combine_by_expert_id: bit-exact against
  oracle/combine.py, with and without the residual, on several shapes.
"""

from __future__ import annotations

import sys
from dataclasses import replace

import pytest
import torch

from oracle import combine, layer, metrics
from vibe_megakernel_amd import cases as C
from vibe_megakernel_amd import submission, workloads

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
GLM = C.case("moe-fp8-glm-5.3-flash-t64")


def _log(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _to(values, device):
    return {k: v.to(device) for k, v in values.items()}


def _compare(case, got, want, exact, rows=None):
    ids, w, y = got["expert_ids"].cpu(), got["expert_weights"].cpu(), got["y"].cpu()
    if rows is not None:
        ids, w, y = ids[rows], w[rows], y[rows]
    assert torch.equal(ids, want["expert_ids"]), f"{case.id}: expert ids differ"
    torch.testing.assert_close(w, want["expert_weights"], rtol=1e-4, atol=0)
    check = metrics.layer_checks(y, want["y"])
    assert check["pass"], f"{case.id}: {check}"
    band = metrics.band(want["y"], y, exact["y"], bf16_rtol=case.bf16_rtol, noise_factor=case.noise_factor)
    assert band["pass"], f"{case.id}: band {band}"
    return check


def _glm_dev():
    base = C.development(GLM)
    return [base, replace(C.development(GLM, tokens=37), id="glm-dev-clamped", weight_std=0.5),
            replace(base, id="glm-dev-unclamped", swiglu_limit=0.0)]


@pytest.mark.parametrize("case", _glm_dev(), ids=lambda c: c.id)
def test_glm_layer_matches_oracle_on_development_geometry(case):
    _log(f"glm parity {case.id} T={case.tokens} w_std={case.weight_std} limit={case.swiglu_limit}")
    for seed in (104729, 104730):
        values = workloads.make_inputs(case, seed, "cpu")
        want, exact = layer.reference(case, values), layer.oracle(case, values)
        got = submission.build(case.to_dict())(_to(values, DEV))
        torch.cuda.synchronize()
        _compare(case, got, want, exact)


def test_glm_full_size_on_every_token():
    case = GLM
    _log(f"glm full size {case.id}")
    values = workloads.make_inputs(case, 104729, DEV)
    got = submission.build(case.to_dict())(values)
    torch.cuda.synchronize()
    cpu = {k: v.cpu() for k, v in values.items()}
    del values
    torch.cuda.empty_cache()
    want, exact = layer.reference_and_oracle(case, cpu)
    _log(f"  {_compare(case, got, want, exact)}")


def test_default_epilogue_equals_plain_forward():
    case = C.development(C.case(C.HEADLINE), tokens=24)
    _log("forward_ex default epilogue")
    values = _to(workloads.make_inputs(case, 9, "cpu"), DEV)
    plain = submission.build(case.to_dict())(values)
    layer_ex = submission.MoELayer(case)
    layer_ex.epilogue = submission._lib.Epilogue(swiglu=0, swiglu_limit=0.0)  # forces megamoe_forward_ex
    ex = layer_ex(values)
    torch.cuda.synchronize()
    for k in ("y", "expert_ids", "expert_weights"):
        assert torch.equal(plain[k], ex[k]), k


@pytest.mark.parametrize("T,K,H,E,residual", [(1, 4, 64, 32, False), (37, 8, 512, 64, True),
                                              (64, 4, 2880, 128, True), (5, 32, 256, 64, False)])
def test_combine_by_expert_id_is_bit_exact(T, K, H, E, residual):
    _log(f"combine by expert id T={T} K={K} H={H}")
    g = torch.Generator().manual_seed(T * 1000 + K)
    out = (torch.randn((T, K, H), generator=g) * 4).to(torch.bfloat16)
    ids = torch.stack([torch.randperm(E, generator=g)[:K] for _ in range(T)])
    w = torch.softmax(torch.randn((T, K), generator=g), -1).to(torch.bfloat16)
    res = torch.randn((T, H), generator=g).to(torch.bfloat16) if residual else None
    want = combine.by_expert_id(out, ids, w, res)
    got = submission.combine_by_expert_id(out.to(DEV), ids.to(DEV), w.to(DEV),
                                          None if res is None else res.to(DEV)).cpu()
    assert torch.equal(got, want)
