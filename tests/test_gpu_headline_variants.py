"""GPU parity of the variants of the headline DeepSeek-V3 shape, through the C ABI.

"-ue8m0": power-of-two (UE8M0) scales for the weights and for the activations quantized in
the layer (x per 128, h per 128), the DeepSeek family's scale format (frontier.py:120,252;
quantization.py:57-59). "-nobias": the routing without the correction bias, ~222 experts hit
at ~2.3 rows each. "-w8a16": bf16 activations into the expert GEMMs (frontier.py:180-183,
quantize=False). "-w8a16-ue8m0": both, the DeepSeek family's expert numerics as the
reference runs them (frontier.py:252-270). Each is checked on its development geometry (two
seeds) and at full size on every token against the oracle, and the single launch equals the
stream-ordered kernels bit for bit on each.
"""

from __future__ import annotations

import sys

import pytest
import torch

from oracle import layer
from test_gpu_layer import _compare, check_every_token
from vibe_megakernel_amd import cases as C
from vibe_megakernel_amd import submission, workloads

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _log(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _same(a, b, what):
    for k in ("y", "expert_ids", "expert_weights"):
        assert torch.equal(a[k], b[k]), f"{what}: {k} differs"


def _pow2(t):
    """Every value a power of two (the UE8M0 grid)."""
    m, _ = torch.frexp(t)
    return bool((m == 0.5).all())


@pytest.mark.parametrize("case", [C.development(c) for c in C.HEADLINE_VARIANTS], ids=lambda c: c.id)
def test_variant_matches_oracle_on_development_geometry(case):
    _log(f"headline variant {case.id} T={case.tokens} H={case.hidden} E={case.experts}")
    one = submission.MoELayer(case)
    five = submission.MoELayer(case, single_launch=False)
    for seed in (104729, 104730):
        values = workloads.make_inputs(case, seed, "cpu")
        if case.power_of_two:
            assert _pow2(values["gate_scale"]) and _pow2(values["shared_down_scale"])
        want, exact = layer.reference(case, values), layer.oracle(case, values)
        gpu = {k: v.to(DEV) for k, v in values.items()}
        a, b = one(gpu), five(gpu)
        torch.cuda.synchronize()
        _same(a, b, f"{case.id} seed {seed}")
        _compare(case, a, want, exact)


def test_ue8m0_activation_scales_reach_the_layer():
    """The same inputs with and without power-of-two activation scales give different y: the
    flag reaches the x and h quantization of the kernels (the weights' scales are inputs)."""
    base = C.development(C.case(C.HEADLINE))
    pw = C.development(C.case(C.HEADLINE + "-ue8m0"))
    values = {k: v.to(DEV) for k, v in workloads.make_inputs(pw, 3, "cpu").items()}
    a = submission.MoELayer(pw)(values)["y"]
    b = submission.MoELayer(base)(values)["y"]
    torch.cuda.synchronize()
    assert not torch.equal(a, b)


@pytest.mark.parametrize("cid", [c.id for c in C.HEADLINE_VARIANTS])
def test_variant_full_size_on_every_token(cid):
    case = C.case(cid)
    _log(f"headline variant full size {cid}")
    values = workloads.make_inputs(case, 104729, DEV)
    got = submission.build(case.to_dict())(values)
    five = submission.MoELayer(case, single_launch=False)(values)
    torch.cuda.synchronize()
    _same(got, five, cid)
    hit = len(torch.unique(got["expert_ids"]))
    _log(f"  {cid}: {hit} experts hit")
    if case.bias == "none":
        assert hit > 200, hit  # the decode regime: most experts hit, ~2.3 rows each
    cpu = {k: v.cpu() for k, v in values.items()}
    del values
    torch.cuda.empty_cache()
    check_every_token(case, got, cpu)
