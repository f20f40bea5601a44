"""GPU parity of the W8A16 form (bf16 activations into the expert GEMMs: frontier.py:180-183
with quantize=False, the DeepSeek family's experts, frontier.py:190,265-270) against the CPU
oracle, through megamoe_layer_forward_w8a16 (one launch, the submission's path), and that
form equal bit for bit to the stream-ordered megamoe_forward_w8a16.

Bars as the W8A8 layer's: expert ids bit-exact, weights within 1e-4 relative of the
reference's, y within the band rule against the widened (FP32) W8A16 oracle and within
max-rel 1e-2 / cosine 0.9999 against its BF16 reference schedule. The FP8 weights enter the
bf16 MFMA exactly (every E4M3 value is a bf16 value); the sums differ from the reference's
fp32 GEMV only in order.
"""

from __future__ import annotations

import sys
from dataclasses import replace

import pytest
import torch

from oracle import layer, metrics
from vibe_megakernel_amd import cases as C
from vibe_megakernel_amd import submission, workloads

from test_gpu_layer import _compare, check_every_token

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
W8A16 = C.case(C.HEADLINE + "-w8a16")


def _log(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _to(values, device):
    return {k: v.to(device) for k, v in values.items()}


def _a16(c):
    return replace(c, activations="bf16")


def _dev_cases():
    return [
        C.development(W8A16),                                   # grouped sigmoid, shared expert
        C.development(W8A16, tokens=37),                        # ragged, chunks of 32 rows and a tail
        C.development(W8A16, tokens=8),                         # the dense schedule (T <= 16, T*K >= E)
        _a16(C.development(C.case("moe-fp8-kimi-k2-t128"), tokens=70, experts=8, topk=4)),  # experts of > 32 rows
        _a16(C.development(C.case("moe-fp8-qwen3-30b-a3b-t32"))),                          # softmax, no shared
        _a16(C.development(C.case("moe-fp8-mixtral-t16"), hidden=4096, intermediate=512, tokens=40)),
        _a16(C.development(C.case("moe-fp8-glm-5.3-flash-t64"))),                          # bf16 SwiGLU, clamp
    ]


@pytest.mark.parametrize("case", _dev_cases(), ids=lambda c: c.id)
def test_w8a16_matches_oracle_on_development_geometry(case):
    _log(f"w8a16 parity {case.id} T={case.tokens} H={case.hidden} E={case.experts} K={case.topk}")
    assert case.activations == "bf16"
    for seed in (104729, 104730):
        values = workloads.make_inputs(case, seed, "cpu")
        want, exact = layer.reference_and_oracle(case, values)
        run = submission.build(case.to_dict())
        assert run.layer.single_launch and run.layer.a16
        got = run(_to(values, DEV))
        torch.cuda.synchronize()
        _compare(case, got, want, exact)


@pytest.mark.parametrize("case", _dev_cases() + [_a16(C.development(C.BLOCK_CASES[0]))], ids=lambda c: c.id)
def test_w8a16_single_launch_equals_stream_ordered(case):
    """The one-launch W8A16 form against its five launches, bit for bit, over consecutive calls
    on one workspace (the control words must come back to zero after each call)."""
    _log(f"w8a16 single vs stream-ordered {case.id}")
    one = submission.MoELayer(case)
    five = submission.MoELayer(case, single_launch=False)
    assert one.single_launch and not five.single_launch
    dev = torch.device(DEV)
    for seed in (5, 6, 7):
        values = _to(workloads.make_inputs(case, seed, "cpu"), DEV)
        a, b = one(values), five(values)
        torch.cuda.synchronize()
        assert not one.gave_up(dev)
        for k in a:
            assert torch.equal(a[k], b[k]), (case.id, seed, k)


def test_w8a16_is_not_the_w8a8_layer():
    """The same inputs through the W8A8 layer land off the W8A16 oracle's band more than the
    W8A16 form does (the quantization noise of x and h is gone)."""
    case = C.development(W8A16, tokens=24)
    _log(f"w8a16 vs w8a8 {case.id}")
    values = workloads.make_inputs(case, 7, "cpu")
    want, exact = layer.reference_and_oracle(case, values)
    a16 = submission.build(case.to_dict())(_to(values, DEV))
    a8 = submission.build(replace(case, activations="fp8").to_dict())(_to(values, DEV))
    torch.cuda.synchronize()
    e16 = metrics.layer_checks(a16["y"].cpu(), exact["y"].to(torch.bfloat16))
    e8 = metrics.layer_checks(a8["y"].cpu(), exact["y"].to(torch.bfloat16))
    assert e16["max_rel"] < e8["max_rel"], (e16, e8)


def test_w8a16_block_form():
    """RMSNorm before (the experts read the normalized rows in bf16) and the residual after."""
    case = _a16(C.development(C.BLOCK_CASES[0]))
    _log(f"w8a16 block {case.id}")
    values = workloads.make_inputs(case, 104729, "cpu")
    want, exact = layer.block_reference(case, values), layer.block_oracle(case, values)
    got = submission.build(case.to_dict())(_to(values, DEV))
    torch.cuda.synchronize()
    assert torch.equal(got["expert_ids"].cpu(), want["expert_ids"])
    check = metrics.layer_checks(got["y"].cpu(), want["y"])
    assert check["pass"], check
    band = metrics.band(want["y"], got["y"].cpu(), exact["y"], bf16_rtol=case.bf16_rtol,
                        noise_factor=case.noise_factor)
    assert band["pass"], band


def test_w8a16_is_deterministic():
    case = C.development(W8A16, tokens=40)
    _log(f"w8a16 determinism {case.id}")
    values = _to(workloads.make_inputs(case, 11, "cpu"), DEV)
    run = submission.build(case.to_dict())
    a, b = run(values), run(values)
    torch.cuda.synchronize()
    for k in a:
        assert torch.equal(a[k], b[k]), k


def test_w8a16_full_size_on_every_token():
    """The headline geometry in the W8A16 form, inputs generated on the GPU; every token."""
    _log(f"w8a16 full size {W8A16.id}")
    values = workloads.make_inputs(W8A16, 104729, DEV)
    got = submission.build(W8A16.to_dict())(values)
    torch.cuda.synchronize()
    cpu = {k: v.cpu() for k, v in values.items()}
    del values
    torch.cuda.empty_cache()
    check_every_token(W8A16, got, cpu)


def test_w8a16_dense_single_launch_over_many_calls():
    """Regression: the W8A16 single launch once quantized x into the region that holds its bf16
    h, leaving write-through copies of those lines in the routing units' XCD L2s, where a
    down unit on the same XCD could read a stale h row (NaN in one 128-column block of y,
    about one call in 470 on this geometry). 3000 consecutive calls of the dense schedule on
    one workspace, each equal to the stream-ordered form bit for bit."""
    base = C.development(C.case("moe-fp8-mixtral-t16"), hidden=4096, intermediate=512)
    case = _a16(replace(base, params={**base.params, "tokens": 4}))
    _log(f"w8a16 dense, many calls {case.id} T={case.tokens} H={case.hidden} E={case.experts}")
    one = submission.MoELayer(case)
    five = submission.MoELayer(case, single_launch=False)
    assert one.single_launch and one.a16
    dev = torch.device(DEV)
    for i in range(3000):
        values = workloads.make_inputs(case, 1000 + i, DEV)
        a, b = one(values), five(values)
        torch.cuda.synchronize()
        for k in a:
            assert torch.equal(a[k], b[k]), f"call {i} (seed {1000 + i}): {k} differs"
        assert not one.gave_up(dev), f"call {i}: a bounded wait gave up"
