"""The single launch under HIP graph capture and replay, through the C ABI.

The reference captures its reference path in a torch.cuda.CUDAGraph for the graph baseline
(megabench/harness/runner.py:178-186). A call of the single launch is one kernel and no
allocation, so it can be captured: the first call (outside capture) makes the workspace and
zeroes it, and each call leaves the control words zero again, so every replay starts from
them as an eager call would. Each replay runs on new contents of the captured inputs, with
eager calls of the same layer and synchronizations between replays, and must equal an eager
call on the same inputs bit for bit (and the oracle, on the development geometry).
"""

from __future__ import annotations

import sys

import pytest
import torch

from oracle import layer, metrics, mx
from vibe_megakernel_amd import cases as C
from vibe_megakernel_amd import submission, workloads

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _log(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _capture(layer_, static, stream):
    """A graph of one call on ``static``, captured on ``stream`` after a call outside capture
    on the same stream (the workspace is per stream, so the capture uses that one)."""
    with torch.cuda.stream(stream):
        layer_(static)
    stream.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        out = layer_(static)
    return graph, out


def _fp8_cases():
    return [C.development(C.case(C.HEADLINE)), C.case("moe-fp8-tiny-t4"),
            C.development(C.case("moe-fp8-mixtral-t16"), hidden=4096, intermediate=512, tokens=40),  # split gate/up
            C.development(C.BLOCK_CASES[0]),
            C.development(C.case(C.HEADLINE), tokens=8),  # the dense schedule with a shared expert
            C.development(C.case(C.HEADLINE + "-w8a16"))]  # the W8A16 form


@pytest.mark.parametrize("case", _fp8_cases(), ids=lambda c: c.id)
def test_captured_layer_replays_equal_eager_calls(case):
    _log(f"graph capture {case.id} T={case.tokens} E={case.experts}")
    captured = submission.MoELayer(case)
    eager = submission.MoELayer(case)
    static = workloads.make_inputs(case, 40, DEV)
    stream = torch.cuda.Stream()
    graph, out = _capture(captured, static, stream)
    for seed in (41, 42, 43, 44):
        fresh = workloads.make_inputs(case, seed, DEV)
        for k, v in fresh.items():
            static[k].copy_(v)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        want = eager(fresh)  # eager work between the replays, on another workspace
        torch.cuda.synchronize()
        for k in ("y", "expert_ids", "expert_weights"):
            assert torch.equal(out[k], want[k]), f"{case.id} seed {seed}: {k} of the replay differs"
        assert torch.isfinite(out["y"].float()).all()
        if seed == 41 and case.hidden <= 1024:
            cpu = {k: v.cpu() for k, v in fresh.items()}
            ref = layer.block_reference(case, cpu) if case.residual else layer.reference(case, cpu)
            assert torch.equal(out["expert_ids"].cpu(), ref["expert_ids"])
            assert metrics.layer_checks(out["y"].cpu(), ref["y"])["pass"]
    # The captured workspace ends every replay with its control words zero: an eager call on
    # it (same stream) still gives the right answer and reports no give-up.
    with torch.cuda.stream(stream):
        again = captured(static)
        assert not captured.gave_up(torch.device(DEV))
    stream.synchronize()
    want = eager(static)
    torch.cuda.synchronize()
    assert torch.equal(again["y"], want["y"])


def test_captured_mx_layer_replays_equal_eager_calls():
    case = C.development(C.case("moe-mxfp4-deepseek-v4-pro-t64"))
    _log(f"graph capture {case.id}")
    captured = submission.MoELayer(case)
    eager = submission.MoELayer(case)
    static = workloads.make_inputs(case, 50, DEV)
    stream = torch.cuda.Stream()
    graph, out = _capture(captured, static, stream)
    for seed in (51, 52, 53):
        fresh = workloads.make_inputs(case, seed, DEV)
        for k, v in fresh.items():
            static[k].copy_(v)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        want = eager(fresh)
        torch.cuda.synchronize()
        assert torch.equal(out["y"], want["y"]), f"seed {seed}"
        if seed == 51:
            ref = mx.reference(case, {k: v.cpu() for k, v in fresh.items()})["y"]
            assert metrics.layer_checks(out["y"].cpu(), ref)["pass"]
