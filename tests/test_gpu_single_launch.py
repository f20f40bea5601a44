"""The layer as one kernel launch (megamoe_layer_forward) on the GPU, through the C ABI.

Its results equal the stream-ordered kernels' (megamoe_forward / megamoe_forward_ex) bit for
bit, on every form (layer, block, clamped bf16 SwiGLU) and on development and full
geometries, over consecutive calls with different inputs on one workspace (the kernel
leaves its control words zero for the next call); and a call launches exactly one kernel,
counted as the reference harness audits it (torch.profiler's device events of one call,
megabench/harness/benchmark.py:73-100). Parity with the CPU oracle is covered by the other
GPU tests, which call the same default path (submission.build)."""

from __future__ import annotations

import sys

import pytest
import torch

from test_gpu_layer import dense_cases
from vibe_megakernel_amd import cases as C
from vibe_megakernel_amd import submission, workloads

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _log(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _to(values):
    return {k: v.to(DEV) for k, v in values.items()}


def _same(a, b, what):
    for k in ("y", "expert_ids", "expert_weights"):
        assert torch.equal(a[k], b[k]), f"{what}: {k} differs"


def _dev_cases():
    out = [C.case("moe-fp8-tiny-t4")]
    out += [C.development(c) for c in C.CASES[1:]]
    out.append(C.development(C.case(C.HEADLINE), tokens=37))
    out.append(C.development(C.case("moe-fp8-kimi-k2-t128"), tokens=70, experts=8, topk=4))
    out.append(C.development(C.case("moe-fp8-mixtral-t16"), hidden=4096, intermediate=512, tokens=40))  # split gate/up
    out += dense_cases() + [C.development(C.BLOCK_CASES[0], tokens=13)]
    out += [C.development(c) for c in C.BLOCK_CASES]
    out += [C.development(c) for c in C.VARIANT_CASES]
    return out


@pytest.mark.parametrize("case", _dev_cases(), ids=lambda c: c.id)
def test_single_launch_equals_stream_ordered_on_development_geometry(case):
    _log(f"single launch {case.id} T={case.tokens} E={case.experts}")
    one = submission.MoELayer(case)
    five = submission.MoELayer(case, single_launch=False)
    assert one.single_launch and not five.single_launch
    for seed in (5, 6, 7):  # consecutive calls on one workspace
        values = _to(workloads.make_inputs(case, seed, "cpu"))
        a, b = one(values), five(values)
        torch.cuda.synchronize()
        _same(a, b, f"{case.id} seed {seed}")
        assert torch.isfinite(a["y"].float()).all()


@pytest.mark.parametrize("cid", [c.id for c in C.CASES])
def test_single_launch_equals_stream_ordered_at_full_size(cid):
    case = C.case(cid)
    _log(f"single launch full size {cid}")
    values = workloads.make_inputs(case, 104729, DEV)
    one = submission.MoELayer(case)
    five = submission.MoELayer(case, single_launch=False)
    for _ in range(2):
        a, b = one(values), five(values)
        torch.cuda.synchronize()
        _same(a, b, cid)


def test_one_call_is_one_kernel_launch():
    from torch.profiler import ProfilerActivity, profile

    case = C.case(C.HEADLINE)
    dev = C.development(case)
    values = _to(workloads.make_inputs(dev, 3, "cpu"))
    run = submission.build(dev.to_dict())
    run(values)  # the workspace is made (and zeroed) on the first call
    torch.cuda.synchronize()
    with profile(activities=[ProfilerActivity.CPU, ProfilerActivity.CUDA]) as prof:
        run(values)
        torch.cuda.synchronize()
    kernels = [e.name for e in prof.events() if e.device_type == torch.autograd.DeviceType.CUDA]
    _log(f"device events of one call: {kernels}")
    assert len(kernels) == 1 and "k_layer" in kernels[0], kernels
    assert dev.max_gpu_launches == 1


def test_a_wait_that_gives_up_is_reported(monkeypatch):
    """The test hook makes the combine units wait for a count the down units never reach, for
    20 us: every kernel ends, y is NaN, and the status word reports it; the next call on the
    same workspace is whole again and reports nothing."""
    case = C.development(C.case(C.HEADLINE))
    layer = submission.MoELayer(case)
    values = _to(workloads.make_inputs(case, 8, "cpu"))
    good = layer(values)
    torch.cuda.synchronize()
    assert not layer.gave_up(torch.device(DEV))
    monkeypatch.setenv("MEGAMOE_FORCE_WAIT_TIMEOUT", "1")
    bad = layer(values)
    torch.cuda.synchronize()
    assert torch.isnan(bad["y"].float()).all()
    assert torch.equal(bad["expert_ids"], good["expert_ids"])
    assert layer.gave_up(torch.device(DEV))
    monkeypatch.delenv("MEGAMOE_FORCE_WAIT_TIMEOUT")
    again = layer(values)
    torch.cuda.synchronize()
    _same(again, good, "after a forced give-up")
    assert not layer.gave_up(torch.device(DEV))


@pytest.mark.parametrize("cid", [C.HEADLINE, "moe-fp8-kimi-k2-t128", "moe-fp8-qwen3-30b-a3b-t32"])
def test_router_units_left_by_their_workgroups_are_rescued(monkeypatch, cid):
    """Router units go to the workgroup of the same index; a routing unit runs (and counts) any
    whose workgroup has not started it, so the layer completes whatever number of workgroups
    the device keeps resident. The test hook makes every odd workgroup leave its unit to them:
    the results equal the stream-ordered form's bit for bit, and no wait gives up."""
    monkeypatch.setenv("MEGAMOE_FORCE_RESCUE", "1")
    for case in (C.development(C.case(cid)), C.case(cid)):
        _log(f"forced rescue {case.id} T={case.tokens} E={case.experts}")
        values = workloads.make_inputs(case, 11, DEV)
        one = submission.MoELayer(case)
        five = submission.MoELayer(case, single_launch=False)
        for _ in range(2):
            a, b = one(values), five(values)
            torch.cuda.synchronize()
            _same(a, b, f"{case.id} with forced rescue")
        assert not one.gave_up(torch.device(DEV))
