"""GPU parity of the MXFP4 form (megamoe.py numerics, serial) against the CPU oracle,
through the C ABI: y within max|y - y_ref| / max|y_ref| <= 1e-2 and cosine >= 0.9999 of
the BF16 reference schedule (oracle.mx.reference) and within the band rule of
megabench/harness/correctness.py:64-85 against the widened oracle; deterministic; inputs
untouched; out-of-range or repeated expert ids give NaN (forced from the host: the
kernels still run to completion)."""

from __future__ import annotations

import sys

import pytest
import torch

from oracle import metrics, mx
from vibe_megakernel_amd import cases as C
from vibe_megakernel_amd import submission, workloads

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
MXCASE = "moe-mxfp4-deepseek-v4-pro-t64"


def _log(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _to(values, device):
    return {k: v.to(device) for k, v in values.items()}


def _check(case, y, want, exact):
    check = metrics.layer_checks(y, want)
    assert check["pass"], f"{case.id}: {check}"
    band = metrics.band(want, y, exact, bf16_rtol=case.bf16_rtol, noise_factor=case.noise_factor)
    assert band["pass"], f"{case.id}: band {band}"
    return check, band


def _dev_cases():
    base = C.case(MXCASE)
    # 1-30 rows per expert (narrow units), about 35 (wide, one tile per wave) and about 150
    # (a wide chunk of 128 rows with two tiles per wave, plus a narrow remainder).
    return [C.development(base), C.development(base, tokens=37, experts=8, topk=4),
            C.development(base, tokens=70, experts=4, topk=2, hidden=512, intermediate=512),
            C.development(base, tokens=300, experts=4, topk=2)]


@pytest.mark.parametrize("case", _dev_cases(), ids=lambda c: f"T{c.tokens}-E{c.experts}-H{c.hidden}")
def test_mx_layer_matches_oracle_on_development_geometry(case):
    _log(f"mx parity {case.id} T={case.tokens} H={case.hidden} I={case.intermediate} E={case.experts}")
    for seed in (104729, 104730):
        values = workloads.make_inputs(case, seed, "cpu")
        want, exact = mx.reference(case, values)["y"], mx.oracle(case, values)["y"]
        got = submission.build(case.to_dict())(_to(values, DEV))["y"].cpu()
        _check(case, got, want, exact)


def test_mx_layer_is_deterministic_and_does_not_mutate_inputs():
    case = C.development(C.case(MXCASE), tokens=24)
    _log("mx determinism")
    values = _to(workloads.make_inputs(case, 5, "cpu"), DEV)
    before = {k: v.clone() for k, v in values.items()}
    run = submission.build(case.to_dict())
    a, b = run(values)["y"], run(values)["y"]
    torch.cuda.synchronize()
    assert torch.equal(a, b)
    u8 = (lambda t: t.view(torch.uint8) if t.dtype == torch.float8_e4m3fn else t)
    for k, v in values.items():
        assert torch.equal(u8(v), u8(before[k])), k


@pytest.mark.parametrize("bad", ["out_of_range", "repeated"])
def test_mx_invalid_ids_give_nan(bad):
    case = C.development(C.case(MXCASE), tokens=8)
    _log(f"mx invalid ids {bad}")
    values = workloads.make_inputs(case, 6, "cpu")
    ids = values["topk_idx"].clone()
    if bad == "out_of_range":
        ids[3, 1] = case.experts
    else:
        ids[2, 1] = ids[2, 0]
    values["topk_idx"] = ids
    y = submission.build(case.to_dict())(_to(values, DEV))["y"].cpu()
    assert torch.isnan(y.float()).all()
    # A valid call on the same workspace afterwards is unaffected.
    good = workloads.make_inputs(case, 6, "cpu")
    y2 = submission.build(case.to_dict())(_to(good, DEV))["y"].cpu()
    assert torch.isfinite(y2.float()).all()


def test_mx_full_size_on_every_token():
    case = C.case(MXCASE)
    _log(f"mx full size {case.id}")
    values = workloads.make_inputs(case, 104729, DEV)
    got = submission.build(case.to_dict())(values)["y"]
    torch.cuda.synchronize()
    cpu = {k: v.cpu() for k, v in values.items()}
    del values
    torch.cuda.empty_cache()
    want, exact = mx.reference_and_oracle(case, cpu)
    check, band = _check(case, got.cpu(), want["y"], exact["y"])
    _log(f"  {case.id}: {check} band_rel={band['relative_error']:.3e}")


def _kernels_of(call):
    """call()'s result and the names of the device kernels it ran."""
    from torch.profiler import ProfilerActivity, profile

    with profile(activities=[ProfilerActivity.CPU, ProfilerActivity.CUDA]) as prof:
        out = call()
        torch.cuda.synchronize()
    return out, [e.name for e in prof.events() if e.device_type == torch.autograd.DeviceType.CUDA]


def test_rows_do_not_depend_on_the_kernel_mode():
    """A row's result depends only on the row and its expert: the same 8 tokens give the same
    bits in a call of 8 tokens (decode units, 16 rows per expert at most) and as the first 8
    of 200 tokens (100 rows per expert on average: batch units, chunks of 64 rows, the
    per-XCD queues). I = 4096 so both calls split the down units into 8 K parts of 2 stages
    (batch mode needs an even stage count per part)."""
    base = C.case(MXCASE)
    small = C.development(base, tokens=8, experts=4, topk=2, hidden=512, intermediate=4096)
    large = C.development(base, tokens=200, experts=4, topk=2, hidden=512, intermediate=4096)
    _log("mx mode independence")
    values = workloads.make_inputs(large, 31, "cpu")
    head = {k: (v[:8] if k in ("x", "x_scales", "topk_idx", "topk_weights") else v) for k, v in values.items()}
    y_small, small_kernels = _kernels_of(lambda: submission.build(small.to_dict())(_to(head, DEV))["y"])
    y_large, large_kernels = _kernels_of(lambda: submission.build(large.to_dict())(_to(values, DEV))["y"])
    assert any("k_experts_mx_batch" in k for k in large_kernels), large_kernels
    assert not any("k_experts_mx_batch" in k for k in small_kernels), small_kernels
    assert torch.equal(y_small, y_large[:8])
    want, exact = mx.reference(large, values)["y"], mx.oracle(large, values)["y"]
    _check(large, y_large.cpu(), want, exact)


@pytest.mark.parametrize("case", _dev_cases() + [C.case(MXCASE)], ids=lambda c: f"T{c.tokens}-E{c.experts}-H{c.hidden}")
def test_mx_single_launch_equals_stream_ordered(case):
    """megamoe_mx_layer_forward (one launch; the batch-shaped geometries take the stream-ordered
    kernels) gives megamoe_mx_forward's bits, over consecutive calls on one workspace."""
    _log(f"mx single launch {case.id} T={case.tokens} E={case.experts}")
    one = submission.MoELayer(case)
    three = submission.MoELayer(case, single_launch=False)
    assert one.single_launch and not three.single_launch
    for seed in (5, 6):
        values = workloads.make_inputs(case, seed, DEV)
        a, b = one(values)["y"], three(values)["y"]
        torch.cuda.synchronize()
        assert torch.equal(a, b), f"{case.id} seed {seed}"
        assert torch.isfinite(a.float()).all()
    assert not one.gave_up(torch.device(DEV))


def test_mx_one_call_is_one_kernel_launch():
    from torch.profiler import ProfilerActivity, profile

    case = C.development(C.case(MXCASE))
    values = _to(workloads.make_inputs(case, 3, "cpu"), DEV)
    run = submission.build(case.to_dict())
    run(values)  # the workspace is made (and zeroed) on the first call
    torch.cuda.synchronize()
    with profile(activities=[ProfilerActivity.CPU, ProfilerActivity.CUDA]) as prof:
        run(values)
        torch.cuda.synchronize()
    kernels = [e.name for e in prof.events() if e.device_type == torch.autograd.DeviceType.CUDA]
    _log(f"device events of one call: {kernels}")
    assert len(kernels) == 1 and "k_layer_mx" in kernels[0], kernels
    assert case.max_gpu_launches == 1


def _bad_ids_cases():
    base = C.case(MXCASE)
    # The decode geometry runs k_layer_mx; the batch-shaped one (100 rows per expert, an even
    # stage count per down part) makes megamoe_mx_layer_forward launch the stream-ordered
    # kernels, which must leave the outcome in the same status word.
    return [C.development(base, tokens=8),
            C.development(base, tokens=200, experts=4, topk=2, hidden=512, intermediate=4096)]


@pytest.mark.parametrize("case", _bad_ids_cases(), ids=lambda c: f"T{c.tokens}-E{c.experts}")
def test_mx_single_launch_reports_bad_ids(case):
    """Bad ids make y NaN and the status word say so; the next good call clears it."""
    _log(f"mx single launch bad ids {case.id} T={case.tokens} E={case.experts}")
    layer = submission.MoELayer(case)
    values = workloads.make_inputs(case, 6, "cpu")
    ids = values["topk_idx"].clone()
    ids[3, 1] = case.experts
    y, kernels = _kernels_of(lambda: layer(_to({**values, "topk_idx": ids}, DEV))["y"])
    batch = case.tokens * case.topk >= 24 * case.experts
    assert any(("k_experts_mx_batch" if batch else "k_layer_mx") in k for k in kernels), kernels
    assert torch.isnan(y.float()).all()
    assert layer.gave_up(torch.device(DEV))
    y2 = layer(_to(values, DEV))["y"]
    torch.cuda.synchronize()
    assert torch.isfinite(y2.float()).all()
    assert not layer.gave_up(torch.device(DEV))
