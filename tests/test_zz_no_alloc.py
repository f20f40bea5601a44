"""megamoe_forward_noalloc on the GPU, through the C ABI: its outputs equal megamoe_forward's
bit for bit on two calls in a row, the second with fewer tokens (the scratch keeps the first
call's contents, which must not matter). The refusal of a geometry beyond the scratch is
checked on the CPU (tests/test_abi.py)."""

from __future__ import annotations

import sys

import pytest
import torch

from vibe_megakernel_amd import _lib
from vibe_megakernel_amd import cases as C
from vibe_megakernel_amd import submission, workloads

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _log(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _to(values):
    return {k: v.to(DEV) for k, v in values.items()}


def _same(a: dict, b: dict, what: str):
    for k in ("y", "expert_ids", "expert_weights"):
        assert torch.equal(a[k], b[k]), f"{what}: {k} differs"


def test_noalloc_equals_forward_on_two_calls_the_second_smaller():
    # First call: Kimi-K2's geometry with 64 experts (a 22 MiB workspace of the 32 MiB
    # scratch); second: a 20-token DeepSeek-V3-routed development geometry (0.3 MiB).
    kimi = C.case("moe-fp8-kimi-k2-t128")
    big = C.Case.from_dict({**kimi.to_dict(), "id": "kimi-k2-e64", "params": {**kimi.params, "experts": 64}})
    small = C.development(C.case(C.HEADLINE), tokens=20)
    sizes = []
    for case, seed in ((big, 41), (small, 42)):
        layer = submission.MoELayer(case, single_launch=False)  # megamoe_forward, the existing entry
        sizes.append(layer.workspace_bytes)
        assert layer.workspace_bytes <= _lib.SCRATCH_BYTES
        _log(f"noalloc {case.id} T={case.tokens} E={case.experts} workspace={layer.workspace_bytes}")
        values = workloads.make_inputs(case, seed, DEV) if case is big else _to(workloads.make_inputs(case, seed, "cpu"))
        want = layer(values)
        got = layer.noalloc(values)
        torch.cuda.synchronize()
        _same(got, want, case.id)
        assert torch.isfinite(got["y"].float()).all()
        del values
        torch.cuda.empty_cache()
    assert sizes[1] < sizes[0]
