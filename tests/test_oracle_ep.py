"""Pins of the expert-parallel restatement (oracle/ep.py) on the CPU.

The send order is checked against a per-owner listing by brute force, the counts against
the listing's sizes, and the whole emulation of ep ranks against the serial MXFP4 layer of
oracle/mx.py bit for bit (the check megabench/verify_megamoe.py:95-105 makes between the EP
and serial runs, at its development geometry, :32). A mistake in the owner rule, the
stability of the order, the segment bookkeeping of either exchange or the slot order of the
combine moves rows between tokens or slots and fails the equality.
"""

from __future__ import annotations

from dataclasses import replace

import numpy as np
import pytest
import torch

from oracle import ep as OE
from oracle import mx as OM
from vibe_megakernel_amd import cases as C
from vibe_megakernel_amd import workloads as W

EP_CASE = C.case("megamoe-layer-deepseek-v4-pro-ep8-t512")


def _dev(ranks: int, tokens: int = 8) -> C.Case:
    """The reference's development geometry (verify_megamoe.py:32), intermediate raised to
    256 so the same geometry also runs on the GPU."""
    return replace(EP_CASE, id=f"ep-dev-{ranks}", gpus=ranks, ep=ranks,
                   params=dict(tokens=tokens, experts=16, topk=4, hidden=256, intermediate=256))


@pytest.mark.parametrize("ep", [1, 2, 4, 8, 16])
def test_send_order_is_stable_by_owner(ep):
    rng = np.random.default_rng(ep)
    ids = np.stack([rng.permutation(32)[:5] for _ in range(40)])
    local = 32 // ep
    order = OE.owner_order(ids, local)
    flat = ids.reshape(-1)
    brute = [i for o in range(ep) for i in range(flat.size) if flat[i] // local == o]
    assert order.tolist() == brute


def test_dispatch_payload_counts_and_slot_rows():
    case = _dev(4)
    values = W.make_mx_inputs(W.serial_case(case), 3)
    send = OE.dispatch(values, case.experts, case.ep)
    ids = values["topk_idx"]
    T, K = ids.shape
    local = case.experts // case.ep
    owners = (ids // local).reshape(-1).tolist()
    assert send["counts"].tolist() == [owners.count(o) for o in range(case.ep)]
    for t in range(T):
        for k in range(K):
            p = int(send["slot_rows"][t, k])
            assert int(send["ids"][p]) == int(ids[t, k])
            assert float(send["weights"][p]) == float(values["topk_weights"][t, k])
            assert torch.equal(send["rows"][p], values["x"][t].view(torch.uint8))
            assert torch.equal(send["row_scales"][p], values["x_scales"][t])
    # Each destination's segment holds its rows only, in (token, slot) order.
    starts = np.concatenate(([0], np.cumsum(send["counts"])))
    source = np.empty(T * K, dtype=np.int64)
    source[send["slot_rows"].reshape(-1).numpy()] = np.arange(T * K)
    for o in range(case.ep):
        seg = slice(int(starts[o]), int(starts[o + 1]))
        assert all(int(i) // local == o for i in send["ids"][seg])
        assert np.all(np.diff(source[seg]) > 0)


@pytest.mark.parametrize("ranks", [1, 2, 4, 8])
def test_expert_parallel_equals_serial_bitwise(ranks):
    case = _dev(ranks)
    serial = W.serial_case(case)
    values = W.make_mx_inputs(serial, 5)
    expected = OM.reference(serial, values)["y"]
    actual = OE.emulate(case, values, ranks)
    assert actual.dtype == torch.bfloat16 and actual.shape == expected.shape
    assert torch.equal(actual, expected)


def test_expert_parallel_widened_equals_serial_oracle():
    case = _dev(4)
    serial = W.serial_case(case)
    values = W.make_mx_inputs(serial, 6)
    assert torch.equal(OE.emulate(case, values, 4, widen=True), OM.oracle(serial, values)["y"])


def test_a_misplaced_return_is_caught():
    """A combine that reads the returned rows of the wrong token differs from the serial
    layer. (The slot order of the fp32 sum is not observable here: a sum of four bf16 rows
    is nearly always exact in fp32.)"""
    case = _dev(2)
    serial = W.serial_case(case)
    values = W.make_mx_inputs(serial, 7)
    expected = OM.reference(serial, values)["y"]
    original = OE.combine

    def reversed_combine(returned, slot_rows):
        return original(returned, slot_rows.roll(1, dims=0))

    try:
        OE.combine = reversed_combine
        moved = OE.emulate(case, values, 2)
    finally:
        OE.combine = original
    assert not torch.equal(moved, expected)


def test_rank_inputs_are_the_serial_problem():
    """Each rank's share holds the serial problem's tokens and its local experts' weights
    (megabench/tests/test_megamoe.py:150-158)."""
    case = _dev(4)
    whole = W.make_mx_inputs(W.serial_case(case), 9)
    local = case.experts // case.ep
    for rank in range(case.ep):
        part = W.make_ep_inputs(case, 9, rank=rank)
        for name in ("x", "x_scales", "topk_idx", "topk_weights"):
            a, b = whole[name], part[name]
            if a.dtype == torch.float8_e4m3fn:
                a, b = a.view(torch.uint8), b.view(torch.uint8)
            assert torch.equal(a, b), name
        for name in ("l1_blocks", "l1_scales", "l2_blocks", "l2_scales"):
            assert torch.equal(whole[name][rank * local:(rank + 1) * local], part[name]), name


def test_catalog_share_geometry():
    c = EP_CASE
    assert (c.gpus, c.ep, c.tokens, c.experts, c.topk, c.hidden, c.intermediate) == (8, 8, 512, 384, 6, 7168, 3072)
    assert c.experts % c.ep == 0 and W.serial_case(c).tokens == 4096
