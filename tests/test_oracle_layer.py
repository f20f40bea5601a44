"""Pins of the oracle's layer composition (CPU only).

The oracle's layer (oracle/layer.py) is compared with an fp64 brute force written
here with explicit loops: per-128 activation scales computed by hand, E4M3 codes from
the plain-C codec and decoded from the format's fields, every dot product in fp64,
and BF16 rounding (for the reference schedule) from the plain-C codec. Both pins are
independent of torch's FP8 cast and of the oracle's own packers.

Planted mistakes (in a patched copy of the oracle, on the CPU) show that the
comparison catches a swapped gate/up operand, a dropped shared expert, a wrong sign
in the SwiGLU and a dropped routed slot. Further invariants: each token's row depends
on that token only; zero down projections leave only the shared expert; the stable
permutation (oracle/codec.c) matches a sort.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import build as oracle_c
from oracle import layer, metrics, routing
from vibe_megakernel_amd import cases as C
from vibe_megakernel_amd import workloads

E4M3_TABLE = np.array([(-1.0 if c & 0x80 else 1.0) * (
    ((c & 7) / 8.0) * 2.0 ** -6 if ((c >> 3) & 15) == 0 else (1.0 + (c & 7) / 8.0) * 2.0 ** (((c >> 3) & 15) - 7))
    for c in range(256)])


def _bf16(v: np.ndarray) -> np.ndarray:
    bits = oracle_c.bf16_encode(np.asarray(v, dtype=np.float32))
    return (bits.astype(np.uint32) << 16).view(np.float32).astype(np.float64)


def _quant_act(v: np.ndarray) -> np.ndarray:
    """Dequantized per-128 E4M3 activation of a row (scale rule: max(amax, 1e-4) / 448)."""
    v32 = np.asarray(v, dtype=np.float32)
    out = np.empty(len(v32), dtype=np.float64)
    for b in range(0, len(v32), 128):
        blk = v32[b:b + 128]
        amax = np.float32(0.0)
        for e in blk:
            amax = max(amax, abs(e))
        s = np.float32(max(amax, np.float32(1e-4)) / np.float32(448.0))
        codes = oracle_c.e4m3_encode(np.clip(blk / s, -448, 448))
        out[b:b + 128] = E4M3_TABLE[codes] * np.float64(s)
    return out


def _weight(values, name, e=None) -> np.ndarray:
    q = values[name] if e is None else values[name][e]
    s = values[name + "_scale"] if e is None else values[name + "_scale"][e]
    codes = q.view(torch.uint8).numpy()
    full = np.repeat(np.repeat(s.double().numpy(), 128, 0), 128, 1)[:codes.shape[0], :codes.shape[1]]
    return E4M3_TABLE[codes] * full


def _mlp(wg, wu, wd, x, widen, quantize=True):
    """One expert on one row; quantize=False is the W8A16 form (x and h enter as they are)."""
    rnd = (lambda v: v.astype(np.float32).astype(np.float64)) if widen else _bf16
    act = _quant_act if quantize else (lambda v: v)
    xd = act(x)
    g, u = rnd(wg @ xd), rnd(wu @ xd)
    h = rnd(g / (1.0 + np.exp(-g)) * u)
    return rnd(wd @ act(h))


def brute_force(case, values, widen=False):
    x = values["x"].float()
    T, H = x.shape
    rnd = (lambda v: v.astype(np.float32).astype(np.float64)) if widen else _bf16
    xin = x.double().numpy() if widen else x.to(torch.bfloat16).double().numpy()
    q = case.activations != "bf16"
    y = np.zeros((T, H))
    for t in range(T):
        ids, w = routing.route(case, values["router"].float() @ x[t], values.get("router_bias"))
        acc = np.zeros(H)
        for slot, e in enumerate(ids.tolist()):
            d = _mlp(_weight(values, "gate", e), _weight(values, "up", e), _weight(values, "down", e), xin[t], widen,
                     q)
            acc += d * np.float64(w[slot])
        if case.shared_experts:
            acc += _mlp(_weight(values, "shared_gate"), _weight(values, "shared_up"), _weight(values, "shared_down"),
                        xin[t], widen, q)
        y[t] = rnd(acc)
    return torch.from_numpy(y)


def _cases():
    return [C.development(C.case("moe-fp8-deepseek-v3-t64"), tokens=5, experts=8, topk=3),
            C.development(C.case("moe-fp8-mixtral-t16"), tokens=4),
            C.development(C.case("moe-fp8-kimi-k2-t128"), tokens=3, experts=8),
            C.development(C.case("moe-fp8-deepseek-v3-t64-w8a16"), tokens=5, experts=8, topk=3),
            C.development(C.case("moe-fp8-deepseek-v3-t64-w8a16-ue8m0"), tokens=5, experts=8, topk=3)]


@pytest.mark.parametrize("case", _cases(), ids=lambda c: c.id)
def test_layer_matches_fp64_brute_force(case):
    values = workloads.make_inputs(case, 21, "cpu")
    ref, ora = layer.reference(case, values), layer.oracle(case, values)
    want_ref, want_ora = brute_force(case, values), brute_force(case, values, widen=True)
    # The BF16 schedule: fp32 vs fp64 accumulation moves a BF16 rounding or an E4M3 code
    # of h now and then; the widened oracle differs only by accumulation order.
    r = metrics.layer_checks(ref["y"], want_ref)
    o = metrics.layer_checks(ora["y"], want_ora)
    assert r["max_rel"] <= 4e-3 and r["cosine"] >= 0.99999, r
    assert o["max_rel"] <= 4e-3 and o["cosine"] >= 0.99999, o
    assert ref["expert_ids"].dtype == torch.int64 and ref["y"].dtype == torch.bfloat16
    assert ora["y"].dtype == torch.float32


class _Planted:
    """Context manager that patches one oracle internal with a wrong variant."""

    def __init__(self, kind):
        self.kind = kind

    def __enter__(self):
        self.saved = (layer._swiglu, layer._expert, layer.route)
        if self.kind == "swap_gate_up":
            orig = layer._expert
            layer._expert = lambda v, n, i=None: orig(v, {"gate": "up", "up": "gate"}.get(n, n), i)
        elif self.kind == "drop_shared":
            orig = layer._expert
            layer._expert = lambda v, n, i=None: orig(v, n, i) * (0.0 if n == "shared_down" else 1.0)
        elif self.kind == "silu_sign":
            layer._swiglu = lambda case, g, u, dt: (torch.nn.functional.silu(-g.float()) * u.float()).to(dt)
        elif self.kind == "drop_slot":
            orig = layer.route

            def route(case, scores, bias):
                ids, w = orig(case, scores, bias)
                w = w.clone()
                w[-1] = 0.0
                return ids, w
            layer.route = route
        return self

    def __exit__(self, *exc):
        layer._swiglu, layer._expert, layer.route = self.saved


@pytest.mark.parametrize("kind", ["swap_gate_up", "drop_shared", "silu_sign", "drop_slot"])
def test_brute_force_catches_planted_mistakes(kind):
    case = C.development(C.case("moe-fp8-deepseek-v3-t64"), tokens=3, experts=8, topk=3)
    values = workloads.make_inputs(case, 23, "cpu")
    want = brute_force(case, values)
    assert metrics.layer_checks(layer.reference(case, values)["y"], want)["pass"]
    with _Planted(kind):
        got = layer.reference(case, values)
    assert not metrics.layer_checks(got["y"], want)["pass"], kind


def test_w8a16_brute_force_catches_a_quantized_activation():
    """The W8A16 oracle quantizing x and h anyway (the W8A8 schedule) fails the W8A16 brute
    force: E4M3 moves each activation by up to 1/16 of its value."""
    case = C.development(C.case("moe-fp8-deepseek-v3-t64-w8a16"), tokens=3, experts=8, topk=3)
    values = workloads.make_inputs(case, 29, "cpu")
    want = brute_force(case, values)
    assert metrics.layer_checks(layer.reference(case, values)["y"], want)["pass"]
    w8a8 = layer.reference(C.development(C.case("moe-fp8-deepseek-v3-t64"), tokens=3, experts=8, topk=3), values)
    assert not metrics.layer_checks(w8a8["y"], want)["pass"]


def test_w8a16_linear_equals_w8a8_on_activations_the_e4m3_grid_holds():
    """frontier.linear's two forms agree bit for bit where quantizing changes nothing: each
    128-block of the activation is E4M3 values times 2^k with one element at +-448 * 2^k, so
    the scale is 2^k and every code is exact (quantization.py:57-59)."""
    g = torch.Generator().manual_seed(31)
    codes = torch.randint(0, 256, (512,), generator=g)
    codes[(codes & 0x7f) == 0x7f] = 0x70  # no NaN codes
    vals = torch.from_numpy(E4M3_TABLE[codes.numpy()]).float()
    vals[::128] = 448.0
    act = (vals * torch.repeat_interleave(2.0 ** torch.tensor([-3.0, 0.0, 2.0, -7.0]), 128)).to(torch.bfloat16)
    assert torch.equal(act.float(), vals * torch.repeat_interleave(2.0 ** torch.tensor([-3.0, 0.0, 2.0, -7.0]), 128))
    w = torch.randn((40, 512), generator=g)
    a8 = layer._linear(w, act, False, torch.bfloat16, True)
    a16 = layer._linear(w, act, False, torch.bfloat16, False)
    assert torch.equal(a8, a16)
    # Off the grid they differ (the activation moves).
    off = act.float() * 1.01
    assert not torch.equal(layer._linear(w, off.to(torch.bfloat16), False, torch.bfloat16, True),
                           layer._linear(w, off.to(torch.bfloat16), False, torch.bfloat16, False))


def test_rows_are_independent_and_token_subsets_agree():
    case = C.development(C.case("moe-fp8-deepseek-v3-t64"), tokens=6, experts=8, topk=3)
    values = workloads.make_inputs(case, 29, "cpu")
    full = layer.reference(case, values)
    part = layer.reference(case, values, tokens=[4, 1])
    assert torch.equal(part["y"], full["y"][[4, 1]])
    assert torch.equal(part["expert_ids"], full["expert_ids"][[4, 1]])


def test_zero_down_projections_leave_the_shared_expert():
    case = C.development(C.case("moe-fp8-deepseek-v3-t64"), tokens=3, experts=8, topk=3)
    values = workloads.make_inputs(case, 31, "cpu")
    values["down"] = torch.zeros_like(values["down"].view(torch.uint8)).view(torch.float8_e4m3fn)
    got = layer.reference(case, values)["y"]
    assert metrics.layer_checks(got, brute_force(case, values))["pass"]
    # Only the shared expert remains: its output alone, rounded once.
    x = values["x"].to(torch.bfloat16).double().numpy()
    shared = np.stack([_mlp(_weight(values, "shared_gate"), _weight(values, "shared_up"),
                            _weight(values, "shared_down"), x[t], False) for t in range(case.tokens)])
    assert torch.equal(got.double(), torch.from_numpy(_bf16(shared)))


def test_stable_permutation_matches_a_sort():
    g = torch.Generator().manual_seed(5)
    for T, K, E in ((64, 8, 256), (7, 3, 5), (1, 1, 1), (128, 8, 384)):
        ids = torch.stack([torch.randperm(E, generator=g)[:K] for _ in range(T)]).numpy()
        counts, offsets, perm, inv, hit = oracle_c.permute(ids, E)
        flat = ids.flatten()
        assert np.array_equal(counts, np.bincount(flat, minlength=E))
        assert offsets[0] == 0 and np.array_equal(np.diff(offsets), counts) and offsets[-1] == T * K
        assert np.array_equal(perm, np.argsort(flat, kind="stable"))
        assert np.array_equal(inv[perm], np.arange(T * K))
        assert hit == len(set(flat.tolist()))
    with pytest.raises(ValueError):
        oracle_c.permute(np.array([[0, 5]]), 5)


def test_brute_force_helpers_are_the_format():
    # 448 and the smallest subnormal decode as the format says; BF16 rounding keeps 8 bits.
    assert E4M3_TABLE[0x7E] == 448.0 and E4M3_TABLE[0x01] == 2.0 ** -9
    assert _bf16(np.array([1.0 + 2.0 ** -8]))[0] == 1.0  # tie to even
    assert _bf16(np.array([1.0 + 3 * 2.0 ** -8]))[0] == 1.0 + 2.0 ** -6
    assert math.isclose(_quant_act(np.full(128, 448.0))[0], 448.0)
