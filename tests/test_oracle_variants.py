"""Pins of the epilogue variants' restatements on the CPU.

SwiGLU forms (oracle/layer.py ``_swiglu``): against an fp64 brute force that rounds to bf16
from the bits (round half to even) at every point the form rounds, on every bf16 gate value
in [-16, 16] with random bf16 up values; planted mistakes (the DeepSeek single rounding for
the bf16 form, the clamp dropped, the clamp applied to the activation instead of its inputs,
up clamped on one side) must differ.

GPT-OSS combine (oracle/combine.py): against a numpy restatement with explicit bf16 rounding
of every product and sum, bit for bit; invariant under permutations of a token's slots;
planted mistakes (router rank order, fp32 accumulation, the residual added first) differ.
"""

from __future__ import annotations

from dataclasses import replace

import numpy as np
import pytest
import torch

from oracle import combine, layer
from vibe_megakernel_amd import cases as C
from vibe_megakernel_amd import workloads

GLM = C.case("moe-fp8-glm-5.3-flash-t64")


def bf16_round(x: np.ndarray) -> np.ndarray:
    """fp64 -> bf16 value (as fp64): round to nearest, ties to even, on the fp64 bits."""
    x = np.asarray(x, dtype=np.float64)
    m, e = np.frexp(x)                        # x = m * 2^e, 0.5 <= |m| < 1
    scaled = np.ldexp(m, 8)                   # 8 significant bits
    r = np.round(scaled)                      # numpy rounds half to even
    return np.ldexp(r, e - 8)


def all_bf16(lo: float, hi: float, tiny: float = 2.0 ** -12) -> np.ndarray:
    """Every bf16 value in [lo, hi] with magnitude 0 or at least ``tiny``. Below 2^-12 the
    fp32 silu of a bf16 gate is exactly g/2 (exp(-g) rounds to 1), so its products with bf16
    up values land on exact bf16 ties, which fp64 breaks the other way half the time."""
    bits = np.arange(0, 1 << 16, dtype=np.uint32) << 16
    v = bits.view(np.float32)
    v = v[np.isfinite(v)].astype(np.float64)
    v = v[(v >= lo) & (v <= hi) & ((np.abs(v) >= tiny) | (v == 0))]
    return np.unique(v)


def brute_swiglu(g: np.ndarray, u: np.ndarray, form: str, limit: float) -> np.ndarray:
    if limit > 0:
        g, u = np.minimum(g, limit), np.clip(u, -limit, limit)
    silu = g / (1.0 + np.exp(-g))
    if form == "bf16":
        return bf16_round(bf16_round(silu) * u)
    return bf16_round(silu * u)


def _grid(seed=0):
    g = all_bf16(-16.0, 16.0)
    rng = np.random.default_rng(seed)
    u = bf16_round(rng.normal(0, 6, g.size))
    return g, u


def _oracle_swiglu(form, limit, g, u):
    case = replace(GLM, swiglu=form, swiglu_limit=limit)
    gt = torch.tensor(g, dtype=torch.float32).to(torch.bfloat16)
    ut = torch.tensor(u, dtype=torch.float32).to(torch.bfloat16)
    return layer._swiglu(case, gt, ut, torch.bfloat16).double().numpy()


@pytest.mark.parametrize("form,limit", [("bf16", 10.0), ("bf16", 0.0), ("fp32", 10.0), ("fp32", 0.0)])
def test_swiglu_forms_against_brute_force(form, limit):
    g, u = _grid()
    got = _oracle_swiglu(form, limit, g, u)
    want = brute_swiglu(g, u, form, limit)
    assert np.array_equal(got, want), np.count_nonzero(got != want)


def test_planted_swiglu_mistakes_are_caught():
    g, u = _grid(1)
    got = _oracle_swiglu("bf16", 10.0, g, u)
    mistakes = {
        "single rounding": brute_swiglu(g, u, "fp32", 10.0),
        "no clamp": brute_swiglu(g, u, "bf16", 0.0),
        "clamp after": np.clip(brute_swiglu(g, u, "bf16", 0.0), -10, 10),
        "up clamped above only": bf16_round(bf16_round(np.minimum(g, 10) / (1 + np.exp(-np.minimum(g, 10))))
                                            * np.minimum(u, 10)),
    }
    for name, wrong in mistakes.items():
        assert np.count_nonzero(got != wrong) > 20, name


def test_glm_layer_clamp_is_exercised_and_matters():
    """With weights large enough for |g| > 10, the layer differs from the unclamped one."""
    case = replace(C.development(GLM), weight_std=0.5)
    values = workloads.make_inputs(case, 3, "cpu")
    clamped = layer.reference(case, values)["y"]
    free = layer.reference(replace(case, swiglu_limit=0.0), values)["y"]
    single = layer.reference(replace(case, swiglu="fp32"), values)["y"]
    assert not torch.equal(clamped, free) and not torch.equal(clamped, single)


def brute_combine(out, ids, w, residual):
    T, K, H = out.shape
    e = out.float().double().numpy()
    p = w.float().double().numpy()
    y = np.empty((T, H))
    for t in range(T):
        acc = np.zeros(H)
        for k in sorted(range(K), key=lambda k: int(ids[t, k])):
            acc = bf16_round(acc + bf16_round(p[t, k] * e[t, k]))
        y[t] = acc if residual is None else bf16_round(residual[t].float().double().numpy() + acc)
    return y


def _combine_inputs(T=9, K=6, H=64, E=40, seed=5):
    g = torch.Generator().manual_seed(seed)
    out = (torch.randn((T, K, H), generator=g) * 3).to(torch.bfloat16)
    ids = torch.stack([torch.randperm(E, generator=g)[:K] for _ in range(T)])
    w = torch.softmax(torch.randn((T, K), generator=g), -1).to(torch.bfloat16)
    res = torch.randn((T, H), generator=g).to(torch.bfloat16)
    return out, ids, w, res


@pytest.mark.parametrize("with_residual", [False, True])
def test_combine_by_expert_id_against_brute_force(with_residual):
    out, ids, w, res = _combine_inputs()
    r = res if with_residual else None
    got = combine.by_expert_id(out, ids, w, r).double().numpy()
    assert np.array_equal(got, brute_combine(out, ids, w, r))


def test_combine_by_expert_id_ignores_slot_order():
    out, ids, w, res = _combine_inputs(seed=6)
    perm = torch.randperm(ids.shape[1], generator=torch.Generator().manual_seed(1))
    a = combine.by_expert_id(out, ids, w, res)
    b = combine.by_expert_id(out[:, perm], ids[:, perm], w[:, perm], res)
    assert torch.equal(a, b)


def test_planted_combine_mistakes_are_caught():
    out, ids, w, res = _combine_inputs(T=32, K=8, H=256, seed=7)
    got = combine.by_expert_id(out, ids, w, res)
    rank_order = torch.empty_like(got)
    fp32_acc = torch.empty_like(got)
    residual_first = torch.empty_like(got)
    for t in range(out.shape[0]):
        o = torch.zeros(out.shape[2], dtype=torch.bfloat16)
        for k in range(out.shape[1]):
            o = o + w[t, k] * out[t, k]
        rank_order[t] = res[t] + o
        f = torch.zeros(out.shape[2])
        for k in ids[t].argsort().tolist():
            f = f + (w[t, k] * out[t, k]).float()
        fp32_acc[t] = res[t] + f.to(torch.bfloat16)
        o = res[t].clone()
        for k in ids[t].argsort().tolist():
            o = o + w[t, k] * out[t, k]
        residual_first[t] = o
    for name, wrong in (("rank order", rank_order), ("fp32 accumulation", fp32_acc),
                        ("residual first", residual_first)):
        assert not torch.equal(got, wrong), name
