"""The FP8 MoE decode layer on the CPU, restated with the reference's rounding points
(test infrastructure).

Per token t (megabench/tasks/frontier.py:343-354, with ``linear`` of :180-186):
    scores      = fp32(router) @ fp32(x[t])                       (one GEMV per token)
    ids, w      = route(scores, bias)                              oracle/routing.py
    for slot, e in enumerate(ids):
        xq, xs  = E4M3 per 128 of x[t]                             quantization.py:87-109
        g, u    = bf16(deq(W_gate[e]) @ deq(xq, xs)), same for up  frontier.py:184-186
        h       = bf16(silu(fp32 g) * fp32 u)                      frontier.py:337
                  (case.swiglu "bf16": bf16(bf16(silu(g)) * u), frontier.py:338 and
                  glm53.py:174; case.swiglu_limit > 0: g, u clamped first, glm53.py:175)
        d       = bf16(deq(W_down[e]) @ deq(E4M3 per 128 of h))
                  (case.activations "bf16", W8A16, frontier.py:182-183 with
                  quantize=False: g, u = bf16(deq(W) @ fp32(x[t])), d = bf16(deq(W_down)
                  @ fp32(h)), nothing quantized)
        acc     = acc + fp32(d) * w[slot]                          frontier.py:349-350
    acc = acc + fp32(shared expert output)                          frontier.py:352
    y[t] = bf16(acc)                                                frontier.py:354 (without
                                                                    the residual add)

Softmax-routed cases use the same expert math with the routing of
megabench/tasks/references/moe.py:68-70.

The loops run per expert rather than per slot so each expert's weights are
dequantized once; every per-row product is still the same GEMV call the
reference makes per token, so the bits do not change. ``widen=True`` is the
FP32 oracle of megabench/tasks/oracle.py: the same graph with every BF16
rounding removed and the FP8 payloads and scales kept.

Pinned by tests/test_oracle_layer.py: an fp64 brute force with explicit loops
on small shapes (both schedules), planted mistakes it must catch (swapped
gate/up, dropped shared expert, SwiGLU sign, dropped slot), row independence
and the zero-down-projection invariant. The exact BF16 bits of the reference's
composed output depend on torch's CPU reduction order; they are not claimed
here, and the graded bars (band rule, max-rel, cosine) do not need them.
"""

from __future__ import annotations

import math

import numpy as np
import torch
import torch.nn.functional as F

from . import formats
from .routing import route


def _linear(w_deq: torch.Tensor, act: torch.Tensor, power_of_two: bool, out_dtype, quantize: bool = True
            ) -> torch.Tensor:
    """frontier.linear (frontier.py:180-186) with the weight already dequantized: W8A8 (the
    activation quantized to E4M3 per 128 first), or with quantize=False W8A16 (the activation
    as it is); an fp32 GEMV, one rounding."""
    if not quantize:
        return (w_deq @ act.float()).to(out_dtype)
    payload, scales = formats.pack_activation(act, power_of_two)
    return (w_deq @ formats.unpack_activation(payload, scales)).to(out_dtype)


def _swiglu(case, g: torch.Tensor, u: torch.Tensor, out_dtype) -> torch.Tensor:
    """g, u in out_dtype (bf16, or fp32 widened). With a limit, gate.clamp(max=L) and
    up.clamp(-L, L) first (glm53.py:175); then the "fp32" form rounds silu(g) * u once
    (frontier.py:337) and the "bf16" form is F.silu(gate) * up on the dtype itself, silu
    rounded before the product (frontier.py:338, glm53.py:174)."""
    limit = getattr(case, "swiglu_limit", 0.0)
    if limit > 0:
        g, u = g.clamp(max=limit), u.clamp(-limit, limit)
    if getattr(case, "swiglu", "fp32") == "bf16":
        return (F.silu(g) * u).to(out_dtype)
    return (F.silu(g.float()) * u.float()).to(out_dtype)


def _expert(values, name: str, index=None):
    q, s = values[name], values[name + "_scale"]
    if index is not None:
        q, s = q[index], s[index]
    return formats.unpack_weight(q, s)


@torch.no_grad()
def _layers(case, values: dict, widens, tokens=None) -> list[dict]:
    """The layer under each schedule of ``widens`` (False: BF16, True: FP32), sharing the
    routing (both schedules route the same fp32 scores of the bf16 input) and each hit
    expert's dequantized weights."""
    x = values["x"].cpu()
    rows = list(range(x.shape[0])) if tokens is None else list(tokens)
    router = values["router"].cpu().float()
    bias = values.get("router_bias")
    bias = None if bias is None else bias.cpu()
    pw = case.power_of_two

    ids, weights = [], []
    for t in rows:
        i, w = route(case, router @ x[t].float(), bias)
        ids.append(i)
        weights.append(w)
    ids_t = torch.stack(ids) if rows else torch.empty((0, case.topk), dtype=torch.int64)
    w_t = torch.stack(weights) if rows else torch.empty((0, case.topk), dtype=torch.float32)

    H = x.shape[1]
    modes = [(torch.float32 if widen else torch.bfloat16) for widen in widens]
    acts = [x.to(bf) for bf in modes]
    down = [{} for _ in modes]  # per mode: (row index, slot) -> [H]
    cpu = {k: v.cpu() for k, v in values.items() if k != "x"}

    q = getattr(case, "activations", "fp8") != "bf16"  # W8A8, or W8A16 (quantize=False)

    def mlp(wg, wu, wd, m, t):
        bf, act = modes[m], acts[m]
        h = _swiglu(case, _linear(wg, act[t], pw, bf, q), _linear(wu, act[t], pw, bf, q), bf)
        return _linear(wd, h, pw, bf, q)

    for e in sorted(set(ids_t.flatten().tolist())):
        wg, wu, wd = _expert(cpu, "gate", e), _expert(cpu, "up", e), _expert(cpu, "down", e)
        for r, t in enumerate(rows):
            for slot in (ids_t[r] == e).nonzero().flatten().tolist():
                for m in range(len(modes)):
                    down[m][(r, slot)] = mlp(wg, wu, wd, m, t)
    shared = [{} for _ in modes]
    if case.shared_experts:
        wg, wu, wd = _expert(cpu, "shared_gate"), _expert(cpu, "shared_up"), _expert(cpu, "shared_down")
        for r, t in enumerate(rows):
            for m in range(len(modes)):
                shared[m][r] = mlp(wg, wu, wd, m, t)

    out = []
    for m, bf in enumerate(modes):
        y = torch.empty((len(rows), H), dtype=bf)
        for r in range(len(rows)):
            acc = torch.zeros(H, dtype=torch.float32)
            for slot in range(case.topk):
                acc = acc + down[m][(r, slot)].float() * w_t[r, slot]
            if case.shared_experts:
                acc = acc + shared[m][r].float()
            y[r] = acc.to(bf)
        out.append({"y": y, "expert_ids": ids_t.clone(), "expert_weights": w_t.clone()})
    return out


def moe_layer(case, values: dict, *, widen: bool = False, tokens=None) -> dict:
    """Outputs {'y', 'expert_ids', 'expert_weights'} for ``tokens`` (default: all)."""
    return _layers(case, values, (widen,), tokens)[0]


def reference_and_oracle(case, values: dict, tokens=None) -> tuple[dict, dict]:
    """``reference`` and ``oracle`` in one pass (each hit expert dequantized once)."""
    want, exact = _layers(case, values, (False, True), tokens)
    return want, exact


def reference(case, values: dict, **kw) -> dict:
    """BF16 rounding schedule of the reference (the graded ``reference``)."""
    return moe_layer(case, values, widen=False, **kw)


def oracle(case, values: dict, **kw) -> dict:
    """FP32 oracle: the same graph without BF16 rounding (megabench/tasks/oracle.py:51-53)."""
    return moe_layer(case, values, widen=True, **kw)


def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float, weight_in_fp32: bool, *,
             widen: bool = False) -> torch.Tensor:
    """common.rms (megabench/tasks/common.py:13-21) for bf16 rows [T, H] and a bf16 gamma [H].

    The sum of squares is taken exactly (each square of a bf16 value is exact in fp64;
    ``math.fsum`` rounds the sum once); then, each operation rounded in fp32:
    m = fp32(s / H), r = 1 / sqrt(m + eps), n = fp32(x) * r, and
    out = bf16(n * w) (weight_in_fp32, the DeepSeek form) or bf16(bf16(n) * w).
    The reference takes the fp32 mean in torch's summation order and torch.rsqrt; the
    two differ from this by an ulp of r at most. ``widen`` drops the bf16 roundings (the
    FP32 oracle of megabench/tasks/oracle.py) and returns fp32.
    """
    xf = x.cpu().float().numpy()
    H = xf.shape[1]
    s = np.array([math.fsum((row.astype(np.float64) ** 2).tolist()) for row in xf], dtype=np.float64)
    m = (s / H).astype(np.float32)
    r = (np.float32(1.0) / np.sqrt((m + np.float32(eps)).astype(np.float32))).astype(np.float32)
    n = (xf * r[:, None]).astype(np.float32)
    w = weight.cpu().float().numpy()
    if widen:
        return torch.from_numpy(n * w)
    if not weight_in_fp32:
        n = torch.from_numpy(n).to(torch.bfloat16).float().numpy()
    return torch.from_numpy((n * w).astype(np.float32)).to(torch.bfloat16)


@torch.no_grad()
def block(case, values: dict, *, widen: bool = False, tokens=None) -> dict:
    """The decoder-block form (frontier.py:335-354): y = x + bf16(layer(rms(x, ln2))) when
    the case sets ``norm`` and ``residual``; ``widen`` is the FP32 oracle of the same graph."""
    x = values["x"].cpu()
    rows = list(range(x.shape[0])) if tokens is None else list(tokens)
    inner = dict(values)
    if case.norm != "none":
        inner["x"] = rms_norm(x, values["ln2"], case.norm_eps, case.norm == "fp32_weight", widen=widen)
    out = moe_layer(case, inner, widen=widen, tokens=tokens)
    if case.residual:
        res = x[rows].float() + out["y"].float()
        out["y"] = res if widen else res.to(torch.bfloat16)
    return out


def block_reference(case, values: dict, **kw) -> dict:
    return block(case, values, widen=False, **kw)


def block_oracle(case, values: dict, **kw) -> dict:
    return block(case, values, widen=True, **kw)
