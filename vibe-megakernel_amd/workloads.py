"""Seeded synthetic inputs of the FP8 MoE decode layer.

``make_inputs(case, seed, device)`` mirrors the reference's task-dispatcher
call (megabench/tasks/workloads.py:30-36). Tensor names follow the reference's
FP8 MoE inputs (megabench/tasks/frontier.py:157-176): ``router``,
``router_bias``, ``gate``/``up``/``down`` expert stacks with ``*_scale`` block
scales, and ``shared_gate``/``shared_up``/``shared_down``.

Every tensor draws from its own generator, seeded from (seed, name) with a
64-bit BLAKE2b digest, so tensors are independent of each other and of the
order they are built in (the scheme of megabench/tasks/distributed.py:25-26).
The stream depends on ``device``: the CPU and GPU generators of PyTorch
produce different numbers, so fixtures are generated on the CPU, and full-size
GPU runs generate on the GPU and copy what a check needs to the host.

Weights are N(0, std) in fp32, quantized to E4M3 with one fp32 scale per
128x128 block: scale = max(block amax, 1e-4) / 448, payload = RNE(clamp(W /
scale, +-448)) (the rule of megabench/tasks/quantization.py:57-59,119-126).
"""

from __future__ import annotations

import hashlib

import torch

from .cases import Case

BLOCK = 128


def seed_for(seed: int, name: str) -> int:
    digest = hashlib.blake2b(f"{seed}/{name}".encode(), digest_size=8).digest()
    return int.from_bytes(digest, "little") & ((1 << 63) - 1)


def _normal(seed: int, name: str, shape, std: float, device) -> torch.Tensor:
    gen = torch.Generator(device=device).manual_seed(seed_for(seed, name))
    return torch.randn(shape, generator=gen, device=device, dtype=torch.float32) * std


def quantize_weight(w: torch.Tensor, power_of_two: bool = False) -> tuple[torch.Tensor, torch.Tensor]:
    """E4M3 payload [R, C] and fp32 scales [ceil(R/128), ceil(C/128)] of an fp32 matrix."""
    rows, cols = w.shape
    pr, pc = (-rows) % BLOCK, (-cols) % BLOCK
    padded = torch.nn.functional.pad(w.float(), (0, pc, 0, pr))
    blocks = padded.view(padded.shape[0] // BLOCK, BLOCK, padded.shape[1] // BLOCK, BLOCK)
    amax = blocks.abs().amax(dim=(1, 3))
    scale = amax.clamp_min(1e-4) / 448.0
    if power_of_two:
        scale = torch.exp2(torch.ceil(torch.log2(scale)))
    q = (blocks / scale[:, None, :, None]).clamp(-448.0, 448.0).to(torch.float8_e4m3fn)
    return q.view(padded.shape)[:rows, :cols].contiguous(), scale


def _expert_stack(seed, name, experts, rows, cols, std, device, power_of_two):
    payload = torch.empty((experts, rows, cols), dtype=torch.float8_e4m3fn, device=device)
    scales = torch.empty((experts, -(-rows // BLOCK), -(-cols // BLOCK)), dtype=torch.float32, device=device)
    for e in range(experts):
        q, s = quantize_weight(_normal(seed, f"{name}:{e}", (rows, cols), std, device), power_of_two)
        payload[e].copy_(q)
        scales[e].copy_(s)
    return payload, scales


def router_bias(case: Case, seed: int, device) -> torch.Tensor | None:
    E = case.experts
    if case.bias == "none":
        return None
    if case.bias == "normal":
        return _normal(seed, "router_bias", (E,), case.bias_std, device)
    # Zipf: the expert at rank r (1-based, over a seeded permutation) gets c * r^-s.
    gen = torch.Generator(device="cpu").manual_seed(seed_for(seed, "router_bias_rank"))
    order = torch.randperm(E, generator=gen)
    ranks = torch.empty(E, dtype=torch.float64)
    ranks[order] = torch.arange(1, E + 1, dtype=torch.float64)
    return (case.zipf_c * ranks.pow(-case.zipf_s)).float().to(device)


def make_inputs(case: Case, seed: int, device="cpu") -> dict[str, torch.Tensor]:
    T, H, E, I, S = case.tokens, case.hidden, case.experts, case.intermediate, case.shared_experts
    std, pw = case.weight_std, case.power_of_two
    values: dict[str, torch.Tensor] = {}
    values["x"] = _normal(seed, "x", (T, H), 1.0, device).to(torch.bfloat16)
    if case.norm != "none":  # the block's ln2 gamma, 1 + N(0, 0.1) in bf16 as frontier.py:87
        values["ln2"] = (_normal(seed, "ln2", (H,), 0.1, device) + 1.0).to(torch.bfloat16)
    values["router"] = _normal(seed, "router", (E, H), case.router_std, device)
    bias = router_bias(case, seed, device)
    if bias is not None:
        values["router_bias"] = bias
    for name, rows, cols in (("gate", I, H), ("up", I, H), ("down", H, I)):
        values[name], values[name + "_scale"] = _expert_stack(seed, name, E, rows, cols, std, device, pw)
    if S:
        for name, rows, cols in (("shared_gate", S * I, H), ("shared_up", S * I, H), ("shared_down", H, S * I)):
            values[name], values[name + "_scale"] = quantize_weight(
                _normal(seed, name, (rows, cols), std, device), pw)
    return values


def input_names(case: Case) -> list[str]:
    names = ["x", "router"]
    if case.norm != "none":
        names.append("ln2")
    if case.bias != "none":
        names.append("router_bias")
    for n in ("gate", "up", "down"):
        names += [n, n + "_scale"]
    if case.shared_experts:
        for n in ("shared_gate", "shared_up", "shared_down"):
            names += [n, n + "_scale"]
    return names


OUTPUTS = ("y", "expert_ids", "expert_weights")
