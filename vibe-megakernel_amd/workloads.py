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
from dataclasses import replace

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
    """E4M3 payload [..., R, C] and fp32 scales [..., ceil(R/128), ceil(C/128)] of fp32
    matrices [..., R, C] (any leading batch dimensions, e.g. a batch of experts)."""
    rows, cols = w.shape[-2:]
    lead = w.shape[:-2]
    pr, pc = (-rows) % BLOCK, (-cols) % BLOCK
    padded = torch.nn.functional.pad(w.float(), (0, pc, 0, pr)) if pr or pc else w.float()
    br, bc = padded.shape[-2] // BLOCK, padded.shape[-1] // BLOCK
    blocks = padded.view(*lead, br, BLOCK, bc, BLOCK)
    amax = blocks.abs().amax(dim=(-3, -1))
    scale = amax.clamp_min(1e-4) / 448.0
    if power_of_two:
        scale = torch.exp2(torch.ceil(torch.log2(scale)))
    q = (blocks / scale[..., :, None, :, None]).clamp_(-448.0, 448.0).to(torch.float8_e4m3fn)
    q = q.view(padded.shape)
    if pr or pc:
        q = q[..., :rows, :cols].contiguous()
    return q, scale


# Expert stacks are generated in batches of at most this many fp32 bytes (one randn and one
# batched quantization per batch, a few dozen kernels per stack instead of ~20 per expert).
STACK_BATCH_BYTES = 2 << 30


def _expert_stack(seed, name, experts, rows, cols, std, device, power_of_two, log=None):
    """E4M3 stack [experts, rows, cols] and its scales. One generator per stack, seeded from
    (seed, name), draws the experts in order, in batches whose size depends on the matrix
    shape only, so a (seed, case) pair always yields the same stack."""
    payload = torch.empty((experts, rows, cols), dtype=torch.float8_e4m3fn, device=device)
    scales = torch.empty((experts, -(-rows // BLOCK), -(-cols // BLOCK)), dtype=torch.float32, device=device)
    gen = torch.Generator(device=device).manual_seed(seed_for(seed, name))
    per = max(1, min(experts, STACK_BATCH_BYTES // (4 * rows * cols)))
    for e0 in range(0, experts, per):
        n = min(per, experts - e0)
        w = torch.randn((n, rows, cols), generator=gen, device=device, dtype=torch.float32).mul_(std)
        q, s = quantize_weight(w, power_of_two)
        del w
        payload[e0:e0 + n].copy_(q)
        scales[e0:e0 + n].copy_(s)
        del q, s
    if log:
        log(f"{name}: {experts} x [{rows}, {cols}] E4M3 in {-(-experts // per)} batch(es)")
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


# -- MXFP4 form (megamoe.py numerics) ---------------------------------------------------

MX = 32       # E8M0 block of the MXFP4 weights and of the E4M3 activations
L1_GAIN = 4   # gate/up outputs of std ~4, so ~1% of them reach the SwiGLU clamp of 10 (megamoe.py:41)


def pack_mxfp4(m: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """E2M1 codes packed two per byte (even element in the low nibble) [..., n/32, 16] and
    E8M0 scales [..., n/32] of an fp32 matrix (the format of quantization.py:13-40): scale
    exponent ceil(log2(amax/6)) clamped to [-126, 127], codes rounded to nearest with ties
    to the even code. The rounding runs per binade of the E2M1 grid: steps of 1/2 below 2,
    of 1 up to 4, of 2 up to 6, each a half-to-even round of the scaled magnitude."""
    g = m.float().unflatten(-1, (-1, MX))
    amax = g.abs().amax(-1)
    e = torch.ceil(torch.log2((amax / 6.0).clamp_min(2.0 ** -126))).clamp(-126, 127).to(torch.int32)
    n = torch.ldexp(g, -e[..., None].float())
    a = n.abs()
    mag = torch.where(a < 2.0, torch.round(a * 2.0) / 2.0,
                      torch.where(a < 4.0, torch.round(a), torch.round(a / 2.0) * 2.0))
    # magnitude -> code: 0, .5, 1, 1.5, 2 -> 0..4; 3 -> 5; 4 -> 6; 6 -> 7
    code = torch.where(mag <= 2.0, mag * 2.0, torch.where(mag == 3.0, 5.0, torch.where(mag == 4.0, 6.0, 7.0)))
    code = code.to(torch.uint8) | ((n < 0).to(torch.uint8) << 3)
    return (code[..., 0::2] | (code[..., 1::2] << 4)).contiguous(), (e + 127).to(torch.uint8)


def pack_e4m3_e8m0(v: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """E4M3 payload and E8M0 scale exponents per row per 32 columns (quantization.py:67-109,
    scale_format='e8m0'): the exponent comes from the fp32 bits of the block amax, raised by
    one where its mantissa exceeds 1.75's, less 448's exponent, floored at 1e-4/448's."""
    g = v.float().unflatten(-1, (-1, MX))
    bits = g.abs().amax(-1).contiguous().view(torch.int32).to(torch.int64)
    e = (((bits + (0x7FFFFF - 0x600000)) >> 23).clamp_min(105 + 8) - 8).to(torch.int32)
    inv = ((254 - e) << 23).view(torch.float32)
    return (g * inv[..., None]).to(torch.float8_e4m3fn).flatten(-2).contiguous(), e.to(torch.uint8)


def mx_routing(case: Case, seed: int, device) -> tuple[torch.Tensor, torch.Tensor]:
    """Distinct experts per token from a log-normal popularity plus Gumbel noise (top-k),
    weights sqrt(softplus(N(0,1))) normalized to the routed scaling (the scheme of
    megamoe.py:59-73, with this build's own seeded streams)."""
    T, E, K = case.tokens, case.experts, case.topk
    pop = _normal(seed, "expert_popularity", (E,), 0.4, device)
    gen = torch.Generator(device=device).manual_seed(seed_for(seed, "route_noise"))
    u = torch.rand((T, E), generator=gen, device=device).clamp(1e-12, 1 - 1e-7)
    idx = (pop + (-torch.log(-torch.log(u)))).topk(K, -1).indices
    score = torch.nn.functional.softplus(_normal(seed, "route_logits", (T, K), 1.0, device)).sqrt()
    return idx.to(torch.int64).contiguous(), (score / score.sum(-1, keepdim=True) * case.routed_scaling).contiguous()


def _mx_experts(case: Case, seed: int, first: int, count: int, device) -> dict[str, torch.Tensor]:
    """MXFP4 weights of experts [first, first + count), each from its own global id's stream."""
    H, I = case.hidden, case.intermediate
    values = {}
    for name, rows, cols, std in (("l1", 2 * I, H, L1_GAIN / H ** 0.5), ("l2", H, I, 1.0 / I ** 0.5)):
        blocks = torch.empty((count, rows, cols // MX, MX // 2), dtype=torch.uint8, device=device)
        scales = torch.empty((count, rows, cols // MX), dtype=torch.uint8, device=device)
        for e in range(count):
            blocks[e], scales[e] = pack_mxfp4(_normal(seed, f"{name}:{first + e}", (rows, cols), std, device))
        values[name + "_blocks"], values[name + "_scales"] = blocks, scales
    return values


def make_mx_inputs(case: Case, seed: int, device="cpu") -> dict[str, torch.Tensor]:
    T, H, E = case.tokens, case.hidden, case.experts
    values = {}
    values["x"], values["x_scales"] = pack_e4m3_e8m0(_normal(seed, "x", (T, H), 1.0, device))
    values["topk_idx"], values["topk_weights"] = mx_routing(case, seed, device)
    values.update(_mx_experts(case, seed, 0, E, device))
    return values


def serial_case(case: Case) -> Case:
    """The single-rank problem of an EP case: every rank's tokens, every expert
    (megabench/verify_megamoe.py:39-40)."""
    return replace(case, gpus=1, ep=1, params=dict(case.params, tokens=case.tokens * case.ep))


def make_ep_inputs(case: Case, seed: int, device="cpu", rank: int = 0) -> dict[str, torch.Tensor]:
    """Inputs of rank ``rank``'s share: x, x_scales, topk_idx and topk_weights of the serial
    problem (all ep * T tokens; rank r's own are rows [r*T, (r+1)*T)) and the MXFP4 weights
    of the rank's local experts [rank*E/ep, (rank+1)*E/ep) only. Every rank's tokens and
    weights are the serial problem's (make_mx_inputs of serial_case), as the reference's rank
    inputs are (megabench/tests/test_megamoe.py:150-158)."""
    serial = serial_case(case)
    local = case.experts // case.ep
    values = {}
    values["x"], values["x_scales"] = pack_e4m3_e8m0(_normal(seed, "x", (serial.tokens, case.hidden), 1.0, device))
    values["topk_idx"], values["topk_weights"] = mx_routing(serial, seed, device)
    values.update(_mx_experts(case, seed, rank * local, local, device))
    return values


def make_inputs(case: Case, seed: int, device="cpu", log=None) -> dict[str, torch.Tensor]:
    """Inputs of ``case``; ``log`` (a callable taking a line of text, or None) hears one line
    per weight stack as it is made."""
    if case.format == "mxfp4":
        return make_mx_inputs(case, seed, device)
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
        values[name], values[name + "_scale"] = _expert_stack(seed, name, E, rows, cols, std, device, pw, log)
    if S:
        for name, rows, cols in (("shared_gate", S * I, H), ("shared_up", S * I, H), ("shared_down", H, S * I)):
            values[name], values[name + "_scale"] = quantize_weight(
                _normal(seed, name, (rows, cols), std, device), pw)
            if log:
                log(f"{name}: [{rows}, {cols}] E4M3")
    return values


def input_names(case: Case) -> list[str]:
    if case.format == "mxfp4":
        return ["x", "x_scales", "topk_idx", "topk_weights", "l1_blocks", "l1_scales", "l2_blocks", "l2_scales"]
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
