"""MXFP4 / UE8M0 numerics of the routed-expert layer, restated on the CPU (test infrastructure).

Formats (megabench/tasks/quantization.py):
  * MXFP4 (:13-51): groups of 32 along the last axis; E8M0 scale 2^(e-127) with
    e = ceil(log2(max(amax / 6, 2^-126))) clamped to [-126, 127] (+127 bias); E2M1 codes
    (sign, 2 exponent bits, 1 mantissa bit: magnitudes 0, .5, 1, 1.5, 2, 3, 4, 6) by
    round-to-nearest with ties to the even code; two codes per byte, the even element in
    the low nibble; packed [..., n/32, 16], scales [..., n/32].
  * E8M0 activation scales (:67-84): the biased exponent from the fp32 bits of the block
    amax, rounded up where its mantissa exceeds 1.75's, minus 448's exponent, floored at
    the exponent of 1e-4/448's; payload = E4M3(x * 2^(127-e)).

The layer (megabench/tasks/megamoe.py:116-182, serial): routing is an input. For each
(token, slot) row, grouped by expert in (token, slot) order:
    l1   = bf16(x @ unpack(l1).T)          x = E4M3 * 2^(e-127), exact in bf16
    gate, up = l1[:, :I], l1[:, I:];  gate = min(gate, limit);  up = clamp(up, +-limit)
    a    = gate / (1 + exp(-gate)) * up * w_slot          (fp32)
    h    = E4M3 per 32 with E8M0 scales of a, dequantized  (exact in bf16)
    d    = bf16(h @ unpack(l2).T)
    y[t] = bf16(sum over slots in order of fp32(d))
``widen=True`` is the FP32 oracle of the same graph: no bf16 roundings and no requant of
h (as the reference's own test widens it: test_megamoe.py:140-143).

Pinned by tests/test_oracle_mx.py: every E2M1 code decoded from its fields, every
midpoint rounded to the even code, the scale rule's minimality and clamps, the E8M0
exponent against DeepGEMM's ceil-to-UE8M0 rule and the edge vectors of
megabench/tests/test_megamoe.py:56-65, and the widened layer against transformers'
DeepseekV4Experts (the check of test_megamoe.py:128-148).
"""

from __future__ import annotations

import numpy as np
import torch

MX_BLOCK = 32
E2M1 = (0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0)
E4M3_MAX_EXPONENT = 8          # 448 = 1.75 * 2^8
E4M3_MAX_MANTISSA = 0x600000   # fp32 mantissa bits of 1.75
E8M0_MIN = 105                 # biased exponent of 2^-22, the scale of the 1e-4 amax floor


def e2m1_value(code: int) -> float:
    """E2M1 decoded from its fields: sign bit 3, exponent bits 2-1 (bias 1), mantissa bit 0."""
    sign = -1.0 if code & 8 else 1.0
    exp, man = (code >> 1) & 3, code & 1
    mag = (man * 0.5) if exp == 0 else (1.0 + 0.5 * man) * 2.0 ** (exp - 1)
    return sign * mag


def _round_e2m1(mag: np.ndarray) -> np.ndarray:
    """Code (0..7) of the nearest E2M1 magnitude, ties to the even code."""
    grid = np.array(E2M1, dtype=np.float64)
    d = np.abs(mag[..., None].astype(np.float64) - grid)
    best = d.min(-1, keepdims=True)
    cand = d == best
    # On a tie two adjacent codes qualify: take the even one.
    even = cand & (np.arange(8) % 2 == 0)
    return np.where(even.any(-1), even.argmax(-1), cand.argmax(-1)).astype(np.uint8)


def pack_mxfp4(matrix: torch.Tensor):
    """(packed uint8 [..., n/32, 16], scales uint8 [..., n/32]) of an fp32 matrix."""
    x = matrix.detach().cpu().float().numpy()
    if x.shape[-1] % MX_BLOCK:
        raise ValueError("the MXFP4 block axis must be a multiple of 32")
    g = x.reshape(*x.shape[:-1], -1, MX_BLOCK)
    amax = np.abs(g).max(-1)
    e = np.ceil(np.log2(np.maximum(amax / 6.0, 2.0 ** -126)))
    e = np.clip(e, -126, 127).astype(np.int32)
    norm = g * np.exp2(-e.astype(np.float64))[..., None]
    codes = _round_e2m1(np.abs(norm)) | ((norm < 0).astype(np.uint8) << 3)
    packed = codes[..., 0::2] | (codes[..., 1::2] << 4)
    return torch.from_numpy(packed.astype(np.uint8)), torch.from_numpy((e + 127).astype(np.uint8))


def unpack_mxfp4(packed: torch.Tensor, scales: torch.Tensor) -> torch.Tensor:
    """fp32 [..., n] (E8M0 255 decodes to NaN)."""
    p = packed.cpu().numpy()
    lut = np.array([e2m1_value(c) for c in range(16)], dtype=np.float32)
    codes = np.stack([p & 15, p >> 4], -1).reshape(*p.shape[:-1], MX_BLOCK)
    s = scales.cpu().numpy().astype(np.int32)
    vals = lut[codes] * np.exp2((s - 127).astype(np.float32))[..., None]
    vals = np.where((s == 255)[..., None], np.float32(np.nan), vals)
    return torch.from_numpy(vals.reshape(*p.shape[:-2], -1).astype(np.float32))


def e8m0_exponent(amax: torch.Tensor) -> torch.Tensor:
    """Biased E8M0 exponent (uint8) that maps ``amax`` into E4M3, from the fp32 bits."""
    bits = amax.float().contiguous().view(torch.int32).to(torch.int64)
    rounded = (bits + (0x7FFFFF - E4M3_MAX_MANTISSA)) >> 23
    return (rounded.clamp_min(E8M0_MIN + E4M3_MAX_EXPONENT) - E4M3_MAX_EXPONENT).to(torch.uint8)


def e8m0_power(e: torch.Tensor, inverse: bool = False) -> torch.Tensor:
    """Exact fp32 2^(e-127), or its reciprocal, from the exponent bits."""
    b = e.to(torch.int32)
    b = 254 - b if inverse else b
    return (b << 23).view(torch.float32)


def pack_activation_e8m0(value: torch.Tensor, block: int = MX_BLOCK):
    """E4M3 payload and E8M0 scales per row per ``block`` columns (quantization.py:87-109,
    scale_format='e8m0'); padding counts as zero."""
    width = value.shape[-1]
    g = torch.nn.functional.pad(value.float(), (0, (-width) % block)).unflatten(-1, (-1, block))
    e = e8m0_exponent(g.abs().amax(-1))
    payload = (g * e8m0_power(e, inverse=True)[..., None]).to(torch.float8_e4m3fn)
    return payload.flatten(-2)[..., :width].contiguous(), e


def unpack_activation_e8m0(payload: torch.Tensor, scales: torch.Tensor, block: int = MX_BLOCK) -> torch.Tensor:
    return payload.float() * e8m0_power(scales).repeat_interleave(block, dim=-1)[..., :payload.shape[-1]]


def swiglu_clamped(l1: torch.Tensor, weights: torch.Tensor, limit: float) -> torch.Tensor:
    """megamoe.py:116-122: clamp in the input dtype, then fp32 (gate * sigmoid) * up * w."""
    gate, up = l1.chunk(2, dim=-1)
    gate = gate.clamp(max=limit).float()
    up = up.clamp(-limit, limit).float()
    return gate / (1 + torch.exp(-gate)) * up * weights[:, None]


@torch.no_grad()
def _layers(case, values: dict, widens, tokens=None) -> list[dict]:
    """The serial layer under each schedule of ``widens``, each expert's weights unpacked once."""
    limit = case.swiglu_limit
    ids = values["topk_idx"].cpu()
    wts = values["topk_weights"].cpu()
    rows = list(range(ids.shape[0])) if tokens is None else list(tokens)
    modes = [(torch.float32 if widen else torch.bfloat16) for widen in widens]
    x32 = unpack_activation_e8m0(values["x"].cpu(), values["x_scales"].cpu())
    H = x32.shape[1]
    d = [{} for _ in modes]
    for e in sorted(set(ids[rows].flatten().tolist())):
        w1_32 = unpack_mxfp4(values["l1_blocks"][e].cpu(), values["l1_scales"][e].cpu())
        w2_32 = unpack_mxfp4(values["l2_blocks"][e].cpu(), values["l2_scales"][e].cpu())
        pairs = [(r, s) for r, t in enumerate(rows) for s in range(ids.shape[1]) if int(ids[t, s]) == e]
        w = torch.stack([wts[rows[r], s] for r, s in pairs])
        for m, bf in enumerate(modes):
            w1, w2 = w1_32.to(bf), w2_32.to(bf)
            xt = torch.stack([x32[rows[r]].to(bf) for r, _ in pairs])
            l1 = (xt.float() @ w1.float().T).to(bf)
            a = swiglu_clamped(l1, w, limit)
            h = a if bf == torch.float32 else unpack_activation_e8m0(*pack_activation_e8m0(a)).to(bf)
            out = (h.float() @ w2.float().T).to(bf)
            for i, key in enumerate(pairs):
                d[m][key] = out[i]
    outs = []
    for m, bf in enumerate(modes):
        y = torch.empty((len(rows), H), dtype=bf)
        for r in range(len(rows)):
            acc = torch.zeros(H, dtype=torch.float32)
            for s in range(ids.shape[1]):
                acc = acc + d[m][(r, s)].float()
            y[r] = acc.to(bf)
        outs.append({"y": y})
    return outs


def layer(case, values: dict, *, widen: bool = False, tokens=None) -> dict:
    """Outputs {'y'} of the serial layer for ``tokens`` (default all)."""
    return _layers(case, values, (widen,), tokens)[0]


def reference_and_oracle(case, values: dict, tokens=None) -> tuple[dict, dict]:
    """``reference`` and ``oracle`` in one pass (each expert's weights unpacked once)."""
    want, exact = _layers(case, values, (False, True), tokens)
    return want, exact


def reference(case, values: dict, **kw) -> dict:
    return layer(case, values, widen=False, **kw)


def oracle(case, values: dict, **kw) -> dict:
    return layer(case, values, widen=True, **kw)
