"""FP8 E4M3 codecs, restated from megabench/tasks/quantization.py (test infrastructure).

Weights: one fp32 scale per 128x128 block, scale = max(block amax, 1e-4) / 448
(or the next power of two), payload = E4M3(clamp(W / scale, +-448)) with
round-to-nearest-even; rows and columns pad to 128 with zeros that take part
in the amax only. Activations: the same rule per row and 128-column block.
Dequantization multiplies the payload by the broadcast scale in fp32.

Pinned by tests/test_oracle_formats.py: explicit per-block loops (the
re-derivation of megabench/tests/test_frontier.py:224-248), the padded
restatement and edge vectors of megabench/tests/test_megamoe.py:56-81, the
E4M3 format decoded field by field for all 256 codes, and round-to-nearest-even
at every midpoint between adjacent codes, each against both torch's cast and
the plain-C codec in oracle/codec.c.
"""

from __future__ import annotations

import torch

BLOCK = 128
FP8_MAX = 448.0


def fp8_scale(amax: torch.Tensor, power_of_two: bool) -> torch.Tensor:
    """quantization.py:57-59"""
    scale = amax.float().clamp_min(1e-4) / FP8_MAX
    if power_of_two:
        scale = torch.exp2(torch.ceil(torch.log2(scale)))
    return scale


def pack_activation(value: torch.Tensor, power_of_two: bool = False, block: int = BLOCK):
    """Per-row, per-``block``-column E4M3 payload and fp32 scales (quantization.py:87-109,
    scale_format="float")."""
    width = value.shape[-1]
    pad = (-width) % block
    grouped = torch.nn.functional.pad(value.float(), (0, pad)).unflatten(-1, (-1, block))
    scales = fp8_scale(grouped.abs().amax(-1), power_of_two)
    payload = (grouped / scales.unsqueeze(-1)).clamp(-FP8_MAX, FP8_MAX).to(torch.float8_e4m3fn)
    return payload.flatten(-2)[..., :width].contiguous(), scales


def unpack_activation(payload: torch.Tensor, scales: torch.Tensor, block: int = BLOCK) -> torch.Tensor:
    """quantization.py:112-116 (fp32 scales)."""
    width = payload.shape[-1]
    return payload.float() * scales.repeat_interleave(block, dim=-1)[..., :width]


def pack_weight(value: torch.Tensor, power_of_two: bool = False):
    """E4M3 payload [R, C] and scales [ceil(R/128), ceil(C/128)] (quantization.py:119-126)."""
    rows, cols = value.shape
    padded = torch.nn.functional.pad(value.float(), (0, (-cols) % BLOCK, 0, (-rows) % BLOCK))
    tiles = padded.view(padded.shape[0] // BLOCK, BLOCK, padded.shape[1] // BLOCK, BLOCK)
    scales = fp8_scale(tiles.abs().amax(dim=(1, 3)), power_of_two)
    payload = (tiles / scales[:, None, :, None]).clamp(-FP8_MAX, FP8_MAX).to(torch.float8_e4m3fn)
    return payload.view(padded.shape)[:rows, :cols].contiguous(), scales


def unpack_weight(payload: torch.Tensor, scales: torch.Tensor) -> torch.Tensor:
    """quantization.py:129-131"""
    full = scales.repeat_interleave(BLOCK, 0).repeat_interleave(BLOCK, 1)
    return payload.float() * full[:payload.shape[0], :payload.shape[1]]
