"""Pins of the oracle's FP8 and BF16 codecs (CPU only).

What fixes each function, independently of the formula it restates:
  * explicit per-block loops (the re-derivation of megabench/tests/test_frontier.py:224-248);
  * the padded restatement and edge vectors of megabench/tests/test_megamoe.py:56-81
    (known-answer data in tests/golden/known_answers.json);
  * the E4M3 format itself: every one of the 256 codes decoded from its sign, exponent
    and mantissa fields, and round-to-nearest-even at every midpoint between adjacent
    codes, checked against both torch's float8_e4m3fn cast and the plain-C codec;
  * BF16 rounding from the bit pattern (RNE on the upper 16 bits).
"""

from __future__ import annotations

import json
import math
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import build as oracle_c
from oracle import formats

GOLDEN = json.loads((Path(__file__).parent / "golden" / "known_answers.json").read_text())


def _e4m3_closed_form(code: int) -> float:
    """Value of an E4M3 (fn) code from its fields: 1 sign, 4 exponent (bias 7), 3 mantissa
    bits; exponent 0 is subnormal; S.1111.111 is NaN; there is no infinity."""
    sign = -1.0 if code & 0x80 else 1.0
    exp, man = (code >> 3) & 0xF, code & 0x7
    if exp == 0xF and man == 0x7:
        return math.nan
    if exp == 0:
        return sign * (man / 8.0) * 2.0 ** -6
    return sign * (1.0 + man / 8.0) * 2.0 ** (exp - 7)


def _scale_rule(block: torch.Tensor, power: bool) -> torch.Tensor:
    scale = block.abs().max().clamp_min(1e-4) / 448
    if power:
        scale = 2 ** torch.ceil(torch.log2(scale))
    return scale


@pytest.mark.parametrize("power", [False, True])
def test_weight_and_activation_scales_match_explicit_block_loops(power):
    torch.manual_seed(13)
    value = torch.randn(137, 259).to(torch.bfloat16)
    payload, scales = formats.pack_weight(value, power_of_two=power)
    expected = torch.empty(value.shape, dtype=torch.float32)
    for row in range(0, 137, 128):
        for col in range(0, 259, 128):
            block = value[row:row + 128, col:col + 128].float()
            scale = _scale_rule(block, power)
            assert scales[row // 128, col // 128] == scale
            expected[row:row + 128, col:col + 128] = (block / scale).to(torch.float8_e4m3fn).float() * scale
    assert torch.equal(formats.unpack_weight(payload, scales), expected)

    payload, scales = formats.pack_activation(value, power_of_two=power)
    for row in (0, 136):
        for col in range(0, 259, 128):
            block = value[row, col:col + 128].float()
            scale = _scale_rule(block, power)
            assert scales[row, col // 128] == scale
            want = (block / scale).to(torch.float8_e4m3fn).float() * scale
            assert torch.equal(formats.unpack_activation(payload, scales)[row, col:col + 128], want)


@pytest.mark.parametrize("power", [False, True])
def test_activation_packing_matches_padded_restatement(power):
    value = torch.randn((3, 300), generator=torch.Generator().manual_seed(5)).to(torch.bfloat16)
    payload, scales = formats.pack_activation(value, power_of_two=power)
    padded = torch.nn.functional.pad(value.float(), (0, 84)).unflatten(-1, (-1, 128))
    want = padded.abs().amax(-1).clamp_min(1e-4) / 448.0
    want = torch.exp2(torch.ceil(torch.log2(want))) if power else want
    assert torch.equal(scales, want)
    expected = (padded / want[..., None]).clamp(-448, 448).to(torch.float8_e4m3fn).flatten(-2)[..., :300]
    assert torch.equal(payload.view(torch.uint8), expected.view(torch.uint8))


@pytest.mark.parametrize("power", [False, True])
def test_reference_edge_values(power):
    """The reference's edge vector (448 and its neighbours, 224, the 1e-4 floor, 0, 896),
    one value per row so each sets its row's amax."""
    edges = torch.tensor(GOLDEN["fp8_edge_values"]["values"], dtype=torch.float32)
    value = torch.zeros((len(edges), 128))
    value[:, 0] = edges
    value[:, 1] = edges / 3  # a second, non-maximal entry per row
    payload, scales = formats.pack_activation(value, power_of_two=power)
    for r, amax in enumerate(edges.tolist()):
        raw = max(amax, 1e-4) / 448.0
        s = float(scales[r, 0])
        if power:
            m, e = math.frexp(s)
            assert m == 0.5, "power-of-two scale"
            assert s / 2 < np.float32(raw) <= s
        else:
            assert s == np.float32(np.float32(max(np.float32(amax), np.float32(1e-4))) / np.float32(448.0))
        restored = formats.unpack_activation(payload, scales)[r, :2]
        # |x / s| <= 448 keeps E4M3 in range: half an ulp of 3 mantissa bits (2^-4 relative), or
        # half the subnormal step 2^-9 of the scale.
        assert bool(((restored - value[r, :2]).abs() <= value[r, :2].abs() * 2 ** -4 + s * 2 ** -10).all())
        assert torch.isfinite(restored).all()
    if not power:
        # 448 maps to scale 1 and payload 448 exactly; 896 to scale 2.
        assert float(scales[0, 0]) == 1.0 and float(payload[0, 0].float()) == 448.0
        assert float(scales[8, 0]) == 2.0 and float(payload[8, 0].float()) == 448.0


def test_e4m3_code_table_is_exhaustively_the_format():
    codes = torch.arange(256, dtype=torch.uint8)
    torch_values = codes.view(torch.float8_e4m3fn).float().tolist()
    lib = oracle_c.load()
    for code in range(256):
        want = _e4m3_closed_form(code)
        got_c = lib.oc_e4m3_to_f32(code)
        if math.isnan(want):
            assert math.isnan(torch_values[code]) and math.isnan(got_c), code
            continue
        assert torch_values[code] == want, code
        assert got_c == want, code
    # Largest finite magnitude and the smallest subnormal.
    assert _e4m3_closed_form(0x7E) == 448.0 and _e4m3_closed_form(0x01) == 2.0 ** -9


def test_e4m3_rounding_is_nearest_even_at_every_midpoint():
    positives = [(c, _e4m3_closed_form(c)) for c in range(0x00, 0x7F)]  # 0 .. 448
    probes, want = [], []
    for (ca, va), (cb, vb) in zip(positives, positives[1:]):
        mid = np.float32((va + vb) / 2)  # exact: both values fit 4 significant bits
        assert float(mid) == (va + vb) / 2
        even = ca if ca % 2 == 0 else cb
        probes += [mid, np.nextafter(mid, np.float32(np.inf)), np.nextafter(mid, np.float32(-np.inf)), va]
        want += [even, cb, ca, ca]
    probes = np.array(probes, dtype=np.float32)
    want = np.array(want, dtype=np.uint8)
    for sign in (1.0, -1.0):
        x = probes * np.float32(sign)
        w = want | (0x80 if sign < 0 else 0)
        w = np.where(x == 0, 0x80 if sign < 0 else 0, w).astype(np.uint8)
        got_torch = torch.from_numpy(x).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
        got_c = oracle_c.e4m3_encode(x)
        assert np.array_equal(got_torch, w)
        assert np.array_equal(got_c, w)


def test_e4m3_codec_agrees_with_torch_on_random_values():
    g = torch.Generator().manual_seed(11)
    x = (torch.randn(400_000, generator=g) * torch.logspace(-12, 3, 400_000).index_select(
        0, torch.randperm(400_000, generator=g))).clamp(-448, 448)
    got_c = oracle_c.e4m3_encode(x.numpy())
    got_torch = x.to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(got_c, got_torch)


def _bf16_from_bits(x: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even of fp32 to its upper 16 bits; NaN -> quiet NaN."""
    u = x.view(np.uint32).astype(np.uint64)
    rounded = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    nan = np.isnan(x)
    rounded[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
    return rounded


def test_bf16_rounding_matches_the_bit_rule_and_torch():
    g = torch.Generator().manual_seed(17)
    x = torch.randn(200_000, generator=g) * torch.logspace(-30, 30, 200_000)
    base = torch.randn(1000, generator=g).to(torch.bfloat16).float()
    # Midpoints between adjacent bf16 values, and one fp32 ulp either side.
    mids = (base.view(torch.int32) + 0x8000).view(torch.float32)
    x = torch.cat([x, mids, torch.nextafter(mids, mids * 2), torch.nextafter(mids, mids * 0)])
    xn = x.numpy()
    want = _bf16_from_bits(xn.copy())
    assert np.array_equal(x.to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16), want)
    assert np.array_equal(oracle_c.bf16_encode(xn), want)
