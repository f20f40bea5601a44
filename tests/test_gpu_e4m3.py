"""The E4M3 encoder of the kernels against the bitwise rounding rule.

The kernels encode E4M3 with gfx950's v_cvt_pk_fp8_f32 (two codes per instruction);
megamoe_e4m3_selftest compares it on the device with the bitwise round-to-nearest-even rule
(quantization.py:106,125 clamp to +-448 first, then cast) on every fp32 magnitude from 0 to
448 with both signs and in every code slot, and on every NaN payload (infinity never reaches
the encoder: the clamp makes it 448, and the bitwise rule is not defined for it). The
quantization tests of test_gpu_layer.py tie the same encoder to the oracle's values.
"""

import pytest
import torch

from vibe_megakernel_amd import _lib

DEV = "cuda:0"


@pytest.mark.gpu
def test_e4m3_encoder_matches_the_rule_on_every_clamped_value():
    lib = _lib.load()
    bad = torch.zeros(1, dtype=torch.int64, device=DEV)
    stream = torch.cuda.current_stream(torch.device(DEV)).cuda_stream
    print("e4m3 self-test: magnitudes 0 .. 448, then NaNs", flush=True)
    assert lib.megamoe_e4m3_selftest(0, 0x43E00000 + 1, bad.data_ptr(), stream) == 0
    assert lib.megamoe_e4m3_selftest(0x7F800001, 0x7FFFFF, bad.data_ptr(), stream) == 0
    torch.cuda.synchronize()
    assert int(bad.item()) == 0
