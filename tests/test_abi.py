"""The C ABI of libmegamoe.so on the CPU: the library loads, exports every function the
header declares, and its host-side checks (geometry, pointers, workspace size) answer
without touching a GPU. No compute entry point runs here."""

from __future__ import annotations

import ctypes
import re
import subprocess
from pathlib import Path

import pytest

from vibe_megakernel_amd import _lib
from vibe_megakernel_amd import cases as C
from vibe_megakernel_amd import submission

HEADER = Path(__file__).resolve().parent.parent / "include" / "megamoe.h"


def _declared() -> set[str]:
    text = HEADER.read_text()
    return set(re.findall(r"^\s*(?:const\s+)?[a-z_0-9]+\s*\*?\s*(megamoe_[a-z_0-9]+)\s*\(", text, flags=re.M))


def test_library_exports_every_declared_function():
    declared = _declared()
    assert declared == set(_lib.SYMBOLS)
    lib = _lib.load()
    for name in declared:
        assert getattr(lib, name) is not None
    out = subprocess.run(["nm", "-D", "--defined-only", str(_lib.LIBRARY)], capture_output=True, text=True,
                         check=True).stdout
    exported = set(re.findall(r"\bT (megamoe_[a-z_0-9]+)$", out, flags=re.M))
    assert declared <= exported


def test_version_and_status_strings():
    lib = _lib.load()
    assert lib.megamoe_abi_version() == _lib.ABI_VERSION == 11
    texts = {code: _lib.status_string(code) for code in range(7)}
    assert texts[_lib.OK] == "ok" and len(set(texts.values())) == 7
    assert _lib.status_string(99) == "unknown status"


@pytest.mark.parametrize("case", C.CASES, ids=lambda c: c.id)
def test_workspace_bytes_for_every_config(case):
    layer = submission.MoELayer(case)
    T, H, K, I, S = case.tokens, case.hidden, case.topk, case.intermediate, case.shared_experts
    # At least the grouped intermediates: quantized x, h rows, bf16 down rows.
    assert layer.workspace_bytes >= T * H + T * K * (I + 2 * H) + T * S * I
    assert layer.workspace_bytes % 256 == 0
    assert layer.workspace_bytes < 64 << 20


def _status(desc, **tensors):
    lib = _lib.load()
    size = ctypes.c_size_t(0)
    return lib.megamoe_workspace_bytes(ctypes.byref(desc), ctypes.byref(size))


@pytest.mark.parametrize("change,status", [
    (dict(hidden=1000), _lib.ERR_SHAPE),                      # H not a multiple of 128
    (dict(intermediate=200), _lib.ERR_SHAPE),
    (dict(topk=300), _lib.ERR_SHAPE),                         # K > E
    (dict(groups=3), _lib.ERR_SHAPE),                         # G does not divide E
    (dict(top_groups=9), _lib.ERR_SHAPE),                     # TG > G
    (dict(groups=64, top_groups=1), _lib.ERR_SHAPE),          # kept groups hold fewer than K experts
    (dict(gate=7), _lib.ERR_SHAPE),
    (dict(tokens=-1), _lib.ERR_SHAPE),
    (dict(experts=2048, groups=1, top_groups=1), _lib.ERR_UNSUPPORTED),
    (dict(topk=40, groups=1, top_groups=1), _lib.ERR_UNSUPPORTED),
    (dict(), _lib.OK),
])
def test_geometry_checks(change, status):
    desc = submission.make_desc(C.case(C.HEADLINE))
    for k, v in change.items():
        setattr(desc, k, v)
    assert _status(desc) == status


def test_null_and_workspace_checks_answer_before_any_gpu_call():
    lib = _lib.load()
    case = C.case(C.HEADLINE)
    desc = submission.make_desc(case)
    size = ctypes.c_size_t(0)
    assert lib.megamoe_workspace_bytes(None, ctypes.byref(size)) == _lib.ERR_INVALID_ARGUMENT
    assert lib.megamoe_workspace_bytes(ctypes.byref(desc), None) == _lib.ERR_INVALID_ARGUMENT
    assert lib.megamoe_forward(ctypes.byref(desc), None, None) == _lib.ERR_INVALID_ARGUMENT
    t = _lib.Tensors()
    assert lib.megamoe_forward(ctypes.byref(desc), ctypes.byref(t), None) == _lib.ERR_INVALID_ARGUMENT
    # Every pointer set (never dereferenced: the workspace check fails first).
    fake = {name: 256 for name, _ in _lib.Tensors._fields_ if name != "workspace_bytes"}
    t = _lib.Tensors(**fake, workspace_bytes=16)
    assert lib.megamoe_forward(ctypes.byref(desc), ctypes.byref(t), None) == _lib.ERR_WORKSPACE
    # Shared expert pointers are required when S > 0.
    t = _lib.Tensors(**{**fake, "shared_down": None}, workspace_bytes=1 << 40)
    assert lib.megamoe_forward(ctypes.byref(desc), ctypes.byref(t), None) == _lib.ERR_INVALID_ARGUMENT
    # No tokens: nothing to do, no pointer needed.
    desc.tokens = 0
    assert lib.megamoe_forward(ctypes.byref(desc), ctypes.byref(_lib.Tensors()), None) == _lib.OK
    assert lib.megamoe_route(ctypes.byref(desc), None, None, None, None, None) == _lib.OK
    desc.tokens = 4
    assert lib.megamoe_route(ctypes.byref(desc), None, None, None, None, None) == _lib.ERR_INVALID_ARGUMENT
    assert lib.megamoe_router_logits(ctypes.byref(desc), None, None, None, None, 0, None) == \
        _lib.ERR_INVALID_ARGUMENT
    assert lib.megamoe_quantize_rows(-1, 128, None, None, None, 0, None) == _lib.ERR_INVALID_ARGUMENT
    assert lib.megamoe_quantize_rows(0, 128, None, None, None, 0, None) == _lib.OK
    assert lib.megamoe_quantize_rows(4, 128, None, None, None, 0, None) == _lib.ERR_INVALID_ARGUMENT
    assert lib.megamoe_e4m3_selftest(0, 16, None, None) == _lib.ERR_INVALID_ARGUMENT
    assert lib.megamoe_e4m3_selftest(0x7F800000, 0x800001, 8, None) == _lib.ERR_INVALID_ARGUMENT


def test_python_errors_follow_the_reference_behaviour():
    """Bad geometry raises ValueError (as the reference's builders do); inputs off the
    GPU are refused before any launch."""
    import torch

    with pytest.raises(ValueError):
        C.Case.from_dict({**C.case(C.HEADLINE).to_dict(), "params": {**C.case(C.HEADLINE).params, "topk": 999}})
    layer = submission.MoELayer(C.development(C.case("moe-fp8-tiny-t4")))
    with pytest.raises(RuntimeError):
        layer({"x": torch.zeros((4, 256), dtype=torch.bfloat16)})
    with pytest.raises(ValueError):
        layer({})
    with pytest.raises(ValueError):
        _lib.check(_lib.ERR_SHAPE, "probe")
    with pytest.raises(_lib.MegaMoEError):
        _lib.check(_lib.ERR_HIP, "probe")


def test_ep_and_variant_entry_points_check_arguments_before_any_gpu_call():
    lib = _lib.load()
    P = ctypes.byref
    desc = _lib.Desc(tokens=64, hidden=7168, experts=384, topk=6, intermediate=3072)
    t, send = _lib.MxTensors(), _lib.EpSend()
    # Dispatch: geometry, limits, pointers.
    assert lib.megamoe_ep_dispatch(None, 8, P(t), P(send), None) == _lib.ERR_INVALID_ARGUMENT
    assert lib.megamoe_ep_dispatch(P(desc), 7, P(t), P(send), None) == _lib.ERR_SHAPE  # 7 does not divide 384
    assert lib.megamoe_ep_dispatch(P(desc), 0, P(t), P(send), None) == _lib.ERR_SHAPE
    assert lib.megamoe_ep_dispatch(P(desc), 384, P(t), P(send), None) == _lib.ERR_UNSUPPORTED  # > 256 ranks
    big = _lib.Desc(tokens=10000, hidden=7168, experts=384, topk=6, intermediate=3072)
    assert lib.megamoe_ep_dispatch(P(big), 8, P(t), P(send), None) == _lib.ERR_UNSUPPORTED  # T*K > 49152
    assert lib.megamoe_ep_dispatch(P(desc), 8, P(t), P(send), None) == _lib.ERR_INVALID_ARGUMENT  # no counts
    fake = _lib.EpSend(**{name: 256 for name in _lib.EP_SEND_FIELDS})
    assert lib.megamoe_ep_dispatch(P(desc), 8, P(t), P(fake), None) == _lib.ERR_INVALID_ARGUMENT  # no x
    odd = _lib.MxTensors(x=257, x_scales=256, topk_idx=256, topk_weights=256)
    assert lib.megamoe_ep_dispatch(P(desc), 8, P(odd), P(fake), None) == _lib.ERR_INVALID_ARGUMENT  # x unaligned
    # Local experts: one slot per row, a valid base.
    assert lib.megamoe_ep_experts(P(desc), 10.0, 0, P(t), None, None) == _lib.ERR_SHAPE  # topk 6
    one = _lib.Desc(tokens=100, hidden=7168, experts=48, topk=1, intermediate=3072)
    assert lib.megamoe_ep_experts(P(one), 10.0, -1, P(t), None, None) == _lib.ERR_SHAPE
    assert lib.megamoe_ep_experts(P(one), 10.0, 48, P(t), None, None) == _lib.ERR_INVALID_ARGUMENT  # no pointers
    assert lib.megamoe_ep_experts(P(one), 0.0, 48, P(t), None, None) == _lib.ERR_INVALID_ARGUMENT  # limit 0
    # Combine at the source.
    assert lib.megamoe_ep_combine(4, 100, 2, None, None, None, None) == _lib.ERR_SHAPE  # H % 8
    assert lib.megamoe_ep_combine(0, 7168, 6, None, None, None, None) == _lib.OK
    assert lib.megamoe_ep_combine(4, 7168, 6, None, None, None, None) == _lib.ERR_INVALID_ARGUMENT
    assert lib.megamoe_ep_combine(4, 7168, 6, 257, 256, 256, None) == _lib.ERR_INVALID_ARGUMENT  # unaligned
    # GPT-OSS combine.
    assert lib.megamoe_combine_by_expert_id(4, 2880, 33, None, None, None, None, None, None) == \
        _lib.ERR_UNSUPPORTED  # K > 32
    assert lib.megamoe_combine_by_expert_id(0, 2880, 4, None, None, None, None, None, None) == _lib.OK
    assert lib.megamoe_combine_by_expert_id(4, 2880, 4, None, None, None, None, None, None) == \
        _lib.ERR_INVALID_ARGUMENT
    # Epilogue variants: the form and the limit are checked.
    d8 = submission.make_desc(C.case(C.HEADLINE))
    ft = _lib.Tensors()
    for bad in (_lib.Epilogue(swiglu=2, swiglu_limit=0.0), _lib.Epilogue(swiglu=1, swiglu_limit=-1.0),
                _lib.Epilogue(swiglu=0, swiglu_limit=float("nan"))):
        assert lib.megamoe_forward_ex(P(d8), P(ft), None, P(bad), None, None) == _lib.ERR_INVALID_ARGUMENT
        assert lib.megamoe_layer_forward(P(d8), P(ft), None, P(bad), None, None) == _lib.ERR_INVALID_ARGUMENT
    ok = _lib.Epilogue(swiglu=1, swiglu_limit=10.0)
    assert lib.megamoe_forward_ex(P(d8), P(ft), None, P(ok), None, None) == _lib.ERR_INVALID_ARGUMENT  # no tensors
    assert lib.megamoe_layer_forward(P(d8), P(ft), None, P(ok), None, None) == _lib.ERR_INVALID_ARGUMENT
    blk = _lib.Block(norm_weight=None, eps=-1.0, weight_in_fp32=1, residual=1)
    assert lib.megamoe_layer_forward(P(d8), P(ft), P(blk), None, None, None) == _lib.ERR_INVALID_ARGUMENT  # eps < 0
    d8.tokens = 0
    assert lib.megamoe_forward_ex(P(d8), P(ft), None, P(ok), None, None) == _lib.OK
    assert lib.megamoe_layer_forward(P(d8), P(ft), None, P(ok), None, None) == _lib.OK


def test_permute_limits_allow_a_full_ep_share():
    """The permute ranks rows without its token bitmap when the bitmap would not fit in LDS,
    so the local experts accept every received-row count a rank can get: ep 8 x 512 tokens x
    6 slots = 24576 rows over 48 local experts (and the fp8 layer any token count whose
    packed counters fit)."""
    lib = _lib.load()
    size = ctypes.c_size_t(0)
    for rows in (1, 10000, 24576, 49152):
        d = _lib.Desc(tokens=rows, hidden=7168, experts=48, topk=1, intermediate=3072)
        assert lib.megamoe_mx_workspace_bytes(ctypes.byref(d), ctypes.byref(size)) == _lib.OK, rows
    for tokens in (64, 4096, 16384):
        d = submission.make_desc(C.Case.from_dict({**C.case(C.HEADLINE).to_dict(), "id": "t",
                                                   "params": {**C.case(C.HEADLINE).params, "tokens": tokens}}))
        assert lib.megamoe_workspace_bytes(ctypes.byref(d), ctypes.byref(size)) == _lib.OK, tokens


def test_case_table_of_the_forms():
    """Every form's case builds its layer (workspace sizing on the CPU) and the catalog
    geometry of the EP share, the MXFP4 and GLM cases is the reference's."""
    for c in C.BLOCK_CASES + C.MX_CASES + C.VARIANT_CASES:
        layer = submission.MoELayer(c)
        assert layer.workspace_bytes > 0 and layer.workspace_bytes % 256 == 0
    glm = C.case("moe-fp8-glm-5.3-flash-t64")
    assert (glm.hidden, glm.experts, glm.topk, glm.intermediate, glm.shared_experts) == (4096, 288, 8, 2048, 1)
    assert (glm.swiglu, glm.swiglu_limit, glm.router, glm.groups) == ("bf16", 10.0, "sigmoid", 1)
    with pytest.raises(ValueError):
        C.Case.from_dict({**glm.to_dict(), "swiglu": "fp16"})
    with pytest.raises(ValueError):
        C.Case.from_dict({**C.case("moe-mxfp4-deepseek-v4-pro-t64").to_dict(), "swiglu": "bf16"})
    with pytest.raises(ValueError):  # expert parallelism is defined for the MXFP4 form
        C.Case.from_dict({**C.case(C.HEADLINE).to_dict(), "gpus": 8, "ep": 8})


def test_noalloc_refuses_a_workspace_beyond_the_scratch():
    """megamoe_forward_noalloc checks the geometry's workspace against MEGAMOE_SCRATCH_BYTES on
    the host and refuses, reading no pointer and launching nothing (so this runs on the CPU);
    every benchmark config fits."""
    lib = _lib.load()
    for case in C.CASES:
        assert submission.MoELayer(case).workspace_bytes <= _lib.SCRATCH_BYTES, case.id
    kimi = C.case("moe-fp8-kimi-k2-t128")
    big = C.Case.from_dict({**kimi.to_dict(), "id": "kimi-k2-t256", "params": {**kimi.params, "tokens": 256}})
    desc = submission.make_desc(big)
    size = ctypes.c_size_t(0)
    assert lib.megamoe_workspace_bytes(ctypes.byref(desc), ctypes.byref(size)) == _lib.OK
    assert size.value > _lib.SCRATCH_BYTES
    assert lib.megamoe_forward_noalloc(ctypes.byref(desc), ctypes.byref(_lib.Tensors()), None) == _lib.ERR_SCRATCH
    assert "scratch" in _lib.status_string(_lib.ERR_SCRATCH)


def test_scratch_size_matches_the_header():
    m = re.search(r"#define MEGAMOE_SCRATCH_BYTES \((\d+)u << (\d+)\)", HEADER.read_text())
    assert m and int(m.group(1)) << int(m.group(2)) == _lib.SCRATCH_BYTES
