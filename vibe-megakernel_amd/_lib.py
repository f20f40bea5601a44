"""ctypes binding of the C ABI in include/megamoe.h (libmegamoe.so, built in-tree).

There is no fallback: if the shared library is missing or cannot be loaded,
``load()`` raises, so nothing on the product path can silently run elsewhere.
"""

from __future__ import annotations

import ctypes
import os
from pathlib import Path

PACKAGE_DIR = Path(__file__).resolve().parent
LIBRARY = PACKAGE_DIR / "libmegamoe.so"

OK, ERR_INVALID_ARGUMENT, ERR_SHAPE, ERR_WORKSPACE, ERR_HIP, ERR_UNSUPPORTED, ERR_SCRATCH = range(7)
SCRATCH_BYTES = 32 << 20  # MEGAMOE_SCRATCH_BYTES
GATE_SOFTMAX, GATE_SIGMOID = 0, 1
STAGES = ("router", "select_quant", "permute", "experts", "combine")
STAGES_MX = ("permute", "experts", "combine")  # the MXFP4 form (routing and x are inputs)

# Every symbol the header declares; tests check the library exports them all.
SYMBOLS = ("megamoe_workspace_bytes", "megamoe_forward", "megamoe_forward_events", "megamoe_forward_timed",
           "megamoe_router_logits", "megamoe_route", "megamoe_quantize_rows", "megamoe_status_string",
           "megamoe_abi_version", "megamoe_block_forward", "megamoe_rms_norm", "megamoe_mx_workspace_bytes",
           "megamoe_mx_forward", "megamoe_ep_dispatch", "megamoe_ep_experts", "megamoe_ep_combine",
           "megamoe_forward_ex", "megamoe_combine_by_expert_id", "megamoe_forward_noalloc",
           "megamoe_layer_forward", "megamoe_layer_status", "megamoe_mx_layer_forward", "megamoe_mx_layer_status",
           "megamoe_e4m3_selftest", "megamoe_forward_w8a16", "megamoe_layer_forward_w8a16")
ABI_VERSION = 11


class Desc(ctypes.Structure):
    _fields_ = [("tokens", ctypes.c_int32), ("hidden", ctypes.c_int32), ("experts", ctypes.c_int32),
                ("topk", ctypes.c_int32), ("intermediate", ctypes.c_int32), ("shared_experts", ctypes.c_int32),
                ("groups", ctypes.c_int32), ("top_groups", ctypes.c_int32), ("gate", ctypes.c_int32),
                ("renormalize", ctypes.c_int32), ("pow2_scales", ctypes.c_int32),
                ("routed_scaling", ctypes.c_float)]


_TENSOR_FIELDS = ("x", "router", "router_bias", "gate", "gate_scale", "up", "up_scale", "down", "down_scale",
                  "shared_gate", "shared_gate_scale", "shared_up", "shared_up_scale", "shared_down",
                  "shared_down_scale", "y", "expert_ids", "expert_weights", "workspace")


class Tensors(ctypes.Structure):
    _fields_ = [(name, ctypes.c_void_p) for name in _TENSOR_FIELDS] + [("workspace_bytes", ctypes.c_size_t)]


class Block(ctypes.Structure):
    _fields_ = [("norm_weight", ctypes.c_void_p), ("eps", ctypes.c_float), ("weight_in_fp32", ctypes.c_int32),
                ("residual", ctypes.c_int32)]


class Epilogue(ctypes.Structure):
    _fields_ = [("swiglu", ctypes.c_int32), ("swiglu_limit", ctypes.c_float)]


MX_TENSOR_FIELDS = ("x", "x_scales", "topk_idx", "topk_weights", "l1_blocks", "l1_scales", "l2_blocks", "l2_scales",
                    "y", "workspace")


class MxTensors(ctypes.Structure):
    _fields_ = [(name, ctypes.c_void_p) for name in MX_TENSOR_FIELDS] + [("workspace_bytes", ctypes.c_size_t)]


EP_SEND_FIELDS = ("rows", "row_scales", "ids", "weights", "counts", "slot_rows")


class EpSend(ctypes.Structure):
    _fields_ = [(name, ctypes.c_void_p) for name in EP_SEND_FIELDS]


class MegaMoEError(RuntimeError):
    def __init__(self, status: int, what: str):
        self.status = status
        super().__init__(f"{what}: {status_string(status)} (status {status})")


_lib = None


def load() -> ctypes.CDLL:
    global _lib
    if _lib is not None:
        return _lib
    if not LIBRARY.exists():
        raise RuntimeError(f"{LIBRARY} is not built; run __graft_entry__.build() (hipcc, gfx950) first")
    lib = ctypes.CDLL(os.fspath(LIBRARY))
    c_int, c_void_p, c_size_t = ctypes.c_int, ctypes.c_void_p, ctypes.c_size_t
    P = ctypes.POINTER
    lib.megamoe_workspace_bytes.argtypes = [P(Desc), P(c_size_t)]
    lib.megamoe_forward.argtypes = [P(Desc), P(Tensors), c_void_p]
    lib.megamoe_forward_noalloc.argtypes = [P(Desc), P(Tensors), c_void_p]
    lib.megamoe_forward_events.argtypes = [P(Desc), P(Tensors), c_void_p, P(c_void_p)]
    lib.megamoe_forward_timed.argtypes = [P(Desc), P(Tensors), c_void_p, P(ctypes.c_float)]
    lib.megamoe_router_logits.argtypes = [P(Desc), c_void_p, c_void_p, c_void_p, c_void_p, c_size_t, c_void_p]
    lib.megamoe_route.argtypes = [P(Desc), c_void_p, c_void_p, c_void_p, c_void_p, c_void_p]
    lib.megamoe_quantize_rows.argtypes = [ctypes.c_int32, ctypes.c_int32, c_void_p, c_void_p, c_void_p,
                                          ctypes.c_int32, c_void_p]
    lib.megamoe_e4m3_selftest.argtypes = [ctypes.c_uint32, ctypes.c_uint32, c_void_p, c_void_p]
    lib.megamoe_block_forward.argtypes = [P(Desc), P(Tensors), P(Block), c_void_p, P(c_void_p)]
    lib.megamoe_rms_norm.argtypes = [ctypes.c_int32, ctypes.c_int32, c_void_p, c_void_p, ctypes.c_float,
                                     ctypes.c_int32, c_void_p, c_void_p]
    lib.megamoe_mx_workspace_bytes.argtypes = [P(Desc), P(c_size_t)]
    lib.megamoe_mx_forward.argtypes = [P(Desc), ctypes.c_float, P(MxTensors), c_void_p, P(c_void_p)]
    lib.megamoe_mx_layer_forward.argtypes = [P(Desc), ctypes.c_float, P(MxTensors), c_void_p, P(c_void_p)]
    lib.megamoe_mx_layer_status.argtypes = [P(Desc), c_void_p, c_size_t, P(ctypes.c_int32), c_void_p]
    lib.megamoe_ep_dispatch.argtypes = [P(Desc), ctypes.c_int32, P(MxTensors), P(EpSend), c_void_p]
    lib.megamoe_ep_experts.argtypes = [P(Desc), ctypes.c_float, ctypes.c_int64, P(MxTensors), c_void_p, P(c_void_p)]
    lib.megamoe_ep_combine.argtypes = [ctypes.c_int32, ctypes.c_int32, ctypes.c_int32, c_void_p, c_void_p, c_void_p,
                                       c_void_p]
    lib.megamoe_forward_ex.argtypes = [P(Desc), P(Tensors), P(Block), P(Epilogue), c_void_p, P(c_void_p)]
    lib.megamoe_forward_w8a16.argtypes = [P(Desc), P(Tensors), P(Block), P(Epilogue), c_void_p, P(c_void_p)]
    lib.megamoe_layer_forward_w8a16.argtypes = [P(Desc), P(Tensors), P(Block), P(Epilogue), c_void_p, P(c_void_p)]
    lib.megamoe_layer_forward.argtypes = [P(Desc), P(Tensors), P(Block), P(Epilogue), c_void_p, P(c_void_p)]
    lib.megamoe_layer_status.argtypes = [P(Desc), c_void_p, c_size_t, P(ctypes.c_int32), c_void_p]
    lib.megamoe_combine_by_expert_id.argtypes = [ctypes.c_int32, ctypes.c_int32, ctypes.c_int32, c_void_p, c_void_p,
                                                 c_void_p, c_void_p, c_void_p, c_void_p]
    lib.megamoe_status_string.argtypes = [c_int]
    lib.megamoe_status_string.restype = ctypes.c_char_p
    lib.megamoe_abi_version.argtypes = []
    for name in SYMBOLS:
        if name != "megamoe_status_string":
            getattr(lib, name).restype = c_int
    _lib = lib
    return lib


def status_string(status: int) -> str:
    return load().megamoe_status_string(status).decode()


def check(status: int, what: str) -> None:
    """Map a status to the reference's error behaviour: bad geometry or arguments raise
    ValueError (as the reference's input builders do), everything else MegaMoEError."""
    if status == OK:
        return
    if status in (ERR_SHAPE, ERR_INVALID_ARGUMENT):
        raise ValueError(f"{what}: {status_string(status)}")
    raise MegaMoEError(status, what)
