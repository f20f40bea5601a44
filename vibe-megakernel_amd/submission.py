"""Drop-in submission for the reference harness: ``build(case) -> run(inputs) -> outputs``.

The contract is the reference's (megabench/README.md:83-104; loaded by path as
megabench/harness/runner.py:69-87 does): ``build`` receives ``Case.to_dict()``
(plus an optional ``execution`` entry, ignored on one GPU), ``run`` takes the
case's input tensors on the GPU, never mutates them, allocates its outputs and
returns ``{"y", "expert_ids", "expert_weights"}`` with the dtypes and shapes of
the reference outputs. All work is issued on torch's current stream through
the C ABI of libmegamoe.so; there is no other code path.

A case in the MXFP4 form (``format="mxfp4"``, megamoe.py numerics) takes ``x`` (E4M3),
``x_scales`` (E8M0 per 32), ``topk_idx``, ``topk_weights`` and the MXFP4 expert stacks
``l1_blocks``/``l1_scales``/``l2_blocks``/``l2_scales`` and returns ``{"y"}`` as
megamoe.reference does, through megamoe_mx_forward.

A case in the block form (``norm``/``residual`` set) takes ``x`` as the block input
and ``ln2`` (bf16 [H]) as the RMSNorm gamma, and returns y = x + bf16(layer(rms(x)))
(frontier.py:335-354).

The fp8 layer and its block and epilogue forms run as ONE kernel launch
(megamoe_layer_forward), within the reference harness's default launch budget of one
(megabench/cases.py:32, audited by megabench/harness/benchmark.py:73-100).
"""

from __future__ import annotations

import contextlib
import ctypes

import torch

from . import _lib
from .cases import Case

_INPUTS = ("x", "router", "router_bias", "gate", "gate_scale", "up", "up_scale", "down", "down_scale",
           "shared_gate", "shared_gate_scale", "shared_up", "shared_up_scale", "shared_down", "shared_down_scale")


_RAW_STREAM = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def _stream_handle(device: torch.device) -> int:
    """torch's current stream of ``device`` as a HIP stream handle (the raw query skips the
    Stream object that torch.cuda.current_stream builds on every call)."""
    if _RAW_STREAM is not None:
        return _RAW_STREAM(device.index)
    return torch.cuda.current_stream(device).cuda_stream


def _on(device: torch.device):
    """A guard making ``device`` current, or none when it is already (the common case)."""
    return contextlib.nullcontext() if torch.cuda.current_device() == device.index else torch.cuda.device(device)


def make_desc(case: Case) -> _lib.Desc:
    return _lib.Desc(tokens=case.tokens, hidden=case.hidden, experts=case.experts, topk=case.topk,
                     intermediate=case.intermediate, shared_experts=case.shared_experts, groups=case.groups,
                     top_groups=case.top_groups,
                     gate=_lib.GATE_SIGMOID if case.router == "sigmoid" else _lib.GATE_SOFTMAX,
                     renormalize=int(case.renormalize), pow2_scales=int(case.power_of_two),
                     routed_scaling=float(case.routed_scaling))


def _expect(t: torch.Tensor, name: str, dtype, shape, device) -> torch.Tensor:
    if not isinstance(t, torch.Tensor):
        raise ValueError(f"{name}: expected a tensor")
    if t.dtype != dtype or tuple(t.shape) != tuple(shape):
        raise ValueError(f"{name}: expected {tuple(shape)} {dtype}, got {tuple(t.shape)} {t.dtype}")
    if t.device != device:
        raise ValueError(f"{name}: on {t.device}, expected {device}")
    if not t.is_contiguous():
        raise ValueError(f"{name}: must be contiguous")
    return t


class MoELayer:
    """The layer for one case; holds one workspace per (device, stream) between calls (the
    work of a call is independent of the last one's, so only calls on one stream share a
    workspace and they are ordered by that stream).

    The fp8 layer (and its block and epilogue forms) runs as one launch,
    megamoe_layer_forward, by default, and the MXFP4 form as megamoe_mx_layer_forward;
    ``single_launch=False`` selects the stream-ordered kernels (megamoe_forward /
    megamoe_forward_ex: router, select + quantization, permute, experts, combine;
    megamoe_mx_forward: permute, experts, combine), whose stage boundaries ``record`` can
    mark. The W8A16 form (case.activations "bf16") runs through megamoe_layer_forward_w8a16
    and megamoe_forward_w8a16 likewise."""

    def __init__(self, case: Case, single_launch: bool = True):
        self.case = case
        self.lib = _lib.load()
        self.desc = make_desc(case)
        self._desc_ref = ctypes.byref(self.desc)
        self._specs = self._input_specs()
        self.mx = case.format == "mxfp4"
        # The W8A16 form (bf16 activations): megamoe_layer_forward_w8a16 (one launch) or
        # megamoe_forward_w8a16 (stream-ordered).
        self.a16 = case.activations == "bf16"
        self.single_launch = single_launch
        self.stages = ("layer",) if self.single_launch else (_lib.STAGES_MX if self.mx else _lib.STAGES)
        size = ctypes.c_size_t(0)
        sizer = self.lib.megamoe_mx_workspace_bytes if self.mx else self.lib.megamoe_workspace_bytes
        _lib.check(sizer(ctypes.byref(self.desc), ctypes.byref(size)), f"{case.id}: workspace size")
        self.workspace_bytes = int(size.value)
        self._workspace: dict[tuple, torch.Tensor] = {}
        self.block = None if case.norm == "none" and not case.residual else (case.norm, case.residual)
        # The epilogue variant of the fp8 form: None is the DeepSeek form.
        self.epilogue = (None if self.mx or (case.swiglu == "fp32" and case.swiglu_limit == 0) else
                         _lib.Epilogue(swiglu=int(case.swiglu == "bf16"), swiglu_limit=float(case.swiglu_limit)))
        self._epi_ref = None if self.epilogue is None else ctypes.byref(self.epilogue)
        # The pointer fields that come from the inputs, in the C struct's order.
        self._ptr_names = tuple(n for n in _INPUTS if (n != "router_bias" or case.bias != "none") and
                                (case.shared_experts or not n.startswith("shared_")))

    def _input_specs(self) -> tuple:
        """(name, dtype, shape) of every input the case reads, in checking order."""
        c = self.case
        T, H, E, K, I, S = c.tokens, c.hidden, c.experts, c.topk, c.intermediate, c.shared_experts
        u8, f8, f32 = torch.uint8, torch.float8_e4m3fn, torch.float32
        if c.format == "mxfp4":
            return (("x", f8, (T, H)), ("x_scales", u8, (T, H // 32)), ("topk_idx", torch.int64, (T, K)),
                    ("topk_weights", f32, (T, K)), ("l1_blocks", u8, (E, 2 * I, H // 32, 16)),
                    ("l1_scales", u8, (E, 2 * I, H // 32)), ("l2_blocks", u8, (E, H, I // 32, 16)),
                    ("l2_scales", u8, (E, H, I // 32)))
        bh, bi = -(-H // 128), -(-I // 128)
        specs = [("x", torch.bfloat16, (T, H)), ("router", f32, (E, H))]
        if c.bias != "none":
            specs.append(("router_bias", f32, (E,)))
        if c.norm != "none":
            specs.append(("ln2", torch.bfloat16, (H,)))
        specs += [("gate", f8, (E, I, H)), ("gate_scale", f32, (E, bi, bh)), ("up", f8, (E, I, H)),
                  ("up_scale", f32, (E, bi, bh)), ("down", f8, (E, H, I)), ("down_scale", f32, (E, bh, bi))]
        if S:
            bs = -(-(S * I) // 128)
            specs += [("shared_gate", f8, (S * I, H)), ("shared_gate_scale", f32, (bs, bh)),
                      ("shared_up", f8, (S * I, H)), ("shared_up_scale", f32, (bs, bh)),
                      ("shared_down", f8, (H, S * I)), ("shared_down_scale", f32, (bh, bs))]
        return tuple((name, dtype, torch.Size(shape)) for name, dtype, shape in specs)

    def _check(self, inputs: dict) -> torch.device:
        """The device of the inputs, after checking every input against the case; raises
        as _expect does (ValueError, or RuntimeError for inputs off the GPU)."""
        x = inputs.get("x")
        if not isinstance(x, torch.Tensor):
            raise ValueError("inputs must hold 'x'")
        device = x.device
        if device.type != "cuda":
            raise RuntimeError(f"the HIP layer runs on a GPU; inputs are on {device}")
        Tensor = torch.Tensor
        for name, dtype, shape in self._specs:
            t = inputs.get(name)
            if (not isinstance(t, Tensor) or t.dtype != dtype or t.shape != shape or t.device != device or
                    not t.is_contiguous()):
                _expect(t, name, dtype, shape, device)
        return device

    def workspace(self, device: torch.device) -> torch.Tensor:
        """The workspace of calls on torch's current stream of ``device``. Zeroed once when it
        is made: the single-launch kernel needs its control words zero when a call starts and
        leaves them zero when it ends (the other entry points need no initialisation)."""
        return self._workspace_on(device, _stream_handle(device))

    def _workspace_on(self, device: torch.device, stream: int) -> torch.Tensor:
        key = (device.index, stream)
        ws = self._workspace.get(key)
        if ws is None:
            ws = torch.zeros(self.workspace_bytes, dtype=torch.uint8, device=device)
            self._workspace[key] = ws
        return ws

    def check_mx_inputs(self, inputs: dict) -> torch.device:
        return self._check(inputs)

    def _call_mx(self, inputs: dict, events=None) -> dict:
        device = self._check(inputs)
        c = self.case
        y = torch.empty((c.tokens, c.hidden), dtype=torch.bfloat16, device=device)
        handle = _stream_handle(device)
        ws = self._workspace_on(device, handle)
        ptr = {name: inputs[name].data_ptr() for name in _lib.MX_TENSOR_FIELDS if name not in ("y", "workspace")}
        tensors = _lib.MxTensors(**ptr, y=y.data_ptr(), workspace=ws.data_ptr(), workspace_bytes=self.workspace_bytes)
        stream = ctypes.c_void_p(handle)
        handles = None if events is None else (ctypes.c_void_p * len(events))(*[e.cuda_event for e in events])
        forward = self.lib.megamoe_mx_layer_forward if self.single_launch else self.lib.megamoe_mx_forward
        with _on(device):
            _lib.check(forward(self._desc_ref, float(c.swiglu_limit), ctypes.byref(tensors), stream, handles),
                       f"{c.id}: forward")
        return {"y": y}

    def check_inputs(self, inputs: dict) -> torch.device:
        return self._check(inputs)

    def _call(self, inputs: dict, timed: bool, events=None, noalloc=False):
        if self.mx:
            if timed:
                raise ValueError("timed() covers the fp8 layer form; use record() for the MXFP4 form")
            return self._call_mx(inputs, events)
        device = self._check(inputs)
        c = self.case
        y = torch.empty((c.tokens, c.hidden), dtype=torch.bfloat16, device=device)
        ids = torch.empty((c.tokens, c.topk), dtype=torch.int64, device=device)
        weights = torch.empty((c.tokens, c.topk), dtype=torch.float32, device=device)
        handle = _stream_handle(device)
        ws = None if noalloc else self._workspace_on(device, handle)
        tensors = _lib.Tensors(*[inputs[name].data_ptr() if name in self._ptr_names else None for name in _INPUTS],
                               y.data_ptr(), ids.data_ptr(), weights.data_ptr(),
                               None if ws is None else ws.data_ptr(), 0 if ws is None else self.workspace_bytes)
        stream = ctypes.c_void_p(handle)
        with _on(device):
            if self.single_launch and not noalloc:
                blk = None
                if self.block is not None:
                    blk = ctypes.byref(_lib.Block(norm_weight=inputs["ln2"].data_ptr() if c.norm != "none" else None,
                                                  eps=float(c.norm_eps), weight_in_fp32=int(c.norm == "fp32_weight"),
                                                  residual=int(c.residual)))
                handles = None if events is None else (ctypes.c_void_p * 2)(*[e.cuda_event for e in events])
                forward = self.lib.megamoe_layer_forward_w8a16 if self.a16 else self.lib.megamoe_layer_forward
                _lib.check(forward(self._desc_ref, ctypes.byref(tensors), blk, self._epi_ref, stream, handles),
                           f"{c.id}: forward")
                return {"y": y, "expert_ids": ids, "expert_weights": weights}
            if noalloc:
                if self.block is not None or self.epilogue is not None or self.a16 or timed or events is not None:
                    raise ValueError("the no-allocation entry point covers the plain layer form")
                _lib.check(self.lib.megamoe_forward_noalloc(ctypes.byref(self.desc), ctypes.byref(tensors), stream),
                           f"{c.id}: forward (no allocation)")
                return {"y": y, "expert_ids": ids, "expert_weights": weights}
            if self.a16:
                if timed:
                    raise ValueError("the W8A16 form runs through megamoe_forward_w8a16 (use record() for stages)")
                blk = None
                if self.block is not None:
                    blk = ctypes.byref(_lib.Block(norm_weight=inputs["ln2"].data_ptr() if c.norm != "none" else None,
                                                  eps=float(c.norm_eps), weight_in_fp32=int(c.norm == "fp32_weight"),
                                                  residual=int(c.residual)))
                handles = (None if events is None else
                           (ctypes.c_void_p * len(events))(*[e.cuda_event for e in events]))
                _lib.check(self.lib.megamoe_forward_w8a16(ctypes.byref(self.desc), ctypes.byref(tensors), blk,
                                                          self._epi_ref, stream, handles), f"{c.id}: forward")
                return {"y": y, "expert_ids": ids, "expert_weights": weights}
            if self.block is not None or self.epilogue is not None:
                if timed:
                    raise ValueError("timed() covers the plain layer form; use record() for the block form and "
                                     "the epilogue variants")
                blk = None
                if self.block is not None:
                    blk = ctypes.byref(_lib.Block(norm_weight=inputs["ln2"].data_ptr() if c.norm != "none" else None,
                                                  eps=float(c.norm_eps), weight_in_fp32=int(c.norm == "fp32_weight"),
                                                  residual=int(c.residual)))
                epi = None if self.epilogue is None else ctypes.byref(self.epilogue)
                handles = (None if events is None else
                           (ctypes.c_void_p * len(events))(*[e.cuda_event for e in events]))
                _lib.check(self.lib.megamoe_forward_ex(ctypes.byref(self.desc), ctypes.byref(tensors), blk, epi,
                                                       stream, handles), f"{c.id}: forward")
                return {"y": y, "expert_ids": ids, "expert_weights": weights}
            if events is not None:
                handles = (ctypes.c_void_p * len(events))(*[e.cuda_event for e in events])
                _lib.check(self.lib.megamoe_forward_events(ctypes.byref(self.desc), ctypes.byref(tensors), stream,
                                                           handles), f"{c.id}: forward")
                return {"y": y, "expert_ids": ids, "expert_weights": weights}
            if timed:
                ms = (ctypes.c_float * len(_lib.STAGES))()
                _lib.check(self.lib.megamoe_forward_timed(ctypes.byref(self.desc), ctypes.byref(tensors), stream,
                                                          ms), f"{c.id}: forward")
                return {"y": y, "expert_ids": ids, "expert_weights": weights}, list(ms)
            _lib.check(self.lib.megamoe_forward(ctypes.byref(self.desc), ctypes.byref(tensors), stream),
                       f"{c.id}: forward")
        return {"y": y, "expert_ids": ids, "expert_weights": weights}

    def __call__(self, inputs: dict) -> dict:
        return self._call(inputs, timed=False)

    def gave_up(self, device: torch.device) -> bool:
        """Whether the last single-launch call on this (device, current stream)'s workspace had
        a bounded wait give up, or (the MXFP4 form) bad expert ids; its y is NaN then.
        Synchronizes the stream (megamoe_layer_status / megamoe_mx_layer_status)."""
        ws = self.workspace(device)
        flag = ctypes.c_int32(0)
        stream = ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)
        status = self.lib.megamoe_mx_layer_status if self.mx else self.lib.megamoe_layer_status
        with torch.cuda.device(device):
            _lib.check(status(ctypes.byref(self.desc), ws.data_ptr(), self.workspace_bytes, ctypes.byref(flag), stream),
                       f"{self.case.id}: status")
        return bool(flag.value)

    def noalloc(self, inputs: dict) -> dict:
        """One call of megamoe_forward_noalloc: the library's fixed device scratch stands in
        for the workspace (the outputs are still allocated here, as the caller's)."""
        return self._call(inputs, timed=False, noalloc=True)

    def timed(self, inputs: dict) -> tuple[dict, list[float]]:
        """One call with a device event between stages; returns (outputs, per-stage ms)."""
        if self.single_launch:
            events = [torch.cuda.Event(enable_timing=True) for _ in range(2)]
            for e in events:
                e.record()  # creates the HIP event
            out = self._call(inputs, timed=False, events=events)
            events[1].synchronize()
            return out, [events[0].elapsed_time(events[1])]
        return self._call(inputs, timed=True)

    def record(self, inputs: dict, events) -> dict:
        """One asynchronous call that records ``events`` (len(STAGES) + 1 torch.cuda.Event
        objects, each recorded once before so its HIP event exists) at the stage boundaries."""
        if len(events) != len(self.stages) + 1 or not all(e.cuda_event for e in events):
            raise ValueError("record() takes len(self.stages) + 1 created events")
        return self._call(inputs, timed=False, events=events)


def build(case: dict):
    layer = MoELayer(Case.from_dict({k: v for k, v in case.items() if k != "execution"}))

    def run(inputs: dict) -> dict:
        return layer(inputs)

    run.layer = layer
    return run


# -- single-stage entry points (the C ABI's test surface) ---------------------------------

def quantize_rows(x: torch.Tensor, power_of_two: bool = False) -> tuple[torch.Tensor, torch.Tensor]:
    """E4M3 payload and fp32 scales per row per 128 columns of a bf16 [rows, cols] tensor."""
    if x.dtype != torch.bfloat16 or x.dim() != 2 or x.device.type != "cuda":
        raise ValueError("quantize_rows takes a 2-D bf16 GPU tensor")
    x = x.contiguous()
    rows, cols = x.shape
    q = torch.empty((rows, cols), dtype=torch.float8_e4m3fn, device=x.device)
    s = torch.empty((rows, -(-cols // 128)), dtype=torch.float32, device=x.device)
    lib = _lib.load()
    with torch.cuda.device(x.device):
        stream = ctypes.c_void_p(torch.cuda.current_stream(x.device).cuda_stream)
        _lib.check(lib.megamoe_quantize_rows(rows, cols, x.data_ptr(), q.data_ptr(), s.data_ptr(),
                                             int(power_of_two), stream), "quantize_rows")
    return q, s


def router_logits(case: Case, x: torch.Tensor, router: torch.Tensor) -> torch.Tensor:
    layer = MoELayer(case)
    logits = torch.empty((case.tokens, case.experts), dtype=torch.float32, device=x.device)
    ws = layer.workspace(x.device)
    with torch.cuda.device(x.device):
        stream = ctypes.c_void_p(torch.cuda.current_stream(x.device).cuda_stream)
        _lib.check(layer.lib.megamoe_router_logits(ctypes.byref(layer.desc), x.contiguous().data_ptr(),
                                                   router.contiguous().data_ptr(), logits.data_ptr(),
                                                   ws.data_ptr(), layer.workspace_bytes, stream), "router_logits")
    return logits


def route(case: Case, logits: torch.Tensor, bias: torch.Tensor | None) -> tuple[torch.Tensor, torch.Tensor]:
    lib = _lib.load()
    desc = make_desc(case)
    T, K = logits.shape[0], case.topk
    desc.tokens = T
    ids = torch.empty((T, K), dtype=torch.int64, device=logits.device)
    w = torch.empty((T, K), dtype=torch.float32, device=logits.device)
    with torch.cuda.device(logits.device):
        stream = ctypes.c_void_p(torch.cuda.current_stream(logits.device).cuda_stream)
        _lib.check(lib.megamoe_route(ctypes.byref(desc), logits.contiguous().data_ptr(),
                                     None if bias is None else bias.contiguous().data_ptr(), ids.data_ptr(),
                                     w.data_ptr(), stream), "route")
    return ids, w


def combine_by_expert_id(expert_out: torch.Tensor, expert_ids: torch.Tensor, weights: torch.Tensor,
                         residual: torch.Tensor | None = None) -> torch.Tensor:
    """GPT-OSS's combine (gptoss.py:112-124) through megamoe_combine_by_expert_id: expert_out
    bf16 [T, K, H], expert_ids int64 [T, K], weights bf16 [T, K], residual bf16 [T, H] or None."""
    T, K, H = expert_out.shape
    device = expert_out.device
    _expect(expert_out, "expert_out", torch.bfloat16, (T, K, H), device)
    _expect(expert_ids, "expert_ids", torch.int64, (T, K), device)
    _expect(weights, "weights", torch.bfloat16, (T, K), device)
    if residual is not None:
        _expect(residual, "residual", torch.bfloat16, (T, H), device)
    y = torch.empty((T, H), dtype=torch.bfloat16, device=device)
    stream = ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)
    with torch.cuda.device(device):
        _lib.check(_lib.load().megamoe_combine_by_expert_id(
            T, H, K, expert_out.data_ptr(), expert_ids.data_ptr(), weights.data_ptr(),
            None if residual is None else residual.data_ptr(), y.data_ptr(), stream), "combine by expert id")
    return y


def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float, weight_in_fp32: bool) -> torch.Tensor:
    """RMSNorm of bf16 rows [rows, cols] with a bf16 gamma [cols] (common.py:13-21)."""
    if x.dtype != torch.bfloat16 or weight.dtype != torch.bfloat16 or x.dim() != 2 or x.device.type != "cuda":
        raise ValueError("rms_norm takes 2-D bf16 rows and a bf16 gamma on the GPU")
    x, weight = x.contiguous(), weight.contiguous()
    rows, cols = x.shape
    if tuple(weight.shape) != (cols,):
        raise ValueError(f"gamma has shape {tuple(weight.shape)}, expected ({cols},)")
    out = torch.empty_like(x)
    lib = _lib.load()
    with torch.cuda.device(x.device):
        stream = ctypes.c_void_p(torch.cuda.current_stream(x.device).cuda_stream)
        _lib.check(lib.megamoe_rms_norm(rows, cols, x.data_ptr(), weight.data_ptr(), float(eps),
                                        int(weight_in_fp32), out.data_ptr(), stream), "rms_norm")
    return out
