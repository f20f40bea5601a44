"""One rank's share of the expert-parallel MXFP4 layer (megabench/tasks/megamoe.py:153-182).

Under expert parallelism over ``ep`` ranks, rank r owns experts [r*E/ep, (r+1)*E/ep) and
holds only their weights. ``reference`` there runs, per rank:

1. ``dispatch``: owner = id // (E/ep) per (token, slot); the rows in a stable order by owner
   (megamoe.py:160-164), the payload of FP8 rows, E8M0 scales, global ids and weights
   gathered in that order (:165-168), and the per-destination counts
   (``exchange_counts``, parallel.py:59-68);
2. the exchange of counts and payload (``all_to_all_single``, parallel.py:52-56);
3. ``experts`` over the received rows (:131-150, ids made local);
4. the exchange back;
5. ``combine``: outputs scattered to their (token, slot) and summed over slots in fp32 in
   slot order (:176-182).

This module holds steps 1, 3 and 5 on the GPU through libmegamoe.so (megamoe_ep_dispatch,
megamoe_ep_experts, megamoe_ep_combine); steps 2 and 4 are the caller's collectives and are
not part of this library. Every call is issued on torch's current stream.
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass

import torch

from . import _lib


def _check(t: torch.Tensor, name: str, dtype, shape, device) -> None:
    if not isinstance(t, torch.Tensor):
        raise ValueError(f"{name}: expected a tensor")
    if t.dtype != dtype or tuple(t.shape) != tuple(shape):
        raise ValueError(f"{name}: expected {tuple(shape)} {dtype}, got {tuple(t.shape)} {t.dtype}")
    if t.device != device or not t.is_contiguous():
        raise ValueError(f"{name}: must be contiguous on {device}")


def _stream(device) -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


@dataclass
class Send:
    """The dispatch of one rank: rows in owner order and where each (token, slot) went."""
    rows: torch.Tensor        # e4m3fn [T*K, H]
    row_scales: torch.Tensor  # uint8 [T*K, H/32]
    ids: torch.Tensor         # int64 [T*K] global expert ids
    weights: torch.Tensor     # fp32 [T*K]
    counts: torch.Tensor      # int64 [ep] rows per destination rank (on the device)
    slot_rows: torch.Tensor   # int32 [T, K] send row of each (token, slot)


def dispatch(x: torch.Tensor, x_scales: torch.Tensor, topk_idx: torch.Tensor, topk_weights: torch.Tensor,
             experts: int, ep: int, send: Send | None = None) -> Send:
    """megamoe.py:160-168 and parallel.py:59-68 (the send half) for this rank's tokens.
    ``send`` (from an earlier call of the same shape) is reused instead of allocating."""
    T, H = x.shape
    K = topk_idx.shape[1] if topk_idx.dim() == 2 else 0
    device = x.device
    if device.type != "cuda":
        raise RuntimeError(f"the HIP layer runs on a GPU; inputs are on {device}")
    if ep <= 0 or experts % ep:
        raise ValueError(f"ep={ep} must divide experts={experts}")
    _check(x, "x", torch.float8_e4m3fn, (T, H), device)
    _check(x_scales, "x_scales", torch.uint8, (T, H // 32), device)
    _check(topk_idx, "topk_idx", torch.int64, (T, K), device)
    _check(topk_weights, "topk_weights", torch.float32, (T, K), device)
    n = T * K
    if send is None:
        send = Send(rows=torch.empty((n, H), dtype=torch.float8_e4m3fn, device=device),
                    row_scales=torch.empty((n, H // 32), dtype=torch.uint8, device=device),
                    ids=torch.empty(n, dtype=torch.int64, device=device),
                    weights=torch.empty(n, dtype=torch.float32, device=device),
                    counts=torch.empty(ep, dtype=torch.int64, device=device),
                    slot_rows=torch.empty((T, K), dtype=torch.int32, device=device))
    else:
        _check(send.rows, "send.rows", torch.float8_e4m3fn, (n, H), device)
        _check(send.row_scales, "send.row_scales", torch.uint8, (n, H // 32), device)
        _check(send.ids, "send.ids", torch.int64, (n,), device)
        _check(send.weights, "send.weights", torch.float32, (n,), device)
        _check(send.counts, "send.counts", torch.int64, (ep,), device)
        _check(send.slot_rows, "send.slot_rows", torch.int32, (T, K), device)
    lib = _lib.load()
    desc = _lib.Desc(tokens=T, hidden=H, experts=experts, topk=K)
    src = _lib.MxTensors(x=x.data_ptr(), x_scales=x_scales.data_ptr(), topk_idx=topk_idx.data_ptr(),
                         topk_weights=topk_weights.data_ptr())
    dst = _lib.EpSend(**{name: getattr(send, name).data_ptr() for name in _lib.EP_SEND_FIELDS})
    with torch.cuda.device(device):
        _lib.check(lib.megamoe_ep_dispatch(ctypes.byref(desc), int(ep), ctypes.byref(src), ctypes.byref(dst),
                                           _stream(device)), "ep dispatch")
    return send


def send_counts(send: Send) -> list[int]:
    """Host copy of the per-destination counts (as exchange_counts' ``send.tolist()``); a
    dispatch that met an expert id outside [0, E) reports -1 counts and raises here."""
    counts = send.counts.tolist()
    if any(c < 0 for c in counts):
        raise ValueError("ep dispatch: an expert id is outside [0, experts)")
    return counts


class Experts:
    """The local experts of one rank (megamoe.py:131-150) over the rows it receives."""

    def __init__(self, l1_blocks: torch.Tensor, l1_scales: torch.Tensor, l2_blocks: torch.Tensor,
                 l2_scales: torch.Tensor, expert_base: int, swiglu_limit: float):
        local, two_i, hb, _ = l1_blocks.shape
        self.local, self.inter, self.hidden = local, two_i // 2, hb * 32
        device = l1_blocks.device
        H, I = self.hidden, self.inter
        _check(l1_blocks, "l1_blocks", torch.uint8, (local, 2 * I, H // 32, 16), device)
        _check(l1_scales, "l1_scales", torch.uint8, (local, 2 * I, H // 32), device)
        _check(l2_blocks, "l2_blocks", torch.uint8, (local, H, I // 32, 16), device)
        _check(l2_scales, "l2_scales", torch.uint8, (local, H, I // 32), device)
        self.weights = (l1_blocks, l1_scales, l2_blocks, l2_scales)
        self.expert_base, self.limit = int(expert_base), float(swiglu_limit)
        self.lib = _lib.load()
        self._ws_bytes: dict[int, int] = {}

    def desc(self, rows: int) -> _lib.Desc:
        return _lib.Desc(tokens=rows, hidden=self.hidden, experts=self.local, topk=1, intermediate=self.inter)

    def workspace_bytes(self, rows: int) -> int:
        if rows not in self._ws_bytes:
            size = ctypes.c_size_t(0)
            _lib.check(self.lib.megamoe_mx_workspace_bytes(ctypes.byref(self.desc(rows)), ctypes.byref(size)),
                       "ep experts: workspace size")
            self._ws_bytes[rows] = int(size.value)
        return self._ws_bytes[rows]

    def __call__(self, rows: torch.Tensor, row_scales: torch.Tensor, ids: torch.Tensor, weights: torch.Tensor,
                 *, workspace: torch.Tensor | None = None, out: torch.Tensor | None = None,
                 events=None) -> torch.Tensor:
        """bf16 [R, H]: each received row's weighted expert output (the returned payload),
        into ``out`` when given."""
        R, H = rows.shape[0], self.hidden
        device = rows.device
        _check(rows, "rows", torch.float8_e4m3fn, (R, H), device)
        _check(row_scales, "row_scales", torch.uint8, (R, H // 32), device)
        _check(ids, "ids", torch.int64, (R,), device)
        _check(weights, "weights", torch.float32, (R,), device)
        desc = self.desc(R)
        need = self.workspace_bytes(R)
        if workspace is None:
            workspace = torch.empty(need, dtype=torch.uint8, device=device)
        elif workspace.numel() < need:
            raise ValueError(f"ep experts: workspace of {workspace.numel()} bytes, {need} needed")
        if out is None:
            out = torch.empty((R, H), dtype=torch.bfloat16, device=device)
        else:
            _check(out, "out", torch.bfloat16, (R, H), device)
        l1, l1s, l2, l2s = self.weights
        t = _lib.MxTensors(x=rows.data_ptr(), x_scales=row_scales.data_ptr(), topk_idx=ids.data_ptr(),
                           topk_weights=weights.data_ptr(), l1_blocks=l1.data_ptr(), l1_scales=l1s.data_ptr(),
                           l2_blocks=l2.data_ptr(), l2_scales=l2s.data_ptr(), y=out.data_ptr(),
                           workspace=workspace.data_ptr(), workspace_bytes=workspace.numel())
        handles = None if events is None else (ctypes.c_void_p * len(events))(*[e.cuda_event for e in events])
        with torch.cuda.device(device):
            _lib.check(self.lib.megamoe_ep_experts(ctypes.byref(desc), self.limit, self.expert_base, ctypes.byref(t),
                                                   _stream(device), handles), "ep experts")
        return out


def combine(returned: torch.Tensor, slot_rows: torch.Tensor, y: torch.Tensor | None = None) -> torch.Tensor:
    """megamoe.py:176-182: y[t] = bf16(sum over slots in order of fp32(returned[slot_rows[t, k]])),
    into ``y`` when given."""
    T, K = slot_rows.shape
    H = returned.shape[1]
    device = returned.device
    _check(returned, "returned", torch.bfloat16, (T * K, H), device)
    _check(slot_rows, "slot_rows", torch.int32, (T, K), device)
    if y is None:
        y = torch.empty((T, H), dtype=torch.bfloat16, device=device)
    else:
        _check(y, "y", torch.bfloat16, (T, H), device)
    with torch.cuda.device(device):
        _lib.check(_lib.load().megamoe_ep_combine(T, H, K, returned.data_ptr(), slot_rows.data_ptr(), y.data_ptr(),
                                                  _stream(device)), "ep combine")
    return y
