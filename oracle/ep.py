"""Expert parallelism of the MXFP4 layer, restated on the CPU (test infrastructure).

megabench/tasks/megamoe.py:153-182 with ``ep`` ranks, every rank emulated in one process:
  * owner of a (token, slot) = id // (E/ep) (:159-160);
  * the send order is a stable sort by owner (:161-164), so each destination receives a
    source's rows in (token, slot) order; the payload is the token's E4M3 row and E8M0
    scales, the global id and the weight (:165-168); the counts are the bincount of the
    owners (parallel.py:59-68);
  * the exchange (parallel.py:52-56) concatenates, per destination, the sources' segments in
    rank order; the reverse exchange hands each source its segments back;
  * each rank runs its local experts over the received rows with ids made local (:131-150,
    megamoe.py:174); each row's output is the serial layer's d row;
  * the source scatters the returned rows to (token, slot) and sums the slots in fp32 in
    slot order (:176-182).

Pinned by tests/test_oracle_ep.py: the send order against a per-owner listing by brute
force, the counts against numpy's bincount, and the whole emulation against the serial
layer of oracle/mx.py bit for bit at ep = 1, 2, 4 and 8 (the equality that
megabench/verify_megamoe.py:95-105 checks between the EP and serial runs).
"""

from __future__ import annotations

import numpy as np
import torch

from . import mx


def owner_order(ids: np.ndarray, local: int) -> np.ndarray:
    """Send order (send row -> flat (token, slot) index): stable by owner rank."""
    owner = np.asarray(ids).reshape(-1) // local
    return np.argsort(owner, kind="stable")


def dispatch(values: dict, experts: int, ep: int) -> dict:
    """The send payload of one rank's values, its counts and the slot -> send row map."""
    ids = values["topk_idx"].cpu()
    T, K = ids.shape
    local = experts // ep
    flat = ids.reshape(-1).numpy()
    order = owner_order(flat, local)
    source = order // K
    slot_rows = np.empty(T * K, dtype=np.int64)
    slot_rows[order] = np.arange(T * K)
    return {"rows": values["x"].cpu().view(torch.uint8)[torch.from_numpy(source)],
            "row_scales": values["x_scales"].cpu()[torch.from_numpy(source)],
            "ids": torch.from_numpy(flat[order].copy()),
            "weights": values["topk_weights"].cpu().reshape(-1)[torch.from_numpy(order)],
            "counts": np.bincount(flat // local, minlength=ep).astype(np.int64),
            "slot_rows": torch.from_numpy(slot_rows.reshape(T, K))}


def experts(case, weights: dict, rows: torch.Tensor, row_scales: torch.Tensor, ids: torch.Tensor,
            wts: torch.Tensor, base: int, *, widen: bool = False) -> torch.Tensor:
    """megamoe.py:131-150 on the received rows: bf16 [R, H], each row's weighted d."""
    R = rows.shape[0]
    if R == 0:
        return torch.empty((0, case.hidden), dtype=torch.float32 if widen else torch.bfloat16)
    one = {"x": rows.view(torch.float8_e4m3fn), "x_scales": row_scales, "topk_idx": (ids - base)[:, None],
           "topk_weights": wts[:, None], **weights}
    return mx.layer(case, one, widen=widen)["y"]


def combine(returned: torch.Tensor, slot_rows: torch.Tensor) -> torch.Tensor:
    T, K = slot_rows.shape
    acc = torch.zeros((T, returned.shape[1]), dtype=torch.float32)
    for k in range(K):
        acc = acc + returned[slot_rows[:, k]].float()
    return acc.to(returned.dtype)


def emulate(case, values: dict, ep: int, *, widen: bool = False) -> torch.Tensor:
    """y of the serial problem in ``values`` computed as ``ep`` ranks would: rank r holds
    tokens [r*T/ep, (r+1)*T/ep) and experts [r*E/ep, (r+1)*E/ep)."""
    T, E = values["x"].shape[0], case.experts
    if T % ep or E % ep:
        raise ValueError("ep must divide the tokens and the experts")
    t, local = T // ep, E // ep
    sends = [dispatch({k: values[k][r * t:(r + 1) * t] for k in ("x", "x_scales", "topk_idx", "topk_weights")},
                      E, ep) for r in range(ep)]
    starts = [np.concatenate(([0], np.cumsum(s["counts"]))) for s in sends]
    outputs = []
    for d in range(ep):
        seg = [slice(int(starts[r][d]), int(starts[r][d + 1])) for r in range(ep)]
        received = {k: torch.cat([sends[r][k][seg[r]] for r in range(ep)])
                    for k in ("rows", "row_scales", "ids", "weights")}
        weights = {k: values[k][d * local:(d + 1) * local] for k in ("l1_blocks", "l1_scales", "l2_blocks",
                                                                        "l2_scales")}
        out = experts(case, weights, received["rows"], received["row_scales"], received["ids"],
                      received["weights"], d * local, widen=widen)
        sizes = [seg[r].stop - seg[r].start for r in range(ep)]
        outputs.append(torch.split(out, sizes))
    ys = []
    for r in range(ep):
        returned = torch.cat([outputs[d][r] for d in range(ep)])
        ys.append(combine(returned, sends[r]["slot_rows"]))
    return torch.cat(ys)
