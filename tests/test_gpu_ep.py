"""GPU parity of one rank's share of the expert-parallel MXFP4 layer (megamoe.py:153-182),
through the C ABI (megamoe_ep_dispatch, megamoe_ep_experts, megamoe_ep_combine).

Every rank of an EP run is emulated in this one process, on the one GPU: each rank's
dispatch and combine run on its own tokens, its local experts on the rows it receives; the
two exchanges between them (collectives in a real run) are torch.cat/split of the send
segments here. Checks:
  * the dispatch equals the oracle's bit for bit (order, payload, counts, slot rows);
  * the emulated EP result equals the serial layer's (megamoe_mx_forward) bit for bit, the
    check megabench/verify_megamoe.py:95-105 makes (the two runs use the same down-projection
    split at these geometries, a condition the layer states);
  * it is within the layer tolerance of oracle.mx.reference and the band of the widened
    oracle;
  * at the catalog share geometry (rank 0 of megamoe-layer-deepseek-v4-pro-ep8-t512) the
    local experts' rows for a sample of experts against the oracle;
  * out-of-range ids: -1 counts from the dispatch, NaN from the experts and the combine.
"""

from __future__ import annotations

import sys
from dataclasses import replace

import numpy as np
import pytest
import torch

from oracle import ep as OE
from oracle import metrics, mx
from vibe_megakernel_amd import cases as C
from vibe_megakernel_amd import ep as EP
from vibe_megakernel_amd import submission, workloads

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
EPCASE = C.case("megamoe-layer-deepseek-v4-pro-ep8-t512")
ROUTING = ("x", "x_scales", "topk_idx", "topk_weights")
WEIGHTS = ("l1_blocks", "l1_scales", "l2_blocks", "l2_scales")


def _log(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _dev(ranks, tokens=8, experts=16, topk=4, hidden=256, intermediate=256):
    return replace(EPCASE, id=f"ep-dev-r{ranks}", gpus=ranks, ep=ranks,
                   params=dict(tokens=tokens, experts=experts, topk=topk, hidden=hidden, intermediate=intermediate))


def _emulate(case, values):
    """y of every rank, concatenated, with the two exchanges done in-process."""
    ep, t, local = case.ep, case.tokens, case.experts // case.ep
    sends = [EP.dispatch(*(values[k][r * t:(r + 1) * t] for k in ROUTING), case.experts, ep) for r in range(ep)]
    counts = [EP.send_counts(s) for s in sends]
    starts = [np.concatenate(([0], np.cumsum(c))) for c in counts]
    outputs = []
    for d in range(ep):
        seg = [slice(int(starts[r][d]), int(starts[r][d + 1])) for r in range(ep)]
        rows = torch.cat([sends[r].rows[seg[r]] for r in range(ep)])
        scales = torch.cat([sends[r].row_scales[seg[r]] for r in range(ep)])
        ids = torch.cat([sends[r].ids[seg[r]] for r in range(ep)])
        wts = torch.cat([sends[r].weights[seg[r]] for r in range(ep)])
        experts = EP.Experts(*(values[k][d * local:(d + 1) * local] for k in WEIGHTS), d * local,
                             case.swiglu_limit)
        out = experts(rows, scales, ids, wts)
        outputs.append(torch.split(out, [s.stop - s.start for s in seg]))
    ys = [EP.combine(torch.cat([outputs[d][r] for d in range(ep)]), sends[r].slot_rows) for r in range(ep)]
    return torch.cat(ys), sends


def test_dispatch_matches_oracle():
    case = _dev(4, tokens=13)
    _log(f"ep dispatch {case.id}")
    values = workloads.make_mx_inputs(workloads.serial_case(case), 21)
    gpu = {k: v.to(DEV) for k, v in values.items()}
    for r in range(case.ep):
        part = {k: values[k][r * case.tokens:(r + 1) * case.tokens] for k in ROUTING}
        want = OE.dispatch(part, case.experts, case.ep)
        got = EP.dispatch(*(gpu[k][r * case.tokens:(r + 1) * case.tokens].contiguous() for k in ROUTING),
                          case.experts, case.ep)
        assert EP.send_counts(got) == want["counts"].tolist()
        assert torch.equal(got.slot_rows.cpu().long(), want["slot_rows"])
        assert torch.equal(got.rows.cpu().view(torch.uint8), want["rows"])
        assert torch.equal(got.row_scales.cpu(), want["row_scales"])
        assert torch.equal(got.ids.cpu(), want["ids"])
        assert torch.equal(got.weights.cpu(), want["weights"])


@pytest.mark.parametrize("ranks,intermediate,tokens,experts", [(1, 256, 8, 16), (2, 256, 8, 16), (8, 256, 8, 16),
                                                               (4, 512, 8, 16), (2, 256, 96, 4)])
def test_expert_parallel_equals_serial_bitwise(ranks, intermediate, tokens, experts):
    """(2, 256, 96, 4): about 96 rows per expert, worked by wide units on both sides."""
    case = _dev(ranks, intermediate=intermediate, tokens=tokens, experts=experts, topk=min(4, experts))
    serial = workloads.serial_case(case)
    _log(f"ep vs serial ranks={ranks} I={intermediate} T={tokens} E={experts}")
    for seed in (104729, 104730):
        values = workloads.make_mx_inputs(serial, seed)
        gpu = {k: v.to(DEV) for k, v in values.items()}
        y_ep, _ = _emulate(case, gpu)
        y_serial = submission.build(serial.to_dict())(gpu)["y"]
        torch.cuda.synchronize()
        assert torch.equal(y_ep, y_serial), f"ranks={ranks} seed={seed}"
        want, exact = mx.reference(serial, values)["y"], mx.oracle(serial, values)["y"]
        check = metrics.layer_checks(y_ep.cpu(), want)
        assert check["pass"], check
        band = metrics.band(want, y_ep.cpu(), exact, bf16_rtol=case.bf16_rtol, noise_factor=case.noise_factor)
        assert band["pass"], band


def test_share_at_catalog_geometry_on_sampled_experts():
    """Rank 0 of the catalog case: its dispatch, its 48 local experts over the rows all 8 ranks
    send it, its combine; the experts' rows of three local experts against the oracle."""
    case = EPCASE
    _log(f"ep share {case.id}")
    values = workloads.make_ep_inputs(case, 104729, DEV, rank=0)
    t, local = case.tokens, case.experts // case.ep
    sends = [EP.dispatch(*(values[k][r * t:(r + 1) * t] for k in ROUTING), case.experts, case.ep)
             for r in range(case.ep)]
    counts = [EP.send_counts(s) for s in sends]
    rows = torch.cat([s.rows[:c[0]] for s, c in zip(sends, counts)])
    scales = torch.cat([s.row_scales[:c[0]] for s, c in zip(sends, counts)])
    ids = torch.cat([s.ids[:c[0]] for s, c in zip(sends, counts)])
    wts = torch.cat([s.weights[:c[0]] for s, c in zip(sends, counts)])
    out = EP.Experts(*(values[k] for k in WEIGHTS), 0, case.swiglu_limit)(rows, scales, ids, wts)
    torch.cuda.synchronize()
    _log(f"  rank 0 receives {rows.shape[0]} rows")
    assert torch.isfinite(out.float()).all()
    ids_cpu = ids.cpu()
    hot = torch.bincount(ids_cpu, minlength=local)
    for e in (int(hot.argmax()), int(hot.argmin()), local // 2):
        sel = (ids_cpu == e).nonzero().flatten()
        if sel.numel() == 0:
            continue
        weights = {k: values[k][e:e + 1].cpu() for k in WEIGHTS}
        args = (rows.cpu()[sel].view(torch.uint8), scales.cpu()[sel], ids_cpu[sel], wts.cpu()[sel])
        want = OE.experts(case, weights, *args, base=e)
        exact = OE.experts(case, weights, *args, base=e, widen=True)
        got = out.cpu()[sel]
        check = metrics.layer_checks(got, want)
        assert check["pass"], (e, check)
        band = metrics.band(want, got, exact, bf16_rtol=case.bf16_rtol, noise_factor=case.noise_factor)
        assert band["pass"], (e, band)
        _log(f"  expert {e}: {sel.numel()} rows {check}")


def test_out_of_range_ids():
    case = _dev(2)
    _log("ep bad ids")
    values = {k: v.to(DEV) for k, v in workloads.make_mx_inputs(workloads.serial_case(case), 3).items()}
    bad = values["topk_idx"][:case.tokens].clone()
    bad[1, 2] = case.experts
    send = EP.dispatch(values["x"][:case.tokens], values["x_scales"][:case.tokens], bad,
                       values["topk_weights"][:case.tokens], case.experts, case.ep)
    with pytest.raises(ValueError):
        EP.send_counts(send)
    assert bool((send.slot_rows == -1).all())
    y = EP.combine(torch.zeros((case.tokens * case.topk, case.hidden), dtype=torch.bfloat16, device=DEV),
                   send.slot_rows)
    assert torch.isnan(y.float()).all()
    # Local experts given a row of another rank's expert: NaN everywhere.
    local = case.experts // case.ep
    experts = EP.Experts(*(values[k][:local] for k in WEIGHTS), 0, case.swiglu_limit)
    n = 5
    ids = torch.tensor([0, 1, local, 2, 0], dtype=torch.int64, device=DEV)
    out = experts(values["x"][:n], values["x_scales"][:n], ids, values["topk_weights"][:n, 0].contiguous())
    assert torch.isnan(out.float()).all()


def test_empty_share():
    case = _dev(2)
    _log("ep empty")
    H = case.hidden
    z8 = torch.empty((0, H), dtype=torch.float8_e4m3fn, device=DEV)
    zs = torch.empty((0, H // 32), dtype=torch.uint8, device=DEV)
    send = EP.dispatch(z8, zs, torch.empty((0, case.topk), dtype=torch.int64, device=DEV),
                       torch.empty((0, case.topk), dtype=torch.float32, device=DEV), case.experts, case.ep)
    assert EP.send_counts(send) == [0] * case.ep
    values = {k: v.to(DEV) for k, v in workloads.make_mx_inputs(workloads.serial_case(case), 3).items()}
    local = case.experts // case.ep
    out = EP.Experts(*(values[k][:local] for k in WEIGHTS), 0, case.swiglu_limit)(
        z8, zs, torch.empty(0, dtype=torch.int64, device=DEV), torch.empty(0, dtype=torch.float32, device=DEV))
    assert out.shape == (0, H)


def test_worst_case_received_rows():
    """A rank that receives every row its 8 senders can send it (ep 8 x 512 tokens x 6 slots =
    24576 rows over its 48 local experts, heavily skewed): beyond the permute's token bitmap,
    so the ranking runs in tiles. Each row's result depends only on the row and its expert,
    so the call equals the same rows worked in eight calls of 3072 (bitmap form), bit for bit,
    and sampled experts are within the layer's bars of the oracle."""
    local, R, H, I = 48, 24576, 256, 256
    case = replace(EPCASE, id="ep-worst", params=dict(tokens=R, experts=local, topk=1, hidden=H, intermediate=I))
    _log(f"ep worst case: {R} received rows over {local} local experts")
    serial = replace(case, gpus=1, ep=1)
    values = workloads.make_mx_inputs(serial, 77)
    g = torch.Generator().manual_seed(5)
    # Zipf-like skew: expert e with weight (e+1)^-1.1, a few hot experts
    p = torch.arange(1, local + 1, dtype=torch.float64).pow(-1.1)
    ids = torch.multinomial(p / p.sum(), R, replacement=True, generator=g).to(torch.int64)
    gpu = {k: v.to(DEV) for k, v in values.items()}
    rows, scales = gpu["x"], gpu["x_scales"]
    wts = gpu["topk_weights"][:, 0].contiguous()
    experts = EP.Experts(*(gpu[k] for k in WEIGHTS), 0, case.swiglu_limit)
    ids_d = ids.to(DEV)
    whole = experts(rows, scales, ids_d, wts)
    parts = torch.cat([experts(rows[i:i + 3072], scales[i:i + 3072], ids_d[i:i + 3072], wts[i:i + 3072])
                       for i in range(0, R, 3072)])
    torch.cuda.synchronize()
    assert torch.isfinite(whole.float()).all()
    assert torch.equal(whole, parts)
    hot = torch.bincount(ids, minlength=local)
    for e in (int(hot.argmax()), int(hot.argmin())):
        sel = (ids == e).nonzero().flatten()[:64]
        weights = {k: values[k][e:e + 1] for k in WEIGHTS}
        args = (values["x"][sel].view(torch.uint8), values["x_scales"][sel], ids[sel], values["topk_weights"][sel, 0])
        want = OE.experts(case, weights, *args, base=e)
        exact = OE.experts(case, weights, *args, base=e, widen=True)
        got = whole.cpu()[sel]
        assert metrics.layer_checks(got, want)["pass"], e
        assert metrics.band(want, got, exact, bf16_rtol=case.bf16_rtol, noise_factor=case.noise_factor)["pass"], e


def test_batch_share_on_few_experts_equals_small_calls():
    """Batch mode (k_experts_mx_batch: 3072 rows for 128 local experts, H 2048, I 512, no K
    split) with the rows on 3 experts (1800, 900 and 372 rows: chunk groups of 29, 15 and 6),
    so 4 of the 8 per-XCD ranges of its work list are empty and their workgroups take units
    from other XCDs' queues. Each row's result depends only on the row and its expert, so the
    call equals the same rows worked in calls of 32 (decode units), bit for bit, and sampled
    experts are within the layer's bars of the oracle."""
    local, H, I = 128, 2048, 512
    per_expert = {3: 1800, 60: 900, 127: 372}
    R = sum(per_expert.values())
    case = replace(EPCASE, id="ep-few", params=dict(tokens=R, experts=local, topk=1, hidden=H, intermediate=I))
    _log(f"ep batch on few experts: {R} rows over {len(per_expert)} of {local} experts")
    serial = replace(case, gpus=1, ep=1)
    gpu = workloads.make_mx_inputs(serial, 91, DEV)
    ids = torch.cat([torch.full((n,), e, dtype=torch.int64) for e, n in per_expert.items()])
    ids = ids[torch.randperm(R, generator=torch.Generator().manual_seed(3))]
    rows, scales = gpu["x"], gpu["x_scales"]
    wts = gpu["topk_weights"][:, 0].contiguous()
    experts = EP.Experts(*(gpu[k] for k in WEIGHTS), 0, case.swiglu_limit)
    ids_d = ids.to(DEV)
    from torch.profiler import ProfilerActivity, profile

    with profile(activities=[ProfilerActivity.CPU, ProfilerActivity.CUDA]) as prof:
        whole = experts(rows, scales, ids_d, wts)
        torch.cuda.synchronize()
    kernels = [e.name for e in prof.events() if e.device_type == torch.autograd.DeviceType.CUDA]
    assert any("k_experts_mx_batch" in k for k in kernels), kernels
    parts = torch.cat([experts(rows[i:i + 32], scales[i:i + 32], ids_d[i:i + 32], wts[i:i + 32])
                       for i in range(0, R, 32)])
    torch.cuda.synchronize()
    assert torch.isfinite(whole.float()).all()
    assert torch.equal(whole, parts)
    x, xs, w0 = gpu["x"].cpu(), gpu["x_scales"].cpu(), gpu["topk_weights"][:, 0].cpu()
    for e in per_expert:
        sel = (ids == e).nonzero().flatten()[:64]
        weights = {k: gpu[k][e:e + 1].cpu() for k in WEIGHTS}
        args = (x[sel].view(torch.uint8), xs[sel], ids[sel], w0[sel])
        want = OE.experts(case, weights, *args, base=e)
        exact = OE.experts(case, weights, *args, base=e, widen=True)
        got = whole.cpu()[sel]
        assert metrics.layer_checks(got, want)["pass"], e
        assert metrics.band(want, got, exact, bf16_rtol=case.bf16_rtol, noise_factor=case.noise_factor)["pass"], e
