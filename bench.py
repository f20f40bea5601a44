"""Benchmark of the FP8 MoE decode layer on one MI355X.

    python bench.py [--steps K] [--warmup W] [--case ID | --all] [--no-cpu-baseline] [--cpu-budget S]

A step is one call of the layer (router, routing, permute, gate/up + SwiGLU,
down, combine) on one batch of synthetic inputs already resident in HBM. W
untimed steps, then K steps bracketed by torch.cuda.synchronize() and device
events; inputs are generated on the GPU (seed 7301). Before either form's warmup
steps the device runs the layer (stream-ordered form) for ~30 ms: after the idle
of input generation, the first ~20 calls run slower while the device ramps up
under this load (warm_device). Steps rotate over as many
independent input sets as it takes to move >= 1 GB per rotation, so the 256 MB
Infinity Cache cannot hold a step's weights.

Printed: one JSON line (rank 0) with the headline metric of the DeepSeek-V3
shape (or --case), the roofline of the dominant kernel (k_experts<false|true>:
gate/up + SwiGLU + down; k_experts_mx for the MXFP4 forms) and the CPU oracle timed on a
bounded sample. Without --case, the line's "configs" also holds the other four
BASELINE.json configs, each measured the same way (time, p50/p95, TB/s, roofline, its
own CPU baseline) in a child process; --all adds the other forms (the block forms, the
MXFP4 layer, rank 0's EP share, the epilogue variants). For an EP case a step is rank 0's
dispatch, local experts and combine (bench_ep_share).

The kernel's duration comes from a second loop of K steps in which the library
records HIP events at its stage boundaries on the stream its kernels run on
(megamoe_forward_events); the mean over those K launches divides the kernel's
algorithmic bytes. ``traffic`` (measured HBM bytes per launch) is read from the
committed rocprofv3 counter summary of the case, when there is one.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import platform
import statistics
import subprocess
import sys
import time
from pathlib import Path

REPO = Path(__file__).resolve().parent
sys.path.insert(0, str(REPO))

import __graft_entry__  # noqa: E402

PROFILES = REPO / "profiles"
PEAK_HBM = 8.0e12          # B/s, MI355X HBM3E
METRIC = "MoE decode layer \u00b5s/step + achieved HBM TB/s (% of peak), DeepSeek-V3 shape, 1 GPU"
PEAK_FP8 = 5.0e15          # flop/s, dense E4M3 MFMA
ROTATE_BYTES = 1.0e9


def _log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def kernel_bytes(case, hit: int) -> dict:
    """Algorithmic HBM bytes of the gate/up and down halves of the expert kernel for U = hit experts."""
    H, I, S, T, K = case.hidden, case.intermediate, case.shared_experts, case.tokens, case.topk
    rows = T * K
    if case.format == "mxfp4":
        # E2M1 weights (half a byte) + one E8M0 byte per 32; x (E4M3 + E8M0 per 32) in; h
        # (E4M3 + E8M0 per 32) out and in; d (bf16) out.
        gu = hit * (2 * I * H // 2 + 2 * I * H // 32) + T * H + T * H // 32 + rows * I + rows * I // 32
        dn = hit * (H * I // 2 + H * I // 32) + rows * I + rows * I // 32 + 2 * rows * H
        return {"gate_up": gu, "down": dn}
    bh, bi = math.ceil(H / 128), math.ceil(I / 128)
    gu = hit * (2 * I * H + 4 * 2 * bi * bh)
    dn = hit * (H * I + 4 * bh * bi)
    if S:
        bs = math.ceil(S * I / 128)
        gu += 2 * S * I * H + 4 * 2 * bs * bh
        dn += H * S * I + 4 * bh * bs
    if case.activations == "bf16":
        # W8A16: x (bf16) in, h (bf16) out / in, d out
        gu += 2 * T * H + 2 * rows * I + (2 * T * S * I if S else 0)
        dn += 2 * rows * I + 2 * rows * H + ((2 * T * S * I + 2 * T * H) if S else 0)
        return {"gate_up": gu, "down": dn}
    # activations in and out: x quantized (T*H + scales) in, h (rows * I + scales) out / in, d out
    gu += T * H + 4 * T * bh + rows * I + 4 * rows * bi + (T * S * I + 4 * T * math.ceil(S * I / 128) if S else 0)
    dn += rows * I + 4 * rows * bi + 2 * rows * H + ((T * S * I + 2 * T * H) if S else 0)
    return {"gate_up": gu, "down": dn}


def mx_kernel(rows: int, experts: int) -> str:
    """The MXFP4 expert kernel of the stream-ordered form: batch mode from 24 rows per expert
    on average (kBatchMinRows in the library), the decode kernel below."""
    return "k_experts_mx_batch" if rows >= 24 * experts else "k_experts_mx"


def _split(case) -> bool:
    """split_gate_up in csrc/megamoe.hip: the split gate/up form when the whole-block gate/up
    units cannot fill one round of a 512-workgroup grid with every expert hit and the rows
    have 32 or more K blocks (never in the W8A16 form)."""
    hit = min(case.experts, case.tokens * case.topk) + case.shared_experts
    return case.activations != "bf16" and hit * (case.intermediate // 128) < 512 and case.hidden // 128 >= 32


def fp8_kernel(case) -> str:
    """The FP8 expert kernel the library runs (k_experts<split, w8a16>)."""
    return f"k_experts<{str(_split(case)).lower()}, {str(case.activations == 'bf16').lower()}>"


def expert_kernel(case) -> str:
    """The expert kernel of the stream-ordered form."""
    if case.format == "mxfp4":
        return mx_kernel(case.tokens * case.topk, case.experts)
    return fp8_kernel(case)


def layer_kernel(case) -> str:
    """The single-launch kernel: k_layer for the fp8 forms (split gate/up as fp8_kernel),
    k_layer_mx for the MXFP4 form."""
    if case.format == "mxfp4":
        return "k_layer_mx"
    return f"k_layer<{str(_split(case)).lower()}, {str(case.activations == 'bf16').lower()}>"


def measured_traffic(case, kernel: str = "k_experts") -> float | None:
    """HBM bytes per launch of ``kernel`` from profiles/<kernel>_<case>_counters.md: the line
    ``traffic_bytes_per_launch: <number>`` (FETCH_SIZE + WRITE_SIZE, calibrated on a copy)."""
    path = PROFILES / f"{kernel}_{case.id}_counters.md"
    if not path.exists():
        return None
    for line in path.read_text().splitlines():
        if line.startswith("traffic_bytes_per_launch:"):
            return float(line.split(":", 1)[1])
    return None


def copy_probe(mib: int) -> None:
    """A plain device copy of ``mib`` MiB, three times: the calibration kernel that a
    rocprofv3 counter run of this script records beside k_experts."""
    import torch

    src = torch.ones(mib << 18, dtype=torch.float32, device="cuda:0")
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    _log(f"[bench] copy probe: 3 x {mib} MiB read + {mib} MiB written")


def cpu_model() -> str:
    """The host CPU's model name (/proc/cpuinfo), or the machine type where it is not listed."""
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or platform.machine()


def cpu_threads() -> int:
    n = len(os.sched_getaffinity(0))
    env = os.environ.get("OMP_NUM_THREADS", "")
    return min(n, int(env)) if env.isdigit() and int(env) > 0 else n


def parity_of(case, y, want: dict, exact: dict, ids=None) -> dict:
    """Outputs of a timed call against the CPU oracle on the same inputs, graded as the
    reference harness grades them: the band rule of megabench/harness/correctness.py:64-85
    against the FP32 oracle (the error may reach twice the BF16 reference's own), expert ids
    equal to the reference's, and cosine >= 0.9999 against the BF16 reference schedule. Also
    reported: max|y - y_ref| / max|y_ref| against that schedule and whether it is <= 1e-2
    ("max_rel_ok"); the reference's own max_rel against the oracle ("reference_max_rel")
    shows the noise floor of that figure on these inputs (an E4M3 requantization near a
    rounding tie turns an ulp of difference upstream into a step of 1/8)."""
    import torch

    from oracle import metrics

    y = y.cpu()
    check = metrics.layer_checks(y, want["y"])
    band = metrics.band(want["y"], y, exact["y"], bf16_rtol=case.bf16_rtol, noise_factor=case.noise_factor)
    ref = metrics.layer_checks(want["y"], exact["y"].to(torch.float32))
    out = {"rows": y.shape[0], "band_pass": band["pass"], "relative_error": band["relative_error"],
           "reference_relative_error": band["reference_relative_error"], "cosine": check["cosine"],
           "max_rel": check["max_rel"], "max_rel_ok": check["max_rel"] <= metrics.MAX_REL,
           "reference_max_rel": ref["max_rel"]}
    ok = band["pass"] and check["cosine"] >= metrics.MIN_COSINE
    if ids is not None and "expert_ids" in want:
        same = int((ids.cpu() == want["expert_ids"]).all(dim=1).sum())
        out["rows_with_equal_ids"] = same
        ok = ok and same == y.shape[0]
    out["ok"] = bool(ok)
    return out


def cpu_baseline(case, values_gpu, hit: int, budget_s: float, got: dict | None = None) -> dict:
    """The CPU oracle (BF16 schedule) on the first tokens of the same inputs, scaled by
    distinct experts computed (the oracle's cost is dominated by dequantizing each hit
    expert once). With ``got`` (the GPU outputs of a timed call on these inputs), the oracle's
    outputs on those tokens check them: the result's "parity" entry."""
    import torch

    from oracle import layer, mx

    threads = cpu_threads()
    torch.set_num_threads(threads)
    cpu = {k: v.cpu() for k, v in values_gpu.items()}
    sample = 1
    while True:
        rows = list(range(sample))
        t0 = time.perf_counter()
        if case.format == "mxfp4":
            reference, oracle = mx.reference, mx.oracle
        elif case.norm != "none" or case.residual:
            reference, oracle = layer.block_reference, layer.block_oracle
        else:
            reference, oracle = layer.reference, layer.oracle
        out = reference(case, cpu, tokens=rows)
        dt = time.perf_counter() - t0
        ids = cpu["topk_idx"][rows] if case.format == "mxfp4" else out["expert_ids"]
        sampled = len(set(ids.flatten().tolist()))
        if dt * 2 > budget_s or sample * 2 > case.tokens:
            break
        sample *= 2
    s = case.shared_experts
    scale = (hit + s) / max(sampled + s, 1)
    parity = None
    if got is not None:  # untimed: the FP32 oracle on the same tokens
        exact = oracle(case, cpu, tokens=rows)
        parity = parity_of(case, got["y"][rows], out, exact, got["expert_ids"][rows] if "expert_ids" in got else None)
        parity["tokens"] = parity.pop("rows")
    return {"value": dt * scale * 1e6, "unit": "us/step", "cores": threads, "kind": "port",
            "cpu_model": cpu_model(), "parity": parity,
            "sample": (f"oracle.{reference.__module__.split('.')[-1]}.{reference.__name__} on tokens 0..{sample - 1} of the timed inputs "
                       f"({sampled} distinct experts{' + shared' if s else ''}, {dt:.2f} s), scaled by "
                       f"{hit + s}/{sampled + s} experts; torch {torch.__version__} CPU, {threads} threads, "
                       f"{cpu_model()}")}


def _p95(values: list[float]) -> float:
    """The 95th percentile with linear interpolation, as megabench/harness/benchmark.py:41-45."""
    ordered = sorted(values)
    at = (len(ordered) - 1) * 0.95
    lo = int(at)
    return ordered[lo] + (ordered[min(lo + 1, len(ordered) - 1)] - ordered[lo]) * (at - lo)


def measure_like_harness(fn, inputs: dict, warmup: int, reps: int) -> dict:
    """The reference harness's timing method (megabench/harness/benchmark.py:13-52): the same
    inputs every call; a device synchronization before each rep; the host clock and a pair
    of device events around each call, the end event waited on. So the host's cost of issuing
    the call (the Python of run(), the C ABI, the launch) counts in both figures, as it does
    when the harness grades a submission. Microseconds."""
    import torch

    for _ in range(warmup):
        fn(inputs)
    torch.cuda.synchronize()
    host, event = [], []
    for _ in range(reps):
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        t0 = time.perf_counter()
        fn(inputs)
        e1.record()
        e1.synchronize()
        event.append(e0.elapsed_time(e1) * 1e3)
        host.append((time.perf_counter() - t0) * 1e6)
    return {"method": "megabench/harness/benchmark.py:_measure (sync before each rep, same inputs)",
            "reps": reps, "host_p50_us": statistics.median(host), "host_p95_us": _p95(host),
            "event_p50_us": statistics.median(event), "event_p95_us": _p95(event)}


DEVICE_WARMUP_MS = 30.0


def warm_device(layer, sets, ms: float = DEVICE_WARMUP_MS) -> int:
    """The device warm-up: the layer, in the form given (the stream-ordered one), run for at
    least ``ms`` milliseconds before any form's warmup steps. After the device has idled (input
    generation ends ~20 ms before the first call), the layer runs slower until the device has
    carried this load for ~20 ms: on the headline shape the first ~20 single-launch calls took
    876 -> 835 us, so 5 warmup calls left the first timed loop ~13 us per call above the next
    ones (841). Copy kernels for as long do not remove the ramp; 20 calls of either form do.
    Returns the number of calls."""
    import torch

    n, t0 = 0, time.perf_counter()
    while (time.perf_counter() - t0) * 1e3 < ms or n < 2:
        layer(sets[n % len(sets)])
        n += 1
        if n % 4 == 0:
            torch.cuda.synchronize()
    torch.cuda.synchronize()
    return n


def _time_layer(layer, sets, steps: int, warmup: int, outs: list | None = None) -> dict:
    """K calls back to back between two device events (the value; also the host's issue time
    per call of that loop), K calls each between its own pair (p50, p95), and K calls in
    which the library records events at its stage boundaries on the stream its kernels run
    on (per-stage means). ``outs`` receives the outputs of the last timed call on each set."""
    import torch

    dev = torch.device("cuda:0")
    n_sets = len(sets)
    # Warmup runs straight into the timed region: a host round trip between them leaves the
    # device idle for a few ms, which measurably slows the first timed calls.
    for i in range(warmup):
        layer(sets[i % n_sets])
    stream = torch.cuda.current_stream(dev)
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    last = [None] * n_sets
    torch.cuda.synchronize()
    start.record(stream)
    t0 = time.perf_counter()
    for i in range(steps):
        last[i % n_sets] = layer(sets[i % n_sets])
    issue_us = (time.perf_counter() - t0) / steps * 1e6
    end.record(stream)
    torch.cuda.synchronize()
    ms = start.elapsed_time(end) / steps
    for i in range(n_sets):  # sets the timed loop did not reach (steps < sets)
        if last[i] is None:
            last[i] = layer(sets[i])
    if outs is not None:
        outs.extend(last)
    del last
    per_step = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
    for i, (e0, e1) in enumerate(per_step):
        e0.record(stream)
        layer(sets[i % n_sets])
        e1.record(stream)
    torch.cuda.synchronize()
    step_ms = [a.elapsed_time(b) for a, b in per_step]
    nev = len(layer.stages) + 1
    events = [[torch.cuda.Event(enable_timing=True) for _ in range(nev)] for _ in range(steps)]
    for row in events:
        for e in row:
            e.record(stream)  # creates the HIP event
    torch.cuda.synchronize()
    for i in range(steps):
        layer.record(sets[i % n_sets], events[i])
    torch.cuda.synchronize()
    stage = [[row[j].elapsed_time(row[j + 1]) for j in range(nev - 1)] for row in events]
    stage_ms = [statistics.mean(s_[j] for s_ in stage) for j in range(nev - 1)]
    return {"ms": ms, "p50_us": statistics.median(step_ms) * 1e3,
            "p95_us": sorted(step_ms)[min(len(step_ms) - 1, int(0.95 * (len(step_ms) - 1) + 0.5))] * 1e3,
            "stage_us": {name: v * 1e3 for name, v in zip(layer.stages, stage_ms)}, "host_issue_us": issue_us}


def bench_case(case, steps: int, warmup: int, want_cpu: bool, cpu_budget: float) -> dict:
    import torch

    __graft_entry__.load_package()
    from vibe_megakernel_amd import cases as C
    from vibe_megakernel_amd import submission, workloads

    dev = torch.device("cuda:0")
    layer = submission.MoELayer(case)  # the submission's path: one launch for the fp8 forms
    per_set = C.algorithmic_bytes(case, round(C.expected_hit_experts(case)))
    n_sets = max(1, min(8, math.ceil(ROTATE_BYTES / per_set)))
    _log(f"[bench] {case.id}: generating {n_sets} input set(s) on the GPU")
    sets = [workloads.make_inputs(case, 7301 + i, dev, log=lambda m, i=i: _log(f"[bench] {case.id} set {i}: {m}"))
            for i in range(n_sets)]
    torch.cuda.synchronize()
    five = submission.MoELayer(case, single_launch=False) if layer.single_launch else layer
    warm_calls = warm_device(five, sets)
    _log(f"[bench] {case.id}: inputs ready, device warmed ({warm_calls} calls); warmup and timing {steps} steps")
    outs: list = []
    r = _time_layer(layer, sets, steps, warmup, outs)
    if case.format == "mxfp4":
        hit = statistics.mean(len(torch.unique(v["topk_idx"])) for v in sets)
    else:
        hit = statistics.mean(len(torch.unique(o["expert_ids"])) for o in outs[:n_sets])
    got0 = {k: v.cpu() for k, v in outs[0].items()}  # the last timed call on sets[0]
    del outs
    harness = measure_like_harness(layer, sets[0], warmup=2, reps=steps)

    bytes_step = C.algorithmic_bytes(case, 0) + (C.algorithmic_bytes(case, 1) - C.algorithmic_bytes(case, 0)) * hit
    ms = r["ms"]
    result = {
        "case": case.id, "ms_per_step": ms, "us_per_step": ms * 1e3, "p50_us": r["p50_us"], "p95_us": r["p95_us"],
        "hit_experts": hit, "bytes_per_step": bytes_step,
        "tb_per_s": bytes_step / (ms * 1e-3) / 1e12,
        "hbm_frac": bytes_step / (ms * 1e-3) / PEAK_HBM,
        "mfma_frac": C.algorithmic_flops(case) / (ms * 1e-3) / PEAK_FP8,
        "launches_per_step": case.max_gpu_launches,
        "stage_us": r["stage_us"], "host_issue_us": r["host_issue_us"], "harness": harness,
        "device_warmup": f"{warm_calls} stream-ordered calls ({DEVICE_WARMUP_MS:.0f} ms) before the warmup steps",
        "rotation_sets": n_sets,
        "dtype": ("e2m1xe4m3->fp32 (E8M0 scales per 32; bf16 out)" if case.format == "mxfp4"
                  else "e4m3xbf16->fp32 (W8A16; bf16 in/out)" if case.activations == "bf16"
                  else "e4m3xe4m3->fp32 (bf16 in/out)"),
    }
    if layer.single_launch:
        # One kernel per step: its roofline is the whole layer's algorithmic bytes over the
        # mean duration of the launch (events the library records around it, on its stream).
        k_ms = r["stage_us"]["layer"] * 1e-3
        result["roofline"] = {"bound": "hbm", "achieved": bytes_step / (k_ms * 1e-3) / 1e9, "peak": PEAK_HBM / 1e9,
                              "unit": "GB/s", "frac": bytes_step / (k_ms * 1e-3) / PEAK_HBM,
                              "traffic": measured_traffic(case, layer_kernel(case).split("<")[0]),
                              "kernel": layer_kernel(case),
                              "kernel_us": k_ms * 1e3, "bytes_per_launch": bytes_step}
        # The stream-ordered kernels of the same layer, for their per-stage times and the
        # expert kernel's own roofline.
        r5 = _time_layer(five, sets, steps, warmup)
        kb = kernel_bytes(case, hit)
        ex_ms = r5["stage_us"]["experts"] * 1e-3
        ex_bytes = kb["gate_up"] + kb["down"]
        result["stream_ordered"] = {
            "us_per_step": r5["ms"] * 1e3, "p50_us": r5["p50_us"], "stage_us": r5["stage_us"],
            "launches_per_step": len(five.stages),
            "expert_kernel": {"kernel": expert_kernel(case), "kernel_us": ex_ms * 1e3, "bytes_per_launch": ex_bytes,
                              "frac": ex_bytes / (ex_ms * 1e-3) / PEAK_HBM,
                              "traffic": measured_traffic(case, expert_kernel(case).split("<")[0])}}
    else:
        kb = kernel_bytes(case, hit)
        ex_ms = r["stage_us"]["experts"] * 1e-3
        ex_bytes = kb["gate_up"] + kb["down"]
        result["roofline"] = {"bound": "hbm", "achieved": ex_bytes / (ex_ms * 1e-3) / 1e9, "peak": PEAK_HBM / 1e9,
                              "unit": "GB/s", "frac": ex_bytes / (ex_ms * 1e-3) / PEAK_HBM,
                              "traffic": measured_traffic(case, expert_kernel(case).split("<")[0]),
                              "kernel": expert_kernel(case),
                              "kernel_us": ex_ms * 1e3, "bytes_per_launch": ex_bytes}
    if want_cpu:
        _log(f"[bench] {case.id}: CPU oracle baseline and parity of the timed outputs")
        base = cpu_baseline(case, sets[0], round(hit), cpu_budget, got0)
        result["parity"] = base.pop("parity")
        result["parity_ok"] = result["parity"]["ok"]
        result["cpu_baseline"] = base
    del sets
    torch.cuda.empty_cache()
    return result


def cpu_baseline_ep(case, experts_cpu: dict, received: dict, hit: int, budget_s: float,
                    got_rows=None) -> dict:
    """The CPU oracle of the local experts (oracle.ep.experts, BF16 schedule) on the rows of
    the first local experts, doubling until the budget, scaled by the hit local experts.
    With ``got_rows`` (the timed steps' local-expert output rows), the oracle's rows check
    them: the result's "parity" entry."""
    import torch

    from oracle import ep as OE

    threads = cpu_threads()
    torch.set_num_threads(threads)
    ids = received["ids"]
    n = 1
    while True:
        sel = (ids < n).nonzero().flatten()
        t0 = time.perf_counter()
        want = OE.experts(case, {k: v[:n] for k, v in experts_cpu.items()}, received["rows"][sel],
                          received["row_scales"][sel], ids[sel], received["weights"][sel], 0)
        dt = time.perf_counter() - t0
        sampled = len(set(ids[sel].tolist()))
        if dt * 2 > budget_s or n * 2 > case.experts // case.ep:
            break
        n *= 2
    parity = None
    if got_rows is not None:  # untimed: the FP32 oracle of the same rows
        exact = OE.experts(case, {k: v[:n] for k, v in experts_cpu.items()}, received["rows"][sel],
                           received["row_scales"][sel], ids[sel], received["weights"][sel], 0, widen=True)
        parity = parity_of(case, got_rows[sel], {"y": want}, {"y": exact})
        parity["local_experts"] = n
    return {"value": dt * hit / max(sampled, 1) * 1e6, "unit": "us/step", "cores": threads, "kind": "port",
            "cpu_model": cpu_model(), "parity": parity,
            "sample": (f"oracle.ep.experts on the received rows of local experts 0..{n - 1} ({sampled} hit, "
                       f"{sel.numel()} rows, {dt:.2f} s), scaled by {hit}/{sampled} experts; dispatch and combine "
                       f"not included; torch {torch.__version__} CPU, {threads} threads, {cpu_model()}")}


def bench_ep_share(case, steps: int, warmup: int, want_cpu: bool, cpu_budget: float) -> dict:
    """Rank 0's share of an EP case: its dispatch (order + pack), its local experts over the
    rows all ranks send it, and its combine, issued back to back on one stream. The rows it
    receives are built before timing from every rank's dispatch (the exchange is a
    collective, not part of the share); the rows it gets back are synthetic bf16 of the
    returned shape (the combine's cost does not depend on their values)."""
    import dataclasses

    import numpy as np
    import torch

    __graft_entry__.load_package()
    from vibe_megakernel_amd import cases as C
    from vibe_megakernel_amd import ep as EP
    from vibe_megakernel_amd import workloads

    dev = torch.device("cuda:0")
    T, K, H, ep = case.tokens, case.topk, case.hidden, case.ep
    local = case.experts // ep
    _log(f"[bench] {case.id}: generating rank 0's share on the GPU")
    v = workloads.make_ep_inputs(case, 7301, dev, rank=0)
    routing = ("x", "x_scales", "topk_idx", "topk_weights")
    sends = [EP.dispatch(*(v[k][r * T:(r + 1) * T] for k in routing), case.experts, ep) for r in range(ep)]
    counts = [EP.send_counts(s_) for s_ in sends]
    received = {name: torch.cat([getattr(s_, name)[:c[0]] for s_, c in zip(sends, counts)])
                for name in ("rows", "row_scales", "ids", "weights")}
    R = received["rows"].shape[0]
    mine = [v[k][:T] for k in routing]
    del sends
    weights = ("l1_blocks", "l1_scales", "l2_blocks", "l2_scales")
    experts = EP.Experts(*(v[k] for k in weights), 0, case.swiglu_limit)
    ws = torch.empty(experts.workspace_bytes(R), dtype=torch.uint8, device=dev)
    returned = torch.randn((T * K, H), device=dev).to(torch.bfloat16)
    args = (received["rows"], received["row_scales"], received["ids"], received["weights"])
    torch.cuda.synchronize()
    _log(f"[bench] {case.id}: rank 0 sends {counts[0]} rows, receives {R}; warmup")

    # Outputs preallocated once, as a serving loop would hold them: the timed steps launch
    # kernels only.
    send = EP.dispatch(*mine, case.experts, ep)
    out = torch.empty((R, H), dtype=torch.bfloat16, device=dev)
    y = torch.empty((T, H), dtype=torch.bfloat16, device=dev)

    def step(events=None):
        EP.dispatch(*mine, case.experts, ep, send=send)
        if events is not None:
            events[0].record(stream)
        experts(*args, workspace=ws, out=out, events=None if events is None else events[1:5])
        EP.combine(returned, send.slot_rows, y=y)
        if events is not None:
            events[5].record(stream)
        return out, y

    stream = torch.cuda.current_stream(dev)
    for _ in range(warmup):
        step()
    _log(f"[bench] {case.id}: timing {steps} steps")
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record(stream)
    for _ in range(steps):
        step()
    end.record(stream)
    torch.cuda.synchronize()
    ms = start.elapsed_time(end) / steps
    per_step = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
    for e0, e1 in per_step:
        e0.record(stream)
        step()
        e1.record(stream)
    torch.cuda.synchronize()
    step_ms = [a.elapsed_time(b) for a, b in per_step]
    # Stage boundaries: before the dispatch's first kernel is not marked (its launch comes
    # first); events[0] follows the dispatch, the library marks the experts' three stages,
    # events[5] follows the combine.
    names = ("dispatch", "permute", "experts", "row_copy", "combine")
    events = [[torch.cuda.Event(enable_timing=True) for _ in range(7)] for _ in range(steps)]
    for row in events:
        for e in row:
            e.record(stream)
    torch.cuda.synchronize()
    for row in events:
        row[0].record(stream)
        step(row[1:])
    torch.cuda.synchronize()
    stage = [[row[j].elapsed_time(row[j + 1]) for j in range(6)] for row in events]
    stage_ms = [statistics.mean(st[j] for st in stage) for j in range(6)]
    # row[1] is recorded after the dispatch and row[2] by the library before its permute
    stage_ms = [stage_ms[0] + stage_ms[1]] + stage_ms[2:]
    harness = measure_like_harness(lambda _: step(), {}, warmup=2, reps=steps)
    hit = len(torch.unique(received["ids"]))
    bytes_step = C.algorithmic_bytes(case, hit)
    rows_case = dataclasses.replace(case, gpus=1, ep=1, params=dict(case.params, tokens=R, topk=1, experts=local))
    kb = kernel_bytes(rows_case, hit)
    ex_ms = stage_ms[names.index("experts")]
    ex_bytes = kb["gate_up"] + kb["down"]
    result = {
        "case": case.id, "ms_per_step": ms, "us_per_step": ms * 1e3,
        "p50_us": statistics.median(step_ms) * 1e3,
        "p95_us": sorted(step_ms)[min(len(step_ms) - 1, int(0.95 * (len(step_ms) - 1) + 0.5))] * 1e3,
        "hit_experts": hit, "bytes_per_step": bytes_step,
        "tb_per_s": bytes_step / (ms * 1e-3) / 1e12, "hbm_frac": bytes_step / (ms * 1e-3) / PEAK_HBM,
        "mfma_frac": 2 * R * 3 * case.intermediate * H / (ms * 1e-3) / PEAK_FP8,
        "stage_us": {name: x * 1e3 for name, x in zip(names, stage_ms)}, "harness": harness,
        "rotation_sets": 1, "received_rows": R, "sent_rows": T * K,
        "roofline": {"bound": "hbm", "achieved": ex_bytes / (ex_ms * 1e-3) / 1e9, "peak": PEAK_HBM / 1e9,
                     "unit": "GB/s", "frac": ex_bytes / (ex_ms * 1e-3) / PEAK_HBM,
                     "traffic": measured_traffic(case, mx_kernel(R, local)),
                     "kernel": mx_kernel(R, local), "kernel_us": ex_ms * 1e3, "bytes_per_launch": ex_bytes},
        "dtype": "e2m1xe4m3->fp32 (E8M0 scales per 32; bf16 out)",
    }
    if want_cpu:
        _log(f"[bench] {case.id}: CPU oracle baseline and parity of the timed outputs")
        base = cpu_baseline_ep(case, {k: v[k].cpu() for k in weights}, {k: x.cpu() for k, x in received.items()},
                               hit, cpu_budget, out.cpu())
        result["parity"] = base.pop("parity")
        result["parity_ok"] = result["parity"]["ok"]
        result["cpu_baseline"] = base
    del v, received
    torch.cuda.empty_cache()
    return result


def _config_entry(r: dict) -> dict:
    """One config's record under "configs": time, bandwidth, roofline and CPU baseline."""
    keep = ("us_per_step", "p50_us", "p95_us", "tb_per_s", "hbm_frac", "mfma_frac", "hit_experts", "bytes_per_step",
            "launches_per_step", "stage_us", "rotation_sets", "roofline", "stream_ordered", "cpu_baseline", "dtype",
            "received_rows", "sent_rows", "host_issue_us", "harness", "parity", "parity_ok", "device_warmup")
    return {k: r[k] for k in keep if k in r}


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--case", default=None, help="measure this case only (its line alone)")
    ap.add_argument("--all", action="store_true",
                    help="also measure the other forms (block, MXFP4, EP share, epilogue variants, the headline "
                         "shape with UE8M0 scales and without the router bias)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-budget", type=float, default=10.0, help="seconds of CPU oracle work per config")
    ap.add_argument("--copy-probe-mib", type=int, default=0,
                    help="run a plain copy of this many MiB first (counter calibration)")
    ap.add_argument("--child", action="store_true", help=argparse.SUPPRESS)
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported by this build "
              "(the layer's multi-GPU sharding is a design note, not built).", file=sys.stderr)
        return 2

    import torch

    __graft_entry__.load_package()
    from vibe_megakernel_amd import cases as C

    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        return 2
    if args.copy_probe_mib > 0:
        copy_probe(args.copy_probe_mib)
    head = C.case(args.case or C.HEADLINE)
    if args.case:
        others = []
    else:
        # The five BASELINE.json configs always; the other forms with --all.
        others = [c for c in C.CASES if c.id != head.id]
        if args.all:
            others += C.BLOCK_CASES + C.MX_CASES + C.EP_CASES + C.VARIANT_CASES + C.HEADLINE_VARIANTS
    run = bench_ep_share if head.ep > 1 else bench_case
    r = run(head, args.steps, args.warmup, not args.no_cpu_baseline, args.cpu_budget)
    # Each other config runs in a child process of its own, on a fresh device heap: after a
    # config's inputs (up to 17 GB) are allocated and freed in this process, the next
    # config's weights land in fragmented memory and its expert kernel measures a few
    # percent slower.
    results = {head.id: r}
    for c in others:
        cmd = [sys.executable, __file__, "--case", c.id, "--steps", str(args.steps), "--warmup", str(args.warmup),
               "--cpu-budget", str(args.cpu_budget), "--child"]
        if args.no_cpu_baseline:
            cmd.append("--no-cpu-baseline")
        child = subprocess.run(cmd, stdout=subprocess.PIPE, text=True)
        if child.returncode != 0:
            print(f"bench.py: the {c.id} run failed (exit {child.returncode})", file=sys.stderr)
            return child.returncode
        results[c.id] = json.loads(child.stdout.strip().splitlines()[-1])["result"]
        _log(f"[bench] {c.id}: {results[c.id]['us_per_step']:.1f} us/step, "
             f"{100 * results[c.id]['hbm_frac']:.1f}% of HBM peak")
    if args.child:
        print(json.dumps({"result": r}), flush=True)
        return 0
    line = {
        "metric": (METRIC if head.id == C.HEADLINE else
                   f"MoE decode layer \u00b5s/step + achieved HBM TB/s (% of peak), {head.id}, 1 GPU"),
        "value": r["us_per_step"], "unit": "us/step", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": r["ms_per_step"], "higher_is_better": False, "scaling": "weak", "vs_baseline": None,
        "dtype": r["dtype"], "data": "synthetic (seeded, generated on the GPU)",
        "config": {"workload": head.id, "tokens": head.tokens, "hidden": head.hidden, "experts": head.experts,
                   "shared_experts": head.shared_experts, "topk": head.topk, "intermediate": head.intermediate,
                   "router": head.router, "groups": head.groups, "top_groups": head.top_groups,
                   "parallelism": (f"rank 0 of ep{head.ep} (its dispatch, local experts and combine; the "
                                   "exchanges are not run)" if head.ep > 1 else "single GPU")},
        "achieved_tb_per_s": r["tb_per_s"], "hbm_frac": r["hbm_frac"], "p50_us": r["p50_us"], "p95_us": r["p95_us"],
        "hit_experts": r["hit_experts"], "bytes_per_step": r["bytes_per_step"], "stage_us": r["stage_us"],
        "mfma_frac": r["mfma_frac"],
        "roofline": r["roofline"],
        "cpu_baseline": r.get("cpu_baseline"),
        "harness": r.get("harness"), "host_issue_us": r.get("host_issue_us"),
        "parity_ok": r.get("parity_ok"), "parity": r.get("parity"),
        "configs": {cid: _config_entry(v) for cid, v in results.items()},
    }
    print(json.dumps(line), flush=True)
    # A config whose timed outputs fail the oracle check fails the run (after the line).
    failed = [cid for cid, v in results.items() if v.get("parity_ok") is False]
    if failed:
        print(f"bench.py: timed outputs differ from the oracle on {failed}", file=sys.stderr)
        return 1
    return 0


if __name__ == "__main__":
    sys.exit(main())
