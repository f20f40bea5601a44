"""GPU parity of the block form (RMSNorm -> layer -> residual add, frontier.py:335-354)
against the CPU oracle, through the C ABI.

Bars: megamoe_rms_norm bit-exact against oracle.layer.rms_norm; in the block, expert ids
bit-exact (routing of the normalized rows), weights as in the layer tests, and y within the
band rule against the widened block oracle and max-rel 1e-2 / cosine 0.9999 against the
BF16 block reference.
"""

from __future__ import annotations

import sys

import pytest
import torch

from oracle import layer, metrics, routing
from vibe_megakernel_amd import cases as C
from vibe_megakernel_amd import submission, workloads

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
LOGIT_RTOL = 1e-4
W_RTOL = 2e-6


def _log(msg):
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.mark.parametrize("fp32_gamma", [True, False])
@pytest.mark.parametrize("shape", [(64, 7168), (37, 2048), (4, 1024), (3, 264), (4096, 1024), (5, 17000)])
def test_rms_norm_bit_exact(shape, fp32_gamma):
    _log(f"rms_norm {shape} fp32_gamma={fp32_gamma}")
    T, H = shape
    g = torch.Generator().manual_seed(T * 31 + H)
    # Row magnitudes over six decades: every row has its own 1/sqrt, and an ulp off in it
    # shows in the rows' bf16 outputs now and then (4096 rows make that likely).
    x = torch.randn((T, H), generator=g) * torch.logspace(-4, 2, T)[:, None]
    x[0] = 0.0
    x = x.to(torch.bfloat16)
    w = (torch.randn((H,), generator=g) * 0.1 + 1.0).to(torch.bfloat16)
    for eps in (1e-6, 1e-5):
        got = submission.rms_norm(x.to(DEV), w.to(DEV), eps, fp32_gamma).cpu()
        want = layer.rms_norm(x, w, eps, fp32_gamma)
        assert torch.equal(got.view(torch.int16), want.view(torch.int16)), f"eps={eps}"


def _to(values, device):
    return {k: v.to(device) for k, v in values.items()}


def _compare(case, got, want, exact, rows=None):
    ids, w, y = got["expert_ids"].cpu(), got["expert_weights"].cpu(), got["y"].cpu()
    if rows is not None:
        ids, w, y = ids[rows], w[rows], y[rows]
    assert torch.equal(ids, want["expert_ids"]), f"{case.id}: expert ids differ"
    torch.testing.assert_close(w, want["expert_weights"], rtol=LOGIT_RTOL, atol=0)
    check = metrics.layer_checks(y, want["y"])
    assert check["pass"], f"{case.id}: {check}"
    band = metrics.band(want["y"], y, exact["y"], bf16_rtol=case.bf16_rtol, noise_factor=case.noise_factor)
    assert band["pass"], f"{case.id}: band {band}"
    return check, band


def _dev_block_cases():
    out = [C.development(c) for c in C.BLOCK_CASES]
    out.append(C.development(C.BLOCK_CASES[0], tokens=37))
    out.append(C.development(C.BLOCK_CASES[0], tokens=13))  # the dense schedule (T <= 16, T*K >= E)
    return out


@pytest.mark.parametrize("case", _dev_block_cases(), ids=lambda c: c.id)
def test_block_matches_oracle_on_development_geometry(case):
    _log(f"block parity {case.id} T={case.tokens} H={case.hidden} norm={case.norm}")
    for seed in (104729, 104730):
        values = workloads.make_inputs(case, seed, "cpu")
        want, exact = layer.block_reference(case, values), layer.block_oracle(case, values)
        got = submission.build(case.to_dict())(_to(values, DEV))
        torch.cuda.synchronize()
        _compare(case, got, want, exact)


def test_block_does_not_mutate_inputs_and_is_deterministic():
    case = C.development(C.BLOCK_CASES[0], tokens=20)
    _log(f"block determinism {case.id}")
    values = _to(workloads.make_inputs(case, 9, "cpu"), DEV)
    before = {k: v.clone() for k, v in values.items()}
    run = submission.build(case.to_dict())
    a, b = run(values), run(values)
    torch.cuda.synchronize()
    for k in a:
        assert torch.equal(a[k], b[k]), k
    for k, v in values.items():
        u = (lambda t: t.view(torch.uint8) if t.dtype == torch.float8_e4m3fn else t)
        assert torch.equal(u(v), u(before[k])), k


@pytest.mark.parametrize("cid", [c.id for c in C.BLOCK_CASES])
def test_full_size_block_on_every_token(cid):
    """Full geometry, inputs generated on the GPU: ids of every token (routing of the
    normalized rows, fp32 GEMV as frontier.py:343, and the correctly rounded logits), y of
    every token against the block oracle."""
    case = C.case(cid)
    _log(f"full size block {cid}")
    values = workloads.make_inputs(case, 104729, DEV)
    got = submission.build(case.to_dict())(values)
    torch.cuda.synchronize()
    cpu = {k: v.cpu() for k, v in values.items()}
    del values
    torch.cuda.empty_cache()
    xn = layer.rms_norm(cpu["x"], cpu["ln2"], case.norm_eps, case.norm == "fp32_weight").float()
    exact_logits = (cpu["router"].double() @ xn.double().T).T.float()
    for t in range(case.tokens):
        wi, ww = routing.route(case, cpu["router"] @ xn[t], cpu.get("router_bias"))
        assert torch.equal(got["expert_ids"][t].cpu(), wi), f"token {t}"
        torch.testing.assert_close(got["expert_weights"][t].cpu(), ww, rtol=LOGIT_RTOL, atol=0)
        ei, ew = routing.route(case, exact_logits[t], cpu.get("router_bias"))
        assert torch.equal(ei, wi), f"token {t}: a top-k margin below the logits' rounding error"
        torch.testing.assert_close(got["expert_weights"][t].cpu(), ew, rtol=W_RTOL, atol=0)
    want, exact = layer.block_reference(case, cpu), layer.block_oracle(case, cpu)
    check, band = _compare(case, got, want, exact)
    _log(f"  {cid}: {check} band_rel={band['relative_error']:.3e}")
