"""Grading rules (test infrastructure).

``band`` restates megabench/harness/correctness.py:64-85: the candidate's
error against the FP32 oracle may reach ``noise_factor`` times the BF16
reference's own error (relative L2, and max-abs plus ``bf16_rtol`` of the
oracle's peak). ``integers_match`` restates the integer rule of
correctness.py:503-521: each element equals the BF16 reference or the oracle.
``layer_checks`` are the layer's stated bars: max|y - y_ref| / max|y_ref| <=
1e-2 and cosine >= 0.9999.
"""

from __future__ import annotations

import torch

MAX_REL = 1e-2
MIN_COSINE = 0.9999


def band(want: torch.Tensor, got: torch.Tensor, exact: torch.Tensor, *, bf16_rtol: float = 0.008,
         rtol: float = 0.0, atol: float = 0.0, noise_factor: float = 2.0) -> dict:
    exact = exact.double().cpu()
    err = got.double().cpu() - exact
    ref_err = want.double().cpu() - exact
    scale = exact.norm().clamp_min(torch.finfo(torch.float64).tiny)
    tol = bf16_rtol if want.dtype == torch.bfloat16 else rtol
    out = {"relative_error": float(err.norm() / scale),
           "reference_relative_error": float(ref_err.norm() / scale),
           "max_abs_error": float(err.abs().max()) if err.numel() else 0.0,
           "reference_max_abs_error": float(ref_err.abs().max()) if err.numel() else 0.0}
    peak = float(exact.abs().max()) if exact.numel() else 0.0
    out["pass"] = bool(out["relative_error"] <= noise_factor * out["reference_relative_error"] + tol and
                       out["max_abs_error"] <= noise_factor * out["reference_max_abs_error"] + atol + tol * peak)
    return out


def integers_match(got: torch.Tensor, want: torch.Tensor, exact: torch.Tensor) -> dict:
    got, want, exact = got.cpu(), want.cpu(), exact.cpu().to(want.dtype)
    neither = (got != want) & (got != exact)
    return {"mismatched_elements": int((got != want).sum()), "unmatched_elements": int(neither.sum()),
            "pass": not bool(neither.any())}


def layer_checks(got: torch.Tensor, ref: torch.Tensor) -> dict:
    g, r = got.double().cpu().flatten(), ref.double().cpu().flatten()
    peak = float(r.abs().max()) if r.numel() else 0.0
    max_rel = float((g - r).abs().max()) / peak if peak > 0 else float((g - r).abs().max() if g.numel() else 0.0)
    denom = float(g.norm() * r.norm())
    cosine = float(g @ r) / denom if denom > 0 else (1.0 if float(g.norm()) == float(r.norm()) == 0 else 0.0)
    return {"max_rel": max_rel, "cosine": cosine, "pass": max_rel <= MAX_REL and cosine >= MIN_COSINE}
