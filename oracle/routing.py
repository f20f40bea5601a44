"""Routing rules of the MoE layer, restated (test infrastructure).

sigmoid (megabench/tasks/frontier.py:229-242), per token:
    p = sigmoid(scores); c = p + bias
    if groups > 1: group score = sum of the two largest c in the group; keep the
        top ``selected_groups`` groups by a stable descending argsort; set c of
        the other groups to -inf
    ids = first topk of a stable descending argsort of c
    w = p[ids] / (sum(p[ids]) + 1e-20) * scaling
softmax (megabench/tasks/distributed.py:174-176; megabench/tasks/references/moe.py:68-70):
    ids = first topk of a stable descending argsort of the logits
    w = softmax(logits[ids]) (renormalize) or softmax(logits)[ids], times scaling

Ties rank the lower expert index first, the order a stable descending sort
gives (megabench/tasks/gptoss.py:106-109 makes it part of the contract).

Pinned by tests/test_oracle_routing.py: the reference's known answer
(megabench/tests/test_frontier.py:297-299), brute force over every group
subset and every expert order on small E, the plain-C selector in
oracle/codec.c, and transformers' DeepseekV3TopkRouter, Qwen3MoE and Mixtral
routers (megabench/tests/test_frontier.py:283-296 pattern).
"""

from __future__ import annotations

import math

import torch


def route_sigmoid(scores: torch.Tensor, bias: torch.Tensor | None, topk: int, groups: int, selected_groups: int,
                  scaling: float = 2.5, renormalize: bool = True):
    prob = scores.float().sigmoid()
    choice = prob if bias is None else prob + bias
    if groups > 1:
        per_group = choice.view(groups, -1)
        top2 = per_group.sort(dim=-1, descending=True, stable=True).values[:, :2]
        keep = top2.sum(-1).argsort(descending=True, stable=True)[:selected_groups]
        mask = torch.ones(groups, dtype=torch.bool, device=scores.device)
        mask[keep] = False
        choice = per_group.masked_fill(mask[:, None], -torch.inf).flatten()
    ids = choice.argsort(descending=True, stable=True)[:topk]
    w = prob[ids]
    if renormalize:
        w = w / (w.sum() + 1e-20)
    return ids, w * scaling


def route_softmax(scores: torch.Tensor, topk: int, renormalize: bool = True, scaling: float = 1.0):
    logits = scores.float()
    ids = logits.argsort(descending=True, stable=True)[:topk]
    w = logits[ids].softmax(-1) if renormalize else logits.softmax(-1)[ids]
    return ids, w * scaling


def route(case, scores: torch.Tensor, bias: torch.Tensor | None):
    """Route one token's logits with the case's rule; returns (ids int64 [K], weights fp32 [K])."""
    if case.router == "sigmoid":
        return route_sigmoid(scores, bias, case.topk, case.groups, case.top_groups, case.routed_scaling,
                             case.renormalize)
    return route_softmax(scores, case.topk, case.renormalize, case.routed_scaling)


def selection_margins(case, scores: torch.Tensor, bias: torch.Tensor | None) -> dict:
    """How far one token's selection is from a tie, on fp64 arithmetic of its fp32 scores.

    The ids (in selection order) are fixed by the order of the top K + 1 candidates, and for
    group-limited routing also by which TG groups are kept. ``expert`` is the smallest gap
    between consecutive candidates among the top K + 1 choice values of the kept groups;
    ``group`` the gap between the TG-th and the (TG+1)-th group score (inf without group
    limiting); ``relative`` the smaller of the two, each divided by the larger magnitude of
    its pair. A gap of 0 is a tie, decided by the lower index (the stable order). A token
    whose relative margin is below the logits' rounding error (~1e-6 for an fp32 GEMV of
    H ~ 7e3) may route differently under fp32 and exact logits; the reference's integer rule
    (correctness.py:503-521) accepts either there."""
    s = scores.double()
    if case.router == "sigmoid":
        prob = torch.sigmoid(s)
        choice = prob if bias is None else prob + bias.double()
    else:
        choice = s
    group_gap, group_rel = math.inf, math.inf
    if case.router == "sigmoid" and case.groups > 1:
        per_group = choice.view(case.groups, -1)
        top2 = per_group.sort(dim=-1, descending=True, stable=True).values[:, :2]
        gscore = top2.sum(-1) if per_group.shape[1] >= 2 else top2[:, 0]
        gs = gscore.sort(descending=True, stable=True)
        if case.top_groups < case.groups:
            a, b = float(gs.values[case.top_groups - 1]), float(gs.values[case.top_groups])
            group_gap = a - b
            group_rel = group_gap / max(abs(a), abs(b), 1e-300)
        mask = torch.ones(case.groups, dtype=torch.bool)
        mask[gs.indices[:case.top_groups]] = False
        choice = per_group.masked_fill(mask[:, None], -math.inf).flatten()
    top = choice.sort(descending=True, stable=True).values[:case.topk + 1]
    finite = top[torch.isfinite(top)]
    expert_gap, expert_rel = math.inf, math.inf
    for i in range(len(finite) - 1):
        a, b = float(finite[i]), float(finite[i + 1])
        gap = a - b
        rel = gap / max(abs(a), abs(b), 1e-300)
        if rel < expert_rel:
            expert_gap, expert_rel = gap, rel
    return {"expert": expert_gap, "group": group_gap, "relative": min(expert_rel, group_rel)}
