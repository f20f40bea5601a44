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
