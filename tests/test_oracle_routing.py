"""Pins of the oracle's routing rules (CPU only).

  * the reference's known answer (megabench/tests/test_frontier.py:297-299, data in
    tests/golden/known_answers.json);
  * brute force: on small E every subset of groups and every subset of experts is
    enumerated, and exactly one of each must dominate its complement under the order
    (value descending, index ascending); inputs sit on a coarse grid so ties are common;
  * the plain-C selector (oracle/codec.c, insertion-sort ranking) on tie-heavy inputs;
  * transformers' routers as independent library routines: DeepseekV3TopkRouter for the
    sigmoid rule (pattern of megabench/tests/test_frontier.py:283-296, compared as sets,
    since it selects with topk(sorted=False)), Qwen3MoeTopKRouter and MixtralTopKRouter
    for softmax top-k with renormalisation.
"""

from __future__ import annotations

import itertools
import json
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import build as oracle_c
from oracle import routing

GOLDEN = json.loads((Path(__file__).parent / "golden" / "known_answers.json").read_text())


def _ranks_before(values, a, b):
    """a before b in (value descending, index ascending)."""
    return values[a] > values[b] or (values[a] == values[b] and a < b)


def _dominant_subset(values, candidates, size):
    """The unique subset of ``candidates`` of ``size`` whose every member ranks before every
    non-member, found by enumeration."""
    found = []
    for subset in itertools.combinations(candidates, size):
        rest = [c for c in candidates if c not in subset]
        if all(_ranks_before(values, a, b) for a in subset for b in rest):
            found.append(set(subset))
    assert len(found) == 1
    return found[0]


def _brute_sigmoid(scores, bias, topk, groups, top_groups, scaling):
    p = [1.0 / (1.0 + np.exp(-np.float64(s))) for s in scores.tolist()]
    prob = scores.float().sigmoid()
    choice = (prob + (bias if bias is not None else 0.0)).tolist()
    E = len(choice)
    n = E // groups
    eligible = list(range(E))
    if groups > 1:
        gscore = []
        for g in range(groups):
            members = sorted(range(g * n, (g + 1) * n), key=lambda e: (-choice[e], e))
            gscore.append(np.float32(np.float32(choice[members[0]]) + np.float32(choice[members[1]])))
        kept = _dominant_subset(gscore, list(range(groups)), top_groups)
        eligible = [e for e in range(E) if e // n in kept]
    chosen = _dominant_subset(choice, eligible, topk)
    ids = sorted(chosen, key=lambda e: (-choice[e], e))
    w = np.array([prob[e].item() for e in ids], dtype=np.float64)
    w = w / (w.sum() + 1e-20) * scaling
    assert all(abs(prob[e].item() - p[e]) < 1e-6 for e in ids)
    return ids, w


def test_reference_known_answer():
    ka = GOLDEN["route_zeros"]
    ids, w = routing.route_sigmoid(torch.tensor(ka["scores"]), torch.tensor(ka["bias"]), ka["topk"], ka["groups"],
                                   ka["top_groups"], ka["routed_scaling"])
    assert ids.tolist() == ka["expert_ids"]
    assert torch.equal(w, torch.tensor(ka["expert_weights"]))


@pytest.mark.parametrize("E,K,G,TG", [(8, 2, 2, 1), (8, 3, 4, 2), (12, 4, 4, 3), (8, 4, 1, 1), (9, 3, 3, 2)])
def test_sigmoid_group_routing_against_brute_force(E, K, G, TG):
    g = torch.Generator().manual_seed(E * 100 + K * 10 + G)
    for trial in range(60):
        scores = (torch.randn(E, generator=g) * 2).round() / 2  # coarse grid: ties in scores and groups
        bias = None if trial % 3 == 0 else (torch.randint(-2, 3, (E,), generator=g).float() / 8)
        ids, w = routing.route_sigmoid(scores, bias, K, G, TG, 2.5)
        want_ids, want_w = _brute_sigmoid(scores, bias, K, G, TG, 2.5)
        assert ids.tolist() == want_ids, (trial, scores, bias)
        np.testing.assert_allclose(w.double().numpy(), want_w, rtol=1e-6)


@pytest.mark.parametrize("E,K", [(8, 2), (16, 5), (7, 7)])
def test_softmax_routing_against_brute_force(E, K):
    g = torch.Generator().manual_seed(E + K)
    for _ in range(60):
        logits = (torch.randn(E, generator=g) * 2).round() / 2
        ids, w = routing.route_softmax(logits, K, renormalize=True)
        vals = logits.tolist()
        chosen = _dominant_subset(vals, list(range(E)), K)
        want = sorted(chosen, key=lambda e: (-vals[e], e))
        assert ids.tolist() == want
        ex = np.exp(np.array([vals[e] for e in want], dtype=np.float64) - max(vals))
        np.testing.assert_allclose(w.double().numpy(), ex / ex.sum(), rtol=1e-6)
        # Without renormalisation the weights are the full softmax at the chosen ids.
        _, w_full = routing.route_softmax(logits, K, renormalize=False)
        full = np.exp(np.array(vals, dtype=np.float64) - max(vals))
        np.testing.assert_allclose(w_full.double().numpy(), full[want] / full.sum(), rtol=1e-6)


@pytest.mark.parametrize("E,K,G,TG", [(256, 8, 8, 4), (384, 8, 1, 1), (64, 6, 8, 3), (128, 8, 1, 1)])
def test_c_selector_matches_oracle_on_tie_heavy_inputs(E, K, G, TG):
    g = torch.Generator().manual_seed(E + 7 * K)
    for trial in range(40):
        choice = (torch.randn(E, generator=g) * 3).round() / 4
        if trial % 4 == 0:
            choice[:] = 0.5  # everything tied
        # The oracle's sigmoid route on scores whose sigmoid + bias equals ``choice`` is not
        # constructible exactly, so compare the selection step itself: route with zero bias
        # on logits, against the C selector fed the same p = sigmoid(logits).
        p = choice.sigmoid()
        ids, _ = routing.route_sigmoid(choice, None, K, G, TG)
        got = oracle_c.select(p.numpy(), K, G, TG)
        assert got.tolist() == ids.tolist(), trial


def test_transformers_deepseek_v3_router_agrees_off_ties():
    from transformers.models.deepseek_v3.configuration_deepseek_v3 import DeepseekV3Config
    from transformers.models.deepseek_v3.modeling_deepseek_v3 import DeepseekV3TopkRouter

    torch.manual_seed(0)
    for E, K, G, TG in ((256, 8, 8, 4), (64, 6, 8, 3), (32, 4, 4, 2)):
        config = DeepseekV3Config(hidden_size=128, n_routed_experts=E, num_experts_per_tok=K, n_group=G,
                                  topk_group=TG, routed_scaling_factor=2.5, norm_topk_prob=True)
        router = DeepseekV3TopkRouter(config).float()
        assert router.num_experts == E
        with torch.no_grad():
            router.weight.normal_()
            router.e_score_correction_bias.copy_(torch.randn(E) * 0.1)
            value = torch.randn(16, 128)
            logits, weights, ids = router(value)
            for t in range(value.shape[0]):
                got_ids, got_w = routing.route_sigmoid(logits[t], router.e_score_correction_bias, K, G, TG, 2.5)
                order, got_order = ids[t].argsort(), got_ids.argsort()
                assert torch.equal(ids[t][order], got_ids[got_order])
                torch.testing.assert_close(weights[t][order], got_w[got_order])


@pytest.mark.parametrize("family", ["qwen3_moe", "mixtral"])
def test_transformers_softmax_routers_agree(family):
    if family == "qwen3_moe":
        from transformers.models.qwen3_moe.configuration_qwen3_moe import Qwen3MoeConfig as Config
        from transformers.models.qwen3_moe.modeling_qwen3_moe import Qwen3MoeTopKRouter as Router
        config = Config(hidden_size=128, num_experts=128, num_experts_per_tok=8, norm_topk_prob=True)
        E, K = 128, 8
    else:
        from transformers.models.mixtral.configuration_mixtral import MixtralConfig as Config
        from transformers.models.mixtral.modeling_mixtral import MixtralTopKRouter as Router
        config = Config(hidden_size=128, num_local_experts=8, num_experts_per_tok=2)
        E, K = 8, 2
    torch.manual_seed(1)
    router = Router(config).float()
    with torch.no_grad():
        router.weight.normal_()
        value = torch.randn(16, 128)
        logits, weights, ids = router(value)
        for t in range(value.shape[0]):
            got_ids, got_w = routing.route_softmax(logits[t], K, renormalize=True)
            order, got_order = ids[t].argsort(), got_ids.argsort()
            assert torch.equal(ids[t][order], got_ids[got_order])
            torch.testing.assert_close(weights[t][order].float(), got_w[got_order], rtol=2e-6, atol=0)
    assert router.weight.shape == (E, 128)


def test_routing_invariants():
    g = torch.Generator().manual_seed(3)
    for _ in range(50):
        s = torch.randn(64, generator=g)
        ids, w = routing.route_sigmoid(s, torch.randn(64, generator=g) * 0.1, 8, 8, 4, 2.5)
        assert len(set(ids.tolist())) == 8 and ids.dtype == torch.int64
        assert len({int(i) // 8 for i in ids}) <= 4  # at most top_groups groups
        torch.testing.assert_close(w.sum(), torch.tensor(2.5), rtol=1e-6, atol=0)
        ids, w = routing.route_softmax(s, 8, renormalize=True)
        assert bool((w[:-1] >= w[1:]).all())
        torch.testing.assert_close(w.sum(), torch.tensor(1.0), rtol=1e-6, atol=0)


class _Rule:
    """The routing fields of a case, for selection_margins."""

    def __init__(self, router, topk, groups=1, top_groups=1):
        self.router, self.topk, self.groups, self.top_groups = router, topk, groups, top_groups


def test_selection_margins_closed_forms():
    # softmax: top K+1 = 3, 2, 1; gaps 1 and 1, relative 1/3 and 1/2.
    m = routing.selection_margins(_Rule("softmax", 2), torch.tensor([3.0, 1.0, 2.0, 0.0]), None)
    assert m["expert"] == 1.0 and m["group"] == float("inf") and m["relative"] == pytest.approx(1 / 3)
    # an exact tie inside the top K + 1 has margin 0
    m = routing.selection_margins(_Rule("softmax", 2), torch.tensor([0.5, 2.0, 0.5, -1.0]), None)
    assert m["expert"] == 0.0 and m["relative"] == 0.0
    # a tie below the (K+1)-th candidate does not matter
    m = routing.selection_margins(_Rule("softmax", 1), torch.tensor([4.0, 2.0, 1.0, 1.0]), None)
    assert m["expert"] == 2.0
    # sigmoid, 2 groups of 2, keep 1: group scores p0+p1 vs p2+p3
    s = torch.tensor([0.0, 0.0, 1.0, -1.0])
    p = torch.sigmoid(s.double())
    m = routing.selection_margins(_Rule("sigmoid", 1, 2, 1), s, None)
    assert m["group"] == pytest.approx(float(p[0] + p[1] - p[2] - p[3]))
    assert m["expert"] == 0.0  # the kept group holds a tie (experts 0 and 1)


@pytest.mark.parametrize("rule", [_Rule("softmax", 8), _Rule("sigmoid", 8, 8, 4), _Rule("sigmoid", 8)])
def test_selection_margins_bound_the_perturbations_that_keep_the_ids(rule):
    # Any change of the scores smaller than a quarter of the smallest absolute gap keeps the
    # ids and their order (sigmoid moves a choice by at most a quarter of the score change,
    # a group score by at most half); moving the (K+1)-th candidate past the K-th changes them.
    g = torch.Generator().manual_seed(17)
    E = 64
    for _ in range(20):
        s = torch.randn(E, generator=g)
        bias = torch.randn(E, generator=g) * 0.1 if rule.router == "sigmoid" else None
        m = routing.selection_margins(rule, s, bias)
        gap = min(m["expert"], m["group"])
        case = type("C", (), {"router": rule.router, "topk": rule.topk, "groups": rule.groups,
                              "top_groups": rule.top_groups, "routed_scaling": 1.0, "renormalize": True})
        ids, _ = routing.route(case, s, bias)
        for _ in range(5):
            noise = (torch.rand(E, generator=g, dtype=torch.float64) * 2 - 1) * gap / 4 * 0.999
            ids2, _ = routing.route(case, (s.double() + noise).float(), bias)
            if gap > 1e-5:  # well above fp32 rounding of the perturbed scores
                assert torch.equal(ids2, ids)
    if rule.router == "softmax":
        s = torch.arange(E, dtype=torch.float32)
        ids, _ = routing.route(case, s, None)
        t = s.clone()
        t[E - rule.topk - 1] += 1.5  # the (K+1)-th passes the K-th: gap 1
        assert routing.selection_margins(rule, s, None)["expert"] == 1.0
        assert not torch.equal(routing.route(case, t, None)[0], ids)
