"""Case family of the FP8 MoE decode layer.

The case record keeps the shape of the reference's ``Case`` contract
(megabench/cases.py:19-113: id, family, model, phase, params, tolerances,
execution geometry, launch budget, band gate) so a ``build(case.to_dict())``
call looks exactly like the reference harness's (megabench/harness/runner.py:
80-87). The reference catalog has no FP8 MoE-layer cases; the five configs
below are the ones this layer is measured on, with routing parameters taken
from each model's published configuration:

* Mixtral / Qwen3-30B-A3B: softmax over the top-k logits (== softmax over all
  experts, then renormalised), megabench/tasks/references/moe.py:68-70,
  megabench/tasks/model_specs.json:24 (``norm_topk_prob``).
* DeepSeek-V3: sigmoid + correction bias, 8 groups / top-4 groups / top-8,
  routed scaling 2.5 (megabench/tasks/model_specs.json:171,204-207).
* Kimi-K2: sigmoid + correction bias, one group (group limit trivially met,
  as in the reference's Kimi use of ``frontier.route(..., 1, 1, ...)``,
  megabench/tasks/kimi_layer.py:200), routed scaling 2.827; the bias is a
  Zipf(s=1.1) profile over a seeded expert permutation, so a few experts are
  hot.
"""

from __future__ import annotations

import math
from dataclasses import asdict, dataclass, field, replace

FAMILY = "moe_fp8_layer"
# The reference harness's launch budget per call for every case of its catalog that does not
# set one (megabench/cases.py:32), audited by megabench/harness/benchmark.py:73-100.
REFERENCE_LAUNCH_BUDGET = 1
ROUTERS = ("softmax", "sigmoid", "given")  # given: topk_idx / topk_weights are inputs
# Expert formats: fp8 = E4M3 weights with fp32 128x128 scales and E4M3 activations with
# fp32 per-128 scales (frontier.py); mxfp4 = E2M1 weights with E8M0 scales per 32 and
# E4M3 activations with E8M0 scales per 32 (megamoe.py, quantization.py:13-116).
FORMATS = ("fp8", "mxfp4")
SWIGLUS = ("fp32", "bf16")
# RMSNorm before the layer (the block form): none, gamma applied in fp32 before the one
# bf16 rounding (DeepSeek), or to the rounded activation (common.py:13-21).
NORMS = ("none", "fp32_weight", "bf16_weight")
BIASES = ("none", "normal", "zipf")
GATES = ("band",)


@dataclass(frozen=True)
class Case:
    """One MoE decode-layer problem (fields as megabench/cases.py:19-56, plus routing)."""

    id: str
    family: str
    model: str
    phase: str
    params: dict
    category: str = "layer"
    suite: str = "p1"
    backend: str = "hip"
    gpus: int = 1
    tp: int = 1
    ep: int = 1
    # The fp8 layer (and its block and epilogue forms) runs as one kernel launch
    # (megamoe_layer_forward), the reference's default budget (REFERENCE_LAUNCH_BUDGET).
    max_gpu_launches: int = 1
    atol: float = 0.0
    rtol: float = 0.0
    bf16_rtol: float = 0.008
    noise_factor: float = 2.0
    ready: bool = True
    note: str = ""
    gate: str = "band"
    # Routing rule (not part of the reference Case; the reference fixes it per task module).
    router: str = "softmax"
    renormalize: bool = True
    routed_scaling: float = 1.0
    bias: str = "none"
    bias_std: float = 0.1
    zipf_s: float = 1.1
    zipf_c: float = 1.0
    power_of_two: bool = False
    weight_std: float = 0.02
    router_std: float = 0.02
    # The block form (frontier.py:335,354): RMSNorm of x with a bf16 gamma ~ 1 + N(0, 0.1)
    # (frontier.py:87) before the layer, and the residual add after it.
    norm: str = "none"
    norm_eps: float = 1e-6
    residual: bool = False
    # The MXFP4 form (megamoe.py numerics): expert format, and the SwiGLU clamp applied
    # to gate (above) and up (both sides) before the activation (megamoe.py:116-122).
    format: str = "fp8"
    swiglu_limit: float = 0.0
    # The SwiGLU form of the fp8 experts: "fp32" h = bf16(silu(g) * u) rounded once
    # (frontier.py:337, DeepSeek), "bf16" h = bf16(bf16(silu(g)) * u) (frontier.py:338,
    # glm53.py:174-175); swiglu_limit > 0 clamps g and u first in either form.
    swiglu: str = "fp32"
    # Activations of the fp8 expert GEMMs: "fp8" quantizes x and h to E4M3 per 128 (W8A8,
    # frontier.py:185-186); "bf16" feeds them in bf16 (W8A16, frontier.py:182-183 with
    # quantize=False: the DeepSeek family's expert GEMMs, frontier.py:190,265-270).
    activations: str = "fp8"

    def __post_init__(self) -> None:
        if not self.id or self.family != FAMILY or not self.model or not self.phase:
            raise ValueError(f"invalid case {self.id}")
        p = self.params
        for name in ("tokens", "hidden", "experts", "topk", "intermediate"):
            if name not in p:
                raise ValueError(f"{self.id}: missing param {name}")
        if any(isinstance(v, bool) or not isinstance(v, int) or v < 1 for v in p.values()):
            raise ValueError(f"invalid dimensions in {self.id}")
        if min(self.gpus, self.tp, self.ep, self.max_gpu_launches) < 1:
            raise ValueError(f"invalid execution geometry in {self.id}")
        if min(self.atol, self.rtol, self.bf16_rtol) < 0 or self.noise_factor < 1:
            raise ValueError(f"invalid tolerance in {self.id}")
        if self.suite not in ("p0", "p1", "p2", "p3") or self.gate not in GATES:
            raise ValueError(f"invalid priority or gate in {self.id}")
        if self.router not in ROUTERS or self.bias not in BIASES:
            raise ValueError(f"invalid routing rule in {self.id}")
        if self.norm not in NORMS or not self.norm_eps >= 0:
            raise ValueError(f"invalid normalization in {self.id}")
        if self.swiglu not in SWIGLUS or not self.swiglu_limit >= 0 or (self.format == "mxfp4" and self.swiglu != "fp32"):
            raise ValueError(f"invalid SwiGLU form in {self.id}")
        if self.format not in FORMATS:
            raise ValueError(f"invalid expert format in {self.id}")
        if self.activations not in ("fp8", "bf16") or (self.activations == "bf16" and self.format != "fp8"):
            raise ValueError(f"{self.id}: bf16 activations (W8A16) are a form of the fp8 experts")
        if (self.format == "mxfp4") != (self.router == "given"):
            raise ValueError(f"{self.id}: the MXFP4 form takes its routing as an input, and only it does")
        if self.format == "mxfp4" and (p["hidden"] % 256 or p["intermediate"] % 256 or p.get("shared_experts", 0)
                                       or self.norm != "none" or self.residual or not self.swiglu_limit > 0):
            raise ValueError(f"{self.id}: the MXFP4 form needs H and I multiples of 256, no shared expert "
                             "or block steps, and a positive SwiGLU limit")
        if self.ep > 1 and (self.format != "mxfp4" or p["experts"] % self.ep or self.gpus != self.ep):
            raise ValueError(f"{self.id}: expert parallelism is defined for the MXFP4 form, over all ranks, "
                             "with ep dividing the experts")
        if self.router == "softmax" and self.bias != "none":
            raise ValueError(f"{self.id}: softmax routing takes no correction bias")
        groups, top = self.groups, self.top_groups
        if p["topk"] > p["experts"] or p["experts"] % groups or top > groups:
            raise ValueError(f"invalid routing geometry in {self.id}")
        if groups > 1 and top * (p["experts"] // groups) < p["topk"]:
            raise ValueError(f"{self.id}: kept groups hold fewer than topk experts")
        object.__setattr__(self, "params", dict(p))

    # -- derived geometry ------------------------------------------------------------
    @property
    def tokens(self) -> int:
        return self.params["tokens"]

    @property
    def hidden(self) -> int:
        return self.params["hidden"]

    @property
    def experts(self) -> int:
        return self.params["experts"]

    @property
    def topk(self) -> int:
        return self.params["topk"]

    @property
    def intermediate(self) -> int:
        return self.params["intermediate"]

    @property
    def shared_experts(self) -> int:
        return self.params.get("shared_experts", 0)

    @property
    def groups(self) -> int:
        return self.params.get("router_groups", 1)

    @property
    def top_groups(self) -> int:
        return self.params.get("router_top_groups", 1)

    def to_dict(self) -> dict:
        values = asdict(self)
        values["params"] = dict(self.params)
        return values

    @classmethod
    def from_dict(cls, values: dict) -> "Case":
        known = {f for f in cls.__dataclass_fields__}
        return cls(**{k: v for k, v in values.items() if k in known})


def _case(cid: str, model: str, *, note: str = "", **kw) -> Case:
    return Case(id=cid, family=FAMILY, model=model, phase="decode", note=note, **kw)


CASES: tuple[Case, ...] = (
    _case("moe-fp8-tiny-t4", "tiny-moe",
          params=dict(tokens=4, hidden=1024, experts=8, topk=2, intermediate=512),
          router="softmax", renormalize=True,
          note="CPU-runnable: x ~ N(0,1) bf16, router N(0,0.02) fp32, experts N(0,0.02) E4M3 128x128"),
    _case("moe-fp8-mixtral-t16", "mistralai/Mixtral-8x7B (MoE shape)",
          params=dict(tokens=16, hidden=4096, experts=8, topk=2, intermediate=14336),
          router="softmax", renormalize=True),
    _case("moe-fp8-qwen3-30b-a3b-t32", "Qwen/Qwen3-30B-A3B (MoE shape)",
          params=dict(tokens=32, hidden=2048, experts=128, topk=8, intermediate=768),
          router="softmax", renormalize=True),
    _case("moe-fp8-deepseek-v3-t64", "deepseek-ai/DeepSeek-V3 (MoE shape)",
          params=dict(tokens=64, hidden=7168, experts=256, topk=8, intermediate=2048, shared_experts=1,
                      router_groups=8, router_top_groups=4),
          router="sigmoid", renormalize=True, routed_scaling=2.5, bias="normal", bias_std=0.1),
    _case("moe-fp8-kimi-k2-t128", "moonshotai/Kimi-K2 (MoE shape, Zipf-skewed router bias)",
          params=dict(tokens=128, hidden=7168, experts=384, topk=8, intermediate=2048, shared_experts=1,
                      router_groups=1, router_top_groups=1),
          router="sigmoid", renormalize=True, routed_scaling=2.827, bias="zipf", zipf_s=1.1, zipf_c=1.0),
)

HEADLINE = "moe-fp8-deepseek-v3-t64"

# Block forms (the next step outward from the layer): the DeepSeek-V3 layer with its ln2
# RMSNorm (gamma in fp32, eps 1e-6) before it and the residual add after it, in one launch.
BLOCK_CASES: tuple[Case, ...] = (
    replace(next(c for c in CASES if c.id == HEADLINE), id=HEADLINE + "-block", norm="fp32_weight",
            norm_eps=1e-6, residual=True,
            note="decoder-block form: rms(x, ln2) -> layer -> x + bf16(out) (frontier.py:335-354)"),
    replace(next(c for c in CASES if c.id == "moe-fp8-qwen3-30b-a3b-t32"), id="moe-fp8-qwen3-30b-a3b-t32-block",
            norm="bf16_weight", norm_eps=1e-5, residual=True,
            note="decoder-block form with the Llama-style RMSNorm (gamma on the rounded activation)"),
)


# The MXFP4 routed-expert layer of megamoe.py (DeepSeek-V4-Pro geometry: 384 experts, top-6,
# H 7168, I 3072, SwiGLU limit 10, routed scaling 2.5; cases.py:380-387), serial, at a decode
# batch of 64 tokens: x arrives as E4M3 with E8M0 scales per 32, routing as ids and weights.
MX_CASES: tuple[Case, ...] = (
    _case("moe-mxfp4-deepseek-v4-pro-t64", "deepseek-ai/DeepSeek-V4-Pro (routed experts, MXFP4)",
          params=dict(tokens=64, hidden=7168, experts=384, topk=6, intermediate=3072),
          router="given", format="mxfp4", swiglu_limit=10.0, routed_scaling=2.5,
          note="megamoe numerics in serial mode: E2M1 x E4M3 scaled MFMA, clamped SwiGLU, E8M0 requant"),
)


# One rank's share of the expert-parallel MXFP4 layer at the reference's catalog geometry
# (megabench/cases.py:380-388: 512 tokens per rank, 8 ranks, 48 local experts each). On one
# GPU the share is the rank's dispatch, its local experts over the rows it receives and its
# combine (megamoe.py:153-182); the exchanges between them are collectives, not built here.
EP_CASES: tuple[Case, ...] = (
    _case("megamoe-layer-deepseek-v4-pro-ep8-t512", "deepseek-ai/DeepSeek-V4-Pro (routed experts, MXFP4, EP8)",
          params=dict(tokens=512, hidden=7168, experts=384, topk=6, intermediate=3072),
          router="given", format="mxfp4", swiglu_limit=10.0, routed_scaling=2.5, gpus=8, ep=8,
          max_gpu_launches=6,
          note="one rank's share: dispatch (order + pack), local experts (permute, experts, row copy), combine"),
)


# Epilogue variants of the fp8 layer: GLM-5.3-Flash's MoE (glm53.py:263-274): sigmoid
# routing with the correction bias and no groups (frontier.route(..., 1, 1), scaling 2.5),
# one shared expert, and SwiGLU in bf16 with the clamp at 10 (glm53.py:30,174-175); the
# geometry of its catalog entry (megabench/cases.py:304-313), 64 tokens as the other
# decode configs.
VARIANT_CASES: tuple[Case, ...] = (
    _case("moe-fp8-glm-5.3-flash-t64", "zai-org/GLM-5.3-Flash (MoE shape, clamped bf16 SwiGLU)",
          params=dict(tokens=64, hidden=4096, experts=288, topk=8, intermediate=2048, shared_experts=1,
                      router_groups=1, router_top_groups=1),
          router="sigmoid", renormalize=True, routed_scaling=2.5, bias="normal", bias_std=0.1,
          swiglu="bf16", swiglu_limit=10.0),
)


# Two variants of the headline shape. "-ue8m0": the DeepSeek family's power-of-two scales
# (UE8M0, "scale_fmt": "ue8m0" in model_specs.json:187), the weights' and the activations'
# alike (frontier.py:120,252 pass power=True to fp8_matrix and linear; quantization.py:57-59).
# "-nobias": the routing without the N(0, 0.1) correction bias. With the bias, the sigmoid
# squeezes the top scores together and the bias decides most selections, so 64 tokens hit
# only ~120 of the 256 experts (the headline's timing inputs: 120); without it ~222 are hit,
# ~2.3 rows each, the uniform-routing expectation that the per-config floors assume.
# "-w8a16": the expert GEMMs with bf16 activations (frontier.py:180-183, quantize=False),
# as the DeepSeek family's TileRT numerics run them (frontier.py:190,265-270).
# "-w8a16-ue8m0": both at once, the expert numerics of the DeepSeek family as the reference
# runs them (frontier.py:252-270: power=True for the weights' scales, quantize=False for
# every expert projection, since gate, up and down are not in DEEPSEEK_FP8_ACTIVATIONS); with
# no activation quantized, the power-of-two rule reaches only the weights.
HEADLINE_VARIANTS: tuple[Case, ...] = (
    replace(next(c for c in CASES if c.id == HEADLINE), id=HEADLINE + "-ue8m0", power_of_two=True,
            note="power-of-two (UE8M0) weight and activation scales"),
    replace(next(c for c in CASES if c.id == HEADLINE), id=HEADLINE + "-nobias", bias="none",
            note="no correction bias: ~222 experts hit, ~2.3 rows each"),
    replace(next(c for c in CASES if c.id == HEADLINE), id=HEADLINE + "-w8a16", activations="bf16",
            note="W8A16: bf16 activations into the expert GEMMs"),
    replace(next(c for c in CASES if c.id == HEADLINE), id=HEADLINE + "-w8a16-ue8m0", activations="bf16",
            power_of_two=True, note="W8A16 with UE8M0 weight scales: the DeepSeek family's expert numerics"),
)


def case(case_id: str) -> Case:
    for c in CASES + BLOCK_CASES + MX_CASES + EP_CASES + VARIANT_CASES + HEADLINE_VARIANTS:
        if c.id == case_id:
            return c
    raise KeyError(case_id)


def development(c: Case, **params) -> Case:
    """Reduced geometry of a catalog case with its routing rule kept.

    Like the reference's development geometries (megabench/verify_megamoe.py:32,
    megabench/tests/test_frontier.py:17-27): small enough for the CPU oracle to
    finish in well under a second, large enough to exercise groups, the shared
    expert and multi-row experts.
    """
    p = dict(c.params)
    small = dict(hidden=256, intermediate=256, experts=min(c.experts, 16), topk=min(c.topk, 4))
    if c.groups > 1:
        small.update(router_groups=4, router_top_groups=2)
    p.update(small)
    p.update(params)
    if p.get("router_groups", 1) > 1 and p["experts"] % p["router_groups"]:
        raise ValueError("development geometry breaks the group split")
    return replace(c, id=c.id + "-dev", params=p)


def algorithmic_bytes(c: Case, hit_experts: int) -> int:
    """HBM bytes one step must move: weights of the hit experts and the shared expert
    (E4M3 payload + fp32 128x128 scales), the fp32 router and bias, x and y in bf16,
    ids (int64) and weights (fp32); in the block form also the bf16 RMSNorm gamma. In the
    MXFP4 form: E2M1 payload (half a byte) + one E8M0 byte per 32 weights, x as E4M3 + E8M0
    per 32, ids and weights, y in bf16."""
    T, H, E, K, I, S = c.tokens, c.hidden, c.experts, c.topk, c.intermediate, c.shared_experts
    if c.format == "mxfp4":  # also one rank's share under EP, hit_experts counting local experts
        # (the HBM terms of megabench/sol.py:160-183)
        per_expert = 3 * I * H // 2 + 3 * I * H // 32
        return hit_experts * per_expert + T * H + T * H // 32 + 12 * T * K + 2 * T * H
    bh, bi = math.ceil(H / 128), math.ceil(I / 128)
    per_expert = 3 * I * H + 4 * (2 * bi * bh + bh * bi)
    shared = 0
    if S:
        si = S * I
        bsi = math.ceil(si / 128)
        shared = 3 * si * H + 4 * (2 * bsi * bh + bh * bsi)
    bias = 4 * E if c.router == "sigmoid" else 0
    gamma = 2 * H if c.norm != "none" else 0  # the block's ln2 (x is read once either way)
    return hit_experts * per_expert + shared + 4 * E * H + bias + gamma + 2 * T * H + 2 * T * H + 12 * T * K


def algorithmic_flops(c: Case) -> int:
    T, H, E, K, I, S = c.tokens, c.hidden, c.experts, c.topk, c.intermediate, c.shared_experts
    if c.format == "mxfp4":  # no router GEMV: routing is an input
        return 2 * T * K * 3 * I * H
    return 2 * T * E * H + 2 * T * K * 3 * I * H + 2 * T * S * 3 * I * H


def expected_hit_experts(c: Case) -> float:
    """E[U] under uniform routing: E * (1 - (1 - K/E)^T)."""
    return c.experts * (1.0 - (1.0 - c.topk / c.experts) ** c.tokens)
