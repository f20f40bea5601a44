"""GPT-OSS's combine of a token's expert outputs, restated on the CPU (test infrastructure).

megabench/tasks/gptoss.py:112-124: the outputs accumulate in ascending expert id order
("independent of router rank"), in bf16, from a bf16 zero row: for each slot in
``selected.argsort()``, ``output = output + probabilities[slot] * expert_output``, where the
probability and the output are bf16, so each product and each sum rounds to bf16; then
``x + output`` in bf16 (the residual add of the decoder step).

Pinned by tests/test_oracle_variants.py against a restatement in numpy with explicit bf16
rounding of every product and sum (from the fp32 bits), invariance under any permutation
of a token's slots, and planted mistakes (rank order, fp32 accumulation, the residual
added before the experts) that it must catch.
"""

from __future__ import annotations

import torch


def by_expert_id(expert_out: torch.Tensor, expert_ids: torch.Tensor, weights: torch.Tensor,
                 residual: torch.Tensor | None = None) -> torch.Tensor:
    """expert_out bf16 [T, K, H], expert_ids int64 [T, K], weights bf16 [T, K], residual
    bf16 [T, H] or None -> bf16 [T, H]."""
    T, K, H = expert_out.shape
    y = torch.empty((T, H), dtype=torch.bfloat16)
    for t in range(T):
        out = torch.zeros(H, dtype=torch.bfloat16)
        for slot in expert_ids[t].argsort(stable=True).tolist():
            out = out + weights[t, slot] * expert_out[t, slot]
        y[t] = out if residual is None else residual[t] + out
    return y
