"""A time-bounded randomized soak of the single launch, through the C ABI.

The single launch hands data between its workgroups (router partials, ids, the lists, h, d)
by write-through stores published by counters, and its waits acquire at workgroup scope:
that is right only if no workgroup reads a line of such data before the line's last write.
A violation would show as a stale value from an earlier call or writer, rarely and
depending on the data. So this runs many calls on random development geometries (the five
configs' families, the block and epilogue forms, random token counts) with random seeds,
consecutive calls sharing one workspace, and checks each against the stream-ordered kernels
bit for bit and the status word after each call (half the calls at 16 tokens or fewer, most
of them in the dense schedule, whose expert units run before the routing is known; a quarter
in the W8A16 form). The MXFP4 layer's one launch (k_layer_mx: the permute, the expert units
and the combine of one queue, the same hand-overs) takes part as well, against its three
stream-ordered kernels. It stops at the first mismatch and names the geometry and seed.
MEGAMOE_SOAK_SECONDS sets the time bound (default 20 s), MEGAMOE_SOAK_SEED the stream of
geometries and seeds (default 20261202).
"""

from __future__ import annotations

import os
import random
import sys
import time

import pytest
import torch

from vibe_megakernel_amd import cases as C
from vibe_megakernel_amd import submission, workloads

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _log(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _geometries(rng):
    """An endless stream of development geometries: a family, then a token count."""
    families = [C.development(c) for c in C.CASES[1:]] + [C.case("moe-fp8-tiny-t4")]
    families += [C.development(C.case("moe-fp8-kimi-k2-t128"), experts=8, topk=4),  # hot experts
                 C.development(C.case("moe-fp8-mixtral-t16"), hidden=4096, intermediate=512),  # split gate/up
                 C.development(C.case("moe-fp8-kimi-k2-t128"), experts=16, topk=4),  # Zipf: many unpicked
                 C.development(C.BLOCK_CASES[0]), C.development(C.VARIANT_CASES[0]),
                 # MXFP4, one launch: ~8 rows per expert or fewer at 64 experts; 16 experts reach
                 # the batch shape (stream-ordered in both forms) from ~100 tokens.
                 C.development(C.MX_CASES[0], experts=64), C.development(C.MX_CASES[0])]
    while True:
        base = rng.choice(families)
        if base.format == "fp8" and rng.random() < 0.25:  # a quarter of the calls in the W8A16 form
            base = C.Case.from_dict({**base.to_dict(), "id": base.id + "-w8a16", "activations": "bf16"})
        # Half the calls at 16 tokens or fewer, where the dense schedule runs (with T*K >= E).
        tokens = rng.randint(1, 16) if rng.random() < 0.5 else rng.randint(17, 130)
        yield C.Case.from_dict({**base.to_dict(), "id": f"{base.id}-soak",
                                "params": {**base.params, "tokens": tokens}})


def _mx_call_inputs(case, seed, weights):
    """An MXFP4 call's inputs on the geometry's expert weights (generating MXFP4 weights takes
    most of a call's time): x and the routing anew from the seed, as make_inputs draws them."""
    x = torch.randn((case.tokens, case.hidden), generator=torch.Generator(device=DEV).manual_seed(seed), device=DEV)
    values = dict(weights)
    values["x"], values["x_scales"] = workloads.pack_e4m3_e8m0(x)
    values["topk_idx"], values["topk_weights"] = workloads.mx_routing(case, seed, DEV)
    return values


def test_randomized_single_launch_soak():
    seconds = float(os.environ.get("MEGAMOE_SOAK_SECONDS", "20"))
    rng = random.Random(int(os.environ.get("MEGAMOE_SOAK_SEED", "20261202")))
    t_end = time.monotonic() + seconds
    calls = geometries = 0
    t_note = time.monotonic() + 30.0
    for case in _geometries(rng):
        if time.monotonic() > t_end:
            break
        if time.monotonic() > t_note:  # a line every 30 s for long runs (shown with pytest -s)
            _log(f"soak: {calls} calls over {geometries} geometries so far")
            t_note += 30.0
        geometries += 1
        one = submission.MoELayer(case)
        five = submission.MoELayer(case, single_launch=False)
        weights = None
        for _ in range(rng.randint(4, 12)):  # consecutive calls on one workspace
            seed = rng.randrange(1 << 30)
            what = f"{case.id} T={case.tokens} H={case.hidden} E={case.experts} K={case.topk} seed {seed}"
            values = _mx_call_inputs(case, seed, weights) if weights is not None else workloads.make_inputs(case, seed, DEV)
            if case.format == "mxfp4":
                weights = {k: v for k, v in values.items() if k.startswith(("l1_", "l2_"))}
            a, b = one(values), five(values)
            torch.cuda.synchronize()
            for k in a:  # y, and the fp8 layers' expert ids and weights
                assert torch.equal(a[k], b[k]), f"{what}: {k} differs after {calls} calls"
            assert not one.gave_up(torch.device(DEV)), f"{what}: a bounded wait gave up"
            calls += 1
    _log(f"soak: {calls} single-launch calls over {geometries} geometries in {seconds:.0f} s, all equal to "
         "the stream-ordered form")
    assert calls > 0
