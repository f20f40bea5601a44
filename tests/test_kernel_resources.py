"""The compiler's resource report for the built library (written by the build).

The expert kernels stream the weights through MFMA loops tuned to stay within two
workgroups' share of the register file: a spill or a stack array there costs time with no
change in the results (one copy of the MXFP4 gate/up units shared by two kernels once
compiled k_experts_mx to 256 VGPRs with scratch and slowed it from 1220 to 1694 us), so
these figures are checked on the CPU after every build.
"""

import json
import subprocess

import pytest

from vibe_megakernel_amd import build as pkg_build


def _report():
    if not pkg_build.REPORT.exists():
        pytest.skip("no resource report: the library has not been built here")
    return json.loads(pkg_build.REPORT.read_text())


def _demangle(names):
    out = subprocess.run(["c++filt"], input="\n".join(names), capture_output=True, text=True, check=True)
    return dict(zip(out.stdout.splitlines(), names))


STREAM_KERNELS = [
    "(anonymous namespace)::k_experts<false, false>",
    "(anonymous namespace)::k_experts<true, false>",
    "(anonymous namespace)::k_experts<false, true>",  # the W8A16 form
    "(anonymous namespace)::k_experts_mx",
    "(anonymous namespace)::k_experts_mx_batch",
]


@pytest.mark.parametrize("kernel", STREAM_KERNELS)
def test_expert_stream_kernels_have_no_scratch(kernel):
    r = _entry(_report(), kernel)
    assert r["scratch_bytes"] == 0 and r["vgpr_spills"] == 0, (kernel, r)
    # Two workgroups of 256 threads per CU (k_experts_mx_batch: one, with its LDS rings).
    assert r["occupancy"] >= (1 if kernel.endswith("_batch") else 2), (kernel, r)


# The single-launch kernels hold the front end (norm, router, routing, permute) and the
# control flow of every phase beside the expert units, all within two workgroups' share of the
# register file. None of them spills a VGPR: the routing keeps its logits, choices and bias in
# LDS (and, from 512 experts, its selection keys), derives its expert indices from an opaque
# lane so they are not hoisted out of the persistent loop, and the combine takes its first
# slots by value. k_layer<false, ...> keeps a 20-byte private segment that no instruction uses.
LAYER_CEILINGS = {
    "(anonymous namespace)::k_layer<false, false>": {"vgpr_spills": 0, "scratch_bytes": 20},
    "(anonymous namespace)::k_layer<true, false>": {"vgpr_spills": 0, "scratch_bytes": 20},
    "(anonymous namespace)::k_layer<false, true>": {"vgpr_spills": 0, "scratch_bytes": 20},  # the W8A16 form
    "(anonymous namespace)::k_layer_mx": {"vgpr_spills": 0, "scratch_bytes": 0},
}


def _entry(report, kernel):
    names = _demangle(list(report))
    # Template instances demangle with their return type, plain functions without.
    match = [m for d, m in names.items() if d.startswith((f"void {kernel}(", f"{kernel}("))]
    assert len(match) == 1, (kernel, sorted(names))
    return report[match[0]]


@pytest.mark.parametrize("kernel", sorted(LAYER_CEILINGS))
def test_single_launch_kernels_spill_no_more_than_now(kernel):
    r = _entry(_report(), kernel)
    for field, ceiling in LAYER_CEILINGS[kernel].items():
        assert r[field] <= ceiling, (kernel, field, r)
    assert r["occupancy"] >= 2, (kernel, r)


def test_parser_reads_hipcc_remarks():
    text = (
        "a.hip:1:1: remark: Function Name: _Z1kv [-Rpass-analysis=kernel-resource-usage]\n"
        "a.hip:1:1: remark:     VGPRs: 237 [-Rpass-analysis=kernel-resource-usage]\n"
        "a.hip:1:1: remark:     ScratchSize [bytes/lane]: 0 [-Rpass-analysis=kernel-resource-usage]\n"
        "a.hip:1:1: remark:     Occupancy [waves/SIMD]: 2 [-Rpass-analysis=kernel-resource-usage]\n"
        "a.hip:1:1: remark:     VGPRs Spill: 6 [-Rpass-analysis=kernel-resource-usage]\n"
        "a.hip:9:1: remark: Function Name: _Z1jv [-Rpass-analysis=kernel-resource-usage]\n"
        "a.hip:9:1: remark:     VGPRs: 12 [-Rpass-analysis=kernel-resource-usage]\n"
    )
    assert pkg_build.resource_report(text) == {
        "_Z1kv": {"vgprs": 237, "scratch_bytes": 0, "occupancy": 2, "vgpr_spills": 6},
        "_Z1jv": {"vgprs": 12},
    }
