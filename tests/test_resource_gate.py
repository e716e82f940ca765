"""CPU gate on the built library's gfx950 code objects (reference
scripts/check_fused_bwd_kernel_gate.py:61-212 gates its kernel on scratch and
spills the same way): no scratch, no spills, LDS within a CU, VGPRs within
the budget that keeps a whole workgroup resident.  Reads only metadata of the
library built in this tree."""
import os

import pytest

import resource_gate as gate

EXPECTED = ("bwd_main_kernel", "bwd_component_kernel", "preprocess_kernel", "rowstats_kernel")


@pytest.fixture(scope="module")
def gated():
    if not os.path.exists(gate.LIB_PATH):
        pytest.fail(f"{gate.LIB_PATH} is not built (make -C flash-attention3_amd)")
    return gate.check(gate.LIB_PATH)


def test_every_kernel_passes(gated):
    kernels, bad = gated
    assert kernels, "no gfx950 code object found"
    assert bad == []


def test_shipped_kernels_present(gated):
    names = [k[".name"] for k in gated[0]]
    for want in EXPECTED:
        assert any(want in n for n in names), want
    # every (head dim, causal, bf16) instantiation of the main kernel with
    # scaled and unscaled resident operands, in the role-major and the
    # head-split job orders (the causal ones also level by level), and the
    # split-plan instantiations of the causal ones (unscaled only), without
    # and with the code for short jobs after pieces: 48, each with its
    # race-check twin (shaobo_fa3_ext_set_race_check), which the gate holds
    # to the same budget
    assert sum("bwd_main_kernel" in n for n in names) == 96
    # the head-split plan's reduction of the per-query-head dK / dV
    assert sum("gqa_reduce_kernel" in n for n in names) == 4


def test_main_kernel_two_waves_per_simd(gated):
    for k in gated[0]:
        if "bwd_main_kernel" in k[".name"]:
            assert k[".max_flat_workgroup_size"] == 512
            assert gate.violations(k) == []


BASE = {".name": "k", ".private_segment_fixed_size": 0, ".uses_dynamic_stack": False,
        ".vgpr_spill_count": 0, ".sgpr_spill_count": 0, ".group_segment_fixed_size": 1024,
        ".max_flat_workgroup_size": 512, ".vgpr_count": 128, ".agpr_count": 0}


@pytest.mark.parametrize("key,value,what", [
    (".private_segment_fixed_size", 16, "scratch"),
    (".uses_dynamic_stack", True, "dynamic stack"),
    (".vgpr_spill_count", 3, "vgpr_spill_count"),
    (".sgpr_spill_count", 1, "sgpr_spill_count"),
    (".group_segment_fixed_size", 160 * 1024 + 4, "LDS"),
    (".vgpr_count", 257, "VGPRs"),
    (".agpr_count", 132, "VGPRs"),  # 128 + 132 > 256
])
def test_planted_violations_are_caught(key, value, what):
    assert gate.violations(BASE) == []
    bad = gate.violations(dict(BASE, **{key: value}))
    assert len(bad) == 1 and what in bad[0]


def test_budget_follows_workgroup_size():
    # 256 threads = one wave per SIMD: the whole 512-register file
    assert gate.violations(dict(BASE, **{".max_flat_workgroup_size": 256, ".vgpr_count": 500})) == []
    assert gate.violations(dict(BASE, **{".max_flat_workgroup_size": 1024, ".vgpr_count": 129}))
