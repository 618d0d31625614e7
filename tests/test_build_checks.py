"""The build's scratch check (ironmlx_amd/build.py): kernels that load into
registers with inline assembly and wait with explicit vmcnt must not use
scratch, and the resource-usage report is parsed per kernel."""
from ironmlx_amd import build

REPORT = """
x.hip:10:1: remark: Function Name: _Z1av [-Rpass-analysis=kernel-resource-usage]
x.hip:10:1: remark:     VGPRs: 128 [-Rpass-analysis=kernel-resource-usage]
x.hip:10:1: remark:     ScratchSize [bytes/lane]: 0 [-Rpass-analysis=kernel-resource-usage]
x.hip:20:1: remark: Function Name: _Z1bv [-Rpass-analysis=kernel-resource-usage]
x.hip:20:1: remark:     VGPRs: 256 [-Rpass-analysis=kernel-resource-usage]
x.hip:20:1: remark:     VGPRs Spill: 12 [-Rpass-analysis=kernel-resource-usage]
x.hip:20:1: remark:     ScratchSize [bytes/lane]: 52 [-Rpass-analysis=kernel-resource-usage]
x.hip:30:1: remark: Function Name: _Z1cv [-Rpass-analysis=kernel-resource-usage]
x.hip:30:1: remark:     ScratchSize [bytes/lane]: 0 [-Rpass-analysis=kernel-resource-usage]
"""


def test_scratch_kernels_parses_report():
    assert build.scratch_kernels(REPORT) == ["_Z1bv"]
    assert build.scratch_kernels("") == []


def test_register_load_files_are_checked():
    # every file whose kernels use the asm register load is in the checked set
    import os
    csrc = os.path.join(os.path.dirname(build.__file__), "csrc")
    users = {n for n in os.listdir(csrc) if n.endswith(".hip") and "gload16(" in open(os.path.join(csrc, n)).read()}
    assert users and users <= build.NO_SCRATCH
