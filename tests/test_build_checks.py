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


REPORT_AGPR = """
y.hip:5:1: remark: Function Name: _Z1dv [-Rpass-analysis=kernel-resource-usage]
y.hip:5:1: remark:     VGPRs: 200 [-Rpass-analysis=kernel-resource-usage]
y.hip:5:1: remark:     AGPRs: 0 [-Rpass-analysis=kernel-resource-usage]
y.hip:5:1: remark:     ScratchSize [bytes/lane]: 0 [-Rpass-analysis=kernel-resource-usage]
y.hip:9:1: remark: Function Name: _Z1ev [-Rpass-analysis=kernel-resource-usage]
y.hip:9:1: remark:     VGPRs: 256 [-Rpass-analysis=kernel-resource-usage]
y.hip:9:1: remark:     AGPRs: 34 [-Rpass-analysis=kernel-resource-usage]
y.hip:9:1: remark:     ScratchSize [bytes/lane]: 0 [-Rpass-analysis=kernel-resource-usage]
y.hip:13:1: remark: Function Name: _Z1fv [-Rpass-analysis=kernel-resource-usage]
y.hip:13:1: remark:     VGPRs: 120 [-Rpass-analysis=kernel-resource-usage]
y.hip:13:1: remark:     AGPRs: 8 [-Rpass-analysis=kernel-resource-usage]
y.hip:13:1: remark:     ScratchSize [bytes/lane]: 0 [-Rpass-analysis=kernel-resource-usage]
"""


def test_spilling_kernels_parses_report():
    assert build.spilling_kernels(REPORT) == ["_Z1bv"]
    assert build.spilling_kernels("") == []
    # at the VGPR limit (copies into AGPRs without scratch) is rejected; AGPRs
    # alone only where MFMA results are meant to stay in VGPRs
    assert build.spilling_kernels(REPORT_AGPR) == ["_Z1ev"]
    assert build.spilling_kernels(REPORT_AGPR, agprs_allowed=False) == ["_Z1ev", "_Z1fv"]


def test_register_load_instantiations():
    # qmm_decode_kernel<XT, NT, MT, GB, S, D, KB, XL, GLU, MAPPED>: XL = 1 takes x
    # through LDS (no register loads), XL = 0 loads x into registers
    xl = "_ZN4iqmm12_GLOBAL__N_117qmm_decode_kernelILi2ELi2ELi2ELi4ELi4ELi2ELi8ELb1ELb1ELb0EEEvNS_7QmmArgsE"
    reg = "_ZN4iqmm12_GLOBAL__N_117qmm_decode_kernelILi2ELi4ELi2ELi2ELi8ELi2ELi4ELb0ELb1ELb0EEEvNS_7QmmArgsE"
    gat = "_ZN4iqmm12_GLOBAL__N_120gather_decode_kernelILi2ELi4ELi2ELi4ELi2ELi4ELb0ELb0ELi1EEEvNS_7QmmArgsElPKl"
    assert not build.register_loads(xl)
    assert build.register_loads(reg) and build.register_loads(gat)


def test_register_load_files_are_checked():
    # every file whose kernels use the asm register load is in the checked set
    import os
    csrc = os.path.join(os.path.dirname(build.__file__), "csrc")
    users = {n for n in os.listdir(csrc) if n.endswith(".hip") and "gload16(" in open(os.path.join(csrc, n)).read()}
    assert users and users <= build.NO_SCRATCH
