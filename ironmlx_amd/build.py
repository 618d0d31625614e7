"""Builds ironmlx_amd/libiqmm.so (the C-ABI HIP library) with hipcc for gfx950.

Every kernel translation unit under csrc/ is compiled in parallel into
ironmlx_amd/_build/*.o, then linked into one shared library next to this
file, so that it travels with the source tree.  Run:  python -m ironmlx_amd.build
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import re
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OBJ = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libiqmm.so")
SOURCES = ["api.hip", "qmv.hip", "qmv_q4.hip", "qmm_mfma.hip", "qmm_gemm.hip", "qmm_skinny.hip", "convert.hip", "moe.hip", "workspace.hip", "qmm_decode.hip", "qmm_gather.hip", "qmm_stream.hip"]
# per-file flags: MFMA results in VGPRs (no AGPR round trip before the VALU epilogue)
FILE_FLAGS = {"qmm_decode.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
              "qmm_stream.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
              "qmm_gather.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"]}
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"
FLAGS = ["-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}",
         # keep the compiler from emitting packed-fp32 VALU ops
         "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
         "-Wno-unused-result"]


# Kernels whose K loops load into registers with inline assembly and wait with
# explicit vmcnt: the compiler treats such an output as written when the asm
# statement issues, so a kernel that spills or copies a register before its
# load has landed (to scratch, or to an AGPR when the 256 VGPRs are used up)
# reads stale data, or has the late load overwrite a register reused
# meanwhile.  Their files are compiled with the resource-usage report and the
# build fails for any kernel that uses scratch, reaches the VGPR limit, or
# (files built with MFMA results in VGPRs) uses AGPRs at all.
NO_SCRATCH = {"qmm_decode.hip", "qmm_gather.hip"}


def register_loads(name: str) -> bool:
    """Whether a qmm_decode_kernel / gather_decode_kernel instantiation loads x
    into registers: its first bool template argument (XL, x through LDS) is 0."""
    m = re.search(r"_kernelI.*?Lb([01])E", name)
    return not (m and m.group(1) == "1")


def spilling_kernels(remarks: str, agprs_allowed: bool = True) -> list[str]:
    """Kernels of a -Rpass-analysis=kernel-resource-usage report that load into
    registers (register_loads) and use scratch, all 256 VGPRs, or
    (agprs_allowed False) any AGPR."""
    out = []
    for block in remarks.split("remark: Function Name: ")[1:]:
        name = block.split()[0]
        if not register_loads(name):
            continue

        def field(key):
            m = re.search(key + r": (\d+)", block)
            return int(m.group(1)) if m else 0
        if (field(r"ScratchSize \[bytes/lane\]") > 0 or field("VGPRs") >= 256
                or (not agprs_allowed and field("AGPRs") > 0)):
            out.append(name)
    return out


def _compile(src: str) -> str:
    obj = os.path.join(OBJ, os.path.splitext(src)[0] + ".o")
    extra = ["-Rpass-analysis=kernel-resource-usage"] if src in NO_SCRATCH else []
    cmd = [HIPCC, *FLAGS, *FILE_FLAGS.get(src, []), *extra, "-c", os.path.join(CSRC, src), "-o", obj]
    p = subprocess.run(cmd, capture_output=True, text=True)
    if p.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{p.stderr}")
    if src in NO_SCRATCH:
        bad = spilling_kernels(p.stderr, agprs_allowed="-amdgpu-mfma-vgpr-form" not in FILE_FLAGS.get(src, []))
        if bad:
            os.remove(obj)
            raise RuntimeError(f"{src}: kernels with register loads in flight use scratch: {bad[:8]}")
    return obj


def build(verbose: bool = True) -> str:
    os.makedirs(OBJ, exist_ok=True)
    with cf.ThreadPoolExecutor(max_workers=min(len(SOURCES), os.cpu_count() or 4)) as ex:
        objs = list(ex.map(_compile, SOURCES))
    cmd = [HIPCC, "-shared", "-fPIC", f"--offload-arch={ARCH}", *objs, "-o", LIB]
    p = subprocess.run(cmd, capture_output=True, text=True)
    if p.returncode != 0:
        raise RuntimeError(f"link failed:\n{p.stderr}")
    if verbose:
        print(f"built {LIB}")
    return LIB


if __name__ == "__main__":
    build()
    sys.exit(0)
