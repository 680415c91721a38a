"""Build recipe for the gfx950 library zero_amd/libzero_amd.so.

Every translation unit in zero_amd/csrc is compiled by hipcc for gfx950
only, in parallel, then linked into one shared library that exports the C
ABI of include/zero_gpu.h.  zero_amd/csrc/module/zg_module.hip is compiled
on its own into the code object zero_amd/zg_kernels.hsaco (an unbundled
gfx950 ELF, the entry points of include/zero_gpu_kernels.h) for hosts that
load kernels with hipModuleLoad.  Packed FP32 VALU instructions are disabled
(-target-feature -packed-fp32-ops) for every device compilation.  MFMA
results are kept in ordinary VGPRs (-amdgpu-mfma-vgpr-form): the prefill
GEMM reads every accumulator after each block, and the AGPR form would add
one v_accvgpr_read per value.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
BUILD = PKG / "_build"
LIB = PKG / "libzero_amd.so"
MODULE_SRC = CSRC / "module" / "zg_module.hip"
MODULE = PKG / "zg_kernels.hsaco"
ARCH = "gfx950"

HIPCC = os.environ.get("HIPCC", shutil.which("hipcc") or "/opt/rocm/bin/hipcc")

DEVICE_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-mllvm", "-amdgpu-mfma-vgpr-form",
    "-Wno-unused-result",
    "-Wno-unused-value",
]


def _compile(src: Path) -> Path:
    obj = BUILD / (src.stem + ".o")
    cmd = [HIPCC, *DEVICE_FLAGS, "-c", str(src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{res.stderr}")
    return obj


def build_module(verbose: bool = True) -> Path:
    """Compile csrc/module/zg_module.hip into the gfx950 code object
    zg_kernels.hsaco (device code only, not an offload bundle)."""
    tmp = MODULE.with_suffix(".hsaco.tmp")
    cmd = [HIPCC, *DEVICE_FLAGS, "--cuda-device-only", "--no-gpu-bundle-output", "-c", str(MODULE_SRC), "-o", str(tmp)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {MODULE_SRC.name}:\n{res.stderr}")
    os.replace(tmp, MODULE)
    if verbose:
        print(f"built {MODULE}", file=sys.stderr)
    return MODULE


def build(verbose: bool = True) -> Path:
    """Compile every csrc/*.hip for gfx950 and link libzero_amd.so, then
    build the code object of csrc/module."""
    BUILD.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    jobs = min(len(sources), int(os.environ.get("MAX_JOBS", "8")))
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(_compile, sources))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB} from {len(sources)} sources", file=sys.stderr)
    build_module(verbose)
    return LIB


if __name__ == "__main__":
    build()
