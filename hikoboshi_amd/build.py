"""Builds the HIP library hikoboshi_amd/libhkbs_pmpnn.so for gfx950 (in-tree).

    python -m hikoboshi_amd.build

hipcc compiles the kernels and the C-ABI layer in one shared object. Packed
FP32 instruction selection is disabled on the device side. build_device_check()
builds the test-only library tests/libdevice_math_check.so (an exhaustive GPU
check of the device GELUs) with the same device flags.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
CSRC = HERE / "csrc"
LIB = HERE / "libhkbs_pmpnn.so"
CHECK_SRC = HERE.parent / "tests" / "csrc" / "device_math_check.hip"
CHECK_LIB = HERE.parent / "tests" / "libdevice_math_check.so"
ARCH = os.environ.get("HKBS_OFFLOAD_ARCH", "gfx950")
SOURCES = ["knn.hip", "features.hip", "encoder.hip", "encoder16.hip", "decoder.hip", "decoder_tf.hip", "capi.hip", "host_noise.cpp",
           "structure_io.cpp"]
# Host-only C++ (no device code), without floating-point contraction.
HOST_FLAGS = ["-ffp-contract=off"]
# The decode kernel keeps many loop-invariant values across its pass loop; sinking
# them back into the loop where that avoids spills leaves registers for the weight
# loads in flight.
# The reference-order encoder adds matrix-core products to its accumulators on
# the VALU; the products have to land in ordinary VGPRs (not AGPRs, which would
# cost a copy per product).
DEVICE_FLAGS = {
    "decoder.hip": ["-mllvm", "-sink-insts-to-avoid-spills"],
    "encoder.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=1"],
    "features.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=1"],
}


def source_flags(src: str) -> list:
    """Extra compiler flags of one source file."""
    return HOST_FLAGS if src.endswith(".cpp") else DEVICE_FLAGS.get(src, [])


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found")


def _common() -> list:
    return [
        hipcc(), "-std=c++17", "-O3", "-fPIC", f"--offload-arch={ARCH}",
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        "-Wno-unused-command-line-argument", "-I", str(HERE.parent / "include"),
    ]


def build(verbose: bool = False) -> Path:
    objs = []
    obj_dir = HERE / "_build"
    obj_dir.mkdir(exist_ok=True)
    common = _common()
    for src in SOURCES:
        obj = obj_dir / (Path(src).stem + ".o")
        cmd = common + source_flags(src) + ["-c", str(CSRC / src), "-o", str(obj)]
        if verbose:
            print(" ".join(cmd), flush=True)
        subprocess.run(cmd, check=True)
        objs.append(str(obj))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [hipcc(), "-shared", "-fPIC", f"--offload-arch={ARCH}", "-o", str(tmp)] + objs
    if verbose:
        print(" ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)
    tmp.replace(LIB)
    return LIB


def build_device_check(verbose: bool = False) -> Path:
    tmp = CHECK_LIB.with_suffix(".so.tmp")
    cmd = _common() + ["-shared", str(CHECK_SRC), "-o", str(tmp)]
    if verbose:
        print(" ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)
    tmp.replace(CHECK_LIB)
    return CHECK_LIB


if __name__ == "__main__":
    build(verbose="-v" in sys.argv)
    build_device_check(verbose="-v" in sys.argv)
    print(LIB)
