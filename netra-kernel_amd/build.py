"""Build the gfx950 artefacts in-tree.

Outputs (git-ignored, shipped with the source tree to the GPU host):
  netra-kernel_amd/lib/netra_moe_gfx950.hsaco  code object loaded by the engine
  netra-kernel_amd/lib/libnetra_engine.so      C-ABI engine runtime
  netra-kernel_amd/lib/libnetra_moe.so         direct entry points (weight prep, no-alloc prefill)
  netra-kernel_amd/lib/libnetra_bridges.so     the reference's per-operation bridge ABIs

Run: python netra-kernel_amd/build.py  (or __graft_entry__.build()).
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
REPO = PKG.parent
CSRC = PKG / "csrc"
LIB = PKG / "lib"
ROCM = Path(os.environ.get("ROCM_PATH", "/opt/rocm"))

HIPCC = str(ROCM / "bin" / "hipcc")
ARCH = "gfx950"
# Packed fp32 VALU ops are disabled for all device code; exact fp32 contract
# order needs contraction off (fmaf is written explicitly where wanted).
# MFMAs take the VGPR form: otherwise the scaled-accumulate GEMM loops route
# every product through one AGPR quad and read it back, which serialises the
# matrix core on its own results.
DEVICE_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-mllvm", "-amdgpu-mfma-vgpr-form=1",
    "-Wall", "-Wno-unused-parameter",
]

HSACO = LIB / "netra_moe_gfx950.hsaco"
ENGINE_SO = LIB / "libnetra_engine.so"
BRIDGE_SO = LIB / "libnetra_moe.so"
OPS_SO = LIB / "libnetra_bridges.so"


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, capture_output=True, text=True)
    noise = "packed-fp32-ops"
    err = "\n".join(l for l in proc.stderr.splitlines() if noise not in l and l.strip())
    if proc.returncode != 0:
        raise RuntimeError(f"build step failed ({proc.returncode}): {' '.join(cmd)}\n{err}")


def build_hsaco() -> Path:
    LIB.mkdir(exist_ok=True)
    tmp = HSACO.with_suffix(".hsaco.tmp")
    _run([HIPCC, *DEVICE_FLAGS, "--genco", "-o", str(tmp), str(CSRC / "kernels" / "moe_kernels.hip")])
    tmp.replace(HSACO)
    return HSACO


def build_engine() -> Path:
    LIB.mkdir(exist_ok=True)
    tmp = ENGINE_SO.with_suffix(".so.tmp")
    cxx = shutil.which("g++") or "g++"
    _run([
        cxx, "-O2", "-std=c++17", "-fPIC", "-shared", "-Wall", "-Wextra",
        "-D__HIP_PLATFORM_AMD__", f"-I{ROCM / 'include'}", f"-I{REPO / 'include'}",
        str(CSRC / "engine" / "manifest.cpp"), str(CSRC / "engine" / "netra_engine.cpp"),
        f"-L{ROCM / 'lib'}", f"-Wl,-rpath,{ROCM / 'lib'}", "-lamdhip64",
        "-o", str(tmp),
    ])
    tmp.replace(ENGINE_SO)
    return ENGINE_SO


def build_bridge() -> Path:
    LIB.mkdir(exist_ok=True)
    tmp = BRIDGE_SO.with_suffix(".so.tmp")
    _run([HIPCC, *DEVICE_FLAGS, "-fPIC", "-shared", "-o", str(tmp),
          str(CSRC / "bridge" / "moe_bridge.hip")])
    tmp.replace(BRIDGE_SO)
    return BRIDGE_SO


def build_op_bridges() -> Path:
    """Host-only library (like the engine): module management and dispatch."""
    LIB.mkdir(exist_ok=True)
    tmp = OPS_SO.with_suffix(".so.tmp")
    cxx = shutil.which("g++") or "g++"
    _run([
        cxx, "-O2", "-std=c++17", "-fPIC", "-shared", "-Wall", "-Wextra",
        "-D__HIP_PLATFORM_AMD__", f"-I{ROCM / 'include'}", f"-I{REPO / 'include'}",
        str(CSRC / "bridge" / "qwen36_bridges.cpp"),
        f"-L{ROCM / 'lib'}", f"-Wl,-rpath,{ROCM / 'lib'}", "-lamdhip64",
        "-o", str(tmp),
    ])
    tmp.replace(OPS_SO)
    return OPS_SO


def build_all() -> list[Path]:
    return [build_hsaco(), build_engine(), build_bridge(), build_op_bridges()]


if __name__ == "__main__":
    for p in build_all():
        print(p.relative_to(REPO))
    sys.exit(0)
