"""Build the gfx950 code object and the loader library in-tree.

  compiler_amd/lib/g950.hsaco     every hot-path kernel (hipcc --genco, gfx950)
  compiler_amd/lib/libg950rt.so   the C-ABI module loader/launcher (include/g950rt.h)
  compiler_amd/lib/g950_exec      the bundle-driven command-line runner

They are written next to the package so they travel with the source tree; the
Python runtime loads exactly the first two.
"""
from __future__ import annotations

import os
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
LIB = PKG / "lib"
HSACO = LIB / "g950.hsaco"
RTLIB = LIB / "libg950rt.so"
EXEC = LIB / "g950_exec"
ARCH = "gfx950"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

# Packed-fp32 VALU forms are disabled for every device compile: hand-written
# and compiler-generated v_pk_{add,mul,fma}_f32 are kept out of all kernels.
DEVICE_FLAGS = ["-O3", f"--offload-arch={ARCH}", "-Xclang", "-target-feature", "-Xclang",
                "-packed-fp32-ops", "-ffp-contract=fast", "-std=c++17"]


def _run(cmd):
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        sys.stderr.write(proc.stdout + proc.stderr)
        raise RuntimeError(f"build step failed ({proc.returncode}): {' '.join(map(str, cmd))}")
    return proc


def build_code_object() -> Path:
    LIB.mkdir(exist_ok=True)
    tmp = HSACO.with_suffix(".hsaco.tmp")
    _run([HIPCC, *DEVICE_FLAGS, "--genco", f"-I{CSRC}", "-o", str(tmp), str(CSRC / "g950_kernels.hip")])
    os.replace(tmp, HSACO)
    return HSACO


def build_runtime() -> Path:
    LIB.mkdir(exist_ok=True)
    tmp = RTLIB.with_name(RTLIB.name + ".tmp")
    # g950_scratch.hip carries the no-alloc entry's static device array: the
    # library holds one gfx950 code object of its own for it
    _run([HIPCC, "-O2", "-std=c++17", "-fPIC", "-shared", "-Wall", f"--offload-arch={ARCH}", "-Xclang",
          "-target-feature", "-Xclang", "-packed-fp32-ops", f"-I{ROOT / 'include'}", f"-I{CSRC}", "-o",
          str(tmp), str(CSRC / "g950rt.cpp"), str(CSRC / "g950_bundle.cpp"), str(CSRC / "g950_scratch.hip")])
    os.replace(tmp, RTLIB)
    return RTLIB


def build_exec() -> Path:
    """g950_exec: the bundle-driven command-line runner (links libg950rt.so)."""
    tmp = EXEC.with_name(EXEC.name + ".tmp")
    _run(["g++", "-O2", "-std=c++17", "-Wall", f"-I{ROOT / 'include'}", "-o", str(tmp),
          str(CSRC / "g950_exec.cpp"), f"-L{LIB}", "-lg950rt", "-Wl,-rpath,$ORIGIN"])
    os.replace(tmp, EXEC)
    return EXEC


def build_all() -> None:
    build_code_object()
    build_runtime()
    build_exec()


if __name__ == "__main__":
    build_all()
    print(HSACO, RTLIB)
