"""Build the oracle's C baseline (test infrastructure): oracle/lib/libg950_oracle.so.

The reference's own hot-path implementation cannot be built here: its
operators are Triton kernels compiled by a100c into RISC-V assembly that needs
the SpacemiT cross toolchain and QEMU (a100_support/env.sh:4-10,
a100c/runtime/build.py:89-110), neither of which is in this image, so there is
no ``oracle/_ref`` build.
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from pathlib import Path

HERE = Path(__file__).resolve().parent
LIB = HERE / "lib" / "libg950_oracle.so"
SRC = HERE / "cpu_baseline.c"


def build() -> Path:
    LIB.parent.mkdir(exist_ok=True)
    tmp = LIB.with_name(LIB.name + ".tmp")
    cmd = ["gcc", "-O3", "-march=x86-64-v3", "-fopenmp", "-fPIC", "-shared", "-o", str(tmp),
           str(SRC), "-lm"]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError("oracle build failed:\n" + proc.stdout + proc.stderr)
    os.replace(tmp, LIB)
    return LIB


def load():
    if not LIB.exists():
        build()
    lib = ctypes.CDLL(str(LIB))
    P = ctypes.c_void_p
    L = ctypes.c_long
    F = ctypes.c_float
    lib.g950o_threads.restype = ctypes.c_int
    lib.g950o_softmax_f32.argtypes = [P, P, L, L]
    lib.g950o_rmsnorm_f32.argtypes = [P, P, P, P, L, L, F]
    lib.g950o_softmax_bf16.argtypes = [P, P, L, L]
    lib.g950o_layernorm_bf16.argtypes = [P, P, P, P, P, P, L, L, F]
    lib.g950o_gemm_bf16.argtypes = [P, P, P, L, L, L, L]
    lib.g950o_gemm_bf16_wide.argtypes = [P, P, P, L, L, L, L]
    lib.g950o_widen_bf16.argtypes = [P, P, L]
    lib.g950o_gemm_i8.argtypes = [P, P, P, P, P, P, L, L, L, L]
    lib.g950o_attention_bf16.argtypes = [P, P, P, P, P, L, L, L, L, L, L, L, L, F, ctypes.c_int]
    return lib


if __name__ == "__main__":
    print(build())
