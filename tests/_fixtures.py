"""Helpers shared by the tests: golden bundle access and dtype decoding."""
from __future__ import annotations

import json
from pathlib import Path

import numpy as np

from compiler_amd import bundle as bundle_mod
from oracle.reference import bf16_from_bits

GOLDEN = Path(__file__).parent / "golden" / "bundles"
INDEX = json.loads((GOLDEN / "index.json").read_text())


def golden_cases(prefix: str):
    return sorted(name for name in INDEX if name.startswith(prefix))


def load(case: str):
    return bundle_mod.read(GOLDEN / case)


def dtype_of(case: str) -> str:
    for name in ("bfloat16", "float16", "float32"):
        if f"-{name}-" in case:
            return name
    raise ValueError(case)


def values(b, name) -> np.ndarray:
    """Decoded float values of one view (bf16 bits -> float32)."""
    v = b.view(name)
    arr = b.array(v)
    if v.dtype == bundle_mod.DTYPE_CODES["bfloat16"]:
        return bf16_from_bits(np.ascontiguousarray(arr))
    return np.ascontiguousarray(arr)
