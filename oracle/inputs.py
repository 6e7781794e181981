"""Seeded synthetic inputs for the five hot-path configurations -- TEST
INFRASTRUCTURE (shared by tests, smoke and bench so that every leg sees the
same data).

Every distribution choice the configurations leave open is fixed here:
  * ``N(0, s)`` with a bare number means standard deviation s (std 3 for the
    reduction inputs, std 0.1 for beta), as the reference scales its normals
    (ops/suite/perf/softmax.py:57 ``standard_normal * 3.0``).
  * GEMM operands ``N(0, 1/sqrt(K))`` are read as VARIANCE 1/sqrt(K) (std
    K**-0.25) so that C ~ N(0, 1); the std reading makes |C| ~ 0.01, below the
    bf16 absolute tolerance, which would make the parity test vacuous.
  * Seeds: configs 1 and 3 state theirs (0 and 1); configs 2, 4 and 5 state
    none and use 2, 4 and 5.
  * bf16 operands are produced by rounding float32 draws with the reference
    RNE rule (``oracle.reference.bf16_round``).
Generation uses ``numpy.random.default_rng`` (PCG64).
"""
from __future__ import annotations

import numpy as np

from .reference import bf16_round

SEEDS = {"c1": 0, "c2": 2, "c3": 1, "c4": 4, "c5": 5}


def config1(rows=4096, cols=4096, seed=SEEDS["c1"]):
    """x[rows, cols] ~ N(0,1) fp32, weight ~ U(0.5,1.5) fp32, eps 1e-6."""
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((rows, cols), dtype=np.float32)
    w = rng.uniform(0.5, 1.5, cols).astype(np.float32)
    return {"x": x, "w": w, "eps": 1e-6}


def config2(rows=8191, cols=3000, seed=SEEDS["c2"], outlier_frac=0.01):
    """x ~ N(0, std 3) with 1% of entries set to +-60, bf16-rounded; LayerNorm
    gamma ~ U(0.5,1.5), beta ~ N(0, std 0.1), eps 1e-5 (all bf16-rounded)."""
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((rows, cols), dtype=np.float32) * np.float32(3.0)
    n = rows * cols
    count = int(round(n * outlier_frac))
    if count:
        idx = rng.choice(n, size=count, replace=False)
        sign = np.where(rng.random(count) < 0.5, -60.0, 60.0).astype(np.float32)
        x.reshape(-1)[idx] = sign
    gamma = rng.uniform(0.5, 1.5, cols).astype(np.float32)
    beta = (rng.standard_normal(cols) * 0.1).astype(np.float32)
    return {"x": bf16_round(x), "gamma": bf16_round(gamma), "beta": bf16_round(beta),
            "eps": 1e-5}


def config3(m=8192, n=8192, k=8192, seed=SEEDS["c3"]):
    """A[m,k] row-major, B logical [k,n] stored column-major as Bt[n,k];
    entries ~ N(0, variance 1/sqrt(K)), bf16-rounded.  Returns float32 arrays
    holding bf16 values: ``a`` [m,k] and ``bt`` [n,k] (B = bt.T)."""
    rng = np.random.default_rng(seed)
    std = np.float32(k ** -0.25)
    a = rng.standard_normal((m, k), dtype=np.float32) * std
    bt = rng.standard_normal((n, k), dtype=np.float32) * std
    return {"a": bf16_round(a), "bt": bf16_round(bt)}


def config4(batch=4, hq=32, hkv=8, seq=4096, dim=128, seed=SEEDS["c4"]):
    """Q[batch,hq,seq,dim], K/V[batch,hkv,seq,dim] ~ N(0,1), bf16-rounded."""
    rng = np.random.default_rng(seed)
    q = rng.standard_normal((batch, hq, seq, dim), dtype=np.float32)
    k = rng.standard_normal((batch, hkv, seq, dim), dtype=np.float32)
    v = rng.standard_normal((batch, hkv, seq, dim), dtype=np.float32)
    return {"q": bf16_round(q), "k": bf16_round(k), "v": bf16_round(v),
            "scale": 1.0 / np.sqrt(dim)}


def config5(m=4096, n=8192, k=8192, seed=SEEDS["c5"]):
    """A int8[m,k], B int8 logical [k,n] stored K-contiguous as Bt[n,k],
    uniform integers in [-127,127]; sa[m], sb[n] ~ U(0.001, 0.02) fp32."""
    rng = np.random.default_rng(seed)
    a = rng.integers(-127, 128, size=(m, k), dtype=np.int8)
    bt = rng.integers(-127, 128, size=(n, k), dtype=np.int8)
    sa = rng.uniform(0.001, 0.02, m).astype(np.float32)
    sb = rng.uniform(0.001, 0.02, n).astype(np.float32)
    return {"a": a, "bt": bt, "sa": sa, "sb": sb}
