"""The OpenMP fp32 CPU path (oracle/cpu_baseline.c, the timed CPU baseline)
agrees with the float64 oracle on small seeded cases -- two independent CPU
restatements of the reference semantics checking each other."""
import numpy as np
import pytest

from oracle import build as obuild
from oracle import inputs
from oracle import reference as ref


@pytest.fixture(scope="module")
def lib():
    return obuild.load()


def p(a):
    return a.ctypes.data


def test_fp32_softmax_rms(lib):
    c = inputs.config1(64, 4096)
    y = np.empty_like(c["x"])
    lib.g950o_softmax_f32(p(c["x"]), p(y), 64, 4096)
    assert ref.max_rel_error(y, ref.softmax(c["x"])) <= 1e-5
    r = np.empty(64, np.float32)
    lib.g950o_rmsnorm_f32(p(c["x"]), p(c["w"]), p(y), p(r), 64, 4096, np.float32(1e-6))
    ey, er = ref.rms_layernorm(c["x"], c["w"], 1e-6)
    assert ref.max_rel_error(r, er) <= 1e-5
    assert ref.isclose_verdict(y, ey, 1e-5, 1e-6)[0]


def test_bf16_layernorm_softmax(lib):
    c = inputs.config2(32, 3000)
    x = ref.bf16_bits(c["x"])
    g, b = ref.bf16_bits(c["gamma"]), ref.bf16_bits(c["beta"])
    y = np.empty_like(x)
    mean, rstd = np.empty(32, np.float32), np.empty(32, np.float32)
    lib.g950o_layernorm_bf16(p(x), p(g), p(b), p(y), p(mean), p(rstd), 32, 3000, np.float32(1e-5))
    ey, em, es = ref.layernorm(c["x"], c["gamma"], c["beta"], 1e-5)
    assert ref.isclose_verdict(ref.bf16_from_bits(y), ey, 1e-2, 1e-2)[0]
    assert ref.max_rel_error(rstd, es) <= 1e-5
    s = np.empty_like(x)
    lib.g950o_softmax_bf16(p(x), p(s), 32, 3000)
    assert ref.isclose_verdict(ref.bf16_from_bits(s), ref.softmax(c["x"]), 1e-2, 1e-2)[0]


def test_gemm_bf16_and_int8(lib):
    c = inputs.config3(70, 50, 128)
    a, bt = ref.bf16_bits(c["a"]), ref.bf16_bits(c["bt"])
    y = np.empty((70, 50), np.uint16)
    lib.g950o_gemm_bf16(p(a), p(bt), p(y), 0, 70, 50, 128)
    assert ref.isclose_verdict(ref.bf16_from_bits(y), ref.matmul(c["a"], c["bt"].T), 2e-2, 2e-2)[0]
    c5 = inputs.config5(40, 30, 256)
    acc = np.empty((40, 30), np.int32)
    y8 = np.empty((40, 30), np.uint16)
    lib.g950o_gemm_i8(p(c5["a"]), p(c5["bt"]), p(c5["sa"]), p(c5["sb"]), p(acc), p(y8), 0, 40, 30, 256)
    exact = ref.matmul_i8(c5["a"], c5["bt"].T)
    assert np.array_equal(acc, exact)
    assert ref.isclose_verdict(ref.bf16_from_bits(y8), ref.dequant(exact, c5["sa"], c5["sb"]), 2e-2, 2e-2)[0]


def test_attention(lib):
    c = inputs.config4(1, 4, 2, 70, 64)
    q, k, v = (np.ascontiguousarray(ref.bf16_bits(c[n][0])) for n in ("q", "k", "v"))
    o = np.empty((4, 70, 64), np.uint16)
    lse = np.empty((4, 70), np.float32)
    lib.g950o_attention_bf16(p(q), p(k), p(v), p(o), p(lse), 4, 2, 70, 64, 0, 4, 0, 70,
                             np.float32(c["scale"]), 1)
    eo, el = ref.attention(c["q"], c["k"], c["v"], c["scale"], causal=True)
    assert ref.isclose_verdict(ref.bf16_from_bits(o), eo[0], 2e-2, 2e-2)[0]
    assert ref.isclose_verdict(lse, el[0], 1e-4, 1e-4)[0]
