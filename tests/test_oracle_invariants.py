"""Pin every oracle function beyond the held fixtures: closed forms, invariants,
special cases and brute force on tiny inputs -- chosen so that a dropped term,
a wrong sign/index or a transposed operand fails one of them."""
import math

import numpy as np
import pytest

from oracle import reference as ref


# ------------------------------------------------------------------ bf16
def test_bf16_round_known_bits():
    cases = {
        0x3F800000: 0x3F80,  # 1.0 exact
        0x3F808000: 0x3F80,  # tie, even mantissa -> down
        0x3F818000: 0x3F82,  # tie, odd mantissa -> up
        0x3F808001: 0x3F81,  # above tie -> up
        0x7F7FFFFF: 0x7F80,  # max float rounds to inf
        0xFF800000: 0xFF80,  # -inf stays
        0x7F800001: 0x7FC0,  # signalling NaN gets the quiet bit
    }
    src = np.array(list(cases), dtype=np.uint32).view(np.float32)
    assert [int(b) for b in ref.bf16_bits(src)] == list(cases.values())


def test_bf16_round_matches_torch_rne():
    torch = pytest.importorskip("torch")
    x = np.random.default_rng(1).standard_normal(100000).astype(np.float32) * 1e3
    t = torch.from_numpy(x).to(torch.bfloat16).to(torch.float32).numpy()
    assert np.array_equal(ref.bf16_round(x), t)


# --------------------------------------------------------------- softmax
def test_softmax_constant_row_and_shift_invariance():
    x = np.full((3, 97), 2.5)
    assert np.allclose(ref.softmax(x), 1 / 97, rtol=0, atol=1e-15)
    rng = np.random.default_rng(2)
    y = rng.standard_normal((5, 33))
    assert np.allclose(ref.softmax(y), ref.softmax(y + 100.0), atol=1e-14)
    assert np.allclose(ref.softmax(y).sum(axis=1), 1.0, atol=1e-14)
    # brute force on one row
    row = y[0]
    bf = [math.exp(v) / sum(math.exp(u) for u in row) for v in row]
    assert np.allclose(ref.softmax(y)[0], bf, atol=1e-15)


# ------------------------------------------------------------- logsumexp
def test_logsumexp_closed_forms_and_library():
    # constant row c of n entries: c + ln n
    for c, n in ((2.5, 97), (-40.0, 16), (0.0, 1)):
        assert np.allclose(ref.logsumexp(np.full((2, n), c)), c + math.log(n), rtol=0, atol=1e-13)
    rng = np.random.default_rng(5)
    x = rng.standard_normal((6, 97)) * 3.0
    scipy_special = pytest.importorskip("scipy.special")
    assert np.allclose(ref.logsumexp(x), scipy_special.logsumexp(x, axis=-1), rtol=1e-14, atol=0)
    # the reference's own ref() form (ops/suite/perf/logsumexp.py:52-56)
    assert np.allclose(ref.logsumexp(x), np.logaddexp.reduce(x, axis=-1), rtol=1e-13, atol=0)
    # shift invariance and brute force on one row
    assert np.allclose(ref.logsumexp(x + 1000.0), ref.logsumexp(x) + 1000.0, rtol=1e-14)
    assert math.isclose(ref.logsumexp(x)[0], math.log(sum(math.exp(v) for v in x[0])), rel_tol=1e-13)
    # bounds: max <= lse <= max + ln n
    assert np.all(ref.logsumexp(x) >= x.max(axis=1))
    assert np.all(ref.logsumexp(x) <= x.max(axis=1) + math.log(97) + 1e-12)


def test_logsumexp_empty_row_is_minus_inf():
    assert np.all(ref.logsumexp(np.zeros((2, 0))) == -np.inf)


def test_logsumexp_special_values():
    x = np.zeros((5, 8))
    x[0, 3] = np.nan                       # NaN anywhere -> NaN
    x[1, 5] = np.inf                       # +inf entry -> +inf
    x[2, :] = -np.inf                      # all -inf -> -inf
    x[3, :4] = -np.inf                     # some -inf -> ln of the finite part
    x[4, 2] = np.nan
    x[4, 6] = np.inf                       # NaN wins over +inf
    y = ref.logsumexp(x)
    assert math.isnan(y[0]) and math.isnan(y[4])
    assert y[1] == np.inf and y[2] == -np.inf
    assert math.isclose(y[3], math.log(4), rel_tol=1e-15)
    # np.logaddexp.reduce (the reference's ref) agrees on every special row
    with np.errstate(invalid="ignore"):
        lib = np.logaddexp.reduce(x, axis=-1)
    assert np.array_equal(np.isnan(lib), np.isnan(y))
    assert np.array_equal(lib[~np.isnan(y)], y[~np.isnan(y)])


# ------------------------------------------------------------ dequantize
def test_dequantize_orientation_brute_force_and_exactness():
    rng = np.random.default_rng(6)
    k, n = 5, 7
    b = rng.integers(-128, 128, (k, n)).astype(np.int8)
    s = rng.random(n).astype(np.float32)
    y = ref.dequantize(b, s)
    # brute force; the scale belongs to the column (a per-row scale fails)
    for i in range(k):
        for j in range(n):
            assert y[i, j] == float(int(b[i, j])) * float(s[j])
    assert not np.allclose(y, np.asarray(b, np.float64) * np.asarray(s[:k], np.float64)[:, None])
    # unit scale is the widened int8; a power-of-two scale is exact scaling
    assert np.array_equal(ref.dequantize(b, np.ones(n)), b.astype(np.float64))
    assert np.array_equal(ref.dequantize(b, np.full(n, 0.125)), b.astype(np.float64) / 8)
    # int8 x bf16/fp16 products fit fp32 exactly: the kernel's fp32 product
    # rounds only once, at the output dtype
    for scale in (ref.bf16_round(s), s.astype(np.float16).astype(np.float32)):
        p = ref.dequantize(b, scale)
        assert np.array_equal(p.astype(np.float32).astype(np.float64), p)


# ---------------------------------------------------------------- norms
def test_rmsnorm_closed_forms():
    w = np.linspace(0.5, 1.5, 64)
    for c in (-3.0, 0.25, 7.0):
        y, r = ref.rms_layernorm(np.full((2, 64), c), w, 0.0)
        assert np.allclose(y, np.sign(c) * w[None, :], atol=1e-14)
        assert np.allclose(r, 1 / abs(c))
    rng = np.random.default_rng(3)
    x = rng.standard_normal((4, 67))
    w = rng.standard_normal(67)
    y, r = ref.rms_layernorm(x, w, 1e-5)
    for i in range(4):
        inv = 1.0 / math.sqrt(sum(v * v for v in x[i]) / 67 + 1e-5)
        assert math.isclose(r[i], inv, rel_tol=1e-14)
        assert np.allclose(y[i], [x[i, j] * inv * w[j] for j in range(67)], atol=1e-14)


def test_layernorm_moments_and_brute_force():
    rng = np.random.default_rng(4)
    x = rng.standard_normal((6, 300)) * 3 + 5
    y, mean, rstd = ref.layernorm(x, np.full(300, 2.0), np.full(300, -1.0), 0.0)
    assert np.allclose(y.mean(axis=1), -1.0, atol=1e-12)
    assert np.allclose(y.std(axis=1), 2.0, atol=1e-12)
    w, b = rng.standard_normal(300), rng.standard_normal(300)
    y, mean, rstd = ref.layernorm(x, w, b, 1e-5)
    for i in range(2):
        m = sum(x[i]) / 300
        var = sum((v - m) ** 2 for v in x[i]) / 300
        rs = 1 / math.sqrt(var + 1e-5)
        assert math.isclose(mean[i], m, rel_tol=1e-13) and math.isclose(rstd[i], rs, rel_tol=1e-12)
        assert np.allclose(y[i], [(x[i, j] - m) * rs * w[j] + b[j] for j in range(300)], atol=1e-12)


# ------------------------------------------------------------------ GEMM
def test_matmul_brute_force_and_orientation():
    rng = np.random.default_rng(5)
    a = rng.standard_normal((5, 7))
    b = rng.standard_normal((7, 3))
    bf = [[sum(a[i, k] * b[k, j] for k in range(7)) for j in range(3)] for i in range(5)]
    assert np.allclose(ref.matmul(a, b), bf, atol=1e-13)
    sq = rng.standard_normal((4, 4))
    assert not np.allclose(ref.matmul(a[:4, :4], sq), ref.matmul(a[:4, :4], sq.T))


def test_int8_exact_brute_force_and_bounds():
    rng = np.random.default_rng(6)
    a = rng.integers(-128, 128, (6, 40), dtype=np.int8)
    b = rng.integers(-128, 128, (40, 5), dtype=np.int8)
    bf = [[sum(int(a[i, k]) * int(b[k, j]) for k in range(40)) for j in range(5)] for i in range(6)]
    assert np.array_equal(ref.matmul_i8(a, b), np.array(bf, dtype=np.int64))
    # worst case of config 5 stays inside int32: K * 127^2
    assert 8192 * 127 * 127 < 2 ** 31
    ext = np.full((1, 8192), -127, np.int8)
    assert ref.matmul_i8(ext, np.full((8192, 1), -127, np.int8))[0, 0] == 8192 * 127 * 127


def test_dequant_closed_form():
    acc = np.array([[3, -4], [100000, 7]], dtype=np.int64)
    sa = np.array([0.5, 0.01], np.float32)
    sb = np.array([2.0, 0.02], np.float32)
    got = ref.dequant(acc, sa, sb)
    for i in range(2):
        for j in range(2):
            assert math.isclose(got[i, j], acc[i, j] * float(sa[i]) * float(sb[j]), rel_tol=1e-15)


# ------------------------------------------------------------- attention
def test_attention_special_cases():
    rng = np.random.default_rng(7)
    q = rng.standard_normal((1, 4, 9, 8))
    k = rng.standard_normal((1, 2, 9, 8))
    v = rng.standard_normal((1, 2, 9, 8))
    o, lse = ref.attention(q, k, v, 0.3, causal=True)
    # causal row 0 sees only key 0: O = V[0], lse = score
    for h in range(4):
        assert np.allclose(o[0, h, 0], v[0, h // 2, 0], atol=1e-14)
        assert math.isclose(lse[0, h, 0], 0.3 * float(q[0, h, 0] @ k[0, h // 2, 0]), rel_tol=1e-12)
    # uniform V -> O = V
    vu = np.broadcast_to(np.arange(8.0), (1, 2, 9, 8)).copy()
    o2, _ = ref.attention(q, k, vu, 0.3, causal=False)
    assert np.allclose(o2, np.arange(8.0), atol=1e-13)
    # equal scores -> lse = s + log(n)
    o3, lse3 = ref.attention(np.zeros((1, 1, 4, 8)), k[:, :1], v[:, :1], 1.0, causal=False)
    assert np.allclose(lse3, ref.lse_equal_scores(0.0, 9), atol=1e-14)
    # GQA map: head h uses kv head h // (Hq/Hkv); swapping kv heads must change heads 0-1 only
    o4, _ = ref.attention(q, k[:, ::-1], v[:, ::-1], 0.3, causal=True)
    assert np.allclose(o4[0, :2], ref.attention(q[:, :2], k[:, 1:], v[:, 1:], 0.3)[0][0])


def test_attention_brute_force():
    rng = np.random.default_rng(8)
    q = rng.standard_normal((1, 1, 5, 3))
    k = rng.standard_normal((1, 1, 5, 3))
    v = rng.standard_normal((1, 1, 5, 3))
    o, lse = ref.attention(q, k, v, 0.7, causal=True)
    for i in range(5):
        s = [0.7 * sum(q[0, 0, i, d] * k[0, 0, j, d] for d in range(3)) for j in range(i + 1)]
        mx = max(s)
        z = sum(math.exp(t - mx) for t in s)
        assert math.isclose(lse[0, 0, i], mx + math.log(z), rel_tol=1e-13)
        for d in range(3):
            od = sum(math.exp(s[j] - mx) / z * v[0, 0, j, d] for j in range(i + 1))
            assert math.isclose(o[0, 0, i, d], od, rel_tol=1e-12, abs_tol=1e-14)
