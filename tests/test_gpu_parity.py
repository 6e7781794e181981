"""GPU parity: every hot-path kernel, called through the C ABI, against the CPU
oracle on the same seeded inputs and against the reference's held fixtures.

Bars (written per test): fp32 reductions <= 1e-5 relative; bf16 reductions
<= 1e-2; bf16 GEMM / attention <= 2e-2 absolute+relative (np.isclose form of
ops/harness/opslib/compare.py:107-140); int8 accumulators bit-exact.
"""
import functools

import numpy as np
import pytest

torch = pytest.importorskip("torch")

from compiler_amd import operators as ops  # noqa: E402
from compiler_amd import runtime as rt  # noqa: E402
from oracle import inputs  # noqa: E402
from oracle import reference as ref  # noqa: E402
from tests._fixtures import dtype_of, golden_cases, load, values  # noqa: E402

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
TD = {"float32": torch.float32, "bfloat16": torch.bfloat16, "float16": torch.float16}


def dev(a, dtype="float32"):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(DEV).to(TD[dtype])


def host(t):
    return t.float().cpu().numpy()


def rel_err(actual, expected, floor):
    a = np.asarray(actual, dtype=np.float64)
    b = np.asarray(expected, dtype=np.float64)
    return float((np.abs(a - b) / np.maximum(np.abs(b), floor)).max())


def close(actual, expected, rtol, atol):
    ok, err = ref.isclose_verdict(actual, expected, rtol, atol)
    assert ok, f"max abs err {err} exceeds rtol={rtol} atol={atol}"


def tile_rows(m, seed, tile=256):
    """Rows to check at full size: a random row in every 256-row output
    tile (so a fault confined to one tile row or one XCD's tiles shows), the
    tile edges, and the ragged last row."""
    rng = np.random.default_rng(seed)
    picks = [t + int(rng.integers(0, min(tile, m - t))) for t in range(0, m, tile)]
    return np.unique(np.r_[0, 1, min(255, m - 1), min(256, m - 1), m // 2, m - 2, m - 1, picks])


# ------------------------------------------------------------ reductions
@pytest.mark.parametrize("rows,cols", [(4096, 4096), (37, 97), (5, 1), (3, 70001)])
def test_softmax_rmsnorm_fp32(rows, cols):
    """Config 1 (and ragged / long-row cases): fp32 <= 1e-5 relative."""
    c = inputs.config1(rows, cols)
    x = dev(c["x"])
    y = ops.softmax(x, sync=True)
    expect = ref.softmax(c["x"])
    assert rel_err(host(y), expect, 1e-30) <= 1e-5
    assert np.allclose(host(y).sum(axis=1), 1.0, atol=1e-5)
    yr, r = ops.rmsnorm(x, dev(c["w"]), c["eps"], sync=True)
    ey, er = ref.rms_layernorm(c["x"], c["w"], c["eps"])
    assert rel_err(host(yr), ey, 1e-6) <= 1e-5
    assert rel_err(host(r), er, 1e-30) <= 1e-5


@pytest.mark.parametrize("rows,cols", [(8191, 3000), (64, 3001), (7, 67)])
def test_layernorm_softmax_bf16_masked_tail(rows, cols):
    """Config 2: bf16 in/out, fp32 statistics, +-60 outliers; <= 1e-2."""
    c = inputs.config2(rows, cols)
    x = dev(c["x"], "bfloat16")
    y, mean, rstd = ops.layernorm(x, dev(c["gamma"], "bfloat16"), dev(c["beta"], "bfloat16"),
                                  c["eps"], sync=True)
    ey, em, es = ref.layernorm(c["x"], c["gamma"], c["beta"], c["eps"])
    close(host(y), ey, 1e-2, 1e-2)
    # fp32 statistics: rstd to 1e-5 relative; the mean of +-60-outlier rows
    # cancels to ~0.05, so it is held to 1e-5 relative or 1e-6 absolute
    # (2e-8 of the rows' mean |x|)
    close(host(mean), em, 1e-5, 1e-6)
    assert rel_err(host(rstd), es, 1e-30) <= 1e-5
    s = ops.softmax(x, sync=True)
    close(host(s), ref.softmax(c["x"]), 1e-2, 1e-2)
    assert np.allclose(host(s).sum(axis=1), 1.0, atol=2e-2)


@pytest.mark.parametrize("dt", ["float32", "bfloat16", "float16"])
@pytest.mark.parametrize("rows,cols", [(4099, 64), (4096, 1000), (4097, 2048), (4100, 3000), (4096, 4096)])
def test_layernorm_parameters_in_lds(rows, cols, dt):
    """Many rows of at most 512 vectors: the LDS-parameter kernels
    (g950_rw_*, every row width class 1..8 vectors per lane) for both
    LayerNorm forms, against the float64 oracle (fp32 <= 1e-5 relative,
    16-bit <= 1e-2); the rows past the last full 8-row workgroup included."""
    c = inputs.config2(rows, cols)
    x = dev(c["x"], dt)
    g, b = dev(c["gamma"], dt), dev(c["beta"], dt)
    xr, gr, br = host(x), host(g), host(b)
    y, mean, rstd = ops.layernorm(x, g, b, c["eps"], sync=True)
    vec = 4 if dt == "float32" else 8
    if (cols // vec) <= 512 and cols % vec == 0:
        assert rt.module().last_kernel.startswith("g950_rw_layernorm_")
    ey, em, es = ref.layernorm(xr, gr, br, c["eps"])
    bar = 1e-5 if dt == "float32" else 1e-2
    close(host(y), ey, bar, bar)
    close(host(mean), em, 1e-5, 1e-6)
    assert rel_err(host(rstd), es, 1e-30) <= 1e-5
    yl = torch.empty_like(x)
    ml = torch.empty(rows, device=DEV)
    sl = torch.empty(rows, device=DEV)
    ops.layer_norm_forward_row(yl, cols, x, cols, g, b, ml, 1, sl, 1, rows, cols, c["eps"], sync=True)
    ey, em, es = ref.layernorm_row(xr, gr, br, c["eps"])
    close(host(yl), ey, bar, bar)
    close(host(ml), em, 1e-5, 1e-6)
    assert rel_err(host(sl), es, 1e-30) <= 1e-5


@pytest.mark.parametrize("dt", ["float32", "bfloat16", "float16"])
@pytest.mark.parametrize("rows,cols,pad", [(8191, 3001, 0), (37, 97, 0), (5, 1, 0), (7, 67, 5), (1000, 1001, 3),
                                           (64, 4089, 0), (33, 1023, 1), (300, 2047, 9)])
def test_masked_row_vectors(rows, cols, pad, dt):
    """Rows that are not whole 16-byte vectors or start off a 16-byte boundary
    (row stride cols + pad): the masked aligned-vector kernels for all five row
    ops, against float64 (fp32 <= 1e-5 relative, 16-bit <= 1e-2); y shares x's
    row stride, and the gap elements between y's rows (sentinels) stay
    untouched by the edge vectors' stores."""
    c = inputs.config2(rows, cols + pad)
    stride = cols + pad
    xd = dev(c["x"], dt)[:, :cols]
    xr = host(xd)
    g, b = dev(c["gamma"][:cols], dt), dev(c["beta"][:cols], dt)
    gr, br = host(g), host(b)
    vec = 4 if dt == "float32" else 8
    masked = (cols % vec != 0 or stride % vec != 0) and cols + vec - 1 <= 8 * 64 * vec

    def out():
        return torch.full((rows, stride), -7.0, dtype=TD[dt], device=DEV)[:, :cols]

    def gaps_intact(y):
        if pad:
            full = torch.as_strided(y, (rows, stride), (stride, 1))
            assert bool((full[:, cols:] == -7.0).all())

    bar = (1e-5, 1e-6) if dt == "float32" else (1e-2, 1e-2)
    y = out()
    ops.softmax_kernel(xd, y, cols, sync=True)
    if masked:
        assert rt.module().last_kernel.startswith("g950_rm_softmax_")
    close(host(y), ref.softmax(xr), *bar)
    gaps_intact(y)
    lse = torch.empty(rows, device=DEV)
    ops.logsumexp_kernel(xd, lse, cols, sync=True)
    close(host(lse), ref.logsumexp(xr), 3e-5, 3e-6)
    y, r = out(), torch.empty(rows, device=DEV)
    ops.rms_layernorm_forward_kernel(y, stride, xd, stride, g, 1, r, 1, cols, 1e-6, sync=True)
    ey, er = ref.rms_layernorm(xr, gr, 1e-6)
    close(host(y), ey, *bar)
    close(host(r), er, 1e-5, 1e-6)
    gaps_intact(y)
    y, mean, rstd = ops.layernorm(xd, g, b, 1e-5, out=out(), sync=True)
    ey, em, es = ref.layernorm(xr, gr, br, 1e-5)
    close(host(y), ey, *(bar if dt != "float32" else (1e-5, 1e-5)))
    close(host(mean), em, 1e-5, 1e-6)
    assert rel_err(host(rstd), es, 1e-30) <= 1e-5
    gaps_intact(y)
    # the row form takes flat buffers addressed by its row-stride scalars
    yfull = torch.full((rows, stride), -7.0, dtype=TD[dt], device=DEV)
    y = yfull[:, :cols]
    ml, sl = torch.empty(rows, device=DEV), torch.empty(rows, device=DEV)
    ops.layer_norm_forward_row(yfull, stride, dev(c["x"], dt), stride, g, b, ml, 1, sl, 1, rows, cols, 1e-5,
                               sync=True)
    ey, em, es = ref.layernorm_row(xr, gr, br, 1e-5)
    close(host(y), ey, *(bar if dt != "float32" else (1e-5, 1e-5)))
    close(host(ml), em, 1e-5, 1e-6)
    gaps_intact(y)


def test_row_reductions_random_shapes_sweep():
    """Thirty-six seeded shapes through the row dispatcher of every row op:
    row lengths log-uniform over 1..200000 (one-wave rows, whole-workgroup
    rows, the split-row pair), up to ~3M elements, the three dtypes in turn,
    and four layouts in turn: whole 16-byte vectors (length a multiple of
    8) packed or with an aligned gap of 8..32 elements between rows, any
    length packed, any length with a gap of 1..9 (rows off a 16-byte
    boundary: the masked kernels); softmax, logsumexp, RMSNorm and LayerNorm
    against float64 at the dtype's bar, the gap elements untouched, and
    every kernel family of the dispatcher reached."""
    rng = np.random.default_rng(4242)
    ran = set()
    for case in range(36):
        dt = ("float32", "bfloat16", "float16")[case % 3]
        layout = case % 4
        cols = int(np.exp(rng.uniform(0, np.log(200000))))
        if layout < 2:
            cols = max(8, cols // 8 * 8)
        rows = int(rng.integers(1, max(2, min(9000, 3_000_000 // cols)) + 1))
        pad = (0, 8 * int(rng.integers(1, 5)), 0, int(rng.integers(1, 10)))[layout]
        stride = cols + pad
        tag = f"case {case}: {dt} rows {rows} cols {cols} stride {stride}"
        c = inputs.config2(rows, stride, seed=100 + case)
        xd = dev(c["x"], dt)[:, :cols]
        xr = host(xd)
        g, b = dev(c["gamma"][:cols], dt), dev(c["beta"][:cols], dt)
        gr, br = host(g), host(b)
        bar = (1e-5, 1e-6) if dt == "float32" else (1e-2, 1e-2)

        def out():
            return torch.full((rows, stride), -7.0, dtype=TD[dt], device=DEV)[:, :cols]

        def checked(what, actual, expected, rtol, atol, y=None):
            ran.add(rt.module().last_kernel)
            ok, err = ref.isclose_verdict(actual, expected, rtol, atol)
            assert ok, f"{tag}: {what} ({rt.module().last_kernel}) max abs err {err}"
            if y is not None and pad:
                full = torch.as_strided(y, (rows, stride), (stride, 1))
                assert bool((full[:, cols:] == -7.0).all()), f"{tag}: {what} wrote between rows"

        y = out()
        ops.softmax_kernel(xd, y, cols, sync=True)
        checked("softmax", host(y), ref.softmax(xr), *bar, y=y)
        lse = torch.empty(rows, device=DEV)
        ops.logsumexp_kernel(xd, lse, cols, sync=True)
        checked("logsumexp", host(lse), ref.logsumexp(xr), 3e-5, 3e-6)
        y, r = out(), torch.empty(rows, device=DEV)
        ops.rms_layernorm_forward_kernel(y, stride, xd, stride, g, 1, r, 1, cols, 1e-6, sync=True)
        ey, er = ref.rms_layernorm(xr, gr, 1e-6)
        checked("rmsnorm", host(y), ey, *bar, y=y)
        checked("rmsnorm r", host(r), er, 1e-5, 1e-6)
        y, mean, rstd = ops.layernorm(xd, g, b, 1e-5, out=out(), sync=True)
        ey, em, es = ref.layernorm(xr, gr, br, 1e-5)
        checked("layernorm", host(y), ey, *(bar if dt != "float32" else (1e-5, 1e-5)), y=y)
        checked("layernorm mean", host(mean), em, 1e-5, 1e-6)
        assert rel_err(host(rstd), es, 1e-30) <= 1e-5, f"{tag}: layernorm rstd"
    for family in ("g950_rr_", "g950_rw_", "g950_rm_", "g950_rs_final_"):
        assert any(k.startswith(family) for k in ran), (family, sorted(ran))
    assert any(k.startswith("g950_rs_final_") and not k.endswith("_v1") for k in ran), sorted(ran)
    assert any(k.startswith("g950_rr_") and k.endswith("_b256") for k in ran), sorted(ran)


@pytest.mark.parametrize("dt", ["float32", "bfloat16", "float16"])
@pytest.mark.parametrize("rows,cols", [(4, 16), (4, 97), (64, 1024), (8191, 3000), (2, 100000)])
def test_logsumexp(rows, cols, dt):
    """ops/suite/perf/logsumexp.py: x ~ 3 N(0,1), expected from the inputs as
    the kernel sees them (rounded to dt); y in float32 to the reference's own
    bar (rtol 3e-5, atol 3e-6, :66), y in dt to the dtype's shared bar."""
    rng = np.random.default_rng(rows * 7 + cols)
    x = (rng.standard_normal((rows, cols)) * 3.0).astype(np.float32)
    xd = dev(x, dt)
    xr = host(xd)
    expect = ref.logsumexp(xr)
    y = ops.logsumexp(xd, sync=True)
    name = rt.module().last_kernel
    assert "logsumexp" in name
    assert name.startswith("g950_rs_final_") == (cols == 100000)
    close(host(y), expect, 3e-5, 3e-6)
    yd = torch.zeros(rows, dtype=TD[dt], device=DEV)
    ops.logsumexp_kernel(xd, yd, cols, sync=True)
    rtol, atol = ref.TOLERANCES[dt]
    close(host(yd), expect, rtol, atol)


def test_logsumexp_empty_rows():
    """n_cols = 0: the kernel's max stays -inf, which is the result
    (logsumexp.py:23-38: maximum = -inf, an infinite maximum is returned)."""
    x = torch.empty((3, 0), dtype=torch.float32, device=DEV)
    y = host(ops.logsumexp(x, sync=True))
    assert np.all(y == -np.inf)


@pytest.mark.parametrize("cols", [97, 3000, 100000])
def test_logsumexp_special_rows(cols):
    """NaN anywhere -> NaN (also beside +inf), +inf -> +inf, all -inf -> -inf,
    partial -inf -> lse of the finite part; a huge-magnitude row stays finite."""
    rng = np.random.default_rng(cols)
    x = rng.standard_normal((7, cols)).astype(np.float32)
    x[0, cols // 2] = np.nan
    x[1, cols - 1] = np.inf
    x[2, :] = -np.inf
    x[3, : cols // 3] = -np.inf
    x[4, 0] = np.nan
    x[4, cols - 1] = np.inf
    x[5, :] = 3.0e38
    x[6, :] = -3.0e38
    y = host(ops.logsumexp(dev(x), sync=True))
    e = ref.logsumexp(x)
    assert np.array_equal(np.isnan(y), np.isnan(e)) and np.isnan(y[[0, 4]]).all()
    assert y[1] == np.inf and y[2] == -np.inf
    fin = np.isfinite(e)
    assert np.isfinite(y[fin]).all()
    close(y[fin], e[fin], 3e-5, 3e-6)


@pytest.mark.parametrize("dt", ["float32", "bfloat16"])
@pytest.mark.parametrize("cols", [97, 3000, 4096])
def test_softmax_special_rows(dt, cols):
    """Rows with huge maxima (|max| >= 2^24: the exponent takes its
    two-rounding form), a row just below that bound (the fma form, whose
    rounded max*log2(e) shifts the whole row's exponents alike), an +inf
    entry (NaN row), an all -inf row (NaN, 0/0), a partly -inf row, and a
    huge row with three tied maxima beside ordinary values (1/3 at the
    maxima, 0 elsewhere)."""
    rng = np.random.default_rng(cols + 1)
    x = rng.standard_normal((8, cols)).astype(np.float32)
    x[0, :] = 3.0e38
    x[1, :] = -3.0e38
    x[2, cols // 2] = np.inf
    x[3, :] = -np.inf
    x[4, : cols // 3] = -np.inf
    x[5, [0, cols // 2, cols - 1]] = 2.5e38
    x[6, :] = 1.5e38 + 0.0 * x[6, :]
    x[7, :] = 1.6e7 + 4.0 * x[7, :]
    if dt == "bfloat16":
        x = ref.bf16_round(x)
    y = host(ops.softmax(dev(x, dt), sync=True)).astype(np.float64)
    e = ref.softmax(x)
    assert np.array_equal(np.isnan(y), np.isnan(e))
    assert np.isnan(y[[2, 3]]).all()
    fin = ~np.isnan(e)
    close(y[fin], e[fin], *((1e-5, 1e-6) if dt == "float32" else (1e-2, 1e-2)))


@pytest.mark.parametrize("dt", ["float32", "bfloat16"])
def test_split_rows_softmax_special_rows(dt):
    """The rows of test_softmax_special_rows at 70000 columns, which take the
    two-launch split (1024-vector chunks merged per row): whole chunks of
    -inf (rows 3 and 4), maxima in three different chunks (row 5), the +inf
    entry in a middle chunk (row 2), and huge rows whose chunk sums merge
    with unit rescale factors."""
    cols = 70000
    rng = np.random.default_rng(cols + 1)
    x = rng.standard_normal((8, cols)).astype(np.float32)
    x[0, :] = 3.0e38
    x[1, :] = -3.0e38
    x[2, cols // 2] = np.inf
    x[3, :] = -np.inf
    x[4, : cols // 3] = -np.inf
    x[5, [0, cols // 2, cols - 1]] = 2.5e38
    x[6, :] = 1.5e38 + 0.0 * x[6, :]
    x[7, :] = 1.6e7 + 4.0 * x[7, :]
    if dt == "bfloat16":
        x = ref.bf16_round(x)
    y = host(ops.softmax(dev(x, dt), sync=True)).astype(np.float64)
    assert rt.module().last_kernel.startswith("g950_rs_final_softmax_")
    e = ref.softmax(x)
    assert np.array_equal(np.isnan(y), np.isnan(e))
    assert np.isnan(y[[2, 3]]).all()
    fin = ~np.isnan(e)
    close(y[fin], e[fin], *((1e-5, 1e-6) if dt == "float32" else (1e-2, 1e-2)))


def test_dequantize_random_sweep():
    """Twelve seeded dequantize shapes, K in 1..3000 and N in 1..3000 (half
    of them N a multiple of 8: the vector kernels; the rest any N: the
    general kernel), the three output dtypes in turn; every element
    bit-exact against the float64 product rounded once."""
    rng = np.random.default_rng(4711)
    for case in range(12):
        dt = ("float32", "bfloat16", "float16")[case % 3]
        k, n = (int(v) for v in rng.integers(1, 3001, 2))
        if case % 2 == 0:
            n = max(8, n // 8 * 8)
        b = rng.integers(-127, 128, (k, n)).astype(np.int8)
        sd = dev(rng.random(n).astype(np.float32), dt)
        y = ops.dequantize(torch.from_numpy(b).to(DEV), sd, sync=True)
        assert np.array_equal(host(y), _dq_expect(b, host(sd), dt)), \
            f"case {case}: {dt} k {k} n {n} ({rt.module().last_kernel})"


def _dq_expect(b, s, dt):
    p = ref.dequantize(b, s)
    if dt == "bfloat16":
        return ref.bf16_round(p.astype(np.float32))
    if dt == "float16":
        return p.astype(np.float16).astype(np.float32)
    return p.astype(np.float32)


@pytest.mark.parametrize("dt", ["float32", "bfloat16", "float16"])
@pytest.mark.parametrize("k,n", [(32, 32), (33, 33), (256, 32), (5, 48), (8192, 8192)])
def test_dequantize_bit_exact(k, n, dt):
    """ops/suite/perf/dequantize_matmul.py: b ~ U{-127..127}, scale ~ U[0,1)
    in dt (make_case :57-60); bit-exact against the float64 product rounded
    once to dt."""
    rng = np.random.default_rng(k * 31 + n)
    b = rng.integers(-127, 128, (k, n)).astype(np.int8)
    sd = dev(rng.random(n).astype(np.float32), dt)
    y = ops.dequantize(torch.from_numpy(b).to(DEV), sd, sync=True)
    vec = n % (4 if dt == "float32" else 8) == 0
    assert rt.module().last_kernel == ("g950_dequant_i8_" + {"float32": "f32", "bfloat16": "bf16",
                                                            "float16": "f16"}[dt] if vec
                                       else "g950_dequant_i8_general")
    assert np.array_equal(host(y), _dq_expect(b, host(sd), dt))


def test_dequantize_strided_views_and_guard():
    """Column-major b (general kernel) and an output with padded rows: the
    pad stays untouched, the values stay exact."""
    rng = np.random.default_rng(44)
    k, n = 64, 96
    b = rng.integers(-128, 128, (k, n)).astype(np.int8)
    bt = torch.from_numpy(np.ascontiguousarray(b.T)).to(DEV).t()  # strides (1, k)
    s = dev(rng.random(n).astype(np.float32), "bfloat16")
    buf = torch.full((k, n + 16), 5.0, dtype=torch.bfloat16, device=DEV)
    y = buf[:, :n]
    ops.dequantize(bt, s, out=y, sync=True)
    assert rt.module().last_kernel == "g950_dequant_i8_general"
    assert np.array_equal(host(y), _dq_expect(b, host(s), "bfloat16"))
    bc = torch.from_numpy(b).to(DEV)
    ops.dequantize(bc, s, out=y, sync=True)
    assert rt.module().last_kernel == "g950_dequant_i8_bf16"
    assert np.array_equal(host(y), _dq_expect(b, host(s), "bfloat16"))
    assert torch.all(buf[:, n:] == 5.0)


SPLIT_SHAPES = [(1, 1 << 20), (3, 70001), (2, 100000), (4, 16384)]


@pytest.mark.parametrize("dt", ["float32", "bfloat16", "float16"])
@pytest.mark.parametrize("rows,cols", SPLIT_SHAPES)
def test_split_rows_all_reductions(rows, cols, dt):
    """Few, long rows take the two-phase split (partials + merge); every
    reduction against the oracle on the dtype-rounded inputs.  Bars: fp32
    outputs <= 1e-5 relative (softmax, RMSNorm), LayerNorm <= 1e-4 absolute
    on unit-scale outputs; 16-bit outputs the dtype's shared bar; statistics
    (r, Mean, Rstd, logsumexp) in fp32 <= 1e-5 relative (Mean: or 1e-6
    absolute).  x has +40 outliers every 97 columns (the centered variance
    and the chunk moments merge must hold them)."""
    rng = np.random.default_rng(rows * 1000 + cols % 997)
    x = (rng.standard_normal((rows, cols)) * 2.0).astype(np.float32)
    x[:, ::97] += 40.0
    w = (rng.standard_normal(cols) * 0.5 + 1.0).astype(np.float32)
    b = (rng.standard_normal(cols) * 0.1).astype(np.float32)
    xd, wd, bd = dev(x, dt), dev(w, dt), dev(b, dt)
    xr, wr, br = host(xd), host(wd), host(bd)
    rtol, atol = ref.TOLERANCES[dt]

    y = ops.softmax(xd, sync=True)
    assert rt.module().last_kernel.startswith("g950_rs_final_softmax_")
    if dt == "float32":
        assert rel_err(host(y), ref.softmax(xr), 1e-30) <= 1e-5
    else:
        close(host(y), ref.softmax(xr), rtol, atol)
    assert np.allclose(host(y).astype(np.float64).sum(axis=1), 1.0, atol=1e-3 if dt != "float32" else 1e-5)

    lse = ops.logsumexp(xd, sync=True)
    assert rt.module().last_kernel.startswith("g950_rs_final_logsumexp_")
    close(host(lse), ref.logsumexp(xr), 3e-5, 3e-6)

    yr, r = ops.rmsnorm(xd, wd, 1e-5, sync=True)
    assert rt.module().last_kernel.startswith("g950_rs_final_rmsnorm_")
    ey, er = ref.rms_layernorm(xr, wr, 1e-5)
    if dt == "float32":
        assert rel_err(host(yr), ey, 1e-6) <= 1e-5
    else:
        close(host(yr), ey, rtol, atol)
    assert rel_err(host(r), er, 1e-30) <= 1e-5

    yl, mean, rstd = ops.layernorm(xd, wd, bd, 1e-5, sync=True)
    assert rt.module().last_kernel.startswith("g950_rs_final_layernorm_")
    ey, em, es = ref.layernorm(xr, wr, br, 1e-5)
    if dt == "float32":
        close(host(yl), ey, 0.0, 1e-4)
    else:
        close(host(yl), ey, rtol, atol)
    close(host(mean), em, 1e-5, 1e-6)
    assert rel_err(host(rstd), es, 1e-30) <= 1e-5


@pytest.mark.parametrize("rows,cols,kernel", [(64, 3000, "g950_r"), (4, 100000, "g950_rs_final_layernorm_")])
def test_layernorm_large_mean_rows(rows, cols, kernel):
    """fp32 rows of mean 1000 and unit spread, in the one-pass register
    kernels and the split path (chunk moments merged per row): the centered
    variance holds (a one-pass E[x^2] - E[x]^2 form misses by 10-100% here),
    and the split's merge keeps Mean and Rstd.  Bar 1e-2 on Y: fp32 sums of
    values near 1000 move the mean by ~1e-3 of the spread."""
    rng = np.random.default_rng(rows + cols)
    x = (1000.0 + rng.standard_normal((rows, cols))).astype(np.float32)
    w = (rng.standard_normal(cols) * 0.5 + 1.0).astype(np.float32)
    b = (rng.standard_normal(cols) * 0.1).astype(np.float32)
    y, mean, rstd = ops.layernorm(dev(x), dev(w), dev(b), 1e-5, sync=True)
    assert rt.module().last_kernel.startswith(kernel)
    ey, em, es = ref.layernorm(x, w, b, 1e-5)
    close(host(y), ey, 1e-2, 1e-2)
    close(host(mean), em, 1e-5, 1e-6)
    close(host(rstd), es, 1e-2, 0.0)


def test_split_rows_guard_and_special_values():
    """Split path: outputs stay inside padded rows; logsumexp keeps the NaN /
    +inf / all -inf rules across chunks (the special value in a later chunk)."""
    rows, cols, pad = 5, 100000, 8
    rng = np.random.default_rng(9)
    x = rng.standard_normal((rows, cols)).astype(np.float32)
    x[0, 77777] = np.nan
    x[1, 99999] = np.inf
    x[2, :] = -np.inf
    x[3, :50000] = -np.inf
    xd = dev(x, "bfloat16")
    buf = torch.full((rows, cols + pad), 7.0, dtype=torch.bfloat16, device=DEV)
    ops.softmax_kernel(dev(np.nan_to_num(x, nan=0.0, posinf=0.0, neginf=0.0), "bfloat16"), buf[:, :cols], cols,
                       sync=True)
    assert rt.module().last_kernel == "g950_rs_final_softmax_bf16_v8"
    assert torch.all(buf[:, cols:] == 7.0)
    y = host(ops.logsumexp(xd, sync=True))
    e = ref.logsumexp(host(xd))
    assert np.isnan(y[0]) and y[1] == np.inf and y[2] == -np.inf
    close(y[3:], e[3:], 3e-5, 3e-6)


def test_reduction_tail_guard_untouched():
    """Outputs are written only inside the view: a poisoned guard behind each
    row stays intact (the masked-tail witness idea of tools/check_masked_tails.py)."""
    rows, cols, pad = 9, 3000, 8
    c = inputs.config2(rows, cols)
    x = dev(c["x"], "bfloat16")
    buf = torch.full((rows, cols + pad), 7.0, dtype=torch.bfloat16, device=DEV)
    y = buf[:, :cols]
    ops.softmax_kernel(x, y, cols, sync=True)
    assert torch.all(buf[:, cols:] == 7.0)
    close(host(y), ref.softmax(c["x"]), 1e-2, 1e-2)


def test_stream_copy_exact():
    x = torch.randn(8191 * 3000, device=DEV).to(torch.bfloat16)
    y = torch.empty_like(x)
    ops.stream_copy(x, y, sync=True)
    assert rt.module().last_kernel == "g950_stream_copy"
    assert torch.equal(x, y)


@pytest.mark.parametrize("case", golden_cases("softmax"))
def test_softmax_reference_fixture(case):
    b = load(case)
    dt = dtype_of(case)
    x = values(b, "x_ptr")
    y = torch.zeros(x.shape, dtype=TD[dt], device=DEV)
    ops.softmax_kernel(dev(x, dt), y, int(b.scalar("n_cols")), sync=True)
    rtol, atol = ref.TOLERANCES[dt]
    close(host(y), values(b, "y_ptr"), rtol, atol)


def test_rms_fixture_shapes_all_dtypes():
    """The reference case shapes of fast_rms_layernorm (:48) in 3 dtypes."""
    for dt in ("float32", "bfloat16", "float16"):
        for rows, cols in ((4, 64), (7, 67)):
            rng = np.random.default_rng(30)
            x = (rng.standard_normal((rows, cols)) * 0.5).astype(np.float32)
            w = (rng.standard_normal(cols) * 0.5 + 1.0).astype(np.float32)
            if dt == "bfloat16":
                x, w = ref.bf16_round(x), ref.bf16_round(w)
            elif dt == "float16":
                x, w = x.astype(np.float16).astype(np.float32), w.astype(np.float16).astype(np.float32)
            yr, r = ops.rmsnorm(dev(x, dt), dev(w, dt), 1e-5, sync=True)
            ey, er = ref.rms_layernorm(x, w, 1e-5)
            rtol, atol = ref.TOLERANCES[dt]
            close(host(yr), ey, rtol, atol)
            close(host(r), er, 1e-5, 1e-6)


# ------------------------------------------------------------------ GEMM
@pytest.mark.parametrize("m,n,k", [(256, 256, 64), (300, 260, 256), (513, 1000, 1024), (1, 7, 64),
                                   (33, 65, 64), (257, 129, 192)])
def test_gemm_bf16_mfma(m, n, k):
    c = inputs.config3(m, n, k)
    y = ops.matmul(dev(c["a"], "bfloat16"), dev(c["bt"], "bfloat16").t(), sync=True)
    assert rt.module().last_kernel == "g950_gemm_bf16_256x256"
    close(host(y), ref.matmul(c["a"], c["bt"].T), 2e-2, 2e-2)


@pytest.mark.parametrize("m,n,k", [(8192, 8192, 8192), (4097, 11008, 4096)])
def test_gemm_bf16_config3_sampled(m, n, k):
    """Config 3 at full size: sampled rows (incl. the ragged last row) and all
    columns checked against float64."""
    c = inputs.config3(m, n, k)
    a = dev(c["a"], "bfloat16")
    y = ops.matmul(a, dev(c["bt"], "bfloat16").t(), sync=True)
    rows = tile_rows(m, 9)
    got = host(y[torch.from_numpy(rows).to(DEV)])
    close(got, ref.matmul(c["a"][rows], c["bt"].T), 2e-2, 2e-2)


@pytest.mark.parametrize("dt", ["bfloat16", "float16"])
@pytest.mark.parametrize("m,n,k", [(32, 32, 32), (33, 33, 48), (256, 256, 128), (300, 260, 192), (16, 4096, 4096),
                                   (1, 1000, 4096), (2048, 2048, 4096), (7, 70, 208), (16, 8192, 8192),
                                   (5, 130, 1040), (1, 8192, 8192), (16, 11008, 4096), (16, 8192, 8000),
                                   (64, 4096, 4096), (4096, 4096, 256), (4100, 4096, 320),
                                   (1100, 8192, 128), (1024, 8192, 128), (17, 8192, 8192), (48, 4096, 1040),
                                   (65, 4096, 4096)])
def test_dequant_matmul_fused(m, n, k, dt):
    """dequantize_matmul fused into the GEMM: a [M,K] in dt, b int8 ~ U{-127..127}
    (K-contiguous), scale ~ U[0,1) / 64 in dt.  Bar 2e-2 (the bf16 GEMM bar,
    np.isclose form) against float64 a . (b * scale) on the rounded inputs; rows
    sampled at the largest shape."""
    rng = np.random.default_rng(m + 7 * n + k)
    a = rng.standard_normal((m, k)).astype(np.float32) * 0.5
    b = rng.integers(-127, 128, (k, n)).astype(np.int8)
    s = (rng.random(n) / 64).astype(np.float32)
    ad, sd = dev(a, dt), dev(s, dt)
    bt = torch.from_numpy(np.ascontiguousarray(b.T)).to(DEV)
    y = ops.dequant_matmul(ad, bt.t(), sd, sync=True)
    short = "bf16" if dt == "bfloat16" else "f16"
    # more 256x256 tiles than half the CUs: B is widened once and the bf16/f16 GEMM runs
    widened = k % 64 == 0 and 2 * -(-m // 256) * -(-n // 256) > 256
    blocks32 = -(-n // 32)
    c16 = m == 1 or blocks32 < 256 or 4 * blocks32 > 5 * 256  # 16 columns per workgroup (256 CUs)
    want = ("g950_gemm_general" if k % 16 else
            f"g950_gemm_w8a16_skinny_c16_{short}" if m <= 16 and c16 else
            f"g950_gemm_w8a16_skinny_{short}" if m <= 16 else
            f"g950_gemm_w8a16_skinny32_{short}" if m <= 32 else
            f"g950_gemm_w8a16_skinny64_{short}" if m <= 64 else
            f"g950_gemm_{short}_256x256" if widened else f"g950_gemm_w8a16_{short}_128x128")
    assert rt.module().last_kernel == want
    rows = np.arange(m) if m <= 512 else np.unique(np.r_[0, 127, 128, m - 1,
                                                        np.random.default_rng(5).integers(0, m, 24)])
    expect = ref.matmul(host(ad)[rows], ref.dequantize(b, host(sd)))
    close(host(y)[rows], expect, 2e-2, 2e-2)
    # no kernel keeps state between calls: a second call reproduces the
    # first bit for bit
    y2 = ops.dequant_matmul(ad, bt.t(), sd, sync=True)
    assert torch.equal(y, y2)


@pytest.mark.parametrize("dt", ["bfloat16", "float16"])
@pytest.mark.parametrize("m,n,k", [(2048, 4096, 4096), (300, 512, 256), (100, 272, 96), (16, 4096, 4096),
                                   (1, 8192, 8192), (64, 1024, 2048)])
def test_dequant_matmul_reference_weight_layout(m, n, k, dt):
    """dequantize_matmul with the reference's own weight layout, int8 b
    row-major [K, N] (stride_bk = N, ops/suite/perf/dequantize_matmul.py:62-65):
    from one 256 tile each way the weights are widened as they lie and the
    row-major-B MFMA kernel runs with the scale in its epilogue; smaller M
    transposes the int8 weights once and takes the fused / decode kernels.
    Bar 2e-2 against float64 a . (b * scale) on the rounded inputs."""
    rng = np.random.default_rng(m + 3 * n + k)
    a = rng.standard_normal((m, k)).astype(np.float32) * 0.5
    b = rng.integers(-127, 128, (k, n)).astype(np.int8)
    s = (rng.random(n) / 64).astype(np.float32)
    ad, sd = dev(a, dt), dev(s, dt)
    y = ops.dequant_matmul(ad, torch.from_numpy(b).to(DEV), sd, sync=True)
    short = "bf16" if dt == "bfloat16" else "f16"
    kern = rt.module().last_kernel
    if m >= 256 and n >= 256 and k % 64 == 0:
        assert kern == f"g950_gemm_{short}_256x256_rb"
    else:
        assert kern.startswith("g950_gemm_w8a16_"), kern
    rows = np.arange(m) if m <= 512 else np.unique(np.r_[0, 255, 256, m - 1,
                                                        np.random.default_rng(5).integers(0, m, 24)])
    expect = ref.matmul(host(ad)[rows], ref.dequantize(b, host(sd)))
    close(host(y)[rows], expect, 2e-2, 2e-2)
    # the K-contiguous layout of the same weights gives the same values (GEMM bar)
    y2 = ops.dequant_matmul(ad, torch.from_numpy(np.ascontiguousarray(b.T)).to(DEV).t(), sd, sync=True)
    close(host(y), host(y2), 2e-2, 2e-2)


def test_dequant_matmul_random_shapes_sweep():
    """Sixteen seeded dequantize_matmul shapes over the routes of both weight
    layouts: decode rows (M 1..64) and larger M (65..1200), N and K
    multiples of 16 (N up to 4096, K up to 2048), K-contiguous int8 weights
    and the reference's row-major [K, N] weights, bf16 and fp16 in turn;
    every row against float64 a . (b * scale) on the rounded inputs (2e-2),
    and the decode, fused and widened row-major-B kernel families reached."""
    rng = np.random.default_rng(31337)
    ran = set()
    for case in range(16):
        dt = ("bfloat16", "float16")[case % 2]
        route = (case // 2) % 4
        m = int(rng.integers(1, 65)) if route < 2 else int(rng.integers(65 if route == 2 else 256, 1201))
        n = 16 * int(rng.integers(1 if route < 3 else 16, 257))
        k = 64 * int(rng.integers(1, 33)) if route == 3 else 16 * int(rng.integers(1, 129))
        rowmajor = route in (1, 3)
        tag = f"case {case}: {dt} m {m} n {n} k {k} {'row-major' if rowmajor else 'K-contiguous'} weights"
        a = rng.standard_normal((m, k)).astype(np.float32) * 0.5
        b = rng.integers(-127, 128, (k, n)).astype(np.int8)
        s = (rng.random(n) / 64).astype(np.float32)
        ad, sd = dev(a, dt), dev(s, dt)
        bw = torch.from_numpy(b).to(DEV) if rowmajor else torch.from_numpy(np.ascontiguousarray(b.T)).to(DEV).t()
        y = ops.dequant_matmul(ad, bw, sd, sync=True)
        kern = rt.module().last_kernel
        ran.add(kern)
        expect = ref.matmul(host(ad), ref.dequantize(b, host(sd)))
        ok, err = ref.isclose_verdict(host(y), expect, 2e-2, 2e-2)
        assert ok, f"{tag}: {kern} max abs err {err}"
    assert any(k.startswith("g950_gemm_w8a16_skinny") for k in ran), sorted(ran)
    assert any(k.startswith("g950_gemm_w8a16_") and k.endswith("_128x128") for k in ran), sorted(ran)
    assert any(k.endswith("_256x256_rb") for k in ran), sorted(ran)


def test_dequant_matmul_general_layouts():
    """Row-major int8 b with rows that are not whole 16-byte vectors, fp32 a
    and a ragged K take the general kernel, same bar (fp32: 1e-4)."""
    rng = np.random.default_rng(12)
    a = rng.standard_normal((70, 40)).astype(np.float32)
    b = rng.integers(-128, 128, (40, 90)).astype(np.int8)
    s = rng.random(90).astype(np.float32)
    for dt, bar in (("float32", 1e-4), ("bfloat16", 2e-2)):
        ad, sd = dev(a, dt), dev(s, dt)
        y = ops.dequant_matmul(ad, torch.from_numpy(b).to(DEV), sd, sync=True)
        assert rt.module().last_kernel == "g950_gemm_general"
        close(host(y), ref.matmul(host(ad), ref.dequantize(b, host(sd))), bar, bar)


def test_gemm_f16_and_general_paths():
    rng = np.random.default_rng(3)
    a = rng.standard_normal((130, 192)).astype(np.float16).astype(np.float32)
    b = rng.standard_normal((192, 70)).astype(np.float16).astype(np.float32)
    expect = ref.matmul(a, b)
    # K-contiguous B -> MFMA f16 kernel
    y = ops.matmul(dev(a, "float16"), dev(b.T.copy(), "float16").t(), sync=True)
    assert rt.module().last_kernel == "g950_gemm_f16_256x256"
    close(host(y), expect, 1e-2, 1e-2)
    # row-major B -> general kernel, fp32 output
    out = torch.empty((130, 70), dtype=torch.float32, device=DEV)
    ops.matmul_kernel(dev(a, "float16"), dev(b, "float16"), out, 130, 70, 192, sync=True)
    assert rt.module().last_kernel == "g950_gemm_general"
    close(host(out), expect, 1e-3, 1e-3)


@pytest.mark.parametrize("dt", ["bfloat16", "float16"])
@pytest.mark.parametrize("m,n,k", [(256, 256, 64), (300, 264, 256), (513, 1000, 1024), (1, 8, 64), (8, 24, 32),
                                   (257, 136, 200), (130, 72, 8), (4096, 4096, 4096), (4097, 11008, 4096),
                                   (256, 520, 192), (777, 264, 128)])
def test_gemm_row_major_b_on_mfma(m, n, k, dt):
    """The reference matmul's own layout (row-major B, ops/suite/perf/matmul.py:33):
    from one 256 tile each way with whole 64-k slabs the MFMA kernel reads B as
    it lies (transposing LDS reads, _rb); smaller shapes and K tails copy B
    once K-contiguous, then the MFMA kernel (the _kt form when K is not a
    whole 64-element slab: the last slab's tail multiplies zeros).  Bar 2e-2
    (bf16) / 1e-2 (fp16) against float64, every column of the rows checked
    (one per 256-row tile at the large shapes, edges included); rows and
    columns outside the output are guarded."""
    c = inputs.config3(m, n, k)
    a, b = dev(c["a"], dt), dev(np.ascontiguousarray(c["bt"].T), dt)   # b: [K, N] row-major
    full = torch.full((m + 2, n + 8), 7.0, dtype=TD[dt], device=DEV)
    y = full[1:m + 1, :n]
    ops.matmul_kernel(a, b, y, m, n, k, sync=True)
    short = "bf16" if dt == "bfloat16" else "f16"
    rb = m >= 256 and n >= 256 and k % 64 == 0
    assert rt.module().last_kernel == f"g950_gemm_{short}_256x256" + ("_rb" if rb else "_kt" if k % 64 else "")
    rows = np.arange(m) if m <= 1024 else tile_rows(m, 3)
    bar = 2e-2 if dt == "bfloat16" else 1e-2
    close(host(y)[rows], ref.matmul(host(a)[rows], host(b)), bar, bar)
    fh = host(full)
    assert (fh[0] == 7).all() and (fh[-1] == 7).all() and (fh[:, n:] == 7).all()


def test_gemm_row_major_b_config3_full_size():
    """C3a in the reference matmul's layout (row-major B [8192, 8192]) through
    the _rb kernel: one row of every 256-row tile plus the edges, all 8192
    columns, against float64; and bit-identical to the column-major kernel
    on the same values (same MFMA sequence per output: both sum the 64-k
    slabs in order with the same fragment k layout)."""
    c = inputs.config3(8192, 8192, 8192)
    a = dev(c["a"], "bfloat16")
    bt = dev(c["bt"], "bfloat16")
    b = bt.t().contiguous()                                          # [K, N] row-major
    y = torch.empty((8192, 8192), dtype=torch.bfloat16, device=DEV)
    ops.matmul_kernel(a, b, y, 8192, 8192, 8192, sync=True)
    assert rt.module().last_kernel == "g950_gemm_bf16_256x256_rb"
    rows = tile_rows(8192, 4)
    close(host(y)[rows], ref.matmul(host(a)[rows], host(b)), 2e-2, 2e-2)
    y2 = torch.empty_like(y)
    ops.matmul_kernel(a, bt.t(), y2, 8192, 8192, 8192, sync=True)
    assert rt.module().last_kernel == "g950_gemm_bf16_256x256"
    assert torch.equal(y, y2)


@pytest.mark.parametrize("colb", [True, False])
@pytest.mark.parametrize("m,n,k", [(256, 256, 32), (300, 260, 256), (513, 1000, 1024), (16, 16, 16), (8, 32, 24),
                                   (4096, 4096, 4096)])
def test_gemm_fp32_mfma(m, n, k, colb):
    """fp32 operands (the matmul corpus's base dtype, ops/suite/perf/matmul.py)
    on v_mfma_f32_32x32x2_f32, both B layouts, K tails included: fp32
    accumulation against float64 within 1e-5 (np.isclose form)."""
    rng = np.random.default_rng(m * 3 + n + k)
    a = rng.standard_normal((m, k)).astype(np.float32)
    bt = rng.standard_normal((n, k)).astype(np.float32)
    ad = torch.from_numpy(a).to(DEV)
    bd = torch.from_numpy(bt).to(DEV).t() if colb else torch.from_numpy(np.ascontiguousarray(bt.T)).to(DEV)
    y = torch.empty((m, n), dtype=torch.float32, device=DEV)
    ops.matmul_kernel(ad, bd, y, m, n, k, sync=True)
    assert rt.module().last_kernel == "g950_gemm_f32_256x256" + ("_kt" if k % 32 else "")
    rows = np.arange(m) if m <= 1024 else tile_rows(m, 5)
    close(y.cpu().numpy()[rows], ref.matmul(a[rows], bt.T), 1e-5, 1e-5 * np.sqrt(k))


def test_gemm_layouts_random_sweep():
    """Eighteen seeded GEMMs across the dispatcher: bf16, fp16 and fp32 in
    turn, K-contiguous or the reference's row-major B, M and N in 1..1300,
    K in 1..2048 (16-bit: half whole 64-k slabs, most of the rest multiples
    of 8 with a tail, now and then any K); every element against float64 (16-bit 2e-2, fp32
    1e-5 with the sqrt(K) absolute term), and the column-major, row-major,
    K-tail and general kernels all reached."""
    rng = np.random.default_rng(6502)
    ran = set()
    for case in range(18):
        dt = ("bfloat16", "float16", "float32")[case % 3]
        m, n = (int(v) for v in rng.integers(1, 1301, 2))
        draw = rng.random()
        if dt != "float32" and draw < 0.5:
            k = 64 * int(rng.integers(1, 33))
        elif dt != "float32" and draw < 0.85:
            k = 8 * int(rng.integers(1, 257))
        else:
            k = int(rng.integers(1, 2049))
        colb = bool(rng.random() < 0.5)
        if not colb and dt != "float32" and rng.random() < 0.7:
            n = max(8, n // 8 * 8)  # 16-byte B rows: the row-major MFMA kernel can read them as they lie
        a = rng.standard_normal((m, k)).astype(np.float32)
        bt = rng.standard_normal((n, k)).astype(np.float32)
        ad = dev(a, dt)
        bd = dev(bt, dt).t() if colb else dev(np.ascontiguousarray(bt.T), dt)
        y = torch.empty((m, n), dtype=TD[dt], device=DEV)
        ops.matmul_kernel(ad, bd, y, m, n, k, sync=True)
        kern = rt.module().last_kernel
        ran.add(kern)
        tag = f"case {case}: {dt} m {m} n {n} k {k} {'K-contiguous' if colb else 'row-major'} B ({kern})"
        expect = ref.matmul(host(ad), host(bd))
        bar = (1e-5, 1e-5 * np.sqrt(k)) if dt == "float32" else (2e-2, 2e-2)
        ok, err = ref.isclose_verdict(host(y), expect, *bar)
        assert ok, f"{tag}: max abs err {err}"
    assert any(k.endswith("_256x256") for k in ran), sorted(ran)
    assert any(k.endswith("_rb") for k in ran), sorted(ran)
    assert any(k.endswith("_kt") for k in ran), sorted(ran)
    assert any("general" in k for k in ran), sorted(ran)


def test_gemm_fp32_ieee_exact_grid():
    """The reference's IEEE check (a100c/tests/test_matrix_breadth.py:454):
    operands on a 1/16 grid make every product and partial sum exact in fp32,
    so the MFMA result must equal the exact (float64) product bit for bit."""
    rng = np.random.default_rng(454)
    a = (rng.integers(-16, 17, (300, 256)) / 16.0).astype(np.float32)
    b = (rng.integers(-16, 17, (256, 200)) / 16.0).astype(np.float32)
    y = torch.empty((300, 200), dtype=torch.float32, device=DEV)
    ops.matmul_kernel(torch.from_numpy(a).to(DEV), torch.from_numpy(b).to(DEV), y, 300, 200, 256, sync=True)
    assert rt.module().last_kernel == "g950_gemm_f32_256x256"
    exact = a.astype(np.float64) @ b.astype(np.float64)
    assert np.array_equal(y.cpu().numpy(), exact.astype(np.float32))


@pytest.mark.parametrize("m,n,k", [(256, 256, 72), (300, 260, 200), (64, 64, 8), (1000, 513, 4104)])
def test_gemm_k_tail_k_contiguous(m, n, k):
    """K-contiguous operands with K a multiple of 8 but not of 64: the _kt
    kernel's zero-filled last slab; the guard columns of a strided output and
    a run-twice bit identity."""
    c = inputs.config3(m, n, k)
    a, bt = dev(c["a"], "bfloat16"), dev(c["bt"], "bfloat16")
    out = torch.full((m, n + 8), -7.0, dtype=torch.bfloat16, device=DEV)
    y = out[:, :n]
    ops.matmul_kernel(a, bt.t(), y, m, n, k, sync=True)
    assert rt.module().last_kernel == "g950_gemm_bf16_256x256_kt"
    close(host(y), ref.matmul(c["a"], c["bt"].T), 2e-2, 2e-2)
    assert bool((out[:, n:] == -7.0).all())
    y2 = torch.empty_like(y)
    ops.matmul_kernel(a, bt.t(), y2, m, n, k, sync=True)
    assert torch.equal(y.contiguous(), y2)


@pytest.mark.parametrize("m,n,k", [(300, 200, 208), (65, 33, 48), (4096, 8192, 8176)])
def test_int8_k_tail_exact(m, n, k):
    """Signed int8 with K a multiple of 16 but not of 128: the _kt kernel,
    int32 bit-exact (zeros add nothing)."""
    c = inputs.config5(m, n, k)
    a, bt = torch.from_numpy(c["a"]).to(DEV), torch.from_numpy(c["bt"]).to(DEV)
    acc = torch.empty((m, n), dtype=torch.int32, device=DEV)
    ops.matmul_i8_kernel(a, bt.t(), acc, m, n, k, sync=True)
    assert rt.module().last_kernel == "g950_gemm_i8_256x256_kt"
    rows = np.arange(m) if m <= 512 else tile_rows(m, 13)
    got = acc[torch.from_numpy(rows).to(DEV)].cpu().numpy()
    assert np.array_equal(got, ref.matmul_i8(c["a"][rows], c["bt"].T))


@pytest.mark.parametrize("case", golden_cases("matmul"))
def test_matmul_reference_fixture(case):
    b = load(case)
    dt = dtype_of(case)
    a, bb = values(b, "a_ptr"), values(b, "b_ptr")
    m, k = a.shape
    n = bb.shape[1]
    rtol, atol = ref.TOLERANCES[dt]
    # the fixture layout (row-major B): the MFMA kernel for 16-bit operands
    y = torch.zeros((m, n), dtype=TD[dt], device=DEV)
    ops.matmul_kernel(dev(a, dt), dev(bb, dt), y, m, n, k, sync=True)
    if dt != "float32" and k % 8 == 0 and n % 8 == 0:
        assert rt.module().last_kernel.startswith("g950_gemm_"), rt.module().last_kernel
        assert "general" not in rt.module().last_kernel
    close(host(y), values(b, "y_ptr"), rtol, atol)
    # ... and the same values column-major, which takes the MFMA kernel when K allows
    if dt != "float32":
        y2 = torch.zeros((m, n), dtype=TD[dt], device=DEV)
        ops.matmul_kernel(dev(a, dt), dev(bb.T.copy(), dt).t(), y2, m, n, k, sync=True)
        close(host(y2), values(b, "y_ptr"), rtol, atol)


# ------------------------------------------------------------------ int8
@pytest.mark.parametrize("m,n,k", [(256, 256, 128), (300, 200, 384), (4096, 8192, 8192), (64, 64, 128),
                                   (300, 200, 256), (65, 33, 640)])
def test_int8_gemm_exact_and_dequant(m, n, k):
    c = inputs.config5(m, n, k)
    a = torch.from_numpy(c["a"]).to(DEV)
    bt = torch.from_numpy(c["bt"]).to(DEV)
    acc = torch.empty((m, n), dtype=torch.int32, device=DEV)
    ops.matmul_i8_kernel(a, bt.t(), acc, m, n, k, sync=True)
    assert rt.module().last_kernel == "g950_gemm_i8_256x256"
    y = torch.empty((m, n), dtype=torch.bfloat16, device=DEV)
    ops.matmul_i8_dequant_kernel(a, bt.t(), torch.from_numpy(c["sa"]).to(DEV),
                                 torch.from_numpy(c["sb"]).to(DEV), y, m, n, k, sync=True)
    rows = np.arange(m) if m * n <= 1 << 20 else tile_rows(m, 11)
    exact = ref.matmul_i8(c["a"][rows], c["bt"].T)
    assert np.abs(exact).max() < 2 ** 31
    got = acc[torch.from_numpy(rows).to(DEV)].cpu().numpy()
    assert np.array_equal(got, exact)  # bit-exact int32
    deq = ref.dequant(exact, c["sa"][rows], c["sb"])
    close(host(y[torch.from_numpy(rows).to(DEV)]), deq, 2e-2, 2e-2)


@pytest.mark.parametrize("m,n,k", [(257, 257, 128), (300, 263, 256), (511, 1001, 640), (256, 259, 128)])
def test_gemm_16x16_edge_windows(m, n, k):
    """M, N >= 256 with whole K slabs take the 16x16-fragment kernel, whose
    edge tiles compute the 256x256 window ending at the matrix edge and store
    only their own rows and columns; N not a multiple of 4 moves those
    windows off 4-column alignment (element stores).  Every output element:
    int8 bit-exact for all four signedness pairs (int32 and the dequant
    epilogue), bf16 / f16 to their bars, and the output's guard rows and
    columns untouched."""
    rng = np.random.default_rng(m * 7 + n)
    pad = 8 - n % 8  # output rows 16-byte aligned, >= 1 guard column after each row
    for adt, bdt in ((np.int8, np.int8), (np.uint8, np.int8), (np.int8, np.uint8), (np.uint8, np.uint8)):
        lo_a, hi_a = (-128, 128) if adt is np.int8 else (0, 256)
        lo_b, hi_b = (-128, 128) if bdt is np.int8 else (0, 256)
        a = rng.integers(lo_a, hi_a, (m, k)).astype(adt)
        bt = rng.integers(lo_b, hi_b, (n, k)).astype(bdt)
        full = torch.full((m + 2, n + pad), -5, dtype=torch.int32, device=DEV)
        acc = full[1:m + 1, :n]
        ops.matmul_i8_kernel(torch.from_numpy(a).to(DEV), torch.from_numpy(bt).to(DEV).t(), acc, m, n, k,
                             sync=True)
        assert rt.module().last_kernel.endswith("_256x256")
        # |a.b| <= 255^2 * 640 < 2^31: the int32 result is the exact product
        assert np.array_equal(acc.cpu().numpy().astype(np.int64), a.astype(np.int64) @ bt.T.astype(np.int64))
        fh = full.cpu().numpy()
        assert (fh[0] == -5).all() and (fh[-1] == -5).all() and (fh[:, n:] == -5).all()
    c = inputs.config5(m, n, k)
    y = torch.empty((m, n), dtype=torch.bfloat16, device=DEV)
    ops.matmul_i8_dequant_kernel(torch.from_numpy(c["a"]).to(DEV), torch.from_numpy(c["bt"]).to(DEV).t(),
                                 torch.from_numpy(c["sa"]).to(DEV), torch.from_numpy(c["sb"]).to(DEV), y, m, n, k,
                                 sync=True)
    assert rt.module().last_kernel == "g950_gemm_i8_256x256"
    close(host(y), ref.dequant(ref.matmul_i8(c["a"], c["bt"].T), c["sa"], c["sb"]), 2e-2, 2e-2)
    for dt in ("bfloat16", "float16"):
        c3 = inputs.config3(m, n, k)
        full = torch.full((m + 2, n + pad), 7.0, dtype=TD[dt], device=DEV)
        y = full[1:m + 1, :n]
        ops.matmul_kernel(dev(c3["a"], dt), dev(c3["bt"], dt).t(), y, m, n, k, sync=True)
        assert rt.module().last_kernel.endswith("_256x256")
        ad, bd = host(dev(c3["a"], dt)), host(dev(c3["bt"], dt))
        close(host(y), ref.matmul(ad, bd.T), *((2e-2, 2e-2) if dt == "bfloat16" else (1e-2, 1e-2)))
        fh = host(full)
        assert (fh[0] == 7).all() and (fh[-1] == 7).all() and (fh[:, n:] == 7).all()


@pytest.mark.parametrize("m,n,k", [(512, 512, 128), (300, 512, 256), (513, 768, 384), (4097, 1024, 128)])
def test_gemm_staged_epilogue_matches_row_stores(m, n, k):
    """Tiles of the 16x16 kernel that own all of their window's columns and
    write a 16-bit output with 16-byte aligned rows stage the output tile
    through LDS and store whole row pieces (a bottom-edge window stores only
    its own rows); an output row stride that is not a multiple of 8 elements
    takes the row-by-row stores.  The two must give the same bits: bf16 and
    f16 GEMM, the int8 dequant epilogue in all four signedness pairs, and the
    W8A16 column scale -- with the guard rows and columns around the output
    untouched."""
    rng = np.random.default_rng(m + 3 * n + k)
    both = functools.partial(_staged_vs_row_stores, m, n)
    c3 = inputs.config3(m, n, k)
    for dt in ("bfloat16", "float16"):
        a, bt = dev(c3["a"], dt), dev(c3["bt"], dt)
        name = "g950_gemm_bf16_256x256" if dt == "bfloat16" else "g950_gemm_f16_256x256"
        y = both(lambda out: ops.matmul_kernel(a, bt.t(), out, m, n, k), dt, name)
        close(host(y), ref.matmul(host(a), host(bt).T), *((2e-2, 2e-2) if dt == "bfloat16" else (1e-2, 1e-2)))
        brow = bt.t().contiguous()
        both(lambda out: ops.matmul_kernel(a, brow, out, m, n, k), dt, name + "_rb")
    sa = torch.from_numpy((rng.random(m) * 0.02 + 0.001).astype(np.float32)).to(DEV)
    sb = torch.from_numpy((rng.random(n) * 0.02 + 0.001).astype(np.float32)).to(DEV)
    for adt, bdt, name in ((np.int8, np.int8, "g950_gemm_i8_256x256"), (np.uint8, np.int8, "g950_gemm_u8s8_256x256"),
                           (np.int8, np.uint8, "g950_gemm_s8u8_256x256"), (np.uint8, np.uint8, "g950_gemm_u8u8_256x256")):
        lo_a, hi_a = (-128, 128) if adt is np.int8 else (0, 256)
        lo_b, hi_b = (-128, 128) if bdt is np.int8 else (0, 256)
        a8 = torch.from_numpy(rng.integers(lo_a, hi_a, (m, k)).astype(adt)).to(DEV)
        b8 = torch.from_numpy(rng.integers(lo_b, hi_b, (n, k)).astype(bdt)).to(DEV)
        both(lambda out: ops.matmul_i8_dequant_kernel(a8, b8.t(), sa, sb, out, m, n, k), "bfloat16", name)


def test_gemm_random_shapes_sweep():
    """Sixteen seeded shapes of the 16x16-fragment kernel (M, N in 256..1300,
    K a multiple of 64): tile counts that are and are not multiples of 8
    (the XCD-contiguous tile order), bottom/right edge windows, both output
    paths (16-byte aligned rows: staged; stride n + 1: row stores) bit-equal,
    and every element against float64."""
    rng = np.random.default_rng(2026)
    for _ in range(16):
        m, n = (int(v) for v in rng.integers(256, 1301, 2))
        k = 64 * int(rng.integers(1, 9))
        c3 = inputs.config3(m, n, k)
        a, bt = dev(c3["a"], "bfloat16"), dev(c3["bt"], "bfloat16")
        y = _staged_vs_row_stores(m, n, lambda out: ops.matmul_kernel(a, bt.t(), out, m, n, k), "bfloat16",
                                  "g950_gemm_bf16_256x256")
        close(host(y), ref.matmul(host(a), host(bt).T), 2e-2, 2e-2)


def test_w8a16_staged_epilogue_matches_row_stores():
    """The widened W8A16 route (more 256x256 tiles than half the CUs: an
    exact bf16 copy of the int8 weights, then the bf16 GEMM with the column
    scale in its epilogue) stages its output like the plain GEMM; the same
    bits as the row-by-row stores, on a shape with a bottom-edge window."""
    m, n, k = 3000, 3072, 128
    rng = np.random.default_rng(5)
    a = dev((rng.standard_normal((m, k)) * 0.1).astype(np.float32), "bfloat16")
    w8 = torch.from_numpy(rng.integers(-127, 128, (n, k)).astype(np.int8)).to(DEV)
    scale = dev((rng.random(n) * 0.02 + 0.001).astype(np.float32), "bfloat16")
    y = _staged_vs_row_stores(m, n, lambda out: ops.dequant_matmul_kernel(a, w8.t(), scale, out, m, n, k),
                              "bfloat16", "g950_gemm_bf16_256x256")
    deq = host(w8.t().float() * scale.float()[None, :])
    close(host(y), ref.matmul(host(a), deq), 2e-2, 2e-2)


def _staged_vs_row_stores(m, n, launch, dt, name):
    """Run ``launch`` into an [m, n] output inside a guarded buffer twice:
    row stride n + 8 (16-byte aligned rows: the staged epilogue) and n + 1
    (the row-by-row stores), both starting 16 bytes (8 elements) into the
    buffer; the same bits, the 8 leading and trailing guard elements and the
    gap after each row untouched."""
    outs = []
    for extra in (8, 1):
        flat = torch.full((16 + m * (n + extra),), 3.0, dtype=TD[dt], device=DEV)
        y = torch.as_strided(flat, (m, n), (n + extra, 1), 8)
        launch(y)
        torch.cuda.synchronize()
        assert rt.module().last_kernel == name
        fh = host(flat)
        rows = fh[8:8 + m * (n + extra)].reshape(m, n + extra)
        assert (fh[:8] == 3).all() and (fh[-8:] == 3).all() and (rows[:, n:] == 3).all()
        outs.append(y.clone())
    assert torch.equal(outs[0], outs[1]), name
    return outs[0]


def test_int8_general_path_exact():
    rng = np.random.default_rng(12)
    a = rng.integers(-128, 128, (37, 100), dtype=np.int8)   # K not a slab multiple
    b = rng.integers(-128, 128, (100, 45), dtype=np.int8)   # row-major
    acc = torch.empty((37, 45), dtype=torch.int32, device=DEV)
    ops.matmul_i8_kernel(torch.from_numpy(a).to(DEV), torch.from_numpy(b).to(DEV), acc, 37, 45, 100,
                         sync=True)
    assert rt.module().last_kernel == "g950_gemm_general_i8"
    assert np.array_equal(acc.cpu().numpy(), ref.matmul_i8(a, b))


# ------------------------------------------------------------- attention
@pytest.mark.parametrize("z,h,hkv,s,d,causal", [
    (1, 4, 2, 200, 128, True), (2, 2, 1, 333, 64, True), (1, 2, 2, 130, 128, False),
    (1, 1, 1, 1, 128, True)])
def test_attention_small(z, h, hkv, s, d, causal):
    c = inputs.config4(z, h, hkv, s, d)
    o, lse = ops.attention(dev(c["q"], "bfloat16"), dev(c["k"], "bfloat16"), dev(c["v"], "bfloat16"),
                           causal=causal, sync=True)
    assert rt.module().last_kernel == f"g950_attn_fwd_bf16_d{d}"
    eo, el = ref.attention(c["q"], c["k"], c["v"], c["scale"], causal=causal)
    close(host(o), eo, 2e-2, 2e-2)
    close(lse.cpu().numpy(), el, 1e-4, 1e-4)


def test_attention_random_shapes_sweep():
    """Twelve seeded shapes of the 16-bit MFMA attention kernels: sequence
    lengths 1..900 (one or several 256-query blocks, the last key tile cut
    anywhere), 1-3 batches, 1-2 KV heads with GQA groups 1, 2 or 4, head
    dim 64 or 128, causal or not, bf16 and fp16 in turn; O and LSE against
    float64 on the 16-bit-rounded inputs."""
    rng = np.random.default_rng(777)
    for case in range(12):
        dt = ("bfloat16", "float16")[case % 2]
        d = (64, 128)[int(rng.integers(0, 2))]
        hkv = int(rng.integers(1, 3))
        h = hkv * (1, 2, 4)[int(rng.integers(0, 3))]
        z = int(rng.integers(1, 4))
        s = int(rng.integers(1, 901))
        causal = bool(rng.random() < 0.5)
        tag = f"case {case}: {dt} z {z} h {h}/{hkv} s {s} d {d} causal {causal}"
        c = inputs.config4(z, h, hkv, s, d, seed=500 + case)
        q, k, v = (dev(c[n], dt) for n in ("q", "k", "v"))
        o, lse = ops.attention(q, k, v, causal=causal, sync=True)
        assert rt.module().last_kernel == f"g950_attn_fwd_{'bf16' if dt == 'bfloat16' else 'f16'}_d{d}", tag
        eo, el = ref.attention(host(q), host(k), host(v), c["scale"], causal=causal)
        ok, err = ref.isclose_verdict(host(o), eo, 2e-2, 2e-2)
        assert ok, f"{tag}: O max abs err {err}"
        ok, err = ref.isclose_verdict(lse.cpu().numpy(), el, 1e-4, 1e-4)
        assert ok, f"{tag}: LSE max abs err {err}"


@pytest.mark.parametrize("dt", ["bfloat16", "float16"])
@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("causal", [True, False])
def test_attention_every_mfma_instantiation(dt, d, causal):
    """Every fixed-length MFMA kernel over many key tiles (the interior tiles
    run the pipelined MFMA phase, the edges the plain one)."""
    c = inputs.config4(1, 4, 2, 520, d)
    o, lse = ops.attention(dev(c["q"], dt), dev(c["k"], dt), dev(c["v"], dt), causal=causal, sync=True)
    assert rt.module().last_kernel == f"g950_attn_fwd_{'bf16' if dt == 'bfloat16' else 'f16'}_d{d}"
    q, k, v = (host(dev(c[n], dt)) for n in ("q", "k", "v"))
    eo, el = ref.attention(q, k, v, c["scale"], causal=causal)
    close(host(o), eo, 2e-2, 2e-2)
    close(lse.cpu().numpy(), el, 1e-4, 1e-4)


@pytest.mark.parametrize("dt", ["bfloat16", "float16"])
@pytest.mark.parametrize("d,s,causal", [(128, 520, True), (64, 333, True), (128, 100, False), (64, 1, True)])
def test_attention_staged_epilogue_matches_row_stores(dt, d, s, causal):
    """With 16-byte aligned output rows the 16-bit kernels stage each wave's
    output tile through LDS and store whole rows (queries past the sequence
    end masked); an output row stride of d + 4 elements takes the per-lane
    8-byte stores.  The two must give the same bits, with the padding after
    each output row untouched, and match the oracle."""
    c = inputs.config4(1, 4, 2, s, d)
    q, k, v = (dev(c[n], dt) for n in ("q", "k", "v"))
    outs = []
    for pad in (8, 4):
        full = torch.full((1, 4, s, d + pad), 5.0, dtype=TD[dt], device=DEV)
        o = full[..., :d]
        lse = torch.empty((1, 4, s), device=DEV)
        ops.attn_fwd_causal_kernel(q, k, v, o, 1, 4, s, c["scale"], *q.stride(), *k.stride(), *v.stride(),
                                   *o.stride(), CAUSAL=causal, lse_ptr=lse, sync=True)
        assert rt.module().last_kernel == f"g950_attn_fwd_{'bf16' if dt == 'bfloat16' else 'f16'}_d{d}"
        assert bool((full[..., d:] == 5.0).all())
        outs.append((o.clone(), lse.clone()))
    assert torch.equal(outs[0][0], outs[1][0]) and torch.equal(outs[0][1], outs[1][1])
    qh, kh, vh = (host(t) for t in (q, k, v))
    eo, el = ref.attention(qh, kh, vh, c["scale"], causal=causal)
    close(host(outs[0][0]), eo, 2e-2, 2e-2)
    close(outs[0][1].cpu().numpy(), el, 1e-4, 1e-4)


@pytest.mark.parametrize("scale", [-0.125, 0.0])
def test_attention_non_positive_scale_takes_fp32_kernel(scale):
    """The 16-bit kernel's running maximum needs scale > 0; other scales run
    the fp32 MFMA kernel (which scales before the maximum) and still match the
    oracle's softmax of the scaled scores."""
    c = inputs.config4(1, 2, 1, 70, 64)
    o, lse = ops.attention(dev(c["q"], "bfloat16"), dev(c["k"], "bfloat16"), dev(c["v"], "bfloat16"),
                           scale=scale, causal=True, sync=True)
    assert rt.module().last_kernel == "g950_attn_fwd_f32mfma_d64"
    eo, el = ref.attention(c["q"], c["k"], c["v"], scale, causal=True)
    close(host(o), eo, 2e-2, 2e-2)
    close(lse.cpu().numpy(), el, 1e-4, 1e-4)


@pytest.mark.parametrize("z,h,hkv,s,d,causal", [
    (1, 4, 2, 200, 128, True), (2, 2, 1, 333, 64, True), (1, 2, 2, 130, 128, False), (1, 1, 1, 1, 128, True),
    (2, 4, 2, 64, 32, False), (1, 8, 8, 257, 32, True), (1, 2, 1, 1000, 64, False)])
def test_attention_fp32(z, h, hkv, s, d, causal):
    """fp32 attention (attn_fwd_causal / attention_forward_triton list float32)
    on the fp32 MFMA kernel: every score once, fp32 probabilities; against
    float64 within 1e-4 (O) and 1e-5 (LSE), np.isclose form."""
    c = inputs.config4(z, h, hkv, s, d)
    q, k, v = (torch.from_numpy(c[n]).to(DEV) for n in ("q", "k", "v"))
    o, lse = ops.attention(q, k, v, causal=causal, sync=True)
    assert rt.module().last_kernel == f"g950_attn_fwd_f32mfma_d{d}"
    eo, el = ref.attention(c["q"], c["k"], c["v"], c["scale"], causal=causal)
    close(o.cpu().numpy(), eo, 1e-4, 1e-5)
    close(lse.cpu().numpy(), el, 1e-5, 1e-5)


def test_attention_fp32_kernel_random_sweep():
    """Ten seeded shapes of the fp32 MFMA attention kernel: fp32 inputs at
    head dim 32, 64 or 128, and (three of the ten) 16-bit inputs at head dim
    32, which that kernel also serves; sequence lengths 1..700, 1-2 batches,
    GQA groups 1/2/4, causal or not.  fp32: O within 1e-4 / 1e-5 and LSE
    within 1e-5 of float64; 16-bit: the 16-bit attention bars."""
    rng = np.random.default_rng(1729)
    for case in range(10):
        dt = ("float32", "float32", "bfloat16", "float32", "float16")[case % 5] if case < 8 else "float32"
        d = 32 if dt != "float32" else (32, 64, 128)[int(rng.integers(0, 3))]
        hkv = int(rng.integers(1, 3))
        h = hkv * (1, 2, 4)[int(rng.integers(0, 3))]
        z = int(rng.integers(1, 3))
        s_len = int(rng.integers(1, 701))
        causal = bool(rng.random() < 0.5)
        tag = f"case {case}: {dt} z {z} h {h}/{hkv} s {s_len} d {d} causal {causal}"
        c = inputs.config4(z, h, hkv, s_len, d, seed=900 + case)
        q, k, v = (dev(c[n], dt) for n in ("q", "k", "v"))
        o, lse = ops.attention(q, k, v, causal=causal, sync=True)
        assert rt.module().last_kernel == f"g950_attn_fwd_f32mfma_d{d}", (tag, rt.module().last_kernel)
        eo, el = ref.attention(host(q), host(k), host(v), c["scale"], causal=causal)
        bars = ((1e-4, 1e-5), (1e-5, 1e-5)) if dt == "float32" else ((2e-2, 2e-2), (1e-4, 1e-4))
        ok, err = ref.isclose_verdict(host(o), eo, *bars[0])
        assert ok, f"{tag}: O max abs err {err}"
        ok, err = ref.isclose_verdict(lse.cpu().numpy(), el, *bars[1])
        assert ok, f"{tag}: LSE max abs err {err}"


@pytest.mark.parametrize("shift,d", [(1, 64), (2, 128), (1, 32)])
def test_attention_fp32_unaligned_kv(shift, d):
    """fp32 K and V views that start one (two) elements into their buffers
    and have row strides that are not whole 16-byte vectors: the fp32 MFMA
    kernel stages them element by element (no 16-byte vector loads at
    unaligned addresses) and still matches the oracle."""
    c = inputs.config4(1, 4, 2, 150, d)
    q = torch.from_numpy(c["q"]).to(DEV)

    def shifted(a):
        z, h, s_, dd = a.shape
        row = dd + shift                     # padded rows: stride dd + shift elements
        buf = torch.zeros(shift + z * h * s_ * row, device=DEV)
        view = buf[shift:].view(z, h, s_, row)[..., :dd]
        view.copy_(torch.from_numpy(a).to(DEV))
        return view
    k, v = shifted(c["k"]), shifted(c["v"])
    assert k.data_ptr() % 16 != 0 and k.stride(2) % 4 != 0
    o, lse = ops.attention(q, k, v, causal=True, sync=True)
    assert rt.module().last_kernel == f"g950_attn_fwd_f32mfma_d{d}"
    eo, el = ref.attention(c["q"], c["k"], c["v"], c["scale"], causal=True)
    close(o.cpu().numpy(), eo, 1e-4, 1e-5)
    close(lse.cpu().numpy(), el, 1e-5, 1e-5)


def test_attention_fp32_config4_scale():
    """C4's shape in fp32 ([4, 32, 4096, 128], 8 KV heads, causal): one query
    head of every KV group of batches 0 and 3 checked in full."""
    c = inputs.config4()
    q, k, v = (torch.from_numpy(c[n]).to(DEV) for n in ("q", "k", "v"))
    o, lse = ops.attention(q, k, v, causal=True, sync=True)
    assert rt.module().last_kernel == "g950_attn_fwd_f32mfma_d128"
    rng = np.random.default_rng(8)
    for zz in (0, 3):
        for g in range(8):
            hh = 4 * g + int(rng.integers(0, 4))
            eo, el = ref.attention(c["q"][zz:zz + 1, hh:hh + 1], c["k"][zz:zz + 1, g:g + 1],
                                   c["v"][zz:zz + 1, g:g + 1], c["scale"], causal=True)
            close(o[zz, hh].cpu().numpy(), eo[0, 0], 1e-4, 1e-5)
            close(lse[zz, hh].cpu().numpy(), el[0, 0], 1e-5, 1e-5)


def test_attention_config4_sampled_heads():
    """Config 4 at full size: one query head of every (batch, KV group) pair --
    32 of 128 heads, each checked in full -- so every KV head's tiles and
    every XCD's share of the grid is compared."""
    c = inputs.config4()
    o, lse = ops.attention(dev(c["q"], "bfloat16"), dev(c["k"], "bfloat16"), dev(c["v"], "bfloat16"),
                           causal=True, sync=True)
    rng = np.random.default_rng(4)
    pairs = [(z, 4 * g + int(rng.integers(0, 4))) for z in range(4) for g in range(8)]
    for z, h in pairs:
        eo, el = ref.attention(c["q"][z:z + 1, h:h + 1], c["k"][z:z + 1, h // 4:h // 4 + 1],
                               c["v"][z:z + 1, h // 4:h // 4 + 1], c["scale"], causal=True)
        close(host(o[z, h]), eo[0, 0], 2e-2, 2e-2)
        close(lse[z, h].cpu().numpy(), el[0, 0], 1e-4, 1e-4)
    # causal row 0 attends to key 0 only: O = V[0] exactly (up to bf16 rounding)
    close(host(o[:, :, 0]), np.repeat(c["v"][:, :, 0], 4, axis=1), 0, 1e-6)


def climbing_scores(s, d):
    """Q/K whose scores climb by about 16 log2 units per 64-key tile: every
    query has a constant component that meets a key component growing with
    the key index, so each row's maximum passes its running reference by more
    than 8 on every tile it reads.  The online softmax then rescales l and O
    and the two half-waves holding a query combine their tile maxima on every
    tile; N(0,1) inputs move the reference on a row's first tile only."""
    c = inputs.config4(1, 4, 2, s, d, seed=31)
    q, k = c["q"].copy(), c["k"].copy()
    q[..., 0] = 4.0
    k[..., 0] = 0.5 * np.arange(s, dtype=np.float32)
    return {**c, "q": inputs.bf16_round(q), "k": inputs.bf16_round(k)}


@pytest.mark.parametrize("dt", ["bfloat16", "float16", "float32"])
@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("causal", [True, False])
def test_attention_reference_max_moves_every_tile(dt, d, causal):
    c = climbing_scores(520, d)
    q, k, v = (dev(c[n], dt) for n in ("q", "k", "v"))
    o, lse = ops.attention(q, k, v, causal=causal, sync=True)
    name = {"bfloat16": f"g950_attn_fwd_bf16_d{d}", "float16": f"g950_attn_fwd_f16_d{d}",
            "float32": f"g950_attn_fwd_f32mfma_d{d}"}[dt]
    assert rt.module().last_kernel == name
    eo, el = ref.attention(host(q), host(k), host(v), c["scale"], causal=causal)
    # fp32: the dot products reach ~1040 before scaling, so fp32 rounding of
    # their partial sums alone moves the probabilities by ~1e-4 relative; a
    # wrong rescale would miss by O(1)
    bar = (1e-3, 1e-4) if dt == "float32" else (2e-2, 2e-2)
    close(host(o), eo, *bar)
    close(lse.cpu().numpy(), el, 1e-5 if dt == "float32" else 1e-4, 1e-4)


@pytest.mark.parametrize("case", golden_cases("attention"))
def test_attention_reference_fixture(case):
    b = load(case)
    dt = dtype_of(case)
    q, k, v = (values(b, n) for n in ("q_ptr", "k_ptr", "v_ptr"))
    out = torch.zeros(q.shape, dtype=TD[dt], device=DEV)
    qd, kd, vd = dev(q, dt), dev(k, dt), dev(v, dt)
    z, h, s, d = q.shape
    ops.attn_fwd_causal_kernel(qd, kd, vd, out, z, h, s, np.float32(b.scalar("scale")),
                               *qd.stride(), *kd.stride(), *vd.stride(), *out.stride(),
                               CAUSAL=False, sync=True)
    rtol, atol = ref.TOLERANCES[dt]
    close(host(out), values(b, "out_ptr"), rtol, atol)


def test_run_twice_bit_identical():
    """Determinism (the runtime's repeat self-check, a100c/runtime/main.c:136-151)."""
    c = inputs.config3(512, 512, 512)
    a, bt = dev(c["a"], "bfloat16"), dev(c["bt"], "bfloat16").t()
    y1 = ops.matmul(a, bt, sync=True)
    y2 = ops.matmul(a, bt, sync=True)
    assert torch.equal(y1, y2)
    q = inputs.config4(1, 4, 2, 256, 128)
    o1, _ = ops.attention(dev(q["q"], "bfloat16"), dev(q["k"], "bfloat16"), dev(q["v"], "bfloat16"), sync=True)
    o2, _ = ops.attention(dev(q["q"], "bfloat16"), dev(q["k"], "bfloat16"), dev(q["v"], "bfloat16"), sync=True)
    assert torch.equal(o1, o2)
