"""GPU parity of the dev-suite kernel signatures and the int8 signedness
variants, called through the C ABI, against the float64 oracle:

  softmax_kernel_inner     ops/suite/dev/softmax_kernel_inner.py (SHAPES (17,), (97,))
  _layer_norm_forward_row  ops/suite/dev/layer_norm_forward_row.py (SHAPES (3,16), (5,128))
  gqa_kernel               ops/suite/dev/gqa.py (SHAPES (2,4,2,32,32), (2,4,2,64,32), (1,4,2,64,32))

each in float32, float16 and bfloat16 (the suite's DTYPES after enrichment),
plus one C2- or C4-scale shape.  Bars: float32 <= 1e-5 relative (reductions)
and the case's 2e-2 for gqa; 16-bit reductions 1e-2; 16-bit attention 2e-2;
integer accumulators bit-exact.
"""
import numpy as np
import pytest

torch = pytest.importorskip("torch")

from compiler_amd import operators as ops  # noqa: E402
from compiler_amd import runtime as rt  # noqa: E402
from oracle import inputs  # noqa: E402
from oracle import reference as ref  # noqa: E402

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
TD = {"float32": torch.float32, "bfloat16": torch.bfloat16, "float16": torch.float16}
DTYPES = ("float32", "float16", "bfloat16")
RED_BAR = {"float32": (1e-5, 1e-6), "float16": (1e-2, 1e-2), "bfloat16": (1e-2, 1e-2)}


def rounded(a, dt):
    a = np.asarray(a, dtype=np.float32)
    if dt == "bfloat16":
        return ref.bf16_round(a)
    if dt == "float16":
        return a.astype(np.float16).astype(np.float32)
    return a


def dev(a, dt):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(DEV).to(TD[dt])


def host(t):
    return t.float().cpu().numpy()


def close(actual, expected, rtol, atol):
    ok, err = ref.isclose_verdict(actual, expected, rtol, atol)
    assert ok, f"max abs err {err} exceeds rtol={rtol} atol={atol}"


def rel_close(actual, expected, rtol, floor):
    a = np.asarray(actual, dtype=np.float64)
    b = np.asarray(expected, dtype=np.float64)
    err = float((np.abs(a - b) / np.maximum(np.abs(b), floor)).max())
    assert err <= rtol, f"max relative error {err} > {rtol}"


# ---------------------------------------------------- softmax_kernel_inner
@pytest.mark.parametrize("dt", DTYPES)
@pytest.mark.parametrize("shape", [(17,), (97,)])
def test_softmax_kernel_inner_reference_shapes(shape, dt):
    """The reference case layer: M = 3 rows of C = max(2, N // 3) from
    N(0, 0.8) in one flat buffer, output pre-filled with -7."""
    m, c = 3, max(2, shape[0] // 3)
    x = rounded(np.random.default_rng(20260901).normal(0, 0.8, m * c), dt)
    out = torch.full((m * c,), -7.0, dtype=TD[dt], device=DEV)
    ops.softmax_kernel_inner(out, dev(x, dt), m, c, 128, False, sync=True)
    assert rt.module().last_kernel.startswith(("g950_rr_softmax_", "g950_rm_softmax_"))
    expect = ref.softmax_inner(x, m, c)
    rtol, atol = RED_BAR[dt]
    if dt == "float32":
        rel_close(host(out), expect, rtol, 1e-30)
    else:
        close(host(out), expect, rtol, atol)


def test_softmax_kernel_inner_c2_scale_and_guard():
    """C2's x (bf16 [8191, 3000] with +-60 outliers) as a flat buffer with a
    guard tail: every row matches, nothing past M*N is written."""
    c = inputs.config2()
    m, n = c["x"].shape
    xd = dev(c["x"].reshape(-1), "bfloat16")
    out = torch.full((m * n + 64,), -7.0, dtype=torch.bfloat16, device=DEV)
    ops.softmax_kernel_inner(out, xd, m, n, sync=True)
    got = host(out)
    assert np.all(got[m * n:] == -7.0)
    rows = np.unique(np.r_[0, m - 1, np.random.default_rng(3).integers(0, m, 64)])
    expect = ref.softmax(c["x"][rows])
    close(got[: m * n].reshape(m, n)[rows], expect, 1e-2, 1e-2)
    assert np.allclose(got[: m * n].reshape(m, n).sum(axis=1), 1.0, atol=2e-2)


@pytest.mark.parametrize("dt", DTYPES)
@pytest.mark.parametrize("m,n,tile", [(3, 32, 16), (3, 32, 8), (5, 3000, 2048), (4, 100, 64)])
def test_softmax_kernel_inner_one_narrow_tile(m, n, tile, dt):
    """ONE_TILE_PER_CTA with TILE_N < N (softmax_kernel_inner.py:13-24): the
    first TILE_N elements of each row are normalised among themselves and
    the rest of the output (pre-filled with -7) stays as it was."""
    x = rounded(np.random.default_rng(7).normal(0, 2.0, m * n), dt)
    before = np.full(m * n + 16, -7.0)
    out = torch.full((m * n + 16,), -7.0, dtype=TD[dt], device=DEV)
    ops.softmax_kernel_inner(out, dev(x, dt), m, n, tile, True, sync=True)
    got = host(out)
    expect = ref.softmax_inner(x, m, n, tile, True, out=before)
    rtol, atol = RED_BAR[dt]
    if dt == "float32":
        rel_close(got[: m * n], expect, rtol, 1e-30)
    else:
        close(got[: m * n], expect, rtol, atol)
    assert np.all(got.reshape(-1)[m * n:] == -7.0)


# ------------------------------------------------- _layer_norm_forward_row
def lnrow_case(rows, cols, dt, seed=20260901):
    rng = np.random.default_rng(seed)
    x = rounded(rng.normal(0, 0.7, (rows, cols)), dt)
    w = rounded(rng.uniform(0.7, 1.3, cols), dt)
    b = rounded(rng.normal(0, 0.1, cols), dt)
    return x, w, b


def run_lnrow(x, w, b, dt, sdt, eps=1e-5):
    rows, cols = x.shape
    y = torch.full((rows * cols,), -7.0, dtype=TD[dt], device=DEV)
    mean = torch.full((rows,), -7.0, dtype=TD[sdt], device=DEV)
    rstd = torch.full((rows,), -7.0, dtype=TD[sdt], device=DEV)
    ops._layer_norm_forward_row(y, cols, dev(x, dt), cols, dev(w, dt), dev(b, dt), mean, 1, rstd, 1, rows, cols,
                                eps, cols, sync=True)
    assert rt.module().last_kernel.startswith(("g950_rr_lnrow_", "g950_rw_lnrow_"))
    return host(y).reshape(rows, cols), host(mean), host(rstd)


@pytest.mark.parametrize("dt", DTYPES)
@pytest.mark.parametrize("shape", [(3, 16), (5, 128)])
def test_layer_norm_forward_row_reference_shapes(shape, dt):
    """Statistics in X's dtype as in the enriched reference case."""
    x, w, b = lnrow_case(*shape, dt)
    y, mean, rstd = run_lnrow(x, w, b, dt, dt)
    ey, em, es = ref.layernorm_row(x, w, b, 1e-5)
    rtol, atol = RED_BAR[dt]
    if dt == "float32":
        rel_close(y, ey, 1e-5, 1e-3)
        rel_close(mean, em, 1e-5, 1e-3)
        rel_close(rstd, es, 1e-5, 1e-30)
    else:
        close(y, ey, rtol, atol)
        close(mean, em, rtol, atol)
        close(rstd, es, rtol, atol)


def test_layer_norm_forward_row_c2_scale():
    """C2's x (bf16 [8191, 3000], +-60 outliers), gamma and beta through the
    row form; fp32 statistics (<= 1e-5 relative; Mean also 1e-6 absolute,
    rows of +-60 outliers cancel to ~0.05), Y <= 1e-2."""
    c = inputs.config2()
    y, mean, rstd = run_lnrow(c["x"], c["gamma"], c["beta"], "bfloat16", "float32")
    ey, em, es = ref.layernorm_row(c["x"], c["gamma"], c["beta"], 1e-5)
    rows = np.unique(np.r_[0, 8190, np.random.default_rng(5).integers(0, 8191, 256)])
    close(y[rows], ey[rows], 1e-2, 1e-2)
    assert np.all(np.abs(mean - em) <= np.maximum(1e-5 * np.abs(em), 1e-6))
    rel_close(rstd, es, 1e-5, 1e-30)


def test_layer_norm_forward_row_strided_rows_and_odd_width():
    """Row strides wider than n_cols (padding between rows left untouched) and
    a row width that is not a whole 16-byte vector."""
    rows, cols, stride = 7, 67, 80
    x, w, b = lnrow_case(rows, cols, "float16", seed=9)
    xp = np.zeros((rows, stride), np.float32)
    xp[:, :cols] = x
    y = torch.full((rows * stride,), -7.0, dtype=torch.float16, device=DEV)
    mean = torch.full((rows * 2,), -7.0, dtype=torch.float32, device=DEV)
    rstd = torch.full((rows * 3,), -7.0, dtype=torch.float32, device=DEV)
    ops._layer_norm_forward_row(y, stride, dev(xp, "float16"), stride, dev(w, "float16"), dev(b, "float16"), mean,
                                2, rstd, 3, rows, cols, 1e-5, sync=True)
    ey, em, es = ref.layernorm_row(x, w, b, 1e-5)
    got = host(y).reshape(rows, stride)
    close(got[:, :cols], ey, 1e-2, 1e-2)
    assert np.all(got[:, cols:] == -7.0)
    rel_close(host(mean)[::2], em, 1e-5, 1e-3)
    rel_close(host(rstd)[::3], es, 1e-5, 1e-30)
    assert np.all(host(mean)[1::2] == -7.0) and np.all(host(rstd)[1::3] == -7.0)


# --------------------------------------------------------------- gqa_kernel
def run_gqa(q, k, v, dt, group, scale=None):
    z, hq, n, d = q.shape
    hkv = k.shape[1]
    scale = 1.0 / np.sqrt(d) if scale is None else scale
    qd, kd, vd = dev(q, dt), dev(k, dt), dev(v, dt)
    out = torch.zeros(q.shape, dtype=TD[dt], device=DEV)
    ops.gqa_kernel(qd, kd, vd, out, n * d, d, 1, n * d, d, 1, n * d, d, 1, n * d, d, 1, hq, hkv, n,
                   np.float32(scale), group, d, 32, sync=True)
    return out, [host(t) for t in (qd, kd, vd)], scale


@pytest.mark.parametrize("dt", DTYPES)
@pytest.mark.parametrize("shape", [(2, 4, 2, 32, 32), (2, 4, 2, 64, 32), (1, 4, 2, 64, 32)])
def test_gqa_kernel_reference_shapes(shape, dt):
    """The reference case: Q, K, V ~ N(0, 1), scale 1/sqrt(d), GROUP = Hq/Hkv;
    bar = the case's allclose 2e-2 (gqa.py:100-101)."""
    z, hq, hkv, n, d = shape
    rng = np.random.default_rng(30)
    q = rounded(rng.standard_normal((z, hq, n, d)), dt)
    k = rounded(rng.standard_normal((z, hkv, n, d)), dt)
    v = rounded(rng.standard_normal((z, hkv, n, d)), dt)
    out, (qh, kh, vh), scale = run_gqa(q, k, v, dt, hq // hkv)
    close(host(out), ref.gqa(qh, kh, vh, scale, hq // hkv), 2e-2, 2e-2)


def test_gqa_kernel_wide_group():
    """GROUP larger than Hq/Hkv sends every query head to KV head 0."""
    rng = np.random.default_rng(31)
    q = rng.standard_normal((2, 4, 40, 32)).astype(np.float32)
    k = rng.standard_normal((2, 2, 40, 32)).astype(np.float32)
    v = rng.standard_normal((2, 2, 40, 32)).astype(np.float32)
    out, (qh, kh, vh), scale = run_gqa(q, k, v, "float32", 4)
    close(host(out), ref.gqa(qh, kh, vh, scale, 4), 2e-2, 2e-2)


@pytest.mark.parametrize("d", [64, 128])
def test_gqa_kernel_mfma_shapes(d):
    """16-bit GQA with d in {64, 128} takes the MFMA kernel (non-causal)."""
    c = inputs.config4(2, 8, 2, 700, d)
    out, (qh, kh, vh), scale = run_gqa(c["q"], c["k"], c["v"], "bfloat16", 4)
    assert rt.module().last_kernel == f"g950_attn_fwd_bf16_d{d}"
    close(host(out), ref.gqa(qh, kh, vh, scale, 4), 2e-2, 2e-2)


def test_gqa_kernel_c4_scale():
    """C4's inputs (bf16 [4, 32, 4096, 128], 8 KV heads) through gqa_kernel
    (non-causal): one query head of every (batch, KV group) checked in full."""
    c = inputs.config4()
    out, _, scale = run_gqa(c["q"], c["k"], c["v"], "bfloat16", 4)
    assert rt.module().last_kernel == "g950_attn_fwd_bf16_d128"
    rng = np.random.default_rng(6)
    for z in range(4):
        for g in range(8):
            h = 4 * g + int(rng.integers(0, 4))
            eo = ref.gqa(c["q"][z:z + 1, h:h + 1], c["k"][z:z + 1, g:g + 1], c["v"][z:z + 1, g:g + 1], scale, 1)
            close(host(out[z, h]), eo[0, 0], 2e-2, 2e-2)


# ------------------------------------------------- dev contracts, random
def test_dev_contracts_random_sweep():
    """Twenty-four seeded cases over the three dev-suite signatures, the
    three dtypes in turn: softmax_kernel_inner with M rows of N in 1..5000
    elements, TILE_N a power of two and ONE_TILE_PER_CTA either way (a
    narrow one-tile case leaves the tail of each output row as it was);
    _layer_norm_forward_row with 1..300 rows of 1..5000 (any width, so
    aligned and masked rows) and statistics in X's dtype; gqa_kernel with
    1-2 batches, GROUP 1/2/4, N_CTX 1..300 and head dim 32/64/128.  Bars as
    in the fixed-shape tests above."""
    rng = np.random.default_rng(2718)
    for case in range(24):
        dt = DTYPES[case % 3]
        kind = (case // 3) % 3
        rtol, atol = RED_BAR[dt]
        if kind == 0:
            m, n = int(rng.integers(1, 51)), int(rng.integers(1, 5001))
            tile = 1 << int(rng.integers(4, 13))
            one = bool(rng.random() < 0.5)
            tag = f"case {case}: softmax_kernel_inner {dt} M {m} N {n} TILE_N {tile} one_tile {one}"
            x = rounded(rng.normal(0, 2.0, m * n), dt)
            before = np.full(m * n + 16, -7.0)
            out = torch.full((m * n + 16,), -7.0, dtype=TD[dt], device=DEV)
            ops.softmax_kernel_inner(out, dev(x, dt), m, n, tile, one, sync=True)
            got = host(out)
            expect = ref.softmax_inner(x, m, n, tile, one, out=before)
            ok, err = ref.isclose_verdict(got[: m * n], expect, rtol, atol)
            assert ok, f"{tag}: max abs err {err}"
            assert np.all(got[m * n:] == -7.0), tag
        elif kind == 1:
            rows, cols = int(rng.integers(1, 301)), int(rng.integers(1, 5001))
            tag = f"case {case}: _layer_norm_forward_row {dt} rows {rows} cols {cols}"
            x, w, b = lnrow_case(rows, cols, dt, seed=3000 + case)
            yd = torch.full((rows * cols,), -7.0, dtype=TD[dt], device=DEV)
            md = torch.full((rows,), -7.0, dtype=TD[dt], device=DEV)
            sd = torch.full((rows,), -7.0, dtype=TD[dt], device=DEV)
            ops._layer_norm_forward_row(yd, cols, dev(x, dt), cols, dev(w, dt), dev(b, dt), md, 1, sd, 1, rows,
                                        cols, 1e-5, cols, sync=True)
            tag += f" ({rt.module().last_kernel})"
            y, mean, rstd = host(yd).reshape(rows, cols), host(md), host(sd)
            ey, em, es = ref.layernorm_row(x, w, b, 1e-5)
            if dt == "float32":
                # y = (x - mean) * rstd * w + b: where the two terms nearly
                # cancel, fp32 rounding of each (~3e-8 near 0.5) is all that
                # is left, so y takes the isclose form with atol 1e-6 (an fp32
                # emulation of the same arithmetic reaches 3.6e-5 relative at
                # |y| = 4e-4 on case 3); the statistics stay relative
                ok, err = ref.isclose_verdict(y, ey, 1e-5, 1e-6)
                assert ok, f"{tag}: y max abs err {err}"
                for what, got, want, floor in (("mean", mean, em, 1e-3), ("rstd", rstd, es, 1e-30)):
                    a, e = np.asarray(got, np.float64), np.asarray(want, np.float64)
                    err = float((np.abs(a - e) / np.maximum(np.abs(e), floor)).max())
                    assert err <= 1e-5, f"{tag}: {what} relative error {err}"
            else:
                for what, got, want in (("y", y, ey), ("mean", mean, em), ("rstd", rstd, es)):
                    ok, err = ref.isclose_verdict(got, want, rtol, atol)
                    assert ok, f"{tag}: {what} max abs err {err}"
        else:
            z, hkv = int(rng.integers(1, 3)), int(rng.integers(1, 3))
            group = (1, 2, 4)[int(rng.integers(0, 3))]
            n, d = int(rng.integers(1, 301)), (32, 64, 128)[int(rng.integers(0, 3))]
            hq = hkv * group
            tag = f"case {case}: gqa_kernel {dt} z {z} heads {hq}/{hkv} n {n} d {d}"
            q = rounded(rng.standard_normal((z, hq, n, d)), dt)
            k = rounded(rng.standard_normal((z, hkv, n, d)), dt)
            v = rounded(rng.standard_normal((z, hkv, n, d)), dt)
            out, (qh, kh, vh), scale = run_gqa(q, k, v, dt, group)
            ok, err = ref.isclose_verdict(host(out), ref.gqa(qh, kh, vh, scale, group), 2e-2, 2e-2)
            assert ok, f"{tag}: max abs err {err}"


# ------------------------------------------------ int8 signedness variants
PAIRS = [("int8", "int8"), ("uint8", "uint8"), ("uint8", "int8"), ("int8", "uint8")]
SHORT = {("int8", "int8"): "i8", ("uint8", "int8"): "u8s8", ("int8", "uint8"): "s8u8", ("uint8", "uint8"): "u8u8"}


def draw(rng, dt, shape):
    lo, hi = (0, 256) if dt == "uint8" else (-128, 128)
    return rng.integers(lo, hi, shape).astype(dt)


@pytest.mark.parametrize("adt,bdt", PAIRS)
@pytest.mark.parametrize("m,n,k", [(300, 260, 256), (33, 65, 128), (4096, 8192, 8192)])
def test_int8_signedness_exact(adt, bdt, m, n, k):
    """Every pair of a100c/plan/tiles.py:121-126 on the MFMA kernel (K-contiguous
    B), int32 bit-exact against the integer product narrowed as the reference
    narrows it; the dequant epilogue at the GEMM bar."""
    rng = np.random.default_rng(m + n + k)
    a = draw(rng, adt, (m, k))
    bt = draw(rng, bdt, (n, k))
    ad, btd = torch.from_numpy(a).to(DEV), torch.from_numpy(bt).to(DEV)
    acc = torch.empty((m, n), dtype=torch.int32, device=DEV)
    ops.matmul_i8_kernel(ad, btd.t(), acc, m, n, k, sync=True)
    assert rt.module().last_kernel == f"g950_gemm_{SHORT[(adt, bdt)]}_256x256"
    rows = np.arange(m) if m <= 512 else np.unique(
        np.r_[[t + int(rng.integers(0, 256)) for t in range(0, m, 256)], 0, m - 1])
    exact = ref.wrap_i32(ref.matmul_i8(a[rows], bt.T))
    assert np.array_equal(acc[torch.from_numpy(rows).to(DEV)].cpu().numpy(), exact)
    sa = (rng.random(m) * 0.019 + 0.001).astype(np.float32)
    sb = (rng.random(n) * 0.019 + 0.001).astype(np.float32)
    y = torch.empty((m, n), dtype=torch.bfloat16, device=DEV)
    ops.matmul_i8_dequant_kernel(ad, btd.t(), torch.from_numpy(sa).to(DEV), torch.from_numpy(sb).to(DEV), y,
                                 m, n, k, sync=True)
    close(host(y[torch.from_numpy(rows).to(DEV)]), ref.dequant(exact, sa[rows], sb), 2e-2, 2e-2)


def test_int8_unsigned_worst_magnitude():
    """u8 x u8 at K = 8192 with every byte 255: each sum is 255^2 * 8192 =
    532,684,800, inside int32 -- the largest magnitude the corrections meet."""
    m, n, k = 256, 256, 8192
    a = torch.full((m, k), 255, dtype=torch.uint8, device=DEV)
    bt = torch.full((n, k), 255, dtype=torch.uint8, device=DEV)
    acc = torch.empty((m, n), dtype=torch.int32, device=DEV)
    ops.matmul_i8_kernel(a, bt.t(), acc, m, n, k, sync=True)
    assert rt.module().last_kernel == "g950_gemm_u8u8_256x256"
    assert bool((acc == 255 * 255 * 8192).all())
    # mixed extremes: uint8 255 x int8 -128
    b2 = torch.full((n, k), -128, dtype=torch.int8, device=DEV)
    ops.matmul_i8_kernel(a, b2.t(), acc, m, n, k, sync=True)
    assert bool((acc == -255 * 128 * 8192).all())


@pytest.mark.parametrize("adt,bdt", PAIRS)
def test_int8_signedness_general_path(adt, bdt):
    """Row-major B and a K that is not a slab multiple: the general kernel."""
    rng = np.random.default_rng(7)
    a = draw(rng, adt, (37, 100))
    b = draw(rng, bdt, (100, 45))
    acc = torch.empty((37, 45), dtype=torch.int32, device=DEV)
    ops.matmul_i8_kernel(torch.from_numpy(a).to(DEV), torch.from_numpy(b).to(DEV), acc, 37, 45, 100, sync=True)
    assert rt.module().last_kernel == "g950_gemm_general_i8"
    assert np.array_equal(acc.cpu().numpy(), ref.wrap_i32(ref.matmul_i8(a, b)))


def test_int8_random_shapes_sweep():
    """Sixteen seeded int8 GEMMs: a random signedness pair each, M and N in
    1..1300, K a multiple of 16 in 16..2048 (whole 128-byte slabs or a K
    tail), K-contiguous or row-major B; every int32 element bit-exact against
    the integer product narrowed modulo 2^32, with both the MFMA kernels and
    the general kernel reached."""
    rng = np.random.default_rng(8128)
    ran = set()
    for case in range(16):
        adt, bdt = PAIRS[case % 4]
        m, n = (int(v) for v in rng.integers(1, 1301, 2))
        k = 16 * int(rng.integers(1, 129))
        colb = bool(rng.random() < 0.75)
        a = draw(rng, adt, (m, k))
        b = draw(rng, bdt, (k, n))
        ad = torch.from_numpy(a).to(DEV)
        bd = torch.from_numpy(np.ascontiguousarray(b.T)).to(DEV).t() if colb else torch.from_numpy(b).to(DEV)
        acc = torch.full((m, n), -7, dtype=torch.int32, device=DEV)
        ops.matmul_i8_kernel(ad, bd, acc, m, n, k, sync=True)
        ran.add(rt.module().last_kernel)
        tag = f"case {case}: {adt} x {bdt} m {m} n {n} k {k} {'K-contiguous' if colb else 'row-major'} B"
        exact = ref.wrap_i32(ref.matmul_i8(a, b))
        assert np.array_equal(acc.cpu().numpy(), exact), f"{tag}: {rt.module().last_kernel}"
    assert any(k.endswith("_256x256") or k.endswith("_256x256_kt") for k in ran), sorted(ran)
    assert "g950_gemm_general_i8" in ran, sorted(ran)


# ------------------------------------------- W8A16 widened-route edge cases
@pytest.mark.parametrize("n,ydt", [(8003, "bfloat16"), (8192, "float32")])
def test_dequant_matmul_widened_ragged_n_and_fp32_out(n, ydt):
    """The widened route (B copied once to bf16, 256x256 GEMM with the column
    scale in its epilogue) with N not a multiple of 256 (and of 4), and with a
    float32 output: the epilogue's column guard, the B row clamp and the fp32
    store."""
    m, k = 1100, 128
    rng = np.random.default_rng(n)
    a = rounded(rng.standard_normal((m, k)) * 0.5, "bfloat16")
    b = rng.integers(-127, 128, (k, n)).astype(np.int8)
    s = rounded(rng.random(n) / 64, "bfloat16")
    ad, sd = dev(a, "bfloat16"), dev(s, "bfloat16")
    bt = torch.from_numpy(np.ascontiguousarray(b.T)).to(DEV)
    y = torch.full((m, n), -7.0, dtype=TD[ydt], device=DEV)
    ops.dequant_matmul_kernel(ad, bt.t(), sd, y, m, n, k, sync=True)
    assert rt.module().last_kernel == "g950_gemm_bf16_256x256"
    rows = np.unique(np.r_[0, 255, 256, m - 1, rng.integers(0, m, 32)])
    expect = ref.matmul(a[rows], ref.dequantize(b, s))
    close(host(y)[rows], expect, 2e-2, 2e-2)


def test_dequant_matmul_k0_writes_zeros():
    """K = 0 with many output tiles: the zero product, from a kernel that reads
    nothing of the empty operands."""
    m, n = 4096, 4096
    a = torch.empty((m, 0), dtype=torch.bfloat16, device=DEV)
    bt = torch.empty((n, 0), dtype=torch.int8, device=DEV)
    s = torch.ones(n, dtype=torch.bfloat16, device=DEV)
    y = torch.full((m, n), -7.0, dtype=torch.bfloat16, device=DEV)
    ops.dequant_matmul_kernel(a, bt.t(), s, y, m, n, 0, sync=True)
    assert rt.module().last_kernel != "g950_gemm_bf16_256x256"
    assert bool((y == 0).all())
