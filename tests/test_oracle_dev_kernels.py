"""Pins of the oracle functions behind the dev-suite kernel signatures
(softmax_kernel_inner, _layer_norm_forward_row, gqa_kernel) and the unsigned
and mixed-sign int8 dot: closed forms, brute force on tiny inputs, and a
planted mistake in each that must fail (planted in the oracle, on the CPU)."""
import math

import numpy as np
import pytest

from oracle import reference as ref


# -------------------------------------------------- _layer_norm_forward_row
def _lnrow_brute(x, w, b, eps):
    y = np.empty_like(x, dtype=np.float64)
    mean = np.empty(x.shape[0])
    rstd = np.empty(x.shape[0])
    for r in range(x.shape[0]):
        row = [float(v) for v in x[r]]
        n = len(row)
        m = sum(row) / n
        msq = sum(v * v for v in row) / n
        s = 1.0 / math.sqrt(msq - m * m + eps)
        mean[r], rstd[r] = m, s
        for c in range(n):
            y[r, c] = (row[c] - m) * s * float(w[c]) + float(b[c])
    return y, mean, rstd


def test_layernorm_row_brute_force_and_closed_forms():
    rng = np.random.default_rng(11)
    x = rng.normal(0, 0.7, (5, 128))
    w = rng.uniform(0.7, 1.3, 128)
    b = rng.normal(0, 0.1, 128)
    got = ref.layernorm_row(x, w, b, 1e-5)
    want = _lnrow_brute(x, w, b, 1e-5)
    for g, e in zip(got, want):
        assert np.allclose(g, e, rtol=1e-12, atol=1e-12)
    # constant row c: mean c, rstd 1/sqrt(eps), Y = B exactly
    y, mean, rstd = ref.layernorm_row(np.full((2, 16), 3.0), w[:16], b[:16], 1e-5)
    assert np.allclose(mean, 3.0) and np.allclose(rstd, 1 / math.sqrt(1e-5)) and np.allclose(y, b[:16][None, :])
    # E[x^2] - mean^2 == var on well-conditioned rows: equals the centered form
    got_c = ref.layernorm(x, w, b, 1e-5)
    for g, e in zip(got, got_c):
        assert np.allclose(g, e, rtol=1e-10, atol=1e-10)


def test_layernorm_row_planted_mistake_fails():
    rng = np.random.default_rng(12)
    x = rng.normal(1.5, 0.7, (3, 16))   # nonzero mean: the mean^2 term matters
    w, b = np.ones(16), np.zeros(16)
    y, mean, rstd = ref.layernorm_row(x, w, b, 1e-5)
    planted = 1.0 / np.sqrt((x * x).mean(1) + 1e-5)      # mean^2 dropped
    assert not np.allclose(planted, rstd, rtol=1e-2)
    assert np.allclose(rstd, _lnrow_brute(x, w, b, 1e-5)[2], rtol=1e-12)


# ---------------------------------------------------- softmax_kernel_inner
def test_softmax_inner_rows_of_flat_buffer():
    rng = np.random.default_rng(13)
    m, n = 3, 32                           # the reference case shape (97,): M=3, C=32
    flat = rng.normal(0, 0.8, m * n + 5)   # trailing elements beyond M*N are not part of it
    got = ref.softmax_inner(flat, m, n)
    assert got.shape == (m * n,)
    for r in range(m):
        row = flat[r * n:(r + 1) * n]
        bf = [math.exp(v) / sum(math.exp(u) for u in row) for v in row]
        assert np.allclose(got[r * n:(r + 1) * n], bf, atol=1e-15)
    # a transposed reading (column-major rows) must differ
    planted = ref.softmax(flat[: m * n].reshape(n, m).T).reshape(-1)
    assert not np.allclose(planted, got, atol=1e-3)


def test_softmax_inner_one_narrow_tile():
    # ONE_TILE_PER_CTA with TILE_N < N (softmax_kernel_inner.py:13-24): the
    # first TILE_N elements of each row normalised among themselves, the
    # rest of the output row as it was
    rng = np.random.default_rng(14)
    m, n, tile = 3, 32, 8
    flat = rng.normal(0, 0.8, m * n)
    before = rng.normal(0, 1.0, m * n)
    got = ref.softmax_inner(flat, m, n, tile, True, out=before)
    for r in range(m):
        row = flat[r * n:r * n + tile]
        bf = [math.exp(v) / sum(math.exp(u) for u in row) for v in row]
        assert np.allclose(got[r * n:r * n + tile], bf, atol=1e-15)
        assert np.array_equal(got[r * n + tile:(r + 1) * n], before[r * n + tile:(r + 1) * n])
    # a whole-row normalisation (the looped form) gives other values on the tile
    assert not np.allclose(got.reshape(m, n)[:, :tile], ref.softmax_inner(flat, m, n).reshape(m, n)[:, :tile])
    # a tile as wide as the row, or the looped form, is the plain row softmax
    for t, one in ((32, True), (64, True), (8, False)):
        assert np.array_equal(ref.softmax_inner(flat, m, n, t, one, out=before), ref.softmax_inner(flat, m, n))


# -------------------------------------------------------------- gqa_kernel
def _gqa_brute(q, k, v, scale, group):
    z, hq, n, d = q.shape
    out = np.zeros((z, hq, n, d))
    for zz in range(z):
        for h in range(hq):
            kv = h // group
            for i in range(n):
                s = [scale * sum(float(q[zz, h, i, e]) * float(k[zz, kv, j, e]) for e in range(d)) for j in range(n)]
                m = max(s)
                p = [math.exp(x - m) for x in s]
                tot = sum(p)
                for e in range(d):
                    out[zz, h, i, e] = sum(p[j] * float(v[zz, kv, j, e]) for j in range(n)) / tot
    return out


def test_gqa_brute_force_and_group_map():
    rng = np.random.default_rng(14)
    q = rng.standard_normal((2, 4, 6, 4))
    k = rng.standard_normal((2, 2, 6, 4))
    v = rng.standard_normal((2, 2, 6, 4))
    for group in (2, 4):                  # Hq/Hkv, and every head on KV head 0
        got = ref.gqa(q, k, v, 0.5, group)
        assert np.allclose(got, _gqa_brute(q, k, v, 0.5, group), atol=1e-13)
    # group = Hq/Hkv is the non-causal attention
    assert np.allclose(ref.gqa(q, k, v, 0.5, 2), ref.attention(q, k, v, 0.5, causal=False)[0], atol=1e-14)
    # a swapped head map (h % Hkv instead of h // group) fails
    planted = np.stack([np.stack([ref.attention(q[zz:zz + 1, h:h + 1], k[zz:zz + 1, h % 2:h % 2 + 1],
                                                v[zz:zz + 1, h % 2:h % 2 + 1], 0.5, causal=False)[0][0, 0]
                                  for h in range(4)]) for zz in range(2)])
    assert not np.allclose(planted, ref.gqa(q, k, v, 0.5, 2), atol=1e-3)
    # uniform V: every output row is that V row
    vu = np.broadcast_to(rng.standard_normal(4), (2, 2, 6, 4))
    assert np.allclose(ref.gqa(q, k, vu, 0.5, 2), vu[:, :1].repeat(4, axis=1), atol=1e-14)
    with pytest.raises(ValueError):
        ref.gqa(q, k, v, 0.5, 1)          # head 2 would read KV head 2 of 2


# ------------------------------------------------- int8 signedness variants
@pytest.mark.parametrize("adt,bdt", [(np.int8, np.int8), (np.uint8, np.uint8), (np.uint8, np.int8),
                                     (np.int8, np.uint8)])
def test_matmul_i8_signedness_brute_force(adt, bdt):
    rng = np.random.default_rng(15)
    lo = lambda dt: 0 if dt == np.uint8 else -128   # noqa: E731
    hi = lambda dt: 256 if dt == np.uint8 else 128  # noqa: E731
    a = rng.integers(lo(adt), hi(adt), (5, 37)).astype(adt)
    b = rng.integers(lo(bdt), hi(bdt), (37, 6)).astype(bdt)
    got = ref.matmul_i8(a, b)
    for i in range(5):
        for j in range(6):
            assert got[i, j] == sum(int(a[i, kk]) * int(b[kk, j]) for kk in range(37))
    # reading an unsigned operand as signed bits gives a different result
    if adt == np.uint8 and (a >= 128).any():
        assert not np.array_equal(ref.matmul_i8(a.view(np.int8), b), got)


def test_wrap_i32_and_worst_case_bounds():
    # u8 x u8 worst case at K = 8192 stays inside int32; one more 255*255 term per step wraps
    assert 255 * 255 * 8192 < 2 ** 31
    a = np.full((1, 8192), 255, np.uint8)
    assert ref.wrap_i32(ref.matmul_i8(a, a.T))[0, 0] == 255 * 255 * 8192
    big = np.array([[2 ** 31 + 5, -(2 ** 31) - 1]], dtype=np.int64)
    assert ref.wrap_i32(big).tolist() == [[-(2 ** 31) + 5, 2 ** 31 - 1]]
