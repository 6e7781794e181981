"""Pin the CPU oracle against the reference's held post-run fixtures.

Each fixture is the reference's own compiled operator output for a seeded case
(tests/golden/make_fixtures.py).  The oracle must agree with it to the
reference comparator's tolerance for the fixture dtype
(ops/harness/opslib/case.py:153-157), and a planted mistake in the oracle must
fail the same check.
"""
import numpy as np
import pytest

from oracle import reference as ref
from tests._fixtures import dtype_of, golden_cases, load, values


def _check(actual, expected, dtype):
    rtol, atol = ref.TOLERANCES[dtype]
    ok, err = ref.isclose_verdict(actual, expected, rtol, atol)
    return ok, err


@pytest.mark.parametrize("case", golden_cases("softmax"))
def test_softmax_oracle_matches_fixture(case):
    b = load(case)
    x = values(b, "x_ptr")
    y = values(b, "y_ptr")
    assert b.scalar("n_cols") == x.shape[1]
    ok, err = _check(ref.softmax(x), y, dtype_of(case))
    assert ok, err
    # planted mistake: dropping the max-subtraction is harmless, dropping the
    # normalisation is not -- the check must see it
    bad = np.exp(x.astype(np.float64))
    assert not _check(bad, y, dtype_of(case))[0]


@pytest.mark.parametrize("case", golden_cases("matmul"))
def test_matmul_oracle_matches_fixture(case):
    b = load(case)
    a = values(b, "a_ptr")
    bb = values(b, "b_ptr")
    y = values(b, "y_ptr")
    m, k = a.shape
    n = bb.shape[1]
    assert (b.scalar("M"), b.scalar("N"), b.scalar("K")) == (m, n, k)
    ok, err = _check(ref.matmul(a, bb), y, dtype_of(case))
    assert ok, err
    # planted mistake: a transposed operand must fail (square cases) or a
    # dropped K block must fail (all cases)
    if k > 8:
        dropped = ref.matmul(a[:, : k - 8], bb[: k - 8])
        assert not _check(dropped, y, dtype_of(case))[0]


@pytest.mark.parametrize("case", golden_cases("attention"))
def test_attention_oracle_matches_fixture(case):
    b = load(case)
    q, k, v, out = (values(b, n) for n in ("q_ptr", "k_ptr", "v_ptr", "out_ptr"))
    scale = b.scalar("scale")
    assert b.scalar("N_CTX") == q.shape[2]
    o, lse = ref.attention(q, k, v, scale, causal=False)
    ok, err = _check(o, out, dtype_of(case))
    assert ok, err
    # planted mistake: the fixtures are non-causal, so a causal oracle must fail
    oc, _ = ref.attention(q, k, v, scale, causal=True)
    assert not _check(oc, out, dtype_of(case))[0]
