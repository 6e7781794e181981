"""Seeded random shapes through every operator family, against the CPU oracle
(the bars of tests/test_gpu_parity.py): odd extents, strided rows and the
kernel-selection boundaries (register configurations, split rows, MFMA vs
general GEMM, attention block edges) that fixed-shape tests can miss."""
import numpy as np
import pytest

torch = pytest.importorskip("torch")

from compiler_amd import operators as ops  # noqa: E402
from oracle import reference as ref  # noqa: E402

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
TD = {"float32": torch.float32, "bfloat16": torch.bfloat16, "float16": torch.float16}


def dev(a, dt):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(DEV).to(TD[dt])


def host(t):
    return t.float().cpu().numpy()


def close(a, e, rtol, atol):
    ok, err = ref.isclose_verdict(a, e, rtol, atol)
    assert ok, f"max abs err {err} (rtol {rtol}, atol {atol})"


@pytest.mark.parametrize("seed", range(12))
def test_row_reductions_random(seed):
    rng = np.random.default_rng(1000 + seed)
    rows = int(rng.choice([1, 2, 3, 7, 63, 64, 65, 257, 1000]))
    cols = int(rng.choice([1, 5, 8, 63, 64, 65, 511, 512, 513, 1024, 4095, 4096, 4097, 8191, 33000, 70001]))
    dt = str(rng.choice(["float32", "bfloat16", "float16"]))
    pad = int(rng.choice([0, 8, 13]))       # padded rows: strided views
    x = (rng.standard_normal((rows, cols + pad)) * 2.0).astype(np.float32)
    xd = dev(x, dt)[:, :cols]
    xr = host(xd)
    rtol, atol = (1e-5, 1e-6) if dt == "float32" else ref.TOLERANCES[dt]
    close(host(ops.softmax(xd, sync=True)), ref.softmax(xr), rtol, atol)
    close(host(ops.logsumexp(xd, sync=True)), ref.logsumexp(xr), 3e-5, 3e-6)
    w = (rng.random(cols) + 0.5).astype(np.float32)
    b = (rng.standard_normal(cols) * 0.1).astype(np.float32)
    wd, bd = dev(w, dt), dev(b, dt)
    y, r = ops.rmsnorm(xd, wd, 1e-5, sync=True)
    ey, er = ref.rms_layernorm(xr, host(wd), 1e-5)
    close(host(y), ey, max(rtol, 1e-5), max(atol, 1e-5))
    close(host(r), er, 1e-5, 1e-6)
    # layernorm_kernel takes one row stride for X and Y: Y shares X's padding
    yl = torch.empty((rows, cols + pad), dtype=TD[dt], device=DEV)[:, :cols]
    y, mean, rstd = ops.layernorm(xd, wd, bd, 1e-5, out=yl, sync=True)
    ey, em, es = ref.layernorm(xr, host(wd), host(bd), 1e-5)
    close(host(y), ey, max(rtol, 1e-4), max(atol, 1e-4))
    close(host(mean), em, 1e-5, 1e-6)
    close(host(rstd), es, 1e-5, 1e-6)


@pytest.mark.parametrize("seed", range(10))
def test_gemm_random(seed):
    rng = np.random.default_rng(2000 + seed)
    m = int(rng.choice([1, 31, 255, 256, 257, 700]))
    n = int(rng.choice([1, 33, 255, 256, 257, 600]))
    k = int(rng.choice([16, 64, 128, 192, 320, 1000, 1024]))
    dt = str(rng.choice(["bfloat16", "float16", "float32"]))
    a = (rng.standard_normal((m, k)) * k ** -0.25).astype(np.float32)
    bt = (rng.standard_normal((n, k)) * k ** -0.25).astype(np.float32)
    ad, btd = dev(a, dt), dev(bt, dt)
    col_major = bool(rng.integers(0, 2))
    bop = btd.t() if col_major else btd.t().contiguous()
    y = ops.matmul(ad, bop, sync=True)
    bar = 1e-4 if dt == "float32" else 2e-2
    close(host(y), ref.matmul(host(ad), host(btd).T), bar, bar)


@pytest.mark.parametrize("seed", range(8))
def test_int8_and_w8a16_random(seed):
    rng = np.random.default_rng(3000 + seed)
    m = int(rng.choice([1, 16, 100, 256, 300]))
    n = int(rng.choice([16, 64, 200, 256, 1000]))
    k = int(rng.choice([128, 256, 640, 1024, 2048]))
    a = rng.integers(-127, 128, (m, k)).astype(np.int8)
    bt = rng.integers(-127, 128, (n, k)).astype(np.int8)
    c = torch.empty((m, n), dtype=torch.int32, device=DEV)
    ops.matmul_i8_kernel(torch.from_numpy(a).to(DEV), torch.from_numpy(bt).to(DEV).t(), c, m, n, k, sync=True)
    assert np.array_equal(c.cpu().numpy().astype(np.int64), ref.matmul_i8(a, bt.T))
    af = (rng.standard_normal((m, k)) * 0.5).astype(np.float32)
    s = (rng.random(n) / 64).astype(np.float32)
    ad, sd = dev(af, "bfloat16"), dev(s, "bfloat16")
    y = ops.dequant_matmul(ad, torch.from_numpy(bt).to(DEV).t(), sd, sync=True)
    close(host(y), ref.matmul(host(ad), ref.dequantize(bt.T, host(sd))), 2e-2, 2e-2)


@pytest.mark.parametrize("seed", range(8))
def test_attention_random(seed):
    rng = np.random.default_rng(4000 + seed)
    z = int(rng.choice([1, 2]))
    hkv = int(rng.choice([1, 2]))
    hq = hkv * int(rng.choice([1, 2, 4]))
    s = int(rng.choice([1, 63, 64, 65, 255, 256, 257, 700]))
    d = int(rng.choice([64, 128]))
    causal = bool(rng.integers(0, 2))
    dt = str(rng.choice(["bfloat16", "float16"]))
    q = rng.standard_normal((z, hq, s, d)).astype(np.float32)
    k = rng.standard_normal((z, hkv, s, d)).astype(np.float32)
    v = rng.standard_normal((z, hkv, s, d)).astype(np.float32)
    qd, kd, vd = dev(q, dt), dev(k, dt), dev(v, dt)
    o = torch.empty_like(qd)
    lse = torch.empty((z, hq, s), dtype=torch.float32, device=DEV)
    scale = 1.0 / np.sqrt(d)
    ops.attn_fwd_causal_kernel(qd, kd, vd, o, z, hq, s, np.float32(scale), *qd.stride(), *kd.stride(),
                               *vd.stride(), *o.stride(), CAUSAL=causal, lse_ptr=lse, sync=True)
    eo, el = ref.attention(host(qd), host(kd), host(vd), scale, causal=causal)
    close(host(o), eo, 2e-2, 2e-2)
    close(lse.cpu().numpy(), el, 1e-4, 1e-4)
