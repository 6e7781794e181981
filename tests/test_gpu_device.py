"""The harness Device protocol (ops/harness/opslib/device.py:79-118) driven the
way the reference's case loop drives it: alloc / upload, a launch with the
kernel object and positional arguments bound by its signature, download.

The kernel objects here are plain functions carrying the reference kernels'
names and parameter lists (ops/suite/perf/softmax.py, logsumexp.py); the
device dispatches on the name, so these stand in for the Triton JIT objects.
"""
import numpy as np
import pytest

torch = pytest.importorskip("torch")

from compiler_amd import runtime as rt  # noqa: E402
from compiler_amd.device import G950Device  # noqa: E402
from oracle import reference as ref  # noqa: E402

pytestmark = pytest.mark.gpu


def softmax_kernel(x_ptr, y_ptr, n_cols, BLOCK_SIZE):  # noqa: N803 - reference names
    raise AssertionError("dispatched by name, never called")


def logsumexp_kernel(x_ptr, y_ptr, n_cols, BLOCK_N):  # noqa: N803
    raise AssertionError("dispatched by name, never called")


def _dequantize_kernel(b_ptr, b_scale_ptr, fpb_ptr, K, N, stride_bk, stride_bn, stride_fpbk,  # noqa: N803
                       stride_fpbn, BLOCK_K, BLOCK_N):
    raise AssertionError("dispatched by name, never called")


class _Config:
    kwargs = {"BLOCK_K": 32, "BLOCK_N": 32}


class _Autotuned:
    """The shape of a triton Autotuner: .fn is the kernel, .configs its tuning
    space; bind_arguments leaves the tuned constexprs out of the positionals."""
    fn = staticmethod(_dequantize_kernel)
    configs = [_Config()]


_dequantize_kernel.__name__ = "dequantize_kernel"


def gelu_kernel(x_ptr, y_ptr, n):
    raise AssertionError("not a hot-path operator")


def test_device_softmax_float32_and_bf16_duality():
    d = G950Device()
    rng = np.random.default_rng(11)
    x = rng.standard_normal((37, 97)).astype(np.float32)
    for dt in ("float32", "bfloat16"):
        xb = d.upload(x, dt)
        yb = d.alloc(x.shape, dt)
        d.launch(softmax_kernel, (37,), (xb, yb, 97), {"BLOCK_SIZE": 128})
        y = d.download(yb)
        assert y.dtype == np.float32 and y.shape == x.shape
        xin = ref.bf16_round(x) if dt == "bfloat16" else x
        rtol, atol = ref.TOLERANCES[dt]
        ok, err = ref.isclose_verdict(y, ref.softmax(xin), rtol, atol)
        assert ok, err
    # uint16 host array = raw bf16 bits
    bits = (ref.bf16_round(x).view(np.uint32) >> 16).astype(np.uint16)
    xb = d.upload(bits, "bfloat16")
    assert np.array_equal(d.download(xb), ref.bf16_round(x))


def test_device_logsumexp_reference_case_shape():
    d = G950Device()
    rng = np.random.default_rng(12)
    x = (rng.standard_normal((64, 1024)) * 3.0).astype(np.float32)
    xb, yb = d.upload(x), d.alloc((64,), np.float32)
    d.launch(logsumexp_kernel, (64,), (xb, yb, 1024), {"BLOCK_N": 1024})
    assert rt.module().last_kernel.startswith("g950_rr_logsumexp_f32")
    ok, err = ref.isclose_verdict(d.download(yb), ref.logsumexp(x), 3e-5, 3e-6)
    assert ok, err


def test_device_dequantize_autotuned_kernel():
    """dequantize_matmul.py case (33, 33) in bf16: the autotuned constexprs
    are absent from the positionals, the scalars are numpy int32."""
    d = G950Device()
    rng = np.random.default_rng(13)
    b = rng.integers(-127, 128, (33, 33)).astype(np.int8)
    s = ref.bf16_round(rng.random(33).astype(np.float32))
    bb, sb, yb = d.upload(b), d.upload(s, "bfloat16"), d.alloc((33, 33), "bfloat16")
    i32 = np.int32
    d.launch(_Autotuned(), None, (bb, sb, yb, i32(33), i32(33), i32(33), i32(1), i32(33), i32(1)), {})
    expect = ref.bf16_round(ref.dequantize(b, s).astype(np.float32))
    assert np.array_equal(d.download(yb), expect)


def matmul_kernel(a_ptr, b_ptr, y_ptr, M, N, K):  # noqa: N803 - ops/suite/perf/matmul.py:21
    raise AssertionError("dispatched by name, never called")


def rms_layernorm_forward_kernel(Y, Y_row_stride, X, X_row_stride, W, W_row_stride, r, r_row_stride,  # noqa
                                 n_cols, eps, BLOCK_SIZE):
    raise AssertionError("dispatched by name, never called")


def attention_forward_kernel(q_ptr, k_ptr, v_ptr, out_ptr, Z, H, N_CTX, scale,  # noqa: N803
                             stride_qz, stride_qh, stride_qm, stride_qk, stride_kz, stride_kh, stride_kn,
                             stride_kk, stride_vz, stride_vh, stride_vk, stride_vn, stride_oz, stride_oh,
                             stride_om, stride_on, HEAD_DIM, BLOCK_N, CAUSAL):
    raise AssertionError("dispatched by name, never called")


def _upload_case(d, b, names, dt):
    """Upload a held bundle's views the way stage_case does: bf16 cases as the
    float32 values (rounded on upload), others in their own dtype."""
    from tests._fixtures import values
    out = {}
    for n in names:
        out[n] = d.upload(values(b, n), dt)
    return out


@pytest.mark.parametrize("case", ["matmul16-bfloat16-t1", "matmul128-float16-t1", "matmul-tail-float32-t1"])
def test_device_matmul_on_held_bundles(case):
    """The held post-run matmul bundles driven through the Device protocol:
    outputs match the reference path's own outputs to the dtype's bar."""
    from tests._fixtures import dtype_of, load, values
    d = G950Device()
    b, dt = load(case), dtype_of(case)
    buf = _upload_case(d, b, ("a_ptr", "b_ptr"), dt)
    y = d.alloc(values(b, "y_ptr").shape, dt)
    M, N, K = (int(b.scalar(n)) for n in ("M", "N", "K"))
    d.launch(matmul_kernel, None, (buf["a_ptr"], buf["b_ptr"], y, M, N, K), {})
    rtol, atol = ref.TOLERANCES[dt]
    ok, err = ref.isclose_verdict(d.download(y), values(b, "y_ptr"), rtol, atol)
    assert ok, err


@pytest.mark.parametrize("case", ["attention-bfloat16-t1", "attention-float32-t1"])
def test_device_attention_on_held_bundles(case):
    from tests._fixtures import dtype_of, load, values
    d = G950Device()
    b, dt = load(case), dtype_of(case)
    buf = _upload_case(d, b, ("q_ptr", "k_ptr", "v_ptr"), dt)
    out = d.alloc(values(b, "out_ptr").shape, dt)
    strides = []
    for t in (buf["q_ptr"], buf["k_ptr"], buf["v_ptr"], out):
        strides += list(t.tensor.stride())
    z, h, s, dd = values(b, "q_ptr").shape
    d.launch(attention_forward_kernel, None,
             (buf["q_ptr"], buf["k_ptr"], buf["v_ptr"], out, z, h, s, np.float32(b.scalar("scale")), *strides,
              dd, 16, False), {})
    rtol, atol = ref.TOLERANCES[dt]
    ok, err = ref.isclose_verdict(d.download(out), values(b, "out_ptr"), rtol, atol)
    assert ok, err


def test_device_rms_layernorm_case_shapes():
    """fast_rms_layernorm.py case shapes (4, 64) and (7, 67) in fp32 and bf16."""
    d = G950Device()
    rng = np.random.default_rng(21)
    for dt in ("float32", "bfloat16"):
        for rows, cols in ((4, 64), (7, 67)):
            x = (rng.standard_normal((rows, cols)) * 0.5).astype(np.float32)
            w = (rng.standard_normal(cols) * 0.5 + 1.0).astype(np.float32)
            xb, wb = d.upload(x, dt), d.upload(w, dt)
            yb, rb = d.alloc((rows, cols), dt), d.alloc((rows,), np.float32)
            d.launch(rms_layernorm_forward_kernel, None, (yb, cols, xb, cols, wb, 1, rb, 1, cols, 1e-5, 128), {})
            xin = ref.bf16_round(x) if dt == "bfloat16" else x
            win = ref.bf16_round(w) if dt == "bfloat16" else w
            ey, er = ref.rms_layernorm(xin, win, 1e-5)
            rtol, atol = ref.TOLERANCES[dt]
            ok, err = ref.isclose_verdict(d.download(yb), ey, rtol, atol)
            assert ok, err
            ok, err = ref.isclose_verdict(d.download(rb), er, 1e-5, 1e-6)
            assert ok, err


def test_device_refuses_other_kernels():
    d = G950Device()
    xb, yb = d.upload(np.zeros(8, np.float32)), d.alloc((8,), np.float32)
    with pytest.raises(NotImplementedError):
        d.launch(gelu_kernel, (1,), (xb, yb, 8), {})


# stand-ins with the reference kernels' names and parameter lists
def attn_fwd_causal_kernel(q_ptr, k_ptr, v_ptr, out_ptr, Z, H, N_CTX, scale,  # noqa: N803
                           stride_qz, stride_qh, stride_qm, stride_qk, stride_kz, stride_kh, stride_kn, stride_kk,
                           stride_vz, stride_vh, stride_vk, stride_vn, stride_oz, stride_oh, stride_om, stride_on,
                           BLOCK_M, BLOCK_N, HEAD_DIM, CAUSAL):
    raise AssertionError("dispatched by name, never called")


def softmax_kernel_inner(output_ptr, input_ptr, M, N, TILE_N, ONE_TILE_PER_CTA):  # noqa: N803
    raise AssertionError("dispatched by name, never called")


def _layer_norm_forward_row(Y_ptr, Y_row_stride, X_ptr, X_row_stride, W_ptr, B_ptr, Mean_ptr,  # noqa: N803
                            Mean_row_stride, RSTD_ptr, RSTD_row_stride, n_rows, n_cols, eps, BLOCK_SIZE):
    raise AssertionError("dispatched by name, never called")


def gqa_kernel(Q, K, V, Out, stride_qh, stride_qm, stride_qk, stride_kh, stride_kn, stride_kk,  # noqa: N803
               stride_vh, stride_vk, stride_vn, stride_oh, stride_om, stride_on, H_Q, H_KV, N_CTX, scale, GROUP,
               HEAD_DIM, BLOCK_N):
    raise AssertionError("dispatched by name, never called")


def test_device_attn_fwd_causal_kernel_perf_lane():
    """The perf-suite name BASELINE config 4 maps to (ops/suite/perf/attn_fwd_causal.py),
    causal, bf16, GQA-free shape as the suite runs it."""
    d = G950Device()
    rng = np.random.default_rng(21)
    z, h, n, hd = 2, 4, 300, 128
    q, k, v = (rng.standard_normal((z, h, n, hd)).astype(np.float32) for _ in range(3))
    qb, kb, vb = (d.upload(a, "bfloat16") for a in (q, k, v))
    ob = d.alloc(q.shape, "bfloat16")
    st = (h * n * hd, n * hd, hd, 1)
    d.launch(attn_fwd_causal_kernel, (3, z * h), (qb, kb, vb, ob, z, h, n, np.float32(hd ** -0.5), *st, *st, *st, *st),
             {"BLOCK_M": 128, "BLOCK_N": 64, "HEAD_DIM": hd, "CAUSAL": True})
    assert rt.module().last_kernel == "g950_attn_fwd_bf16_d128"
    qr, kr, vr = (ref.bf16_round(a) for a in (q, k, v))
    eo, _ = ref.attention(qr, kr, vr, hd ** -0.5, causal=True)
    ok, err = ref.isclose_verdict(d.download(ob), eo, 2e-2, 2e-2)
    assert ok, err


def test_device_dev_suite_kernels():
    """softmax_kernel_inner, _layer_norm_forward_row and gqa_kernel as the
    reference case layer calls them (flat buffers, the 2-D X_ptr, 4-D GQA
    arrays, constexprs in the keywords)."""
    d = G950Device()
    rng = np.random.default_rng(22)
    x = rng.normal(0, 0.8, 96)
    xb, yb = d.upload(x.astype(np.float32)), d.upload(np.full(96, -7.0, np.float32))
    d.launch(softmax_kernel_inner, (3,), (yb, xb, 3, 32), {"TILE_N": 128, "ONE_TILE_PER_CTA": False})
    assert np.allclose(d.download(yb), ref.softmax_inner(x.astype(np.float32), 3, 32), rtol=1e-5, atol=1e-7)

    r, c = 5, 128
    xs = rng.normal(0, 0.7, (r, c)).astype(np.float32)
    w = rng.uniform(0.7, 1.3, c).astype(np.float32)
    b = rng.normal(0, 0.1, c).astype(np.float32)
    bufs = {"Y": d.upload(np.full(r * c, -7.0, np.float32)), "X": d.upload(xs), "W": d.upload(w),
            "B": d.upload(b), "M": d.upload(np.full(r, -7.0, np.float32)), "R": d.upload(np.full(r, -7.0, np.float32))}
    d.launch(_layer_norm_forward_row, (r,), (bufs["Y"], c, bufs["X"], c, bufs["W"], bufs["B"], bufs["M"], 1,
                                             bufs["R"], 1),
             {"n_rows": r, "n_cols": c, "eps": 1e-5, "BLOCK_SIZE": c})
    ey, em, es = ref.layernorm_row(xs, w, b, 1e-5)
    assert np.allclose(d.download(bufs["Y"]).reshape(r, c), ey, rtol=1e-4, atol=1e-4)
    assert np.allclose(d.download(bufs["M"]), em, rtol=1e-4, atol=1e-6)
    assert np.allclose(d.download(bufs["R"]), es, rtol=1e-4)

    z, hq, hkv, n, hd = 2, 4, 2, 64, 32
    q = rng.standard_normal((z, hq, n, hd)).astype(np.float32)
    k = rng.standard_normal((z, hkv, n, hd)).astype(np.float32)
    v = rng.standard_normal((z, hkv, n, hd)).astype(np.float32)
    qb, kb, vb = d.upload(q), d.upload(k), d.upload(v)
    ob = d.alloc(q.shape, np.float32)
    st = (n * hd, hd, 1)
    d.launch(gqa_kernel, (2, z * hq), (qb, kb, vb, ob, *st, *st, *st, *st, hq, hkv, n, np.float32(hd ** -0.5)),
             {"GROUP": 2, "HEAD_DIM": hd, "BLOCK_N": 32})
    ok, err = ref.isclose_verdict(d.download(ob), ref.gqa(q, k, v, hd ** -0.5, 2), 2e-2, 2e-2)
    assert ok, err


def test_device_timer_and_release():
    """timer(): device events around one launch, the way the reference
    benchmark measures (benchmark/run.py:155-170); the launch has finished
    when the block ends.  release() frees the entry's buffers."""
    d = G950Device()
    rng = np.random.default_rng(23)
    x = rng.standard_normal((8191, 3000)).astype(np.float32)
    xb, yb = d.upload(x, "bfloat16"), d.alloc(x.shape, "bfloat16")
    timer = d.timer()
    times = []
    for _ in range(5):
        with timer:
            d.launch(softmax_kernel, (8191,), (xb, yb, 3000), {"BLOCK_SIZE": 4096})
        times.append(timer.seconds)
    # the result is complete at the end of the block
    ok, err = ref.isclose_verdict(d.download(yb)[:4], ref.softmax(ref.bf16_round(x[:4])), 2e-2, 2e-2)
    assert ok, err
    # 98 MB through HBM: tens of microseconds, far below a host round trip of milliseconds
    assert all(0 < t < 5e-3 for t in times), times
    before = torch.cuda.memory_allocated()
    d.release({"x_ptr": xb, "y_ptr": yb})
    assert xb.tensor is None and yb.tensor is None
    assert torch.cuda.memory_allocated() < before
