"""g950_launch_noalloc against g950_launch through the C ABI: every route
that takes workspace from the library's static scratch array
gives the regular entry's results (same kernels: bit for bit), on two calls
in a row with the second smaller; a call that needs more scratch than the
array holds is refused with G950_USAGE."""
import numpy as np
import pytest

torch = pytest.importorskip("torch")

from compiler_amd import operators as ops  # noqa: E402
from compiler_amd import runtime as rt  # noqa: E402

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def both(call, kernels=False):
    """(regular result, no-alloc result, kernel the no-alloc call ran[, kernel
    the regular call ran]).  Both calls run on a fresh stream, the no-alloc
    one first, so no workspace of the regular entry exists yet for it to
    reuse, and the library must hold no workspace for that stream after it."""
    mod = rt.module()
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        assert mod.workspace_bytes(s) == 0
        with rt.no_alloc():
            out = call()
            kernel = mod.last_kernel
        s.synchronize()
        assert mod.workspace_bytes(s) == 0, "g950_launch_noalloc allocated workspace"
        ref_out = call()
        ref_kernel = mod.last_kernel
        s.synchronize()
    return (ref_out, out, kernel, ref_kernel) if kernels else (ref_out, out, kernel)


def split_rows_softmax(rows, cols, seed):
    x = torch.from_numpy(np.random.default_rng(seed).standard_normal((rows, cols), dtype=np.float32)).to(DEV)
    x = x.to(torch.bfloat16)
    return lambda: ops.softmax(x, sync=True)


def test_split_rows_two_calls():
    for rows, cols, seed in ((4, 65536, 1), (3, 40000, 2)):   # few long rows: the two-launch split path
        a, b, kernel = both(split_rows_softmax(rows, cols, seed))
        assert kernel.startswith("g950_rs_final_softmax_bf16")
        assert torch.equal(a, b)


def w8a16(m, n, k, seed):
    rng = np.random.default_rng(seed)
    a = torch.from_numpy(rng.standard_normal((m, k), dtype=np.float32)).to(DEV).to(torch.bfloat16)
    bt = torch.from_numpy(rng.integers(-127, 128, (n, k)).astype(np.int8)).to(DEV)
    s = torch.from_numpy((rng.random(n) / 64).astype(np.float32)).to(DEV).to(torch.bfloat16)
    return lambda: ops.dequant_matmul(a, bt.t(), s, sync=True)


def test_w8a16_few_rows_two_calls():
    # 17..64 rows: the B-streaming kernels need no workspace
    for m, n, k, seed in ((64, 4096, 4096, 3), (48, 2048, 2048, 4)):
        a, b, kernel = both(w8a16(m, n, k, seed))
        assert kernel == "g950_gemm_w8a16_skinny64_bf16"
        assert torch.equal(a, b)


def test_w8a16_widened_copy_in_scratch_two_calls():
    # many output tiles (2 x 5 x 32 = 320 > 256 CUs), B small enough for its
    # bf16 copy to fit the scratch
    for m, n, k, seed in ((1100, 8192, 128, 5), (1025, 8192, 64, 6)):
        a, b, kernel, ref_kernel = both(w8a16(m, n, k, seed), kernels=True)
        assert kernel == ref_kernel == "g950_gemm_bf16_256x256"
        assert torch.equal(a, b)


def test_w8a16_widened_copy_too_large_takes_fused_kernel():
    # 2048 x 8192 x 4096: 2 x 8 x 32 = 512 tiles > 256 CUs take the widened
    # route, and its 64 MiB bf16 copy of B exceeds the 32 MiB scratch: the
    # regular call widens into its workspace, the no-alloc call runs the fused
    # kernel (no workspace); different kernels, so the GEMM bar (2e-2)
    a, b, kernel, ref_kernel = both(w8a16(2048, 8192, 4096, 7), kernels=True)
    assert ref_kernel == "g950_gemm_bf16_256x256"
    assert kernel == "g950_gemm_w8a16_bf16_128x128"
    ok = torch.isclose(b.float(), a.float(), rtol=2e-2, atol=2e-2).all()
    assert bool(ok)


def rowmajor_gemm(m, n, k, seed):
    rng = np.random.default_rng(seed)
    a = torch.from_numpy(rng.standard_normal((m, k), dtype=np.float32)).to(DEV).to(torch.bfloat16)
    b = torch.from_numpy(rng.standard_normal((k, n), dtype=np.float32)).to(DEV).to(torch.bfloat16)
    return lambda: ops.matmul(a, b, sync=True)   # b: the reference's row-major [K, N]


def test_row_major_b_read_directly_two_calls():
    # from one 256 tile each way the MFMA kernel reads row-major B as it lies:
    # no workspace on either entry, the same kernel, the same bits
    for m, n, k, seed in ((2048, 4096, 4096, 11), (300, 264, 256, 12)):
        a, b, kernel, ref_kernel = both(rowmajor_gemm(m, n, k, seed), kernels=True)
        assert kernel == ref_kernel == "g950_gemm_bf16_256x256_rb"
        assert torch.equal(a, b)


def test_row_major_b_copy_in_scratch_two_calls():
    # fewer than 256 rows: B is copied K-contiguous first; a 2 MiB (then
    # 0.5 MiB) copy fits the scratch, so both entries run the same kernels
    for m, n, k, seed in ((128, 1024, 1024, 13), (100, 512, 512, 14)):
        a, b, kernel, ref_kernel = both(rowmajor_gemm(m, n, k, seed), kernels=True)
        assert kernel == ref_kernel == "g950_gemm_bf16_256x256"
        assert torch.equal(a, b)


def test_row_major_b_copy_too_large_takes_general_kernel():
    # 128 x 8192 x 4096: the K-contiguous copy of B (64 MiB) exceeds the
    # 32 MiB scratch, so the no-alloc call runs the general kernel (the
    # documented fallback); the regular call copies into its workspace
    a, b, kernel, ref_kernel = both(rowmajor_gemm(128, 8192, 4096, 15), kernels=True)
    assert ref_kernel == "g950_gemm_bf16_256x256"
    assert kernel == "g950_gemm_general"
    ok = torch.isclose(b.float(), a.float(), rtol=2e-2, atol=2e-2).all()
    assert bool(ok)


def unsigned_gemm(m, n, k, seed):
    rng = np.random.default_rng(seed)
    a = torch.from_numpy(rng.integers(0, 256, (m, k)).astype(np.uint8)).to(DEV)
    bt = torch.from_numpy(rng.integers(0, 256, (n, k)).astype(np.uint8)).to(DEV)

    def call():
        c = torch.empty((m, n), dtype=torch.int32, device=DEV)
        ops.matmul_i8_kernel(a, bt.t(), c, m, n, k, sync=True)
        return c
    return call


def test_unsigned_int8_sums_two_calls():
    for m, n, k, seed in ((512, 512, 1024, 8), (300, 260, 256, 9)):
        a, b, kernel = both(unsigned_gemm(m, n, k, seed))
        assert kernel == "g950_gemm_u8u8_256x256"
        assert torch.equal(a, b)


def test_no_scratch_route_unchanged():
    a, b, kernel = both(split_rows_softmax(64, 3000, 10))   # one wave per row, no workspace
    assert kernel.startswith("g950_rr_softmax_bf16")
    assert torch.equal(a, b)


def test_request_beyond_scratch_is_refused():
    # uint8 x uint8 with 9M columns: its column sums need 36 MB of workspace,
    # more than the scratch holds -- refused before any kernel runs
    n = 9_000_000
    a = torch.zeros((1, 128), dtype=torch.uint8, device=DEV)
    bt = torch.empty((n, 128), dtype=torch.uint8, device=DEV)
    c = torch.full((1, n), 7, dtype=torch.int32, device=DEV)
    with rt.no_alloc():
        with pytest.raises(rt.G950Error) as err:
            ops.matmul_i8_kernel(a, bt.t(), c, 1, n, 128, sync=True)
    assert err.value.code == rt.USAGE and "scratch" in str(err.value)
    assert bool((c == 7).all())
    del bt
    torch.cuda.empty_cache()
