"""C-ABI library checks that need no GPU: it loads, exports every function
include/g950rt.h declares, and its host-side contract checks and kernel
selection (g950_validate, which never touches a device) behave as specified.
"""
import ctypes
import re
from pathlib import Path

import numpy as np
import pytest

from compiler_amd import runtime as rt

HEADER = Path(__file__).resolve().parents[1] / "include" / "g950rt.h"
BASE = 0x7F0000000000  # fake device address: validate compares, never dereferences


def declared_functions():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\s*\*?\s*(g950_\w+)\s*\(", text, re.M)))


def test_library_exports_every_declared_function():
    lib = rt.load_library()
    names = declared_functions()
    assert set(names) == set(rt.EXPORTS)
    for name in names:
        assert hasattr(lib, name), name


def test_record_layouts_match_reference_abi():
    # a100c/runtime/a100rt.h:186-199 pins these sizes and offsets
    assert ctypes.sizeof(rt.View) == 56
    assert rt.View.data.offset == 0 and rt.View.shape.offset == 8
    assert rt.View.strides.offset == 16 and rt.View.storage_size.offset == 24
    assert rt.View.dtype.offset == 32 and rt.View.ndim.offset == 36
    assert rt.View.flags.offset == 40 and rt.View.storage.offset == 48
    assert ctypes.sizeof(rt.Scalar) == 16 and rt.Scalar.bits.offset == 8


def test_strerror_codes():
    lib = rt.load_library()
    assert lib.g950_strerror(0) == b"ok"
    assert b"refused" in lib.g950_strerror(2)
    assert b"rejected" in lib.g950_strerror(3)
    # a100c/runtime/a100rt.h:54: exit 5 = repeats produced different outputs
    assert rt.REPEAT_MISMATCH == 5 and b"repeats" in lib.g950_strerror(5)


class Args:
    """Builds fake views (host shape/stride arrays, fake device addresses)."""

    ITEM = {rt.DT_F32: 4, rt.DT_BF16: 2, rt.DT_F16: 2, rt.DT_INT8: 1, rt.DT_UINT8: 1, rt.DT_INT32: 4, rt.DT_INT64: 8}

    def __init__(self):
        self.specs = []
        self.keep = []
        self.next = BASE

    def view(self, shape, dtype, strides=None, output=False, offset=0, storage_extra=0):
        isz = self.ITEM[dtype]
        if strides is None:
            strides = []
            acc = 1
            for n in reversed(shape):
                strides.insert(0, acc)
                acc *= n
        reach = sum((n - 1) * s for n, s in zip(shape, strides)) + 1 if all(shape) else 0
        storage = self.next
        self.next += ((reach + offset) * isz + storage_extra + 4096 + 255) // 256 * 256
        self.specs.append((shape, [s * isz for s in strides], dtype, output, storage + offset * isz,
                           storage, (reach + offset) * isz + storage_extra))
        return self

    def build(self):
        arr = (rt.View * len(self.specs))()
        for i, (shape, strides, dtype, output, data, storage, size) in enumerate(self.specs):
            s = (ctypes.c_int64 * len(shape))(*shape)
            st = (ctypes.c_int64 * len(shape))(*strides)
            self.keep += [s, st]
            arr[i].data, arr[i].shape, arr[i].strides = data, s, st
            arr[i].storage_size, arr[i].dtype, arr[i].ndim = size, dtype, len(shape)
            arr[i].flags, arr[i].storage = int(output), storage
        return arr


def validate(op, args, scalars):
    lib = rt.load_library()
    views = args.build()
    sc = (rt.Scalar * max(len(scalars), 1))(*[rt.scalar(*s) if isinstance(s, tuple) else rt.scalar(s)
                                              for s in scalars])
    rc = lib.g950_validate(op, views, len(args.specs), sc, len(scalars))
    return rc, lib.g950_last_kernel().decode(), lib.g950_last_error().decode()


def softmax_args(rows, cols, dtype):
    return Args().view([rows, cols], dtype).view([rows, cols], dtype, output=True)


@pytest.mark.parametrize("rows,cols,dtype,kernel", [
    (4096, 4096, rt.DT_F32, "g950_rr_softmax_f32_v4_i16_b64"),
    (8191, 3000, rt.DT_BF16, "g950_rr_softmax_bf16_v8_i6_b64"),
    (4, 97, rt.DT_F32, "g950_rm_softmax_f32_v4_i1"),      # odd rows: masked aligned vectors
    (8191, 3001, rt.DT_BF16, "g950_rm_softmax_bf16_v8_i6"),
    (4, 16, rt.DT_F16, "g950_rr_softmax_f16_v8_i1_b64"),
    (2, 100000, rt.DT_F32, "g950_rs_final_softmax_f32_v4"),
    (3, 70001, rt.DT_F32, "g950_rs_final_softmax_f32_v1"),
    (1, 1 << 20, rt.DT_BF16, "g950_rs_final_softmax_bf16_v8"),
    (4, 16384, rt.DT_F32, "g950_rs_final_softmax_f32_v4"),     # few rows: split
    (4, 4096, rt.DT_F32, "g950_rr_softmax_f32_v4_i16_b64"),    # one chunk: no split
    (200, 16384, rt.DT_F32, "g950_rr_softmax_f32_v4_i16_b256"),  # enough rows
])
def test_softmax_kernel_selection(rows, cols, dtype, kernel):
    rc, name, err = validate(rt.OP_SOFTMAX, softmax_args(rows, cols, dtype), [cols])
    assert rc == 0, err
    assert name == kernel


def test_odd_rows_masked_vectors_need_a_shared_phase():
    # y rows in another 16-byte phase than x rows: the element-wise v1 kernel
    a = Args().view([300, 3001], rt.DT_BF16).view([300, 3001], rt.DT_BF16, strides=[3004, 1], output=True)
    rc, name, err = validate(rt.OP_SOFTMAX, a, [3001])
    assert rc == 0 and name.startswith("g950_rr_softmax_bf16_v1"), err
    # rows longer than one wave's eight vectors per lane: the v1 kernels / split rows
    a = softmax_args(64, 4097, rt.DT_BF16)
    rc, name, err = validate(rt.OP_SOFTMAX, a, [4097])
    assert rc == 0 and "_v1" in name, err


def test_softmax_refusals():
    rc, _, err = validate(rt.OP_SOFTMAX, softmax_args(4, 97, rt.DT_F32), [96])
    assert rc == rt.USAGE and "n_cols" in err
    # output view without the output flag
    a = Args().view([4, 97], rt.DT_F32).view([4, 97], rt.DT_F32, output=False)
    assert validate(rt.OP_SOFTMAX, a, [97])[0] == rt.REJECTED
    # mixed dtypes
    a = Args().view([4, 97], rt.DT_F32).view([4, 97], rt.DT_BF16, output=True)
    assert validate(rt.OP_SOFTMAX, a, [97])[0] == rt.USAGE
    # wrong arity
    assert validate(rt.OP_SOFTMAX, softmax_args(4, 97, rt.DT_F32), [97, 1])[0] == rt.USAGE
    # a stride whose reach wraps 64 bits (4 row steps x 2^62 bytes = 2^64, which
    # wraps to 0) is outside any storage
    a = Args().view([5, 97], rt.DT_F32).view([5, 97], rt.DT_F32, output=True)
    shape, strides, dtype, output, data, storage, size = a.specs[0]
    a.specs[0] = (shape, [1 << 62, 4], dtype, output, data, storage, size)
    rc, _, err = validate(rt.OP_SOFTMAX, a, [97])
    assert rc == rt.REJECTED and "reach" in err, err


@pytest.mark.parametrize("rows,cols,dtype,ydt,kernel", [
    (4, 16, rt.DT_F32, rt.DT_F32, "g950_rr_logsumexp_f32_v4_i1_b64"),
    (64, 1024, rt.DT_BF16, rt.DT_F32, "g950_rr_logsumexp_bf16_v8_i2_b64"),
    (4, 97, rt.DT_F16, rt.DT_F16, "g950_rm_logsumexp_f16_v8_i1"),
    (2, 100000, rt.DT_F32, rt.DT_F32, "g950_rs_final_logsumexp_f32_v4"),
])
def test_logsumexp_contract(rows, cols, dtype, ydt, kernel):
    a = Args().view([rows, cols], dtype).view([rows], ydt, output=True)
    rc, name, err = validate(rt.OP_LOGSUMEXP, a, [cols])
    assert rc == 0, err
    assert name == kernel


def test_logsumexp_refusals():
    ok = Args().view([4, 97], rt.DT_F32).view([4], rt.DT_F32, output=True)
    assert validate(rt.OP_LOGSUMEXP, ok, [96])[0] == rt.USAGE
    assert validate(rt.OP_LOGSUMEXP, ok, [97, 1])[0] == rt.USAGE
    short = Args().view([4, 97], rt.DT_F32).view([3], rt.DT_F32, output=True)
    rc, _, err = validate(rt.OP_LOGSUMEXP, short, [97])
    assert rc == rt.USAGE and "per row" in err
    ints = Args().view([4, 97], rt.DT_F32).view([4], rt.DT_INT32, output=True)
    assert validate(rt.OP_LOGSUMEXP, ints, [97])[0] == rt.USAGE
    unflagged = Args().view([4, 97], rt.DT_F32).view([4], rt.DT_F32, output=False)
    assert validate(rt.OP_LOGSUMEXP, unflagged, [97])[0] == rt.REJECTED


def dq_args(k, n, ydt, b_strides=None):
    return (Args().view([k, n], rt.DT_INT8, strides=b_strides).view([n], ydt)
            .view([k, n], ydt, output=True))


@pytest.mark.parametrize("k,n,ydt,kernel", [
    (32, 32, rt.DT_F32, "g950_dequant_i8_f32"),
    (8192, 8192, rt.DT_BF16, "g950_dequant_i8_bf16"),
    (256, 32, rt.DT_F16, "g950_dequant_i8_f16"),
    (33, 33, rt.DT_F32, "g950_dequant_i8_general"),
])
def test_dequantize_contract(k, n, ydt, kernel):
    rc, name, err = validate(rt.OP_DEQUANTIZE, dq_args(k, n, ydt), [np.int32(k), np.int32(n), np.int32(n),
                                                                     np.int32(1), np.int32(n), np.int32(1)])
    assert rc == 0, err
    assert name == kernel


def test_dequantize_refusals():
    good = [np.int32(32), np.int32(32), np.int32(32), np.int32(1), np.int32(32), np.int32(1)]
    # a stride scalar that disagrees with its view
    bad = list(good)
    bad[2] = np.int32(31)
    rc, _, err = validate(rt.OP_DEQUANTIZE, dq_args(32, 32, rt.DT_F32), bad)
    assert rc == rt.USAGE and "stride_bk" in err
    assert validate(rt.OP_DEQUANTIZE, dq_args(32, 32, rt.DT_F32), good[:5])[0] == rt.USAGE
    # scale and output dtypes must agree; b must be int8
    a = Args().view([32, 32], rt.DT_INT8).view([32], rt.DT_F32).view([32, 32], rt.DT_BF16, output=True)
    assert validate(rt.OP_DEQUANTIZE, a, good)[0] == rt.USAGE
    a = Args().view([32, 32], rt.DT_UINT8).view([32], rt.DT_F32).view([32, 32], rt.DT_F32, output=True)
    assert validate(rt.OP_DEQUANTIZE, a, good)[0] == rt.USAGE
    # a column-major b takes the general kernel
    rc, name, err = validate(rt.OP_DEQUANTIZE, dq_args(32, 32, rt.DT_F32, b_strides=[1, 32]),
                             [np.int32(32), np.int32(32), np.int32(1), np.int32(32), np.int32(32), np.int32(1)])
    assert rc == 0 and name == "g950_dequant_i8_general", err


NP_DT = {"float32": rt.DT_F32, "float16": rt.DT_F16, "bfloat16": rt.DT_BF16, "int32": rt.DT_INT32,
         "uint64": rt.DT_UINT64}


def varlen_validate(a, meta, dt="bfloat16", **override):
    """g950_validate for a flash_varlen case: 12 flat views + 46 scalars, sorted."""
    from compiler_amd.operators import _VARLEN_SCALARS, _VARLEN_VIEWS
    merged = {**a, **meta, **override}
    args = Args()
    for name in sorted(_VARLEN_VIEWS):
        arr = np.asarray(merged[name])
        code = dt if name in ("q_ptr", "k_ptr", "v_ptr", "o_ptr") else arr.dtype.name
        args.view([arr.size], NP_DT.get(code, rt.DT_F32) if code != "uint64" else rt.DT_INT64,
                  output=name in ("o_ptr", "softmax_lse_ptr"))
    scal = []
    for name in sorted(_VARLEN_SCALARS):
        val = merged[name]
        scal.append(np.float32(val) if isinstance(val, float) else (np.int32(1 if val else 0)
                    if isinstance(val, bool) else np.int32(val)))
    return validate(rt.OP_FLASH_VARLEN, args, scal)


def test_flash_varlen_contract():
    from oracle import inputs
    a, meta = inputs.varlen_case()                       # the reference case: d=16 -> general kernel
    rc, name, err = varlen_validate(a, meta)
    assert rc == 0 and name == "g950_attn_varlen_general", err
    a, meta = inputs.varlen_case(batches=3, max_q=300, max_k=400, h=8, hk=2, d=128)
    rc, name, err = varlen_validate(a, meta)
    assert rc == 0 and name == "g950_attn_fwd_bf16_d128_varlen", err
    rc, name, err = varlen_validate(a, meta, dt="float16")
    assert rc == 0 and name == "g950_attn_fwd_f16_d128_varlen", err
    a, meta = inputs.varlen_case(batches=3, max_q=64, max_k=200, h=4, hk=4, d=64, paged=True, block_size=16,
                                 causal=True, window_right=0)
    rc, name, err = varlen_validate(a, meta)
    assert rc == 0 and name == "g950_attn_fwd_bf16_d64_varlen_pl", err   # 16-key pages: per-lane lookups
    a, meta = inputs.varlen_case(batches=3, max_q=64, max_k=200, h=4, hk=4, d=64, paged=True, block_size=64,
                                 causal=True, window_right=0)
    rc, name, err = varlen_validate(a, meta)
    assert rc == 0 and name == "g950_attn_fwd_bf16_d64_varlen_pt", err   # whole-tile pages
    a, meta = inputs.varlen_case(strided=True, d=64)      # padded strides: not 16-byte multiples
    rc, name, err = varlen_validate(a, meta)
    assert rc == 0 and name == "g950_attn_varlen_general", err


def test_flash_varlen_refusals():
    from oracle import inputs
    a, meta = inputs.varlen_case()
    for flag in ("is_softcap", "is_dropout", "return_softmax", "is_alibi", "seqlenq_ngroups_swapped"):
        rc, _, err = varlen_validate(a, meta, **{flag: True})
        assert rc == rt.USAGE and flag in err
    rc, _, err = varlen_validate(a, meta, scale_softmax_log2=0.5)
    assert rc == rt.USAGE and "scale_softmax_log2" in err
    rc, _, err = varlen_validate(a, meta, h_hk_ratio=3)
    assert rc == rt.USAGE
    rc, _, err = varlen_validate(a, meta, total_q=a["total_q"] + 1)   # lse too small for h x total_q
    assert rc == rt.USAGE and "softmax_lse_ptr" in err
    rc, _, err = varlen_validate(a, meta, cu_seqlens_q_ptr=a["cu_seqlens_q_ptr"].astype(np.float32))
    assert rc == rt.USAGE and "int32" in err
    a2, meta2 = inputs.varlen_case(var_q=False, var_k=False)
    rc, _, err = varlen_validate(a2, meta2, seqlen_q=a2["seqlen_q"] + 1)
    assert rc == rt.USAGE and "seqlen_q" in err
    rc, _, err = varlen_validate(a2, meta2, seqlen_k=a2["seqlen_k"] + 5)
    assert rc == rt.USAGE and "seqlen_k" in err


def test_dequant_matmul_contract():
    def args(m, n, k, adt=rt.DT_BF16, col_b=True, sdt=None):
        return (Args().view([m, k], adt).view([k, n], rt.DT_INT8, strides=[1, k] if col_b else None)
                .view([n], sdt or adt).view([m, n], adt, output=True))
    rc, name, err = validate(rt.OP_DEQUANT_MATMUL, args(256, 512, 1024), [1024, 256, 512])
    assert rc == 0 and name == "g950_gemm_w8a16_bf16_128x128", err
    rc, name, err = validate(rt.OP_DEQUANT_MATMUL, args(16, 8192, 8192, rt.DT_F16), [8192, 16, 8192])
    assert rc == 0 and name == "g950_gemm_w8a16_skinny_f16", err   # decode shape (M <= 16)
    # 16 columns per workgroup: a 32-column grid short of the CUs (128 < 256),
    # more than a quarter past them (344 > 320), or one row of A
    for m, n in ((16, 4096), (16, 11008), (1, 8192)):
        rc, name, err = validate(rt.OP_DEQUANT_MATMUL, args(m, n, 4096), [4096, m, n])
        assert rc == 0 and name == "g950_gemm_w8a16_skinny_c16_bf16", (m, n, err)
    rc, name, err = validate(rt.OP_DEQUANT_MATMUL, args(17, 4096, 4096), [4096, 17, 4096])
    assert rc == 0 and name == "g950_gemm_w8a16_skinny32_bf16", err   # 17..32 rows
    rc, name, err = validate(rt.OP_DEQUANT_MATMUL, args(64, 4096, 4096, rt.DT_F16), [4096, 64, 4096])
    assert rc == 0 and name == "g950_gemm_w8a16_skinny64_f16", err   # 33..64 rows
    rc, name, err = validate(rt.OP_DEQUANT_MATMUL, args(65, 4096, 4096), [4096, 65, 4096])
    assert rc == 0 and name == "g950_gemm_w8a16_bf16_128x128", err   # 65 rows: the tiled kernel
    rc, name, err = validate(rt.OP_DEQUANT_MATMUL, args(4096, 4096, 256), [256, 4096, 4096])
    assert rc == 0 and name == "g950_gemm_bf16_256x256", err   # B widened once, 256 tiles
    rc, name, err = validate(rt.OP_DEQUANT_MATMUL, args(1024, 8192, 128), [128, 1024, 8192])
    assert rc == 0 and name == "g950_gemm_w8a16_bf16_128x128", err   # 128 tiles: half the CUs
    rc, name, err = validate(rt.OP_DEQUANT_MATMUL, args(1025, 8192, 128), [128, 1025, 8192])
    assert rc == 0 and name == "g950_gemm_bf16_256x256", err   # 160 tiles
    rc, name, err = validate(rt.OP_DEQUANT_MATMUL, args(4096, 4096, 208), [208, 4096, 4096])
    assert rc == 0 and name == "g950_gemm_w8a16_bf16_128x128", err   # K not a multiple of 64
    # the reference's own weight layout, row-major int8 b [K, N]
    # (dequantize_matmul.py:62-65): widened as it lies + the row-major-B MFMA
    # kernel from one 256 tile each way (whole 64-k slabs), else transposed
    # once to K-contiguous and the fused / decode kernels
    rc, name, err = validate(rt.OP_DEQUANT_MATMUL, args(64, 64, 64, col_b=False), [64, 64, 64])
    assert rc == 0 and name == "g950_gemm_w8a16_skinny64_bf16", err
    rc, name, err = validate(rt.OP_DEQUANT_MATMUL, args(2048, 4096, 4096, col_b=False), [4096, 2048, 4096])
    assert rc == 0 and name == "g950_gemm_bf16_256x256_rb", err
    rc, name, err = validate(rt.OP_DEQUANT_MATMUL, args(300, 512, 256, rt.DT_F16, col_b=False), [256, 300, 512])
    assert rc == 0 and name == "g950_gemm_f16_256x256_rb", err
    rc, name, err = validate(rt.OP_DEQUANT_MATMUL, args(100, 272, 96, col_b=False), [96, 100, 272])
    assert rc == 0 and name == "g950_gemm_w8a16_bf16_128x128", err   # M < 256: transposed, fused kernel
    rc, name, err = validate(rt.OP_DEQUANT_MATMUL, args(1, 8192, 8192, col_b=False), [8192, 1, 8192])
    assert rc == 0 and name == "g950_gemm_w8a16_skinny_c16_bf16", err
    rc, name, err = validate(rt.OP_DEQUANT_MATMUL, args(64, 72, 64, col_b=False), [64, 64, 72])
    assert rc == 0 and name == "g950_gemm_general", err   # N not whole 16-byte int8 rows
    rc, name, err = validate(rt.OP_DEQUANT_MATMUL, args(64, 64, 40), [40, 64, 64])
    assert rc == 0 and name == "g950_gemm_general", err
    assert validate(rt.OP_DEQUANT_MATMUL, args(64, 64, 64, sdt=rt.DT_F32), [64, 64, 64])[0] == rt.USAGE
    assert validate(rt.OP_DEQUANT_MATMUL, args(64, 64, 64), [64, 64, 65])[0] == rt.USAGE
    wrong_b = Args().view([64, 64], rt.DT_BF16).view([64, 64], rt.DT_BF16).view([64], rt.DT_BF16) \
        .view([64, 64], rt.DT_BF16, output=True)
    assert validate(rt.OP_DEQUANT_MATMUL, wrong_b, [64, 64, 64])[0] == rt.USAGE


def test_empty_views_may_be_null_nonempty_may_not():
    a = Args().view([3, 0], rt.DT_F32).view([3], rt.DT_F32, output=True)
    shape, strides, dtype, out, data, storage, size = a.specs[0]
    a.specs[0] = (shape, strides, dtype, out, 0, 0, 0)          # empty x with null pointers
    rc, name, err = validate(rt.OP_LOGSUMEXP, a, [0])
    assert rc == 0, err
    b = Args().view([3, 4], rt.DT_F32).view([3], rt.DT_F32, output=True)
    shape, strides, dtype, out, data, storage, size = b.specs[0]
    b.specs[0] = (shape, strides, dtype, out, 0, 0, size)
    rc, _, err = validate(rt.OP_LOGSUMEXP, b, [4])
    assert rc == rt.REJECTED and "null" in err


def test_empty_rows_never_take_the_masked_kernels():
    # a [3, 0] view whose data pointer is not 16-byte aligned: the masked
    # kernels would read the aligned block at or below an address no
    # allocation backs; empty rows keep the element-wise kernel (no loads)
    a = Args().view([3, 0], rt.DT_F32).view([3], rt.DT_F32, output=True)
    shape, strides, dtype, out, data, storage, size = a.specs[0]
    a.specs[0] = (shape, strides, dtype, out, BASE + 8, BASE + 8, 0)
    rc, name, err = validate(rt.OP_LOGSUMEXP, a, [0])
    assert rc == 0, err
    assert not name.startswith("g950_rm_"), name


def test_view_reach_outside_storage_is_rejected():
    a = softmax_args(4, 97, rt.DT_F32)
    shape, strides, dtype, out, data, storage, size = a.specs[0]
    a.specs[0] = (shape, strides, dtype, out, data, storage, size - 4)  # one element short
    rc, _, err = validate(rt.OP_SOFTMAX, a, [97])
    assert rc == rt.REJECTED and "outside" in err


def test_rms_and_layernorm_contracts():
    a = (Args().view([3000], rt.DT_BF16).view([8191, 3000], rt.DT_BF16)
         .view([8191, 3000], rt.DT_BF16, output=True).view([8191], rt.DT_F32, output=True))
    scal = [1, 3000, 3000, np.float32(1e-6), 3000, 1]
    rc, name, err = validate(rt.OP_RMS_LAYERNORM, a, scal)
    assert rc == 0, err
    assert name == "g950_rr_rmsnorm_bf16_v8_i6_b64"
    bad = [1, 2999, 3000, np.float32(1e-6), 3000, 1]
    assert validate(rt.OP_RMS_LAYERNORM, a, bad)[0] == rt.USAGE
    ln = (Args().view([3000], rt.DT_BF16).view([8191], rt.DT_F32, output=True)
          .view([8191], rt.DT_F32, output=True).view([3000], rt.DT_BF16)
          .view([8191, 3000], rt.DT_BF16).view([8191, 3000], rt.DT_BF16, output=True))
    rc, name, err = validate(rt.OP_LAYERNORM, ln, [3000, np.float32(1e-5), 3000])
    assert rc == 0, err
    assert name == "g950_rw_layernorm_bf16_v8_i6"    # many rows: parameters in LDS, 8 rows per workgroup
    few = (Args().view([3000], rt.DT_BF16).view([64], rt.DT_F32, output=True)
           .view([64], rt.DT_F32, output=True).view([3000], rt.DT_BF16)
           .view([64, 3000], rt.DT_BF16).view([64, 3000], rt.DT_BF16, output=True))
    rc, name, err = validate(rt.OP_LAYERNORM, few, [3000, np.float32(1e-5), 3000])
    assert rc == 0 and name == "g950_rr_layernorm_bf16_v8_i6_b64", err
    assert validate(rt.OP_LAYERNORM, ln, [3000, np.float32(1e-5), 3001])[0] == rt.USAGE


def gemm_args(m, n, k, dtype, col_major_b=True, out=rt.DT_BF16):
    a = Args().view([m, k], dtype)
    if col_major_b:
        a.view([k, n], dtype, strides=[1, k])
    else:
        a.view([k, n], dtype)
    return a.view([m, n], out, output=True)


@pytest.mark.parametrize("m,n,k,colb,kernel", [
    (8192, 8192, 8192, True, "g950_gemm_bf16_256x256"),
    (4097, 11008, 4096, True, "g950_gemm_bf16_256x256"),
    (8192, 8192, 8192, False, "g950_gemm_bf16_256x256_rb"),  # row-major B (matmul.py:33), read as it lies
    (4097, 11008, 4096, False, "g950_gemm_bf16_256x256_rb"),
    (300, 264, 256, False, "g950_gemm_bf16_256x256_rb"),
    (256, 256, 96, False, "g950_gemm_bf16_256x256_kt"),  # row-major B, K tail: copied K-contiguous
    (255, 4096, 4096, False, "g950_gemm_bf16_256x256"),  # row-major B under one tile of rows: copied
    (128, 128, 128, False, "g950_gemm_bf16_256x256"),   # the corpus fixtures' layout
    (8, 24, 32, False, "g950_gemm_bf16_256x256_kt"),     # matmul-tail fixture shape [8,32,24]: K tail
    (64, 64, 96, True, "g950_gemm_bf16_256x256_kt"),    # K not a whole 64-element (128-byte) slab
    (64, 64, 100, True, "g950_gemm_general"),           # K rows not 16-byte multiples
    (64, 60, 64, False, "g950_gemm_general"),           # row-major B rows not 16-byte multiples
    (33, 65, 64, True, "g950_gemm_bf16_256x256"),       # a single slab
])
def test_matmul_selection(m, n, k, colb, kernel):
    rc, name, err = validate(rt.OP_MATMUL, gemm_args(m, n, k, rt.DT_BF16, colb), [k, m, n])
    assert rc == 0, err
    assert name == kernel


def test_matmul_rows_past_4gib_take_64bit_kernels():
    # the whole-slab kernels address DMA rows by 32-bit offsets from the
    # operand base; a row stride that puts the last row at 4 GiB or beyond
    # selects the _kt kernels (64-bit addresses), or the general kernel for
    # unsigned int8 operands (no _kt form)
    near = Args().view([2, 64], rt.DT_BF16, strides=[(1 << 31) - 128, 1]) \
        .view([64, 64], rt.DT_BF16, strides=[1, 64]).view([2, 64], rt.DT_BF16, output=True)
    rc, name, err = validate(rt.OP_MATMUL, near, [64, 2, 64])
    assert rc == 0 and name == "g950_gemm_bf16_256x256", err
    far = Args().view([2, 64], rt.DT_BF16, strides=[1 << 31, 1]) \
        .view([64, 64], rt.DT_BF16, strides=[1, 64]).view([2, 64], rt.DT_BF16, output=True)
    rc, name, err = validate(rt.OP_MATMUL, far, [64, 2, 64])
    assert rc == 0 and name == "g950_gemm_bf16_256x256_kt", err
    farb = Args().view([2, 64], rt.DT_BF16).view([64, 2], rt.DT_BF16, strides=[1, 1 << 31]) \
        .view([2, 2], rt.DT_BF16, output=True)
    rc, name, err = validate(rt.OP_MATMUL, farb, [64, 2, 2])
    assert rc == 0 and name == "g950_gemm_bf16_256x256_kt", err
    for adt, want in ((rt.DT_INT8, "g950_gemm_i8_256x256_kt"), (rt.DT_UINT8, "g950_gemm_general_i8")):
        c = (Args().view([2, 128], adt, strides=[1 << 32, 1]).view([128, 64], rt.DT_INT8, strides=[1, 128])
             .view([2, 64], rt.DT_INT32, output=True))
        rc, name, err = validate(rt.OP_MATMUL_I8, c, [128, 2, 64])
        assert rc == 0 and name == want, err


def test_matmul_fp32_and_int8_tails():
    # fp32 operands (the corpus base dtype) take the fp32 MFMA kernel in both B
    # layouts; mixed operand dtypes and unaligned rows the general kernel
    rc, name, err = validate(rt.OP_MATMUL, gemm_args(128, 128, 128, rt.DT_F32, False, out=rt.DT_F32), [128, 128, 128])
    assert rc == 0 and name == "g950_gemm_f32_256x256", err
    rc, name, err = validate(rt.OP_MATMUL, gemm_args(16, 16, 16, rt.DT_F32, True, out=rt.DT_F32), [16, 16, 16])
    assert rc == 0 and name == "g950_gemm_f32_256x256_kt", err
    rc, name, err = validate(rt.OP_MATMUL, gemm_args(8, 32, 24, rt.DT_F32, False, out=rt.DT_F32), [24, 8, 32])
    assert rc == 0 and name == "g950_gemm_f32_256x256_kt", err
    rc, name, err = validate(rt.OP_MATMUL, gemm_args(8, 30, 24, rt.DT_F32, False, out=rt.DT_F32), [24, 8, 30])
    assert rc == 0 and name == "g950_gemm_general", err
    mixed = Args().view([64, 64], rt.DT_F32).view([64, 64], rt.DT_BF16, strides=[1, 64]) \
        .view([64, 64], rt.DT_F32, output=True)
    rc, name, err = validate(rt.OP_MATMUL, mixed, [64, 64, 64])
    assert rc == 0 and name == "g950_gemm_general", err
    # int8 with a K tail takes the _kt kernel
    c = (Args().view([300, 208], rt.DT_INT8).view([208, 200], rt.DT_INT8, strides=[1, 208])
         .view([300, 200], rt.DT_INT32, output=True))
    rc, name, err = validate(rt.OP_MATMUL_I8, c, [208, 300, 200])
    assert rc == 0 and name == "g950_gemm_i8_256x256_kt", err
    # an unsigned operand with a K tail: the zero tail would flip to -128, so the general kernel
    c = (Args().view([300, 208], rt.DT_UINT8).view([208, 200], rt.DT_INT8, strides=[1, 208])
         .view([300, 200], rt.DT_INT32, output=True))
    rc, name, err = validate(rt.OP_MATMUL_I8, c, [208, 300, 200])
    assert rc == 0 and name == "g950_gemm_general_i8", err


def test_matmul_refusals():
    assert validate(rt.OP_MATMUL, gemm_args(64, 64, 64, rt.DT_BF16), [64, 64, 65])[0] == rt.USAGE
    a = Args().view([64, 64], rt.DT_BF16).view([32, 64], rt.DT_BF16).view([64, 64], rt.DT_BF16, output=True)
    assert validate(rt.OP_MATMUL, a, [64, 64, 64])[0] == rt.USAGE


def test_int8_selection():
    a = (Args().view([4096, 8192], rt.DT_INT8).view([8192, 8192], rt.DT_INT8, strides=[1, 8192])
         .view([4096], rt.DT_F32).view([8192], rt.DT_F32).view([4096, 8192], rt.DT_BF16, output=True))
    rc, name, err = validate(rt.OP_MATMUL_I8_DEQUANT, a, [8192, 4096, 8192])
    assert rc == 0, err
    assert name == "g950_gemm_i8_256x256"
    c = (Args().view([64, 100], rt.DT_INT8).view([100, 64], rt.DT_INT8)
         .view([64, 64], rt.DT_INT32, output=True))
    rc, name, err = validate(rt.OP_MATMUL_I8, c, [100, 64, 64])
    assert rc == 0 and name == "g950_gemm_general_i8", err


def attn_args(z, h, hkv, s, d, dtype, lse=True):
    a = Args().view([z, hkv, s, d], dtype)
    if lse:
        a.view([z, h, s], rt.DT_F32, output=True)
    a.view([z, h, s, d], dtype, output=True).view([z, h, s, d], dtype).view([z, hkv, s, d], dtype)
    return a


def attn_scalars(z, h, hkv, s, d, causal=True):
    qs = [h * s * d, s * d, d, 1]
    ks = [hkv * s * d, s * d, d, 1]
    # sorted: CAUSAL H N_CTX Z scale stride_k(h,k,n,z) stride_o(h,m,n,z) stride_q(h,k,m,z) stride_v(h,k,n,z)
    return [bool(causal), np.int32(h), np.int32(s), np.int32(z), np.float32(d ** -0.5),
            ks[1], ks[3], ks[2], ks[0], qs[1], qs[2], qs[3], qs[0],
            qs[1], qs[3], qs[2], qs[0], ks[1], ks[2], ks[3], ks[0]]


def test_attention_selection_and_refusals():
    rc, name, err = validate(rt.OP_ATTENTION_LSE, attn_args(4, 32, 8, 4096, 128, rt.DT_BF16),
                             attn_scalars(4, 32, 8, 4096, 128))
    assert rc == 0, err
    assert name == "g950_attn_fwd_bf16_d128"
    rc, name, err = validate(rt.OP_ATTENTION_LSE, attn_args(4, 4, 4, 32, 64, rt.DT_F32),
                             attn_scalars(4, 4, 4, 32, 64, causal=False))
    assert rc == 0 and name == "g950_attn_fwd_f32mfma_d64", err   # fp32: the fp32 MFMA kernel
    rc, name, err = validate(rt.OP_ATTENTION_LSE, attn_args(4, 32, 8, 4096, 128, rt.DT_F32),
                             attn_scalars(4, 32, 8, 4096, 128))
    assert rc == 0 and name == "g950_attn_fwd_f32mfma_d128", err
    rc, name, err = validate(rt.OP_ATTENTION_LSE, attn_args(1, 2, 2, 40, 48, rt.DT_F32),
                             attn_scalars(1, 2, 2, 40, 48))
    assert rc == 0 and name == "g950_attn_fwd_general", err        # head dim 48: the general kernel
    neg = attn_scalars(1, 2, 1, 70, 64)
    neg[4] = np.float32(-0.125)                                      # scale <= 0: not the 16-bit kernel
    rc, name, err = validate(rt.OP_ATTENTION_LSE, attn_args(1, 2, 1, 70, 64, rt.DT_BF16), neg)
    assert rc == 0 and name == "g950_attn_fwd_f32mfma_d64", err
    bad = attn_scalars(4, 32, 8, 4096, 128)
    bad[5] += 1  # stride_kh disagrees with the k view
    rc, _, err = validate(rt.OP_ATTENTION_LSE, attn_args(4, 32, 8, 4096, 128, rt.DT_BF16), bad)
    assert rc == rt.USAGE and "stride_kh" in err
    # Hq not a multiple of Hkv
    rc, _, err = validate(rt.OP_ATTENTION_LSE, attn_args(1, 6, 4, 64, 64, rt.DT_BF16),
                          attn_scalars(1, 6, 4, 64, 64))
    assert rc == rt.USAGE


def test_unknown_operator_refused():
    rc, _, err = validate(99, softmax_args(4, 16, rt.DT_F32), [16])
    assert rc == rt.USAGE and "unknown" in err


# ------------------------------------------------------- dev-suite contracts
def test_softmax_inner_contract():
    # the reference case (97,): M = 3 rows of C = 32 in a flat buffer
    a = Args().view([96], rt.DT_F32).view([96], rt.DT_F32, output=True)
    rc, name, err = validate(rt.OP_SOFTMAX_INNER, a, [3, 32])
    assert rc == 0 and name == "g950_rr_softmax_f32_v4_i1_b64", err
    # (17,): M = 3, C = 5 -- not a whole 16-byte vector per row
    a = Args().view([15], rt.DT_BF16).view([15], rt.DT_BF16, output=True)
    rc, name, err = validate(rt.OP_SOFTMAX_INNER, a, [3, 5])
    assert rc == 0 and name == "g950_rm_softmax_bf16_v8_i1", err
    # C2 scale through the flat contract
    a = Args().view([8191 * 3000], rt.DT_BF16).view([8191 * 3000], rt.DT_BF16, output=True)
    rc, name, err = validate(rt.OP_SOFTMAX_INNER, a, [8191, 3000])
    assert rc == 0 and name == "g950_rr_softmax_bf16_v8_i6_b64", err
    # a 2-D contiguous view is a flat buffer too
    a = Args().view([3, 32], rt.DT_F32).view([96], rt.DT_F32, output=True)
    assert validate(rt.OP_SOFTMAX_INNER, a, [3, 32])[0] == 0
    # refusals: M x N past the buffer, mixed dtypes, a non-contiguous view, arity
    a = Args().view([96], rt.DT_F32).view([95], rt.DT_F32, output=True)
    rc, _, err = validate(rt.OP_SOFTMAX_INNER, a, [3, 32])
    assert rc == rt.USAGE and "exceed" in err
    a = Args().view([96], rt.DT_F32).view([96], rt.DT_F16, output=True)
    assert validate(rt.OP_SOFTMAX_INNER, a, [3, 32])[0] == rt.USAGE
    a = Args().view([3, 32], rt.DT_F32, strides=[64, 1]).view([96], rt.DT_F32, output=True)
    rc, _, err = validate(rt.OP_SOFTMAX_INNER, a, [3, 32])
    assert rc == rt.USAGE and "contiguous" in err
    a = Args().view([96], rt.DT_F32).view([96], rt.DT_F32, output=True)
    assert validate(rt.OP_SOFTMAX_INNER, a, [3])[0] == rt.USAGE
    # nothing to do
    assert validate(rt.OP_SOFTMAX_INNER, a, [0, 32])[0] == 0


def test_softmax_inner_one_tile_contract():
    # the constexprs as scalars (M, N, ONE_TILE_PER_CTA, TILE_N): one tile
    # narrower than the row normalises the first TILE_N elements, read and
    # written at row stride N -- 16 fp32 = whole 16-byte vectors of 32-element rows
    a = Args().view([96], rt.DT_F32).view([96], rt.DT_F32, output=True)
    rc, name, err = validate(rt.OP_SOFTMAX_INNER, a, [3, 32, True, 16])
    assert rc == 0 and name.startswith("g950_rr_softmax_f32_v4"), err
    # a tile as wide as the row, or the looped form, covers the row
    for sc in ([3, 32, True, 32], [3, 32, True, 64], [3, 32, False, 16]):
        rc, name, err = validate(rt.OP_SOFTMAX_INNER, a, sc)
        assert rc == 0 and name == "g950_rr_softmax_f32_v4_i1_b64", (sc, err)
    # bf16 rows of 3000 with a 2048-wide tile: 4096-byte tile rows at a 6000-byte stride
    a = Args().view([8191 * 3000], rt.DT_BF16).view([8191 * 3000], rt.DT_BF16, output=True)
    rc, name, err = validate(rt.OP_SOFTMAX_INNER, a, [8191, 3000, True, 2048])
    assert rc == 0 and name.startswith("g950_r") and "softmax_bf16" in name, err
    a = Args().view([96], rt.DT_F32).view([96], rt.DT_F32, output=True)
    rc, _, err = validate(rt.OP_SOFTMAX_INNER, a, [3, 32, True, 0])
    assert rc == rt.USAGE and "TILE_N" in err
    assert validate(rt.OP_SOFTMAX_INNER, a, [3, 32, True])[0] == rt.USAGE


def lnrow_args(rows, cols, dt, sdt=None, x2d=True):
    sdt = sdt or dt
    a = Args().view([cols], dt).view([rows], sdt, output=True).view([rows], sdt, output=True).view([cols], dt)
    a.view([rows, cols] if x2d else [rows * cols], dt)
    return a.view([rows * cols], dt, output=True)


def lnrow_scalars(rows, cols, xs=None, ys=None, ms=1, rs=1, eps=1e-5):
    # sorted: Mean_row_stride RSTD_row_stride X_row_stride Y_row_stride eps n_cols n_rows
    return [ms, rs, cols if xs is None else xs, cols if ys is None else ys, np.float32(eps), cols, rows]


def test_layernorm_row_contract():
    for rows, cols, dt, kernel in ((3, 16, rt.DT_F32, "g950_rr_lnrow_f32_v4_i1_b64"),
                                   (5, 128, rt.DT_BF16, "g950_rr_lnrow_bf16_v8_i1_b64"),
                                   (8191, 3000, rt.DT_BF16, "g950_rw_lnrow_bf16_v8_i6"),
                                   (7, 67, rt.DT_F16, "g950_rm_lnrow_f16_v8_i1")):
        rc, name, err = validate(rt.OP_LAYERNORM_ROW, lnrow_args(rows, cols, dt), lnrow_scalars(rows, cols))
        assert rc == 0 and name == kernel, err
    # statistics in another float dtype than X (each pair must agree)
    rc, _, err = validate(rt.OP_LAYERNORM_ROW, lnrow_args(3, 16, rt.DT_BF16, rt.DT_F32), lnrow_scalars(3, 16))
    assert rc == 0, err
    # refusals
    rc, _, err = validate(rt.OP_LAYERNORM_ROW, lnrow_args(3, 16, rt.DT_F32), lnrow_scalars(3, 16, xs=17))
    assert rc == rt.USAGE and "exceed" in err
    rc, _, err = validate(rt.OP_LAYERNORM_ROW, lnrow_args(3, 16, rt.DT_F32), lnrow_scalars(3, 16, ys=8))
    assert rc == rt.USAGE and "overlap" in err
    rc, _, err = validate(rt.OP_LAYERNORM_ROW, lnrow_args(3, 16, rt.DT_F32), lnrow_scalars(3, 16, ms=2))
    assert rc == rt.USAGE
    mixed = (Args().view([16], rt.DT_F32).view([3], rt.DT_F32, output=True).view([3], rt.DT_F32, output=True)
             .view([16], rt.DT_BF16).view([3, 16], rt.DT_F32).view([48], rt.DT_F32, output=True))
    assert validate(rt.OP_LAYERNORM_ROW, mixed, lnrow_scalars(3, 16))[0] == rt.USAGE
    bad = lnrow_scalars(3, 16)
    bad[5] = 0
    assert validate(rt.OP_LAYERNORM_ROW, lnrow_args(3, 16, rt.DT_F32), bad)[0] == rt.USAGE
    # a row stride whose reach overflows 64 bits ((n_rows - 1) * stride wraps
    # negative) is still refused
    rc, _, err = validate(rt.OP_LAYERNORM_ROW, lnrow_args(3, 16, rt.DT_F32), lnrow_scalars(3, 16, xs=1 << 62))
    assert rc == rt.USAGE and "exceed" in err, err


def gqa_args(z, hq, hkv, n, d, dt):
    # sorted views: K, Out, Q, V
    return (Args().view([z, hkv, n, d], dt).view([z, hq, n, d], dt, output=True).view([z, hq, n, d], dt)
            .view([z, hkv, n, d], dt))


def gqa_scalars(hq, hkv, n, d, group=None):
    group = hq // hkv if group is None else group
    # sorted: GROUP HEAD_DIM H_KV H_Q N_CTX scale stride_k(h,k,n) stride_o(h,m,n) stride_q(h,k,m) stride_v(h,k,n)
    return [group, d, hkv, hq, n, np.float32(d ** -0.5), n * d, 1, d, n * d, d, 1, n * d, 1, d, n * d, d, 1]


def test_gqa_contract():
    for shape, dt, kernel in (((2, 4, 2, 32, 32), rt.DT_F32, "g950_attn_fwd_f32mfma_d32"),
                              ((1, 4, 2, 64, 32), rt.DT_BF16, "g950_attn_fwd_f32mfma_d32"),
                              ((4, 32, 8, 4096, 128), rt.DT_BF16, "g950_attn_fwd_bf16_d128"),
                              ((2, 8, 2, 500, 64), rt.DT_F16, "g950_attn_fwd_f16_d64")):
        z, hq, hkv, n, d = shape
        rc, name, err = validate(rt.OP_GQA, gqa_args(*shape, dt), gqa_scalars(hq, hkv, n, d))
        assert rc == 0 and name == kernel, err
    # GROUP larger than Hq/Hkv: all heads on the first KV heads (valid)
    assert validate(rt.OP_GQA, gqa_args(2, 4, 2, 32, 32, rt.DT_F32), gqa_scalars(4, 2, 32, 32, group=4))[0] == 0
    # GROUP that sends a head past the KV heads
    rc, _, err = validate(rt.OP_GQA, gqa_args(2, 4, 2, 32, 32, rt.DT_F32), gqa_scalars(4, 2, 32, 32, group=1))
    assert rc == rt.USAGE and "GROUP" in err
    # a stride scalar that disagrees with its view
    bad = gqa_scalars(4, 2, 32, 32)
    bad[6] += 1
    rc, _, err = validate(rt.OP_GQA, gqa_args(2, 4, 2, 32, 32, rt.DT_F32), bad)
    assert rc == rt.USAGE and "stride_kh" in err
    # a batch stride other than heads x head stride (the kernel's batch offset)
    a = (Args().view([2, 2, 32, 32], rt.DT_F32, strides=[4096, 1024, 32, 1])
         .view([2, 4, 32, 32], rt.DT_F32, output=True).view([2, 4, 32, 32], rt.DT_F32)
         .view([2, 2, 32, 32], rt.DT_F32))
    rc, _, err = validate(rt.OP_GQA, a, gqa_scalars(4, 2, 32, 32))
    assert rc == rt.USAGE and "batch stride" in err
    # N_CTX disagreeing with the views, and arity
    bad = gqa_scalars(4, 2, 32, 32)
    bad[4] = 31
    assert validate(rt.OP_GQA, gqa_args(2, 4, 2, 32, 32, rt.DT_F32), bad)[0] == rt.USAGE
    assert validate(rt.OP_GQA, gqa_args(2, 4, 2, 32, 32, rt.DT_F32), gqa_scalars(4, 2, 32, 32)[:17])[0] == rt.USAGE


@pytest.mark.parametrize("adt,bdt,kernel", [
    (rt.DT_INT8, rt.DT_INT8, "g950_gemm_i8_256x256"),
    (rt.DT_UINT8, rt.DT_INT8, "g950_gemm_u8s8_256x256"),
    (rt.DT_INT8, rt.DT_UINT8, "g950_gemm_s8u8_256x256"),
    (rt.DT_UINT8, rt.DT_UINT8, "g950_gemm_u8u8_256x256"),
])
def test_int8_signedness_selection(adt, bdt, kernel):
    a = (Args().view([4096, 8192], adt).view([8192, 8192], bdt, strides=[1, 8192])
         .view([4096, 8192], rt.DT_INT32, output=True))
    rc, name, err = validate(rt.OP_MATMUL_I8, a, [8192, 4096, 8192])
    assert rc == 0 and name == kernel, err
    # row-major B: the general kernel handles every pair
    c = Args().view([64, 100], adt).view([100, 64], bdt).view([64, 64], rt.DT_INT32, output=True)
    rc, name, err = validate(rt.OP_MATMUL_I8, c, [100, 64, 64])
    assert rc == 0 and name == "g950_gemm_general_i8", err


def test_int8_refuses_other_integer_types():
    a = Args().view([64, 128], rt.DT_INT32).view([128, 64], rt.DT_INT8, strides=[1, 128]) \
        .view([64, 64], rt.DT_INT32, output=True)
    rc, _, err = validate(rt.OP_MATMUL_I8, a, [128, 64, 64])
    assert rc == rt.USAGE and "uint8" in err


def test_dequant_matmul_k0_never_takes_the_widened_route():
    # K = 0 with many output tiles: the 256x256 GEMM would DMA slab 0 of an empty
    # operand; the fused kernel (no K loop) writes the zero product instead
    a = (Args().view([4096, 0], rt.DT_BF16).view([0, 4096], rt.DT_INT8, strides=[1, 0])
         .view([4096], rt.DT_BF16).view([4096, 4096], rt.DT_BF16, output=True))
    rc, name, err = validate(rt.OP_DEQUANT_MATMUL, a, [0, 4096, 4096])
    assert rc == 0, err
    assert name != "g950_gemm_bf16_256x256"
    assert name == "g950_gemm_w8a16_bf16_128x128"
