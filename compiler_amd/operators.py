"""The hot-path operators behind the reference kernels' own call signatures.

Each function takes the arguments of the reference Triton kernel it replaces
(same names, same meaning; pointer arguments are torch-ROCm device tensors,
runtime scalars are ints/floats) and launches the gfx950 kernel through the
C ABI.  Views and scalars are handed over in sorted argument-name order, the
layout the reference host packer produces (a100_support/native_io.py:74,81).

The triton launch grid and constexpr block sizes of the reference are not
arguments here: the launcher derives the grid from the view extents, and the
constexprs only shaped the reference's tiles.  The one constexpr with
semantics, attention's ``CAUSAL``, is a keyword argument.
"""
from __future__ import annotations

import math

import numpy as np

from . import runtime as rt


def _launch(op, named_tensors: dict, outputs: set, named_scalars: dict, stream=None, sync=False,
            prepare=False):
    names = sorted(named_tensors)
    tensors = [named_tensors[n] for n in names]
    outs = [n in outputs for n in names]
    scalars = [named_scalars[n] if isinstance(named_scalars[n], rt.Scalar) else rt.scalar(named_scalars[n])
               for n in sorted(named_scalars)]
    if prepare:
        return rt.module().prepare(op, tensors, outs, scalars, stream=stream)
    return rt.module().launch(op, tensors, outs, scalars, stream=stream, sync=sync)


def softmax_kernel(x_ptr, y_ptr, n_cols, *, stream=None, sync=False, prepare=False):
    """Row softmax (ops/suite/perf/softmax.py:21-32).  x/y: [rows, n_cols]."""
    return _launch(rt.OP_SOFTMAX, {"x_ptr": x_ptr, "y_ptr": y_ptr}, {"y_ptr"},
                   {"n_cols": n_cols}, stream, sync, prepare)


def softmax_kernel_inner(output_ptr, input_ptr, M, N, TILE_N=None, ONE_TILE_PER_CTA=None, *, stream=None,
                         sync=False, prepare=False):
    """Row softmax over flat buffers (ops/suite/dev/softmax_kernel_inner.py:12-72):
    row m is the N contiguous elements at input_ptr + m*N, written to
    output_ptr + m*N.  With both constexprs given they travel as scalars: the
    one-tile form (ONE_TILE_PER_CTA) with TILE_N < N normalises only the first
    TILE_N elements of each row and leaves the rest of the output untouched,
    as the reference's single masked tile does (:13-24)."""
    scalars = {"M": M, "N": N}
    if TILE_N is not None and ONE_TILE_PER_CTA is not None:
        scalars.update(ONE_TILE_PER_CTA=bool(ONE_TILE_PER_CTA), TILE_N=int(TILE_N))
    return _launch(rt.OP_SOFTMAX_INNER, {"input_ptr": input_ptr, "output_ptr": output_ptr}, {"output_ptr"},
                   scalars, stream, sync, prepare)


def layer_norm_forward_row(Y_ptr, Y_row_stride, X_ptr, X_row_stride, W_ptr, B_ptr, Mean_ptr, Mean_row_stride,
                           RSTD_ptr, RSTD_row_stride, n_rows, n_cols, eps, BLOCK_SIZE=None, *, stream=None,
                           sync=False, prepare=False):
    """Row LayerNorm forward (ops/suite/dev/layer_norm_forward_row.py:11-36):
    mean and rstd from sum(x) and sum(x^2) (E[x^2] - mean^2), x_hat rounded to
    X's dtype, Y = x_hat*W + B.  Buffers are flat, addressed by the row-stride
    scalars.  The reference loads BLOCK_SIZE columns unmasked, so BLOCK_SIZE
    must equal n_cols (a wider block would read the next row)."""
    if BLOCK_SIZE is not None and int(BLOCK_SIZE) != int(n_cols):
        raise rt.G950Error(rt.USAGE, "_layer_norm_forward_row: BLOCK_SIZE must equal n_cols (the reference "
                                     "loads BLOCK_SIZE columns without a mask)")
    return _launch(rt.OP_LAYERNORM_ROW, {"B_ptr": B_ptr, "Mean_ptr": Mean_ptr, "RSTD_ptr": RSTD_ptr, "W_ptr": W_ptr,
                                         "X_ptr": X_ptr, "Y_ptr": Y_ptr}, {"Y_ptr", "Mean_ptr", "RSTD_ptr"},
                   {"Mean_row_stride": Mean_row_stride, "RSTD_row_stride": RSTD_row_stride,
                    "X_row_stride": X_row_stride, "Y_row_stride": Y_row_stride,
                    "eps": np.float32(eps) if not isinstance(eps, np.generic) else eps,
                    "n_cols": n_cols, "n_rows": n_rows}, stream, sync, prepare)


# the reference's kernel name (a leading underscore in ops/suite/dev/layer_norm_forward_row.py:11)
_layer_norm_forward_row = layer_norm_forward_row


def gqa_kernel(Q, K, V, Out, stride_qh, stride_qm, stride_qk, stride_kh, stride_kn, stride_kk,
               stride_vh, stride_vk, stride_vn, stride_oh, stride_om, stride_on, H_Q, H_KV, N_CTX, scale,
               GROUP, HEAD_DIM=None, BLOCK_N=None, *, stream=None, sync=False, prepare=False):
    """Non-causal GQA attention forward (ops/suite/dev/gqa.py:20-59): Q/Out
    [Z, H_Q, N_CTX, HEAD_DIM], K/V [Z, H_KV, N_CTX, HEAD_DIM]; query head h
    reads KV head h // GROUP.  BLOCK_N only shaped the reference's tile."""
    head_dim = Q.shape[-1] if HEAD_DIM is None else HEAD_DIM
    return _launch(rt.OP_GQA, {"K": K, "Out": Out, "Q": Q, "V": V}, {"Out"},
                   {"GROUP": GROUP, "HEAD_DIM": head_dim, "H_KV": H_KV, "H_Q": H_Q, "N_CTX": N_CTX,
                    "scale": np.float32(scale) if not isinstance(scale, np.generic) else scale,
                    "stride_kh": stride_kh, "stride_kk": stride_kk, "stride_kn": stride_kn,
                    "stride_oh": stride_oh, "stride_om": stride_om, "stride_on": stride_on,
                    "stride_qh": stride_qh, "stride_qk": stride_qk, "stride_qm": stride_qm,
                    "stride_vh": stride_vh, "stride_vk": stride_vk, "stride_vn": stride_vn},
                   stream, sync, prepare)


def logsumexp_kernel(x_ptr, y_ptr, n_cols, *, stream=None, sync=False, prepare=False):
    """Row logsumexp (ops/suite/perf/logsumexp.py:16-38).  x: [rows, n_cols],
    y: [rows] (float32 in the reference): max over non-NaN entries plus
    log(sum(exp(x - max))); NaN for a row holding a NaN; an infinite max is
    returned as is."""
    return _launch(rt.OP_LOGSUMEXP, {"x_ptr": x_ptr, "y_ptr": y_ptr}, {"y_ptr"},
                   {"n_cols": n_cols}, stream, sync, prepare)


def dequantize_kernel(b_ptr, b_scale_ptr, fpb_ptr, K, N, stride_bk, stride_bn, stride_fpbk, stride_fpbn,
                      *, stream=None, sync=False, prepare=False):
    """int8 weight dequantisation fpb = b * b_scale[None, :]
    (ops/suite/perf/dequantize_matmul.py:28-43).  b: int8 [K, N]; b_scale [N]
    and fpb [K, N] share one float dtype; the stride scalars are element
    strides and must match the tensors'."""
    return _launch(rt.OP_DEQUANTIZE, {"b_ptr": b_ptr, "b_scale_ptr": b_scale_ptr, "fpb_ptr": fpb_ptr},
                   {"fpb_ptr"}, {"K": K, "N": N, "stride_bk": stride_bk, "stride_bn": stride_bn,
                                 "stride_fpbk": stride_fpbk, "stride_fpbn": stride_fpbn},
                   stream, sync, prepare)


_VARLEN_VIEWS = ("q_ptr", "k_ptr", "v_ptr", "o_ptr", "p_ptr", "softmax_lse_ptr", "cu_seqlens_q_ptr",
                 "cu_seqlens_k_ptr", "seqused_k_ptr", "philox_args", "alibi_slopes_ptr", "page_table_ptr")
_VARLEN_SCALARS = ("q_row_stride", "k_row_stride", "v_row_stride", "q_head_stride", "k_head_stride",
                   "v_head_stride", "o_row_stride", "o_head_stride", "q_batch_stride", "k_batch_stride",
                   "v_batch_stride", "o_batch_stride", "is_cu_seqlens_q", "is_cu_seqlens_k", "is_seqused_k",
                   "b", "bk", "h", "hk", "h_hk_ratio", "seqlen_q", "seqlen_k", "seqlen_q_rounded",
                   "seqlen_k_rounded", "d", "is_softcap", "softcap", "scale_softmax", "scale_softmax_log2",
                   "is_dropout", "p_dropout", "rp_dropout", "p_dropout_in_uint8_t", "return_softmax",
                   "is_causal", "is_local", "window_size_left", "window_size_right", "seqlenq_ngroups_swapped",
                   "is_paged", "is_alibi", "alibi_slopes_batch_stride", "total_q", "page_table_batch_stride",
                   "block_size", "k_page_stride")
# tile-shape constexprs of the reference kernel: accepted, no semantics here
_VARLEN_TILE = ("BLOCK_M", "BLOCK_N", "BLOCK_K", "KERNEL_NUM_WARPS", "PIPELINE_STAGES", "d_rounded")


def flash_varlen_fwd_kernel(*, stream=None, sync=False, prepare=False, **args):
    """Variable-length attention forward (ops/suite/dev/flash_varlen_fwd_kernel.py:22-320),
    called with the reference kernel's argument names: cu_seqlens / fixed-length
    batches, seqused_k, GQA, causal and local windows, paged K/V.  Pointer
    arguments are device tensors (flattened to 1-D views); softcap, dropout,
    alibi, return_softmax and seqlenq_ngroups_swapped must be off."""
    unknown = set(args) - set(_VARLEN_VIEWS) - set(_VARLEN_SCALARS) - set(_VARLEN_TILE)
    if unknown:
        raise TypeError(f"flash_varlen_fwd_kernel: unexpected arguments {sorted(unknown)}")
    missing = [n for n in _VARLEN_VIEWS + _VARLEN_SCALARS if n not in args]
    if missing:
        raise TypeError(f"flash_varlen_fwd_kernel: missing arguments {missing}")
    views = {n: args[n].reshape(-1) for n in _VARLEN_VIEWS}
    scalars = {n: args[n] for n in _VARLEN_SCALARS}
    return _launch(rt.OP_FLASH_VARLEN, views, {"o_ptr", "softmax_lse_ptr"}, scalars, stream, sync, prepare)


def dequant_matmul_kernel(a_ptr, b_ptr, b_scale_ptr, y_ptr, M, N, K, *, stream=None, sync=False, prepare=False):
    """dequantize_matmul fused into one GEMM: y = a . (b * b_scale[None, :])
    (ops/suite/perf/dequantize_matmul.py:28-43 then matmul.py:21-37).  a: [M, K]
    float, b: int8 logical [K, N] (pass ``bt.t()`` of a row-major [N, K] for the
    MFMA path), b_scale: [N] in a's dtype, y: [M, N]."""
    return _launch(rt.OP_DEQUANT_MATMUL, {"a_ptr": a_ptr, "b_ptr": b_ptr, "b_scale_ptr": b_scale_ptr,
                                          "y_ptr": y_ptr}, {"y_ptr"}, {"M": M, "N": N, "K": K},
                   stream, sync, prepare)


def rms_layernorm_forward_kernel(Y, Y_row_stride, X, X_row_stride, W, W_row_stride, r,
                                 r_row_stride, n_cols, eps, *, stream=None, sync=False, prepare=False):
    """RMSNorm forward (ops/suite/perf/fast_rms_layernorm.py:20-42)."""
    return _launch(rt.OP_RMS_LAYERNORM, {"Y": Y, "X": X, "W": W, "r": r}, {"Y", "r"},
                   {"Y_row_stride": Y_row_stride, "X_row_stride": X_row_stride,
                    "W_row_stride": W_row_stride, "r_row_stride": r_row_stride,
                    "n_cols": n_cols, "eps": np.float32(eps)}, stream, sync, prepare)


def layernorm_kernel(X, Y, W, B, Mean, Rstd, stride, N, eps, *, stream=None, sync=False, prepare=False):
    """LayerNorm forward with Mean/Rstd outputs
    (ops/suite/dev/fused_layernorm_triton.py:27-42)."""
    return _launch(rt.OP_LAYERNORM, {"X": X, "Y": Y, "W": W, "B": B, "Mean": Mean, "Rstd": Rstd},
                   {"Y", "Mean", "Rstd"}, {"stride": stride, "N": N, "eps": np.float32(eps)},
                   stream, sync, prepare)


def matmul_kernel(a_ptr, b_ptr, y_ptr, M, N, K, *, stream=None, sync=False, prepare=False):
    """Y = A.B with fp32 accumulation (ops/suite/perf/matmul.py:21-37).
    ``b_ptr`` is the logical [K, N] operand in either layout: column-major
    (K-contiguous, e.g. ``bt.t()`` of a row-major [N, K] tensor) or the
    reference's row-major [K, N], which the MFMA kernel reads as it lies
    (transposing LDS reads) from one 256 tile each way."""
    return _launch(rt.OP_MATMUL, {"a_ptr": a_ptr, "b_ptr": b_ptr, "y_ptr": y_ptr}, {"y_ptr"},
                   {"M": M, "N": N, "K": K}, stream, sync, prepare)


def matmul_i8_kernel(a_ptr, b_ptr, c_ptr, M, N, K, *, stream=None, sync=False, prepare=False):
    """8-bit integer dot -> int32, bit-exact modular accumulation, for the
    four signedness pairs of the i8 family (a100c/plan/tiles.py:118-131:
    int8/uint8 a_ptr and b_ptr in any combination)."""
    return _launch(rt.OP_MATMUL_I8, {"a_ptr": a_ptr, "b_ptr": b_ptr, "c_ptr": c_ptr}, {"c_ptr"},
                   {"M": M, "N": N, "K": K}, stream, sync, prepare)


def matmul_i8_dequant_kernel(a_ptr, b_ptr, sa_ptr, sb_ptr, y_ptr, M, N, K, *, stream=None,
                             sync=False, prepare=False):
    """int8 GEMM + dequant epilogue: y = bf16(acc * sa[m] * sb[n])
    (per-column rule of ops/suite/perf/dequantize_matmul.py:29-38)."""
    return _launch(rt.OP_MATMUL_I8_DEQUANT,
                   {"a_ptr": a_ptr, "b_ptr": b_ptr, "sa_ptr": sa_ptr, "sb_ptr": sb_ptr,
                    "y_ptr": y_ptr}, {"y_ptr"}, {"M": M, "N": N, "K": K}, stream, sync, prepare)


def attn_fwd_causal_kernel(q_ptr, k_ptr, v_ptr, out_ptr, Z, H, N_CTX, scale,
                           stride_qz, stride_qh, stride_qm, stride_qk,
                           stride_kz, stride_kh, stride_kn, stride_kk,
                           stride_vz, stride_vh, stride_vk, stride_vn,
                           stride_oz, stride_oh, stride_om, stride_on,
                           *, CAUSAL=True, lse_ptr=None, stream=None, sync=False,
                           prepare=False):
    """Attention forward (ops/suite/perf/attn_fwd_causal.py:20-55), with GQA
    when k/v carry fewer heads (ops/suite/dev/gqa.py:29) and the optional
    per-row logsumexp (ops/suite/dev/flash_varlen_fwd_kernel.py:309,318-320)."""
    tensors = {"q_ptr": q_ptr, "k_ptr": k_ptr, "v_ptr": v_ptr, "out_ptr": out_ptr}
    outputs = {"out_ptr"}
    op = rt.OP_ATTENTION
    if lse_ptr is not None:
        tensors["lse_ptr"] = lse_ptr
        outputs.add("lse_ptr")
        op = rt.OP_ATTENTION_LSE
    scalars = {"CAUSAL": bool(CAUSAL), "Z": Z, "H": H, "N_CTX": N_CTX,
               "scale": np.float32(scale) if not isinstance(scale, np.generic) else scale,
               "stride_qz": stride_qz, "stride_qh": stride_qh, "stride_qm": stride_qm,
               "stride_qk": stride_qk, "stride_kz": stride_kz, "stride_kh": stride_kh,
               "stride_kn": stride_kn, "stride_kk": stride_kk, "stride_vz": stride_vz,
               "stride_vh": stride_vh, "stride_vk": stride_vk, "stride_vn": stride_vn,
               "stride_oz": stride_oz, "stride_oh": stride_oh, "stride_om": stride_om,
               "stride_on": stride_on}
    return _launch(op, tensors, outputs, scalars, stream, sync, prepare)


def stream_copy(x, y, *, stream=None, sync=False, prepare=False):
    """y = x through the streaming-copy kernel (nontemporal 16-byte loads and
    stores, the row kernels' memory path); used to calibrate HBM counters."""
    return _launch(rt.OP_COPY, {"x": x, "y": y}, {"y"}, {}, stream, sync, prepare)


# ------------------------------------------------------ tensor conveniences
def softmax(x, out=None, **kw):
    import torch
    y = torch.empty_like(x) if out is None else out
    softmax_kernel(x, y, x.shape[-1], **kw)
    return y


def logsumexp(x, out=None, **kw):
    import torch
    y = torch.empty(x.shape[0], dtype=torch.float32, device=x.device) if out is None else out
    logsumexp_kernel(x, y, x.shape[-1], **kw)
    return y


def dequantize(b, scale, out=None, **kw):
    """b: int8 [K, N] tensor, scale: [N] float tensor -> b * scale in scale's dtype."""
    import torch
    y = torch.empty(b.shape, dtype=scale.dtype, device=b.device) if out is None else out
    dequantize_kernel(b, scale, y, b.shape[0], b.shape[1], b.stride(0), b.stride(1), y.stride(0),
                      y.stride(1), **kw)
    return y


def dequant_matmul(a, b, scale, out=None, **kw):
    """a [M,K] @ (b [K,N] int8 * scale[N]); pass ``bt.t()`` for a K-contiguous b."""
    import torch
    m, k = a.shape
    n = b.shape[1]
    y = torch.empty((m, n), dtype=a.dtype, device=a.device) if out is None else out
    dequant_matmul_kernel(a, b, scale, y, m, n, k, **kw)
    return y


def rmsnorm(x, w, eps, out=None, r=None, **kw):
    import torch
    y = torch.empty_like(x) if out is None else out
    r = torch.empty(x.shape[0], dtype=torch.float32, device=x.device) if r is None else r
    rms_layernorm_forward_kernel(y, y.stride(0), x, x.stride(0), w, 1, r, r.stride(0),
                                 x.shape[1], eps, **kw)
    return y, r


def layernorm(x, w, b, eps, out=None, mean=None, rstd=None, **kw):
    import torch
    y = torch.empty_like(x) if out is None else out
    mean = torch.empty(x.shape[0], dtype=torch.float32, device=x.device) if mean is None else mean
    rstd = torch.empty(x.shape[0], dtype=torch.float32, device=x.device) if rstd is None else rstd
    layernorm_kernel(x, y, w, b, mean, rstd, x.stride(0), x.shape[1], eps, **kw)
    return y, mean, rstd


def matmul(a, b, out=None, **kw):
    """a [M,K] @ b [K,N] (row-major b, or ``bt.t()`` for a K-contiguous one)."""
    import torch
    m, k = a.shape
    n = b.shape[1]
    y = torch.empty((m, n), dtype=a.dtype, device=a.device) if out is None else out
    matmul_kernel(a, b, y, m, n, k, **kw)
    return y


def attention(q, k, v, scale=None, causal=True, out=None, lse=None, **kw):
    import torch
    z, h, s, d = q.shape
    scale = 1.0 / math.sqrt(d) if scale is None else scale
    o = torch.empty_like(q) if out is None else out
    if lse is None:
        lse = torch.empty((z, h, s), dtype=torch.float32, device=q.device)
    attn_fwd_causal_kernel(q, k, v, o, z, h, s, scale, *q.stride(), *k.stride(), *v.stride(),
                           *o.stride(), CAUSAL=causal, lse_ptr=lse, **kw)
    return o, lse
