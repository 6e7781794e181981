"""CPU oracle for the g950 hot path -- TEST INFRASTRUCTURE ONLY.

This module is the checker, never the product: only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
import it.  The product path (``compiler_amd``) never routes through it.

Each function restates, in numpy float64, the reference operator's own ``ref``
semantics (file:line cited per function, paths relative to the reference
checkout).  Low-precision rounding follows the reference host conversion
``_bf16_host`` (``ops/harness/opslib/case.py:214-220``).

How each function is pinned (besides restating the formula):
  * ``softmax``              -- reference-held post-run fixtures softmax16/97 in
                                3 dtypes; rows sum to 1; constant row -> 1/n.
  * ``rms_layernorm``        -- closed form: constant row c -> sign(c)*w (eps->0);
                                scale invariance; brute-force loop on tiny rows.
  * ``layernorm``            -- per-row output mean == beta, std == gamma when
                                gamma/beta are constant; brute-force loop.
  * ``layernorm_row``        -- constant row c -> mean c, rstd 1/sqrt(eps), Y = B;
                                equals ``layernorm`` on well-conditioned rows
                                (E[x^2] - mean^2 == var); brute-force loop;
                                a dropped mean^2 term fails.
  * ``gqa``                  -- ``attention`` (non-causal) when GROUP = Hq/Hkv;
                                GROUP > Hq/Hkv maps several groups onto the
                                first KV heads (brute force); uniform V -> V.
  * ``matmul``               -- reference-held matmul16/128/tail fixtures in 3
                                dtypes + matmul256 fp16; brute-force triple loop.
  * ``matmul_i8``            -- exact integer brute force on tiny shapes; int32
                                no-overflow bound 8192*127^2 < 2^31.
  * ``dequant``              -- closed form vs a scalar loop; bf16 RNE rule.
  * ``attention``            -- reference-held attention fixtures (non-causal) in
                                3 dtypes; causal row 0 == V[0]; uniform V -> V;
                                LSE of equal scores == s + log(n).
  * ``flash_varlen``         -- per-sequence equality with ``attention`` (dense
                                and causal, GQA); local window 0 picks V[i];
                                huge windows == dense; permuted pages ==
                                contiguous; seqused_k == truncated keys;
                                brute-force loop with bottom-right causal mask.
  * ``bf16_round``           -- known bit patterns (ties-to-even, NaN quieting,
                                overflow to inf) and torch's RNE conversion.
"""
from __future__ import annotations

import math

import numpy as np

__all__ = [
    "bf16_round", "bf16_bits", "bf16_from_bits", "softmax", "rms_layernorm",
    "layernorm", "matmul", "matmul_i8", "dequant", "attention", "isclose_verdict",
    "TOLERANCES",
    "logsumexp",
    "dequantize",
    "flash_varlen",
    "layernorm_row",
    "gqa",
    "softmax_inner",
    "wrap_i32",
]

# Shared value tolerances per dtype (ops/harness/opslib/case.py:153-157) and the
# tighter bars the hot-path contract states for the build's own configs.
TOLERANCES = {
    "float32": (1e-3, 1e-3),
    "float16": (1e-2, 1e-2),
    "bfloat16": (2e-2, 2e-2),
}


# --------------------------------------------------------------------- bf16
def bf16_round(array) -> np.ndarray:
    """float32 values rounded to bfloat16, returned as float32.

    Round-to-nearest-even on the upper 16 bits; NaN keeps its payload with the
    quiet bit set (ops/harness/opslib/case.py:214-220).
    """
    values = np.ascontiguousarray(array, dtype=np.float32)
    bits = values.view(np.uint32)
    rounded = (bits + np.uint32(0x7FFF) + ((bits >> 16) & np.uint32(1))) & np.uint32(0xFFFF0000)
    rounded = np.where(np.isnan(values), bits | np.uint32(0x00400000), rounded)
    return rounded.astype(np.uint32).view(np.float32)


def bf16_bits(array) -> np.ndarray:
    """uint16 storage bits of ``bf16_round(array)``."""
    return (bf16_round(array).view(np.uint32) >> 16).astype(np.uint16)


def bf16_from_bits(bits) -> np.ndarray:
    """Decode uint16 bf16 storage to float32 (exact widening)."""
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


# --------------------------------------------------------------- reductions
def softmax(x) -> np.ndarray:
    """Row softmax over the last axis in float64.

    ops/suite/perf/softmax.py:40-45: ``e = exp(x - max); e / sum(e)``.  The
    masked-tail form (ops/suite/dev/softmax_kernel_inner.py:12-72) pads with
    -inf, which contributes exp(-inf) = 0, so the unpadded row is the result.
    """
    x64 = np.asarray(x, dtype=np.float64)
    e = np.exp(x64 - x64.max(axis=-1, keepdims=True))
    return e / e.sum(axis=-1, keepdims=True)


def logsumexp(x) -> np.ndarray:
    """Row logsumexp over the last axis in float64 (ops/suite/perf/logsumexp.py).

    ref (:52-56) is ``np.logaddexp.reduce`` in float64; the kernel (:16-38)
    takes the max over non-NaN entries, returns NaN for a row holding a NaN,
    the max itself when it is infinite, else ``max + log(sum(exp(x - max)))``.
    Both agree on every row: a NaN row reduces to NaN in logaddexp, a +inf
    entry to +inf, an all -inf row to -inf.
    """
    x64 = np.asarray(x, dtype=np.float64)
    nan = np.isnan(x64).any(axis=-1)
    finite_or_inf = np.where(np.isnan(x64), -np.inf, x64)
    # the kernel's running max starts at -inf (:23), so an empty row gives -inf
    mx = finite_or_inf.max(axis=-1, initial=-np.inf)
    with np.errstate(invalid="ignore", over="ignore", divide="ignore"):
        safe = np.where(np.isfinite(mx), mx, 0.0)
        s = np.exp(finite_or_inf - safe[..., None]).sum(axis=-1)
        out = np.where(np.isfinite(mx), safe + np.log(s), mx)
    return np.where(nan, np.nan, out)


def dequantize(b, scale) -> np.ndarray:
    """int8 weight dequantisation in float64 (ops/suite/perf/dequantize_matmul.py):
    ``ref`` (:47-50) is ``b * s[None, :]`` in float64, cast to fpb's dtype;
    the kernel (:28-43) widens b and s to fp32 and multiplies.  The product of
    an int8 and a float32/bf16/fp16 value is exact in float64, so rounding it
    to the output dtype is the single rounding both forms perform."""
    return np.asarray(b, dtype=np.float64) * np.asarray(scale, dtype=np.float64)[None, :]


def rms_layernorm(x, w, eps):
    """RMSNorm forward: returns (Y, r) in float64.

    ops/suite/perf/fast_rms_layernorm.py:52-61: ``var = sum(x*x)/n``,
    ``inv = 1/sqrt(var + eps)``, ``Y = (x*inv)*w``, ``r[row] = inv``.
    """
    x64 = np.asarray(x, dtype=np.float64)
    w64 = np.asarray(w, dtype=np.float64)
    n_cols = x64.shape[-1]
    var = (x64 * x64).sum(axis=-1, keepdims=True) / n_cols
    inv = 1.0 / np.sqrt(var + float(eps))
    y = (x64 * inv) * w64[None, :]
    return y, inv.reshape(-1)


def layernorm(x, w, b, eps):
    """LayerNorm forward: returns (Y, Mean, Rstd) in float64.

    ops/suite/dev/fused_layernorm_triton.py:49-60: centered variance
    ``var = mean((x-mean)^2)`` (numpy ``var``), ``rstd = 1/sqrt(var+eps)``,
    ``Y = (x-mean)*rstd*w + b``.
    """
    x64 = np.asarray(x, dtype=np.float64)
    w64 = np.asarray(w, dtype=np.float64)
    b64 = np.asarray(b, dtype=np.float64)
    mean = x64.mean(axis=-1)
    var = x64.var(axis=-1)
    rstd = 1.0 / np.sqrt(var + float(eps))
    y = (x64 - mean[:, None]) * rstd[:, None] * w64[None, :] + b64[None, :]
    return y, mean, rstd


def layernorm_row(x, w, b, eps):
    """Row LayerNorm forward of ``_layer_norm_forward_row``: returns (Y, Mean,
    Rstd) in float64.

    ops/suite/dev/layer_norm_forward_row.py:65-67: ``mean = x.mean(1)``,
    ``rstd = 1/sqrt((x*x).mean(1) - mean*mean + eps)`` (the E[x^2] - mean^2
    form, not the centered variance), ``Y = (x - mean)*rstd*W + B``.
    """
    x64 = np.asarray(x, dtype=np.float64)
    w64 = np.asarray(w, dtype=np.float64)
    b64 = np.asarray(b, dtype=np.float64)
    mean = x64.mean(axis=-1)
    rstd = 1.0 / np.sqrt((x64 * x64).mean(axis=-1) - mean * mean + float(eps))
    y = (x64 - mean[:, None]) * rstd[:, None] * w64[None, :] + b64[None, :]
    return y, mean, rstd


def softmax_inner(flat, m, n, tile_n=None, one_tile=False, out=None) -> np.ndarray:
    """``softmax_kernel_inner`` (ops/suite/dev/softmax_kernel_inner.py, ref):
    the flat buffer's first m*n elements as m rows of n, row softmax in
    float64, returned flat.  The one-tile form with ``tile_n < n`` loads
    ``tl.arange(0, TILE_N)`` of each row (masked by ``< N``, so all of them)
    and stores the same positions (:13-24): the first ``tile_n`` elements
    of a row are normalised among themselves and the rest of the output row
    keeps what ``out`` (the output buffer before the call, flat) held."""
    x = np.asarray(flat).reshape(-1)[: m * n].reshape(m, n)
    if not (one_tile and tile_n is not None and tile_n < n):
        return softmax(x).reshape(-1)
    res = np.array(np.asarray(out).reshape(-1)[: m * n], dtype=np.float64).reshape(m, n)
    res[:, :tile_n] = softmax(x[:, :tile_n])
    return res.reshape(-1)


# -------------------------------------------------------------------- GEMM
def matmul(a, b) -> np.ndarray:
    """``Y = A @ B`` in float64 (ops/suite/perf/matmul.py:46-50).

    ``b`` is the logical [K, N] operand whatever its memory order.
    """
    return np.asarray(a, dtype=np.float64) @ np.asarray(b, dtype=np.float64)


def matmul_i8(a, b) -> np.ndarray:
    """Exact integer ``C = A @ B`` for int8 / uint8 operands, returned as int64.

    Semantics of the i8 dot family: signed or unsigned operands in the four
    pairs s x s, u x u, u x s, s x u, 32-bit accumulator (a100c/plan/tiles.py:
    118-131; a100c/tests/test_matrix_breadth.py:365-452 accumulates in int64
    and narrows to int32, see ``wrap_i32``).  float64 BLAS is exact here:
    every partial sum is an integer below 2**53 (|a*b| <= 255*255, K <= 2**20).
    """
    a = np.asarray(a)
    b = np.asarray(b)
    if a.shape[1] > (1 << 20):
        raise ValueError("K too large for the exact float64 path")
    return np.rint(a.astype(np.float64) @ b.astype(np.float64)).astype(np.int64)


def wrap_i32(acc) -> np.ndarray:
    """The int64 accumulator narrowed to int32 modulo 2**32, as the reference
    test narrows it (a100c/tests/test_matrix_breadth.py:389-390)."""
    return np.asarray(acc, dtype=np.int64).astype(np.int32)


def dequant(acc, sa, sb) -> np.ndarray:
    """Dequant epilogue ``acc[m,n] * sa[m] * sb[n]`` in float64.

    The per-column scale is the ``dequantize_kernel`` rule
    (ops/suite/perf/dequantize_matmul.py:29-38, ref :49-52); the per-row A
    scale is the symmetric-activation half of the same rule.
    """
    acc64 = np.asarray(acc, dtype=np.float64)
    return acc64 * np.asarray(sa, dtype=np.float64)[:, None] * np.asarray(sb, dtype=np.float64)[None, :]


# --------------------------------------------------------------- attention
def attention(q, k, v, scale, causal=True, block_rows=512, group=None):
    """Flash-style attention forward in float64: returns (O, LSE).

    Scores and softmax follow ops/suite/perf/attn_fwd_causal.py:63-76 (causal
    mask ``j <= i``); the GQA head map ``h_kv = h // group`` (``group`` =
    Hq // Hkv unless given) follows ops/suite/dev/gqa.py:29 and the LSE rule
    ``rowmax + log(rowsum)`` on scaled scores (natural log, ``+inf`` for an
    empty or NaN row) follows ops/suite/dev/flash_varlen_fwd_kernel.py:309 and
    :411-418.

    q: [Z, Hq, S, D]; k, v: [Z, Hkv, S, D].  Computed per (z, h) in row blocks
    so that the score tensor never exceeds ``block_rows * S`` doubles.
    """
    q = np.asarray(q)
    k = np.asarray(k)
    v = np.asarray(v)
    z_count, hq, s_q, d = q.shape
    hkv = k.shape[1]
    if group is None:
        if hq % hkv:
            raise ValueError("Hq must be a multiple of Hkv")
        group = hq // hkv
    if (hq - 1) // group >= hkv:
        raise ValueError("group maps a query head past the KV heads")
    s_k = k.shape[2]
    out = np.empty((z_count, hq, s_q, d), dtype=np.float64)
    lse = np.empty((z_count, hq, s_q), dtype=np.float64)
    for z in range(z_count):
        for h in range(hq):
            kh = k[z, h // group].astype(np.float64)
            vh = v[z, h // group].astype(np.float64)
            for r0 in range(0, s_q, block_rows):
                r1 = min(s_q, r0 + block_rows)
                qb = q[z, h, r0:r1].astype(np.float64)
                s = (qb @ kh.T) * float(scale)
                if causal:
                    rows = np.arange(r0, r1)[:, None]
                    cols = np.arange(s_k)[None, :]
                    s = np.where(cols <= rows, s, -np.inf)
                m = s.max(axis=1, keepdims=True)
                finite = np.isfinite(m)
                m_safe = np.where(finite, m, 0.0)
                p = np.exp(s - m_safe)
                l = p.sum(axis=1, keepdims=True)
                empty = (l == 0) | np.isnan(l)
                out[z, h, r0:r1] = np.where(empty, 0.0, p / np.where(empty, 1.0, l)) @ vh
                with np.errstate(divide="ignore"):
                    row_lse = (m_safe + np.log(l))[:, 0]
                lse[z, h, r0:r1] = np.where(empty[:, 0], np.inf, row_lse)
    return out, lse


def gqa(q, k, v, scale, group):
    """``gqa_kernel``'s output in float64 (ops/suite/dev/gqa.py:69-85):
    non-causal softmax(q k^T * scale) v per (z, h) with KV head h // group."""
    return attention(q, k, v, scale, causal=False, group=group)[0]


# ------------------------------------------------------------- comparison
def flash_varlen(q, k, v, *, b, h, hk, d, scale, q_row_stride, k_row_stride, v_row_stride,
                 q_head_stride, k_head_stride, v_head_stride, o_row_stride, o_head_stride,
                 q_batch_stride=0, k_batch_stride=0, v_batch_stride=0, o_batch_stride=0,
                 seqlen_q=0, seqlen_k=0, total_q=0, cu_seqlens_q=None, cu_seqlens_k=None,
                 seqused_k=None, causal=False, local=False, window_left=-1, window_right=-1,
                 page_table=None, page_table_batch_stride=0, block_size=1, k_page_stride=0,
                 o, lse):
    """Variable-length attention forward in float64 over flat buffers:
    returns (o, lse) copies with every written position set.

    Follows ops/suite/dev/flash_varlen_fwd_kernel.py:22-320: per batch ``bid``
    the query rows are ``cu_seqlens_q[bid] ..`` (row-stride addressed) or
    ``bid * q_batch_stride`` with ``seqlen_q`` rows (:25-36), keys likewise
    (:37-48) with ``seqused_k`` overriding the key count (:49-52); query head
    ``hid`` reads key head ``hid // (h // hk)`` (:69-72).  Row ``i`` sees keys
    ``j < k_len`` with ``j <= i + k_len - q_len + window_right`` when causal or
    local and ``j >= i + k_len - q_len - window_left`` when local (:132-145).
    Paged K/V (:99-117): key ``j`` lives at ``page_table[bid *
    page_table_batch_stride + j // block_size] * k_page_stride + (j %
    block_size) * k_row_stride`` past the head offset, for K and V alike.
    LSE = log(sum(exp(scale * s))) in natural log, at ``h * total_q +
    (cu_seqlens_q[bid] or bid * seqlen_q) + i``; a row without keys gets O = 0
    and LSE = +inf (:309-312).  ``o`` and ``lse`` are the flat output
    buffers' initial contents (positions no row writes keep them).
    """
    q = np.asarray(q, dtype=np.float64).reshape(-1)
    k = np.asarray(k, dtype=np.float64).reshape(-1)
    v = np.asarray(v, dtype=np.float64).reshape(-1)
    ratio = h // hk
    out = np.asarray(o, dtype=np.float64).reshape(-1).copy()
    lse_out = np.asarray(lse, dtype=np.float64).reshape(-1).copy()
    dim = np.arange(d)
    for bid in range(b):
        if cu_seqlens_q is not None:
            q_bos, q_len = int(cu_seqlens_q[bid]), int(cu_seqlens_q[bid + 1]) - int(cu_seqlens_q[bid])
            q_off, o_off, lse_off = q_bos * q_row_stride, q_bos * o_row_stride, q_bos
        else:
            q_len = seqlen_q
            q_off, o_off, lse_off = bid * q_batch_stride, bid * o_batch_stride, bid * seqlen_q
        if cu_seqlens_k is not None:
            k_bos = int(cu_seqlens_k[bid])
            k_len = int(cu_seqlens_k[bid + 1]) - k_bos
            k_off, v_off = k_bos * k_row_stride, k_bos * v_row_stride
        else:
            k_len = seqlen_k
            k_off, v_off = bid * k_batch_stride, bid * v_batch_stride
        if seqused_k is not None:
            k_len = int(seqused_k[bid])
        keys = np.arange(k_len)
        if page_table is not None:
            phys = np.asarray(page_table).reshape(-1)[bid * page_table_batch_stride + keys // block_size]
            k_rows = phys.astype(np.int64) * k_page_stride + (keys % block_size) * k_row_stride
            v_rows = k_rows
        else:
            k_rows = k_off + keys * k_row_stride
            v_rows = v_off + keys * v_row_stride
        rows = np.arange(q_len)
        allowed = np.ones((q_len, k_len), dtype=bool)
        diag = rows[:, None] + (k_len - q_len)
        if causal or local:
            allowed &= keys[None, :] <= diag + window_right
        if local:
            allowed &= keys[None, :] >= diag - window_left
        for hid in range(h):
            kh = hid // ratio
            qt = q[q_off + hid * q_head_stride + rows[:, None] * q_row_stride + dim[None, :]]
            kt = k[k_rows[:, None] + kh * k_head_stride + dim[None, :]]
            vt = v[v_rows[:, None] + kh * v_head_stride + dim[None, :]]
            s = np.where(allowed, (qt @ kt.T) * float(scale), -np.inf)
            m = s.max(axis=1, keepdims=True) if k_len else np.full((q_len, 1), -np.inf)
            m_safe = np.where(np.isfinite(m), m, 0.0)
            p = np.exp(s - m_safe)
            l = p.sum(axis=1, keepdims=True)
            empty = l == 0
            out[o_off + hid * o_head_stride + rows[:, None] * o_row_stride + dim[None, :]] = (
                np.where(empty, 0.0, p / np.where(empty, 1.0, l)) @ vt if k_len else 0.0)
            with np.errstate(divide="ignore"):
                lse_out[hid * total_q + lse_off + rows] = np.where(empty[:, 0], np.inf, (m_safe + np.log(l))[:, 0])
    return out, lse_out


def isclose_verdict(actual, expected, rtol, atol, equal_nan=True):
    """(ok, max_abs_error) with the corpus comparator rule.

    Verdict is ``np.isclose`` (|a-b| <= atol + rtol*|b|) and the error metric
    ignores exactly-equal entries (ops/harness/opslib/compare.py:107-140).
    """
    a = np.asarray(actual).reshape(-1)
    b = np.asarray(expected).reshape(-1)
    close = np.isclose(a, b, rtol=rtol, atol=atol, equal_nan=equal_nan)
    with np.errstate(invalid="ignore", over="ignore"):
        delta = np.abs(a.astype(np.float64) - b.astype(np.float64))
        equal = a == b
        if equal_nan:
            equal = equal | (np.isnan(a) & np.isnan(b))
        err = float(np.where(equal, 0.0, delta).max(initial=0.0))
    return bool(close.all()), err


def max_rel_error(actual, expected, floor=1e-30) -> float:
    """max |a-b| / max(|b|, floor) over all entries (the north-star 'relative')."""
    a = np.asarray(actual, dtype=np.float64)
    b = np.asarray(expected, dtype=np.float64)
    return float((np.abs(a - b) / np.maximum(np.abs(b), floor)).max(initial=0.0))


def lse_equal_scores(score: float, n: int) -> float:
    """LSE of n equal scaled scores: s + log(n) (closed form used as a pin)."""
    return score + math.log(n)
