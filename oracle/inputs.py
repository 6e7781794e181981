"""Seeded synthetic inputs for the five hot-path configurations -- TEST
INFRASTRUCTURE (shared by tests, smoke and bench so that every leg sees the
same data).

Every distribution choice the configurations leave open is fixed here:
  * ``N(0, s)`` with a bare number means standard deviation s (std 3 for the
    reduction inputs, std 0.1 for beta), as the reference scales its normals
    (ops/suite/perf/softmax.py:57 ``standard_normal * 3.0``).
  * GEMM operands ``N(0, 1/sqrt(K))`` are read as VARIANCE 1/sqrt(K) (std
    K**-0.25) so that C ~ N(0, 1); the std reading makes |C| ~ 0.01, below the
    bf16 absolute tolerance, which would make the parity test vacuous.
  * Seeds: configs 1 and 3 state theirs (0 and 1); configs 2, 4 and 5 state
    none and use 2, 4 and 5.
  * bf16 operands are produced by rounding float32 draws with the reference
    RNE rule (``oracle.reference.bf16_round``).
Generation uses ``numpy.random.default_rng`` (PCG64).
"""
from __future__ import annotations

import numpy as np

from .reference import bf16_round

SEEDS = {"c1": 0, "c2": 2, "c3": 1, "c4": 4, "c5": 5}


def config1(rows=4096, cols=4096, seed=SEEDS["c1"]):
    """x[rows, cols] ~ N(0,1) fp32, weight ~ U(0.5,1.5) fp32, eps 1e-6."""
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((rows, cols), dtype=np.float32)
    w = rng.uniform(0.5, 1.5, cols).astype(np.float32)
    return {"x": x, "w": w, "eps": 1e-6}


def config2(rows=8191, cols=3000, seed=SEEDS["c2"], outlier_frac=0.01):
    """x ~ N(0, std 3) with 1% of entries set to +-60, bf16-rounded; LayerNorm
    gamma ~ U(0.5,1.5), beta ~ N(0, std 0.1), eps 1e-5 (all bf16-rounded)."""
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((rows, cols), dtype=np.float32) * np.float32(3.0)
    n = rows * cols
    count = int(round(n * outlier_frac))
    if count:
        idx = rng.choice(n, size=count, replace=False)
        sign = np.where(rng.random(count) < 0.5, -60.0, 60.0).astype(np.float32)
        x.reshape(-1)[idx] = sign
    gamma = rng.uniform(0.5, 1.5, cols).astype(np.float32)
    beta = (rng.standard_normal(cols) * 0.1).astype(np.float32)
    return {"x": bf16_round(x), "gamma": bf16_round(gamma), "beta": bf16_round(beta),
            "eps": 1e-5}


def config3(m=8192, n=8192, k=8192, seed=SEEDS["c3"]):
    """A[m,k] row-major, B logical [k,n] stored column-major as Bt[n,k];
    entries ~ N(0, variance 1/sqrt(K)), bf16-rounded.  Returns float32 arrays
    holding bf16 values: ``a`` [m,k] and ``bt`` [n,k] (B = bt.T)."""
    rng = np.random.default_rng(seed)
    std = np.float32(k ** -0.25)
    a = rng.standard_normal((m, k), dtype=np.float32) * std
    bt = rng.standard_normal((n, k), dtype=np.float32) * std
    return {"a": bf16_round(a), "bt": bf16_round(bt)}


def config4(batch=4, hq=32, hkv=8, seq=4096, dim=128, seed=SEEDS["c4"]):
    """Q[batch,hq,seq,dim], K/V[batch,hkv,seq,dim] ~ N(0,1), bf16-rounded."""
    rng = np.random.default_rng(seed)
    q = rng.standard_normal((batch, hq, seq, dim), dtype=np.float32)
    k = rng.standard_normal((batch, hkv, seq, dim), dtype=np.float32)
    v = rng.standard_normal((batch, hkv, seq, dim), dtype=np.float32)
    return {"q": bf16_round(q), "k": bf16_round(k), "v": bf16_round(v),
            "scale": 1.0 / np.sqrt(dim)}


def config5(m=4096, n=8192, k=8192, seed=SEEDS["c5"]):
    """A int8[m,k], B int8 logical [k,n] stored K-contiguous as Bt[n,k],
    uniform integers in [-127,127]; sa[m], sb[n] ~ U(0.001, 0.02) fp32."""
    rng = np.random.default_rng(seed)
    a = rng.integers(-127, 128, size=(m, k), dtype=np.int8)
    bt = rng.integers(-127, 128, size=(n, k), dtype=np.int8)
    sa = rng.uniform(0.001, 0.02, m).astype(np.float32)
    sb = rng.uniform(0.001, 0.02, n).astype(np.float32)
    return {"a": a, "bt": bt, "sa": sa, "sb": sb}


def varlen_case(batches=2, max_q=17, max_k=19, h=4, hk=2, d=16, var_q=True, var_k=True,
                strided=False, seed=20260826, paged=False, block_size=16, causal=False,
                local=False, window_left=-1, window_right=-1, seqused_trim=0):
    """A flash_varlen_fwd_kernel case over flat fp32 buffers, laid out as the
    reference case layer lays it out (ops/suite/dev/flash_varlen_fwd_kernel.py
    make_case: sequence b has max_q - 2b query and max_k - 3b key rows, q/k/v
    ~ N(0, 0.25), o pre-filled with -0.875, lse with -inf, row stride h*d or
    hk*d, head stride d; ``strided`` pads K and V heads/rows/batches by
    3/5/7 and 7/11/13 elements).  ``paged`` re-homes every sequence's keys
    into pages of ``block_size`` rows placed in a shuffled page pool (one
    page table row per batch); ``seqused_trim`` keys are dropped from the end
    of every sequence through ``seqused_k``.  Returns (args, meta): args by
    the reference argument names (numpy arrays and ints), meta the
    constexprs with semantics."""
    import math
    rng = np.random.default_rng(seed)
    q_lens = np.array([max_q - 2 * i for i in range(batches)], dtype=np.int32)
    k_lens = np.array([max_k - 3 * i for i in range(batches)], dtype=np.int32)
    if not var_q:
        q_lens[:] = max_q
    if not var_k:
        k_lens[:] = max_k
    if q_lens.min() <= 0 or k_lens.min() <= 0:
        raise ValueError("too many batches for the maximum lengths")
    cu_q = np.concatenate(([0], np.cumsum(q_lens))).astype(np.int32)
    cu_k = np.concatenate(([0], np.cumsum(k_lens))).astype(np.int32)
    total_q, total_k = int(cu_q[-1]), int(cu_k[-1])
    q_rows = total_q if var_q else batches * max_q
    k_rows = total_k if var_k else batches * max_k
    q = rng.normal(0.0, 0.25, q_rows * h * d).astype(np.float32)
    kl = rng.normal(0.0, 0.25, (k_rows, hk, d)).astype(np.float32)
    vl = rng.normal(0.0, 0.25, (k_rows, hk, d)).astype(np.float32)
    a = {"q_ptr": q, "o_ptr": np.full(q_rows * h * d, -0.875, dtype=np.float32),
         "softmax_lse_ptr": np.full(h * max(total_q, q_rows), -np.inf, dtype=np.float32),
         "p_ptr": np.zeros(1, np.float32), "philox_args": np.array([seed, 0], np.uint64),
         "alibi_slopes_ptr": np.zeros(1, np.float32),
         "cu_seqlens_q_ptr": cu_q, "cu_seqlens_k_ptr": cu_k, "seqused_k_ptr": k_lens - seqused_trim,
         "q_row_stride": h * d, "q_head_stride": d, "o_row_stride": h * d, "o_head_stride": d,
         "q_batch_stride": max_q * h * d, "o_batch_stride": max_q * h * d,
         "b": batches, "bk": batches, "seqlen_q": max_q, "seqlen_k": max_k,
         "seqlen_q_rounded": (max_q + 127) // 128 * 128, "seqlen_k_rounded": (max_k + 31) // 32 * 32,
         "total_q": max(total_q, q_rows) if not var_q else total_q,
         "page_table_ptr": np.zeros(1, np.int32), "k_page_stride": 0}
    if not var_q:
        a["total_q"] = batches * max_q
    starts = cu_k[:-1] if var_k else np.arange(batches) * max_k
    if paged:
        # pages of block_size key rows; row stride hk*d (k and v share it)
        row = hk * d
        pages_per = [(int(n) + block_size - 1) // block_size for n in k_lens]
        npages = sum(pages_per)
        order = rng.permutation(npages)
        kp = np.full(npages * block_size * row, -3.0, np.float32)
        vp = np.full(npages * block_size * row, -3.0, np.float32)
        table = np.zeros((batches, max(pages_per)), np.int32)
        nxt = 0
        for bi in range(batches):
            for pg in range(pages_per[bi]):
                phys = int(order[nxt]); nxt += 1
                table[bi, pg] = phys
                lo = pg * block_size
                hi = min(int(k_lens[bi]), lo + block_size)
                src = slice(int(starts[bi]) + lo, int(starts[bi]) + hi)
                dst = phys * block_size * row
                kp[dst:dst + (hi - lo) * row] = kl[src].reshape(-1)
                vp[dst:dst + (hi - lo) * row] = vl[src].reshape(-1)
        a.update({"k_ptr": kp, "v_ptr": vp, "k_row_stride": row, "v_row_stride": row,
                  "k_head_stride": d, "v_head_stride": d, "k_batch_stride": 0, "v_batch_stride": 0,
                  "page_table_ptr": table.reshape(-1), "k_page_stride": block_size * row})
        pt_stride = table.shape[1]
    else:
        pt_stride = 0
        for name, src, pads in (("k", kl, (3, 5, 7)), ("v", vl, (7, 11, 13))):
            if strided:
                hs = d + pads[0]
                rs = hk * hs + pads[1]
                bs = max_k * rs + pads[2]
            else:
                hs, rs, bs = d, hk * d, max_k * hk * d
            extent = (k_rows * rs) if var_k else batches * bs
            buf = np.full(max(extent, 1), -3.0, np.float32)
            for bi in range(batches):
                base = int(starts[bi]) * rs if var_k else bi * bs
                n = int(k_lens[bi])
                idx = (base + np.arange(n)[:, None, None] * rs + np.arange(hk)[None, :, None] * hs
                       + np.arange(d)[None, None, :])
                buf[idx] = src[int(starts[bi]):int(starts[bi]) + n]
            a.update({f"{name}_ptr": buf, f"{name}_row_stride": rs, f"{name}_head_stride": hs,
                      f"{name}_batch_stride": bs})
    scale = 1.0 / math.sqrt(d)
    meta = {"is_cu_seqlens_q": var_q, "is_cu_seqlens_k": var_k and not paged,
            "is_seqused_k": bool(seqused_trim) or paged, "h": h, "hk": hk, "h_hk_ratio": h // hk,
            "d": d, "scale_softmax": scale, "scale_softmax_log2": scale * math.log2(math.e),
            "is_causal": causal, "is_local": local, "window_size_left": window_left,
            "window_size_right": window_right, "is_paged": paged, "block_size": block_size,
            "page_table_batch_stride": pt_stride, "is_softcap": False, "softcap": 0.0,
            "is_dropout": False, "p_dropout": 1.0, "rp_dropout": 1.0, "p_dropout_in_uint8_t": 255,
            "return_softmax": False, "seqlenq_ngroups_swapped": False, "is_alibi": False,
            "alibi_slopes_batch_stride": 0}
    return a, meta


def varlen_oracle(a, meta):
    """The oracle's outputs for a ``varlen_case`` (inputs taken as given)."""
    from .reference import flash_varlen
    return flash_varlen(
        a["q_ptr"], a["k_ptr"], a["v_ptr"], b=a["b"], h=meta["h"], hk=meta["hk"], d=meta["d"],
        scale=meta["scale_softmax"], q_row_stride=a["q_row_stride"], k_row_stride=a["k_row_stride"],
        v_row_stride=a["v_row_stride"], q_head_stride=a["q_head_stride"], k_head_stride=a["k_head_stride"],
        v_head_stride=a["v_head_stride"], o_row_stride=a["o_row_stride"], o_head_stride=a["o_head_stride"],
        q_batch_stride=a["q_batch_stride"], k_batch_stride=a["k_batch_stride"],
        v_batch_stride=a["v_batch_stride"], o_batch_stride=a["o_batch_stride"], seqlen_q=a["seqlen_q"],
        seqlen_k=a["seqlen_k"], total_q=a["total_q"],
        cu_seqlens_q=a["cu_seqlens_q_ptr"] if meta["is_cu_seqlens_q"] else None,
        cu_seqlens_k=a["cu_seqlens_k_ptr"] if meta["is_cu_seqlens_k"] else None,
        seqused_k=a["seqused_k_ptr"] if meta["is_seqused_k"] else None,
        causal=meta["is_causal"], local=meta["is_local"], window_left=meta["window_size_left"],
        window_right=meta["window_size_right"],
        page_table=a["page_table_ptr"] if meta["is_paged"] else None,
        page_table_batch_stride=meta["page_table_batch_stride"], block_size=meta["block_size"],
        k_page_stride=a["k_page_stride"], o=a["o_ptr"], lse=a["softmax_lse_ptr"])
