"""Pins of ``oracle.reference.flash_varlen`` (variable-length attention with
causal / local windows, GQA, seqused_k and paged K/V), each an independent
route to the same numbers: the dense ``attention`` oracle (itself pinned by the
reference's held attention fixtures) per sequence, closed forms of degenerate
windows, layout invariances, and a brute-force loop."""
import math

import numpy as np
import pytest

from oracle import inputs
from oracle import reference as ref


def seq_tensors(a, meta, bid):
    """(q [1,h,q_len,d], k/v [1,hk,k_len,d]) of one sequence, read through the
    case's own offsets (contiguous or strided layouts, no paging)."""
    h, hk, d = meta["h"], meta["hk"], meta["d"]
    if meta["is_cu_seqlens_q"]:
        q0, q1 = a["cu_seqlens_q_ptr"][bid], a["cu_seqlens_q_ptr"][bid + 1]
        qoff, ql = q0 * a["q_row_stride"], q1 - q0
    else:
        qoff, ql = bid * a["q_batch_stride"], a["seqlen_q"]
    if meta["is_cu_seqlens_k"]:
        k0, k1 = a["cu_seqlens_k_ptr"][bid], a["cu_seqlens_k_ptr"][bid + 1]
        koff, voff, kl = k0 * a["k_row_stride"], k0 * a["v_row_stride"], k1 - k0
    else:
        koff, voff, kl = bid * a["k_batch_stride"], bid * a["v_batch_stride"], a["seqlen_k"]
    if meta["is_seqused_k"]:
        kl = a["seqused_k_ptr"][bid]
    dim = np.arange(d)
    qt = np.stack([a["q_ptr"][qoff + hh * a["q_head_stride"] + np.arange(ql)[:, None] * a["q_row_stride"] + dim]
                   for hh in range(h)])
    kt = np.stack([a["k_ptr"][koff + hh * a["k_head_stride"] + np.arange(kl)[:, None] * a["k_row_stride"] + dim]
                   for hh in range(hk)])
    vt = np.stack([a["v_ptr"][voff + hh * a["v_head_stride"] + np.arange(kl)[:, None] * a["v_row_stride"] + dim]
                   for hh in range(hk)])
    return qt[None], kt[None], vt[None], int(ql), int(kl)


def split_out(a, meta, o, lse, bid, ql):
    h, d = meta["h"], meta["d"]
    if meta["is_cu_seqlens_q"]:
        q0 = a["cu_seqlens_q_ptr"][bid]
        ooff, loff = q0 * a["o_row_stride"], q0
    else:
        ooff, loff = bid * a["o_batch_stride"], bid * a["seqlen_q"]
    dim = np.arange(d)
    ot = np.stack([o[ooff + hh * a["o_head_stride"] + np.arange(ql)[:, None] * a["o_row_stride"] + dim]
                   for hh in range(h)])
    lt = np.stack([lse[hh * a["total_q"] + loff + np.arange(ql)] for hh in range(h)])
    return ot, lt


@pytest.mark.parametrize("kw", [
    dict(),                                             # the reference case (2,17,19,4,2,16)
    dict(batches=3, max_q=17, max_k=19, h=6, hk=2, d=32),
    dict(var_q=False, var_k=False),                     # batch-stride addressing
    dict(strided=True),                                 # padded K/V heads/rows/batches
    dict(var_q=False, var_k=True, strided=True),
])
def test_dense_equals_attention_per_sequence(kw):
    a, meta = inputs.varlen_case(**kw)
    o, lse = inputs.varlen_oracle(a, meta)
    for bid in range(a["b"]):
        qt, kt, vt, ql, kl = seq_tensors(a, meta, bid)
        eo, el = ref.attention(qt, kt, vt, meta["scale_softmax"], causal=False)
        ot, lt = split_out(a, meta, o, lse, bid, ql)
        assert np.allclose(ot, eo[0], atol=1e-12) and np.allclose(lt, el[0], atol=1e-12)


def test_causal_square_equals_attention_causal():
    a, meta = inputs.varlen_case(max_q=19, max_k=19, causal=True, window_right=0)
    # sequence lengths differ between q (19-2b) and k (19-3b): take batch 0 only
    o, lse = inputs.varlen_oracle(a, meta)
    qt, kt, vt, ql, kl = seq_tensors(a, meta, 0)
    assert ql == kl
    eo, el = ref.attention(qt, kt, vt, meta["scale_softmax"], causal=True)
    ot, lt = split_out(a, meta, o, lse, 0, ql)
    assert np.allclose(ot, eo[0], atol=1e-12) and np.allclose(lt, el[0], atol=1e-12)


def test_bottom_right_causal_brute_force():
    """q_len < k_len: row i sees keys j <= i + k_len - q_len + wr (brute force)."""
    a, meta = inputs.varlen_case(batches=2, max_q=5, max_k=9, h=2, hk=1, d=4, causal=True, window_right=0)
    o, lse = inputs.varlen_oracle(a, meta)
    for bid in range(2):
        qt, kt, vt, ql, kl = seq_tensors(a, meta, bid)
        qt, kt, vt = (t.astype(np.float64) for t in (qt, kt, vt))
        ot, lt = split_out(a, meta, o, lse, bid, ql)
        for hh in range(2):
            for i in range(ql):
                js = [j for j in range(kl) if j <= i + kl - ql]
                sc = [meta["scale_softmax"] * sum(float(qt[0, hh, i, e]) * float(kt[0, 0, j, e]) for e in range(4))
                      for j in js]
                mx = max(sc)
                w = [math.exp(s - mx) for s in sc]
                for e in range(4):
                    val = sum(wj * float(vt[0, 0, j, e]) for wj, j in zip(w, js)) / sum(w)
                    assert abs(ot[hh, i, e] - val) < 1e-12
                assert abs(lt[hh, i] - (mx + math.log(sum(w)))) < 1e-12


def test_local_window_zero_picks_own_key_and_huge_window_is_dense():
    a, meta = inputs.varlen_case(max_q=19, max_k=19, var_q=False, var_k=False, local=True,
                                 window_left=0, window_right=0)
    o, lse = inputs.varlen_oracle(a, meta)
    for bid in range(2):
        qt, kt, vt, ql, kl = seq_tensors(a, meta, bid)
        ot, lt = split_out(a, meta, o, lse, bid, ql)
        for hh in range(meta["h"]):
            kh = hh // meta["h_hk_ratio"]
            assert np.allclose(ot[hh], vt[0, kh, :ql], atol=1e-15)
            own = meta["scale_softmax"] * (qt[0, hh] * kt[0, kh, :ql]).sum(axis=1)
            assert np.allclose(lt[hh], own, atol=1e-12)
    a, meta = inputs.varlen_case(local=True, window_left=10**6, window_right=10**6)
    o1, l1 = inputs.varlen_oracle(a, meta)
    meta["is_local"] = False
    o2, l2 = inputs.varlen_oracle(a, meta)
    assert np.array_equal(o1, o2) and np.array_equal(l1, l2)


def test_fully_masked_rows_are_zero_with_infinite_lse():
    """A left window beyond every key (row i sees j >= i + k_len - q_len - wl
    with wl very negative) leaves rows empty: O = 0, LSE = +inf."""
    a, meta = inputs.varlen_case(local=True, window_left=-100, window_right=100)
    o, lse = inputs.varlen_oracle(a, meta)
    for bid in range(2):
        _, _, _, ql, _ = seq_tensors(a, meta, bid)
        ot, lt = split_out(a, meta, o, lse, bid, ql)
        assert np.all(ot == 0.0) and np.all(np.isinf(lt)) and np.all(lt > 0)


def test_paged_and_seqused_and_gqa_invariances():
    base, meta = inputs.varlen_case(batches=3, max_q=17, max_k=40, h=4, hk=2, d=16)
    o0, l0 = inputs.varlen_oracle(base, meta)
    for bs in (1, 4, 16):
        a, m = inputs.varlen_case(batches=3, max_q=17, max_k=40, h=4, hk=2, d=16, paged=True, block_size=bs)
        o, lse = inputs.varlen_oracle(a, m)
        assert np.array_equal(o, o0) and np.array_equal(lse, l0)
    # seqused_k trims keys: equal to the dense oracle on the trimmed sequences
    a, m = inputs.varlen_case(batches=2, max_q=9, max_k=12, h=2, hk=1, d=8, seqused_trim=3)
    o, lse = inputs.varlen_oracle(a, m)
    for bid in range(2):
        qt, kt, vt, ql, kl = seq_tensors(a, m, bid)
        assert kl == 12 - 3 * bid - 3
        eo, el = ref.attention(qt, kt, vt, m["scale_softmax"], causal=False)
        ot, lt = split_out(a, m, o, lse, bid, ql)
        assert np.allclose(ot, eo[0], atol=1e-12) and np.allclose(lt, el[0], atol=1e-12)
    # GQA: duplicating each KV head into its query heads gives the same result
    qt, kt, vt, ql, kl = seq_tensors(base, meta, 1)
    eo, _ = ref.attention(qt, np.repeat(kt, 2, axis=1), np.repeat(vt, 2, axis=1), meta["scale_softmax"],
                          causal=False)
    ot, _ = split_out(base, meta, o0, l0, 1, ql)
    assert np.allclose(ot, eo[0], atol=1e-12)


def test_untouched_positions_keep_their_initial_values():
    a, meta = inputs.varlen_case(var_q=False, var_k=False)
    o, lse = inputs.varlen_oracle(a, meta)
    assert not np.any(o == -0.875) and np.all(np.isfinite(lse))
