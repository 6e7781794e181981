"""GPU parity of flash_varlen_fwd_kernel (variable-length attention with
cu_seqlens / fixed-length batches, seqused_k, GQA, causal and local windows,
paged K/V) through the C ABI against the CPU oracle on the same inputs.

Cases: the reference's own case shapes (ops/suite/dev/flash_varlen_fwd_kernel.py
:320-330, d = 16/32/64) and MFMA-path cases at d = 64/128 with the features
the reference case layer leaves at their defaults.  Bars are the reference
case's own (:348-354 with :412): fp32 1e-4, bf16 1e-2, fp16 3e-2 (rtol = atol,
np.isclose form) on O -- including the positions no row writes, which must
keep their initial value -- and on LSE (+inf for rows without keys).
"""
import numpy as np
import pytest

torch = pytest.importorskip("torch")

from compiler_amd import operators as ops  # noqa: E402
from compiler_amd import runtime as rt  # noqa: E402
from compiler_amd.operators import _VARLEN_SCALARS, _VARLEN_VIEWS  # noqa: E402
from oracle import inputs  # noqa: E402
from oracle import reference as ref  # noqa: E402

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
TD = {"float32": torch.float32, "bfloat16": torch.bfloat16, "float16": torch.float16}
BAR = {"float32": 1e-4, "bfloat16": 1e-2, "float16": 3e-2}


def run(a, meta, dt):
    t = {}
    for n in _VARLEN_VIEWS:
        arr = np.ascontiguousarray(a[n])
        if arr.dtype == np.uint64:
            arr = arr.view(np.int64)
        t[n] = torch.from_numpy(arr).to(DEV)
        if n in ("q_ptr", "k_ptr", "v_ptr", "o_ptr"):
            t[n] = t[n].to(TD[dt])
    rounded = {n: t[n].float().cpu().numpy() for n in ("q_ptr", "k_ptr", "v_ptr", "o_ptr")}
    merged = {**a, **meta}
    ops.flash_varlen_fwd_kernel(**t, **{n: merged[n] for n in _VARLEN_SCALARS}, sync=True)
    expect_o, expect_lse = inputs.varlen_oracle({**a, **rounded}, meta)
    return t["o_ptr"].float().cpu().numpy(), t["softmax_lse_ptr"].cpu().numpy(), expect_o, expect_lse


def check(a, meta, dt, kernel_prefix):
    o, lse, eo, el = run(a, meta, dt)
    assert rt.module().last_kernel.startswith(kernel_prefix), rt.module().last_kernel
    bar = BAR[dt]
    ok, err = ref.isclose_verdict(o, eo, bar, bar)
    assert ok, f"O max err {err}"
    ok, err = ref.isclose_verdict(lse, el, bar, bar)
    assert ok, f"LSE max err {err}"
    assert np.array_equal(np.isinf(lse), np.isinf(el))


REF_SHAPES = [(2, 17, 19, 4, 2, 16), (3, 17, 19, 6, 2, 32), (3, 33, 35, 6, 2, 32), (4, 65, 67, 8, 4, 64),
              (2, 17, 35, 4, 2, 16, 0, 0, 1), (2, 17, 35, 4, 2, 16, 1, 1, 1), (2, 17, 35, 4, 2, 16, 1, 0, 1),
              (2, 17, 35, 4, 2, 16, 0, 1, 1), (3, 17, 19, 4, 2, 16)]


@pytest.mark.parametrize("dt", ["float16", "bfloat16", "float32"])
@pytest.mark.parametrize("shape", REF_SHAPES)
def test_reference_case_shapes(shape, dt):
    b, mq, mk, h, hk, d = shape[:6]
    var_q, var_k, strided = (True, True, False) if len(shape) == 6 else map(bool, shape[6:])
    a, meta = inputs.varlen_case(b, mq, mk, h, hk, d, var_q=var_q, var_k=var_k, strided=strided)
    mfma = dt != "float32" and d in (64, 128) and not strided
    check(a, meta, dt, "g950_attn_fwd_" if mfma else "g950_attn_varlen_general")


MFMA_CASES = {
    "dense": dict(batches=3, max_q=700, max_k=900, h=8, hk=2, d=128),
    "causal": dict(batches=3, max_q=700, max_k=900, h=8, hk=2, d=128, causal=True, window_right=0),
    "causal_square": dict(batches=2, max_q=600, max_k=600, h=4, hk=4, d=64, var_q=False, var_k=False,
                          causal=True, window_right=0),
    "local": dict(batches=3, max_q=700, max_k=900, h=8, hk=2, d=128, local=True, window_left=100,
                  window_right=50),
    "local_empty_rows": dict(batches=2, max_q=300, max_k=300, h=4, hk=2, d=64, local=True, window_left=-40,
                             window_right=80),
    "paged16": dict(batches=3, max_q=500, max_k=777, h=8, hk=2, d=128, paged=True, block_size=16),
    "paged64_causal": dict(batches=3, max_q=500, max_k=777, h=8, hk=2, d=64, paged=True, block_size=64,
                           causal=True, window_right=0),
    "seqused": dict(batches=3, max_q=400, max_k=520, h=8, hk=8, d=128, seqused_trim=37),
    "fixed_len": dict(batches=2, max_q=513, max_k=700, h=4, hk=2, d=128, var_q=False, var_k=False),
}


@pytest.mark.parametrize("dt", ["bfloat16", "float16"])
@pytest.mark.parametrize("case", sorted(MFMA_CASES))
def test_mfma_varlen_features(case, dt):
    """Every feature on the MFMA kernels; the paging mode is compiled into
    the kernel: contiguous rows (`_varlen`), pages of whole 64-key tiles
    (`_varlen_pt`), other page sizes (`_varlen_pl`)."""
    c = MFMA_CASES[case]
    a, meta = inputs.varlen_case(**c)
    suffix = "" if not c.get("paged") else "_pt" if c["block_size"] % 64 == 0 else "_pl"
    name = f"g950_attn_fwd_{'bf16' if dt == 'bfloat16' else 'f16'}_d{c['d']}_varlen{suffix}"
    check(a, meta, dt, name)
    assert rt.module().last_kernel == name


@pytest.mark.parametrize("paged", [False, True])
@pytest.mark.parametrize("dt", ["bfloat16", "float16"])
def test_mfma_varlen_empty_sequences(dt, paged):
    """Whole sequences without keys or queries on the MFMA kernels, inside
    the contract that seqlen_q bounds every sequence's rows (the reference's
    grid has ceil(seqlen_q / BLOCK_M) q-blocks, flash_varlen_fwd_kernel.py:470):
    sequence 1 gets seqused_k = 0 (no key tile at all: every row O = 0,
    LSE = +inf, :309-312); sequence 2 gets no queries (equal cu_seqlens_q
    entries); sequence 3 keeps its 294 queries over 100 keys, so under the
    bottom-right causal alignment its first 194 rows see no key; the rows
    after cu_seqlens_q[-1] belong to no sequence and keep their initial
    values (O -0.875, LSE -inf)."""
    extra = dict(paged=True, block_size=64) if paged else {}
    a, meta = inputs.varlen_case(batches=4, max_q=300, max_k=400, h=8, hk=2, d=128, seqused_trim=5,
                                 causal=True, window_right=0, **extra)
    a = dict(a)
    used = a["seqused_k_ptr"].copy()
    used[1] = 0
    used[3] = 100
    a["seqused_k_ptr"] = used
    cu = a["cu_seqlens_q_ptr"].copy()
    q3 = cu[4] - cu[3]
    cu[3] = cu[2]
    cu[4] = cu[2] + q3
    a["cu_seqlens_q_ptr"] = cu
    o, lse, eo, el = run(a, meta, dt)
    assert rt.module().last_kernel.endswith("_varlen_pt" if paged else "_varlen"), rt.module().last_kernel
    o3, l2 = o.reshape(-1, 8, 128), lse.reshape(8, -1)
    assert np.all(o3[cu[1]:cu[2]] == 0.0)
    assert np.all(np.isposinf(l2[:, cu[1]:cu[2]]))
    assert int(np.isposinf(l2[:, cu[3]:cu[4]]).sum()) == 8 * 194
    assert np.all(o3[cu[4]:] == -0.875) and np.all(np.isneginf(l2[:, cu[4]:]))
    bar = BAR[dt]
    ok, err = ref.isclose_verdict(o, eo, bar, bar)
    assert ok, f"O max err {err}"
    ok, err = ref.isclose_verdict(lse, el, bar, bar)
    assert ok, f"LSE max err {err}"
    assert np.array_equal(np.isinf(lse), np.isinf(el))


def test_mfma_varlen_random_sweep():
    """Sixteen seeded varlen cases on the MFMA kernels: 1-4 sequences of up
    to 700 queries and 900 keys, GQA 1/2/4 over 1-2 KV heads, head dim 64 or
    128, and a random mix of the features -- causal, a local window (random
    left/right sizes, some of them negative), paged K/V with 16-, 64- or
    128-key pages, seqused_k trimming, fixed-length rows -- bf16 and fp16
    in turn; O and LSE against the oracle at the case's bar, and all three
    paging forms of the kernel reached."""
    rng = np.random.default_rng(90210)
    ran = set()
    for case in range(16):
        dt = ("bfloat16", "float16")[case % 2]
        batches = int(rng.integers(1, 5))
        max_q = int(rng.integers(2 * batches + 1, 701))
        max_k = int(rng.integers(3 * batches + 1, 901))
        hk = int(rng.integers(1, 3))
        kw = dict(batches=batches, max_q=max_q, max_k=max_k, hk=hk, h=hk * (1, 2, 4)[int(rng.integers(0, 3))],
                  d=(64, 128)[int(rng.integers(0, 2))], seed=1000 + case)
        feature = int(rng.integers(0, 4))
        if feature == 1:
            kw.update(causal=True, window_right=0)
        elif feature == 2:
            kw.update(local=True, window_left=int(rng.integers(-50, 300)), window_right=int(rng.integers(-50, 300)))
        elif feature == 3:
            kw.update(var_q=False, var_k=False)
        if feature != 3 and rng.random() < 0.5:
            kw.update(paged=True, block_size=(16, 64, 128)[int(rng.integers(0, 3))])
        if rng.random() < 0.3:
            kw.update(seqused_trim=int(rng.integers(1, 3 * batches + 1)))
        a, meta = inputs.varlen_case(**kw)
        o, lse, eo, el = run(a, meta, dt)
        kern = rt.module().last_kernel
        ran.add(kern.split("_varlen")[-1])
        tag = f"case {case}: {dt} {kw} ({kern})"
        bar = BAR[dt]
        ok, err = ref.isclose_verdict(o, eo, bar, bar)
        assert ok, f"{tag}: O max err {err}"
        ok, err = ref.isclose_verdict(lse, el, bar, bar)
        assert ok, f"{tag}: LSE max err {err}"
        assert np.array_equal(np.isinf(lse), np.isinf(el)), tag
    assert {"", "_pt", "_pl"} <= ran, sorted(ran)


def test_general_kernel_features_fp32():
    """The same features through the fp32 one-thread-per-row kernel."""
    for kw in (dict(causal=True, window_right=0), dict(local=True, window_left=3, window_right=2),
               dict(paged=True, block_size=4), dict(seqused_trim=2), dict(strided=True, causal=True,
                                                                          window_right=1)):
        a, meta = inputs.varlen_case(batches=3, max_q=17, max_k=24, h=4, hk=2, d=16, **kw)
        check(a, meta, "float32", "g950_attn_varlen_general")


def test_invalid_device_lengths_leave_memory_alone():
    """cu_seqlens that would address past q/o make that sequence empty: no
    write outside the views (guard bytes behind o stay), the valid sequence
    is still right."""
    a, meta = inputs.varlen_case(batches=2, max_q=17, max_k=19, h=4, hk=2, d=64)
    a = dict(a)
    cu = a["cu_seqlens_q_ptr"].copy()
    cu[2] = cu[1] + 10_000          # second sequence claims rows far past the buffers
    a["cu_seqlens_q_ptr"] = cu
    t = {n: torch.from_numpy(np.ascontiguousarray(a[n]).view(np.int64) if a[n].dtype == np.uint64
                             else np.ascontiguousarray(a[n])).to(DEV) for n in _VARLEN_VIEWS}
    for n in ("q_ptr", "k_ptr", "v_ptr"):
        t[n] = t[n].to(torch.bfloat16)
    guard = torch.full((t["o_ptr"].numel() + 64,), 5.0, dtype=torch.bfloat16, device=DEV)
    guard[: t["o_ptr"].numel()] = -0.875
    t["o_ptr"] = guard[: t["o_ptr"].numel()]
    merged = {**a, **meta}
    ops.flash_varlen_fwd_kernel(**t, **{n: merged[n] for n in _VARLEN_SCALARS}, sync=True)
    assert torch.all(guard[t["o_ptr"].numel():] == 5.0)
    first = int(a["cu_seqlens_q_ptr"][1]) * meta["h"] * meta["d"]
    rounded = {n: t[n].float().cpu().numpy() for n in ("q_ptr", "k_ptr", "v_ptr")}
    ok_case = dict(a, **rounded)
    ok_case["cu_seqlens_q_ptr"] = inputs.varlen_case(batches=2, max_q=17, max_k=19, h=4, hk=2,
                                                     d=64)[0]["cu_seqlens_q_ptr"]
    eo, _ = inputs.varlen_oracle(dict(ok_case, o_ptr=np.full(t["o_ptr"].numel(), -0.875, np.float32)), meta)
    got = t["o_ptr"].float().cpu().numpy()
    ok, err = ref.isclose_verdict(got[:first], eo[:first], 1e-2, 1e-2)
    assert ok, err
    assert np.all(got[first:] == -0.875)
