"""gfx950 micro-probes: the hardware rates the kernel designs are built on.

Measurement only (``python bench.py --hw-probe``): loads
``lib/g950_probes.hsaco`` (``compiler_amd/csrc/g950_probes.hip``) with the HIP
module API and reports, per probe, the mean over waves of the best-of-four
``s_memtime`` cycle count, at 1, 4 and 8 waves per CU (one workgroup per CU,
256 workgroups).  ``s_memtime`` counts shader-clock cycles; the ``clock``
entry checks that against the 100 MHz real-time counter.
"""
from __future__ import annotations

import ctypes
from pathlib import Path

from .build import PROBES, STAMPS

RATE = {
    "lds_b128": ("g950p_lds_b128", "64 ds_read_b128 (1 KiB each)", 64 * 1024),
    "lds_tr_b16": ("g950p_lds_tr_b16", "64 ds_read_b64_tr_b16 (512 B each)", 64 * 512),
    "exp": ("g950p_exp", "256 v_exp_f32, 8 chains", 0),
    "fma": ("g950p_fma", "256 v_fma_f32, 8 chains", 0),
    "mfma": ("g950p_mfma", "64 v_mfma_f32_32x32x16_bf16, 4 accumulators", 0),
    "mfma_exp2": ("g950p_mfma_exp2", "64 MFMA, each + 2 v_exp_f32", 0),
    "mfma_fma4": ("g950p_mfma_fma4", "64 MFMA, each + 4 v_fma_f32", 0),
    "mfma_fma8": ("g950p_mfma_fma8", "64 MFMA, each + 8 v_fma_f32", 0),
    "mfma_lds": ("g950p_mfma_lds", "64 MFMA, each + 1 ds_read_b128 (4 in flight)", 0),
    "mfma_mix": ("g950p_mfma_mix", "64 MFMA, each + one softmax step (fma, exp, add, 1/2 cvt_pk, 9/16 max3)", 0),
    "mfma_mix_lds": ("g950p_mfma_mix_lds", "64 MFMA, each + the softmax step + 1 ds_read_b128", 0),
}
ISSUE = {
    "issue_lds_dma": ("g950p_issue_lds_dma", "8 global_load_lds_dwordx4 per wave"),
    "issue_global": ("g950p_issue_global", "8 global_load_dwordx4 per wave"),
}
BLOCKS = 256


class _Hip:
    def __init__(self):
        self.lib = ctypes.CDLL("libamdhip64.so")
        self.mod = ctypes.c_void_p()
        path = Path(PROBES)
        if not path.exists():
            raise RuntimeError(f"{path} is not built (run __graft_entry__.build())")
        rc = self.lib.hipModuleLoad(ctypes.byref(self.mod), str(path).encode())
        if rc:
            raise RuntimeError(f"hipModuleLoad({path}) failed: {rc}")

    def launch(self, name, threads, args, stream):
        f = ctypes.c_void_p()
        rc = self.lib.hipModuleGetFunction(ctypes.byref(f), self.mod, name.encode())
        if rc:
            raise RuntimeError(f"hipModuleGetFunction({name}) failed: {rc}")
        vals = [a if isinstance(a, ctypes._SimpleCData) else ctypes.c_void_p(a) for a in args]
        ptrs = (ctypes.c_void_p * len(vals))(*[ctypes.addressof(v) for v in vals])
        rc = self.lib.hipModuleLaunchKernel(f, BLOCKS, 1, 1, threads, 1, 1, 0, stream, ptrs, None)
        if rc:
            raise RuntimeError(f"hipModuleLaunchKernel({name}) failed: {rc}")


def run(torch) -> dict:
    """All probes on cuda:0; returns {probe: {waves_per_cu: result}}."""
    hip = _Hip()
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    out = torch.zeros(BLOCKS * 16 * 2, dtype=torch.int64, device="cuda")
    sink = torch.zeros(512 * 4, dtype=torch.int32, device="cuda")
    res: dict = {}
    for key, (name, what, nbytes) in RATE.items():
        res[key] = {"what": what}
        for waves in (1, 4, 8):
            for _ in range(2):  # the second launch is the one kept
                out.zero_()
                hip.launch(name, 64 * waves, [out.data_ptr(), sink.data_ptr()], stream)
                torch.cuda.synchronize()
            cyc = out[: BLOCKS * 16].view(BLOCKS, 16)[:, :waves].double()
            row = {"cycles": round(cyc.mean().item(), 1)}
            if nbytes:
                # bytes the workgroup's waves read / cycles of its slowest wave
                row["bytes_per_clk_per_cu"] = round(nbytes * waves / cyc.max(dim=1).values.mean().item(), 1)
            res[key][waves] = row
    src = torch.zeros(BLOCKS * 16 * 8 * 1024 // 4, dtype=torch.float32, device="cuda").normal_()
    for key, (name, what) in ISSUE.items():
        res[key] = {"what": what}
        for waves in (4, 8):
            for _ in range(3):
                out.zero_()
                hip.launch(name, 64 * waves, [src.data_ptr(), out.data_ptr(), sink.data_ptr()], stream)
                torch.cuda.synchronize()
            o = out.view(BLOCKS, 16, 2)[:, :waves].double()
            res[key][waves] = {"issue_cycles": round(o[..., 0].mean().item(), 1),
                               "to_data_cycles": round(o[..., 1].mean().item(), 1)}
    for _ in range(2):
        out.zero_()
        hip.launch("g950p_clock", 64, [out.data_ptr()], stream)
        torch.cuda.synchronize()
    c = out[: BLOCKS * 2].view(BLOCKS, 2).double()
    res["clock"] = {"memtime_mhz": round(100.0 * c[:, 0].mean().item() / c[:, 1].mean().item(), 1)}
    res["mfma_shape"] = mfma_shape_rates(torch, hip, stream)
    res["attention_phases"] = attention_phases(torch)
    return res


STAMP_WG = 1000  # G950_ATT_STAMP_WG of g950_att_stamps.hip


def attention_phases(torch, t_lo=8, t_hi=40) -> dict:
    """Where an iteration of the bf16 attention main loop goes: one launch of
    the stamped code object (lib/g950_att_stamps.hsaco) at the non-causal
    [4, 32 / 8 KV heads, 4096, 128] shape, after the product kernel warmed
    the clock; workgroup STAMP_WG writes its s_memtime stamps (loop top,
    after the barrier, after the DMA issue, after the first-half softmax,
    after the MFMA phase, after the lead waves' softmax) over its output.
    Mean shader cycles per iteration over tiles t_lo..t_hi-1, for the lead
    waves 0-3 (DMA, MFMA phase, softmax) and waves 4-7 (softmax, MFMA phase)."""
    import math
    import time

    from . import operators as ops
    from . import runtime as rt
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev)
    g.manual_seed(0)
    B, H, HK, S, D = 4, 32, 8, 4096, 128
    q = torch.randn((B, H, S, D), device=dev, generator=g).to(torch.bfloat16)
    k = torch.randn((B, HK, S, D), device=dev, generator=g).to(torch.bfloat16)
    v = torch.randn((B, HK, S, D), device=dev, generator=g).to(torch.bfloat16)
    o = torch.empty_like(q)
    lse = torch.empty((B, H, S), device=dev)
    args = (q, k, v, o, B, H, S, 1.0 / math.sqrt(D), *q.stride(), *k.stride(), *v.stride(), *o.stride())
    call = ops.attn_fwd_causal_kernel(*args, CAUSAL=False, lse_ptr=lse, prepare=True)
    t_end = time.perf_counter() + 0.5
    while time.perf_counter() < t_end:  # clock ramp on the product kernel
        call()
        torch.cuda.synchronize()
    devi = torch.cuda.current_device()
    prod = rt.module()
    stamped = rt.Module(str(STAMPS))
    try:
        rt._modules[devi] = stamped
        ops.attn_fwd_causal_kernel(*args, CAUSAL=False, lse_ptr=lse, prepare=True)()
        torch.cuda.synchronize()
    finally:
        rt._modules[devi] = prod
        stamped.close()
    # the workgroup -> (q-block, batch, head) map of the kernel: longest
    # q-blocks first, the G query heads of one KV head 8 ids apart
    nqb, per_qb, G = S // 256, B * H, H // HK
    qb = nqb - 1 - STAMP_WG // per_qb
    i = STAMP_WG % per_qb
    xcd, j = i & 7, i >> 3
    zk = xcd + 8 * (j // G)
    z, h = zk // HK, (zk % HK) * G + j % G
    raw = o[z, h, qb * 256:qb * 256 + 256].contiguous().view(torch.int64).cpu()
    st = raw.view(8, -1)[:, :64 * 6].view(8, 64, 6).double()
    out = {"shape": "non-causal bf16 [4, 32/8, 4096, 128]", "tiles": [t_lo, t_hi], "workgroup": STAMP_WG}
    for grp, ws, cols in (("lead", range(0, 4), (("barrier", 0, 1), ("dma_issue", 1, 2), ("mfma_phase", 3, 4),
                                                  ("softmax", 4, 5))),
                          ("other", range(4, 8), (("barrier", 0, 1), ("softmax", 2, 3), ("mfma_phase", 3, 4)))):
        sel = st[list(ws), t_lo:t_hi]
        row = {name: round((sel[..., b] - sel[..., a]).mean().item(), 1) for name, a, b in cols}
        row["period"] = round((st[list(ws), t_lo + 1:t_hi + 1, 0] - sel[..., 0]).mean().item(), 1)
        out[grp] = row
    return out


def mfma_shape_rates(torch, hip, stream, seconds=1.0) -> dict:
    """Sustained bf16 MFMA TFLOP/s of the 32x32x16 and 16x16x32 forms
    (g950p_mfma_rate32 / _rate16: 8 waves per CU, random operands rotating
    through eight registers), each timed with HIP events over about
    ``seconds`` of back-to-back launches so the power limit sets the clock;
    each shape is measured twice, interleaved."""
    import time
    words = torch.randint(0, 2 ** 31 - 1, (65536 * 4,), dtype=torch.int32, device="cuda")
    words = (words & 0x807F807F) | 0x3F003F00  # random signs and mantissas, exponents near 1
    sink = torch.empty(BLOCKS * 512, dtype=torch.float32, device="cuda")
    iters = 2000
    out = {}
    for name, key in (("g950p_mfma_rate32", "32x32x16"), ("g950p_mfma_rate16", "16x16x32")) * 2:
        args = [words.data_ptr(), sink.data_ptr(), ctypes.c_int(iters)]
        for _ in range(3):
            hip.launch(name, 512, args, stream)
        torch.cuda.synchronize()
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        t0 = time.perf_counter()
        e0.record()
        n = 0
        while time.perf_counter() - t0 < seconds:
            hip.launch(name, 512, args, stream)
            n += 1
            if n % 8 == 0:
                torch.cuda.synchronize()
        e1.record()
        e1.synchronize()
        flop = n * BLOCKS * 8 * iters * 32 * 32768  # per wave per iteration: 32 x 32768 = 64 x 16384
        out.setdefault(key, []).append(round(flop / (e0.elapsed_time(e1) * 1e-3) / 1e12, 1))
    return {"what": "bf16 MFMA, random operands, 8 waves/CU, ~1 s of back-to-back launches each",
            "tflops": out}
