"""Benchmark of the gfx950 hot path on one MI355X.

Headline workload: masked-tail bf16 row reductions
on x[8191, 3000] -- one step = one LayerNorm pass + one softmax pass over one
batch; value = algorithmic HBM bytes per step / step time (GB/s).  Inputs are
resident in HBM before the timed region; the timed region rotates 6 buffer
sets (~885 MB > the 256 MB Infinity Cache) so that successive steps cannot be
served from MALL.

The same line carries
  * roofline: the dominant kernel's achieved GB/s (algorithmic bytes per launch
    / its average launch time, HIP events on the launch stream) against the
    8 TB/s HBM peak;
  * cpu_baseline: the OpenMP fp32 CPU path (oracle/cpu_baseline.c, the a100c
    worker-pool restatement) on the same workload, on this host's cores, with
    the numpy float64 oracle (the reference ref() semantics) beside it;
  * suite: every other BASELINE config (fp32 RMSNorm/softmax GB/s, bf16 GEMM,
    causal GQA attention and int8 GEMM TFLOP/s) with its own roofline fraction
    and, for each BASELINE config, both CPU baselines on a bounded sample
    (rows of A, query heads, rows of x) sized to about a second each.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "GEMM/attn TFLOP/s + norm/softmax HBM GB/s vs roofline, 1×MI355X"
HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFS = 2516.6   # dense, 256 CU x 2.4 GHz x 4096 FLOP/clk
INT8_PEAK_TOPS = 5033.2  # dense, 8192 OP/clk/CU
FP32_PEAK_TFS = 157.3    # dense fp32 MFMA
ROTATE = 6   # rotating buffer sets: >= 512 MiB touched per cycle, so the 256 MB MALL cannot hold them


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def warm(torch, launch, seconds):
    """Launch repeatedly for about ``seconds`` of wall time: MI355X engine
    clocks ramp over the first few hundred milliseconds of sustained load
    (measured: 1.46 -> 1.86 GHz across four back-to-back 1 ms kernels), so a
    handful of warmup launches under-reports a kernel's steady rate."""
    import time
    t_end = time.perf_counter() + seconds
    i = 0
    while time.perf_counter() < t_end:
        for _ in range(4):
            launch(i)
            i += 1
        torch.cuda.synchronize()


def event_time(torch, launch, iters, warmup, warm_s=0.0):
    """Average ms per launch of ``launch(i)``: HIP events on the launch stream
    around a batch of back-to-back launches of prepared calls (whose host cost
    is well below the kernel time, so the queue never drains and the average
    is the kernel's own duration plus the inter-dispatch gap)."""
    if warm_s > 0:
        warm(torch, launch, warm_s)
    for i in range(warmup):
        launch(i)
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record()
    for i in range(iters):
        launch(i)
    end.record()
    end.synchronize()
    return start.elapsed_time(end) / iters


def headline(torch, ops, args):
    """Config 2: LayerNorm + softmax, bf16 [8191, 3000]."""
    from oracle import inputs
    rows, cols = 8191, 3000
    dev = "cuda:0"
    sets = []
    for s in range(ROTATE):
        c = inputs.config2(rows, cols, seed=inputs.SEEDS["c2"] + s)
        bf = lambda a: torch.from_numpy(a).to(dev).to(torch.bfloat16)  # noqa: E731
        sets.append({
            "x": bf(c["x"]), "g": bf(c["gamma"]), "b": bf(c["beta"]),
            "y": torch.empty((rows, cols), dtype=torch.bfloat16, device=dev),
            "s": torch.empty((rows, cols), dtype=torch.bfloat16, device=dev),
            "mean": torch.empty(rows, dtype=torch.float32, device=dev),
            "rstd": torch.empty(rows, dtype=torch.float32, device=dev),
        })
    eps = 1e-5
    ln_bytes = 2 * rows * cols * 2 + 2 * cols * 2 + 2 * rows * 4
    sm_bytes = 2 * rows * cols * 2

    ln_calls = [ops.layernorm_kernel(d["x"], d["y"], d["g"], d["b"], d["mean"], d["rstd"], cols, cols,
                                     eps, prepare=True) for d in sets]
    sm_calls = [ops.softmax_kernel(d["x"], d["s"], cols, prepare=True) for d in sets]

    def ln(i):
        ln_calls[i % ROTATE]()

    def sm(i):
        sm_calls[i % ROTATE]()

    def step(i):
        ln(i)
        sm(i)

    # per-kernel launch times: events around many back-to-back launches of one
    # kernel (its average launch duration), and the reference's per-launch median
    ln_t = timed(torch, ln, 200, 10, warm_s=0.3)
    ln_ms = ln_t["mean_ms"]
    ln_kernel = ln_calls[0].kernel
    sm_t = timed(torch, sm, 200, 10)
    sm_ms = sm_t["mean_ms"]
    sm_kernel = sm_calls[0].kernel

    # the timed steps: barrier-free single process, synchronize on both sides
    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record()
    for i in range(args.steps):
        step(i)
    end.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_step = start.elapsed_time(end) / args.steps
    value = (ln_bytes + sm_bytes) / (ms_step * 1e-3) / 1e9
    dom = ("layernorm", ln_kernel, ln_bytes, ln_ms) if ln_ms >= sm_ms else ("softmax", sm_kernel, sm_bytes, sm_ms)
    achieved = dom[2] / (dom[3] * 1e-3) / 1e9
    roof = {"bound": "hbm", "kernel": dom[1], "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
            "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic_for(dom[1]),
            "algorithmic_bytes": dom[2], "avg_launch_us": round(dom[3] * 1e3, 2)}
    per_kernel = {
        "layernorm": {"kernel": ln_kernel, "us": round(ln_ms * 1e3, 2),
                      "GB/s": round(ln_bytes / (ln_ms * 1e-3) / 1e9, 1), "bytes": ln_bytes,
                      "median_us": round(ln_t["median_ms"] * 1e3, 2), "n_samples": ln_t["n"]},
        "softmax": {"kernel": sm_kernel, "us": round(sm_ms * 1e3, 2),
                    "GB/s": round(sm_bytes / (sm_ms * 1e-3) / 1e9, 1), "bytes": sm_bytes,
                    "median_us": round(sm_t["median_ms"] * 1e3, 2), "n_samples": sm_t["n"]},
    }
    roof["median_us"] = per_kernel[dom[0]]["median_us"]
    roof["frac_median"] = round(dom[2] / (roof["median_us"] * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)
    del sets
    return value, ms_step, wall, roof, per_kernel, ln_bytes + sm_bytes


def cpu_baseline(seconds=10.0):
    """OpenMP fp32 CPU path on config 2 (full workload, repeated ~`seconds`)."""
    from oracle import build as obuild
    from oracle import inputs
    from oracle.reference import bf16_bits
    lib = obuild.load()
    rows, cols = 8191, 3000
    c = inputs.config2(rows, cols)
    x = bf16_bits(c["x"])
    g, b = bf16_bits(c["gamma"]), bf16_bits(c["beta"])
    y = np.empty_like(x)
    s = np.empty_like(x)
    mean = np.empty(rows, np.float32)
    rstd = np.empty(rows, np.float32)
    p = lambda a: a.ctypes.data  # noqa: E731
    reps = 0
    t0 = time.perf_counter()
    while True:
        lib.g950o_layernorm_bf16(p(x), p(g), p(b), p(y), p(mean), p(rstd), rows, cols, 1e-5)
        lib.g950o_softmax_bf16(p(x), p(s), rows, cols)
        reps += 1
        el = time.perf_counter() - t0
        if el >= seconds or reps >= 1000:
            break
    nbytes = (2 * rows * cols * 2 + 2 * cols * 2 + 2 * rows * 4) + 2 * rows * cols * 2
    from oracle import reference as ref

    def f64(nrows):
        ref.layernorm(c["x"][:nrows], c["gamma"], c["beta"], 1e-5)
        ref.softmax(c["x"][:nrows])
    n, t = sized_time(f64, 256, rows)
    per_row = nbytes / rows
    return {"value": round(nbytes * reps / el / 1e9, 2), "unit": "GB/s", "cores": int(lib.g950o_threads()),
            "kind": "port",
            "sample": f"full config-2 workload (LayerNorm + softmax, bf16 [8191,3000]) x {reps} passes, "
                      f"{el:.1f} s, oracle/cpu_baseline.c OpenMP fp32",
            "cpu": _cpu_model(),
            "numpy_f64": {"value": round(per_row * n / t / 1e9, 3), "unit": "GB/s",
                          "threads": _blas_threads() or "numpy (reductions single-threaded)",
                          "sample": f"{n} rows of the same workload, {t:.2f} s, oracle/reference.py float64"}}


CPU_TARGET_S = 1.0   # seconds of CPU work per timed baseline sample


def _blas_threads():
    keys = ("OMP_NUM_THREADS", "OPENBLAS_NUM_THREADS", "MKL_NUM_THREADS")
    return {k: os.environ[k] for k in keys if k in os.environ}


def sized_time(run, n0, n_max, target_s=CPU_TARGET_S):
    """Time ``run(n)`` on a bounded sample: a warm-up call with ``n0`` units
    (first touch, thread-pool start), a probe call with ``n0`` units, then
    calls with ``n`` scaled so one takes about ``target_s`` (at most
    ``n_max``, the whole config), repeated until about ``target_s`` has
    passed.  Returns (units timed, seconds)."""
    run(n0)
    t0 = time.perf_counter()
    run(n0)
    probe = max(time.perf_counter() - t0, 1e-6)
    n = int(min(n_max, max(n0, n0 * target_s / probe)))
    done, t0 = 0, time.perf_counter()
    while True:
        run(n)
        done += n
        el = time.perf_counter() - t0
        if el >= target_s or done >= 100 * n:
            return done, el


def cpu_legs(port_run, f64_run, work_per_unit, unit, scale, what, n0, n_max):
    """Both CPU baselines of one config on a bounded sample of ``what`` units:
    the OpenMP fp32 port (oracle/cpu_baseline.c, the a100c worker-pool
    partition) and the numpy float64 oracle (oracle/reference.py restating the
    reference ``ref()``).  ``work_per_unit`` is bytes or FLOP per unit; the
    value is work / time / ``scale`` in ``unit``."""
    from oracle import build as obuild
    lib = obuild.load()
    n, t = sized_time(port_run, n0, n_max)
    out = {"value": round(work_per_unit * n / t / scale, 3), "unit": unit, "cores": int(lib.g950o_threads()),
           "kind": "port", "sample": f"{n} {what}, {t:.2f} s, oracle/cpu_baseline.c OpenMP fp32",
           "cpu": _cpu_model()}
    if f64_run is not None:
        n, t = sized_time(f64_run, n0, n_max)
        out["numpy_f64"] = {"value": round(work_per_unit * n / t / scale, 3), "unit": unit,
                            "threads": _blas_threads() or f"numpy BLAS default ({os.cpu_count()} CPUs visible)",
                            "sample": f"{n} {what}, {t:.2f} s, oracle/reference.py float64"}
    return out


def _cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def event_samples(torch, launch, min_samples=50, min_time_s=0.2, max_samples=1000, floor=10):
    """The reference benchmark's statistic (ops/harness/benchmark/run.py:141-186,
    benchmark/README.md:64-67): one HIP-event pair around each launch on the
    launch stream, each launch waited for before the next (the harness
    Device's launch returns once the kernel has finished), sampled until
    EITHER >= 50 samples or >= 0.2 s of kernel time, never fewer than 10, at
    most 1000.  Returns the samples in ms; the reference reports their median."""
    stream = torch.cuda.current_stream()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    times = []
    i = 0
    while True:
        start.record(stream)
        launch(i)
        end.record(stream)
        end.synchronize()
        times.append(start.elapsed_time(end))
        i += 1
        n = len(times)
        if n >= max(min_samples, floor) or (n >= floor and sum(times) >= min_time_s * 1e3) or n >= max_samples:
            return times


def timed(torch, launch, iters, warmup, warm_s=0.0):
    """Both statistics of one prepared launch: the batched mean (events around
    ``iters`` back-to-back launches after a ``warm_s`` warm-up: the kernel's
    average launch duration plus the inter-dispatch gap) and the reference's
    per-launch median (``event_samples``)."""
    mean_ms = event_time(torch, launch, iters, warmup, warm_s=warm_s)
    s = sorted(event_samples(torch, launch))
    pick = lambda f: s[min(len(s) - 1, round(f * (len(s) - 1)))]  # noqa: E731
    return {"mean_ms": mean_ms, "median_ms": float(np.median(s)), "p10_ms": pick(0.1), "p90_ms": pick(0.9),
            "n": len(s)}


def make_row(name, kernel, work, unit, scale, peak, bound, t):
    """One suite row: value and roofline fraction from the batched mean (the
    average launch duration, as rocprofv3 sees the kernel back to back), the
    reference statistic (median of per-launch samples) beside it."""
    v = work / (t["mean_ms"] * 1e-3) / scale
    vm = work / (t["median_ms"] * 1e-3) / scale
    return {"config": name, "kernel": kernel, "us": round(t["mean_ms"] * 1e3, 2), "value": round(v, 1),
            "unit": unit, "bound": bound, "frac": round(v / peak, 4),
            "median_us": round(t["median_ms"] * 1e3, 2), "n_samples": t["n"],
            "p10_us": round(t["p10_ms"] * 1e3, 2), "p90_us": round(t["p90_ms"] * 1e3, 2),
            "value_median": round(vm, 1), "frac_median": round(vm / peak, 4)}


# suite sections (bench.py --only KEY[,KEY...] runs just these, without the
# headline or the CPU legs: one rocprofv3 trace per config)
SECTIONS = ("c1", "lse", "dequantize", "c3a", "c3b", "c3a_rowb", "gemm_f32", "c4", "attn_f32", "odd", "split",
            "w8a16", "w8a16_16", "w8a16_1", "w8a16_rowb", "varlen", "varlen_paged", "c5")


def suite(torch, ops, cpu=True, only=None):
    """Every other BASELINE config, timed per kernel with HIP events; with
    ``cpu`` each BASELINE config row also carries its CPU baselines (both
    legs) on a bounded sample of the same inputs.  ``only``: the section keys
    to run (SECTIONS), all when None."""
    from oracle import build as obuild
    from oracle import inputs
    from oracle import reference as ref
    from oracle.reference import bf16_bits
    lib = obuild.load() if cpu else None
    P = lambda a: a.ctypes.data  # noqa: E731
    dev = "cuda:0"
    out = []

    def want(key):
        return only is None or key in only

    # C1: fp32 RMSNorm + softmax [4096, 4096], 6 rotating sets (768 MiB)
    if want("c1"):
        sets = []
        for s in range(ROTATE):
            c = inputs.config1(seed=inputs.SEEDS["c1"] + s)
            sets.append({"x": torch.from_numpy(c["x"]).to(dev), "w": torch.from_numpy(c["w"]).to(dev),
                         "y": torch.empty((4096, 4096), device=dev), "r": torch.empty(4096, device=dev)})
        rb = 2 * 4096 * 4096 * 4 + 2 * 4096 * 4
        sb = 2 * 4096 * 4096 * 4
        rms_calls = [ops.rms_layernorm_forward_kernel(d["y"], 4096, d["x"], 4096, d["w"], 1, d["r"], 1,
                                                      4096, 1e-6, prepare=True) for d in sets]
        smx_calls = [ops.softmax_kernel(d["x"], d["y"], 4096, prepare=True) for d in sets]
        for name, calls, nbytes in (("C1a rmsnorm fp32 [4096,4096]", rms_calls, rb),
                                    ("C1b softmax fp32 [4096,4096]", smx_calls, sb)):
            t = timed(torch, lambda i: calls[i % ROTATE](), 200, 10, warm_s=0.3)
            out.append(make_row(name, calls[0].kernel, nbytes, "GB/s", 1e9, HBM_PEAK_GBS, "hbm", t))
        del sets, rms_calls, smx_calls
        torch.cuda.empty_cache()
        if cpu:
            c1 = inputs.config1()
            x1, w1 = c1["x"], c1["w"]
            y1, r1 = np.empty_like(x1), np.empty(4096, np.float32)
            out[-2]["cpu_baseline"] = cpu_legs(
                lambda n: lib.g950o_rmsnorm_f32(P(x1), P(w1), P(y1), P(r1), n, 4096, 1e-6),
                lambda n: ref.rms_layernorm(x1[:n], w1, 1e-6), rb / 4096, "GB/s", 1e9, "rows of [4096,4096]", 256,
                4096)
            out[-1]["cpu_baseline"] = cpu_legs(
                lambda n: lib.g950o_softmax_f32(P(x1), P(y1), n, 4096),
                lambda n: ref.softmax(x1[:n]), sb / 4096, "GB/s", 1e9, "rows of [4096,4096]", 256, 4096)
            del c1, x1, y1

    # next-row operators at their BASELINE-sized shapes, 6 rotating sets each:
    # row logsumexp bf16 [8191, 3000] -> fp32, int8 weight dequant [8192, 8192] -> bf16
    g = torch.Generator(device=dev)
    g.manual_seed(7)
    if want("lse"):
        lse_sets = [(torch.randn((8191, 3000), device=dev, generator=g).mul_(3.0).to(torch.bfloat16),
                     torch.empty(8191, device=dev)) for _ in range(ROTATE)]
        calls = [ops.logsumexp_kernel(x, y, 3000, prepare=True) for x, y in lse_sets]
        t = timed(torch, lambda i: calls[i % ROTATE](), 200, 10, warm_s=0.3)
        out.append(make_row("F logsumexp bf16 [8191,3000] -> fp32", calls[0].kernel, 8191 * 3000 * 2 + 8191 * 4,
                            "GB/s", 1e9, HBM_PEAK_GBS, "hbm", t))
        del lse_sets, calls
    if want("dequantize"):
        dq_sets = [(torch.randint(-127, 127, (8192, 8192), device=dev, generator=g, dtype=torch.int8),
                    torch.rand(8192, device=dev, generator=g).to(torch.bfloat16),
                    torch.empty((8192, 8192), dtype=torch.bfloat16, device=dev)) for _ in range(ROTATE)]
        calls = [ops.dequantize_kernel(b, sc, y, 8192, 8192, 8192, 1, 8192, 1, prepare=True) for b, sc, y in dq_sets]
        t = timed(torch, lambda i: calls[i % ROTATE](), 50, 10, warm_s=0.3)
        out.append(make_row("F dequantize int8 [8192,8192] -> bf16", calls[0].kernel, 8192 * 8192 * 3 + 8192 * 2,
                            "GB/s", 1e9, HBM_PEAK_GBS, "hbm", t))
        del dq_sets, calls
    torch.cuda.empty_cache()

    # C3: bf16 GEMM, A row-major, B column-major
    for key, (m, n, k) in (("c3a", (8192, 8192, 8192)), ("c3b", (4097, 11008, 4096))):
        if not want(key):
            continue
        c = inputs.config3(m, n, k)
        a = torch.from_numpy(c["a"]).to(dev).to(torch.bfloat16)
        bt = torch.from_numpy(c["bt"]).to(dev).to(torch.bfloat16)
        y = torch.empty((m, n), dtype=torch.bfloat16, device=dev)
        call = ops.matmul_kernel(a, bt.t(), y, m, n, k, prepare=True)
        t = timed(torch, lambda i: call(), 20, 3, warm_s=0.5)
        out.append(make_row(f"C3 gemm bf16 {m}x{n}x{k}", call.kernel, 2.0 * m * n * k, "TFLOP/s", 1e12,
                            BF16_PEAK_TFS, "mfma", t))
        del a, bt, y
        torch.cuda.empty_cache()
        if cpu:
            # rows of A against all of B (inputs resident: B widened once
            # outside the timed sample, as the GPU's B is resident in HBM)
            ab, btb = bf16_bits(c["a"]), bf16_bits(c["bt"])
            b32 = np.empty(btb.shape, np.float32)
            lib.g950o_widen_bf16(P(btb), P(b32), btb.size)
            cbuf = np.empty((m, n), np.uint16)
            b64 = c["bt"].T.astype(np.float64)
            a64 = c["a"].astype(np.float64)
            out[-1]["cpu_baseline"] = cpu_legs(
                lambda r: lib.g950o_gemm_bf16_wide(P(ab), P(b32), P(cbuf), 0, r, n, k),
                lambda r: a64[:r] @ b64, 2.0 * n * k, "TFLOP/s", 1e12, f"rows of A ({m}x{n}x{k})", 8, m)
            del ab, btb, b32, cbuf, b64, a64
        del c

    # the reference matmul's own layout: row-major B [K, N] (ops/suite/perf/matmul.py:33),
    # read as it lies by the MFMA kernel (transposing LDS reads)
    if want("c3a_rowb"):
        c = inputs.config3(8192, 8192, 8192)
        a = torch.from_numpy(c["a"]).to(dev).to(torch.bfloat16)
        b = torch.from_numpy(np.ascontiguousarray(c["bt"].T)).to(dev).to(torch.bfloat16)
        del c
        y = torch.empty((8192, 8192), dtype=torch.bfloat16, device=dev)
        call = ops.matmul_kernel(a, b, y, 8192, 8192, 8192, prepare=True)
        t = timed(torch, lambda i: call(), 20, 3, warm_s=0.5)
        out.append(make_row("F gemm bf16 8192^3, row-major B (reference layout)", call.kernel, 2.0 * 8192 ** 3,
                            "TFLOP/s", 1e12, BF16_PEAK_TFS, "mfma", t))
        del a, b, y
        torch.cuda.empty_cache()

    # fp32 operands (the matmul corpus's base dtype) on the fp32 MFMA kernel
    if want("gemm_f32"):
        g32 = torch.Generator(device=dev)
        g32.manual_seed(5)
        a = torch.randn((4096, 4096), device=dev, generator=g32)
        b = torch.randn((4096, 4096), device=dev, generator=g32)
        y = torch.empty((4096, 4096), device=dev)
        call = ops.matmul_kernel(a, b, y, 4096, 4096, 4096, prepare=True)
        t = timed(torch, lambda i: call(), 10, 2, warm_s=0.3)
        out.append(make_row("F gemm fp32 4096^3, row-major B", "g950_transpose_b32 + " + call.kernel,
                            2.0 * 4096 ** 3, "TFLOP/s", 1e12, FP32_PEAK_TFS, "mfma", t))
        del a, b, y
        torch.cuda.empty_cache()

    # C4: causal GQA attention bf16 (4, 32/8, 4096, 128) with LSE
    if want("c4"):
        c = inputs.config4()
        bf = lambda a: torch.from_numpy(a).to(dev).to(torch.bfloat16)  # noqa: E731
        q, k, v = bf(c["q"]), bf(c["k"]), bf(c["v"])
        o = torch.empty_like(q)
        lse = torch.empty((4, 32, 4096), dtype=torch.float32, device=dev)
        call = ops.attn_fwd_causal_kernel(q, k, v, o, 4, 32, 4096, 1 / math.sqrt(128), *q.stride(), *k.stride(),
                                          *v.stride(), *o.stride(), CAUSAL=True, lse_ptr=lse, prepare=True)
        t = timed(torch, lambda i: call(), 10, 2, warm_s=0.5)
        out.append(make_row("C4 causal GQA attention bf16 (4,32/8,4096,128)", call.kernel,
                            4.0 * 4 * 32 * 128 * 4096 * 4096 / 2, "TFLOP/s", 1e12, BF16_PEAK_TFS, "mfma", t))
        del q, k, v, o, lse
        torch.cuda.empty_cache()
        if cpu:
            # whole (batch 0, head) slices: 4096 causal query rows each
            qb, kb, vb = (bf16_bits(c[n][0]) for n in ("q", "k", "v"))
            ob = np.empty((32, 4096, 128), np.uint16)
            lb = np.empty((32, 4096), np.float32)
            head_flops = 4.0 * 128 * 4096 * 4096 / 2
            out[-1]["cpu_baseline"] = cpu_legs(
                lambda hn: lib.g950o_attention_bf16(P(qb), P(kb), P(vb), P(ob), P(lb), 32, 8, 4096, 128, 0, hn, 0,
                                                    4096, 1 / math.sqrt(128), 1),
                lambda hn: ref.attention(c["q"][:1, :hn], c["k"][:1, :(hn + 3) // 4], c["v"][:1, :(hn + 3) // 4],
                                         1 / math.sqrt(128), causal=True, group=4),
                head_flops, "TFLOP/s", 1e12, "(batch 0, query head) slices of 4096 causal rows", 1, 32)
            del qb, kb, vb, ob, lb
        del c

    # the same causal GQA attention in fp32 (the fp32 MFMA kernel)
    if want("attn_f32"):
        c = inputs.config4()
        q, k, v = (torch.from_numpy(c[n]).to(dev) for n in ("q", "k", "v"))
        del c
        o = torch.empty_like(q)
        lse = torch.empty((4, 32, 4096), dtype=torch.float32, device=dev)
        call = ops.attn_fwd_causal_kernel(q, k, v, o, 4, 32, 4096, 1 / math.sqrt(128), *q.stride(), *k.stride(),
                                          *v.stride(), *o.stride(), CAUSAL=True, lse_ptr=lse, prepare=True)
        t = timed(torch, lambda i: call(), 3, 1, warm_s=0.3)
        out.append(make_row("F causal GQA attention fp32 (4,32/8,4096,128)", call.kernel,
                            4.0 * 4 * 32 * 128 * 4096 * 4096 / 2, "TFLOP/s", 1e12, FP32_PEAK_TFS, "mfma", t))
        del q, k, v, o, lse
        torch.cuda.empty_cache()

    # rows whose length is not a whole number of 16-byte vectors: bf16 [8191, 3001]
    # (C2's distribution), LayerNorm and softmax, 6 rotating sets
    if want("odd"):
        odd = []
        for sidx in range(ROTATE):
            c = inputs.config2(8191, 3001, seed=inputs.SEEDS["c2"] + 10 + sidx)
            bf = lambda a: torch.from_numpy(a).to(dev).to(torch.bfloat16)  # noqa: E731
            odd.append((bf(c["x"]), bf(c["gamma"]), bf(c["beta"]),
                        torch.empty((8191, 3001), dtype=torch.bfloat16, device=dev),
                        torch.empty(8191, device=dev), torch.empty(8191, device=dev)))
        lno = [ops.layernorm_kernel(x, y, g_, b_, mm, rr, 3001, 3001, 1e-5, prepare=True)
               for x, g_, b_, y, mm, rr in odd]
        smo = [ops.softmax_kernel(x, y, 3001, prepare=True) for x, g_, b_, y, mm, rr in odd]
        for name, calls, nbytes in (("F layernorm bf16 [8191,3001] (odd rows)", lno,
                                     2 * 8191 * 3001 * 2 + 2 * 3001 * 2 + 2 * 8191 * 4),
                                    ("F softmax bf16 [8191,3001] (odd rows)", smo, 2 * 8191 * 3001 * 2)):
            t = timed(torch, lambda i: calls[i % ROTATE](), 100, 10, warm_s=0.3)
            out.append(make_row(name, calls[0].kernel, nbytes, "GB/s", 1e9, HBM_PEAK_GBS, "hbm", t))
        del odd, lno, smo
        torch.cuda.empty_cache()

    # few long rows (split-row two-phase path): softmax bf16 [4, 2^22]
    if want("split"):
        xs = [torch.randn((4, 1 << 22), device=dev, generator=g).to(torch.bfloat16) for _ in range(ROTATE)]
        ys = [torch.empty_like(x) for x in xs]
        calls = [ops.softmax_kernel(x, y, 1 << 22, prepare=True) for x, y in zip(xs, ys)]
        t = timed(torch, lambda i: calls[i % ROTATE](), 100, 10, warm_s=0.3)
        out.append(make_row("F split-row softmax bf16 [4,4194304]", calls[0].kernel, 2 * 4 * (1 << 22) * 2, "GB/s",
                            1e9, HBM_PEAK_GBS, "hbm", t))
        del xs, ys, calls

    # dequantize_matmul fused into the GEMM (W8A16): 8192^3 and two decode
    # shapes (16 rows and one row: the B-streaming kernels), bf16 activations,
    # int8 K-contiguous weights; and 8192^3 with the reference's own row-major
    # int8 weights [K, N] (dequantize_matmul.py:62-65)
    for key, (m_, n_, k_), rowq in (("w8a16", (8192, 8192, 8192), False), ("w8a16_16", (16, 8192, 8192), False),
                                    ("w8a16_1", (1, 8192, 8192), False), ("w8a16_rowb", (8192, 8192, 8192), True)):
        if not want(key):
            continue
        # decode shapes are HBM-bound: six rotating input sets (384 MiB of
        # weights), so the 64 MiB weight matrix cannot stay in the MALL
        nsets = 1 if m_ > 1000 else ROTATE
        calls = []
        for _ in range(nsets):
            a_ = torch.randn((m_, k_), device=dev, generator=g).to(torch.bfloat16)
            bt_ = torch.randint(-127, 127, (n_, k_), device=dev, generator=g, dtype=torch.int8)
            s_ = torch.rand(n_, device=dev, generator=g).to(torch.bfloat16)
            y_ = torch.empty((m_, n_), device=dev, dtype=torch.bfloat16)
            b_ = bt_.t().contiguous() if rowq else bt_.t()
            calls.append(ops.dequant_matmul_kernel(a_, b_, s_, y_, m_, n_, k_, prepare=True))
        call = calls[0]
        t = timed(torch, lambda i: calls[i % nsets](), 10 if m_ > 1000 else 50, 3, warm_s=0.3)
        if m_ > 1000:
            # large M: one exact int8 -> bf16 copy of B, then the bf16 GEMM (both timed)
            kern = call.kernel if "w8a16" in call.kernel else "g950_widen_i8_bf16 + " + call.kernel
            label = ", row-major int8 weights (reference layout)" if rowq else ""
            out.append(make_row(f"F dequant_matmul W8A16 bf16 {m_}x{n_}x{k_}{label}", kern, 2.0 * m_ * n_ * k_,
                                "TFLOP/s", 1e12, BF16_PEAK_TFS, "mfma", t))
        else:
            out.append(make_row(f"F dequant_matmul W8A16 bf16 {m_}x{n_}x{k_} (decode)", call.kernel,
                                n_ * k_ + m_ * k_ * 2 + m_ * n_ * 2, "GB/s", 1e9, HBM_PEAK_GBS, "hbm", t))
        del a_, bt_, b_, s_, y_, calls, call
    torch.cuda.empty_cache()

    # varlen attention (flash_varlen_fwd_kernel): 8 sequences of 4096 - 256 i
    # tokens (q = k lengths, causal), 32 query / 8 KV heads, d 128, bf16;
    # contiguous and paged (64-token pages, shuffled) K/V
    if want("varlen") or want("varlen_paged"):
        out.extend(varlen_rows(torch, ops, contiguous=want("varlen"), paged=want("varlen_paged")))
        torch.cuda.empty_cache()

    # C5: int8 GEMM 4096x8192x8192 + dequant
    if want("c5"):
        c = inputs.config5()
        a = torch.from_numpy(c["a"]).to(dev)
        bt = torch.from_numpy(c["bt"]).to(dev)
        sa = torch.from_numpy(c["sa"]).to(dev)
        sbv = torch.from_numpy(c["sb"]).to(dev)
        y = torch.empty((4096, 8192), dtype=torch.bfloat16, device=dev)
        call = ops.matmul_i8_dequant_kernel(a, bt.t(), sa, sbv, y, 4096, 8192, 8192, prepare=True)
        t = timed(torch, lambda i: call(), 20, 3, warm_s=0.5)
        out.append(make_row("C5 int8 gemm 4096x8192x8192 + dequant", call.kernel, 2.0 * 4096 * 8192 * 8192, "TOP/s",
                            1e12, INT8_PEAK_TOPS, "mfma", t))
        del a, bt, sa, sbv, y
        torch.cuda.empty_cache()
        if cpu:
            yc = np.empty((4096, 8192), np.uint16)
            b64 = c["bt"].T.astype(np.float64)
            a64 = c["a"].astype(np.float64)
            out[-1]["cpu_baseline"] = cpu_legs(
                lambda r: lib.g950o_gemm_i8(P(c["a"]), P(c["bt"]), P(c["sa"]), P(c["sb"]), None, P(yc), 0, r, 8192,
                                            8192),
                lambda r: ref.dequant(np.rint(a64[:r] @ b64), c["sa"][:r], c["sb"]),
                2.0 * 8192 * 8192, "TOP/s", 1e12, "rows of A (4096x8192x8192, int32 exact + dequant)", 8, 4096)
            del yc, b64, a64
        del c
    return out


def varlen_rows(torch, ops, contiguous=True, paged=True):
    """flash_varlen_fwd_kernel at the C4 scale: 8 causal sequences of
    4096 - 256 i tokens, 32 query / 8 KV heads, d 128, bf16; contiguous and
    paged (64-token pages, shuffled) K/V."""
    dev = "cuda:0"
    lens = [4096 - 256 * i for i in range(8)]
    tq = sum(lens)
    cu = torch.tensor([0] + list(np.cumsum(lens)), dtype=torch.int32, device=dev)
    g = torch.Generator(device=dev)
    g.manual_seed(11)
    qv = torch.randn((tq, 32, 128), device=dev, generator=g).mul_(0.5).to(torch.bfloat16)
    kv = torch.randn((tq, 8, 128), device=dev, generator=g).mul_(0.5).to(torch.bfloat16)
    vv = torch.randn((tq, 8, 128), device=dev, generator=g).to(torch.bfloat16)
    ov = torch.empty_like(qv)
    lsev = torch.empty((32, tq), device=dev)
    pages = [(n + 63) // 64 for n in lens]
    perm = torch.randperm(sum(pages), device=dev, generator=g)
    table = torch.zeros((8, max(pages)), dtype=torch.int32, device=dev)
    kp = torch.empty((sum(pages) * 64, 8, 128), dtype=torch.bfloat16, device=dev)
    vp = torch.empty_like(kp)
    nxt = 0
    for b, n in enumerate(lens):
        for pg in range(pages[b]):
            ph = int(perm[nxt])
            nxt += 1
            table[b, pg] = ph
            lo, hi = pg * 64, min(n, pg * 64 + 64)
            kp[ph * 64:ph * 64 + hi - lo] = kv[int(cu[b]) + lo:int(cu[b]) + hi]
            vp[ph * 64:ph * 64 + hi - lo] = vv[int(cu[b]) + lo:int(cu[b]) + hi]
    used = torch.tensor(lens, dtype=torch.int32, device=dev)
    zero1 = torch.zeros(1, device=dev)
    philox = torch.zeros(2, dtype=torch.int64, device=dev)
    scal = dict(q_row_stride=32 * 128, k_row_stride=8 * 128, v_row_stride=8 * 128, q_head_stride=128,
                k_head_stride=128, v_head_stride=128, o_row_stride=32 * 128, o_head_stride=128, q_batch_stride=0,
                k_batch_stride=0, v_batch_stride=0, o_batch_stride=0, is_cu_seqlens_q=True,
                is_cu_seqlens_k=True, is_seqused_k=False, b=8, bk=8, h=32, hk=8, h_hk_ratio=4, seqlen_q=4096,
                seqlen_k=4096, seqlen_q_rounded=4096, seqlen_k_rounded=4096, d=128, is_softcap=False,
                softcap=0.0, scale_softmax=1 / math.sqrt(128), scale_softmax_log2=math.log2(math.e) / math.sqrt(128),
                is_dropout=False, p_dropout=1.0, rp_dropout=1.0, p_dropout_in_uint8_t=255, return_softmax=False,
                is_causal=True, is_local=False, window_size_left=-1, window_size_right=0,
                seqlenq_ngroups_swapped=False, is_paged=False, is_alibi=False, alibi_slopes_batch_stride=0,
                total_q=tq, page_table_batch_stride=0, block_size=1, k_page_stride=0)
    ptrs = dict(q_ptr=qv, k_ptr=kv, v_ptr=vv, o_ptr=ov, p_ptr=zero1, softmax_lse_ptr=lsev, cu_seqlens_q_ptr=cu,
                cu_seqlens_k_ptr=cu, seqused_k_ptr=used, philox_args=philox, alibi_slopes_ptr=zero1,
                page_table_ptr=table)
    flops = sum(4.0 * 32 * 128 * n * (n + 1) / 2 for n in lens)
    rows = []
    for on, name, extra in ((contiguous, "F varlen causal GQA bf16 (8 seqs 4096..2304, 32/8, d128)", {}),
                            (paged, "F varlen paged(64) causal GQA bf16 (same)",
                             dict(k_ptr=kp, v_ptr=vp, is_paged=True, is_cu_seqlens_k=False, is_seqused_k=True,
                                  page_table_batch_stride=max(pages), block_size=64, k_page_stride=64 * 8 * 128))):
        if not on:
            continue
        call = ops.flash_varlen_fwd_kernel(**{**ptrs, **scal, **extra}, prepare=True)
        t = timed(torch, lambda i: call(), 10, 2, warm_s=0.5)
        rows.append(make_row(name, call.kernel, flops, "TFLOP/s", 1e12, BF16_PEAK_TFS, "mfma", t))
    return rows


def pmc_probe(torch, ops):
    """Counter-collection workload (run under rocprofv3 --pmc): the streaming
    copy kernel on exactly the bytes of one x (the calibration kernel: same
    nontemporal 16-byte loads/stores as the row kernels), then 8 launches of
    each HBM-bound kernel on 6 rotating buffer sets, as in the timed region:
    C2, C1, int8 dequantisation and the next-row kernels."""
    from oracle import inputs
    rows, cols = 8191, 3000
    dev = "cuda:0"
    srcs = [torch.empty(rows * cols, dtype=torch.bfloat16, device=dev).normal_() for _ in range(ROTATE)]
    dsts = [torch.empty_like(x) for x in srcs]
    copies = [ops.stream_copy(x, y, prepare=True) for x, y in zip(srcs, dsts)]
    torch.cuda.synchronize()
    for i in range(8):
        copies[i % ROTATE]()
    torch.cuda.synchronize()
    src = srcs[0]
    del dsts
    sets = []
    for s in range(ROTATE):
        c = inputs.config2(rows, cols, seed=inputs.SEEDS["c2"] + s)
        bf = lambda a: torch.from_numpy(a).to(dev).to(torch.bfloat16)  # noqa: E731
        sets.append((bf(c["x"]), bf(c["gamma"]), bf(c["beta"]), torch.empty((rows, cols), dtype=torch.bfloat16, device=dev),
                     torch.empty(rows, device=dev), torch.empty(rows, device=dev)))
    ln = [ops.layernorm_kernel(x, y, g, b, m, r, cols, cols, 1e-5, prepare=True) for x, g, b, y, m, r in sets]
    sm = [ops.softmax_kernel(x, y, cols, prepare=True) for x, g, b, y, m, r in sets]
    lr = [ops.layer_norm_forward_row(y.view(-1), cols, x, cols, g, b, m, 1, r, 1, rows, cols, 1e-5, prepare=True)
          for x, g, b, y, m, r in sets]
    torch.cuda.synchronize()
    for calls in (ln, sm, lr):
        for i in range(8):
            calls[i % ROTATE]()
        torch.cuda.synchronize()
    del sets, ln, sm, lr
    # C1 fp32 [4096, 4096] RMSNorm and softmax, 6 rotating sets
    c1 = [(torch.randn((4096, 4096), device=dev), torch.rand(4096, device=dev) + 0.5,
           torch.empty((4096, 4096), device=dev), torch.empty(4096, device=dev)) for _ in range(ROTATE)]
    rms = [ops.rms_layernorm_forward_kernel(y, 4096, x, 4096, w, 1, r, 1, 4096, 1e-6, prepare=True)
           for x, w, y, r in c1]
    smf = [ops.softmax_kernel(x, y, 4096, prepare=True) for x, w, y, r in c1]
    for calls in (rms, smf):
        for i in range(8):
            calls[i % ROTATE]()
        torch.cuda.synchronize()
    del c1, rms, smf
    # int8 weight dequantisation [8192, 8192] -> bf16, 6 rotating sets
    dq = [(torch.randint(-127, 127, (8192, 8192), device=dev, dtype=torch.int8),
           torch.rand(8192, device=dev).to(torch.bfloat16),
           torch.empty((8192, 8192), dtype=torch.bfloat16, device=dev)) for _ in range(ROTATE)]
    dqc = [ops.dequantize_kernel(b, sc, y, 8192, 8192, 8192, 1, 8192, 1, prepare=True) for b, sc, y in dq]
    for i in range(8):
        dqc[i % ROTATE]()
    torch.cuda.synchronize()
    del dq, dqc
    # next-row kernels: row logsumexp bf16 [8191, 3000] -> fp32; odd rows
    # bf16 [8191, 3001] LayerNorm and softmax; split rows bf16 [4, 2^22]
    # softmax; W8A16 decode 16 x 8192 x 8192 and 1 x 8192 x 8192
    gen = torch.Generator(device=dev)
    gen.manual_seed(7)
    lse = [(torch.randn((8191, 3000), device=dev, generator=gen).mul_(3.0).to(torch.bfloat16),
            torch.empty(8191, device=dev)) for _ in range(ROTATE)]
    lsec = [ops.logsumexp_kernel(x, y, 3000, prepare=True) for x, y in lse]
    odd = [(torch.randn((8191, 3001), device=dev, generator=gen).mul_(3.0).to(torch.bfloat16),
            torch.rand(3001, device=dev, generator=gen).add_(0.5).to(torch.bfloat16),
            torch.randn(3001, device=dev, generator=gen).mul_(0.1).to(torch.bfloat16),
            torch.empty((8191, 3001), dtype=torch.bfloat16, device=dev),
            torch.empty(8191, device=dev), torch.empty(8191, device=dev)) for _ in range(ROTATE)]
    lno = [ops.layernorm_kernel(x, y, g_, b_, m_, r_, 3001, 3001, 1e-5, prepare=True) for x, g_, b_, y, m_, r_ in odd]
    smo = [ops.softmax_kernel(x, y, 3001, prepare=True) for x, g_, b_, y, m_, r_ in odd]
    for calls in (lsec, lno, smo):
        for i in range(8):
            calls[i % ROTATE]()
        torch.cuda.synchronize()
    del lse, lsec, odd, lno, smo
    xs = [torch.randn((4, 1 << 22), device=dev, generator=gen).to(torch.bfloat16) for _ in range(ROTATE)]
    spc = [ops.softmax_kernel(x, torch.empty_like(x), 1 << 22, prepare=True) for x in xs]
    for i in range(8):
        spc[i % ROTATE]()
    torch.cuda.synchronize()
    del xs, spc
    for m_ in (16, 1):
        dec = [(torch.randn((m_, 8192), device=dev, generator=gen).to(torch.bfloat16),
                torch.randint(-127, 127, (8192, 8192), device=dev, generator=gen, dtype=torch.int8),
                torch.rand(8192, device=dev, generator=gen).to(torch.bfloat16),
                torch.empty((m_, 8192), device=dev, dtype=torch.bfloat16)) for _ in range(ROTATE)]
        decc = [ops.dequant_matmul_kernel(a_, b_.t(), s_, y_, m_, 8192, 8192, prepare=True) for a_, b_, s_, y_ in dec]
        for i in range(8):
            decc[i % ROTATE]()
        torch.cuda.synchronize()
        del dec, decc
    log(f"pmc probe: copy {src.numel() * 2} B read + write; C2 layernorm/softmax/layer_norm_forward_row, "
        "C1 rmsnorm/softmax fp32, dequantize int8->bf16 8192^2, logsumexp bf16 [8191,3000], odd-row "
        "layernorm/softmax [8191,3001], split-row softmax [4,2^22], W8A16 decode 16/1 x 8192 x 8192: x8 each")


def load_probe(torch, ops, which, seconds):
    """Power/clock workload: one config's kernel back to back for `seconds`
    (C4 causal attention, the C3 GEMM at 8192^3, or C2 softmax on six
    rotating sets), so `amd-smi metric --power` / `rocm-smi --showclocks`
    can sample the chip under it from another process.  Prints the launch
    count and the mean time per launch (host waits between ~8 ms batches
    included)."""
    from oracle import inputs
    dev = "cuda:0"
    if which == "attn":
        c = inputs.config4()
        bf = lambda x: torch.from_numpy(x).to(dev).to(torch.bfloat16)  # noqa: E731
        q, k, v = bf(c["q"]), bf(c["k"]), bf(c["v"])
        del c
        o = torch.empty_like(q)
        lse = torch.empty((4, 32, 4096), dtype=torch.float32, device=dev)
        call = ops.attn_fwd_causal_kernel(q, k, v, o, 4, 32, 4096, 1 / math.sqrt(128), *q.stride(), *k.stride(),
                                          *v.stride(), *o.stride(), CAUSAL=True, lse_ptr=lse, prepare=True)
        launch = lambda i: call()  # noqa: E731
    elif which == "gemm":
        c = inputs.config3(8192, 8192, 8192)
        a = torch.from_numpy(c["a"]).to(dev).to(torch.bfloat16)
        bt = torch.from_numpy(c["bt"]).to(dev).to(torch.bfloat16)
        del c
        y = torch.empty((8192, 8192), dtype=torch.bfloat16, device=dev)
        call = ops.matmul_kernel(a, bt.t(), y, 8192, 8192, 8192, prepare=True)
        launch = lambda i: call()  # noqa: E731
    elif which == "softmax":
        xs = [torch.from_numpy(inputs.config2(8191, 3000, seed=inputs.SEEDS["c2"] + s)["x"]).to(dev)
              .to(torch.bfloat16) for s in range(ROTATE)]
        ys = [torch.empty_like(x) for x in xs]
        calls = [ops.softmax_kernel(x, y, 3000, prepare=True) for x, y in zip(xs, ys)]
        launch = lambda i: calls[i % ROTATE]()  # noqa: E731
    else:
        sys.exit(f"bench.py: --load takes attn, gemm or softmax (not {which!r})")
    torch.cuda.synchronize()
    # host waits once per ~8 ms of queued work, so the GPU never idles long
    batch = 400 if which == "softmax" else 16
    log(f"load {which}: started, {seconds} s")
    n, t_end = 0, time.perf_counter() + seconds
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    while time.perf_counter() < t_end:
        for _ in range(batch):
            launch(n)
            n += 1
        torch.cuda.synchronize()
    end.record()
    end.synchronize()
    print(json.dumps({"load": which, "seconds": seconds, "launches": n,
                      "mean_us": round(start.elapsed_time(end) / n * 1e3, 2)}), flush=True)


def mfma_probe(torch, ops):
    """Counter-collection workload for the MFMA-bound kernels (run under
    rocprofv3 --pmc): C3 bf16 GEMM 8192^3 and 4097x11008x4096, C4 causal GQA
    attention and the C5 int8 GEMM, three launches each after one warm-up
    launch."""
    import math
    from oracle import inputs
    dev = "cuda:0"
    for m, n, k in ((8192, 8192, 8192), (4097, 11008, 4096)):
        c = inputs.config3(m, n, k)
        a = torch.from_numpy(c["a"]).to(dev).to(torch.bfloat16)
        bt = torch.from_numpy(c["bt"]).to(dev).to(torch.bfloat16)
        del c
        y = torch.empty((m, n), dtype=torch.bfloat16, device=dev)
        gemm = ops.matmul_kernel(a, bt.t(), y, m, n, k, prepare=True)
        for _ in range(4):
            gemm()
        torch.cuda.synchronize()
        if m == 8192:
            # comparator, not the product: hipBLASLt (torch.matmul) on the
            # same operands, for its counters beside this kernel's
            for _ in range(4):
                torch.matmul(a, bt.t())
            torch.cuda.synchronize()
            # the reference layout, row-major B, read as it lies (_rb)
            b = bt.t().contiguous()
            rbg = ops.matmul_kernel(a, b, y, m, n, k, prepare=True)
            for _ in range(4):
                rbg()
            torch.cuda.synchronize()
            del b
        del a, bt, y
    c5 = inputs.config5()
    a8, b8 = torch.from_numpy(c5["a"]).to(dev), torch.from_numpy(c5["bt"]).to(dev)
    sa, sb = torch.from_numpy(c5["sa"]).to(dev), torch.from_numpy(c5["sb"]).to(dev)
    y8 = torch.empty((4096, 8192), dtype=torch.bfloat16, device=dev)
    i8 = ops.matmul_i8_dequant_kernel(a8, b8.t(), sa, sb, y8, 4096, 8192, 8192, prepare=True)
    for _ in range(4):
        i8()
    torch.cuda.synchronize()
    del a8, b8, y8, c5
    c = inputs.config4()
    bf = lambda x: torch.from_numpy(x).to(dev).to(torch.bfloat16)  # noqa: E731
    q, kk, v = bf(c["q"]), bf(c["k"]), bf(c["v"])
    o = torch.empty_like(q)
    lse = torch.empty((4, 32, 4096), dtype=torch.float32, device=dev)
    attn = ops.attn_fwd_causal_kernel(q, kk, v, o, 4, 32, 4096, 1 / math.sqrt(128), *q.stride(), *kk.stride(),
                                      *v.stride(), *o.stride(), CAUSAL=True, lse_ptr=lse, prepare=True)
    for _ in range(4):
        attn()
    torch.cuda.synchronize()
    log(f"mfma probe: {gemm.kernel} x4 (two shapes), {rbg.kernel} x4, {i8.kernel} x4, {attn.kernel} x4")


def traffic_for(kernel):
    """HBM bytes per launch measured for `kernel` (profiles/hbm_traffic.json,
    from the rocprofv3 FETCH_SIZE / WRITE_SIZE passes, copy-calibrated)."""
    path = os.path.join(ROOT, "profiles", "hbm_traffic.json")
    try:
        with open(path) as f:
            data = json.load(f)
    except (OSError, ValueError):
        return None
    row = data.get("kernels", {}).get(kernel)
    return None if row is None else int(row["traffic_bytes"])


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-suite", action="store_true", help="headline workload only")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--cpu-seconds", type=float, default=3.0)
    ap.add_argument("--pmc-probe", action="store_true",
                    help="run only the counter-collection workload (for rocprofv3 --pmc)")
    ap.add_argument("--mfma-probe", action="store_true",
                    help="run only the GEMM + attention counter workload (for rocprofv3 --pmc)")
    ap.add_argument("--load", default=None, choices=("attn", "gemm", "softmax"),
                    help="run one config's kernel back to back for --seconds (power/clock sampling beside it)")
    ap.add_argument("--seconds", type=float, default=10.0)
    ap.add_argument("--only", default=None,
                    help="comma-separated suite sections (" + ",".join(SECTIONS) + ", or 'headline'): run just "
                         "these, without the CPU legs, and print their rows (one rocprofv3 trace per config)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU only (asked for {args.gpus}); the multi-GPU "
              "sharding plan is design-only", file=sys.stderr)
        sys.exit(2)

    import torch
    from compiler_amd import operators as ops
    if not torch.cuda.is_available():
        sys.exit("bench.py needs the MI355X")
    if args.pmc_probe:
        pmc_probe(torch, ops)
        return
    if args.mfma_probe:
        mfma_probe(torch, ops)
        return
    if args.load:
        load_probe(torch, ops, args.load, args.seconds)
        return
    if args.only:
        only = set(args.only.split(","))
        bad = only - set(SECTIONS) - {"headline"}
        if bad:
            sys.exit(f"bench.py: unknown --only sections {sorted(bad)} (known: headline, {', '.join(SECTIONS)})")
        rows = {}
        if "headline" in only:
            value, ms_step, wall, roof, per_kernel, step_bytes = headline(torch, ops, args)
            rows["headline"] = {"value": round(value, 1), "unit": "GB/s", "ms_per_step": round(ms_step, 5),
                                "roofline": roof, "kernels": per_kernel}
        rows["suite"] = suite(torch, ops, cpu=False, only=only - {"headline"})
        for r in rows["suite"]:
            log(f"bench:   {r['config']}: {r['value']} {r['unit']} ({r['frac'] * 100:.1f}% of peak; "
                f"median {r['median_us']} us of {r['n_samples']})")
        print(json.dumps({"only": sorted(only), **rows}), flush=True)
        return
    log("bench: headline (config 2) ...")
    value, ms_step, wall, roof, per_kernel, step_bytes = headline(torch, ops, args)
    log(f"bench: headline {value:.1f} GB/s, {ms_step * 1e3:.1f} us/step")
    suite_rows = []
    if not args.no_suite:
        log("bench: suite ...")
        suite_rows = suite(torch, ops, cpu=not args.no_cpu)
        for r in suite_rows:
            log(f"bench:   {r['config']}: {r['value']} {r['unit']} ({r['frac'] * 100:.1f}% of peak)")
    cpu = None
    if not args.no_cpu:
        log("bench: cpu baseline ...")
        cpu = cpu_baseline(args.cpu_seconds)
    line = {
        "metric": METRIC, "value": round(value, 1), "unit": "GB/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms_step, 5),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic (seeded numpy draws of the BASELINE distributions, oracle/inputs.py)",
        "config": {"workload": "C2 masked-tail bf16 LayerNorm + softmax, x[8191,3000] (1% +-60), "
                               "fp32 statistics, 6 rotating buffer sets",
                   "rows": 8191, "cols": 3000, "bytes_per_step": step_bytes},
        "roofline": roof, "kernels": per_kernel, "cpu_baseline": cpu, "suite": suite_rows,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
