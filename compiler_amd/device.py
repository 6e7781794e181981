"""A harness ``Device`` for the gfx950 hot path.

It implements the reference harness's Device protocol
(ops/harness/opslib/device.py:79-118: alloc / upload / download / pointer /
synchronize / compare / launch) so the reference's own case loop
(``stage_case`` -> ``StagedCase.launch`` -> ``Device.launch``, device.py:323-415)
can drive these kernels unchanged.  ``launch`` receives the reference kernel
object (or any callable with the same parameter names), binds the positional
arguments by that signature exactly as ``bind_arguments`` produced them
(device.py:232-260), and dispatches by the kernel's NAME to the matching
operator of ``compiler_amd.operators``.  Kernels outside the hot path are
refused with ``NotImplementedError`` -- there is no fallback.

bf16 follows the harness's pointer duality (ops/harness/compiler_api/
AGENT_GUIDE.md:253): a float32 host array is rounded to bf16 on upload, a
uint16 host array is taken as raw bf16 bits; bf16 buffers download as float32
values.  Launches are synchronous, as the contract requires
(ops/harness/compiler_api/COMPILE_CONTRACT.md:73-74).
"""
from __future__ import annotations

import inspect

import numpy as np

from . import operators as ops

_NP_TO_TORCH = {"float32": "float32", "float16": "float16", "bfloat16": "bfloat16",
                "int8": "int8", "uint8": "uint8", "int16": "int16", "int32": "int32",
                "int64": "int64", "float64": "float64", "bool": "bool"}


class G950Buffer:
    """A device buffer: a torch-ROCm tensor plus its logical dtype name."""

    def __init__(self, tensor, dtype_name: str):
        self.tensor = tensor
        self._dtype = dtype_name

    def data_ptr(self):
        return self.tensor.data_ptr()

    @property
    def dtype(self):
        return self._dtype

    @property
    def shape(self):
        return tuple(self.tensor.shape)


def _kernel_name(kernel) -> str:
    target = kernel
    for attr in ("fn", "fn"):  # autotuner -> JITFunction -> python function
        target = getattr(target, attr, target)
    return getattr(target, "__name__", str(kernel))


def _kernel_params(kernel):
    """Parameter names in the order ``bind_arguments`` emits positional values:
    constexprs an autotuner supplies are skipped (device.py:241-252)."""
    configs = getattr(kernel, "configs", None)
    tuned = set((getattr(configs[0], "kwargs", {}) or {}).keys()) if configs else set()
    target = kernel
    for attr in ("fn", "fn"):
        target = getattr(target, attr, target)
    return [p for p in inspect.signature(target).parameters if p not in tuned]


def _softmax(a, sync):
    ops.softmax_kernel(a["x_ptr"], a["y_ptr"], a["n_cols"], sync=sync)


def _softmax_inner(a, sync):
    ops.softmax_kernel_inner(a["output_ptr"], a["input_ptr"], a["M"], a["N"], a.get("TILE_N"),
                             a.get("ONE_TILE_PER_CTA"), sync=sync)


def _layer_norm_row(a, sync):
    ops.layer_norm_forward_row(a["Y_ptr"], a["Y_row_stride"], a["X_ptr"], a["X_row_stride"], a["W_ptr"],
                               a["B_ptr"], a["Mean_ptr"], a["Mean_row_stride"], a["RSTD_ptr"],
                               a["RSTD_row_stride"], a["n_rows"], a["n_cols"], a["eps"], a.get("BLOCK_SIZE"),
                               sync=sync)


def _gqa(a, sync):
    names = ["stride_qh", "stride_qm", "stride_qk", "stride_kh", "stride_kn", "stride_kk", "stride_vh",
             "stride_vk", "stride_vn", "stride_oh", "stride_om", "stride_on"]
    ops.gqa_kernel(a["Q"], a["K"], a["V"], a["Out"], *[a[n] for n in names], a["H_Q"], a["H_KV"], a["N_CTX"],
                   a["scale"], a["GROUP"], a.get("HEAD_DIM"), sync=sync)


def _logsumexp(a, sync):
    ops.logsumexp_kernel(a["x_ptr"], a["y_ptr"], a["n_cols"], sync=sync)


def _dequantize(a, sync):
    ops.dequantize_kernel(a["b_ptr"], a["b_scale_ptr"], a["fpb_ptr"], a["K"], a["N"], a["stride_bk"],
                          a["stride_bn"], a["stride_fpbk"], a["stride_fpbn"], sync=sync)


def _flash_varlen(a, sync):
    from .operators import _VARLEN_SCALARS, _VARLEN_VIEWS
    ops.flash_varlen_fwd_kernel(**{n: a[n] for n in _VARLEN_VIEWS + _VARLEN_SCALARS}, sync=sync)


def _rms(a, sync):
    ops.rms_layernorm_forward_kernel(a["Y"], a["Y_row_stride"], a["X"], a["X_row_stride"], a["W"],
                                     a["W_row_stride"], a["r"], a["r_row_stride"], a["n_cols"],
                                     a["eps"], sync=sync)


def _layernorm(a, sync):
    ops.layernorm_kernel(a["X"], a["Y"], a["W"], a["B"], a["Mean"], a["Rstd"], a["stride"], a["N"],
                         a["eps"], sync=sync)


def _matmul(a, sync):
    ops.matmul_kernel(a["a_ptr"], a["b_ptr"], a["y_ptr"], a["M"], a["N"], a["K"], sync=sync)


def _attention(a, causal_default, sync):
    names = ["stride_qz", "stride_qh", "stride_qm", "stride_qk", "stride_kz", "stride_kh",
             "stride_kn", "stride_kk", "stride_vz", "stride_vh", "stride_vk", "stride_vn",
             "stride_oz", "stride_oh", "stride_om", "stride_on"]
    ops.attn_fwd_causal_kernel(a["q_ptr"], a["k_ptr"], a["v_ptr"], a["out_ptr"], a["Z"], a["H"],
                               a["N_CTX"], a["scale"], *[a[n] for n in names],
                               CAUSAL=bool(a.get("CAUSAL", causal_default)), sync=sync)


# reference kernel name -> operator (hot path only)
KERNELS = {
    "softmax_kernel": _softmax,
    "softmax_kernel_inner": _softmax_inner,
    "_layer_norm_forward_row": _layer_norm_row,
    "gqa_kernel": _gqa,
    "logsumexp_kernel": _logsumexp,
    "dequantize_kernel": _dequantize,
    "flash_varlen_fwd_kernel": _flash_varlen,
    "rms_layernorm_forward_kernel": _rms,
    "layernorm_kernel": _layernorm,
    "matmul_kernel": _matmul,
    "attn_fwd_causal_kernel": lambda a, sync: _attention(a, True, sync),
    "attention_forward_kernel": lambda a, sync: _attention(a, False, sync),
}


class G950Timer:
    """``with timer: launch()`` brackets the launch with two HIP events on
    the launch stream.  Inside the block the device launches without a host
    wait, so the end event lands right behind the kernels; leaving the block
    waits for it, so the launch has finished when the block ends (the
    contract of COMPILE_CONTRACT.md:73-74).  ``seconds`` is the elapsed GPU
    time between the events."""

    def __init__(self, device):
        torch = device.torch
        self._device = device
        self._start = torch.cuda.Event(enable_timing=True)
        self._end = torch.cuda.Event(enable_timing=True)
        self.seconds = None

    def __enter__(self):
        torch = self._device.torch
        self._stream = torch.cuda.current_stream(self._device.device)
        self._start.record(self._stream)
        self._device._timing = True
        return self

    def __exit__(self, *exc):
        self._device._timing = False
        self._end.record(self._stream)
        self._end.synchronize()
        self.seconds = self._start.elapsed_time(self._end) / 1000.0
        return False


class G950Device:
    """Device protocol implementation over torch-ROCm memory and the g950 C ABI."""

    name = "g950"

    def __init__(self, device: str = "cuda:0"):
        import torch
        if not torch.cuda.is_available():
            raise RuntimeError("G950Device needs an MI355X (gfx950) GPU")
        self.torch = torch
        self.device = torch.device(device)
        self._timing = False   # inside a timer: launches stay asynchronous

    # -- memory -----------------------------------------------------------
    def _tdtype(self, name):
        return getattr(self.torch, _NP_TO_TORCH[name])

    def alloc(self, shape, dtype):
        name = np.dtype(dtype).name if dtype != "bfloat16" else "bfloat16"
        return G950Buffer(self.torch.zeros(tuple(shape), dtype=self._tdtype(name), device=self.device), name)

    def upload(self, array, dtype=None):
        array = np.ascontiguousarray(array)
        target = dtype if dtype is not None else array.dtype.name
        if target == "bfloat16":
            if array.dtype == np.uint16:
                t = self.torch.from_numpy(array.view(np.int16)).to(self.device).view(self.torch.bfloat16)
            else:
                t = self.torch.from_numpy(array.astype(np.float32)).to(self.device).to(self.torch.bfloat16)
            return G950Buffer(t, "bfloat16")
        t = self.torch.from_numpy(array.astype(target, copy=False)).to(self.device)
        return G950Buffer(t, target)

    def download(self, buffer):
        t = buffer.tensor
        if buffer.dtype == "bfloat16":
            return t.float().cpu().numpy()
        return t.cpu().numpy()

    def pointer(self, buffer):
        return buffer.data_ptr()

    def synchronize(self):
        self.torch.cuda.synchronize(self.device)

    def compare(self, buffer, expected, policy):
        return None  # host comparison by the harness

    def timer(self):
        """Device-event timing for the reference benchmark
        (ops/harness/benchmark/run.py:126-133,255): ``with timer: launch()``
        then ``timer.seconds``."""
        return G950Timer(self)

    def release(self, buffers):
        """Free buffers (a dict or iterable of G950Buffer) the reference
        benchmark is done with (benchmark/run.py:126-133); their memory goes
        back to torch's allocator for the next entry."""
        items = buffers.values() if isinstance(buffers, dict) else buffers
        for b in items:
            if isinstance(b, G950Buffer):
                b.tensor = None

    def properties(self):
        p = self.torch.cuda.get_device_properties(self.device)
        return {"name": p.name, "gcn_arch": getattr(p, "gcnArchName", ""),
                "multiprocessors": p.multi_processor_count, "total_memory": p.total_memory}

    # -- launch -----------------------------------------------------------
    def launch(self, kernel, grid, positional, keywords):
        name = _kernel_name(kernel)
        if name not in KERNELS:
            raise NotImplementedError(f"{name} is not a g950 hot-path operator")
        params = _kernel_params(kernel)
        values = dict(zip(params, positional))
        values.update(keywords or {})
        args = {k: (v.tensor if isinstance(v, G950Buffer) else v) for k, v in values.items()}
        with self.torch.cuda.device(self.device):
            KERNELS[name](args, not self._timing)
