"""ctypes binding of the gfx950 loader/launcher (include/g950rt.h).

The product path is: torch-ROCm tensors (allocation, I/O, stream) ->
``g950_view``/``g950_scalar`` records -> ``g950_launch`` -> a kernel of the
single gfx950 code object.  There is no fallback: if the library or code
object is missing, or no GPU is present, loading raises ``G950Error``.
"""
from __future__ import annotations

import ctypes
import threading
from pathlib import Path

import numpy as np

PKG = Path(__file__).resolve().parent
LIB_PATH = PKG / "lib" / "libg950rt.so"
HSACO_PATH = PKG / "lib" / "g950.hsaco"

OK, USAGE, REJECTED, RESOURCE, REPEAT_MISMATCH, SYNC = 0, 2, 3, 4, 5, 6

# operator contracts (include/g950rt.h)
OP_SOFTMAX = 1
OP_RMS_LAYERNORM = 2
OP_LAYERNORM = 3
OP_MATMUL = 4
OP_MATMUL_I8 = 5
OP_MATMUL_I8_DEQUANT = 6
OP_ATTENTION = 7
OP_ATTENTION_LSE = 8
OP_COPY = 9
OP_LOGSUMEXP = 10
OP_DEQUANTIZE = 11
OP_FLASH_VARLEN = 12
OP_DEQUANT_MATMUL = 13
OP_SOFTMAX_INNER = 14
OP_LAYERNORM_ROW = 15
OP_GQA = 16

# dtype codes (a100c/runtime/a100rt.h:58-72)
DT_BOOL, DT_INT8, DT_UINT8, DT_INT16, DT_UINT16, DT_INT32 = 1, 2, 3, 4, 5, 6
DT_UINT32, DT_INT64, DT_UINT64, DT_F16, DT_BF16, DT_F32, DT_F64 = 7, 8, 9, 10, 11, 12, 13

EXPORTS = ("g950_open", "g950_launch", "g950_launch_noalloc", "g950_workspace_bytes", "g950_validate",
           "g950_last_kernel", "g950_sync", "g950_strerror",
           "g950_last_error", "g950_close", "g950_bundle_open", "g950_bundle_check", "g950_bundle_reason",
           "g950_bundle_count", "g950_bundle_view", "g950_bundle_scalar", "g950_bundle_exec",
           "g950_bundle_close")


class G950Error(RuntimeError):
    def __init__(self, code: int, message: str):
        super().__init__(f"[g950 {code}] {message}")
        self.code = code


class View(ctypes.Structure):
    _fields_ = [("data", ctypes.c_void_p), ("shape", ctypes.POINTER(ctypes.c_int64)),
                ("strides", ctypes.POINTER(ctypes.c_int64)), ("storage_size", ctypes.c_uint64),
                ("dtype", ctypes.c_uint32), ("ndim", ctypes.c_uint32), ("flags", ctypes.c_uint32),
                ("reserved_", ctypes.c_uint32), ("storage", ctypes.c_void_p)]


class Scalar(ctypes.Structure):
    _fields_ = [("dtype", ctypes.c_uint32), ("size", ctypes.c_uint32), ("bits", ctypes.c_uint64)]


assert ctypes.sizeof(View) == 56 and ctypes.sizeof(Scalar) == 16

_lib = None
_lib_lock = threading.Lock()

# G950_NOALLOC_SCRATCH_BYTES (include/g950rt.h)
NOALLOC_SCRATCH_BYTES = 32 << 20

_mode = threading.local()


class no_alloc:
    """Within ``with no_alloc():`` every operator call on this thread goes
    through ``g950_launch_noalloc``: no device allocation, workspace from the
    library's static scratch array (calls that need more are refused)."""

    def __enter__(self):
        self._prev = getattr(_mode, "noalloc", False)
        _mode.noalloc = True
        return self

    def __exit__(self, *exc):
        _mode.noalloc = self._prev
        return False


def noalloc_active() -> bool:
    return getattr(_mode, "noalloc", False)


def load_library():
    """Load libg950rt.so (does not touch the GPU)."""
    global _lib
    with _lib_lock:
        if _lib is not None:
            return _lib
        if not LIB_PATH.exists():
            raise G950Error(RESOURCE, f"{LIB_PATH} is not built (run __graft_entry__.build())")
        lib = ctypes.CDLL(str(LIB_PATH))
        lib.g950_open.argtypes = [ctypes.c_char_p, ctypes.POINTER(ctypes.c_void_p)]
        lib.g950_open.restype = ctypes.c_int
        lib.g950_launch.argtypes = [ctypes.c_void_p, ctypes.c_uint32, ctypes.POINTER(View),
                                    ctypes.c_uint32, ctypes.POINTER(Scalar), ctypes.c_uint32,
                                    ctypes.c_void_p]
        lib.g950_launch.restype = ctypes.c_int
        lib.g950_launch_noalloc.argtypes = lib.g950_launch.argtypes
        lib.g950_launch_noalloc.restype = ctypes.c_int
        lib.g950_workspace_bytes.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
        lib.g950_workspace_bytes.restype = ctypes.c_size_t
        lib.g950_validate.argtypes = [ctypes.c_uint32, ctypes.POINTER(View), ctypes.c_uint32,
                                      ctypes.POINTER(Scalar), ctypes.c_uint32]
        lib.g950_validate.restype = ctypes.c_int
        lib.g950_last_kernel.restype = ctypes.c_char_p
        lib.g950_sync.argtypes = [ctypes.c_void_p]
        lib.g950_sync.restype = ctypes.c_int
        lib.g950_strerror.argtypes = [ctypes.c_int]
        lib.g950_strerror.restype = ctypes.c_char_p
        lib.g950_last_error.restype = ctypes.c_char_p
        lib.g950_close.argtypes = [ctypes.c_void_p]
        lib.g950_close.restype = None
        vp, u32, i32p = ctypes.c_void_p, ctypes.c_uint32, ctypes.POINTER(ctypes.c_int)
        lib.g950_bundle_open.argtypes = [ctypes.c_char_p, u32, ctypes.POINTER(vp), i32p]
        lib.g950_bundle_check.argtypes = [ctypes.c_char_p, ctypes.c_uint64, i32p]
        lib.g950_bundle_reason.argtypes = [ctypes.c_int]
        lib.g950_bundle_reason.restype = ctypes.c_char_p
        lib.g950_bundle_count.argtypes = [vp, ctypes.c_int]
        lib.g950_bundle_count.restype = u32
        lib.g950_bundle_view.argtypes = [vp, u32, ctypes.POINTER(View)]
        lib.g950_bundle_scalar.argtypes = [vp, u32, ctypes.POINTER(Scalar)]
        lib.g950_bundle_exec.argtypes = [vp, vp, u32, ctypes.POINTER(Scalar), u32, u32, vp, i32p]
        lib.g950_bundle_close.argtypes = [vp]
        _lib = lib
        return lib


def bundle_check(image: bytes) -> str | None:
    """Native a100-native-io/v1 validation of an in-memory image: None if the
    image is valid, else the reference reader's reason name."""
    lib = load_library()
    reason = ctypes.c_int(0)
    rc = lib.g950_bundle_check(bytes(image), len(image), ctypes.byref(reason))
    return None if rc == OK else lib.g950_bundle_reason(reason.value).decode()


def _torch_dtype_code(t) -> int:
    import torch
    table = {torch.float32: DT_F32, torch.bfloat16: DT_BF16, torch.float16: DT_F16,
             torch.int8: DT_INT8, torch.uint8: DT_UINT8, torch.int16: DT_INT16,
             torch.int32: DT_INT32, torch.int64: DT_INT64, torch.float64: DT_F64,
             torch.bool: DT_BOOL}
    if t.dtype not in table:
        raise G950Error(USAGE, f"unsupported tensor dtype {t.dtype}")
    return table[t.dtype]


def scalar(value, dtype: str | None = None) -> Scalar:
    """Encode a scalar the way the reference host packer does
    (a100_support/native_io.py:29-46): numpy scalars keep their dtype, Python
    ints become int64, floats float64, bools bool."""
    if dtype is not None:
        arr = np.asarray(value, dtype=dtype)
    elif isinstance(value, np.generic):
        arr = np.asarray(value)
    elif isinstance(value, bool):
        arr = np.asarray(value, dtype=np.bool_)
    elif isinstance(value, int):
        arr = np.asarray(value, dtype=np.int64)
    elif isinstance(value, float):
        arr = np.asarray(value, dtype=np.float64)
    else:
        raise G950Error(USAGE, f"unsupported scalar {type(value).__name__}")
    codes = {"bool": DT_BOOL, "int8": DT_INT8, "uint8": DT_UINT8, "int16": DT_INT16,
             "uint16": DT_UINT16, "int32": DT_INT32, "uint32": DT_UINT32, "int64": DT_INT64,
             "uint64": DT_UINT64, "float16": DT_F16, "float32": DT_F32, "float64": DT_F64}
    bits = int.from_bytes(arr.astype(arr.dtype.newbyteorder("<")).tobytes(), "little")
    return Scalar(codes[arr.dtype.name], arr.itemsize, bits)


class _ViewArray:
    """Keeps the ctypes shape/stride arrays alive for the duration of a call."""

    def __init__(self, tensors, outputs):
        n = len(tensors)
        self.views = (View * max(n, 1))()
        self._keep = []
        for i, (t, out) in enumerate(zip(tensors, outputs)):
            if not t.is_cuda:
                raise G950Error(USAGE, "g950 operators take device (cuda/hip) tensors")
            nd = t.dim()
            shape = (ctypes.c_int64 * max(nd, 1))(*t.shape)
            strides = (ctypes.c_int64 * max(nd, 1))(*[s * t.element_size() for s in t.stride()])
            self._keep += [shape, strides]
            storage = t.untyped_storage()
            v = self.views[i]
            v.data = t.data_ptr()
            v.shape = shape
            v.strides = strides
            v.storage_size = storage.nbytes()
            v.dtype = _torch_dtype_code(t)
            v.ndim = nd
            v.flags = 1 if out else 0
            v.storage = storage.data_ptr()


class Module:
    """One loaded code object on the current device."""

    def __init__(self, hsaco: Path | str = HSACO_PATH):
        import torch
        lib = load_library()
        if not torch.cuda.is_available():
            raise G950Error(RESOURCE, "no HIP device: the g950 kernels need an MI355X (gfx950)")
        if not Path(hsaco).exists():
            raise G950Error(RESOURCE, f"{hsaco} is not built (run __graft_entry__.build())")
        torch.cuda.init()
        self.device = torch.cuda.current_device()
        handle = ctypes.c_void_p()
        rc = lib.g950_open(str(hsaco).encode(), ctypes.byref(handle))
        if rc != OK:
            raise G950Error(rc, lib.g950_last_error().decode())
        self._lib = lib
        self._handle = handle
        self.last_kernel = ""

    def launch(self, op: int, tensors, outputs, scalars, stream=None, sync=False):
        """Launch operator ``op``.  ``tensors``/``scalars`` are in sorted
        argument-name order; ``outputs`` flags the output views."""
        import torch
        views = _ViewArray(tensors, outputs)
        sc = (Scalar * max(len(scalars), 1))(*scalars)
        if stream is None:
            stream = torch.cuda.current_stream(self.device)
        handle = ctypes.c_void_p(stream.cuda_stream if hasattr(stream, "cuda_stream") else stream)
        entry = self._lib.g950_launch_noalloc if noalloc_active() else self._lib.g950_launch
        rc = entry(self._handle, op, views.views, len(tensors), sc, len(scalars), handle)
        if rc != OK:
            raise G950Error(rc, self._lib.g950_last_error().decode())
        self.last_kernel = self._lib.g950_last_kernel().decode()
        if sync:
            rc = self._lib.g950_sync(handle)
            if rc != OK:
                raise G950Error(rc, self._lib.g950_last_error().decode())
        return self.last_kernel

    def workspace_bytes(self, stream=None) -> int:
        """Device workspace bytes the library holds for ``stream`` (the
        current stream by default); g950_launch_noalloc never changes it."""
        import torch
        if stream is None:
            stream = torch.cuda.current_stream(self.device)
        handle = ctypes.c_void_p(stream.cuda_stream if hasattr(stream, "cuda_stream") else stream)
        return int(self._lib.g950_workspace_bytes(self._handle, handle))

    def prepare(self, op: int, tensors, outputs, scalars, stream=None):
        """Pack the call once; the returned object re-launches it with one C
        call (the launcher still validates every launch)."""
        return Prepared(self, op, tensors, outputs, scalars, stream)

    def close(self):
        if getattr(self, "_handle", None):
            self._lib.g950_close(self._handle)
            self._handle = None


_modules: dict = {}


def module() -> Module:
    """The process-wide module for the current device (loaded once)."""
    import torch
    dev = torch.cuda.current_device() if torch.cuda.is_available() else -1
    mod = _modules.get(dev)
    if mod is None:
        mod = Module()
        _modules[dev] = mod
    return mod


class Prepared:
    """A packed operator call: views, scalars and stream built once."""

    def __init__(self, module: Module, op, tensors, outputs, scalars, stream=None):
        import torch
        self._module = module
        self._tensors = list(tensors)  # keep the storages alive
        self._views = _ViewArray(self._tensors, outputs)
        self._n = len(self._tensors)
        self._scalars = (Scalar * max(len(scalars), 1))(*scalars)
        self._ns = len(scalars)
        self._op = op
        if stream is None:
            stream = torch.cuda.current_stream(module.device)
        self._stream = ctypes.c_void_p(stream.cuda_stream if hasattr(stream, "cuda_stream") else stream)
        self.kernel = ""

    def __call__(self):
        lib = self._module._lib
        rc = lib.g950_launch(self._module._handle, self._op, self._views.views, self._n,
                             self._scalars, self._ns, self._stream)
        if rc != OK:
            raise G950Error(rc, lib.g950_last_error().decode())
        if not self.kernel:
            self.kernel = lib.g950_last_kernel().decode()
            self._module.last_kernel = self.kernel
