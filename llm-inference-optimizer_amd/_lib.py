"""ctypes binding of the gfx950 kernel library ``libmi355_fused.so``.

The library exposes the C ABI declared in ``include/mi355_fused.h``; this
module loads it once, declares the argument types, checks the ABI version and
turns a non-zero status into an exception carrying the library's message.

There is no fallback: if the library has not been built, every kernel call
raises ``KernelLibraryMissing`` (build it with ``python -c "import
__graft_entry__ as g; g.build()"`` or ``python
llm-inference-optimizer_amd/build.py``).
"""
from __future__ import annotations

import ctypes
import threading
from pathlib import Path

import torch

LIB_PATH = Path(__file__).resolve().parent / "libmi355_fused.so"
ABI_VERSION = 1

# dtype codes of the C ABI (enum mi355_dtype)
F32, F16, BF16 = 0, 1, 2
DTYPE_CODE = {torch.float32: F32, torch.float16: F16, torch.bfloat16: BF16}

EXPORTED_SYMBOLS = ("mi355_abi_version", "mi355_last_error", "mi355_rmsnorm_fwd", "mi355_add_rmsnorm_fwd",
                    "mi355_silu_mul_fwd", "mi355_gate_up_silu_fwd", "mi355_w8a16_linear_fwd",
                    "mi355_quantize_int8_fwd", "mi355_gate_up_silu_w8a16_fwd", "mi355_linear16_fwd")


class KernelLibraryMissing(RuntimeError):
    """The HIP kernel library is not built (no silent CPU fallback exists)."""


class KernelError(RuntimeError):
    """A C-ABI call returned a non-zero status."""

    def __init__(self, fn: str, status: int, message: str):
        super().__init__(f"{fn} failed with status {status}: {message}")
        self.status = status


_lock = threading.Lock()
_lib: ctypes.CDLL | None = None
_ext = None


def _declare(L: ctypes.CDLL, path: Path) -> ctypes.CDLL:
    """Declares the C ABI's argument and return types on `L` and checks its
    ABI version."""
    vp, i64, i32 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int
    L.mi355_abi_version.argtypes = []
    L.mi355_abi_version.restype = i32
    L.mi355_last_error.argtypes = []
    L.mi355_last_error.restype = ctypes.c_char_p
    L.mi355_rmsnorm_fwd.argtypes = [vp, vp, vp, i64, i64, i64, i64, ctypes.c_float, i32, i32, i32, vp]
    L.mi355_rmsnorm_fwd.restype = i32
    L.mi355_add_rmsnorm_fwd.argtypes = [vp, vp, vp, vp, vp, i64, i64, i64, i64, i64, i64, ctypes.c_float,
                                        i32, i32, i32, vp]
    L.mi355_add_rmsnorm_fwd.restype = i32
    L.mi355_silu_mul_fwd.argtypes = [vp, vp, vp, i64, i32, i32, vp]
    L.mi355_silu_mul_fwd.restype = i32
    L.mi355_gate_up_silu_fwd.argtypes = [vp, vp, vp, vp, i64, i64, i64, i64, i64, i64, i32, i32, vp]
    L.mi355_gate_up_silu_fwd.restype = i32
    L.mi355_w8a16_linear_fwd.argtypes = [vp, vp, vp, vp, vp, i64, i64, i64, i64, i64, i64, i32, i32, i32, i32,
                                         vp]
    L.mi355_w8a16_linear_fwd.restype = i32
    L.mi355_quantize_int8_fwd.argtypes = [vp, vp, vp, i64, i64, i64, i64, i32, vp]
    L.mi355_quantize_int8_fwd.restype = i32
    L.mi355_gate_up_silu_w8a16_fwd.argtypes = [vp, vp, vp, vp, vp, vp, i64, i64, i64, i64, i64, i64, i32, i32,
                                               i32, vp]
    L.mi355_gate_up_silu_w8a16_fwd.restype = i32
    L.mi355_linear16_fwd.argtypes = [vp, vp, vp, vp, i64, i64, i64, i64, i64, i64, i32, i32, i32, vp]
    L.mi355_linear16_fwd.restype = i32
    ver = L.mi355_abi_version()
    if ver != ABI_VERSION:
        raise KernelLibraryMissing(f"{path} has ABI version {ver}, expected {ABI_VERSION}; rebuild it")
    return L


def load() -> ctypes.CDLL:
    """Load (once) and return the kernel library."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not LIB_PATH.exists():
            raise KernelLibraryMissing(
                f"{LIB_PATH} is not built; run `python -c \"import __graft_entry__ as g; g.build()\"` "
                "from the repository root (there is no CPU fallback)")
        _lib = _declare(ctypes.CDLL(str(LIB_PATH)), LIB_PATH)
    return _lib


def ext():
    """The host-side launchers (``_mi355_torch``, a torch extension over this
    library's C ABI; see csrc/torch_launchers.cpp), loaded once.  Raises
    KernelLibraryMissing when it is not built."""
    global _ext
    if _ext is not None:
        return _ext
    load()
    with _lock:
        if _ext is None:
            try:
                from . import _mi355_torch as mod
            except ImportError as e:
                raise KernelLibraryMissing(
                    f"the torch launcher extension _mi355_torch is not built next to {LIB_PATH} ({e}); run "
                    "`python -c \"import __graft_entry__ as g; g.build()\"` from the repository root") from e
            if mod.abi_version() != ABI_VERSION:
                raise KernelLibraryMissing(f"_mi355_torch was built against ABI {mod.abi_version()}, "
                                           f"expected {ABI_VERSION}; rebuild it")
            mod.set_kernel_error(KernelError)
            _ext = mod
    return _ext


def check(fn: str, status: int) -> None:
    if status != 0:
        raise KernelError(fn, status, load().mi355_last_error().decode(errors="replace"))


_raw_stream = torch._C._cuda_getCurrentRawStream   # device index -> hipStream_t as int
_current_device = torch._C._cuda_getDevice


def stream_handle(device) -> int:
    """hipStream_t of torch's current stream on ``device`` (torch.device or
    index), as an integer."""
    idx = device if isinstance(device, int) else device.index
    return _raw_stream(_current_device() if idx is None else idx)


def launch(fn: str, device_index: int, *args) -> None:
    """Calls C-ABI entry point `fn` with `args` plus torch's current stream on
    `device_index`, with that device current; raises KernelError on failure.
    The hot path of the Python launchers (a few hundred ns above the call)."""
    f = getattr(load(), fn)
    if device_index == _current_device():
        st = f(*args, _raw_stream(device_index))
    else:
        with torch.cuda.device(device_index):
            st = f(*args, _raw_stream(device_index))
    if st != 0:
        check(fn, st)


def rmsnorm_fwd(x_ptr: int, w_ptr: int, y_ptr: int, rows: int, n: int, x_row_stride: int,
                y_row_stride: int, eps: float, x_dtype: int, w_dtype: int, y_dtype: int, stream: int) -> None:
    check("mi355_rmsnorm_fwd",
          load().mi355_rmsnorm_fwd(x_ptr, w_ptr, y_ptr, rows, n, x_row_stride, y_row_stride, eps,
                                   x_dtype, w_dtype, y_dtype, stream))


def add_rmsnorm_fwd(x_ptr: int, r_ptr: int, w_ptr: int, y_ptr: int, ro_ptr: int, rows: int, n: int,
                    x_row_stride: int, r_row_stride: int, y_row_stride: int, ro_row_stride: int, eps: float,
                    x_dtype: int, w_dtype: int, y_dtype: int, stream: int) -> None:
    check("mi355_add_rmsnorm_fwd",
          load().mi355_add_rmsnorm_fwd(x_ptr, r_ptr, w_ptr, y_ptr, ro_ptr, rows, n, x_row_stride, r_row_stride,
                                       y_row_stride, ro_row_stride, eps, x_dtype, w_dtype, y_dtype, stream))


def silu_mul_fwd(gate_ptr: int, up_ptr: int, out_ptr: int, numel: int, in_dtype: int, out_dtype: int,
                 stream: int) -> None:
    check("mi355_silu_mul_fwd",
          load().mi355_silu_mul_fwd(gate_ptr, up_ptr, out_ptr, numel, in_dtype, out_dtype, stream))


def gate_up_silu_fwd(x_ptr: int, wg_ptr: int, wu_ptr: int, out_ptr: int, rows: int, k: int, n_out: int,
                     x_row_stride: int, w_row_stride: int, out_row_stride: int, dtype: int, out_dtype: int,
                     stream: int) -> None:
    check("mi355_gate_up_silu_fwd",
          load().mi355_gate_up_silu_fwd(x_ptr, wg_ptr, wu_ptr, out_ptr, rows, k, n_out, x_row_stride, w_row_stride,
                                        out_row_stride, dtype, out_dtype, stream))


def w8a16_linear_fwd(x_ptr: int, q_ptr: int, scale_ptr: int, bias_ptr: int | None, out_ptr: int, rows: int, k: int,
                     n: int, x_row_stride: int, w_row_stride: int, out_row_stride: int, x_dtype: int,
                     scale_dtype: int, bias_dtype: int, out_dtype: int, stream: int) -> None:
    check("mi355_w8a16_linear_fwd",
          load().mi355_w8a16_linear_fwd(x_ptr, q_ptr, scale_ptr, bias_ptr, out_ptr, rows, k, n, x_row_stride,
                                        w_row_stride, out_row_stride, x_dtype, scale_dtype, bias_dtype, out_dtype,
                                        stream))


def gate_up_silu_w8a16_fwd(x_ptr: int, qg_ptr: int, qu_ptr: int, sg_ptr: int, su_ptr: int, out_ptr: int, rows: int,
                           k: int, n_out: int, x_row_stride: int, w_row_stride: int, out_row_stride: int,
                           x_dtype: int, scale_dtype: int, out_dtype: int, stream: int) -> None:
    check("mi355_gate_up_silu_w8a16_fwd",
          load().mi355_gate_up_silu_w8a16_fwd(x_ptr, qg_ptr, qu_ptr, sg_ptr, su_ptr, out_ptr, rows, k, n_out,
                                              x_row_stride, w_row_stride, out_row_stride, x_dtype, scale_dtype,
                                              out_dtype, stream))


def quantize_int8_fwd(w_ptr: int, q_ptr: int, scale_ptr: int, n: int, k: int, w_row_stride: int,
                      q_row_stride: int, w_dtype: int, stream: int) -> None:
    check("mi355_quantize_int8_fwd",
          load().mi355_quantize_int8_fwd(w_ptr, q_ptr, scale_ptr, n, k, w_row_stride, q_row_stride, w_dtype, stream))


def linear16_fwd(x_ptr: int, w_ptr: int, bias_ptr: int | None, out_ptr: int, rows: int, k: int, n: int,
                 x_row_stride: int, w_row_stride: int, out_row_stride: int, dtype: int, bias_dtype: int,
                 out_dtype: int, stream: int) -> None:
    check("mi355_linear16_fwd",
          load().mi355_linear16_fwd(x_ptr, w_ptr, bias_ptr, out_ptr, rows, k, n, x_row_stride, w_row_stride,
                                    out_row_stride, dtype, bias_dtype, out_dtype, stream))
