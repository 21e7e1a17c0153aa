"""ctypes binding of libdscq.so (include/dscq.h).

The library is built in-tree by ``python -m dscquant_amd.build``.  torch is
imported first so that the HIP runtime torch ships is the one libdscq binds
to (both are ``libamdhip64.so.7``): tensors, streams and kernels then share
one runtime.  There is no fallback: if the library is missing, every entry
point raises.
"""
from __future__ import annotations

import ctypes
import os
import threading

import torch  # noqa: F401  (loads torch's HIP runtime before libdscq)

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "lib", "libdscq.so")

F16, F32 = 0, 1

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None

# name -> argtypes, in include/dscq.h order.
_P, _I, _I64, _F = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_float
SIGNATURES = {
    "dscq_quantize": [_P, _I, _I64, _I64, _F, _I, _I, _P, _P, _P, _P, _P],
    "dscq_silu_mul_quantize": [_P, _P, _I64, _I64, _I64, _F, _I, _P, _P, _P, _P, _P],
    "dscq_matmul_silu_mul": [_P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _P, _P],
    "dscq_activation_codes": [_P, _I, _I64, _I64, _F, _I, _I, _P, _P, _P, _P],
    "dscq_pack_weight": [_P, _I, _I64, _I64, _F, _I, _P, _P, _P, _P, _P],
    "dscq_weight_codes": [_P, _I, _I64, _I64, _F, _I, _I, _P, _P, _P],
    "dscq_matmul": [_P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I, _I, _I, _P, _P, _P],
    "dscq_matmul_ws": [_P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I, _I, _I, _P, _P,
                       _P, _I64, _P],
    "dscq_matmul_noalloc": [_P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I, _I, _I, _P, _P,
                            _P],
    "dscq_matmul_workspace_bytes": [_I64, _I64, _I64, _I],
    "dscq_linear_decode": [_P, _I, _I64, _I64, _F, _I, _P, _P, _P, _P, _I64, _I, _P, _P],
    "dscq_linear_decode_supported": [_I64, _I64],
    "dscq_pack_int4": [_P, _I64, _I64, _P, _P],
    "dscq_unpack_int4": [_P, _I64, _I64, _I64, _P, _P],
    "dscq_time_next_kernel": [_P, _P],
    "dscq_set_gemm_kernel": [_I],
    "dscq_stream_probe": [_P, _I64, _P, _I64, _I, _P],
    "dscq_mfma_probe": [_I64, _I, _I64, _P, _P],
    "dscq_device_supported": [],
    "dscq_last_error": [],
    "dscq_version": [],
}


def lib() -> ctypes.CDLL:
    """The loaded library (raises if it has not been built)."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise RuntimeError(
                    f"libdscq.so not found at {LIB_PATH}: build it with "
                    "`python -m dscquant_amd.build` (the HIP path has no fallback)")
            L = ctypes.CDLL(LIB_PATH)
            for name, argtypes in SIGNATURES.items():
                fn = getattr(L, name)
                fn.argtypes = argtypes
                fn.restype = ctypes.c_int
            L.dscq_last_error.restype = ctypes.c_char_p
            L.dscq_version.restype = ctypes.c_char_p
            L.dscq_matmul_workspace_bytes.restype = ctypes.c_int64
            _lib = L
    return _lib


def call(name: str, *args) -> None:
    """Calls a dscq_* entry point; raises RuntimeError with its message on failure."""
    L = lib()
    rc = getattr(L, name)(*args)
    if rc != 0:
        msg = L.dscq_last_error().decode(errors="replace")
        raise RuntimeError(msg or f"{name} failed with code {rc}")


def ptr(t) -> int | None:
    """Device pointer of a tensor (None for None / empty tensors)."""
    if t is None or t.numel() == 0:
        return None
    return t.data_ptr()


def stream(device: torch.device) -> int:
    """hipStream_t of torch's current stream on `device`."""
    return torch.cuda.current_stream(device).cuda_stream


_supported: dict[int, bool] = {}


def require_gfx950(device: torch.device) -> None:
    """The gfx950 check that replaces kernel/w4a4.cu:204-206."""
    idx = device.index if device.index is not None else torch.cuda.current_device()
    ok = _supported.get(idx)
    if ok is None:
        with torch.cuda.device(idx):
            ok = lib().dscq_device_supported() == 1
        _supported[idx] = ok
    if not ok:
        name = torch.cuda.get_device_properties(idx).gcnArchName
        raise RuntimeError(f"This W4A4 backend targets gfx950 (MI355X); device {idx} is {name}")
