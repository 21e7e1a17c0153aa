"""ctypes front end of oracle/dscq_oracle.c (test infrastructure only).

All arrays are numpy; fp16 inputs are widened to fp32 exactly before they
reach C.  See dscq_oracle.c for the reference citations of each rule.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "lib", "liboracle.so")
_lib = None


def build() -> str:
    """Compile the C oracle with its Makefile (gcc, -ffp-contract=off)."""
    import subprocess

    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return LIB_PATH


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"oracle library missing at {LIB_PATH}; run `make -C oracle`")
        L = ctypes.CDLL(LIB_PATH)
        P, I64, F, I = ctypes.c_void_p, ctypes.c_int64, ctypes.c_float, ctypes.c_int
        L.oracle_activation_codes.argtypes = [P, I64, I64, F, I, P, P, P]
        L.oracle_weight_codes.argtypes = [P, I64, I64, F, I, P, P]
        L.oracle_fwht_rows.argtypes = [P, I64, I64, I]
        L.oracle_quantize_rows.argtypes = [P, I64, I64, F, P, P, P, P]
        L.oracle_pack_int4.argtypes = [P, I64, I64, P]
        L.oracle_unpack_int4.argtypes = [P, I64, I64, I64, P]
        L.oracle_pack_weight.argtypes = [P, I64, I64, F, I, P, P, P, P, P]
        L.oracle_gemm_raw.argtypes = [P, P, I64, I64, I64, P]
        L.oracle_gemm_raw.restype = ctypes.c_int
        L.oracle_restore.argtypes = [P, P, P, P, P, P, I64, I64, P]
        for fn in ("oracle_activation_codes", "oracle_weight_codes",
                   "oracle_fwht_rows", "oracle_quantize_rows",
                   "oracle_pack_int4", "oracle_unpack_int4",
                   "oracle_pack_weight", "oracle_restore"):
            getattr(L, fn).restype = None
        _lib = L
    return _lib


def _p(a: np.ndarray):
    assert a.flags.c_contiguous
    return a.ctypes.data_as(ctypes.c_void_p)


def _f32(x) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(x), dtype=np.float32)


def ceil_to(v: int, m: int) -> int:
    return (v + m - 1) // m * m


def activation_codes(x, bits: int = 4, clip: float = 1.0):
    """core/quantization.py:13-21 -> (codes u8 [M,K], scale f32 [M], zero f32 [M])."""
    x = _f32(x)
    M, K = x.shape
    codes = np.empty((M, K), np.uint8)
    scales = np.empty(M, np.float32)
    zeros = np.empty(M, np.float32)
    lib().oracle_activation_codes(_p(x), M, K, float(np.float32(clip)), bits,
                                  _p(codes), _p(scales), _p(zeros))
    return codes, scales, zeros


def weight_codes(w, bits: int = 4, clip: float = 1.0):
    """core/quantization.py:7-11 -> (codes int8 [N,K], scale f32 [N])."""
    w = _f32(w)
    N, K = w.shape
    codes = np.empty((N, K), np.int8)
    scales = np.empty(N, np.float32)
    lib().oracle_weight_codes(_p(w), N, K, float(np.float32(clip)), bits,
                              _p(codes), _p(scales))
    return codes, scales


def fwht_rows(x, block: int = 128) -> np.ndarray:
    """Unnormalised Sylvester FWHT on each `block`-wide chunk of every row."""
    y = _f32(x).copy()
    M, K = y.shape
    lib().oracle_fwht_rows(_p(y), M, K, block)
    return y


def quantize_rows(x, clip: float = 1.0, rotate_block: int = 0,
                  want_codes: bool = False):
    """kernel/w4a4.cu:20-68 quantize (+ optional online rotation first).

    Returns (packed u8 [MP, KP/2], scales f32 [MP], zeros i32 [MP]
    [, codes u8 [MP, KP]]).
    """
    x = _f32(x)
    if rotate_block:
        x = fwht_rows(x, rotate_block)
    M, K = x.shape
    MP, KP = ceil_to(M, 8), ceil_to(K, 64)
    packed = np.empty((MP, KP // 2), np.uint8)
    scales = np.empty(MP, np.float32)
    zeros = np.empty(MP, np.int32)
    codes = np.empty((MP, KP), np.uint8) if want_codes else None
    lib().oracle_quantize_rows(_p(x), M, K, float(np.float32(clip)), _p(packed),
                               _p(scales), _p(zeros),
                               _p(codes) if want_codes else None)
    if want_codes:
        return packed, scales, zeros, codes
    return packed, scales, zeros


def pack_int4(codes) -> np.ndarray:
    """core/quantization.py:31-40 (range checks are the caller's)."""
    c = np.ascontiguousarray(codes, dtype=np.int8)
    R, C = c.shape
    out = np.empty((R, (C + 1) // 2), np.uint8)
    lib().oracle_pack_int4(_p(c), R, C, _p(out))
    return out


def unpack_int4(packed, width: int) -> np.ndarray:
    """core/quantization.py:42-45."""
    p = np.ascontiguousarray(packed, dtype=np.uint8)
    R, CB = p.shape
    out = np.empty((R, width), np.int8)
    lib().oracle_unpack_int4(_p(p), R, CB, width, _p(out))
    return out


def pack_weight(w, clip: float = 1.0, rotate_block: int = 0):
    """Weight glue for the GEMM: (packed u8 [NP,KP/2], sw f32 [NP], sums i32 [NP])."""
    w = _f32(w)
    N, K = w.shape
    NP, KP = ceil_to(N, 8), ceil_to(K, 64)
    scratch = np.empty((N, K), np.float32)
    cscratch = np.empty((N, K), np.int8)
    packed = np.empty((NP, KP // 2), np.uint8)
    sw = np.empty(NP, np.float32)
    sums = np.empty(NP, np.int32)
    lib().oracle_pack_weight(_p(w), N, K, float(np.float32(clip)), rotate_block,
                             _p(scratch), _p(cscratch), _p(packed), _p(sw),
                             _p(sums))
    return packed, sw, sums


def gemm_raw(a, b, M: int, N: int) -> np.ndarray:
    """kernel/w4a4.cu:80-154 raw int32 accumulators [M, N]."""
    a = np.ascontiguousarray(a, dtype=np.uint8)
    b = np.ascontiguousarray(b, dtype=np.uint8)
    KP = a.shape[1] * 2
    assert b.shape[1] * 2 == KP and a.shape[0] >= M and b.shape[0] >= N
    raw = np.empty((M, N), np.int32)
    rc = lib().oracle_gemm_raw(_p(a), _p(b), M, N, KP, _p(raw))
    if rc != 0:
        raise OverflowError("int32 accumulator overflow")
    return raw


def restore(raw, sx, zx, sw, sums, bias=None, out_dtype=np.float16):
    """kernel/w4a4.cu:70-78 epilogue; fp32 result narrowed RNE to out_dtype."""
    raw = np.ascontiguousarray(raw, dtype=np.int32)
    M, N = raw.shape
    sx, sw = _f32(sx), _f32(sw)
    zx = np.ascontiguousarray(zx, dtype=np.int32)
    sums = np.ascontiguousarray(sums, dtype=np.int32)
    b = None if bias is None or np.size(bias) == 0 else _f32(bias)
    out = np.empty((M, N), np.float32)
    lib().oracle_restore(_p(raw), _p(sx), _p(zx), _p(sw), _p(sums),
                         _p(b) if b is not None else None, M, N, _p(out))
    return out.astype(out_dtype)


def linear_w4a4(x, w, bias=None, clip_a: float = 1.0, clip_w: float = 1.0,
                rotate_block: int = 0, out_dtype=np.float16):
    """Whole W4A4 linear through the oracle: quantize -> gemm -> restore.

    Returns (out, raw, (packed_a, sx, zx), (packed_w, sw, sums)).
    """
    x = _f32(x)
    M = x.shape[0]
    N = np.shape(w)[0]
    pa, sx, zx = quantize_rows(x, clip_a, rotate_block)
    pw, sw, sums = pack_weight(w, clip_w, rotate_block)
    raw = gemm_raw(pa, pw, M, N)
    out = restore(raw, sx, zx, sw, sums, bias, out_dtype)
    return out, raw, (pa, sx, zx), (pw, sw, sums)


def gemm_raw_blas(a, b, M: int, N: int) -> np.ndarray:
    """Same result as gemm_raw for large shapes, via float64 BLAS on the
    unpacked codes.  Exact: every product is an integer with |p| <= 64 and
    every partial sum an integer below 64 * K < 2^53, so no rounding occurs
    in any summation order.  Pinned against gemm_raw in tests/test_oracle.py.
    """
    a = np.ascontiguousarray(a, dtype=np.uint8)
    b = np.ascontiguousarray(b, dtype=np.uint8)
    KP = a.shape[1] * 2
    ia = unpack_int4(a[:M], KP).astype(np.float64)
    ib = unpack_int4(b[:N], KP).astype(np.float64)
    r = ia @ ib.T
    if np.abs(r).max(initial=0) > 2**31 - 1:
        raise OverflowError("int32 accumulator overflow")
    return r.astype(np.int32)
