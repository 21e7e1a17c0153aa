"""Vectorised numpy restatement of the W4A4 rules (test infrastructure only).

Written independently of dscq_oracle.c so the two cross-check each other.
numpy float32 arithmetic is IEEE (correctly rounded, no contraction) and
``np.rint`` rounds half to even, matching torch.round / __float2int_rn.
"""
from __future__ import annotations

import numpy as np

F32 = np.float32


def activation_codes(x, bits: int = 4, clip: float = 1.0):
    """core/quantization.py:13-21."""
    xf = np.asarray(x, dtype=F32)
    qmax = F32(2 ** bits - 1)
    clip = F32(clip)
    lo = np.minimum(xf.min(axis=-1, keepdims=True), F32(0)) * clip
    hi = np.maximum(xf.max(axis=-1, keepdims=True), F32(0)) * clip
    scale = np.maximum((hi - lo) / qmax, F32(1e-8))
    zero = np.clip(np.rint(-lo / scale), F32(0), qmax)
    code = np.clip(np.rint(xf / scale + zero), F32(0), qmax)
    return code.astype(np.uint8), scale[..., 0], zero[..., 0]


def weight_codes(w, bits: int = 4, clip: float = 1.0):
    """core/quantization.py:7-11."""
    wf = np.asarray(w, dtype=F32)
    bound = F32(2 ** (bits - 1) - 1)
    scale = np.maximum(np.abs(wf).max(axis=1, keepdims=True) * F32(clip) / bound,
                       F32(1e-8))
    code = np.clip(np.rint(wf / scale), -bound, bound)
    return code.astype(np.int8), scale[:, 0]


def pack_int4(codes) -> np.ndarray:
    """core/quantization.py:31-40."""
    c = np.asarray(codes).astype(np.int16)
    if c.shape[1] % 2:
        c = np.pad(c, ((0, 0), (0, 1)))
    u = c & 15
    return (u[:, ::2] | (u[:, 1::2] << 4)).astype(np.uint8)


def unpack_int4(packed, width: int) -> np.ndarray:
    """core/quantization.py:42-45."""
    p = np.asarray(packed, dtype=np.uint8)
    code = np.stack((p & 15, p >> 4), axis=-1).reshape(p.shape[0], -1).astype(np.int16)
    signed = np.where(code >= 8, code - 16, code)
    return signed[:, :width].astype(np.int8)


def fwht_rows(x, block: int = 128) -> np.ndarray:
    """Unnormalised Sylvester FWHT per block, bit 0 first (same order as the C)."""
    y = np.array(x, dtype=F32, copy=True)
    M, K = y.shape
    v = y.reshape(M, K // block, block)
    h = 1
    while h < block:
        v = v.reshape(M, K // block, block // (2 * h), 2, h)
        u, w = v[:, :, :, 0, :].copy(), v[:, :, :, 1, :].copy()
        v[:, :, :, 0, :] = u + w
        v[:, :, :, 1, :] = u - w
        v = v.reshape(M, K // block, block)
        h *= 2
    return v.reshape(M, K)


def sylvester(n: int) -> np.ndarray:
    """Dense Sylvester Hadamard matrix of order n (power of two), float64."""
    H = np.ones((1, 1))
    while H.shape[0] < n:
        H = np.block([[H, H], [H, -H]])
    return H
