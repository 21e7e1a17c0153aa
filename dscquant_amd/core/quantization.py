"""Quantization primitives with the reference's names and signatures
(core/quantization.py:4-45), computed by the gfx950 kernels of libdscq.

``weight_codes`` / ``activation_codes`` return the same float-valued codes,
scales and zero-points as the reference (round half to even, IEEE fp32
division, the 1e-8 scale floor), bit for bit, for finite inputs on a CUDA
(HIP) device.  These are inference primitives: the codes carry no gradient
(the reference's straight-through estimator serves calibration, which stays
outside this path).  A CPU tensor raises -- there is no CPU fallback.
"""
from __future__ import annotations

import torch

from .. import _lib

__all__ = ["ste_round", "weight_codes", "activation_codes", "quantize_weight",
           "quantize_activation", "pack_int4", "unpack_int4"]

_MAX_ROWS = 65528  # rows per kernel call: a multiple of 8 below 65535


def ste_round(x):
    """core/quantization.py:4-5: round in the forward pass, identity gradient."""
    return x + (x.round() - x).detach()


def _as_kernel_input(t: torch.Tensor, what: str) -> torch.Tensor:
    if not t.is_cuda:
        raise RuntimeError(f"{what}: dscquant_amd runs on the GPU (HIP); got a "
                           f"{t.device.type} tensor")
    if t.dtype not in (torch.float16, torch.float32):
        t = t.float()  # bf16 / fp64 -> fp32; the reference widens with .float() too
    return t.contiguous()


def _dtype_code(t: torch.Tensor) -> int:
    return _lib.F16 if t.dtype == torch.float16 else _lib.F32


def _clip_value(clip) -> float:
    return float(clip.detach().float().item()) if torch.is_tensor(clip) else float(clip)


def weight_codes(weight, bits, clip=1.0):
    """core/quantization.py:7-11 -> (code f32 [N, K], scale f32 [N, 1])."""
    w = _as_kernel_input(weight, "weight_codes")
    if w.dim() != 2:
        raise ValueError("weight_codes expects a [out_features, in_features] matrix")
    bits, clip = int(bits), _clip_value(clip)
    N, K = w.shape
    NP, KP = (N + 7) // 8 * 8, (K + 63) // 64 * 64
    codes = torch.empty((NP, KP), dtype=torch.int8, device=w.device)
    scales = torch.empty((NP,), dtype=torch.float32, device=w.device)
    _lib.require_gfx950(w.device)
    with torch.cuda.device(w.device):
        _lib.call("dscq_weight_codes", w.data_ptr(), _dtype_code(w), N, K, clip, bits, 0,
                  codes.data_ptr(), scales.data_ptr(), _lib.stream(w.device))
    return codes[:N, :K].float(), scales[:N, None]


def activation_codes(x, bits, clip=1.0):
    """core/quantization.py:13-21 -> (code, scale, zero), codes in [0, 2^bits-1].

    Shapes follow the reference: code like x, scale / zero ``x.shape[:-1] + (1,)``,
    all float32.
    """
    xk = _as_kernel_input(x, "activation_codes")
    bits, clip = int(bits), _clip_value(clip)
    K = xk.shape[-1]
    rows = xk.reshape(-1, K)
    M = rows.shape[0]
    KP = (K + 63) // 64 * 64
    code = torch.empty((M, K), dtype=torch.float32, device=xk.device)
    scale = torch.empty((M,), dtype=torch.float32, device=xk.device)
    zero = torch.empty((M,), dtype=torch.float32, device=xk.device)
    _lib.require_gfx950(xk.device)
    with torch.cuda.device(xk.device):
        for r0 in range(0, M, _MAX_ROWS):
            part = rows[r0:r0 + _MAX_ROWS]
            m = part.shape[0]
            mp = (m + 7) // 8 * 8
            c = torch.empty((mp, KP), dtype=torch.uint8, device=xk.device)
            s = torch.empty((mp,), dtype=torch.float32, device=xk.device)
            z = torch.empty((mp,), dtype=torch.int32, device=xk.device)
            _lib.call("dscq_activation_codes", part.data_ptr(), _dtype_code(part), m, K, clip,
                      bits, 0, c.data_ptr(), s.data_ptr(), z.data_ptr(),
                      _lib.stream(xk.device))
            code[r0:r0 + m] = c[:m, :K]
            scale[r0:r0 + m] = s[:m]
            zero[r0:r0 + m] = z[:m]
    lead = x.shape[:-1]
    return code.reshape(*lead, K), scale.reshape(*lead, 1), zero.reshape(*lead, 1)


def quantize_weight(weight, bits, clip=1.0):
    """core/quantization.py:23-25: fake-quantized weight in its own dtype."""
    code, scale = weight_codes(weight, bits, clip)
    return (code * scale).to(weight.dtype)


def quantize_activation(x, bits, clip=1.0):
    """core/quantization.py:27-29: fake-quantized activation in its own dtype."""
    code, scale, zero = activation_codes(x, bits, clip)
    return ((code - zero) * scale).to(x.dtype)


def pack_int4(codes):
    """core/quantization.py:31-40: signed [-8, 7] codes -> u8 [R, ceil(C/2)]."""
    if codes.ndim != 2:
        raise ValueError('Packed weights must be a matrix.')
    c = codes.to(torch.int8)
    if bool(((c < -8) | (c > 7)).any()):
        raise ValueError('Signed INT4 code out of range.')
    if not c.is_cuda:
        raise RuntimeError("pack_int4: dscquant_amd runs on the GPU (HIP); got a "
                           f"{c.device.type} tensor")
    c = c.contiguous()
    R, C = c.shape
    out = torch.empty((R, (C + 1) // 2), dtype=torch.uint8, device=c.device)
    with torch.cuda.device(c.device):
        _lib.call("dscq_pack_int4", _lib.ptr(c), R, C, _lib.ptr(out), _lib.stream(c.device))
    return out


def unpack_int4(packed, width):
    """core/quantization.py:42-45: u8 [R, CB] -> signed int8 [R, width]."""
    if not packed.is_cuda:
        raise RuntimeError("unpack_int4: dscquant_amd runs on the GPU (HIP); got a "
                           f"{packed.device.type} tensor")
    p = packed.to(torch.uint8).contiguous()
    R, CB = p.shape
    width = int(width)
    width = min(width, 2 * CB)  # slicing semantics of the reference's [:, :width]
    out = torch.empty((R, width), dtype=torch.int8, device=p.device)
    with torch.cuda.device(p.device):
        _lib.call("dscq_unpack_int4", _lib.ptr(p), R, CB, width, _lib.ptr(out),
                  _lib.stream(p.device))
    return out
