"""torch-CPU restatement of the reference's fake-quant W4A4 forward.

TEST INFRASTRUCTURE / CPU BASELINE ONLY.  ``QuantLinear.forward`` with
``enabled=True`` (core/linear.py:48-52) quantizes the activation
(core/quantization.py:13-21, 27-29) and the weight (:7-11, 23-25) to integer
codes, dequantizes them back to the input dtype, and runs ``F.linear``.  The
weight is re-quantized on every call (linear.py:51-52).  This module restates
that composition in torch on the CPU so bench.py can time it beside the GPU
path, and so tests can check that the integer path lands within tolerance of
the fake-quant output.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F


def _round(x: torch.Tensor) -> torch.Tensor:
    # ste_round (core/quantization.py:4-5) forward value: x + (round(x) - x).
    return x + (x.round() - x)


def weight_codes(weight: torch.Tensor, bits: int, clip=1.0):
    """core/quantization.py:7-11."""
    bound = 2 ** (bits - 1) - 1
    scale = (weight.float().abs().amax(dim=1, keepdim=True) * clip / bound).clamp_min(1e-08)
    code = _round(weight.float() / scale).clamp(-bound, bound)
    return code, scale


def activation_codes(x: torch.Tensor, bits: int, clip=1.0):
    """core/quantization.py:13-21."""
    xf = x.float()
    lo = torch.minimum(xf.amin(dim=-1, keepdim=True), torch.zeros_like(xf[..., :1])) * clip
    hi = torch.maximum(xf.amax(dim=-1, keepdim=True), torch.zeros_like(xf[..., :1])) * clip
    maximum = 2 ** bits - 1
    scale = ((hi - lo) / maximum).clamp_min(1e-08)
    zero = _round(-lo / scale).clamp(0, maximum)
    code = _round(xf / scale + zero).clamp(0, maximum)
    return code, scale, zero


def quantize_weight(weight, bits, clip=1.0):
    """core/quantization.py:23-25."""
    code, scale = weight_codes(weight, bits, clip)
    return (code * scale).to(weight.dtype)


def quantize_activation(x, bits, clip=1.0):
    """core/quantization.py:27-29."""
    code, scale, zero = activation_codes(x, bits, clip)
    return ((code - zero) * scale).to(x.dtype)


def forward(x, weight, bias=None, bits=4, clip_a=1.0, clip_w=1.0, w_hat=None):
    """core/linear.py:48-52 with an optional pre-quantized weight.

    With ``w_hat=None`` the weight is fake-quantized on this call, as the
    reference does on every forward; passing ``w_hat`` times the
    "weights cached" variant.
    """
    if w_hat is None:
        w_hat = quantize_weight(weight, bits, clip_w)
    return F.linear(quantize_activation(x, bits, clip_a), w_hat, bias)
