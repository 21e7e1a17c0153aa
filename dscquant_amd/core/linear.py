"""QuantLinear with the reference's constructor, attributes and fold rules
(core/linear.py:8-52), running the W4A4 path on gfx950.

When ``enabled`` and the module is configured for 4-bit weights and 4-bit
activations, ``forward`` runs the integer path instead of the reference's
fake-quant composition:

    quantize(x [, online block-Hadamard])  -> packed int4 x, sx, zx   (HIP)
    matmul(packed x, packed W, ...)         -> out (fp16 / fp32)       (HIP)

The packed weight (``pack_weight``: weight_codes at 4 bits, pack_int4, the
per-channel scale and code sums) is cached on the module (non-persistent,
so state_dict keys are unchanged) and rebuilt when the weight, the clip or
the rotation changes.  The integer result equals the reference's
F.linear(quantize_activation(x), quantize_weight(W)) in exact arithmetic; the
reference additionally rounds x_hat and W_hat to the input dtype before its
GEMM, so outputs agree within the fp16 tolerance, while codes and int32
accumulators are bit-exact.

Other bit widths run the reference composition with GPU-computed codes.
``rotate_block`` (default 0) is an attribute like ``enabled``: set it to 128
to rotate activations online with H_128 and fold W H_128 / 128 into the
packed weight (the computational-invariance rule of core/linear.py:34-37).
"""
from __future__ import annotations

import weakref

import torch
import torch.nn.functional as F
from torch import nn

from .. import w4a4
from .quantization import quantize_activation, quantize_weight

_MAX_ROWS = 65528


class QuantLinear(nn.Module):

    def __init__(self, base, config, interface=None, role=None, repeat=1):
        super().__init__()
        self.base = base
        self.config = config
        self.role, self.repeat = (role, repeat)
        self._interface = None if interface is None else weakref.ref(interface)
        self.weight_clip = nn.Parameter(torch.tensor(1.0, device=base.weight.device),
                                        requires_grad=False)
        self.activation_clip = nn.Parameter(torch.tensor(1.0, device=base.weight.device),
                                            requires_grad=False)
        self.enabled = False
        self.rotate_block = 0
        self._packed = None  # (key, packed, sw, sums): a cache, not module state
        for param in self.base.parameters():
            param.requires_grad_(False)

    # core/linear.py:22-46
    def transformed(self):
        weight, bias = (self.base.weight, self.base.bias)
        interface = self._interface() if self._interface else None
        if interface is None:
            return (weight, bias)
        if hasattr(interface, "matrices") and hasattr(interface, "head_dim"):
            # Rotation (core/transforms.py:33-52): per-head orthogonal R.
            matrices = interface.matrices()
            if self.role == 'v':
                shaped = weight.float().reshape(interface.heads, interface.head_dim, -1)
                weight = (matrices.transpose(-1, -2) @ shaped).reshape_as(weight).to(weight.dtype)
                if bias is not None:
                    bias = (matrices.transpose(-1, -2)
                            @ bias.float().reshape(interface.heads, -1, 1)).flatten().to(bias.dtype)
            elif self.role == 'o':
                matrices = matrices.repeat_interleave(self.repeat, dim=0)
                shaped = weight.float().reshape(weight.shape[0], len(matrices), interface.head_dim)
                weight = torch.matmul(shaped.transpose(0, 1), matrices.contiguous()) \
                    .transpose(0, 1).reshape_as(weight).to(weight.dtype)
        else:
            # Scaling (core/transforms.py:66-72): diagonal exp(log-scale).
            scale = interface.diagonal()
            if self.role == 'up':
                weight = (weight.float() / scale[:, None]).to(weight.dtype)
                if bias is not None:
                    bias = (bias.float() / scale).to(bias.dtype)
            else:
                weight = (weight.float() * scale[None, :]).to(weight.dtype)
        return (weight, bias)

    # ---------------------------------------------------------------- int path
    def _is_w4a4(self) -> bool:
        return (getattr(self.config, "weight_bits", None) == 4
                and getattr(self.config, "activation_bits", None) == 4)

    def packed_weight(self):
        """(packed u8 [NP, KP/2], sw f32 [NP], sums i32 [NP]) for the current weight."""
        weight, _ = self.transformed()
        wclip = float(self.weight_clip.detach().float().item())
        interface = self._interface() if self._interface else None
        key = (weight.data_ptr(), weight._version, tuple(weight.shape), wclip,
               int(self.rotate_block))
        if interface is None and self._packed is not None and self._packed[0] == key:
            return self._packed[1:]
        w = weight.detach()
        if w.dtype not in (torch.float16, torch.float32):
            w = w.float()
        packed, sw, sums = w4a4.pack_weight(w.contiguous(), wclip, int(self.rotate_block))
        if interface is None:
            self._packed = (key, packed, sw, sums)
        return packed, sw, sums

    def _forward_w4a4(self, x):
        if x.requires_grad and torch.is_grad_enabled():
            raise RuntimeError("the W4A4 HIP path is inference-only (codes carry no gradient)")
        packed_w, sw, sums = self.packed_weight()
        _, bias = self.transformed()
        N = self.base.weight.shape[0]
        K = x.shape[-1]
        lead = x.shape[:-1]
        xr = x.reshape(-1, K)
        if xr.dtype not in (torch.float16, torch.float32):
            xr = xr.float()
        xr = xr.contiguous()
        fp32 = xr.dtype != torch.float16
        out_dtype = torch.float32 if fp32 else torch.float16
        b = (torch.empty(0, dtype=out_dtype, device=x.device) if bias is None
             else bias.detach().to(out_dtype).contiguous())
        aclip = float(self.activation_clip.detach().float().item())
        M = xr.shape[0]
        if (M > 0 and xr.data_ptr() % 16 == 0
                and w4a4.linear_decode_supported(M, K)):
            # A few tokens: quantize and multiply in one launch (bit-identical).
            out = w4a4.linear_decode(xr, aclip, int(self.rotate_block), packed_w, sw, sums, b,
                                     N, fp32)
            return out.reshape(*lead, N).to(x.dtype)
        out = torch.empty((M, N), dtype=out_dtype, device=x.device)
        for r0 in range(0, max(M, 1), _MAX_ROWS):
            part = xr[r0:r0 + _MAX_ROWS]
            m = part.shape[0]
            if m == 0:
                break
            pa, sx, zx = w4a4.quantize(part, aclip, True, int(self.rotate_block))
            o, _ = w4a4.matmul(pa, packed_w, sx, zx, sw, sums, b, m, N, True, False, fp32)
            if M <= _MAX_ROWS:
                out = o
            else:
                out[r0:r0 + m] = o
        return out.reshape(*lead, N).to(x.dtype)

    # core/linear.py:48-52
    def forward(self, x):
        if not self.enabled:
            return self.base(x)
        if self._is_w4a4():
            return self._forward_w4a4(x)
        if self.rotate_block:
            raise RuntimeError("rotate_block applies to the W4A4 integer path only")
        weight, bias = self.transformed()
        return F.linear(quantize_activation(x, self.config.activation_bits, self.activation_clip),
                        quantize_weight(weight, self.config.weight_bits, self.weight_clip), bias)
