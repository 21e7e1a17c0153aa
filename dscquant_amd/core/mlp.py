"""SiLU-gated MLP block on the W4A4 path: down(act_fn(gate(x)) * up(x)).

The reference quantizes each projection of a Llama MLP through its own
QuantLinear (core/linear.py:48-52; core/model_ops.py drives the model) and
runs the activation in between unquantized in torch.  ``QuantMLP`` keeps the
three QuantLinear modules (their weights, clips, folds and rotations) and
runs the block in four launches:

    quantize(x)                                  -> packed x        (HIP)
    matmul_silu_mul(packed x, gate/up weights)   -> h [M, N]        (HIP)
    quantize(h)                                  -> packed h        (HIP)
    matmul(packed h, down weights)               -> out             (HIP)

gate and up read the same quantized x, so they run as one GEMM against the
packed weights interleaved in 64-row blocks, whose epilogue computes
h = fp16(fp16(silu(g)) * u) (an fp16 model's roundings) from the two halves
of each output tile.  When N is not a multiple of 64 the gate|up GEMM writes
[M, 2N] against the row-concatenated weights instead, and one kernel applies
the SiLU, the product and the down projection's input quantization
(silu_mul_quantize); both give the same h and the same packed h.
"""
from __future__ import annotations

import torch
from torch import nn

from .. import w4a4
from .linear import QuantLinear

_MAX_ROWS = 65528


def _clip(p) -> float:
    return float(p.detach().float().item())


class QuantMLP(nn.Module):
    """Fused W4A4 form of ``down(silu(gate(x)) * up(x))`` over three QuantLinear."""

    def __init__(self, gate: QuantLinear, up: QuantLinear, down: QuantLinear):
        super().__init__()
        self.gate, self.up, self.down = gate, up, down
        self._packed = None  # (key, gate|up packed, sw, sums, bias, down packed, sw, sums)

    def _fusable(self) -> bool:
        mods = (self.gate, self.up, self.down)
        return (all(m.enabled and m._is_w4a4() for m in mods)
                and self.gate.rotate_block == self.up.rotate_block
                and _clip(self.gate.activation_clip) == _clip(self.up.activation_clip)
                and self.gate.base.weight.shape[0] % 8 == 0)

    def packed(self):
        """(gate|up packed, sw, sums, gate|up bias or None, down packed, sw, sums)."""
        key = []
        for m in (self.gate, self.up, self.down):
            w, _ = m.transformed()
            key.append((w.data_ptr(), w._version, _clip(m.weight_clip), int(m.rotate_block)))
        key = tuple(key)
        if self._packed is not None and self._packed[0] == key:
            return self._packed[1:]
        pg, swg, sg = self.gate.packed_weight()
        pu, swu, su = self.up.packed_weight()
        _, bg = self.gate.transformed()
        _, bu = self.up.transformed()
        N = self.gate.base.weight.shape[0]
        bias = None
        if bg is not None or bu is not None:
            zero = torch.zeros(N, dtype=torch.float16, device=pg.device)
            bias = (zero if bg is None else bg.detach().half(),
                    zero if bu is None else bu.detach().half())
        # gate and up rows interleaved in 64-row blocks for matmul_silu_mul,
        # else concatenated for the [M, 2N] GEMM + silu_mul_quantize
        join = w4a4.interleave_gate_up if self._gated_gemm() else (lambda a, b: torch.cat([a, b]))
        pd, swd, sd = self.down.packed_weight()
        self._packed = (key, join(pg, pu), join(swg, swu), join(sg, su),
                        None if bias is None else join(*bias), pd, swd, sd)
        return self._packed[1:]

    def _gated_gemm(self) -> bool:
        """Whether gate and up run as one GEMM with the SiLU-gated epilogue."""
        return self.gate.base.weight.shape[0] % 64 == 0

    def forward(self, x):
        if not self._fusable():
            from torch.nn import functional as F
            return self.down(F.silu(self.gate(x)) * self.up(x))
        if x.requires_grad and torch.is_grad_enabled():
            raise RuntimeError("the W4A4 HIP path is inference-only (codes carry no gradient)")
        pgu, swgu, sgu, bgu, pd, swd, sd = self.packed()
        N = self.gate.base.weight.shape[0]
        NO = self.down.base.weight.shape[0]
        K = x.shape[-1]
        lead = x.shape[:-1]
        xr = x.reshape(-1, K)
        if xr.dtype not in (torch.float16, torch.float32):
            xr = xr.float()
        xr = xr.contiguous()
        fp32 = xr.dtype != torch.float16
        out_dtype = torch.float32 if fp32 else torch.float16
        _, bd = self.down.transformed()
        bdown = (torch.empty(0, dtype=out_dtype, device=x.device) if bd is None
                 else bd.detach().to(out_dtype).contiguous())
        bgu = torch.empty(0, dtype=torch.float16, device=x.device) if bgu is None else bgu
        aclip, dclip = _clip(self.gate.activation_clip), _clip(self.down.activation_clip)
        rot_in, rot_down = int(self.gate.rotate_block), int(self.down.rotate_block)
        M = xr.shape[0]
        out = torch.empty((M, NO), dtype=out_dtype, device=x.device)
        for r0 in range(0, max(M, 1), _MAX_ROWS):
            part = xr[r0:r0 + _MAX_ROWS]
            m = part.shape[0]
            if m == 0:
                break
            pa, sx, zx = w4a4.quantize(part, aclip, True, rot_in)
            if self._gated_gemm():
                h = w4a4.matmul_silu_mul(pa, pgu, sx, zx, swgu, sgu, bgu, m, N)
                ph, sh, zh = w4a4.quantize(h, dclip, True, rot_down)
            else:
                gu, _ = w4a4.matmul(pa, pgu, sx, zx, swgu, sgu, bgu, m, 2 * N, True, False, False)
                ph, sh, zh = w4a4.silu_mul_quantize(gu, dclip, rot_down)
            o, _ = w4a4.matmul(ph, pd, sh, zh, swd, sd, bdown, m, NO, True, False, fp32)
            out[r0:r0 + m] = o
        return out.reshape(*lead, NO).to(x.dtype)
