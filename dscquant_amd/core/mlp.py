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
(silu_mul_quantize); both give the same h and the same packed h.  The
block computes h in fp16, so it takes fp16 inputs; fp32 and bf16 inputs run
the composition through the three modules (each on the integer path), as the
reference would.
"""
from __future__ import annotations

import torch
from torch import nn

from .. import w4a4
from .linear import QuantLinear, _stamp

_MAX_ROWS = 65528


class QuantMLP(nn.Module):
    """Fused W4A4 form of ``down(silu(gate(x)) * up(x))`` over three QuantLinear."""

    def __init__(self, gate: QuantLinear, up: QuantLinear, down: QuantLinear):
        super().__init__()
        self.gate, self.up, self.down = gate, up, down
        self._packed = None  # (key, pins, gate|up packed, sw, sums, bias, down packed, sw, sums)

    def _fusable(self, x) -> bool:
        """The fused block computes h in fp16 (an fp16 model's roundings), so it
        takes fp16 inputs only; other dtypes run the three modules in turn."""
        mods = (self.gate, self.up, self.down)
        return (x.dtype == torch.float16
                and all(m.enabled and m._is_w4a4() for m in mods)
                and self.gate.rotate_block == self.up.rotate_block
                and self.gate.clip_value("activation_clip")
                == self.up.clip_value("activation_clip")
                and self.gate.base.weight.shape[0] % 8 == 0)

    def packed(self):
        """(gate|up packed, sw, sums, gate|up bias or None, down packed, sw, sums).

        Built from the three modules' own packed weights and cached while those
        are the same objects (each module re-packs when its weight, fold, clip or
        rotation changes, and then hands out new tensors)."""
        parts = [m.packed_weight() for m in (self.gate, self.up, self.down)]
        biases = [m.packed_bias(torch.float16) for m in (self.gate, self.up)]
        items = [(f"w{i}.{j}", t) for i, p in enumerate(parts) for j, t in enumerate(p)]
        items += [(f"b{i}", b) for i, b in enumerate(biases)]
        key, pins = _stamp(items + [("gated", self._gated_gemm())])
        if self._packed is not None and self._packed[0] == key:
            return self._packed[2:]
        (pg, swg, sg), (pu, swu, su), (pd, swd, sd) = parts
        bg, bu = biases
        N = self.gate.base.weight.shape[0]
        bias = None
        if bg.numel() or bu.numel():
            zero = torch.zeros(N, dtype=torch.float16, device=pg.device)
            bias = (bg if bg.numel() else zero, bu if bu.numel() else zero)
        # gate and up rows interleaved in 64-row blocks for matmul_silu_mul,
        # else concatenated for the [M, 2N] GEMM + silu_mul_quantize
        join = w4a4.interleave_gate_up if self._gated_gemm() else (lambda a, b: torch.cat([a, b]))
        self._packed = (key, pins, join(pg, pu), join(swg, swu), join(sg, su),
                        None if bias is None else join(*bias), pd, swd, sd)
        return self._packed[2:]

    def _gated_gemm(self) -> bool:
        """Whether gate and up run as one GEMM with the SiLU-gated epilogue."""
        return self.gate.base.weight.shape[0] % 64 == 0

    def forward(self, x):
        if not self._fusable(x):
            from torch.nn import functional as F
            return self.down(F.silu(self.gate(x)) * self.up(x))
        if x.requires_grad and torch.is_grad_enabled():
            raise RuntimeError("the W4A4 HIP path is inference-only (codes carry no gradient)")
        pgu, swgu, sgu, bgu, pd, swd, sd = self.packed()
        N = self.gate.base.weight.shape[0]
        NO = self.down.base.weight.shape[0]
        K = x.shape[-1]
        lead = x.shape[:-1]
        xr = x.reshape(-1, K).contiguous()
        bdown = self.down.packed_bias(torch.float16)
        bgu = torch.empty(0, dtype=torch.float16, device=x.device) if bgu is None else bgu
        aclip = self.gate.clip_value("activation_clip")
        dclip = self.down.clip_value("activation_clip")
        rot_in, rot_down = int(self.gate.rotate_block), int(self.down.rotate_block)
        M = xr.shape[0]

        def block(part):
            m = part.shape[0]
            pa, sx, zx = w4a4.quantize(part, aclip, True, rot_in)
            if self._gated_gemm():
                h = w4a4.matmul_silu_mul(pa, pgu, sx, zx, swgu, sgu, bgu, m, N)
                ph, sh, zh = w4a4.quantize(h, dclip, True, rot_down)
            else:
                gu, _ = w4a4.matmul(pa, pgu, sx, zx, swgu, sgu, bgu, m, 2 * N, True, False, False)
                ph, sh, zh = w4a4.silu_mul_quantize(gu, dclip, rot_down)
            return w4a4.matmul(ph, pd, sh, zh, swd, sd, bdown, m, NO, True, False, False)[0]

        if 0 < M <= _MAX_ROWS:
            return block(xr).reshape(*lead, NO)
        out = torch.empty((M, NO), dtype=torch.float16, device=x.device)
        for r0 in range(0, M, _MAX_ROWS):
            out[r0:r0 + _MAX_ROWS] = block(xr[r0:r0 + _MAX_ROWS])
        return out.reshape(*lead, NO)
