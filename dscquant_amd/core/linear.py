"""QuantLinear with the reference's constructor, attributes and fold rules
(core/linear.py:8-52), running the W4A4 path on gfx950.

When ``enabled`` and the module is configured for 4-bit weights and 4-bit
activations, ``forward`` runs the integer path instead of the reference's
fake-quant composition:

    quantize(x [, online block-Hadamard])  -> packed int4 x, sx, zx   (HIP)
    matmul(packed x, packed W, ...)         -> out (fp16 / fp32)       (HIP)

The integer result equals the reference's F.linear(quantize_activation(x),
quantize_weight(W)) in exact arithmetic; the reference additionally rounds
x_hat and W_hat to the input dtype before its GEMM, so outputs agree within
the fp16 tolerance, while codes and int32 accumulators are bit-exact.

Derived state is cached on the module, never in its state_dict:

* the folded weight and bias (``transformed()``), recomputed when the base
  weight / bias or any tensor or scalar attribute of the interface changes;
* the packed weight (``pack_weight``: weight_codes at 4 bits, pack_int4, the
  per-channel scale and code sums), recomputed when the folded weight, the
  weight clip or ``rotate_block`` changes;
* the clip values as Python floats, so a steady-state forward issues no
  device-to-host read and can be captured in a HIP graph.

A change is seen through tensor identity, PyTorch's version counter, the
storage address, dtype and device: in-place updates under ``torch.no_grad()``,
``load_state_dict``, optimizer steps, assigning new tensors and the module
casts and moves (``.half()``, ``.to()``, ``.cuda()``) are all seen.  In-place
writes through ``.data`` are not; call ``invalidate_cache()`` after such a
write.

An empty batch (``x`` with no rows) returns an empty ``[..., 0, N]`` output in
``x``'s dtype without launching anything, as ``F.linear`` does.

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
_SCALARS = (int, float, bool, str, type(None))


def _stamp(objects):
    """(key, pins) for a sequence of (name, value) pairs.

    A tensor is keyed by identity, version counter, storage address, dtype and
    device (plain values, safe to compare with ==): ``Module.half()`` / ``.to()``
    / ``.cuda()`` swap a parameter's ``.data`` without changing its identity or
    version, but never its storage, dtype and device together.  ``pins`` keeps
    the tensors alive so that their ids cannot be reused by new tensors while
    the key is held."""
    key, pins = [], []
    for name, value in objects:
        if isinstance(value, torch.Tensor):
            key.append((name, id(value), value._version, value.data_ptr(), value.dtype,
                        value.device))
            pins.append(value)
        elif isinstance(value, _SCALARS):
            key.append((name, type(value).__name__, value))
        else:
            key.append((name, "obj", id(value)))
            pins.append(value)
    return tuple(key), tuple(pins)


def interface_state(interface):
    """Every tensor and scalar an interface's transform can depend on: its
    parameters and buffers (alpha, beta, the bases, core/transforms.py:9-14) and
    its public plain attributes (probe, override, heads, head_dim, ...)."""
    items = []
    if isinstance(interface, nn.Module):
        items += [("p." + n, t) for n, t in interface.named_parameters()]
        items += [("b." + n, t) for n, t in interface.named_buffers()]
    items += sorted((("a." + n, v) for n, v in vars(interface).items()
                     if not n.startswith("_") and not isinstance(v, nn.Module)
                     and (isinstance(v, torch.Tensor) or isinstance(v, _SCALARS))),
                    key=lambda kv: kv[0])
    return items


def _per_head_transpose_product(m, blocks):
    """m with the rows of head h (rows h*d .. h*d + d - 1) replaced by
    blocks[h]^T @ those rows, in fp32.  m: [H*d, C]; blocks: [H, d, d]."""
    H, d, _ = blocks.shape
    lhs = blocks.float().transpose(1, 2).contiguous()
    return torch.bmm(lhs, m.float().reshape(H, d, -1).contiguous()).reshape(m.shape)


def fold_interface(interface, role, repeat, weight, bias):
    """The equivalence transform of ``interface`` folded into one projection
    (core/linear.py:22-46), in fp32, cast back to the tensors' dtypes.

    Rotation (per-head orthogonal R_h, core/transforms.py:51-52): the v
    projection's output channels of head h become R_h^T W_h (bias likewise);
    the o projection's input channels of query head j become W_j R_(j // repeat),
    which is the same per-head product applied to W^T, since
    (W R)^T = R^T W^T.  Other roles are unchanged.
    Scaling (diagonal s, core/transforms.py:71-72): the up projection's rows
    are divided by s (bias likewise); any other role has its columns
    multiplied by s.
    """
    if callable(getattr(interface, "matrices", None)):
        R = interface.matrices()
        if role == "v":
            w = _per_head_transpose_product(weight, R).to(weight.dtype)
            b = None if bias is None else \
                _per_head_transpose_product(bias.reshape(-1, 1), R).reshape(-1).to(bias.dtype)
            return w, b
        if role == "o":
            Rq = R.repeat_interleave(repeat, dim=0)
            w = _per_head_transpose_product(weight.t(), Rq).t().contiguous().to(weight.dtype)
            return w, bias
        return weight, bias
    s = interface.diagonal().float()
    if role == "up":
        w = (weight.float() / s.unsqueeze(1)).to(weight.dtype)
        b = None if bias is None else (bias.float() / s).to(bias.dtype)
        return w, b
    return (weight.float() * s.unsqueeze(0)).to(weight.dtype), bias


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
        for param in self.base.parameters():
            param.requires_grad_(False)
        self.invalidate_cache()

    # ---------------------------------------------------------------- caches
    def invalidate_cache(self) -> None:
        """Drops the folded weight, the packed weight and the clip values, so the
        next forward recomputes them (needed after writes through ``.data``)."""
        self._fold = None     # (key, pins, weight, bias)
        self._pack = None     # (key, pins, (packed, sw, sums))
        self._biases = {}     # dtype -> (key, pins, bias in that dtype)
        self._clips = {}      # name -> (parameter, stamp, float)
        self._fold_gen = getattr(self, "_fold_gen", 0) + 1

    def clip_value(self, name: str) -> float:
        """``weight_clip`` / ``activation_clip`` as a float, read from the device
        only when the parameter changed."""
        p = getattr(self, name)
        stamp = (p._version, p.data_ptr(), p.dtype, p.device)
        hit = self._clips.get(name)
        if hit is not None and hit[0] is p and hit[1] == stamp:
            return hit[2]
        value = float(p.detach().float().item())
        self._clips[name] = (p, stamp, value)
        return value

    def _fold_key(self, interface):
        items = [("weight", self.base.weight), ("bias", self.base.bias),
                 ("role", self.role), ("repeat", self.repeat), ("interface", id(interface))]
        return _stamp(items + interface_state(interface))

    # core/linear.py:22-46
    def transformed(self):
        """(weight, bias) with the interface's transform folded in.

        Without an interface: the base tensors.  The fold is cached while the
        base tensors and the interface's state are unchanged; when autograd
        would record it (grad enabled and an interface tensor requiring grad,
        as during calibration) it is computed afresh, graph attached."""
        interface = self._interface() if self._interface else None
        if interface is None:
            return (self.base.weight, self.base.bias)
        key, pins = self._fold_key(interface)
        tracked = torch.is_grad_enabled() and any(
            isinstance(t, torch.Tensor) and t.requires_grad for t in pins)
        if tracked:
            return fold_interface(interface, self.role, self.repeat,
                                  self.base.weight, self.base.bias)
        if self._fold is None or self._fold[0] != key:
            weight, bias = fold_interface(interface, self.role, self.repeat,
                                          self.base.weight, self.base.bias)
            self._fold = (key, pins, weight, bias)
            self._fold_gen += 1
        return self._fold[2], self._fold[3]

    # ---------------------------------------------------------------- int path
    def _is_w4a4(self) -> bool:
        return (getattr(self.config, "weight_bits", None) == 4
                and getattr(self.config, "activation_bits", None) == 4)

    def _folded(self):
        with torch.no_grad():
            return self.transformed()

    def _source_stamp(self, tensor, name):
        # A folded tensor is a cache entry: its generation names it.  A base
        # tensor is named by identity and version.
        interface = self._interface() if self._interface else None
        return (name + "@fold", self._fold_gen) if interface is not None else (name, tensor)

    def packed_weight(self):
        """(packed u8 [NP, KP/2], sw f32 [NP], sums i32 [NP]) for the current weight."""
        weight, _ = self._folded()
        wclip = self.clip_value("weight_clip")
        key, pins = _stamp([self._source_stamp(weight, "weight"), ("clip", wclip),
                            ("rotate", int(self.rotate_block))])
        if self._pack is None or self._pack[0] != key:
            w = weight.detach()
            if w.dtype not in (torch.float16, torch.float32):
                w = w.float()
            packed = tuple(w4a4.pack_weight(w.contiguous(), wclip, int(self.rotate_block)))
            self._pack = (key, pins, packed)
        return self._pack[2]

    def packed_bias(self, dtype):
        """The folded bias in the output dtype (an empty tensor when there is none)."""
        _, bias = self._folded()
        key, pins = _stamp([self._source_stamp(bias, "bias"), ("dtype", str(dtype))])
        hit = self._biases.get(dtype)
        if hit is None or hit[0] != key:
            b = (torch.empty(0, dtype=dtype, device=self.base.weight.device) if bias is None
                 else bias.detach().to(dtype).contiguous())
            hit = self._biases[dtype] = (key, pins, b)
        return hit[2]

    def _forward_w4a4(self, x):
        if x.requires_grad and torch.is_grad_enabled():
            raise RuntimeError("the W4A4 HIP path is inference-only (codes carry no gradient)")
        N, KW = self.base.weight.shape
        K = x.shape[-1]
        lead = x.shape[:-1]
        if K != KW:
            # F.linear's own check (core/linear.py:52); packing pads K to 64, so the
            # kernels alone would not see a mismatch inside one padding step.
            raise RuntimeError(f"mat1 and mat2 shapes cannot be multiplied "
                               f"({x.numel() // max(K, 1)}x{K} and {KW}x{N})")
        if x.numel() == 0:
            # An empty batch: F.linear returns [..., 0, N] in x's dtype
            # (core/linear.py:48-52); nothing is launched.
            return torch.empty((*lead, N), dtype=x.dtype, device=x.device)
        packed_w, sw, sums = self.packed_weight()
        xr = x.reshape(-1, K)
        if xr.dtype not in (torch.float16, torch.float32):
            xr = xr.float()
        xr = xr.contiguous()
        fp32 = xr.dtype != torch.float16
        out_dtype = torch.float32 if fp32 else torch.float16
        b = self.packed_bias(out_dtype)
        aclip = self.clip_value("activation_clip")
        rot = int(self.rotate_block)
        M = xr.shape[0]
        if (M > 0 and xr.data_ptr() % 16 == 0
                and w4a4.linear_decode_supported(M, K)):
            # A few tokens: quantize and multiply in one launch (bit-identical).
            out = w4a4.linear_decode(xr, aclip, rot, packed_w, sw, sums, b, N, fp32)
            return out.reshape(*lead, N).to(x.dtype)
        if M <= _MAX_ROWS:
            pa, sx, zx = w4a4.quantize(xr, aclip, True, rot)
            out, _ = w4a4.matmul(pa, packed_w, sx, zx, sw, sums, b, M, N, True, False, fp32)
            return out.reshape(*lead, N).to(x.dtype)
        out = torch.empty((M, N), dtype=out_dtype, device=x.device)
        for r0 in range(0, M, _MAX_ROWS):
            part = xr[r0:r0 + _MAX_ROWS]
            m = part.shape[0]
            pa, sx, zx = w4a4.quantize(part, aclip, True, rot)
            out[r0:r0 + m], _ = w4a4.matmul(pa, packed_w, sx, zx, sw, sums, b, m, N, True,
                                            False, fp32)
        return out.reshape(*lead, N).to(x.dtype)

    # core/linear.py:48-52
    def forward(self, x):
        if not self.enabled:
            return self.base(x)
        if self._is_w4a4():
            return self._forward_w4a4(x)
        if self.rotate_block:
            raise RuntimeError("rotate_block applies to the W4A4 integer path only")
        if x.requires_grad and torch.is_grad_enabled():
            raise RuntimeError("the GPU quantization codes carry no gradient: run the "
                               "quantized forward under torch.no_grad()")
        weight, bias = self.transformed()
        xq = quantize_activation(x, self.config.activation_bits, self.activation_clip)
        wq = quantize_weight(weight, self.config.weight_bits, self.weight_clip)
        return F.linear(xq, wq, bias)
