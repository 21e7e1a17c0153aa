"""The W4A4 extension API, MI355X edition.

Drop-in for the reference's compiled extension (kernel/w4a4.cu:227-230),
which exports

    quantize(x, clip, fused) -> [packed, scales, zeros]
    matmul(a, b, sx, zx, sw, sums, bias, M, N, fused, force_decode, fp32)
        -> [out, raw]

with the same argument meaning, padded layouts, dtypes and RuntimeError
messages (kernel/w4a4.cu:12-17, 164-225).  Outputs are allocated by torch's
caching allocator on the input's device; kernels run asynchronously on the
current stream.  Two additions that the reference leaves to the caller:

    quantize(..., rotate_block=128)   online block-Hadamard before quantizing
    pack_weight(w, clip, rotate_block) -> [packed, sw, sums]   the weight glue

Every argument check runs on the host before any GPU call, so tests can
exercise all of them without a GPU (``check_quantize_args`` /
``check_matmul_args``).
"""
from __future__ import annotations

import torch

from . import _lib

__all__ = ["quantize", "matmul", "pack_weight", "silu_mul_quantize", "linear_decode",
           "linear_decode_supported", "matmul_silu_mul", "interleave_gate_up", "padded",
           "check_quantize_args", "check_matmul_args", "workspace_bytes"]


def padded(v: int, m: int) -> int:
    return (v + m - 1) // m * m


def _check_cuda(t: torch.Tensor) -> None:
    # kernel/w4a4.cu:12-14
    if not (t.is_cuda and t.is_contiguous()):
        raise RuntimeError("Expected contiguous CUDA tensor")


def _check_float(t: torch.Tensor) -> None:
    # kernel/w4a4.cu:15-18
    if t.dtype not in (torch.float16, torch.float32):
        raise RuntimeError("Only FP16 and FP32 inputs are supported")


def check_quantize_args(x: torch.Tensor, clip: float, rotate_block: int = 0,
                        require_cuda: bool = True) -> None:
    """kernel/w4a4.cu:165-168 (+ the rotation's divisibility rule)."""
    if require_cuda:
        _check_cuda(x)
    _check_float(x)
    if not (x.dim() == 2 and 0 < x.size(0) <= 65535 and 0 < x.size(1) <= 1048576):
        raise RuntimeError("Require 1<=M<=65535 and 1<=K<=1048576")
    if not (0.5 <= clip <= 1.0):
        raise RuntimeError("Activation clip must be in [0.5,1]")
    if rotate_block not in (0, 128):
        raise RuntimeError(f"rotate_block must be 0 or 128 (got {rotate_block})")
    if rotate_block and x.size(1) % rotate_block:
        raise RuntimeError(
            f"Rotation needs K to be a multiple of {rotate_block} (got K={x.size(1)})")


def quantize(x: torch.Tensor, clip: float = 1.0, fused: bool = True,
             rotate_block: int = 0):
    """Per-token int4 quantization + packing (kernel/w4a4.cu:164-187).

    Returns [packed u8 [MP, KP/2], scales f32 [MP], zeros i32 [MP]] with
    MP = ceil8(M), KP = ceil64(K).  ``fused=False`` runs the reference's
    two-pass form (codes kernel, then pack kernel); results are identical.
    """
    clip = float(clip)
    check_quantize_args(x, clip, rotate_block)
    dev = x.device
    _lib.require_gfx950(dev)
    M, K = x.shape
    MP, KP = padded(M, 8), padded(K, 64)
    packed = torch.empty((MP, KP // 2), dtype=torch.uint8, device=dev)
    scales = torch.empty((MP,), dtype=torch.float32, device=dev)
    zeros = torch.empty((MP,), dtype=torch.int32, device=dev)
    codes = None if fused else torch.empty((MP, KP), dtype=torch.uint8, device=dev)
    with torch.cuda.device(dev):
        _lib.call("dscq_quantize", x.data_ptr(),
                  _lib.F16 if x.dtype == torch.float16 else _lib.F32, M, K, clip,
                  1 if fused else 0, rotate_block, packed.data_ptr(),
                  scales.data_ptr(), zeros.data_ptr(), _lib.ptr(codes), _lib.stream(dev))
    return [packed, scales, zeros]


def check_matmul_args(a, b, sx, zx, sw, sums, bias, M: int, N: int, fp32: bool,
                      require_cuda: bool = True) -> int:
    """kernel/w4a4.cu:192-202; returns KP."""
    for t in (a, b, sx, zx, sw, sums, bias):
        if require_cuda:
            _check_cuda(t)
        if t.device != a.device:
            raise RuntimeError("All buffers must be on the same device")
    if not (a.dim() == 2 and b.dim() == 2 and a.dtype == torch.uint8 and b.dtype == torch.uint8):
        raise RuntimeError("Packed operands must be byte matrices")
    KP = a.size(1) * 2
    MP, NP = padded(M, 8), padded(N, 8)
    if not (0 < M <= 65535 and N > 0 and 0 < KP <= 1048576 and KP % 64 == 0):
        raise RuntimeError("Invalid dimensions")
    if not (a.size(0) >= MP and b.size(0) >= NP and b.size(1) == a.size(1)):
        raise RuntimeError("Invalid padded operand shapes")
    if not (sx.dtype == torch.float32 and sw.dtype == torch.float32
            and zx.dtype == torch.int32 and sums.dtype == torch.int32):
        raise RuntimeError("Invalid metadata dtypes")
    if not (sx.numel() >= MP and zx.numel() >= MP and sw.numel() >= NP and sums.numel() >= NP):
        raise RuntimeError("Metadata too short")
    dtype = torch.float32 if fp32 else torch.float16
    if not (bias.dtype == dtype and (bias.numel() == 0 or bias.numel() == N)):
        raise RuntimeError("Bias shape/dtype mismatch")
    return KP


def matmul(a, b, sx, zx, sw, sums, bias, M: int, N: int, fused: bool = True,
           force_decode: bool = False, fp32: bool = False):
    """Packed W4A4 GEMM + dequant epilogue (kernel/w4a4.cu:189-225).

    Returns [out [M, N] fp16 (fp32 if ``fp32``), raw i32 [M, N] (or [0] when
    ``fused``)].  ``bias`` is an empty tensor or [N] of the output dtype.
    """
    M, N = int(M), int(N)
    KP = check_matmul_args(a, b, sx, zx, sw, sums, bias, M, N, fp32)
    dev = a.device
    _lib.require_gfx950(dev)
    out = torch.empty((M, N), dtype=torch.float32 if fp32 else torch.float16, device=dev)
    raw = torch.empty((0,) if fused else (M, N), dtype=torch.int32, device=dev)
    with torch.cuda.device(dev):
        # Shapes whose K loop the library splits over workgroups take a scratch
        # workspace, allocated here like the outputs (dscq_matmul_ws); the size
        # depends on the device's compute units, so it is asked on that device.
        ws_bytes = workspace_bytes(M, N, KP, force_decode)
        ws = torch.empty((ws_bytes,), dtype=torch.uint8, device=dev) if ws_bytes else None
        _lib.call("dscq_matmul_ws", a.data_ptr(), b.data_ptr(), sx.data_ptr(), zx.data_ptr(),
                  sw.data_ptr(), sums.data_ptr(), _lib.ptr(bias), M, N, KP,
                  1 if fused else 0, 1 if force_decode else 0, 1 if fp32 else 0,
                  out.data_ptr(), _lib.ptr(raw), _lib.ptr(ws), ws_bytes, _lib.stream(dev))
    return [out, raw]


def workspace_bytes(M: int, N: int, KP: int, force_decode: bool = False) -> int:
    """Scratch bytes ``matmul`` passes to dscq_matmul_ws for this shape (0: none)."""
    n = int(_lib.lib().dscq_matmul_workspace_bytes(int(M), int(N), int(KP),
                                                   1 if force_decode else 0))
    if n < 0:
        raise RuntimeError(_lib.lib().dscq_last_error().decode())
    return n


def linear_decode_supported(M: int, K: int) -> bool:
    """Whether ``linear_decode`` takes an [M, K] input (a few tokens; see include/dscq.h)."""
    return bool(_lib.lib().dscq_linear_decode_supported(int(M), int(K)))


def linear_decode(x: torch.Tensor, clip: float, rotate_block: int, b, sw, sums, bias,
                  N: int, fp32: bool = False) -> torch.Tensor:
    """quantize(x, clip, True, rotate_block) followed by matmul(..., fused=True) in one
    launch, for few tokens; bit-identical to the two calls.  ``b``, ``sw``, ``sums``,
    ``bias`` as for ``matmul``.  Returns out [M, N] fp16 (fp32 if ``fp32``)."""
    clip = float(clip)
    check_quantize_args(x, clip, rotate_block)
    M, K = x.shape
    N = int(N)
    KP = padded(K, 64)
    for t in (b, sw, sums, bias):
        _check_cuda(t)
        if t.device != x.device:
            raise RuntimeError("All buffers must be on the same device")
    if not (b.dim() == 2 and b.dtype == torch.uint8 and b.size(1) * 2 == KP
            and b.size(0) >= padded(N, 8) and N > 0):
        raise RuntimeError("Invalid padded operand shapes")
    if not (sw.dtype == torch.float32 and sums.dtype == torch.int32
            and sw.numel() >= padded(N, 8) and sums.numel() >= padded(N, 8)):
        raise RuntimeError("Invalid metadata dtypes")
    dtype = torch.float32 if fp32 else torch.float16
    if not (bias.dtype == dtype and (bias.numel() == 0 or bias.numel() == N)):
        raise RuntimeError("Bias shape/dtype mismatch")
    dev = x.device
    _lib.require_gfx950(dev)
    out = torch.empty((M, N), dtype=dtype, device=dev)
    with torch.cuda.device(dev):
        _lib.call("dscq_linear_decode", x.data_ptr(),
                  _lib.F16 if x.dtype == torch.float16 else _lib.F32, M, K, clip, rotate_block,
                  b.data_ptr(), sw.data_ptr(), sums.data_ptr(), _lib.ptr(bias), N,
                  1 if fp32 else 0, out.data_ptr(), _lib.stream(dev))
    return out


def pack_weight(w: torch.Tensor, clip: float = 1.0, rotate_block: int = 0,
                return_codes: bool = False):
    """Weight glue for ``matmul``: [packed u8 [NP, KP/2], sw f32 [NP], sums i32 [NP]].

    Codes follow weight_codes (core/quantization.py:7-11) at 4 bits and are
    packed as pack_int4 (:31-40); ``sums[n] = sum_k code[n, k]`` feeds the
    zero-point correction of the epilogue (kernel/w4a4.cu:74).  With
    ``rotate_block=128`` the weight is first folded as W H_128 / 128, the
    partner of ``quantize(..., rotate_block=128)``.  ``return_codes`` appends
    the signed int8 codes [NP, KP].
    """
    _check_cuda(w)
    if w.dtype == torch.bfloat16:
        w = w.float()
    _check_float(w)
    if w.dim() != 2:
        raise RuntimeError("Weights must be a matrix")
    clip = float(clip)
    N, K = w.shape
    NP, KP = padded(N, 8), padded(K, 64)
    dev = w.device
    _lib.require_gfx950(dev)
    packed = torch.empty((NP, KP // 2), dtype=torch.uint8, device=dev)
    sw = torch.empty((NP,), dtype=torch.float32, device=dev)
    sums = torch.empty((NP,), dtype=torch.int32, device=dev)
    codes = torch.empty((NP, KP), dtype=torch.int8, device=dev) if return_codes else None
    with torch.cuda.device(dev):
        _lib.call("dscq_pack_weight", w.data_ptr(),
                  _lib.F16 if w.dtype == torch.float16 else _lib.F32, N, K, clip,
                  rotate_block, packed.data_ptr(), sw.data_ptr(), sums.data_ptr(),
                  _lib.ptr(codes), _lib.stream(dev))
    if return_codes:
        return [packed, sw, sums, codes]
    return [packed, sw, sums]


def silu_mul_quantize(gate_up: torch.Tensor, clip: float = 1.0, rotate_block: int = 0,
                      return_h: bool = False):
    """Quantize + pack the gated activation of a SiLU-gated MLP.

    ``gate_up`` is the fp16 [M, 2N] output of one W4A4 GEMM against the
    concatenated gate and up weights (gate in columns [0, N), up in [N, 2N)).
    The rows quantized are h = fp16(fp16(silu(g)) * u), the down projection's
    input; the result is what ``quantize(h, clip, True, rotate_block)`` returns:
    [packed u8 [MP, KP/2], scales f32 [MP], zeros i32 [MP]] (KP = ceil64(N)),
    plus h [M, N] fp16 when ``return_h``.
    """
    _check_cuda(gate_up)
    if gate_up.dtype != torch.float16:
        raise RuntimeError("silu_mul_quantize: gate|up must be fp16")
    if gate_up.dim() != 2 or gate_up.size(1) % 2:
        raise RuntimeError("silu_mul_quantize: expected [M, 2N]")
    clip = float(clip)
    if not (0.5 <= clip <= 1.0):
        raise RuntimeError("Activation clip must be in [0.5,1]")
    M, N = gate_up.size(0), gate_up.size(1) // 2
    if rotate_block not in (0, 128) or (rotate_block and N % rotate_block):
        raise RuntimeError(f"Rotation needs N to be a multiple of {rotate_block} (got N={N})")
    dev = gate_up.device
    _lib.require_gfx950(dev)
    MP, KP = padded(M, 8), padded(N, 64)
    packed = torch.empty((MP, KP // 2), dtype=torch.uint8, device=dev)
    scales = torch.empty((MP,), dtype=torch.float32, device=dev)
    zeros = torch.empty((MP,), dtype=torch.int32, device=dev)
    h = torch.empty((M, N), dtype=torch.float16, device=dev) if return_h else None
    with torch.cuda.device(dev):
        _lib.call("dscq_silu_mul_quantize", gate_up.data_ptr(), gate_up.data_ptr() + 2 * N,
                  2 * N, M, N, clip, rotate_block, packed.data_ptr(), scales.data_ptr(),
                  zeros.data_ptr(), _lib.ptr(h), _lib.stream(dev))
    out = [packed, scales, zeros]
    if return_h:
        out.append(h)
    return out


def interleave_gate_up(gate, up, block: int = 64) -> torch.Tensor:
    """Rows of two [N, ...] tensors (packed weights, sw, sums or bias of a gate and
    an up projection) interleaved in ``block``-row blocks, the weight order
    ``matmul_silu_mul`` reads: gate rows 64t .. 64t+63, then up rows 64t .. 64t+63."""
    if gate.shape != up.shape or gate.size(0) % block:
        raise RuntimeError(f"interleave_gate_up: need equal shapes with rows % {block} == 0")
    rest = tuple(gate.shape[1:])
    g = gate.reshape(gate.size(0) // block, block, *rest)
    u = up.reshape(up.size(0) // block, block, *rest)
    return torch.stack([g, u], dim=1).reshape(2 * gate.size(0), *rest).contiguous()


def matmul_silu_mul(a, b_gu, sx, zx, sw, sums, bias, M: int, N: int) -> torch.Tensor:
    """h [M, N] fp16 = fp16(fp16(silu(g)) * u) of the gate and up projections in one
    GEMM (include/dscq.h: dscq_matmul_silu_mul).  ``a``, ``sx``, ``zx`` as for
    ``matmul``; ``b_gu``, ``sw``, ``sums`` and ``bias`` (empty or fp16 [2N]) hold
    the gate and up rows in ``interleave_gate_up`` order.  Needs N % 64 == 0."""
    for t in (a, b_gu, sx, zx, sw, sums, bias):
        _check_cuda(t)
        if t.device != a.device:
            raise RuntimeError("All buffers must be on the same device")
    M, N = int(M), int(N)
    if not (a.dim() == 2 and a.dtype == torch.uint8 and b_gu.dim() == 2
            and b_gu.dtype == torch.uint8 and a.size(1) == b_gu.size(1)
            and a.size(0) >= padded(M, 8) and b_gu.size(0) == 2 * N):
        raise RuntimeError("Invalid padded operand shapes")
    if not (sx.dtype == torch.float32 and zx.dtype == torch.int32 and sw.dtype == torch.float32
            and sums.dtype == torch.int32 and sx.numel() >= padded(M, 8)
            and zx.numel() >= padded(M, 8) and sw.numel() == 2 * N and sums.numel() == 2 * N):
        raise RuntimeError("Invalid metadata dtypes")
    if not (bias.numel() == 0 or (bias.dtype == torch.float16 and bias.numel() == 2 * N)):
        raise RuntimeError("Bias shape/dtype mismatch")
    dev = a.device
    _lib.require_gfx950(dev)
    h = torch.empty((M, N), dtype=torch.float16, device=dev)
    with torch.cuda.device(dev):
        _lib.call("dscq_matmul_silu_mul", a.data_ptr(), b_gu.data_ptr(), sx.data_ptr(),
                  zx.data_ptr(), sw.data_ptr(), sums.data_ptr(), _lib.ptr(bias), M, N,
                  a.size(1) * 2, h.data_ptr(), _lib.stream(dev))
    return h
