"""On-disk format of pre-packed W4A4 weights.

A packed linear layer is what ``dscq_pack_weight`` produces -- the operand every
GEMM of this package reads -- plus what is needed to use it again:

    packed  u8  [NP, KP/2]  byte j of a row holds the codes of k = 2j (low nibble)
                            and 2j+1 (high nibble), each as (c & 15), c in [-7, 7]
                            (core/quantization.py:31-40; padding: code 0)
    sw      f32 [NP]        per-output-channel scale (core/quantization.py:7-11)
    sums    i32 [NP]        per-row code sums (the epilogue's zero-point term,
                            kernel/w4a4.cu:74-75)
    bias    optional [N] fp16/fp32

with NP = ceil(N/8)*8 and KP = ceil(K/64)*64 (the shape contract of
kernel/w4a4.cu:195-200).  Files are safetensors (no code runs on load); the
metadata records the format version, K, N, the rotation the weights were
folded with (0 or 128: activations must be quantized with the same
``rotate_block``) and the weight clip.
"""
from __future__ import annotations

import torch

FORMAT = "dscq-w4-packed/1"


def _padded(v: int, m: int) -> int:
    return (v + m - 1) // m * m


def _check(packed, sw, sums, bias, K: int, N: int) -> None:
    NP, KP = _padded(N, 8), _padded(K, 64)
    if not (packed.dtype == torch.uint8 and tuple(packed.shape) == (NP, KP // 2)):
        raise ValueError(f"packed must be uint8 [{NP}, {KP // 2}] for N={N}, K={K}, "
                         f"got {packed.dtype} {tuple(packed.shape)}")
    if not (sw.dtype == torch.float32 and tuple(sw.shape) == (NP,)):
        raise ValueError(f"sw must be float32 [{NP}]")
    if not (sums.dtype == torch.int32 and tuple(sums.shape) == (NP,)):
        raise ValueError(f"sums must be int32 [{NP}]")
    if bias is not None and not (bias.dtype in (torch.float16, torch.float32)
                                 and tuple(bias.shape) == (N,)):
        raise ValueError(f"bias must be fp16/fp32 [{N}]")


def save_packed(path: str, packed, sw, sums, K: int, N: int, rotate_block: int = 0,
                weight_clip: float = 1.0, bias=None) -> None:
    """Writes one packed linear layer to ``path`` (safetensors)."""
    from safetensors.torch import save_file
    K, N = int(K), int(N)
    if rotate_block not in (0, 128):
        raise ValueError(f"rotate_block must be 0 or 128 (got {rotate_block})")
    _check(packed, sw, sums, bias, K, N)
    tensors = {"packed": packed.detach().contiguous().cpu(),
               "sw": sw.detach().contiguous().cpu(),
               "sums": sums.detach().contiguous().cpu()}
    if bias is not None:
        tensors["bias"] = bias.detach().contiguous().cpu()
    meta = {"format": FORMAT, "K": str(K), "N": str(N), "rotate_block": str(int(rotate_block)),
            "weight_clip": repr(float(weight_clip))}
    save_file(tensors, path, metadata=meta)


def load_packed(path: str, device=None) -> dict:
    """Reads a file written by ``save_packed``: a dict with ``packed``, ``sw``,
    ``sums``, ``bias`` (or None), ``K``, ``N``, ``rotate_block``, ``weight_clip``."""
    from safetensors import safe_open
    with safe_open(path, framework="pt", device="cpu") as f:
        meta = f.metadata() or {}
        if meta.get("format") != FORMAT:
            raise ValueError(f"{path}: not a {FORMAT} file (format={meta.get('format')!r})")
        names = set(f.keys())
        t = {k: f.get_tensor(k) for k in names}
    K, N = int(meta["K"]), int(meta["N"])
    bias = t.get("bias")
    _check(t["packed"], t["sw"], t["sums"], bias, K, N)
    out = {"packed": t["packed"], "sw": t["sw"], "sums": t["sums"], "bias": bias, "K": K, "N": N,
           "rotate_block": int(meta["rotate_block"]), "weight_clip": float(meta["weight_clip"])}
    if device is not None:
        for k in ("packed", "sw", "sums", "bias"):
            if out[k] is not None:
                out[k] = out[k].to(device)
    return out
