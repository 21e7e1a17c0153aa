"""The measurement probes (include/dscq.h: dscq_stream_probe, dscq_mfma_probe)
compute what they say, so the ceilings bench.py reports time real work."""
import numpy as np
import pytest
import torch

from dscquant_amd import _lib

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("pieces", [1, 2, 4, 8, 16])
def test_stream_probe_writes_the_xor_of_its_pieces(gpu, pieces):
    n = 1 << 16  # output pieces
    print(f"case: stream probe, {pieces} pieces per thread", flush=True)
    src = torch.randint(0, 256, (n * pieces * 16,), dtype=torch.uint8, device=gpu)
    dst = torch.zeros(n * 16, dtype=torch.uint8, device=gpu)
    _lib.call("dscq_stream_probe", src.data_ptr(), src.numel(), dst.data_ptr(), dst.numel(),
              pieces, _lib.stream(gpu))
    torch.cuda.synchronize()
    want = np.bitwise_xor.reduce(src.cpu().numpy().reshape(pieces, n, 16), axis=0)
    assert np.array_equal(dst.cpu().numpy().reshape(n, 16), want)
    # the read-only form leaves dst alone unless some thread hits the constant
    dst.zero_()
    _lib.call("dscq_stream_probe", src.data_ptr(), src.numel(), dst.data_ptr(), 0, pieces,
              _lib.stream(gpu))
    torch.cuda.synchronize()
    assert int(dst.count_nonzero()) == 0


def _part(seed, idx):
    h = ((seed * 0x9E3779B1) ^ (idx * 0x85EBCA77)) & 0xFFFFFFFF
    return (((h >> 13) ^ (h >> 7)) & 7) * 16 - 64


def _increment(sx, sy):
    """What one MFMA of operand sets sx, sy adds to the sum of its 32 x 32
    accumulator: sum_k (Fx + 32 gx(k)) (Fy + 32 gy(k)) over the 32 k values
    (half, p), F = sum over the 32 rows of f (the kernel's probe_operand)."""
    def fg(seed):
        F = sum(_part(seed, 64 + i) for i in range(32))
        g = [_part(seed ^ 0x5BD1E995, h * 16 + p) for h in range(2) for p in range(16)]
        return F, g
    (Fx, gx), (Fy, gy) = fg(sx), fg(sy)
    return sum((Fx + 32 * a) * (Fy + 32 * b) for a, b in zip(gx, gy))


@pytest.mark.parametrize("wgs,waves,mfmas", [(256, 8, 512), (3, 5, 24)])
def test_mfma_probe_checksum(gpu, wgs, waves, mfmas):
    print(f"case: mfma probe {wgs}x{waves} waves, {mfmas} MFMAs each", flush=True)
    out = torch.zeros(wgs * waves, dtype=torch.int32, device=gpu)
    _lib.call("dscq_mfma_probe", wgs, waves, mfmas, out.data_ptr(), _lib.stream(gpu))
    torch.cuda.synchronize()
    steps = mfmas // 4
    # four accumulators per wave, each step one MFMA per accumulator; sets
    # (b0, a0) and (b1, a1) alternate
    want = 4 * (steps // 2) * (_increment(2, 1) + _increment(4, 3))
    want &= 0xFFFFFFFF
    want = want - (1 << 32) if want >= (1 << 31) else want
    assert out.cpu().numpy().tolist() == [want] * (wgs * waves)
