"""Seeded random shapes through the fused decode linear (dscq_linear_decode)
against the two-launch path and the oracle, bit for bit.

The kernel picks from M and K the product form (v_dot8 for M <= 2, MFMA
beyond), the activation layout (16 lanes per block for up to 64 blocks, a quad
per block beyond) and the weight pieces per lane (4, 8 or 12).  This sweep
draws M, K (a multiple of 128 with rotation, any multiple of 8 without), N
(ragged or a multiple of 16), clip, bias and the input / output dtypes over the
shapes the kernel accepts.
"""
import numpy as np
import pytest
import torch

from dscquant_amd import w4a4
from oracle import native
from tests.conftest import activations, weights, sweep_size

pytestmark = pytest.mark.gpu


def _fits(M, K):
    """The kernel's limits (dscq_linear_decode_supported), restated so that the
    cases are drawn without loading the library; the test checks they agree."""
    KP = (K + 63) // 64 * 64
    KB, nblk = KP // 2, (KP + 127) // 128
    return (1 <= M <= 8 and K % 8 == 0 and M * nblk <= 128 and M * KB <= 16384
            and (KB + 63) // 64 <= 8 * 12 and (KB + 511) // 512 <= 12)


def _cases(n, seed):
    rng = np.random.default_rng(seed)
    out = []
    while len(out) < n:
        M = int(rng.integers(1, 5))
        rot = 128 if rng.random() < 0.7 else 0
        K = int(rng.integers(1, 97)) * 128 if rot else int(rng.integers(1, 1500)) * 8
        if not _fits(M, K):
            continue
        N = int(rng.choice([rng.integers(1, 300), rng.integers(300, 12000)]))
        if rng.random() < 0.5:
            N = (N + 15) // 16 * 16
        clip = 1.0 if rng.random() < 0.6 else float(np.float32(rng.uniform(0.5, 1.0)))
        out.append((M, K, N, rot, clip, bool(rng.random() < 0.3), bool(rng.random() < 0.4),
                    bool(rng.random() < 0.3)))
    return out


CASES = _cases(*sweep_size(28, 31337))


@pytest.mark.parametrize("M,K,N,rot,clip,x32,bias,fp32", CASES,
                         ids=[f"M{c[0]}-K{c[1]}-N{c[2]}-rot{c[3]}" for c in CASES])
def test_linear_decode_random_shapes(gpu, M, K, N, rot, clip, x32, bias, fp32):
    print(f"decode sweep case M{M} K{K} N{N} rot{rot} clip{clip} x32{x32} bias{bias} "
          f"fp32{fp32}", flush=True)
    assert w4a4.linear_decode_supported(M, K)
    x = activations(M, K, seed=M * 101 + K + N, dtype=np.float32 if x32 else np.float16)
    w = weights(N, K, seed=N * 13 + K)
    out_np = np.float32 if fp32 else np.float16
    b = (np.random.default_rng(N).standard_normal(N) * 0.1).astype(out_np) if bias else None
    xt = torch.from_numpy(x).to(gpu)
    pw, sw, sums = w4a4.pack_weight(torch.from_numpy(w).to(gpu), 1.0, rot)
    out_dtype = torch.float32 if fp32 else torch.float16
    bt = torch.empty(0, dtype=out_dtype, device=gpu) if b is None else torch.from_numpy(b).to(gpu)
    y = w4a4.linear_decode(xt, clip, rot, pw, sw, sums, bt, N, fp32)
    pa, sx, zx = w4a4.quantize(xt, clip, True, rot)
    y2, _ = w4a4.matmul(pa, pw, sx, zx, sw, sums, bt, M, N, True, False, fp32)
    torch.cuda.synchronize()
    assert torch.equal(y, y2)
    ref, *_ = native.linear_w4a4(x.astype(np.float32), w.astype(np.float32), b, clip_a=clip,
                                 rotate_block=rot, out_dtype=out_np)
    np.testing.assert_array_equal(y.cpu().numpy(), ref)
