"""Seeded random shapes through dscq_matmul against the oracle, bit for bit.

The GEMM dispatch picks among the skinny-M kernel, the pipelined kernel with
256x128 / 128x128 / 64x128 tiles of four or eight waves, and the general tiled
kernel from M, N, KP and the output alignment; the rules move as kernels get
tuned.  This sweep draws M, N (ragged or a multiple of 8) and K over the ranges
where those choices change, with bias, fp32 output and forced decode at random,
and holds every case to the oracle's int32 accumulators and epilogue in both the
raw-accumulator and fused modes (the same checks as test_gpu_matmul.py).
"""
import numpy as np
import pytest
import torch

from dscquant_amd import w4a4
from oracle import native
from tests.conftest import sweep_size
from tests.test_gpu_matmul import _operands, _oracle_raw

pytestmark = pytest.mark.gpu


def _cases(n, seed):
    rng = np.random.default_rng(seed)
    out = []
    while len(out) < n:
        M = int(rng.choice([rng.integers(1, 64), rng.integers(64, 400), rng.integers(400, 1100)]))
        N = int(rng.choice([rng.integers(1, 600), rng.integers(600, 3000),
                            rng.integers(3000, 12000)]))
        if rng.random() < 0.6:
            N = (N + 7) // 8 * 8
        K = int(rng.choice([rng.integers(1, 1200), rng.integers(1200, 5000),
                            rng.integers(4000, 9000)]))
        if M * N * ((K + 63) // 64 * 64) > 2.5e9:
            continue
        out.append((M, N, K, bool(rng.random() < 0.5), bool(rng.random() < 0.3),
                    bool(rng.random() < 0.1)))
    return out


CASES = _cases(*sweep_size(48, 2026))


@pytest.mark.parametrize("M,N,K,use_bias,fp32,force_decode", CASES,
                         ids=[f"M{c[0]}-N{c[1]}-K{c[2]}" for c in CASES])
def test_matmul_random_shapes(gpu, M, N, K, use_bias, fp32, force_decode):
    print(f"sweep case M{M} N{N} K{K} bias{use_bias} fp32{fp32} decode{force_decode}",
          flush=True)
    a, b, sx, zx, sw, sums = _operands(M, N, K, seed=M * 7919 + N * 31 + K)
    out_dtype = np.float32 if fp32 else np.float16
    bias = (np.random.default_rng(N + K).standard_normal(N).astype(out_dtype)
            if use_bias else None)
    T = lambda v: torch.from_numpy(v).to(gpu)  # noqa: E731
    tbias = T(bias) if use_bias else torch.empty(0, dtype=torch.float32 if fp32 else torch.float16,
                                                 device=gpu)
    out, raw = w4a4.matmul(T(a), T(b), T(sx), T(zx), T(sw), T(sums), tbias, M, N,
                           fused=False, force_decode=force_decode, fp32=fp32)
    out_f, _ = w4a4.matmul(T(a), T(b), T(sx), T(zx), T(sw), T(sums), tbias, M, N,
                           fused=True, force_decode=force_decode, fp32=fp32)
    torch.cuda.synchronize()
    raw_ref = _oracle_raw(a, b, M, N)
    np.testing.assert_array_equal(raw.cpu().numpy(), raw_ref)
    out_ref = native.restore(raw_ref, sx, zx, sw, sums, bias, out_dtype=out_dtype)
    np.testing.assert_array_equal(out.cpu().numpy(), out_ref)
    np.testing.assert_array_equal(out_f.cpu().numpy(), out_ref)
