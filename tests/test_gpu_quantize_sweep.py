"""Seeded random shapes through dscq_quantize and dscq_pack_weight against the
oracle, bit for bit.

The row-quantization dispatch picks, from M and K, the waves per row (1, 2, 4),
the 128-blocks per quad (1, 2, 4), how the row fills those blocks (whole
blocks exactly, whole blocks with quads past the row, a partial last block),
the clamp-free form (clip 1), one row per workgroup (two waves per row over
2048+ rows), the LDS-staged packed stores (rows that fill every block) and,
past 32768 elements, the streaming kernel.  This sweep draws M, K, clip, the
rotation, the input dtype and the fused / two-pass mode over the ranges where
those choices change and holds every case to the oracle's codes, scales and
zero-points (activations) and packed weights, scales and code sums (weights).
"""
import numpy as np
import pytest
import torch

from dscquant_amd import w4a4
from oracle import native
from tests.conftest import activations, weights, sweep_size

pytestmark = pytest.mark.gpu


def _cases(n, seed):
    rng = np.random.default_rng(seed)
    out = []
    while len(out) < n:
        M = int(rng.choice([rng.integers(1, 64), rng.integers(64, 1500),
                            rng.integers(1900, 3200)]))
        K = int(rng.choice([rng.integers(1, 40) * 128, rng.integers(8, 5000),
                            rng.integers(5000, 32000), rng.integers(1, 17) * 2048,
                            rng.integers(32776, 40000)]))
        K = max(8, K // 8 * 8) if rng.random() < 0.85 else max(1, K)
        if M * K > 3.5e7:
            continue
        rot = 128 if K % 128 == 0 and rng.random() < 0.7 else 0
        clip = 1.0 if rng.random() < 0.6 else float(np.float32(rng.uniform(0.5, 1.0)))
        dtype = np.float16 if rng.random() < 0.7 else np.float32
        fused = bool(rng.random() < 0.8)
        out.append((M, K, rot, clip, dtype, fused))
    return out


CASES = _cases(*sweep_size(40, 4242))


@pytest.mark.parametrize("M,K,rot,clip,dtype,fused", CASES,
                         ids=[f"M{c[0]}-K{c[1]}-rot{c[2]}-{np.dtype(c[4]).name}" for c in CASES])
def test_quantize_random_shapes(gpu, M, K, rot, clip, dtype, fused):
    print(f"quantize sweep case M{M} K{K} rot{rot} clip{clip} {np.dtype(dtype).name} "
          f"fused{fused}", flush=True)
    x = activations(M, K, seed=M * 131 + K, dtype=dtype)
    packed, scales, zeros = w4a4.quantize(torch.from_numpy(x).to(gpu), clip, fused, rot)
    torch.cuda.synchronize()
    p_ref, s_ref, z_ref = native.quantize_rows(x.astype(np.float32), clip, rot)
    np.testing.assert_array_equal(scales.cpu().numpy(), s_ref)
    np.testing.assert_array_equal(zeros.cpu().numpy(), z_ref)
    np.testing.assert_array_equal(packed.cpu().numpy(), p_ref)


WCASES = [c for c in _cases(60, seed=777) if c[0] * c[1] <= 1.2e7][:16]


@pytest.mark.parametrize("N,K,rot,clip,dtype,_fused", WCASES,
                         ids=[f"N{c[0]}-K{c[1]}-rot{c[2]}" for c in WCASES])
def test_pack_weight_random_shapes(gpu, N, K, rot, clip, dtype, _fused):
    print(f"pack_weight sweep case N{N} K{K} rot{rot} clip{clip}", flush=True)
    w = weights(N, K, seed=N * 17 + K, dtype=dtype)
    packed, sw, sums = w4a4.pack_weight(torch.from_numpy(w).to(gpu), clip, rot)
    torch.cuda.synchronize()
    p_ref, sw_ref, sums_ref = native.pack_weight(w.astype(np.float32), clip, rot)
    np.testing.assert_array_equal(sw.cpu().numpy(), sw_ref)
    np.testing.assert_array_equal(sums.cpu().numpy(), sums_ref)
    np.testing.assert_array_equal(packed.cpu().numpy(), p_ref)
