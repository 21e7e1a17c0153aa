"""Full-size parity at the Llama-70B linear shapes (M=4096; q/o K=N=8192,
gate/up K=8192 -> N=28672, down K=28672 -> N=8192), where a whole-output
oracle product would be slow.

The activation quantization (rotate + quantize + pack, 4096 x 28672) and the
weight packing are checked bit for bit against the oracle in full; the GEMM's
int32 accumulators and fp16 outputs are checked exactly on a seeded sample of
96 rows x 96 columns (int64 dot products of the oracle-unpacked codes), plus a
size-independent identity over the whole output: the row sums of raw equal
the unpacked activation codes times the column sums of the weight codes.
"""
import numpy as np
import pytest
import torch

from dscquant_amd import w4a4
from oracle import native
from tests.conftest import weights

pytestmark = pytest.mark.gpu


def _activations(M, K, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(M, K, generator=g)
    idx = torch.randperm(K, generator=torch.Generator().manual_seed(seed + 2))[:int(np.ceil(0.01 * K))]
    x[:, idx] *= 50
    return x.half()


@pytest.mark.parametrize("M,N,K", [(4096, 8192, 8192), (4096, 28672, 8192), (4096, 8192, 28672)])
def test_70b_shapes_full_quantize_and_sampled_gemm(gpu, M, N, K):
    print(f"70B-shape case M{M} N{N} K{K}", flush=True)
    rot = 128
    x = _activations(M, K, seed=11)
    w = torch.from_numpy(weights(N, K, seed=12))
    pa, sx, zx = w4a4.quantize(x.to(gpu), 1.0, True, rot)
    pw, sw, sums = w4a4.pack_weight(w.to(gpu), 1.0, rot)
    out, raw = w4a4.matmul(pa, pw, sx, zx, sw, sums,
                           torch.empty(0, dtype=torch.float16, device=gpu), M, N, fused=False)
    torch.cuda.synchronize()

    # activations and weights in full, bit for bit
    pa_ref, sx_ref, zx_ref = native.quantize_rows(x.float().numpy(), 1.0, rot)
    np.testing.assert_array_equal(pa.cpu().numpy(), pa_ref)
    np.testing.assert_array_equal(sx.cpu().numpy(), sx_ref)
    np.testing.assert_array_equal(zx.cpu().numpy(), zx_ref)
    pw_ref, sw_ref, sums_ref = native.pack_weight(w.float().numpy(), 1.0, rot)
    np.testing.assert_array_equal(pw.cpu().numpy(), pw_ref)
    np.testing.assert_array_equal(sums.cpu().numpy(), sums_ref)

    KP = pa_ref.shape[1] * 2
    rng = np.random.default_rng(M + N + K)
    rows = np.sort(rng.choice(M, 96, replace=False))
    cols = np.sort(rng.choice(N, 96, replace=False))
    ia = native.unpack_int4(pa_ref[rows], KP).astype(np.int64)
    ib = native.unpack_int4(pw_ref[cols], KP).astype(np.int64)
    raw_ref = ia @ ib.T
    raw_gpu = raw.cpu().numpy()
    np.testing.assert_array_equal(raw_gpu[np.ix_(rows, cols)], raw_ref)
    out_ref = native.restore(raw_ref.astype(np.int32), sx_ref[rows], zx_ref[rows],
                             sw_ref[cols], sums_ref[cols], None)
    np.testing.assert_array_equal(out.cpu().numpy()[np.ix_(rows, cols)], out_ref)

    # whole output: sum_n raw[m, n] = sum_k a[m, k] * (sum_n b[n, k]), exact in int64
    colsum_b = np.zeros(KP, np.int64)
    for r0 in range(0, N, 1024):
        colsum_b += native.unpack_int4(pw_ref[r0:min(r0 + 1024, N)], KP).sum(0, dtype=np.int64)
    for r0 in range(0, M, 512):
        a_blk = native.unpack_int4(pa_ref[r0:r0 + 512], KP).astype(np.int64)
        np.testing.assert_array_equal(raw_gpu[r0:r0 + 512].sum(1, dtype=np.int64),
                                      a_blk @ colsum_b)
