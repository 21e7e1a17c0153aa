"""GPU parity of the W4A4 GEMM (int8 MFMA path and skinny-M path).

raw int32 accumulators are compared bit-exactly with the oracle's integer
GEMM; the dequantized output is compared bit-exactly with the oracle's fp32
epilogue narrowed to fp16 (same operation order, no fma), and additionally
held to the max relative error 1e-3 against a float64 dequant of the same
accumulators.  Operands are random bytes (every nibble value, both signs at
the extremes) with random metadata, plus the end-to-end config data.
"""
import numpy as np
import pytest
import torch

from dscquant_amd import w4a4
from oracle import native
from tests.conftest import activations, weights

pytestmark = pytest.mark.gpu


def _operands(M, N, K, seed):
    rng = np.random.default_rng(seed)
    MP, NP, KP = (M + 7) // 8 * 8, (N + 7) // 8 * 8, (K + 63) // 64 * 64
    a = rng.integers(0, 256, size=(MP, KP // 2), dtype=np.uint8)
    b = rng.integers(0, 256, size=(NP, KP // 2), dtype=np.uint8)
    sx = (rng.random(MP).astype(np.float32) + 0.5) * 0.05
    zx = rng.integers(0, 16, size=MP).astype(np.int32)
    sw = (rng.random(NP).astype(np.float32) + 0.5) * 0.002
    sums = rng.integers(-2000, 2000, size=NP).astype(np.int32)
    return a, b, sx, zx, sw, sums


def _oracle_raw(a, b, M, N):
    KP = a.shape[1] * 2
    if M * N * KP > 3e8:
        return native.gemm_raw_blas(a, b, M, N)
    return native.gemm_raw(a, b, M, N)


def _dequant64(raw, sx, zx, sw, sums, bias, M, N):
    corr = raw.astype(np.int64) + (8 - zx[:M, None].astype(np.int64)) * sums[None, :N]
    out = corr.astype(np.float64) * sx[:M, None] * sw[None, :N]
    if bias is not None:
        out = out + bias[None, :N].astype(np.float64)
    return out


MM_CASES = [
    # (M, N, K, bias, fp32, force_decode)
    (1, 4096, 4096, False, False, False),
    (4, 11008, 4096, False, False, False),
    (7, 100, 64, True, False, False),
    (8, 4096, 4096, False, False, False),
    (16, 4096, 4096, True, False, False),
    (16, 11008, 4096, False, False, False),
    (16, 4096, 4096, False, False, True),
    (33, 72, 192, True, True, False),
    (64, 264, 320, False, False, True),
    (128, 256, 4096, False, False, False),
    (300, 520, 1088, True, False, False),
    (512, 11008, 4096, False, False, False),
    (512, 4096, 11008, False, False, False),
    (1000, 1000, 1024, True, True, False),
    (2048, 4096, 4096, False, False, False),
    # packed rows ending halfway through a 256-nibble K slice (K % 256 == 128)
    (96, 136, 128, True, False, False),
    (200, 264, 384, False, True, False),
    (256, 512, 4224, True, False, False),
    # 64 x 128 tiles past one round (280 tiles): four waves per workgroup
    (448, 5120, 512, True, False, False),
    # mid-M with 65 column tiles and a K tail: eight-wave 64 x 128 tiles
    (40, 8200, 320, True, False, False),
    (24, 8200, 192, False, True, False),
    (17, 8264, 4096, True, False, False),
    # one round of 128 x 128 tiles (224 of them): eight waves per workgroup
    (192, 14336, 320, True, True, False),
    # 128 x 128 tiles past one round (688), two workgroups per CU
    (512, 22016, 64, False, False, False),
    # M >= 64 with few weight rows: the skinny-M kernel (ceil(M/16) * N <= 16384)
    (100, 1000, 4096, True, True, False),
    (144, 1024, 4160, False, False, False),
    # K split over workgroups (few 64 x 128 tiles, long K): 4 and 5 parts
    (130, 2056, 8384, True, True, False),
    (64, 4104, 11072, False, False, False),
    # K split with an fp16 bias: mid-M (pipelined 64 x 128 tiles, 2 parts) and
    # M = 128 down projection (4 parts)
    (32, 11008, 11008, True, False, False),
    (128, 4096, 11008, True, False, False),
    # one round of 64 x 128 tiles with K >= 4096: the k-group kernel (padded
    # rows with an fp32 bias; N past the last full tile with a K tail)
    (300, 2048, 8192, True, True, False),
    (64, 8200, 4352, True, False, False),
    # 256 x 128 tiles past one round: two rounds (even slice count), 448
    # tiles (a 75% last round, odd slice count, fp32 out), a K tail with an
    # fp32 bias, and a single slice
    (2048, 8192, 512, True, False, False),
    (3584, 4096, 4352, False, True, False),
    (2048, 8192, 4160, True, True, False),
    (2048, 8192, 256, False, False, False),
    # wide N in whole rounds: each XCD's workgroups of a round on a 4 x 8 block
    # of tiles (1024 x 16384: two rounds of 256 tiles)
    (1024, 16384, 320, True, False, False),
    # skinny-M workgroups with two or three tiles of 16 columns: N = 14336
    # (two), ragged N = 8200 (three, the last workgroup short), forced decode
    # over three row blocks with ragged N (two)
    (16, 14336, 4096, True, True, False),
    (8, 8200, 4096, True, False, False),
    (40, 5000, 1024, False, False, True),
]


@pytest.mark.parametrize("M,N,K,use_bias,fp32,force_decode", MM_CASES,
                         ids=[f"M{c[0]}-N{c[1]}-K{c[2]}-bias{int(c[3])}-fp32{int(c[4])}"
                              f"-decode{int(c[5])}" for c in MM_CASES])
def test_matmul_matches_oracle(gpu, M, N, K, use_bias, fp32, force_decode):
    print(f"matmul case M{M} N{N} K{K} bias{use_bias} fp32{fp32} decode{force_decode}",
          flush=True)
    a, b, sx, zx, sw, sums = _operands(M, N, K, seed=M + 3 * N + 7 * K)
    out_dtype = np.float32 if fp32 else np.float16
    bias = (np.random.default_rng(K).standard_normal(N).astype(out_dtype)
            if use_bias else None)
    T = lambda v: torch.from_numpy(v).to(gpu)  # noqa: E731
    tbias = T(bias) if use_bias else torch.empty(0, dtype=torch.float32 if fp32 else torch.float16,
                                                 device=gpu)
    out, raw = w4a4.matmul(T(a), T(b), T(sx), T(zx), T(sw), T(sums), tbias, M, N,
                           fused=False, force_decode=force_decode, fp32=fp32)
    out_f, raw_f = w4a4.matmul(T(a), T(b), T(sx), T(zx), T(sw), T(sums), tbias, M, N,
                               fused=True, force_decode=force_decode, fp32=fp32)
    torch.cuda.synchronize()
    assert raw_f.numel() == 0
    raw_ref = _oracle_raw(a, b, M, N)
    np.testing.assert_array_equal(raw.cpu().numpy(), raw_ref)
    out_ref = native.restore(raw_ref, sx, zx, sw, sums, bias, out_dtype=out_dtype)
    got = out.cpu().numpy()
    np.testing.assert_array_equal(got, out_ref)
    np.testing.assert_array_equal(out_f.cpu().numpy(), got)
    # max relative error 1e-3 against a float64 dequant of the accumulators
    exact = _dequant64(raw_ref, sx, zx, sw, sums, bias, M, N)
    rel = np.abs(got.astype(np.float64) - exact) / np.maximum(np.abs(exact), 1e-30)
    big = np.abs(exact) > 1e-2
    assert rel[big].max() <= 1e-3


def test_matmul_extreme_nibbles(gpu):
    """All -8 x -8 and -8 x +7 at K = 4096: the largest |products| and sums."""
    M, N, K = 40, 72, 4096
    a = np.full((40, K // 2), 0x88, np.uint8)
    b = np.full((72, K // 2), 0x88, np.uint8)
    b[36:] = 0x77
    T = lambda v: torch.from_numpy(v).to(gpu)  # noqa: E731
    ones = lambda n: torch.ones(n, device=gpu)  # noqa: E731
    zeros_i = lambda n: torch.full((n,), 8, dtype=torch.int32, device=gpu)  # noqa: E731
    out, raw = w4a4.matmul(T(a), T(b), ones(40), zeros_i(40), ones(72),
                           torch.zeros(72, dtype=torch.int32, device=gpu),
                           torch.empty(0, dtype=torch.float32, device=gpu), M, N,
                           fused=False, fp32=True)
    r = raw.cpu().numpy()
    assert (r[:, :36] == 64 * K).all() and (r[:, 36:] == -56 * K).all()


def test_matmul_long_k(gpu):
    """K beyond 65536 drains the scaled accumulator (worst-case magnitudes)."""
    M, N, K = 16, 64, 139264
    rng = np.random.default_rng(9)
    a = np.full((16, K // 2), 0x88, np.uint8)
    a[:, ::3] = rng.integers(0, 256, size=a[:, ::3].shape, dtype=np.uint8)
    b = np.full((64, K // 2), 0x88, np.uint8)
    T = lambda v: torch.from_numpy(v).to(gpu)  # noqa: E731
    sx = np.ones(16, np.float32)
    zx = np.full(16, 8, np.int32)
    sw = np.ones(64, np.float32)
    sums = np.zeros(64, np.int32)
    out, raw = w4a4.matmul(T(a), T(b), T(sx), T(zx), T(sw), T(sums),
                           torch.empty(0, dtype=torch.float32, device=gpu), M, N,
                           fused=False, fp32=True)
    np.testing.assert_array_equal(raw.cpu().numpy(), native.gemm_raw(a, b, M, N))


@pytest.mark.parametrize("M,N,K,rot", [(16, 4096, 4096, 128), (2048, 4096, 4096, 128),
                                       (5, 11008, 4096, 0), (512, 11008, 4096, 128)])
def test_end_to_end_config_data(gpu, M, N, K, rot):
    """quantize -> pack_weight -> matmul on the config distributions vs the oracle."""
    print(f"end-to-end case M{M} N{N} K{K} rot{rot}", flush=True)
    x = activations(M, K, seed=0)
    w = weights(N, K, seed=1)
    T = lambda v: torch.from_numpy(v).to(gpu)  # noqa: E731
    pa, sx, zx = w4a4.quantize(T(x), 1.0, True, rot)
    pw, sw, sums = w4a4.pack_weight(T(w), 1.0, rot)
    out, raw = w4a4.matmul(pa, pw, sx, zx, sw, sums,
                           torch.empty(0, dtype=torch.float16, device=gpu), M, N, fused=False)
    pa_ref, sx_ref, zx_ref = native.quantize_rows(x.astype(np.float32), 1.0, rot)
    pw_ref, sw_ref, sums_ref = native.pack_weight(w.astype(np.float32), 1.0, rot)
    np.testing.assert_array_equal(pa.cpu().numpy(), pa_ref)
    np.testing.assert_array_equal(pw.cpu().numpy(), pw_ref)
    raw_ref = _oracle_raw(pa_ref, pw_ref, M, N)
    np.testing.assert_array_equal(raw.cpu().numpy(), raw_ref)
    out_ref = native.restore(raw_ref, sx_ref, zx_ref, sw_ref, sums_ref, None)
    np.testing.assert_array_equal(out.cpu().numpy(), out_ref)


@pytest.mark.parametrize("M,N,K", [(1, 8, 1048576), (65535, 8, 64), (3, 24, 262144)])
def test_matmul_size_limits(gpu, M, N, K):
    """The largest K (2^20, the quantize limit) and M (65535) the path accepts,
    random nibbles, raw accumulators against the oracle's integer GEMM."""
    print(f"matmul limits M{M} N{N} K{K}", flush=True)
    a, b, sx, zx, sw, sums = _operands(M, N, K, seed=M + N + K)
    T = lambda v: torch.from_numpy(v).to(gpu)  # noqa: E731
    out, raw = w4a4.matmul(T(a), T(b), T(sx), T(zx), T(sw), T(sums),
                           torch.empty(0, dtype=torch.float32, device=gpu), M, N,
                           fused=False, fp32=True)
    torch.cuda.synchronize()
    raw_ref = native.gemm_raw(a, b, M, N)
    np.testing.assert_array_equal(raw.cpu().numpy(), raw_ref)
    np.testing.assert_array_equal(out.cpu().numpy(),
                                  native.restore(raw_ref, sx, zx, sw, sums, None,
                                                 out_dtype=np.float32))
