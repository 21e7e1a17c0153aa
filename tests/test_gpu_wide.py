"""GPU parity of the wide-tile GEMM kernel (256 x 256 and 256 x 128 tiles, one
wave per SIMD, LDS-DMA operand loads; dscq_set_gemm_kernel selects it, and
its tile width, for any shape it applies to).

Its fp16 outputs are compared bit for bit with the oracle's epilogue on the
oracle's int32 accumulators (kernel/w4a4.cu:70-161) at ragged shapes (partial
tiles in M and N, one to five K slices, tiny M), with and without bias, and
with the largest accumulator and zero-point-correction magnitudes, and at
seeded random shapes inside its contract; at the
70B shapes, where the automatic choice takes it, its whole output is compared
with the pipelined kernel's (itself checked against the oracle there).
"""
import numpy as np
import pytest
import torch

from dscquant_amd import _lib, w4a4
from oracle import native
from tests.conftest import sweep_size
from tests.test_gpu_matmul import _dequant64, _operands, _oracle_raw

pytestmark = pytest.mark.gpu


class gemm_kernel:
    """Selects the GEMM kernel for this thread (dscq_set_gemm_kernel) for a block."""

    def __init__(self, which):
        self.which = which

    def __enter__(self):
        self.prev = _lib.lib().dscq_set_gemm_kernel(self.which)
        assert self.prev >= 0

    def __exit__(self, *exc):
        _lib.lib().dscq_set_gemm_kernel(self.prev)


WIDE_CASES = [
    # (M, N, K, bias)
    (256, 256, 256, False),     # one tile, one slice
    (256, 264, 512, True),      # N past a whole tile by 8 columns, two slices
    (300, 520, 768, True),      # partial tiles in M and N, three slices
    (512, 1024, 4096, False),   # sixteen slices
    (1000, 1032, 1280, True),   # five slices, ragged both ways
    (64, 256, 256, False),      # M = 64: one tile mostly past the rows
    (72, 4104, 512, True),      # padded rows (MP = 72), 17 column tiles
]


@pytest.mark.parametrize("width", [256, 128])
@pytest.mark.parametrize("M,N,K,use_bias", WIDE_CASES,
                         ids=[f"M{c[0]}-N{c[1]}-K{c[2]}-bias{int(c[3])}" for c in WIDE_CASES])
def test_wide_kernel_matches_oracle(gpu, M, N, K, use_bias, width):
    print(f"wide case M{M} N{N} K{K} bias{use_bias} width{width}", flush=True)
    a, b, sx, zx, sw, sums = _operands(M, N, K, seed=11 * M + N + 3 * K)
    bias = np.random.default_rng(K + 1).standard_normal(N).astype(np.float16) if use_bias else None
    T = lambda v: torch.from_numpy(v).to(gpu)  # noqa: E731
    tbias = T(bias) if use_bias else torch.empty(0, dtype=torch.float16, device=gpu)
    with gemm_kernel(3 if width == 256 else 4):
        out, raw = w4a4.matmul(T(a), T(b), T(sx), T(zx), T(sw), T(sums), tbias, M, N,
                               fused=True)
    with gemm_kernel(2):
        out_pipe, _ = w4a4.matmul(T(a), T(b), T(sx), T(zx), T(sw), T(sums), tbias, M, N,
                                  fused=True)
    torch.cuda.synchronize()
    assert raw.numel() == 0
    raw_ref = _oracle_raw(a, b, M, N)
    out_ref = native.restore(raw_ref, sx, zx, sw, sums, bias)
    got = out.cpu().numpy()
    np.testing.assert_array_equal(got, out_ref)
    np.testing.assert_array_equal(out_pipe.cpu().numpy(), out_ref)
    exact = _dequant64(raw_ref, sx, zx, sw, sums, bias, M, N)
    rel = np.abs(got.astype(np.float64) - exact) / np.maximum(np.abs(exact), 1e-30)
    big = np.abs(exact) > 1e-2
    assert rel[big].max() <= 1e-3


def _random_cases(n, seed):
    """Seeded shapes inside the wide kernel's contract (N % 8 == 0, K a
    multiple of 256): ragged M and N, 1-39 slices, either tile width."""
    rng = np.random.default_rng(seed)
    out = []
    while len(out) < n:
        M = int(rng.integers(1, 1400))
        N = int(rng.integers(1, 1600)) * 8
        K = int(rng.integers(1, 40)) * 256
        if M * N * K > 2.0e9:
            continue
        out.append((M, N, K, bool(rng.random() < 0.5), int(rng.choice([256, 128]))))
    return out


RANDOM_CASES = _random_cases(*sweep_size(12, 8086))


@pytest.mark.parametrize("M,N,K,use_bias,width", RANDOM_CASES,
                         ids=[f"M{c[0]}-N{c[1]}-K{c[2]}-w{c[4]}" for c in RANDOM_CASES])
def test_wide_kernel_random_shapes(gpu, M, N, K, use_bias, width):
    test_wide_kernel_matches_oracle(gpu, M, N, K, use_bias, width)


@pytest.mark.parametrize("width", [256, 128])
@pytest.mark.parametrize("zero_point", [0, 8, 15])
def test_wide_kernel_extreme_magnitudes(gpu, zero_point, width):
    """K = 65536 (the kernel's limit) with all -8 x -8 and -8 x +7 products: the
    largest scaled accumulators (2^30), and zero-points 0 / 15 with the largest
    code sums (the (8 - zx) * 256 * sums term at 2^29.8)."""
    M, N, K = 256, 264, 65536
    print(f"wide extreme case zx={zero_point}", flush=True)
    a = np.full((M, K // 2), 0x88, np.uint8)
    b = np.full((N, K // 2), 0x88, np.uint8)
    b[N // 2:] = 0x77
    sx = np.full(M, 2.0 ** -12, np.float32)
    zx = np.full(M, zero_point, np.int32)
    sw = np.full(N, 2.0 ** -10, np.float32)
    sums = np.where(np.arange(N) < N // 2, -7 * K, 7 * K).astype(np.int32)
    T = lambda v: torch.from_numpy(v).to(gpu)  # noqa: E731
    with gemm_kernel(3 if width == 256 else 4):
        out, _ = w4a4.matmul(T(a), T(b), T(sx), T(zx), T(sw), T(sums),
                             torch.empty(0, dtype=torch.float16, device=gpu), M, N, fused=True)
    torch.cuda.synchronize()
    raw_ref = np.where(np.arange(N) < N // 2, 64 * K, -56 * K).astype(np.int32)[None, :].repeat(M, 0)
    np.testing.assert_array_equal(out.cpu().numpy(), native.restore(raw_ref, sx, zx, sw, sums))


@pytest.mark.parametrize("M,N,K", [(4096, 8192, 8192), (4096, 8192, 28672)])
def test_wide_kernel_whole_output_at_70b_shapes(gpu, M, N, K):
    """The automatic choice takes the wide-tile kernel at these shapes (two or
    more rounds of 256 x 256 tiles): its whole fp16 output equals the pipelined
    kernel's, and a seeded 64 x 64 sample equals the oracle's."""
    print(f"wide 70B case M{M} N{N} K{K}", flush=True)
    rng = np.random.default_rng(M + N + K)
    a = rng.integers(0, 256, size=(M, K // 2), dtype=np.uint8)
    b = rng.integers(0, 256, size=(N, K // 2), dtype=np.uint8)
    sx = (rng.random(M).astype(np.float32) + 0.5) * 0.05
    zx = rng.integers(0, 16, size=M).astype(np.int32)
    sw = (rng.random(N).astype(np.float32) + 0.5) * 0.002
    sums = rng.integers(-20000, 20000, size=N).astype(np.int32)
    T = lambda v: torch.from_numpy(v).to(gpu)  # noqa: E731
    args = (T(a), T(b), T(sx), T(zx), T(sw), T(sums),
            torch.empty(0, dtype=torch.float16, device=gpu), M, N)
    out = w4a4.matmul(*args, fused=True)[0]
    with gemm_kernel(2):
        out_pipe = w4a4.matmul(*args, fused=True)[0]
    torch.cuda.synchronize()
    assert torch.equal(out, out_pipe)
    rows = np.sort(rng.choice(M, 64, replace=False))
    cols = np.sort(rng.choice(N, 64, replace=False))
    KP = K
    ia = native.unpack_int4(a[rows], KP).astype(np.int64)
    ib = native.unpack_int4(b[cols], KP).astype(np.int64)
    raw_ref = (ia @ ib.T).astype(np.int32)
    np.testing.assert_array_equal(out.cpu().numpy()[np.ix_(rows, cols)],
                                  native.restore(raw_ref, sx[rows], zx[rows], sw[cols], sums[cols]))


def test_set_gemm_kernel_contract(gpu):
    L = _lib.lib()
    prev = L.dscq_set_gemm_kernel(1)
    assert L.dscq_set_gemm_kernel(2) == 1
    assert L.dscq_set_gemm_kernel(0) == 2
    assert L.dscq_set_gemm_kernel(5) == -1
    L.dscq_set_gemm_kernel(prev)
