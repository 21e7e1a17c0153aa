"""The product path captured in a HIP graph (torch.cuda.CUDAGraph), as bench.py
times it: every replay must read the current contents of its input buffers and
give, bit for bit, what eager calls give on the same data.  Each replay is
followed by eager work on the same stream and a synchronisation, and the inputs
change between replays.  Covered: rotate+quantize+pack -> pipelined GEMM
(prefill shape class, the prefill shape itself) and -> wide-tile GEMM (forced
at both tile widths, and by the automatic rule), quantize -> skinny-M GEMM (16
tokens, one and three column tiles per workgroup), the fused decode kernel (one
and three tiles per workgroup, both product forms), the SiLU-gated
requantization, and the gated GEMM on the wide-tile and pipelined kernels.
"""
import numpy as np
import pytest
import torch

from dscquant_amd import w4a4
from tests.conftest import activations, weights

pytestmark = pytest.mark.gpu


def _capture(fn, static_in):
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn(static_in)  # warm the captured path outside capture
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = fn(static_in)
    return g, out


def _replay_and_compare(fn, inputs):
    static_in = inputs[0].clone()
    g, static_out = _capture(fn, static_in)
    for rep, x in enumerate(inputs + inputs[::-1]):
        static_in.copy_(x)
        g.replay()
        eager = fn(x)
        torch.cuda.synchronize()
        outs = static_out if isinstance(static_out, (list, tuple)) else [static_out]
        refs = eager if isinstance(eager, (list, tuple)) else [eager]
        for o, r in zip(outs, refs):
            assert torch.equal(o, r), f"replay {rep} differs from eager"


@pytest.mark.parametrize("M,K,N", [(256, 4096, 1024), (16, 4096, 4096), (128, 11008, 4096),
                                   (16, 4096, 11008), (2048, 4096, 4096)])
def test_quantize_matmul_graph(gpu, M, K, N):
    print(f"graph quantize+matmul M{M} K{K} N{N}", flush=True)
    pw, sw, sums = w4a4.pack_weight(torch.from_numpy(weights(N, K, seed=9)).to(gpu), 1.0, 128)
    bias = torch.empty(0, dtype=torch.float16, device=gpu)

    def run(x):
        pa, sx, zx = w4a4.quantize(x, 1.0, True, 128)
        out, _ = w4a4.matmul(pa, pw, sx, zx, sw, sums, bias, M, N)
        return [out, pa, sx, zx]

    xs = [torch.from_numpy(activations(M, K, seed=s).astype(np.float16)).to(gpu)
          for s in (1, 2, 3)]
    _replay_and_compare(run, xs)


@pytest.mark.parametrize("M,K,N,which,use_bias", [(512, 4096, 2048, 3, False),
                                                   (300, 2048, 1032, 4, True),
                                                   (4096, 4096, 4096, 0, False)])
def test_quantize_wide_matmul_graph(gpu, M, K, N, which, use_bias):
    """The wide-tile GEMM (LDS DMA) captured and replayed: forced with 256 x 256
    or 256 x 128 tiles, and chosen by the automatic rule at 4096 x 4096 x 4096."""
    from tests.test_gpu_wide import gemm_kernel
    print(f"graph quantize+wide matmul M{M} K{K} N{N} kernel{which} bias{use_bias}", flush=True)
    pw, sw, sums = w4a4.pack_weight(torch.from_numpy(weights(N, K, seed=12)).to(gpu), 1.0, 128)
    bias = (torch.from_numpy((np.random.default_rng(1).standard_normal(N) * 0.1)
                             .astype(np.float16)).to(gpu) if use_bias
            else torch.empty(0, dtype=torch.float16, device=gpu))

    def run(x):
        with gemm_kernel(which):
            pa, sx, zx = w4a4.quantize(x, 1.0, True, 128)
            out, _ = w4a4.matmul(pa, pw, sx, zx, sw, sums, bias, M, N)
        return [out, pa, sx, zx]

    xs = [torch.from_numpy(activations(M, K, seed=s).astype(np.float16)).to(gpu)
          for s in (7, 8, 9)]
    _replay_and_compare(run, xs)


@pytest.mark.parametrize("M,N", [(2, 4096), (4, 11008), (1, 11008)])
def test_linear_decode_graph(gpu, M, N):
    K = 4096
    print(f"graph linear_decode M{M} K{K} N{N}", flush=True)
    assert w4a4.linear_decode_supported(M, K)
    pw, sw, sums = w4a4.pack_weight(torch.from_numpy(weights(N, K, seed=5)).to(gpu), 1.0, 128)
    bias = torch.from_numpy((np.random.default_rng(0).standard_normal(N) * 0.1)
                            .astype(np.float16)).to(gpu)

    def run(x):
        return w4a4.linear_decode(x, 1.0, 128, pw, sw, sums, bias, N)

    xs = [torch.from_numpy(activations(M, K, seed=s).astype(np.float16)).to(gpu)
          for s in (4, 5, 6)]
    _replay_and_compare(run, xs)


def test_silu_mul_quantize_graph(gpu):
    M, N = 64, 1024
    print(f"graph silu_mul_quantize M{M} N{N}", flush=True)

    def run(gu):
        return w4a4.silu_mul_quantize(gu, 1.0, 128, return_h=True)

    rng = np.random.default_rng(7)
    xs = [torch.from_numpy((rng.standard_normal((M, 2 * N)) * 2).astype(np.float16)).to(gpu)
          for _ in range(3)]
    _replay_and_compare(run, xs)


@pytest.mark.parametrize("M,K,N,which", [(512, 4096, 2048, 3), (512, 4096, 2048, 2)])
def test_quantize_matmul_silu_mul_graph(gpu, M, K, N, which):
    """The gated GEMM (gate|up with the SiLU-gated epilogue) captured and
    replayed on the wide-tile kernel (forced) and on the pipelined kernel."""
    from tests.test_gpu_wide import gemm_kernel
    print(f"graph quantize+matmul_silu_mul M{M} K{K} N{N} kernel{which}", flush=True)
    pg, swg, sg = w4a4.pack_weight(torch.from_numpy(weights(N, K, seed=31)).to(gpu), 1.0, 0)
    pu, swu, su = w4a4.pack_weight(torch.from_numpy(weights(N, K, seed=32)).to(gpu), 1.0, 0)
    il = w4a4.interleave_gate_up
    b, sw, sums = il(pg, pu), il(swg, swu), il(sg, su)
    empty = torch.empty(0, dtype=torch.float16, device=gpu)

    def run(x):
        with gemm_kernel(which):
            pa, sx, zx = w4a4.quantize(x, 1.0, True, 0)
            h = w4a4.matmul_silu_mul(pa, b, sx, zx, sw, sums, empty, M, N)
        return [h, pa]

    xs = [torch.from_numpy(activations(M, K, seed=s).astype(np.float16)).to(gpu)
          for s in (10, 11, 12)]
    _replay_and_compare(run, xs)
