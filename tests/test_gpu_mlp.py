"""SiLU-gated W4A4 MLP block on the GPU.

The gated activation h = fp16(fp16(silu(g)) * u) depends on exp, whose last
bit differs between the GPU's and the CPU's libraries, so h is checked
against torch's CPU fp16 composition within a few fp16 ulps (and equal on
more than 99% of the elements).  Everything after
h is integer or fixed-order fp32 and is checked bit for bit against the
oracle applied to the kernel's own h: packed codes, scales and zero-points of
the down projection's input (with its online rotation) and the block output.
"""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

from dscquant_amd import w4a4
from dscquant_amd.core.linear import QuantLinear
from dscquant_amd.core.mlp import QuantMLP
from oracle import native
from tests.conftest import activations, weights

pytestmark = pytest.mark.gpu


def _h_reference(gu: torch.Tensor) -> torch.Tensor:
    """An fp16 model's act_fn(gate) * up on the CPU."""
    N = gu.shape[1] // 2
    g, u = gu[:, :N].cpu(), gu[:, N:].cpu()
    return F.silu(g.float()).half() * u


@pytest.mark.parametrize("M,N,rot", [(1, 512, 0), (16, 11008, 128), (37, 1024, 128),
                                     (512, 11008, 128), (64, 640, 0)])
def test_silu_mul_quantize_matches_oracle(gpu, M, N, rot):
    print(f"silu_mul_quantize case M{M} N{N} rot{rot}", flush=True)
    g = torch.Generator().manual_seed(M + N)
    gu = (torch.randn(M, 2 * N, generator=g) * 2.0).half().to(gpu)
    packed, sx, zx, h = w4a4.silu_mul_quantize(gu, 1.0, rot, return_h=True)
    torch.cuda.synchronize()
    h_ref = _h_reference(gu)
    hk = h.cpu()
    # A last-bit exp difference can flip the fp16 rounding of silu(g), which
    # the product carries into h as up to ~2.5 fp16 ulps; exact elsewhere.
    diff = (hk.float() - h_ref.float()).abs()
    assert (diff <= torch.maximum(hk.float().abs(), torch.tensor(6.1e-5)) * 2.0 ** -8).all()
    assert (diff == 0).float().mean() > 0.99
    # codes of the kernel's own h: bit-exact against the oracle
    pa, sx_ref, zx_ref = native.quantize_rows(hk.float().numpy(), 1.0, rot)
    np.testing.assert_array_equal(packed.cpu().numpy(), pa)
    np.testing.assert_array_equal(sx.cpu().numpy(), sx_ref)
    np.testing.assert_array_equal(zx.cpu().numpy(), zx_ref)
    # without the h output the kernel writes the same codes
    p2, s2, z2 = w4a4.silu_mul_quantize(gu, 1.0, rot)
    assert torch.equal(p2, packed) and torch.equal(s2, sx) and torch.equal(z2, zx)


class Cfg:
    weight_bits = 4
    activation_bits = 4


def _deinterleave(gu_i, N):
    """Columns of a GEMM against interleave_gate_up weights back to [gate | up]."""
    M = gu_i.shape[0]
    blocks = gu_i.reshape(M, N // 64, 2, 64)
    return torch.cat([blocks[:, :, 0].reshape(M, N), blocks[:, :, 1].reshape(M, N)], dim=1)


@pytest.mark.parametrize("M,K,N,bias", [(1, 4096, 11008, False), (5, 1088, 640, True),
                                        (16, 4096, 2816, False), (17, 1000, 1024, True),
                                        (64, 4096, 11008, False), (300, 1088, 64, True),
                                        (512, 4096, 11008, True), (96, 1088, 11008, True)])
def test_matmul_silu_mul_matches_unfused_path(gpu, M, K, N, bias):
    """The gated GEMM's h equals the [M, 2N] GEMM + silu_mul_quantize path's h bit
    for bit (the skinny-M kernel for M <= 16, the tiled kernel above; K with a
    partial last slice; gate/up bias), and quantize(h) its packed output."""
    print(f"matmul_silu_mul case M{M} K{K} N{N} bias{bias}", flush=True)
    x = torch.from_numpy(activations(M, K, seed=M + K)).to(gpu)
    wg = torch.from_numpy(weights(N, K, seed=11)).to(gpu)
    wu = torch.from_numpy(weights(N, K, seed=12)).to(gpu)
    pg, swg, sg = w4a4.pack_weight(wg, 1.0, 0)
    pu, swu, su = w4a4.pack_weight(wu, 1.0, 0)
    gen = torch.Generator().manual_seed(N)
    bg = (torch.randn(N, generator=gen) * 0.1).half().to(gpu) if bias else None
    bu = (torch.randn(N, generator=gen) * 0.1).half().to(gpu) if bias else None
    empty = torch.empty(0, dtype=torch.float16, device=gpu)
    pa, sx, zx = w4a4.quantize(x, 1.0, True, 0)
    gu, _ = w4a4.matmul(pa, torch.cat([pg, pu]), sx, zx, torch.cat([swg, swu]),
                        torch.cat([sg, su]), torch.cat([bg, bu]) if bias else empty, M, 2 * N)
    p_ref, s_ref, z_ref, h_ref = w4a4.silu_mul_quantize(gu, 1.0, 128 if N % 128 == 0 else 0,
                                                        return_h=True)
    il = w4a4.interleave_gate_up
    h = w4a4.matmul_silu_mul(pa, il(pg, pu), sx, zx, il(swg, swu), il(sg, su),
                             il(bg, bu) if bias else empty, M, N)
    p, s_, z = w4a4.quantize(h, 1.0, True, 128 if N % 128 == 0 else 0)
    torch.cuda.synchronize()
    assert torch.equal(h, h_ref)
    assert torch.equal(p, p_ref) and torch.equal(s_, s_ref) and torch.equal(z, z_ref)


@pytest.mark.parametrize("M,K,N,bias", [(512, 4096, 11008, True), (512, 4096, 11008, False),
                                        (1000, 2048, 2880, True), (64, 4096, 1024, False),
                                        (256, 512, 64, True), (300, 8192, 4160, False)])
def test_matmul_silu_mul_wide_tiles(gpu, M, K, N, bias):
    """The gated GEMM on the wide-tile kernel (dscq_set_gemm_kernel(3): 256 x 256
    tiles, each wave's 128 columns the gate and up rows of 64 outputs; partial
    tiles in M and N, one to 32 slices) gives the unfused path's h bit for bit,
    and the pipelined kernel's."""
    from tests.test_gpu_wide import gemm_kernel
    print(f"matmul_silu_mul wide case M{M} K{K} N{N} bias{bias}", flush=True)
    x = torch.from_numpy(activations(M, K, seed=M + 3 * K)).to(gpu)
    wg = torch.from_numpy(weights(N, K, seed=21)).to(gpu)
    wu = torch.from_numpy(weights(N, K, seed=22)).to(gpu)
    pg, swg, sg = w4a4.pack_weight(wg, 1.0, 0)
    pu, swu, su = w4a4.pack_weight(wu, 1.0, 0)
    gen = torch.Generator().manual_seed(N + 1)
    bg = (torch.randn(N, generator=gen) * 0.1).half().to(gpu) if bias else None
    bu = (torch.randn(N, generator=gen) * 0.1).half().to(gpu) if bias else None
    empty = torch.empty(0, dtype=torch.float16, device=gpu)
    pa, sx, zx = w4a4.quantize(x, 1.0, True, 0)
    gu, _ = w4a4.matmul(pa, torch.cat([pg, pu]), sx, zx, torch.cat([swg, swu]),
                        torch.cat([sg, su]), torch.cat([bg, bu]) if bias else empty, M, 2 * N)
    _, _, _, h_ref = w4a4.silu_mul_quantize(gu, 1.0, 0, return_h=True)
    il = w4a4.interleave_gate_up
    args = (pa, il(pg, pu), sx, zx, il(swg, swu), il(sg, su), il(bg, bu) if bias else empty, M, N)
    with gemm_kernel(3):
        h_wide = w4a4.matmul_silu_mul(*args)
    with gemm_kernel(2):
        h_pipe = w4a4.matmul_silu_mul(*args)
    torch.cuda.synchronize()
    assert torch.equal(h_wide, h_ref)
    assert torch.equal(h_pipe, h_ref)


def test_matmul_silu_mul_rejects_bad_shapes(gpu):
    pa = torch.zeros((64, 64), dtype=torch.uint8, device=gpu)
    sx = torch.ones(64, device=gpu)
    zx = torch.zeros(64, dtype=torch.int32, device=gpu)
    b = torch.zeros((192, 64), dtype=torch.uint8, device=gpu)  # N = 96: not a multiple of 64
    sw = torch.ones(192, device=gpu)
    sums = torch.zeros(192, dtype=torch.int32, device=gpu)
    with pytest.raises(RuntimeError, match="N % 64 == 0"):
        w4a4.matmul_silu_mul(pa, b, sx, zx, sw, sums, torch.empty(0, dtype=torch.float16,
                                                                  device=gpu), 64, 96)


def _linear(n_out, n_in, seed, gpu, bias=False):
    lin = torch.nn.Linear(n_in, n_out, bias=bias)
    with torch.no_grad():
        lin.weight.copy_(torch.from_numpy(weights(n_out, n_in, seed=seed).astype(np.float32)))
        if bias:
            lin.bias.copy_(torch.randn(n_out, generator=torch.Generator().manual_seed(seed)) * 0.1)
    return lin.half().to(gpu)


@pytest.mark.parametrize("M,K,N,bias", [(16, 1024, 2816, False), (128, 4096, 11008, False),
                                        (40, 512, 1024, True)])
def test_quant_mlp_matches_oracle(gpu, M, K, N, bias):
    print(f"QuantMLP case M{M} K{K} N{N} bias{bias}", flush=True)
    gate = QuantLinear(_linear(N, K, 1, gpu, bias), Cfg())
    up = QuantLinear(_linear(N, K, 2, gpu, bias), Cfg())
    down = QuantLinear(_linear(K, N, 3, gpu, bias), Cfg())
    for m in (gate, up, down):
        m.enabled = True
    down.rotate_block = 128
    mlp = QuantMLP(gate, up, down)
    x = torch.from_numpy(activations(M, K, seed=7)).to(gpu)
    with torch.no_grad():
        y = mlp(x)
    torch.cuda.synchronize()
    assert y.shape == (M, K) and y.dtype == torch.float16

    # the same chain through the oracle, starting from the kernel's own h
    xf = x.float().cpu().numpy()
    wg, wu, wd = (m.base.weight.float().cpu().numpy() for m in (gate, up, down))
    bgu = (np.concatenate([gate.base.bias.cpu().numpy(), up.base.bias.cpu().numpy()])
           if bias else None)
    gu_ref, *_ = native.linear_w4a4(xf, np.concatenate([wg, wu]), bgu)
    pa, sx, zx = w4a4.quantize(x, 1.0, True, 0)
    pgu, swgu, sgu, bgu_t, *_ = mlp.packed()
    gu, _ = w4a4.matmul(pa, pgu, sx, zx, swgu, sgu,
                        bgu_t if bgu_t is not None else torch.empty(0, dtype=torch.float16,
                                                                    device=gpu),
                        M, 2 * N, True, False, False)
    if mlp._gated_gemm():  # weights interleaved in 64-row blocks: back to [gate | up]
        gu = _deinterleave(gu, N)
    np.testing.assert_array_equal(gu.cpu().numpy(), gu_ref)
    _, _, _, h = w4a4.silu_mul_quantize(gu, 1.0, 128, return_h=True)
    bd = down.base.bias.cpu().numpy() if bias else None
    y_ref, *_ = native.linear_w4a4(h.float().cpu().numpy(), wd, bd, rotate_block=128)
    np.testing.assert_array_equal(y.cpu().numpy(), y_ref)

    # tolerance against the unquantized fp32 block (W4A4 error, not a parity bar)
    with torch.no_grad():
        xf_t = x.float().cpu()
        ref = F.linear(F.silu(F.linear(xf_t, torch.from_numpy(wg))) *
                       F.linear(xf_t, torch.from_numpy(wu)), torch.from_numpy(wd))
    rel = (y.float().cpu() - ref).norm() / ref.norm()
    assert rel < 0.5, rel
