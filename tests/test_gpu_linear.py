"""QuantLinear on the GPU: the integer W4A4 forward against the oracle.

The module keeps the reference's state and fold rules; when enabled at 4/4
bits its output must equal the oracle's quantize -> GEMM -> epilogue chain bit
for bit, and sit within fp16 tolerance of the reference's fake-quant
composition (which rounds x_hat and W_hat to fp16 before F.linear).
"""
import numpy as np
import pytest
import torch

from dscquant_amd.core.linear import QuantLinear
from oracle import fakequant, native
from tests.conftest import activations, weights

pytestmark = pytest.mark.gpu


class Cfg:
    def __init__(self, wb=4, ab=4):
        self.weight_bits = wb
        self.activation_bits = ab


def _layer(N, K, gpu, bias=True, dtype=torch.float16):
    base = torch.nn.Linear(K, N, bias=bias)
    with torch.no_grad():
        base.weight.copy_(torch.from_numpy(weights(N, K, seed=1).astype(np.float32)))
        if bias:
            base.bias.copy_(torch.randn(N, generator=torch.Generator().manual_seed(3)) * 0.1)
    return base.to(device=gpu, dtype=dtype)


@pytest.mark.parametrize("M,N,K,rot,bias", [(16, 4096, 4096, 0, True), (16, 4096, 4096, 128, False),
                                            (3, 1024, 512, 0, True), (257, 768, 1024, 128, True)])
def test_quant_linear_w4a4_matches_oracle(gpu, M, N, K, rot, bias):
    print(f"QuantLinear case M{M} N{N} K{K} rot{rot} bias{bias}", flush=True)
    layer = QuantLinear(_layer(N, K, gpu, bias), Cfg())
    layer.enabled = True
    layer.rotate_block = rot
    x = activations(M, K, seed=0)
    with torch.no_grad():
        y = layer(torch.from_numpy(x).to(gpu).reshape(1, M, K))
    assert y.shape == (1, M, N) and y.dtype == torch.float16
    w = layer.base.weight.detach().float().cpu().numpy()
    b = layer.base.bias.detach().cpu().numpy() if bias else None
    out_ref, *_ = native.linear_w4a4(x.astype(np.float32), w, b, rotate_block=rot)
    np.testing.assert_array_equal(y[0].cpu().numpy(), out_ref)
    if rot == 0:
        fq = fakequant.forward(torch.from_numpy(x).float(), torch.from_numpy(w),
                               None if b is None else torch.from_numpy(b).float()).numpy()
        assert np.abs(y[0].cpu().float().numpy() - fq).max() <= 2e-3 * np.abs(fq).max()
    # the packed weight is cached until the weight changes
    p1 = layer.packed_weight()[0]
    assert layer.packed_weight()[0] is p1
    with torch.no_grad():
        layer.base.weight.mul_(2)
    assert layer.packed_weight()[0] is not p1


def test_quant_linear_fp32_and_bf16_inputs(gpu):
    layer = QuantLinear(_layer(256, 512, gpu, True, torch.float32), Cfg())
    layer.enabled = True
    x = activations(8, 512, seed=4, dtype=np.float32)
    with torch.no_grad():
        y = layer(torch.from_numpy(x).to(gpu))
        yb = layer(torch.from_numpy(x).to(gpu).to(torch.bfloat16))
    assert y.dtype == torch.float32 and yb.dtype == torch.bfloat16
    w = layer.base.weight.detach().cpu().numpy()
    b = layer.base.bias.detach().cpu().numpy()
    out_ref, *_ = native.linear_w4a4(x, w, b, out_dtype=np.float32)
    np.testing.assert_array_equal(y.cpu().numpy(), out_ref)


def test_quant_linear_other_bit_widths_use_gpu_codes(gpu):
    layer = QuantLinear(_layer(128, 256, gpu, True, torch.float32), Cfg(8, 6))
    layer.enabled = True
    x = torch.from_numpy(activations(4, 256, seed=5, dtype=np.float32)).to(gpu)
    with torch.no_grad():
        y = layer(x)
    w = layer.base.weight.detach().cpu()
    xa = fakequant.quantize_activation(x.cpu(), 6)
    wq = fakequant.quantize_weight(w, 8)
    ref = torch.nn.functional.linear(xa, wq, layer.base.bias.detach().cpu())
    torch.testing.assert_close(y.cpu(), ref, rtol=1e-5, atol=1e-5)


def test_quant_linear_w4a4_with_learned_transforms(gpu):
    """Folds of core/linear.py:22-46 (per-head rotation on the o projection, diagonal
    scaling on up / down) on the integer path: the module's folded weight agrees with
    the fold formula in fp32 tolerance (matmul order is the device's), and the output
    is bit-exact against the oracle fed that same folded weight."""

    class Rot(torch.nn.Module):
        def __init__(self, heads, head_dim):
            super().__init__()
            self.heads, self.head_dim = heads, head_dim
            q, _ = torch.linalg.qr(torch.randn(heads, head_dim, head_dim,
                                               generator=torch.Generator().manual_seed(5)))
            self.m = q.to(gpu)

        def matrices(self):
            return self.m

    class Scl(torch.nn.Module):
        def __init__(self, n):
            super().__init__()
            self.s = (torch.rand(n, generator=torch.Generator().manual_seed(6)) + 0.5).to(gpu)

        def diagonal(self):
            return self.s

    M = 24
    cases = [(Rot(8, 64), "o", 512, 512), (Scl(1024), "up", 1024, 512), (Scl(512), "down", 256, 512)]
    for interface, role, N, K in cases:
        print(f"QuantLinear fold case role {role} N{N} K{K}", flush=True)
        layer = QuantLinear(_layer(N, K, gpu, bias=False), Cfg(), interface, role)
        layer.enabled = True
        x = torch.from_numpy(activations(M, K, seed=8)).to(gpu)
        with torch.no_grad():
            y = layer(x)
        w_fold, _ = layer.transformed()
        w0 = layer.base.weight.float()
        if role == "o":
            R = interface.m.float()
            ref = torch.einsum("ohd,hde->ohe", w0.reshape(N, 8, 64), R).reshape(N, K)
        elif role == "up":
            ref = w0 / interface.s[:, None]
        else:
            ref = w0 * interface.s[None, :]
        torch.testing.assert_close(w_fold.float(), ref.half().float(), rtol=2e-3, atol=2e-5)
        out_ref, *_ = native.linear_w4a4(x.float().cpu().numpy(),
                                         w_fold.float().cpu().numpy(), None)
        np.testing.assert_array_equal(y.cpu().numpy(), out_ref)
