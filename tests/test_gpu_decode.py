"""Fused decode linear (dscq_linear_decode) on the GPU.

The fused kernel quantizes the few activation rows inside every workgroup and
multiplies them with its weight stripe in the same launch.  Its output must
equal, bit for bit, the two-launch path (quantize, then matmul) and the
oracle's whole linear (quantize_rows -> gemm_raw -> restore), at the decode
shapes (M <= 4, K = 4096; M = 1 up to K = 12288) and at the edges: K not a
multiple of 128 (no rotation), KB % 64 == 32 (a half-empty last k block),
N not a multiple of 16, clip < 1 (clamped codes), fp32 input and output,
bias, and rows that are all zero, constant, or hold exact rounding ties.
"""
import numpy as np
import pytest
import torch

from dscquant_amd import w4a4
from dscquant_amd.core.linear import QuantLinear
from oracle import native
from tests.conftest import activations, weights

pytestmark = pytest.mark.gpu

CASES = [
    # M, K, N, rot, clip, x dtype, bias, fp32 out
    (1, 4096, 4096, 128, 1.0, torch.float16, False, False),
    (4, 4096, 4096, 128, 1.0, torch.float16, True, False),
    (3, 4096, 11008, 128, 0.9, torch.float16, False, False),
    (2, 8192, 1000, 128, 1.0, torch.float16, False, True),
    (1, 11008, 4096, 128, 1.0, torch.float16, True, False),
    (3, 1000, 264, 0, 1.0, torch.float32, True, True),
    (2, 192, 40, 0, 0.5, torch.float16, False, False),
    (1, 64, 8, 0, 1.0, torch.float16, False, False),
    (4, 2048, 24, 128, 1.0, torch.float32, False, False),
    # M <= 2 (the v_dot8 form): the longest row (K = 12288, twelve 16-byte weight
    # pieces per lane), and fp32 in / out with bias at N = 11008
    (1, 12288, 520, 128, 1.0, torch.float16, True, False),
    (2, 4096, 11008, 128, 1.0, torch.float32, True, True),
    # M >= 3 with two or three 16-column tiles per workgroup (up to three
    # tiles per CU: N = 11008 three, ragged N = 8200 three with a short last
    # workgroup, N = 6000 two) and two past that (N = 14336)
    (4, 4096, 11008, 128, 1.0, torch.float16, True, False),
    (3, 5376, 8200, 0, 0.9, torch.float16, False, True),
    (4, 2048, 6000, 128, 1.0, torch.float32, True, False),
    (4, 4096, 14336, 128, 0.8, torch.float16, False, False),
    # M <= 2 with several tiles per workgroup (up to four weight pieces per
    # lane): N = 14336 two, ragged N = 8200 three; K = 8192 keeps one (N = 8192)
    (1, 4096, 14336, 128, 1.0, torch.float16, True, False),
    (2, 2048, 8200, 0, 0.7, torch.float32, False, True),
    (1, 8192, 8192, 128, 1.0, torch.float16, False, False),
]


def _inputs(M, K, N, xdtype, bias, fp32, seed):
    x = activations(M, K, seed=seed).astype(np.float32)
    if M >= 2:
        x[1] = 0.0                      # all-zero row: scale 1e-8, zero 0
    if M >= 3:
        x[2] = 0.25                     # constant row
    w = weights(N, K, seed=seed + 1)
    b = (np.random.default_rng(seed).standard_normal(N) * 0.1).astype(
        np.float32 if fp32 else np.float16) if bias else None
    return x.astype(np.float16 if xdtype == torch.float16 else np.float32), w, b


@pytest.mark.parametrize("M,K,N,rot,clip,xdtype,bias,fp32", CASES)
def test_linear_decode_matches_two_launch_path_and_oracle(gpu, M, K, N, rot, clip, xdtype,
                                                          bias, fp32):
    print(f"linear_decode case M{M} K{K} N{N} rot{rot} clip{clip} {xdtype} bias{bias} "
          f"fp32{fp32}", flush=True)
    assert w4a4.linear_decode_supported(M, K)
    x, w, b = _inputs(M, K, N, xdtype, bias, fp32, seed=M * 7 + K)
    xt = torch.from_numpy(x).to(gpu)
    pw, sw, sums = w4a4.pack_weight(torch.from_numpy(w).to(gpu), 1.0, rot)
    out_dtype = torch.float32 if fp32 else torch.float16
    bt = (torch.empty(0, dtype=out_dtype, device=gpu) if b is None
          else torch.from_numpy(b).to(gpu))
    y = w4a4.linear_decode(xt, clip, rot, pw, sw, sums, bt, N, fp32)
    pa, sx, zx = w4a4.quantize(xt, clip, True, rot)
    y2, _ = w4a4.matmul(pa, pw, sx, zx, sw, sums, bt, M, N, True, False, fp32)
    torch.cuda.synchronize()
    assert torch.equal(y, y2)
    ref, *_ = native.linear_w4a4(x.astype(np.float32), w.astype(np.float32), b, clip_a=clip,
                                 rotate_block=rot,
                                 out_dtype=np.float32 if fp32 else np.float16)
    np.testing.assert_array_equal(y.cpu().numpy(), ref)


def test_linear_decode_exact_ties(gpu):
    """Rows with elements at exact x / scale + zero = k + 0.5 ties (the guard's
    exact-division path), no rotation: bit-exact against the oracle."""
    M, K, N = 2, 512, 64
    x = np.zeros((M, K), np.float32)
    # scale = (hi - lo) / 15 = 1 with lo = -7.5 (zero = rne(7.5) = 8), hi = 7.5;
    # interior elements at j + 0.5 - 8 for j = 0..14 hit exact ties.
    x[:, 0], x[:, 1] = -7.5, 7.5
    vals = np.arange(15, dtype=np.float32) + 0.5 - 8.0
    x[:, 2:2 + 15 * 30] = np.tile(vals, 30)
    x[1] *= 0.5
    xt = torch.from_numpy(x.astype(np.float16)).to(gpu)
    w = weights(N, K, seed=3)
    pw, sw, sums = w4a4.pack_weight(torch.from_numpy(w).to(gpu), 1.0, 0)
    bt = torch.empty(0, dtype=torch.float16, device=gpu)
    y = w4a4.linear_decode(xt, 1.0, 0, pw, sw, sums, bt, N, False)
    torch.cuda.synchronize()
    ref, *_ = native.linear_w4a4(x.astype(np.float16).astype(np.float32), w.astype(np.float32))
    np.testing.assert_array_equal(y.cpu().numpy(), ref)


class _Cfg:
    weight_bits = 4
    activation_bits = 4


@pytest.mark.parametrize("M,rot", [(1, 128), (4, 0)])
def test_quant_linear_uses_fused_decode(gpu, monkeypatch, M, rot):
    """QuantLinear's integer path takes the fused kernel for a few tokens and
    returns the oracle's output (3-D input, bias)."""
    calls = []
    real = w4a4.linear_decode
    monkeypatch.setattr(w4a4, "linear_decode", lambda *a, **k: calls.append(1) or real(*a, **k))
    K, N = 4096, 512
    lin = torch.nn.Linear(K, N, bias=True)
    with torch.no_grad():
        lin.weight.copy_(torch.from_numpy(weights(N, K, seed=5).astype(np.float32)))
        lin.bias.copy_(torch.randn(N, generator=torch.Generator().manual_seed(6)) * 0.1)
    lin = lin.half().to(gpu)
    q = QuantLinear(lin, _Cfg())
    q.enabled = True
    q.rotate_block = rot
    x = torch.from_numpy(activations(M, K, seed=9)).to(gpu).reshape(1, M, K)
    with torch.no_grad():
        y = q(x)
    torch.cuda.synchronize()
    assert y.shape == (1, M, N) and y.dtype == torch.float16
    assert calls == [1]
    ref, *_ = native.linear_w4a4(x[0].float().cpu().numpy(), lin.weight.float().cpu().numpy(),
                                 lin.bias.cpu().numpy(), rotate_block=rot)
    np.testing.assert_array_equal(y[0].cpu().numpy(), ref)


def test_linear_decode_rejects_large_inputs(gpu):
    assert not w4a4.linear_decode_supported(5, 4096)
    assert not w4a4.linear_decode_supported(2, 11008)
    assert not w4a4.linear_decode_supported(1, 4100)     # K % 8 != 0
    x = torch.zeros(5, 4096, dtype=torch.float16, device=gpu)
    pw = torch.zeros(8, 2048, dtype=torch.uint8, device=gpu)
    sw = torch.zeros(8, device=gpu)
    sums = torch.zeros(8, dtype=torch.int32, device=gpu)
    with pytest.raises(RuntimeError, match="exceed the fused decode kernel"):
        w4a4.linear_decode(x, 1.0, 0, pw, sw, sums,
                           torch.empty(0, dtype=torch.float16, device=gpu), 8)
