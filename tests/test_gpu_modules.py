"""QuantLinear and QuantMLP as modules on the GPU: the decode workloads through
the module, learned interfaces with cached folds, HIP-graph capture of the
module forwards, and the non-fp16 MLP inputs.

Outputs are checked bit for bit against the oracle (oracle/dscq_oracle.c) fed
the module's own folded weight, or, where the two computations are the same
kernels on the same data, against a freshly built module.
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
from tests.interfaces import LearnedRotation, LearnedScaling

pytestmark = pytest.mark.gpu


class Cfg:
    weight_bits = 4
    activation_bits = 4


def _base(N, K, seed, gpu, bias=False, dtype=torch.float16):
    lin = torch.nn.Linear(K, N, bias=bias)
    with torch.no_grad():
        lin.weight.copy_(torch.from_numpy(weights(N, K, seed=seed).astype(np.float32)))
        if bias:
            lin.bias.copy_(torch.randn(N, generator=torch.Generator().manual_seed(seed)) * 0.1)
    return lin.to(device=gpu, dtype=dtype)


def _enabled(*mods, rot=0):
    for m in mods:
        m.enabled = True
        m.rotate_block = rot
    return mods


@pytest.fixture
def pack_calls(monkeypatch):
    calls = []
    real = w4a4.pack_weight

    def counting(*args, **kwargs):
        calls.append(args[0].shape)
        return real(*args, **kwargs)

    monkeypatch.setattr(w4a4, "pack_weight", counting)
    return calls


@pytest.mark.parametrize("M", [1, 4, 8, 16])
def test_quant_linear_decode_workloads_n11008(gpu, M):
    """The decode workloads' shapes (K=4096 -> N=11008, 128-wide rotation) through
    the module: the fused decode kernel (M <= 4) or quantize + skinny-M GEMM."""
    K, N = 4096, 11008
    print(f"QuantLinear decode case M{M} N{N} K{K}", flush=True)
    (layer,) = _enabled(QuantLinear(_base(N, K, 21, gpu, bias=True), Cfg()), rot=128)
    x = activations(M, K, seed=M)
    with torch.no_grad():
        y = layer(torch.from_numpy(x).to(gpu))
    torch.cuda.synchronize()
    w = layer.base.weight.float().cpu().numpy()
    b = layer.base.bias.cpu().numpy()
    out_ref, *_ = native.linear_w4a4(x.astype(np.float32), w, b, rotate_block=128)
    np.testing.assert_array_equal(y.cpu().numpy(), out_ref)


def test_learned_rotation_folds_and_packs_once(gpu, pack_calls):
    """An o projection with a learned per-head rotation: repeated forwards fold and
    pack once; an update of the interface refolds and repacks once; every output
    is bit-exact against the oracle fed the module's folded weight."""
    heads, hd, N, M = 4, 128, 1024, 48
    K = heads * hd
    rot = LearnedRotation(heads, hd, seed=3).to(gpu)
    (layer,) = _enabled(QuantLinear(_base(N, K, 22, gpu), Cfg(), rot, "o"), rot=128)
    x = torch.from_numpy(activations(M, K, seed=9)).to(gpu)
    with torch.no_grad():
        ys = [layer(x) for _ in range(3)]
    torch.cuda.synchronize()
    assert len(pack_calls) == 1 and rot._calls == 1
    assert all(torch.equal(y, ys[0]) for y in ys)
    with torch.no_grad():  # the cached fold (with grad enabled it would be refolded)
        w_fold = layer.transformed()[0]
    ref, *_ = native.linear_w4a4(x.float().cpu().numpy(), w_fold.float().cpu().numpy(), None,
                                 rotate_block=128)
    np.testing.assert_array_equal(ys[0].cpu().numpy(), ref)

    with torch.no_grad():
        rot.alpha.add_(0.5)
        y2 = layer(x)
        y3 = layer(x)
    torch.cuda.synchronize()
    assert len(pack_calls) == 2 and rot._calls == 2
    assert torch.equal(y2, y3) and not torch.equal(y2, ys[0])
    with torch.no_grad():
        w_fold2 = layer.transformed()[0]
    ref2, *_ = native.linear_w4a4(x.float().cpu().numpy(), w_fold2.float().cpu().numpy(), None,
                                  rotate_block=128)
    np.testing.assert_array_equal(y2.cpu().numpy(), ref2)


def test_mlp_follows_interface_updates(gpu, pack_calls):
    """QuantMLP with a learned scaling folded into up (rows) and down (columns):
    after the interface changes, the block equals a freshly built block."""
    K, N, M = 1024, 2816, 40
    scl = LearnedScaling(N, seed=4).to(gpu)

    def block():
        gate = QuantLinear(_base(N, K, 31, gpu, bias=True), Cfg())
        up = QuantLinear(_base(N, K, 32, gpu, bias=True), Cfg(), scl, "up")
        down = QuantLinear(_base(K, N, 33, gpu), Cfg(), scl, "down")
        _enabled(gate, up)
        _enabled(down, rot=128)
        return QuantMLP(gate, up, down)

    mlp = block()
    x = torch.from_numpy(activations(M, K, seed=10)).to(gpu)
    with torch.no_grad():
        y1 = mlp(x)
        mlp(x)
    assert len(pack_calls) == 3  # gate, up, down once each
    with torch.no_grad():
        scl.alpha.mul_(-1.5)
        y2 = mlp(x)
        mlp(x)
    assert len(pack_calls) == 5  # up and down repacked, gate kept
    with torch.no_grad():
        y_fresh = block()(x)
    torch.cuda.synchronize()
    assert not torch.equal(y1, y2)
    assert torch.equal(y2, y_fresh)


def _capture_and_check(fn, x_static, inputs):
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn(x_static)  # warm-up (and any caches) outside capture
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = fn(x_static)
    for rep, x in enumerate(inputs + inputs[::-1]):
        x_static.copy_(x)
        g.replay()
        eager = fn(x)
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"replay {rep} differs from eager"


@pytest.mark.parametrize("M", [1, 256])
def test_quant_linear_forward_in_a_graph(gpu, pack_calls, M):
    """QuantLinear.forward with a learned rotation and the online Hadamard,
    captured in a HIP graph (decode: the fused kernel; prefill: quantize +
    pipelined GEMM); replays equal eager calls, and no call repacks."""
    heads, hd, N = 32, 128, 4096
    K = heads * hd
    print(f"graph QuantLinear M{M} K{K} N{N}", flush=True)
    rot = LearnedRotation(heads, hd, seed=5).to(gpu)
    (layer,) = _enabled(QuantLinear(_base(N, K, 23, gpu, bias=True), Cfg(), rot, "o"), rot=128)
    xs = [torch.from_numpy(activations(M, K, seed=s)).to(gpu) for s in (1, 2, 3)]
    with torch.no_grad():
        _capture_and_check(layer, xs[0].clone(), xs)
    assert len(pack_calls) == 1 and rot._calls == 1


def test_quant_mlp_forward_in_a_graph(gpu, pack_calls):
    K, N, M = 1024, 2816, 64
    print(f"graph QuantMLP M{M} K{K} N{N}", flush=True)
    gate, up, down = (QuantLinear(_base(n, k, s, gpu, bias=True), Cfg())
                      for n, k, s in ((N, K, 41), (N, K, 42), (K, N, 43)))
    _enabled(gate, up)
    _enabled(down, rot=128)
    mlp = QuantMLP(gate, up, down)
    xs = [torch.from_numpy(activations(M, K, seed=s)).to(gpu) for s in (4, 5, 6)]
    with torch.no_grad():
        _capture_and_check(mlp, xs[0].clone(), xs)
    assert len(pack_calls) == 3


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_quant_mlp_non_fp16_inputs_run_the_composition(gpu, monkeypatch, dtype):
    """fp32 / bf16 inputs skip the fp16 fused block: each projection runs the
    integer path in fp32 and the activation runs in the input dtype, as
    down(silu(gate(x)) * up(x)) does.  Each projection is bit-exact against the
    oracle on its own input."""
    K, N, M = 512, 1024, 24
    gated = []
    monkeypatch.setattr(w4a4, "matmul_silu_mul", lambda *a, **k: gated.append(1))
    gate, up, down = (QuantLinear(_base(n, k, s, gpu, bias=True, dtype=torch.float32), Cfg())
                      for n, k, s in ((N, K, 51), (N, K, 52), (K, N, 53)))
    _enabled(gate, up, down)
    mlp = QuantMLP(gate, up, down)
    x = torch.from_numpy(activations(M, K, seed=11, dtype=np.float32)).to(gpu).to(dtype)
    with torch.no_grad():
        y = mlp(x)
        g, u = gate(x), up(x)
        h = F.silu(g) * u
        y_comp = down(h)
    torch.cuda.synchronize()
    assert not gated and y.dtype == dtype and torch.equal(y, y_comp)

    def ref(mod, inp):
        out, *_ = native.linear_w4a4(inp.float().cpu().numpy(),
                                     mod.base.weight.cpu().numpy(),
                                     mod.base.bias.cpu().numpy(), out_dtype=np.float32)
        return torch.from_numpy(out).to(dtype)

    assert torch.equal(g.cpu(), ref(gate, x)) and torch.equal(u.cpu(), ref(up, x))
    assert torch.equal(y.cpu(), ref(down, h))


@pytest.mark.parametrize("lead", [(0,), (2, 0)])
@pytest.mark.parametrize("rot,bias", [(0, False), (128, True)])
def test_quant_linear_empty_batch(gpu, lead, rot, bias):
    """An empty batch gives an empty [..., 0, N] output in x's dtype, as F.linear
    does (core/linear.py:48-52), and a following forward is unaffected."""
    K, N = 512, 256
    q = QuantLinear(_base(N, K, 3, gpu, bias=bias), Cfg())
    _enabled(q, rot=rot)
    with torch.no_grad():
        y = q(torch.empty(*lead, K, dtype=torch.float16, device=gpu))
        assert y.shape == (*lead, N) and y.dtype == torch.float16 and y.device == gpu
        x = torch.from_numpy(activations(4, K, seed=5)).to(gpu)
        y1 = q(x)
        y2 = QuantLinear(q.base, Cfg())
        _enabled(y2, rot=rot)
        torch.testing.assert_close(y1, y2(x), rtol=0, atol=0)
