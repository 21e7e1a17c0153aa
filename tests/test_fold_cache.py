"""QuantLinear's cached fold (transformed()) and clip values, on the CPU.

The fold of a learned interface (core/linear.py:22-46) is recomputed only when
something it depends on changes: the base weight / bias, or any parameter,
buffer or plain attribute of the interface (alpha, beta, the bases, probe,
override; core/transforms.py:6-31).  With autograd recording through the
interface (calibration), every call folds afresh with the graph attached, as
the reference does.
"""
import pytest
import torch
from torch import nn

from dscquant_amd.core.linear import QuantLinear
from tests.interfaces import LearnedRotation as _LearnedRotation
from tests.interfaces import LearnedScaling as _LearnedScaling


def _linear(n_out, n_in, seed, bias=True):
    g = torch.Generator().manual_seed(seed)
    lin = nn.Linear(n_in, n_out, bias=bias)
    with torch.no_grad():
        lin.weight.copy_(torch.randn(n_out, n_in, generator=g) * 0.05)
        if bias:
            lin.bias.copy_(torch.randn(n_out, generator=g) * 0.1)
    return lin


def _v_fold_formula(rot, lin):
    R = rot.matrices().detach()
    w = (R.transpose(-1, -2) @ lin.weight.reshape(rot.heads, rot.head_dim, -1)).reshape_as(lin.weight)
    b = (R.transpose(-1, -2) @ lin.bias.reshape(rot.heads, -1, 1)).flatten()
    return w, b


def test_fold_is_cached_until_the_interface_changes():
    rot = _LearnedRotation(2, 8)
    lin = _linear(16, 24, seed=1)
    q = QuantLinear(lin, None, rot, "v")
    with torch.no_grad():
        w1, b1 = q.transformed()
        w2, b2 = q.transformed()
        assert rot._calls == 1 and w2 is w1 and b2 is b1
        # a learned coefficient updated in place (an optimizer step does the same)
        rot.alpha.add_(0.25)
        w3, b3 = q.transformed()
        assert rot._calls == 2 and w3 is not w1
        assert (w3 - w1).abs().max() > 1e-4
        ref_w, ref_b = _v_fold_formula(rot, lin)
        torch.testing.assert_close(w3, ref_w, rtol=1e-5, atol=1e-6)
        torch.testing.assert_close(b3, ref_b, rtol=1e-5, atol=1e-6)
        # override / probe are plain attributes: setting or clearing one refolds
        n = rot.rec_basis.shape[0]
        rot.override = torch.full((n,), 0.01)
        w4, _ = q.transformed()
        assert rot._calls == 4 and w4 is not w3  # (one extra call from the formula above)
        rot.override = None
        w5, _ = q.transformed()
        assert rot._calls == 5
        torch.testing.assert_close(w5, w3)
        # a new basis tensor (Interface.set_basis assigns one)
        rot.rec_basis = rot.rec_basis.clone() * 2
        q.transformed()
        assert rot._calls == 6
        # the base weight itself
        lin.weight.mul_(2)
        w7, _ = q.transformed()
        assert rot._calls == 7
        torch.testing.assert_close(w7, _v_fold_formula(rot, lin)[0], rtol=1e-5, atol=1e-6)
        rot._calls = 0
        q.transformed()
        assert rot._calls == 0  # rebuilt formula above did not disturb the cache


def test_fold_records_autograd_when_the_interface_is_trained():
    scl = _LearnedScaling(32)
    up = QuantLinear(_linear(32, 16, seed=2), None, scl, "up")
    w1, b1 = up.transformed()
    w2, _ = up.transformed()
    assert scl._calls == 2 and w1.grad_fn is not None and b1.grad_fn is not None
    (w1.sum() + w2.sum()).backward()
    assert scl.alpha.grad is not None and scl.alpha.grad.abs().sum() > 0
    # without grad the same fold is computed once and cached
    scl._calls = 0
    with torch.no_grad():
        a, _ = up.transformed()
        b, _ = up.transformed()
    assert scl._calls == 1 and a is b
    torch.testing.assert_close(a, w1.detach())


def test_o_projection_fold_repeats_each_rotation_over_its_query_heads():
    rot = _LearnedRotation(2, 4, seed=3)
    repeat = 3
    lin = _linear(10, 2 * repeat * 4, seed=4, bias=False)
    q = QuantLinear(lin, None, rot, "o", repeat=repeat)
    with torch.no_grad():
        w, b = q.transformed()
    assert b is None
    R = rot.matrices().detach()
    for j in range(2 * repeat):
        cols = slice(4 * j, 4 * j + 4)
        torch.testing.assert_close(w[:, cols], lin.weight[:, cols] @ R[j // repeat],
                                   rtol=1e-5, atol=1e-6)


def test_data_writes_need_invalidate_cache():
    scl = _LearnedScaling(16)
    dn = QuantLinear(_linear(8, 16, seed=5, bias=False), None, scl, "down")
    with torch.no_grad():
        w1, _ = dn.transformed()
    scl.alpha.data.add_(0.5)  # bypasses the version counter
    with torch.no_grad():
        assert dn.transformed()[0] is w1
    dn.invalidate_cache()
    with torch.no_grad():
        w2, _ = dn.transformed()
    assert (w2 - w1).abs().max() > 1e-4
    torch.testing.assert_close(w2, dn.base.weight * scl.diagonal().detach()[None, :])


def test_clip_values_follow_in_place_updates():
    q = QuantLinear(_linear(8, 16, seed=6), None)
    assert q.clip_value("weight_clip") == 1.0
    with torch.no_grad():
        q.weight_clip.fill_(0.75)
    assert q.clip_value("weight_clip") == 0.75
    q.load_state_dict({**q.state_dict(), "activation_clip": torch.tensor(0.5)})
    assert q.clip_value("activation_clip") == 0.5
    q.weight_clip = nn.Parameter(torch.tensor(0.625), requires_grad=False)
    assert q.clip_value("weight_clip") == 0.625
    q.weight_clip.data.fill_(0.875)  # not seen until the cache is dropped
    assert q.clip_value("weight_clip") == 0.625
    q.invalidate_cache()
    assert q.clip_value("weight_clip") == 0.875


def test_dead_interface_falls_back_to_the_base_weight():
    rot = _LearnedRotation(2, 8)
    lin = _linear(16, 24, seed=7)
    q = QuantLinear(lin, None, rot, "v")
    with torch.no_grad():
        w1, _ = q.transformed()
    assert w1 is not lin.weight
    del rot
    import gc
    gc.collect()
    w, b = q.transformed()
    assert w is lin.weight and b is lin.bias


def test_non_w4a4_path_refuses_gradients():
    class Cfg:
        weight_bits, activation_bits = 8, 6
    q = QuantLinear(_linear(8, 16, seed=8), Cfg())
    q.enabled = True
    x = torch.randn(2, 16, requires_grad=True)
    with pytest.raises(RuntimeError, match="no gradient"):
        q(x)


def test_fold_follows_module_casts():
    """Module.half() swaps each parameter's .data (same object, same version):
    the cached fold and clip values must follow the new dtype."""
    rot = _LearnedRotation(2, 8)
    lin = _linear(16, 24, seed=9)
    q = QuantLinear(lin, None, rot, "v")
    with torch.no_grad():
        w1, b1 = q.transformed()
    assert w1.dtype == torch.float32
    q.half()
    assert lin.weight.dtype == torch.float16
    with torch.no_grad():
        w2, b2 = q.transformed()
    assert w2.dtype == torch.float16 and b2.dtype == torch.float16
    assert q.clip_value("weight_clip") == 1.0
    q.float()
    with torch.no_grad():
        w3, _ = q.transformed()
    assert w3.dtype == torch.float32 and w3 is not w1


def test_clip_value_follows_module_casts():
    q = QuantLinear(_linear(8, 16, seed=10), None)
    assert q.clip_value("activation_clip") == 1.0
    q.activation_clip.data = torch.tensor(0.75)  # what Module._apply does per parameter
    assert q.clip_value("activation_clip") == 0.75


class _W4A4:
    weight_bits, activation_bits = 4, 4


@pytest.mark.parametrize("lead", [(0,), (3, 0), (0, 5)])
@pytest.mark.parametrize("rotate", [0, 128])
def test_empty_batch_returns_empty_output_without_launching(monkeypatch, lead, rotate):
    """F.linear of an empty batch is an empty [..., 0, N] tensor in x's dtype
    (core/linear.py:48-52); the integer path returns it without a library call."""
    from dscquant_amd import _lib

    def no_call(*a, **k):
        raise AssertionError("library called for an empty batch")
    monkeypatch.setattr(_lib, "call", no_call)
    q = QuantLinear(_linear(32, 256, seed=11), _W4A4())
    q.enabled, q.rotate_block = True, rotate
    for dtype in (torch.float16, torch.float32):
        x = torch.empty(*lead, 256, dtype=dtype)
        with torch.no_grad():
            y = q(x)
        assert y.shape == (*lead, 32) and y.dtype == dtype


def test_feature_mismatch_raises_like_f_linear(monkeypatch):
    """K inside the same 64-element padding step as the weight's K would pass the
    packed-shape checks; the module rejects it as F.linear does."""
    from dscquant_amd import _lib
    monkeypatch.setattr(_lib, "call", lambda *a, **k: (_ for _ in ()).throw(AssertionError()))
    q = QuantLinear(_linear(32, 256, seed=12), _W4A4())
    q.enabled = True
    for shape in [(4, 250), (0, 250), (2, 3, 260)]:
        with pytest.raises(RuntimeError, match="cannot be multiplied"):
            with torch.no_grad():
                q(torch.zeros(*shape, dtype=torch.float16))
