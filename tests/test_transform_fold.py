"""The weight folds of QuantLinear.transformed (core/linear.py:22-46) pinned by
the invariance they exist for, on the CPU in fp32.

* Per-head rotation: v's output rows become R^T W_v per kv head (bias too) and
  o's input columns W_o R per query head, R repeated over the `repeat` query
  heads that share a kv head.  Attention mixes v's head outputs only within a
  head, so the composed map o . expand . v must be unchanged:
  W_o' E W_v' = W_o E W_v and W_o' E b_v' = W_o E b_v, E the kv -> query head
  expansion.  R is orthogonal and not symmetric, so R in place of R^T, or the
  rotation applied on the wrong axis, changes the product.
* Diagonal scaling: up's output rows are divided by s, down's input columns
  multiplied by s, so W_down' diag(g) W_up' = W_down diag(g) W_up for any gate
  factor g (SiLU(gate) multiplies up's output elementwise) and the up bias maps
  the same way.  A scale on the wrong axis, or multiplied where it divides,
  changes the product.
"""
import torch

from dscquant_amd.core.linear import QuantLinear


class _Rot(torch.nn.Module):
    def __init__(self, heads, head_dim, seed):
        super().__init__()
        self.heads, self.head_dim = heads, head_dim
        g = torch.Generator().manual_seed(seed)
        a = torch.randn(heads, head_dim, head_dim, generator=g, dtype=torch.float64)
        # exp of a skew-symmetric matrix is orthogonal with det +1 (a learned
        # rotation basis), computed in float64 and stored as fp32
        self.m = torch.linalg.matrix_exp(0.3 * (a - a.transpose(-1, -2))).float()

    def matrices(self):
        return self.m


class _Scl(torch.nn.Module):
    def __init__(self, n, seed):
        super().__init__()
        g = torch.Generator().manual_seed(seed)
        self.s = torch.exp(torch.randn(n, generator=g) * 0.5)

    def diagonal(self):
        return self.s


def _linear(n_out, n_in, seed, bias=True):
    g = torch.Generator().manual_seed(seed)
    lin = torch.nn.Linear(n_in, n_out, bias=bias)
    with torch.no_grad():
        lin.weight.copy_(torch.randn(n_out, n_in, generator=g) * 0.05)
        if bias:
            lin.bias.copy_(torch.randn(n_out, generator=g) * 0.1)
    return lin


def _close(a, b):
    torch.testing.assert_close(a, b, rtol=1e-4, atol=1e-5)


def test_rotation_fold_preserves_attention_value_output_map():
    hidden, kv_heads, head_dim, repeat = 96, 4, 16, 2
    rot = _Rot(kv_heads, head_dim, seed=1)
    v = QuantLinear(_linear(kv_heads * head_dim, hidden, seed=2), None, rot, "v")
    o = QuantLinear(_linear(hidden, kv_heads * repeat * head_dim, seed=3, bias=False),
                    None, rot, "o", repeat=repeat)

    def expand(t):  # kv-head blocks of rows -> query-head blocks
        return t.reshape(kv_heads, head_dim, -1).repeat_interleave(repeat, dim=0) \
                .reshape(kv_heads * repeat * head_dim, -1)

    wv, bv = v.base.weight.double(), v.base.bias.double()
    wo = o.base.weight.double()
    wv_f, bv_f = (t.double() for t in v.transformed())
    wo_f, bo_f = o.transformed()
    assert bo_f is None
    wo_f = wo_f.double()

    _close(wo_f @ expand(wv_f), wo @ expand(wv))
    _close(wo_f @ expand(bv_f[:, None]), wo @ expand(bv[:, None]))
    # the fold changed the weights themselves (the rotation is not the identity)
    assert (wv_f - wv).abs().max() > 1e-2 and (wo_f - wo).abs().max() > 1e-2
    # per-head orthogonality: the folded v rows keep each head's Gram matrix over K
    g0 = torch.einsum("hdk,hek->hde", wv.reshape(kv_heads, head_dim, -1),
                      wv.reshape(kv_heads, head_dim, -1))
    g1 = torch.einsum("hdk,hek->hde", wv_f.reshape(kv_heads, head_dim, -1),
                      wv_f.reshape(kv_heads, head_dim, -1))
    rm = rot.m.double()
    _close(g1, rm.transpose(-1, -2) @ g0 @ rm)


def test_scaling_fold_preserves_gated_mlp_map():
    hidden, inter = 64, 160
    scl = _Scl(inter, seed=4)
    up = QuantLinear(_linear(inter, hidden, seed=5), None, scl, "up")
    down = QuantLinear(_linear(hidden, inter, seed=6, bias=False), None, scl, "down")
    gate = torch.rand(inter, generator=torch.Generator().manual_seed(7), dtype=torch.float64)

    wu, bu = up.base.weight.double(), up.base.bias.double()
    wd = down.base.weight.double()
    wu_f, bu_f = (t.double() for t in up.transformed())
    wd_f = down.transformed()[0].double()

    _close(wd_f @ (gate[:, None] * wu_f), wd @ (gate[:, None] * wu))
    _close(wd_f @ (gate * bu_f), wd @ (gate * bu))
    assert (wu_f - wu).abs().max() > 1e-3 and (wd_f - wd).abs().max() > 1e-3


def test_no_interface_is_identity():
    lin = _linear(32, 48, seed=8)
    w, b = QuantLinear(lin, None).transformed()
    assert w is lin.weight and b is lin.bias
