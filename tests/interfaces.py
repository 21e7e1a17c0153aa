"""Test-side stand-ins for the reference's learned interfaces (core/transforms.py:
Interface, Rotation, Scaling): the same state layout (a reconstruction basis
buffer, learned coefficients ``alpha``, ``probe`` / ``override`` increments,
``heads`` / ``head_dim``) and the same duck-typed methods QuantLinear folds
through, ``matrices()`` and ``diagonal()``.  They count their calls in
``_calls`` so tests can see when a fold was recomputed.
"""
import math

import torch
from torch import nn


class LearnedRotation(nn.Module):
    """A per-head rotation with the reference Interface's state layout: a
    reconstruction basis and its coefficients alpha, an increment that an
    override or probe replaces; R_h = exp(skew(basis @ alpha + increment))."""

    def __init__(self, heads, head_dim, seed=0):
        super().__init__()
        self.heads, self.head_dim = heads, head_dim
        n = heads * head_dim * (head_dim - 1) // 2
        g = torch.Generator().manual_seed(seed)
        self.register_buffer("rec_basis", torch.randn(n, 3, generator=g) * 0.2)
        self.alpha = nn.Parameter(torch.randn(3, generator=g))
        self.probe = None
        self.override = None
        self._calls = 0

    def _skew(self, coord):
        d = self.head_dim
        iu = torch.triu_indices(d, d, offset=1, device=coord.device)
        out = coord.new_zeros(self.heads, d, d)
        out[:, iu[0], iu[1]] = coord.reshape(self.heads, -1) / math.sqrt(2)
        return out - out.transpose(-1, -2)

    def matrices(self):
        self._calls += 1
        coord = self.rec_basis @ self.alpha
        inc = self.override if self.override is not None else self.probe
        if inc is not None:
            coord = coord + inc
        return torch.linalg.matrix_exp(self._skew(coord))


class LearnedScaling(nn.Module):
    def __init__(self, n, seed=0):
        super().__init__()
        g = torch.Generator().manual_seed(seed)
        self.register_buffer("rec_basis", torch.randn(n, 2, generator=g) * 0.3)
        self.alpha = nn.Parameter(torch.randn(2, generator=g))
        self.override = None
        self._calls = 0

    def diagonal(self):
        self._calls += 1
        v = self.rec_basis @ self.alpha
        if self.override is not None:
            v = v + self.override
        return torch.exp(v - v.mean())
