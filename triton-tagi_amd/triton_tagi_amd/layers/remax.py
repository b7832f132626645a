"""Remax activation (mirrors triton_tagi/layers/remax.py:33-191).

Per row: MixtureReLU moments of M = max(0, Z) (floored at 1e-6), log-normal moments of
M and its row sum, mu_A renormalised to sum 1, S_A = (exp(var_ln_A) - 1) mu_A^2 and the
Jacobian J = min(sqrt(S_A S_Z), cov(A, M)/max(Phi, 1e-6)) / S_Z. One wavefront per row.
"""

from __future__ import annotations

import torch
from torch import Tensor

from .. import _lib
from ..base import Layer
from .relu import jacobian_backward


def remax(mu_z: Tensor, var_z: Tensor):
    """(mu_a, var_a, J) over the last dim of a (B, K) or (K,) tensor (remax.py:122-159)."""
    squeeze = mu_z.dim() == 1
    if squeeze:
        mu_z, var_z = mu_z.unsqueeze(0), var_z.unsqueeze(0)
    mu_z = _lib.check(mu_z.contiguous(), "mu_z")
    var_z = _lib.check(var_z.contiguous(), "var_z")
    if mu_z.dim() != 2 or var_z.shape != mu_z.shape:
        raise ValueError(f"remax: expected matching (B, K) tensors, got {tuple(mu_z.shape)}")
    B, K = mu_z.shape
    mu_a, var_a, J = torch.empty_like(mu_z), torch.empty_like(mu_z), torch.empty_like(mu_z)
    _lib.call("tagi_remax_fwd", mu_z.data_ptr(), var_z.data_ptr(), mu_a.data_ptr(), var_a.data_ptr(),
              J.data_ptr(), B, K, _lib.stream_of(mu_z))
    if squeeze:
        return mu_a.squeeze(0), var_a.squeeze(0), J.squeeze(0)
    return mu_a, var_a, J


triton_remax = remax


class Remax(Layer):
    """Softmax alternative for Bayesian nets (sum of output means ~ 1)."""

    def __init__(self) -> None:
        self.J: Tensor | None = None

    def forward(self, mz: Tensor, Sz: Tensor) -> tuple[Tensor, Tensor]:
        mu_a, Sa, J = remax(mz, Sz)
        self.J = J
        return mu_a, Sa

    def backward(self, delta_ma: Tensor, delta_Sa: Tensor) -> tuple[Tensor, Tensor]:
        return jacobian_backward(delta_ma, delta_Sa, self.J)

    def __repr__(self) -> str:
        return "Remax()"
