"""EvenSoftplus for heteroscedastic (TAGI-V) outputs (mirrors triton_tagi/layers/even_softplus.py:38-194).

The output holds interleaved (mean, noise-variance) pairs. Odd flat positions get the
second-order Gaussian moments of softplus, with s = sigmoid(mu):
    mu_a = max(softplus(mu) + S s (1 - s) / 2, 1e-9),  S_a = max(s^2 S, 1e-9),  J = s
and even positions pass through (J = 1). Backward: delta_mu J, delta_S J^2.
"""

from __future__ import annotations

import torch
from torch import Tensor

from .. import _lib
from ..base import Layer
from .relu import jacobian_backward


def even_softplus(mz: Tensor, Sz: Tensor, half_width: int):
    """(ma, Sa, J) of the flat moments (even_softplus.py:93-124); half_width is not needed
    by the rule (odd flat positions are the odd positions of every 2K-wide row)."""
    mz = _lib.check(mz.contiguous(), "mz")
    Sz = _lib.check(Sz.contiguous(), "Sz")
    if Sz.shape != mz.shape:
        raise ValueError("even_softplus: mz and Sz shapes differ")
    ma, Sa, J = torch.empty_like(mz), torch.empty_like(mz), torch.empty_like(mz)
    _lib.call("tagi_even_softplus_fwd", mz.data_ptr(), Sz.data_ptr(), ma.data_ptr(), Sa.data_ptr(), J.data_ptr(),
              mz.numel(), _lib.stream_of(mz))
    return ma, Sa, J


class EvenSoftplus(Layer):
    def __init__(self, half_width: int) -> None:
        self.half_width = half_width
        self.J = None

    def forward(self, mz: Tensor, Sz: Tensor) -> tuple[Tensor, Tensor]:
        shape = mz.shape
        ma, Sa, J = even_softplus(mz.reshape(-1), Sz.reshape(-1), self.half_width)
        self.J = J.view(shape)
        return ma.view(shape), Sa.view(shape)

    def backward(self, delta_ma: Tensor, delta_Sa: Tensor) -> tuple[Tensor, Tensor]:
        return jacobian_backward(delta_ma, delta_Sa, self.J)

    def __repr__(self):
        return f"EvenSoftplus(half_width={self.half_width})"
