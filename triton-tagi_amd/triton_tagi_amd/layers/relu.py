"""Bayesian ReLU (mirrors triton_tagi/layers/relu.py:43-172).

With alpha = mu_z / sigma_z:
    mu_a = sigma phi(alpha) + mu Phi(alpha)
    S_a  = max(-mu_a^2 + 2 mu_a mu - mu sigma phi + (S - mu^2) Phi, 0)
    J    = Phi(alpha)   (Phi ~ phi/(-alpha) below alpha = -5)
Backward: delta_mu * J, delta_S * J^2.
"""

from __future__ import annotations

import torch
from torch import Tensor

from .. import _lib
from ..base import Layer


def bayesian_relu(mz, Sz):
    """(ma, Sa, J) of max(0, z), z ~ N(mz, Sz), elementwise (relu.py:94-122)."""
    mz = _lib.check(_lib.dense(mz), "mz")
    Sz = _lib.check(_lib.like(Sz, mz), "Sz")
    if Sz.shape != mz.shape:
        raise ValueError("bayesian_relu: mz and Sz shapes differ")
    ma, Sa, J = torch.empty_like(mz), torch.empty_like(mz), torch.empty_like(mz)
    _lib.call("tagi_relu_fwd", mz.data_ptr(), Sz.data_ptr(), ma.data_ptr(), Sa.data_ptr(), J.data_ptr(),
              mz.numel(), _lib.stream_of(mz))
    return ma, Sa, J


def jacobian_backward(delta_m, delta_S, J):
    """(delta_m * J, delta_S * J^2), one HIP launch."""
    dm = _lib.check(_lib.like(delta_m.reshape(J.shape), J), "delta_m")
    dS = _lib.check(_lib.like(delta_S.reshape(J.shape), J), "delta_S")
    if dm.numel() != J.numel() or dS.numel() != J.numel():
        raise ValueError(f"Jacobian backward: delta {tuple(dm.shape)} vs stored Jacobian {tuple(J.shape)}")
    om, oS = torch.empty_like(dm), torch.empty_like(dS)
    _lib.call("tagi_jacobian_bwd", dm.data_ptr(), dS.data_ptr(), J.data_ptr(), om.data_ptr(), oS.data_ptr(),
              dm.numel(), _lib.stream_of(dm))
    return om, oS


class ReLU(Layer):
    """Rectified-Gaussian activation; stores J for the backward pass."""

    def __init__(self) -> None:
        self.J = None

    def forward(self, mz: Tensor, Sz: Tensor) -> tuple[Tensor, Tensor]:
        ma, Sa, J = bayesian_relu(mz, Sz)
        self.J = J
        return ma, Sa

    def backward(self, delta_mz: Tensor, delta_Sz: Tensor) -> tuple[Tensor, Tensor]:
        return jacobian_backward(delta_mz, delta_Sz, self.J)

    def __repr__(self):
        return "ReLU()"
