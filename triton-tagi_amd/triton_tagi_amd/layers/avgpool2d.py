"""Bayesian AvgPool2D (mirrors triton_tagi/layers/avgpool2d.py:329-434).

Activations are kept channels-last. Non-overlapping k x k windows: mu_out = sum mu / k^2; S_out = sum S / k^4
(spatial_correlation=False) or / k^2 (True). Backward spreads delta_mu/k^2 and
delta_S * (the same variance scale) to every input of the window.
"""

from __future__ import annotations

import torch
from torch import Tensor

from .. import _lib
from ..base import Layer


class AvgPool2D(Layer):
    def __init__(self, kernel_size: int, spatial_correlation: bool = False) -> None:
        self.k = kernel_size
        self.spatial_correlation = spatial_correlation
        self.input_shape = None

    def _var_scale(self) -> float:
        inv_k2 = 1.0 / (self.k * self.k)
        return inv_k2 if self.spatial_correlation else inv_k2 * inv_k2

    def forward(self, ma: Tensor, Sa: Tensor) -> tuple[Tensor, Tensor]:
        ma = _lib.check(_lib.channels_last(ma), "ma")
        Sa = _lib.check(_lib.channels_last(Sa), "Sa")
        self.input_shape = ma.shape
        N, C, H, W = ma.shape
        k = self.k
        mo = _lib.empty_cl(N, C, H // k, W // k, ma.device)
        So = _lib.empty_cl(N, C, H // k, W // k, ma.device)
        _lib.call("tagi_avgpool2d_fwd", ma.data_ptr(), Sa.data_ptr(), mo.data_ptr(), So.data_ptr(), N, C, H, W, k,
                  self._var_scale(), _lib.stream_of(ma))
        return mo, So

    def backward(self, dm: Tensor, ds: Tensor) -> tuple[Tensor, Tensor]:
        N, C, H, W = self.input_shape
        dm = _lib.check(_lib.channels_last(dm.reshape(N, C, H // self.k, W // self.k)), "dm")
        ds = _lib.check(_lib.channels_last(ds.reshape(N, C, H // self.k, W // self.k)), "ds")
        om = _lib.empty_cl(N, C, H, W, dm.device)
        oS = _lib.empty_cl(N, C, H, W, dm.device)
        _lib.call("tagi_avgpool2d_bwd", dm.data_ptr(), ds.data_ptr(), om.data_ptr(), oS.data_ptr(), N, C, H, W,
                  self.k, self._var_scale(), _lib.stream_of(dm))
        return om, oS

    def __repr__(self):
        sc = "on" if self.spatial_correlation else "off"
        return f"AvgPool2D(kernel={self.k}, spatial_correlation={sc})"
