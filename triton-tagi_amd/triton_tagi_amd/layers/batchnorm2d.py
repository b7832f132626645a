"""Bayesian BatchNorm2D (mirrors triton_tagi/layers/batchnorm2d.py:238-538).

Training forward normalises with the batch statistics
    mean_c = E[mu],  var_c = (E[S] + E[mu^2] - mean_c^2) * n/(n-1),  n = N*H*W
and keeps running statistics: the first call copies the batch statistics (and, with
preserve_var, sets gamma := sqrt(var + eps)); later calls apply an EMA with momentum.
    mhat = (mu - mean)/sqrt(var+eps),  Shat = S/(var+eps)
    mu_out = g mhat + b,  S_out = g^2 Shat + Sg (mhat^2 + Shat) + Sb
Backward: delta_mz = delta_mu g/sqrt(var+eps), delta_Sz = delta_S g^2/(var+eps), and
delta_g = Sg sum(delta_mu mhat), delta_Sg = Sg^2 sum(delta_S mhat^2), delta_b = Sb sum
delta_mu, delta_Sb = Sb^2 sum delta_S (sums over N, H, W). Activations are kept channels-last.
"""

from __future__ import annotations

import torch
from torch import Tensor

from .. import _lib
from ..base import LearnableLayer
from ..param_init import init_weight_bias_norm
from ..update.parameters import update_parameters


class BatchNorm2D(LearnableLayer):
    def __init__(self, num_features: int, momentum: float = 0.1, eps: float = 1e-5, device: str = "cuda",
                 gain_w: float = 1.0, gain_b: float = 1.0, preserve_var: bool = True) -> None:
        self.num_features = num_features
        self.momentum = momentum
        self.eps = eps
        self.device = torch.device(device)
        self.training = True
        self.preserve_var = preserve_var
        self._is_initialized = False
        self.mw, self.Sw, self.mb, self.Sb = init_weight_bias_norm(
            num_features, gain_w=gain_w, gain_b=gain_b, device=self.device
        )
        self.has_bias = True
        self.running_mean = torch.zeros(num_features, device=self.device)
        self.running_var = torch.ones(num_features, device=self.device)
        self.m_hat = None
        self.S_hat = None  # not materialised (the backward pass does not read it)
        self.input_shape = None
        self._norm_var = None
        self.delta_mw = self.delta_Sw = self.delta_mb = self.delta_Sb = None

    def train(self) -> None:
        self.training = True

    def eval(self) -> None:
        self.training = False

    def forward(self, mz: Tensor, Sz: Tensor) -> tuple[Tensor, Tensor]:
        mz = _lib.check(_lib.channels_last(mz), "mz")
        Sz = _lib.check(_lib.channels_last(Sz), "Sz")
        self.input_shape = mz.shape
        N, C, H, W = mz.shape
        if C != self.num_features:
            raise ValueError(f"BatchNorm2D: expected {self.num_features} channels, got {C}")
        HW = H * W
        dev = mz.device
        st = _lib.stream_of(mz)
        if self.training:
            bmean = torch.empty(C, device=dev, dtype=torch.float32)
            bvar = torch.empty(C, device=dev, dtype=torch.float32)
            first = not self._is_initialized
            ws = _lib.workspace(_lib.query("tagi_bn_stats_ws_bytes", N, C, HW), dev)
            wp, wb = _lib.ws_args(ws)
            _lib.call("tagi_bn_stats", mz.data_ptr(), Sz.data_ptr(), bmean.data_ptr(), bvar.data_ptr(),
                      _lib.check(self.running_mean, "running_mean").data_ptr(),
                      _lib.check(self.running_var, "running_var").data_ptr(), _lib.check(self.mw, "mw").data_ptr(),
                      N, C, HW, float(self.momentum), float(self.eps), int(first), int(self.preserve_var), wp, wb, st)
            self._is_initialized = True
            norm_mean, norm_var = bmean, bvar
        else:
            norm_mean, norm_var = self.running_mean, self.running_var
        self._norm_var = norm_var
        ma, Sa, mhat = torch.empty_like(mz), torch.empty_like(mz), torch.empty_like(mz)
        _lib.call("tagi_bn_fwd", mz.data_ptr(), Sz.data_ptr(), norm_mean.data_ptr(), norm_var.data_ptr(),
                  self.mw.data_ptr(), _lib.check(self.Sw, "Sw").data_ptr(), _lib.check(self.mb, "mb").data_ptr(),
                  _lib.check(self.Sb, "Sb").data_ptr(), ma.data_ptr(), Sa.data_ptr(), mhat.data_ptr(), None, N, C, HW,
                  float(self.eps), st)
        self.m_hat = mhat
        return ma, Sa

    def backward(self, delta_ma: Tensor, delta_Sa: Tensor) -> tuple[Tensor, Tensor]:
        dma = _lib.check(_lib.channels_last(delta_ma.reshape(self.input_shape)), "delta_ma")
        dSa = _lib.check(_lib.channels_last(delta_Sa.reshape(self.input_shape)), "delta_Sa")
        N, C, H, W = self.input_shape
        HW = H * W
        dev = dma.device
        dmz, dSz = torch.empty_like(dma), torch.empty_like(dSa)
        self.delta_mw = torch.empty(C, device=dev, dtype=torch.float32)
        self.delta_Sw = torch.empty_like(self.delta_mw)
        self.delta_mb = torch.empty_like(self.delta_mw)
        self.delta_Sb = torch.empty_like(self.delta_mw)
        ws = _lib.workspace(_lib.query("tagi_bn_bwd_ws_bytes", N, C, HW), dev)
        wp, wb = _lib.ws_args(ws)
        _lib.call("tagi_bn_bwd", dma.data_ptr(), dSa.data_ptr(), self.m_hat.data_ptr(), self._norm_var.data_ptr(),
                  self.mw.data_ptr(), self.Sw.data_ptr(), self.Sb.data_ptr(), dmz.data_ptr(), dSz.data_ptr(),
                  self.delta_mw.data_ptr(), self.delta_Sw.data_ptr(), self.delta_mb.data_ptr(),
                  self.delta_Sb.data_ptr(), N, C, HW, float(self.eps), wp, wb, _lib.stream_of(dma))
        return dmz, dSz

    def _update_items(self):
        return [(self.mw, self.Sw, self.delta_mw, self.delta_Sw), (self.mb, self.Sb, self.delta_mb, self.delta_Sb)]

    def update(self, cap_factor: float) -> None:
        for m, S, dm, dS in self._update_items():
            update_parameters(m, S, dm, dS, cap_factor)

    @property
    def num_parameters(self) -> int:
        return 2 * (self.mw.numel() + self.mb.numel())

    def __repr__(self):
        return f"BatchNorm2D(num_features={self.num_features}, momentum={self.momentum}, eps={self.eps})"
