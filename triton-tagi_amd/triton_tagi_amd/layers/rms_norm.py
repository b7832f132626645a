"""Bayesian RMSNorm (mirrors triton_tagi/layers/rms_norm.py:42-150).

Per row r of length ni:  rms = mean(mu^2 + S),  inv = 1/sqrt(rms + eps)
    mu_z = inv mu g,   S_z = inv^2 (S (g^2 + Sg) + Sg mu^2)
Backward: delta_mu inv g, delta_S (inv g)^2;  delta_g = Sg sum_r inv mu delta_mu,
delta_Sg = Sg^2 sum_r inv^2 mu^2 delta_S.
"""

from __future__ import annotations

import torch
from torch import Tensor

from .. import _lib
from ..base import LearnableLayer
from ..param_init import init_weight_bias_norm
from ..update.parameters import update_parameters


class RMSNorm(LearnableLayer):
    def __init__(self, normalized_shape, eps: float = 1e-6, gain_w: float = 1.0, device: str = "cuda") -> None:
        if isinstance(normalized_shape, int):
            normalized_shape = [normalized_shape]
        if len(normalized_shape) != 1:
            raise ValueError(f"RMSNorm only supports a single normalized dimension, got {normalized_shape}")
        self.normalized_shape = list(normalized_shape)
        self.ni = normalized_shape[0]
        self.eps = eps
        self.gain_w = gain_w
        self.device = torch.device(device)
        self.has_bias = False
        mu_w, Sw, _, _ = init_weight_bias_norm(self.ni, gain_w=gain_w, gain_b=1.0, device=self.device)
        self.mw, self.Sw = mu_w, Sw
        self.mb = self.Sb = None
        self.ma_in = None
        self.inv_rms = None
        self._input_shape = None
        self.delta_mw = self.delta_Sw = self.delta_mb = self.delta_Sb = None

    def forward(self, ma: Tensor, Sa: Tensor) -> tuple[Tensor, Tensor]:
        self._input_shape = ma.shape
        ma_flat = _lib.check(ma.reshape(-1, self.ni).contiguous(), "ma")
        Sa_flat = _lib.check(Sa.reshape(-1, self.ni).contiguous(), "Sa")
        rows = ma_flat.shape[0]
        mz, Sz = torch.empty_like(ma_flat), torch.empty_like(ma_flat)
        inv = torch.empty(rows, 1, device=ma.device, dtype=torch.float32)
        _lib.call("tagi_rmsnorm_fwd", ma_flat.data_ptr(), Sa_flat.data_ptr(), self.mw.data_ptr(), self.Sw.data_ptr(),
                  mz.data_ptr(), Sz.data_ptr(), inv.data_ptr(), rows, self.ni, float(self.eps), _lib.stream_of(ma_flat))
        self.ma_in = ma_flat
        self.inv_rms = inv
        return mz.reshape(self._input_shape), Sz.reshape(self._input_shape)

    def backward(self, delta_mz: Tensor, delta_Sz: Tensor) -> tuple[Tensor, Tensor]:
        shape = delta_mz.shape
        dm = _lib.check(delta_mz.reshape(-1, self.ni).contiguous(), "delta_mz")
        dS = _lib.check(delta_Sz.reshape(-1, self.ni).contiguous(), "delta_Sz")
        rows = dm.shape[0]
        dev = dm.device
        dma, dSa = torch.empty_like(dm), torch.empty_like(dS)
        self.delta_mw = torch.empty(self.ni, device=dev, dtype=torch.float32)
        self.delta_Sw = torch.empty_like(self.delta_mw)
        ws = _lib.workspace(_lib.query("tagi_rmsnorm_bwd_ws_bytes", rows, self.ni), dev)
        wp, wb = _lib.ws_args(ws)
        _lib.call("tagi_rmsnorm_bwd", dm.data_ptr(), dS.data_ptr(), self.ma_in.data_ptr(), self.inv_rms.data_ptr(),
                  self.mw.data_ptr(), self.Sw.data_ptr(), dma.data_ptr(), dSa.data_ptr(), self.delta_mw.data_ptr(),
                  self.delta_Sw.data_ptr(), rows, self.ni, wp, wb, _lib.stream_of(dm))
        return dma.reshape(shape), dSa.reshape(shape)

    def _update_items(self):
        return [(self.mw, self.Sw, self.delta_mw, self.delta_Sw)]

    def update(self, cap_factor: float) -> None:
        update_parameters(self.mw, self.Sw, self.delta_mw, self.delta_Sw, cap_factor)

    @property
    def num_parameters(self) -> int:
        return 2 * self.mw.numel()

    def __repr__(self) -> str:
        return f"RMSNorm(normalized_shape={self.normalized_shape}, eps={self.eps}, gain_w={self.gain_w})"
