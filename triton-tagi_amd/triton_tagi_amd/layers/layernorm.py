"""Bayesian LayerNorm over the feature dimension (mirrors triton_tagi/layers/layernorm.py:51-202).

Per sample b (statistics of the means, with the input variances added to the spread):
    mu_ra = mean_i mu_i,   var_ra = (sum_i (mu_i - mu_ra)^2 + sum_i S_i) / (D - 1)
    inv = 1 / sqrt(var_ra + eps)
    mu_z = inv (mu - mu_ra) g + b,   S_z = inv^2 (S (g^2 + Sg) + Sg (mu - mu_ra)^2) + Sb
Backward with the diagonal Jacobian J = inv g: delta_mu J, delta_S J^2, and the parameter
deltas Sg sum inv (mu - mu_ra) delta_mu, Sg^2 sum inv^2 (mu - mu_ra)^2 delta_S,
Sb sum delta_mu, Sb^2 sum delta_S over the rows.
"""

from __future__ import annotations

import torch
from torch import Tensor

from .. import _lib
from ..base import LearnableLayer
from ..param_init import init_weight_bias_norm
from ..update.parameters import update_parameters


class LayerNorm(LearnableLayer):
    def __init__(self, normalized_shape: int, eps: float = 1e-5, bias: bool = True, device: str = "cuda",
                 gain_w: float = 1.0, gain_b: float = 1.0) -> None:
        self.normalized_shape = normalized_shape
        self.ni = normalized_shape
        self.eps = eps
        self.has_bias = bias
        self.device = torch.device(device)
        self.mw, self.Sw, self.mb, self.Sb = init_weight_bias_norm(
            normalized_shape, gain_w=gain_w, gain_b=gain_b, device=self.device
        )
        if not bias:
            self.mb = torch.zeros(normalized_shape, device=self.device)
            self.Sb = torch.zeros(normalized_shape, device=self.device)
        self.ma_in: Tensor | None = None
        self.mu_ra: Tensor | None = None   # (B, 1)
        self.var_ra: Tensor | None = None  # (B, 1)
        self.delta_mw = self.delta_Sw = self.delta_mb = self.delta_Sb = None
        self._shape = None

    def forward(self, ma: Tensor, Sa: Tensor) -> tuple[Tensor, Tensor]:
        D = self.ni
        if ma.shape[-1] != D:
            raise ValueError(f"LayerNorm: expected {D} features, got {ma.shape[-1]}")
        self._shape = ma.shape
        m = _lib.check(ma.reshape(-1, D).contiguous(), "ma")
        S = _lib.check(Sa.reshape(-1, D).contiguous(), "Sa")
        rows = m.shape[0]
        mz, Sz = torch.empty_like(m), torch.empty_like(m)
        mu_ra = torch.empty(rows, 1, device=m.device, dtype=torch.float32)
        var_ra = torch.empty(rows, 1, device=m.device, dtype=torch.float32)
        _lib.call("tagi_layernorm_fwd", m.data_ptr(), S.data_ptr(), _lib.check(self.mw, "mw").data_ptr(),
                  _lib.check(self.Sw, "Sw").data_ptr(), _lib.check(self.mb, "mb").data_ptr(),
                  _lib.check(self.Sb, "Sb").data_ptr(), mz.data_ptr(), Sz.data_ptr(), mu_ra.data_ptr(),
                  var_ra.data_ptr(), rows, D, float(self.eps), _lib.stream_of(m))
        self.ma_in, self.mu_ra, self.var_ra = m, mu_ra, var_ra
        return mz.reshape(self._shape), Sz.reshape(self._shape)

    def backward(self, delta_mz: Tensor, delta_Sz: Tensor) -> tuple[Tensor, Tensor]:
        D = self.ni
        dm = _lib.check(delta_mz.reshape(-1, D).contiguous(), "delta_mz")
        dS = _lib.check(delta_Sz.reshape(-1, D).contiguous(), "delta_Sz")
        rows = dm.shape[0]
        if rows != self.ma_in.shape[0]:
            raise ValueError(f"LayerNorm: {rows} delta rows for {self.ma_in.shape[0]} forward rows")
        dev = dm.device
        dma, dSa = torch.empty_like(dm), torch.empty_like(dS)
        self.delta_mw = torch.empty(D, device=dev, dtype=torch.float32)
        self.delta_Sw = torch.empty_like(self.delta_mw)
        self.delta_mb = torch.empty_like(self.delta_mw)
        self.delta_Sb = torch.empty_like(self.delta_mw)
        ws = _lib.workspace(_lib.query("tagi_layernorm_bwd_ws_bytes", rows, D), dev)
        wp, wb = _lib.ws_args(ws)
        _lib.call("tagi_layernorm_bwd", dm.data_ptr(), dS.data_ptr(), self.ma_in.data_ptr(), self.mu_ra.data_ptr(),
                  self.var_ra.data_ptr(), self.mw.data_ptr(), self.Sw.data_ptr(), self.Sb.data_ptr(), dma.data_ptr(),
                  dSa.data_ptr(), self.delta_mw.data_ptr(), self.delta_Sw.data_ptr(), self.delta_mb.data_ptr(),
                  self.delta_Sb.data_ptr(), rows, D, float(self.eps), wp, wb, _lib.stream_of(dm))
        return dma.reshape(delta_mz.shape), dSa.reshape(delta_Sz.shape)

    def _update_items(self):
        items = [(self.mw, self.Sw, self.delta_mw, self.delta_Sw)]
        if self.has_bias:
            items.append((self.mb, self.Sb, self.delta_mb, self.delta_Sb))
        return items

    def update(self, cap_factor: float) -> None:
        for m, S, dm, dS in self._update_items():
            update_parameters(m, S, dm, dS, cap_factor)

    @property
    def num_parameters(self) -> int:
        n = self.mw.numel() + (self.mb.numel() if self.has_bias else 0)
        return 2 * n

    def __repr__(self):
        return f"LayerNorm(normalized_shape={self.normalized_shape}, eps={self.eps}, bias={self.has_bias})"
