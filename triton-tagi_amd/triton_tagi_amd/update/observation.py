"""Dense output innovation (mirrors triton_tagi/update/observation.py:24-46,119-163).

    delta_mu = (y - mu) / (var + sigma_v^2),   delta_var = -1 / (var + sigma_v^2)
"""

from __future__ import annotations

import torch

from .. import _lib


def compute_innovation(y, y_pred_mu, y_pred_var, sigma_v):
    """Innovation deltas for observations y of the predicted output (mu, var)."""
    if y_pred_mu.shape[-1] == 2 * y.shape[-1]:
        raise NotImplementedError(
            "heteroscedastic (2x-wide) output heads are not part of this engine's step path"
        )
    y = _lib.check(y.contiguous(), "y")
    mu = _lib.check(y_pred_mu.contiguous(), "y_pred_mu")
    var = _lib.check(y_pred_var.contiguous(), "y_pred_var")
    if mu.numel() != y.numel() or var.numel() != y.numel():
        raise ValueError(f"compute_innovation: y {tuple(y.shape)} vs prediction {tuple(mu.shape)}")
    dm = torch.empty_like(y)
    dS = torch.empty_like(y)
    _lib.call("tagi_innovation", y.data_ptr(), mu.data_ptr(), var.data_ptr(), float(sigma_v) ** 2,
              dm.data_ptr(), dS.data_ptr(), y.numel(), _lib.stream_of(y))
    return dm, dS
