"""Output innovation (mirrors triton_tagi/update/observation.py:24-224).

Dense:            delta_mu = (y - mu) / (var + sigma_v^2),  delta_var = -1 / (var + sigma_v^2)
Heteroscedastic:  a prediction twice as wide as y holds interleaved (mean, noise-variance)
                  pairs; the noise outputs are learned (TAGI-V) instead of sigma_v.
Sparse (HRC):     the dense rule at the selected tree nodes of each row, zeros elsewhere.
"""

from __future__ import annotations

import torch

from .. import _lib


def compute_innovation(y, y_pred_mu, y_pred_var, sigma_v):
    """Innovation deltas for observations y of the predicted output (mu, var).

    If the prediction's last dimension is twice y's, the heteroscedastic rule runs
    (observation.py:137) and the deltas have the prediction's shape; sigma_v is unused.
    """
    y = _lib.check(y.contiguous(), "y")
    mu = _lib.check(y_pred_mu.contiguous(), "y_pred_mu")
    var = _lib.check(y_pred_var.contiguous(), "y_pred_var")
    if y_pred_mu.shape[-1] == 2 * y.shape[-1]:
        if mu.numel() != 2 * y.numel() or var.numel() != mu.numel():
            raise ValueError(f"compute_innovation: y {tuple(y.shape)} vs prediction {tuple(mu.shape)}")
        dm, dS = torch.empty_like(mu), torch.empty_like(var)
        _lib.call("tagi_innovation_heteros", y.data_ptr(), mu.data_ptr(), var.data_ptr(), dm.data_ptr(),
                  dS.data_ptr(), y.numel(), _lib.stream_of(y))
        return dm, dS
    if mu.numel() != y.numel() or var.numel() != y.numel():
        raise ValueError(f"compute_innovation: y {tuple(y.shape)} vs prediction {tuple(mu.shape)}")
    dm = torch.empty_like(y)
    dS = torch.empty_like(y)
    _lib.call("tagi_innovation", y.data_ptr(), mu.data_ptr(), var.data_ptr(), float(sigma_v) ** 2,
              dm.data_ptr(), dS.data_ptr(), y.numel(), _lib.stream_of(y))
    return dm, dS


def compute_innovation_with_indices(ma, Sa, y_obs, var_obs, selected_idx):
    """Sparse innovation at 1-indexed nodes ``selected_idx`` (observation.py:171-224).

    ma, Sa: (B, n_nodes); y_obs, var_obs, selected_idx: (B, n_obs). Returns (B, n_nodes)
    deltas, zero except at the selected nodes (a node selected twice gets both terms).
    """
    ma = _lib.check(ma.contiguous(), "ma")
    Sa = _lib.check(Sa.contiguous(), "Sa")
    y_obs = _lib.check(y_obs.contiguous(), "y_obs")
    var_obs = _lib.check(var_obs.contiguous(), "var_obs")
    if not isinstance(selected_idx, torch.Tensor) or selected_idx.dtype.is_floating_point:
        raise TypeError("compute_innovation_with_indices: selected_idx must be an integer tensor")
    idx = selected_idx.to(device=ma.device, dtype=torch.int32).contiguous()
    if ma.dim() != 2 or Sa.shape != ma.shape:
        raise ValueError(f"compute_innovation_with_indices: ma/Sa must be (B, n_nodes), got {tuple(ma.shape)}")
    B = ma.shape[0]
    if y_obs.dim() != 2 or y_obs.shape[0] != B or var_obs.shape != y_obs.shape or idx.shape != y_obs.shape:
        raise ValueError("compute_innovation_with_indices: y_obs, var_obs and selected_idx must be (B, n_obs)")
    dm, dS = torch.empty_like(ma), torch.empty_like(Sa)
    _lib.call("tagi_innovation_indexed", ma.data_ptr(), Sa.data_ptr(), y_obs.data_ptr(), var_obs.data_ptr(),
              idx.data_ptr(), dm.data_ptr(), dS.data_ptr(), B, ma.shape[1], y_obs.shape[1], _lib.stream_of(ma))
    return dm, dS


def hrc_innovation(ma, Sa, labels, hrc, sigma_v):
    """Sparse innovation of integer class labels on an HRC output (network.py:196-214 in
    one launch: label encoding, the constant noise sigma_v^2 and the innovation).

    ma, Sa: (N, n_nodes) with n_nodes >= hrc.len; labels: N integers. A label outside
    [0, n_classes) makes its row of deltas NaN.
    """
    ma = _lib.check(ma.contiguous(), "ma")
    Sa = _lib.check(Sa.contiguous(), "Sa")
    if ma.dim() != 2 or Sa.shape != ma.shape:
        raise ValueError(f"hrc_innovation: moments must be (N, n_nodes), got {tuple(ma.shape)}")
    if ma.shape[1] < hrc.len:
        raise ValueError(f"hrc_innovation: output width {ma.shape[1]} < tree size {hrc.len}")
    lab = labels.to(device=ma.device, dtype=torch.int64).reshape(-1).contiguous()
    if lab.numel() != ma.shape[0]:
        raise ValueError(f"hrc_innovation: {lab.numel()} labels for {ma.shape[0]} output rows")
    obs, idx = hrc.tables(ma.device)
    dm, dS = torch.empty_like(ma), torch.empty_like(Sa)
    _lib.call("tagi_hrc_innovation", ma.data_ptr(), Sa.data_ptr(), lab.data_ptr(), obs.data_ptr(), idx.data_ptr(),
              float(sigma_v) ** 2, dm.data_ptr(), dS.data_ptr(), ma.shape[0], ma.shape[1], hrc.n_obs, obs.shape[0],
              _lib.stream_of(ma))
    return dm, dS
