"""Gaussian priors of TAGI parameters (mirrors triton_tagi/param_init.py:22-198).

Means are drawn from N(0, scale) with ``torch.randn(shape, device=device)``, weights
before bias; variances are the constant (gain * scale)^2. BatchNorm/RMSNorm scales
start at mean 1 with variance gain^2 / C.
"""

from __future__ import annotations

import math

import torch


def he_init(fan_in: float) -> float:
    """He scale sqrt(1/fan_in), so the prior variance is gain^2/fan_in (param_init.py:22-36)."""
    return math.sqrt(1.0 / fan_in)


def xavier_init(fan_in: float, fan_out: float) -> float:
    """Xavier scale sqrt(2/(fan_in+fan_out)) (param_init.py:39-49)."""
    return math.sqrt(2.0 / (fan_in + fan_out))


def gaussian_param_init(scale: float, gain: float, shape, device="cuda"):
    """m ~ N(0, scale) elementwise, S = (gain*scale)^2 (param_init.py:57-78)."""
    m = torch.randn(shape, device=device) * scale
    S = torch.full(shape if isinstance(shape, tuple) else (shape,), (gain * scale) ** 2, device=device)
    return m, S


def _scale(method: str, fan_in: float, fan_out: float) -> float:
    if method.lower() == "xavier":
        return xavier_init(fan_in, fan_out)
    if method.lower() == "he":
        return he_init(fan_in)
    raise ValueError(f"Unsupported init method: {method}")


def init_weight_bias_linear(input_size, output_size, init_method="He", gain_w=1.0, gain_b=1.0, bias=True,
                            device="cuda"):
    """Linear priors: weights (in, out), bias (1, out) (param_init.py:86-126)."""
    scale = _scale(init_method, input_size, output_size)
    mu_w, var_w = gaussian_param_init(scale, gain_w, (input_size, output_size), device)
    if bias:
        mu_b, var_b = gaussian_param_init(scale, gain_b, (1, output_size), device)
    else:
        mu_b = torch.zeros(1, output_size, device=device)
        var_b = torch.zeros(1, output_size, device=device)
    return mu_w, var_w, mu_b, var_b


def init_weight_bias_conv2d(kernel_size, in_channels, out_channels, init_method="He", gain_w=1.0, gain_b=1.0,
                            device="cuda"):
    """Conv2D priors: weights (C_in*k*k, C_out) rows ordered (c, kh, kw), bias (1, C_out)
    (param_init.py:129-168)."""
    fan_in = kernel_size**2 * in_channels
    fan_out = kernel_size**2 * out_channels
    scale = _scale(init_method, fan_in, fan_out)
    K = in_channels * kernel_size * kernel_size
    mu_w, var_w = gaussian_param_init(scale, gain_w, (K, out_channels), device)
    mu_b, var_b = gaussian_param_init(scale, gain_b, (1, out_channels), device)
    return mu_w, var_w, mu_b, var_b


def init_weight_bias_norm(num_features, gain_w=1.0, gain_b=1.0, device="cuda"):
    """Normalisation priors: gamma ~ (1, gain_w^2/C), beta ~ (0, gain_b^2/C)
    (param_init.py:171-198; scale 2/(C+C))."""
    scale = 2.0 / (num_features + num_features)
    mu_gamma = torch.ones(num_features, device=device)
    var_gamma = torch.full((num_features,), scale * gain_w**2, device=device)
    mu_beta = torch.zeros(num_features, device=device)
    var_beta = torch.full((num_features,), scale * gain_b**2, device=device)
    return mu_gamma, var_gamma, mu_beta, var_beta
