"""triton_tagi_amd: the TAGI step (Tractable Approximate Gaussian Inference) on MI355X.

Drop-in for the step path of triton-tagi: the same layer classes, ``Sequential.step``
and update rules, with every moment computation in hand-written HIP kernels for gfx950
(fp32 MFMA for the moment GEMMs) behind the C ABI of ``libtagi_hip.so``.
"""

from .base import Layer, LearnableLayer
from .layers import (
    Add,
    AvgPool2D,
    BatchNorm2D,
    Conv2D,
    Embedding,
    Flatten,
    Linear,
    MultiheadAttentionV2,
    PositionalEncoding,
    ReLU,
    Remax,
    ResBlock,
    RMSNorm,
)
from .network import Sequential
from .param_init import (
    gaussian_param_init,
    he_init,
    init_weight_bias_conv2d,
    init_weight_bias_linear,
    init_weight_bias_norm,
    xavier_init,
)
from .update import compute_innovation, get_cap_factor, update_parameters

__version__ = "0.1.0"
__all__ = [
    "Layer", "LearnableLayer", "Sequential", "Add", "AvgPool2D", "BatchNorm2D", "Conv2D", "Embedding", "Flatten",
    "Linear", "MultiheadAttentionV2", "PositionalEncoding", "RMSNorm", "ReLU", "Remax", "ResBlock", "he_init",
    "xavier_init", "gaussian_param_init", "init_weight_bias_linear", "init_weight_bias_conv2d",
    "init_weight_bias_norm", "compute_innovation", "get_cap_factor", "update_parameters",
]
