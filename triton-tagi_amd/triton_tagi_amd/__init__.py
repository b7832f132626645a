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
    EvenSoftplus,
    Flatten,
    LayerNorm,
    Linear,
    MaxPool2D,
    MultiheadAttentionV2,
    PositionalEncoding,
    ReLU,
    Remax,
    ResBlock,
    RMSNorm,
)
from .checkpoint import RunDir, load_model
from .hrc_softmax import HierarchicalSoftmax, class_to_obs, get_predicted_labels, labels_to_hrc, obs_to_class_probs
from .network import Sequential
from .param_init import (
    gaussian_param_init,
    he_init,
    init_weight_bias_conv2d,
    init_weight_bias_linear,
    init_weight_bias_norm,
    xavier_init,
)
from .update import (
    compute_innovation,
    compute_innovation_with_indices,
    get_cap_factor,
    hrc_innovation,
    update_parameters,
)

__version__ = "0.1.0"
__all__ = [
    "Layer", "LearnableLayer", "Sequential", "Add", "AvgPool2D", "BatchNorm2D", "Conv2D", "Embedding", "Flatten",
    "Linear", "MultiheadAttentionV2", "PositionalEncoding", "RMSNorm", "ReLU", "Remax", "ResBlock", "he_init",
    "xavier_init", "gaussian_param_init", "init_weight_bias_linear", "init_weight_bias_conv2d",
    "init_weight_bias_norm", "compute_innovation", "get_cap_factor", "update_parameters", "EvenSoftplus",
    "LayerNorm", "MaxPool2D", "RunDir", "load_model", "HierarchicalSoftmax", "class_to_obs", "labels_to_hrc",
    "obs_to_class_probs", "get_predicted_labels", "compute_innovation_with_indices", "hrc_innovation",
]
