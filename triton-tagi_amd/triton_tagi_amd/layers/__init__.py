"""TAGI layers on HIP kernels."""

from .avgpool2d import AvgPool2D
from .batchnorm2d import BatchNorm2D
from .conv2d import Conv2D
from .embedding import Embedding
from .even_softplus import EvenSoftplus, even_softplus
from .flatten import Flatten
from .layernorm import LayerNorm
from .linear import Linear
from .maxpool2d import MaxPool2D
from .multihead_attention import MultiheadAttentionV2
from .positional_encoding import PositionalEncoding
from .relu import ReLU, bayesian_relu
from .remax import Remax, remax, triton_remax
from .resblock import Add, ResBlock, add_shortcut, delta_merge, triton_add_shortcut, triton_delta_merge
from .rms_norm import RMSNorm

__all__ = [
    "Add", "AvgPool2D", "BatchNorm2D", "Conv2D", "Embedding", "EvenSoftplus", "Flatten", "LayerNorm", "Linear",
    "MaxPool2D", "MultiheadAttentionV2", "even_softplus",
    "PositionalEncoding", "RMSNorm", "ReLU", "Remax", "ResBlock", "add_shortcut", "bayesian_relu", "delta_merge",
    "remax", "triton_add_shortcut", "triton_delta_merge", "triton_remax",
]
