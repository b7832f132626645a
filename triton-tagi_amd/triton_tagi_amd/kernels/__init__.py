"""Python entry points of the HIP kernels (reference names kept as aliases)."""

from .attention import bmm_shared_left, bmm_shared_right, bmm_tagi, bmm_tagi_var
from .common import (
    fused_backward_delta,
    fused_var_forward,
    fused_weight_grad,
    linear_forward,
    linear_param_deltas,
    triton_fused_backward_delta,
    triton_fused_var_forward,
    triton_fused_weight_grad,
)

__all__ = [
    "bmm_shared_left", "bmm_shared_right", "bmm_tagi", "bmm_tagi_var",
    "fused_backward_delta", "fused_var_forward", "fused_weight_grad", "linear_forward",
    "linear_param_deltas", "triton_fused_backward_delta", "triton_fused_var_forward",
    "triton_fused_weight_grad",
]
