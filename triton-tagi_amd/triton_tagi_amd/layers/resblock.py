"""Residual block and moment add (mirrors triton_tagi/layers/resblock.py:138-472).

Main path Conv3x3(stride) -> ReLU -> BN -> Conv3x3 -> ReLU -> BN; shortcut is identity
or, when the stride or the channel count changes, Conv 2x2 stride 2 -> ReLU -> BN. The
block output is main + shortcut (means and variances add; no post-activation).
Backward sends the incoming deltas to both branches and sums what comes back.

Layers here never write their inputs, so neither direction needs the reference's
defensive copies: the add writes into the main branch's fresh output.
"""

from __future__ import annotations

import torch
from torch import Tensor

from .. import _lib
from ..base import LearnableLayer
from .batchnorm2d import BatchNorm2D
from .conv2d import Conv2D
from .relu import ReLU


def add_shortcut(mu_s, var_s, mu_a, var_a) -> None:
    """In place: mu_a += mu_s, var_a += var_s (resblock.py:138-154)."""
    assert mu_s.shape == mu_a.shape, f"Shape mismatch: shortcut={mu_s.shape} vs output={mu_a.shape}"
    _lib.check(mu_a, "mu_a"), _lib.check(var_a, "var_a")
    if var_a.stride() != mu_a.stride():
        raise ValueError("add_shortcut: mu_a and var_a must share one storage order")
    mu_s = _lib.check(_lib.like(mu_s, mu_a), "mu_s")
    var_s = _lib.check(_lib.like(var_s, mu_a), "var_s")
    _lib.call("tagi_add_inplace", mu_s.data_ptr(), var_s.data_ptr(), mu_a.data_ptr(), var_a.data_ptr(),
              mu_s.numel(), _lib.stream_of(mu_a))


def delta_merge(d_mu_skip, d_var_skip, d_mu_out, d_var_out) -> None:
    """In place: d_mu_out += d_mu_skip, d_var_out += d_var_skip (resblock.py:157-175)."""
    assert d_mu_skip.shape == d_mu_out.shape, f"Shape mismatch: skip={d_mu_skip.shape} vs out={d_mu_out.shape}"
    add_shortcut(d_mu_skip, d_var_skip, d_mu_out, d_var_out)


triton_add_shortcut = add_shortcut
triton_delta_merge = delta_merge


class Add:
    """Element-wise sum of two Gaussian streams (resblock.py:183-213)."""

    def forward(self, mu_z, var_z, mu_x, var_x):
        assert mu_z.shape == mu_x.shape
        mu_s, var_s = mu_z.clone(), var_z.clone()
        add_shortcut(mu_x, var_x, mu_s, var_s)
        return mu_s, var_s

    def backward(self, delta_mu_s, delta_var_s):
        return (delta_mu_s.clone(), delta_var_s.clone()), (delta_mu_s.clone(), delta_var_s.clone())

    def __repr__(self):
        return "Add()"


class ResBlock(LearnableLayer):
    def __init__(self, in_channels: int, out_channels: int, stride: int = 1, device: str = "cuda",
                 gain_w: float = 1.0, gain_b: float = 1.0) -> None:
        self.in_channels = in_channels
        self.out_channels = out_channels
        self.stride = stride
        self.device = device
        self.training = True
        kw = dict(device=device, gain_w=gain_w, gain_b=gain_b)
        self.conv1 = Conv2D(in_channels, out_channels, kernel_size=3, stride=stride, padding=1,
                            padding_type=2 if stride > 1 else 1, **kw)
        self.relu1 = ReLU()
        self.bn1 = BatchNorm2D(out_channels, preserve_var=False, **kw)
        self.conv2 = Conv2D(out_channels, out_channels, kernel_size=3, stride=1, padding=1, **kw)
        self.relu2 = ReLU()
        self.bn2 = BatchNorm2D(out_channels, preserve_var=False, **kw)
        self._main_layers = [self.conv1, self.relu1, self.bn1, self.conv2, self.relu2, self.bn2]
        self.use_projection = (stride != 1) or (in_channels != out_channels)
        if self.use_projection:
            self.proj_conv = Conv2D(in_channels, out_channels, kernel_size=2, stride=stride, padding=0, **kw)
            self.proj_relu = ReLU()
            self.proj_bn = BatchNorm2D(out_channels, preserve_var=False, **kw)
            self._proj_layers = [self.proj_conv, self.proj_relu, self.proj_bn]
        else:
            self.proj_conv = self.proj_relu = self.proj_bn = None
            self._proj_layers = []
        self._learnable = [self.conv1, self.bn1, self.conv2, self.bn2]
        if self.use_projection:
            self._learnable.extend([self.proj_conv, self.proj_bn])

    def sublayers(self) -> tuple:
        return tuple(self._main_layers + self._proj_layers)

    def train(self) -> None:
        self.training = True
        for layer in self._learnable:
            if hasattr(layer, "train"):
                layer.train()

    def eval(self) -> None:
        self.training = False
        for layer in self._learnable:
            if hasattr(layer, "eval"):
                layer.eval()

    def forward(self, mu_in: Tensor, var_in: Tensor) -> tuple[Tensor, Tensor]:
        """main(x) + shortcut(x) (resblock.py:354-385). The shortcut runs first so its
        output can be added inside the main branch's last pass."""
        from .fused import forward_chain

        mu_x, var_x = forward_chain(self._proj_layers, mu_in, var_in) if self._proj_layers else (mu_in, var_in)
        return forward_chain(self._main_layers, mu_in, var_in, add=(mu_x, var_x))

    def backward(self, delta_mu: Tensor, delta_var: Tensor) -> tuple[Tensor, Tensor]:
        """Deltas through both branches, summed (resblock.py:387-430); the shortcut's
        deltas are added inside the main branch's first input-delta GEMM."""
        from .fused import resblock_backward

        return resblock_backward(self, delta_mu, delta_var)

    def _update_items(self):
        items = []
        for layer in self._learnable:
            items.extend(layer._update_items())
        return items

    def update(self, cap_factor: float) -> None:
        for layer in self._learnable:
            layer.update(cap_factor)

    @property
    def mw(self):
        return self.conv1.mw

    @mw.setter
    def mw(self, value):
        self.conv1.mw = value

    @property
    def Sw(self):
        return self.conv1.Sw

    @property
    def mb(self):
        return self.conv1.mb

    @property
    def Sb(self):
        return self.conv1.Sb

    @property
    def num_parameters(self) -> int:
        return sum(layer.num_parameters for layer in self._learnable)

    def __repr__(self):
        proj = "projection" if self.use_projection else "identity"
        return f"ResBlock({self.in_channels}→{self.out_channels}, stride={self.stride}, skip={proj})"
