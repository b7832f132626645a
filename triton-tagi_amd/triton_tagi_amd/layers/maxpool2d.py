"""Bayesian MaxPool2D, hard-argmax rule (mirrors triton_tagi/layers/maxpool2d.py:30-132).

The output takes the mean of the window position with the largest mean and the variance
at that same position; the backward pass routes each delta to that position (Jacobian 1
there, 0 elsewhere), adding up where overlapping windows picked the same input.
Tensors keep the storage order they arrive in (NCHW or channels-last).
"""

from __future__ import annotations

import torch
from torch import Tensor

from .. import _lib
from ..base import Layer


class MaxPool2D(Layer):
    def __init__(self, kernel_size: int, stride: int | None = None, padding: int = 0) -> None:
        self.kernel_size = kernel_size
        self.stride = stride if stride is not None else kernel_size
        self.padding = padding
        self.pool_idx: Tensor | None = None  # (N, C, H_out, W_out) int32, h * W + w of each pick
        self.input_shape: tuple | None = None
        self._cl = False

    def _out_hw(self, H: int, W: int) -> tuple[int, int]:
        k, s, p = self.kernel_size, self.stride, self.padding
        return (H + 2 * p - k) // s + 1, (W + 2 * p - k) // s + 1

    def forward(self, ma: Tensor, Sa: Tensor) -> tuple[Tensor, Tensor]:
        if ma.dim() != 4:
            raise ValueError(f"MaxPool2D: expected (N, C, H, W) moments, got {tuple(ma.shape)}")
        ma = _lib.check(_lib.dense(ma), "ma")
        Sa = _lib.check(_lib.like(Sa, ma), "Sa")
        N, C, H, W = ma.shape
        self.input_shape = (N, C, H, W)
        cl = not ma.is_contiguous() and ma.is_contiguous(memory_format=torch.channels_last)
        self._cl = cl
        Ho, Wo = self._out_hw(H, W)
        fmt = torch.channels_last if cl else torch.contiguous_format
        mz = torch.empty((N, C, Ho, Wo), device=ma.device, dtype=torch.float32, memory_format=fmt)
        Sz = torch.empty_like(mz)
        idx = torch.empty((N, C, Ho, Wo), device=ma.device, dtype=torch.int32, memory_format=fmt)
        _lib.call("tagi_maxpool2d_fwd", ma.data_ptr(), Sa.data_ptr(), mz.data_ptr(), Sz.data_ptr(), idx.data_ptr(),
                  N, C, H, W, self.kernel_size, self.stride, self.padding, int(cl), _lib.stream_of(ma))
        self.pool_idx = idx
        return mz, Sz

    def backward(self, delta_mz: Tensor, delta_Sz: Tensor) -> tuple[Tensor, Tensor]:
        N, C, H, W = self.input_shape
        Ho, Wo = self._out_hw(H, W)
        fmt = torch.channels_last if self._cl else torch.contiguous_format
        dm = _lib.check(delta_mz.reshape(N, C, Ho, Wo).contiguous(memory_format=fmt), "delta_mz")
        dS = _lib.check(delta_Sz.reshape(N, C, Ho, Wo).contiguous(memory_format=fmt), "delta_Sz")
        om = torch.empty((N, C, H, W), device=dm.device, dtype=torch.float32, memory_format=fmt)
        oS = torch.empty_like(om)
        _lib.call("tagi_maxpool2d_bwd", dm.data_ptr(), dS.data_ptr(), self.pool_idx.data_ptr(), om.data_ptr(),
                  oS.data_ptr(), N, C, H, W, self.kernel_size, self.stride, self.padding, int(self._cl),
                  _lib.stream_of(dm))
        return om, oS

    def __repr__(self):
        return f"MaxPool2D(kernel_size={self.kernel_size}, stride={self.stride}, padding={self.padding})"
