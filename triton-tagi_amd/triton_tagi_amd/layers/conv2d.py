"""Bayesian Conv2D layer as implicit GEMM (mirrors triton_tagi/layers/conv2d.py:189-390).

The reference unfolds patches (im2col), runs the Linear kernels on them and folds the
input deltas back (col2im). Here the three GEMMs gather patches straight from the
activation tensors inside the kernels:
    forward      mu_z = P(mu_a) @ mw + mb ;  S_z = P(mu_a)^2 @ Sw + P(S_a) @ (mw^2 + Sw) + Sb
    input delta  fold(delta_z @ mw^T) as a transposed implicit GEMM (no col2im)
    deltas       delta_mw = Sw * P^T @ delta_mz, delta_Sw = Sw^2 * (P^2)^T @ delta_Sz (+ bias)
padding_type 1 pads p on every side; padding_type 2 pads p on the right/bottom only
(conv2d.py:280-291). Activations and deltas are kept channels-last (NHWC storage of the
(N, C, H, W) tensors) so every patch row the kernels gather is a contiguous run of channels.
"""

from __future__ import annotations

import contextlib

import torch
from torch import Tensor

from .. import _lib, _overlap
from ..base import LearnableLayer
from ..param_init import init_weight_bias_conv2d
from ..update.parameters import update_parameters
from ._bn_pending import bias_deltas_formed


class Conv2D(LearnableLayer):
    """2-D convolution with Gaussian weights; mw, Sw are (C_in*k*k, C_out), rows (c, kh, kw)."""

    def __init__(self, C_in: int, C_out: int, kernel_size: int, stride: int = 1, padding: int = 0,
                 padding_type: int = 1, device: str = "cuda", init_method: str = "He", gain_w: float = 1.0,
                 gain_b: float = 1.0) -> None:
        self.C_in = C_in
        self.C_out = C_out
        self.kH = self.kW = kernel_size
        self.stride = stride
        self.padding = padding
        self.padding_type = padding_type
        self.device = torch.device(device)
        self.mw, self.Sw, self.mb, self.Sb = init_weight_bias_conv2d(
            kernel_size, C_in, C_out, init_method=init_method, gain_w=gain_w, gain_b=gain_b, device=self.device
        )
        self.has_bias = True
        self.ma_in = None
        self.input_shape = None
        self.spatial = None
        self.delta_mw = self.delta_Sw = self.delta_mb = self.delta_Sb = None

    def _geom(self, N, C, H, W) -> _lib.ConvGeom:
        k, s, p = self.kH, self.stride, self.padding
        if self.padding_type == 2 and p > 0:
            Ho, Wo, pt = (H + p - k) // s + 1, (W + p - k) // s + 1, 0
        else:
            Ho, Wo, pt = (H + 2 * p - k) // s + 1, (W + 2 * p - k) // s + 1, p
        if Ho <= 0 or Wo <= 0:
            raise ValueError(f"Conv2D: input {H}x{W} too small for kernel {k} stride {s} padding {p}")
        return _lib.ConvGeom(N, C, H, W, self.C_out, k, s, pt, pt, Ho, Wo)

    def forward(self, ma: Tensor, Sa: Tensor) -> tuple[Tensor, Tensor]:
        ma, Sa, mz, Sz, g = self._forward_prepare(ma, Sa)
        ws = _lib.workspace(_lib.query("tagi_conv2d_fwd_ws_bytes", g), mz.device)
        wp, wb = _lib.ws_args(ws)
        _lib.call("tagi_conv2d_fwd", ma.data_ptr(), _lib.ptr(Sa), self.mw.data_ptr(), self.Sw.data_ptr(),
                  self.mb.data_ptr(), self.Sb.data_ptr(), mz.data_ptr(), Sz.data_ptr(), g, wp, wb,
                  _lib.stream_of(mz))
        return mz, Sz

    def _forward_prepare(self, ma: Tensor, Sa: Tensor):
        """Checks the input, records what backward needs and allocates the output moments.

        Returns (ma, Sa, mz, Sz, geometry) with the inputs channels-last; the caller
        launches the forward. Sa None: a deterministic input (zero variance), passed on."""
        if ma.dim() != 4 or ma.shape[1] != self.C_in:
            raise ValueError(f"Conv2D: expected (N, {self.C_in}, H, W), got {tuple(ma.shape)}")
        ma = _lib.check(_lib.channels_last(ma), "ma")
        if Sa is not None:
            Sa = _lib.check(_lib.channels_last(Sa), "Sa")
            if Sa.shape != ma.shape:
                raise ValueError(f"Conv2D: Sa {tuple(Sa.shape)} does not match ma {tuple(ma.shape)}")
        N, C, H, W = ma.shape
        self.input_shape = (N, C, H, W)
        g = self._geom(N, C, H, W)
        self.spatial = (g.Ho, g.Wo)
        self.ma_in = ma
        mz = _lib.empty_cl(N, self.C_out, g.Ho, g.Wo, ma.device)
        Sz = _lib.empty_cl(N, self.C_out, g.Ho, g.Wo, ma.device)
        return ma, Sa, mz, Sz, g

    def backward(self, delta_mz: Tensor, delta_Sz: Tensor) -> tuple[Tensor, Tensor]:
        return self._backward(delta_mz, delta_Sz, True)

    def backward_param_deltas(self, delta_mz: Tensor, delta_Sz: Tensor) -> None:
        """The parameter deltas of ``backward`` without forming the input deltas."""
        self._backward(delta_mz, delta_Sz, False)

    def _output_deltas(self, delta_mz: Tensor, delta_Sz: Tensor):
        """The geometry and the output deltas as channels-last (N, C_out, Ho, Wo) tensors."""
        N, C, H, W = self.input_shape
        g = self._geom(N, C, H, W)
        dmz = _lib.check(_lib.channels_last(delta_mz.reshape(N, self.C_out, g.Ho, g.Wo)), "delta_mz")
        dSz = _lib.check(_lib.channels_last(delta_Sz.reshape(N, self.C_out, g.Ho, g.Wo)), "delta_Sz")
        if tuple(dmz.shape) != (N, self.C_out, g.Ho, g.Wo):
            raise ValueError(f"Conv2D.backward: delta shape {tuple(dmz.shape)} != output shape")
        return g, dmz, dSz

    def _backward(self, delta_mz: Tensor, delta_Sz: Tensor, input_deltas: bool,
                  add: tuple[Tensor, Tensor] | None = None):
        """Parameter deltas, then (if asked) the input deltas, plus ``add`` when given."""
        N, C, H, W = self.input_shape
        g, dmz, dSz = self._output_deltas(delta_mz, delta_Sz)
        self._param_deltas(g, dmz, dSz)
        if not input_deltas:
            return None
        dev = dmz.device
        st = _lib.stream_of(dmz)
        d_ma = _lib.empty_cl(N, C, H, W, dev)
        d_Sa = _lib.empty_cl(N, C, H, W, dev)
        ws = _lib.workspace(_lib.query("tagi_conv2d_bwd_delta_ws_bytes", g), dev)
        wp, wb = _lib.ws_args(ws)
        if add is None:
            _lib.call("tagi_conv2d_bwd_delta", dmz.data_ptr(), dSz.data_ptr(), self.mw.data_ptr(), d_ma.data_ptr(),
                      d_Sa.data_ptr(), g, wp, wb, st)
        else:
            am = _lib.check(_lib.like(add[0].reshape(N, C, H, W), d_ma), "add_m")
            aS = _lib.check(_lib.like(add[1].reshape(N, C, H, W), d_ma), "add_S")
            _lib.call("tagi_conv2d_bwd_delta_add", dmz.data_ptr(), dSz.data_ptr(), self.mw.data_ptr(),
                      am.data_ptr(), aS.data_ptr(), d_ma.data_ptr(), d_Sa.data_ptr(), g, wp, wb, st)
        return d_ma, d_Sa

    def _param_deltas(self, g, dmz: Tensor, dSz: Tensor) -> None:
        """delta_mw / delta_Sw (and the bias deltas unless a fused pass formed them), on the
        side stream of an overlapped step when the product is large."""
        N = self.input_shape[0]
        dev = dmz.device
        K = self.C_in * self.kH * self.kW
        ctx = _overlap.active()
        big = N * g.Ho * g.Wo * K * self.C_out >= _overlap.MIN_MACS_CONV
        # bias deltas already formed by the fused BatchNorm2D -> ReLU pass that produced these
        # deltas (finalized with the BatchNorm parameter deltas): no bias row in the GEMM
        bias_done = bias_deltas_formed(self)
        side = ctx.fork(dev, self.ma_in, dmz, dSz) if ctx is not None and big else None
        with torch.cuda.stream(side) if side is not None else contextlib.nullcontext():
            self.delta_mw = torch.empty(K, self.C_out, device=dev, dtype=torch.float32)
            self.delta_Sw = torch.empty_like(self.delta_mw)
            if not bias_done:
                self.delta_mb = torch.empty(1, self.C_out, device=dev, dtype=torch.float32)
                self.delta_Sb = torch.empty_like(self.delta_mb)
            ws = _lib.workspace(_lib.query("tagi_conv2d_wgrad_ws_bytes", g), dev)
            wp, wb = _lib.ws_args(ws)
            _lib.call("tagi_conv2d_wgrad", self.ma_in.data_ptr(), dmz.data_ptr(), dSz.data_ptr(), self.Sw.data_ptr(),
                      self.Sb.data_ptr(), self.delta_mw.data_ptr(), self.delta_Sw.data_ptr(),
                      None if bias_done else self.delta_mb.data_ptr(),
                      None if bias_done else self.delta_Sb.data_ptr(), g, wp, wb, _lib.stream_of(dmz))

    def _update_items(self):
        return [(self.mw, self.Sw, self.delta_mw, self.delta_Sw), (self.mb, self.Sb, self.delta_mb, self.delta_Sb)]

    def update(self, cap_factor: float) -> None:
        for m, S, dm, dS in self._update_items():
            update_parameters(m, S, dm, dS, cap_factor)

    @property
    def num_parameters(self) -> int:
        return 2 * (self.mw.numel() + self.mb.numel())

    def __repr__(self):
        return f"Conv2D({self.C_in}, {self.C_out}, kernel={self.kH}, stride={self.stride}, pad={self.padding})"
