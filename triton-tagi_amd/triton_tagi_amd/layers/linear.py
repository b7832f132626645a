"""Bayesian Linear layer (mirrors triton_tagi/layers/linear.py:30-181).

Forward (one fused fp32-MFMA launch):
    mu_z = mu_a @ mu_w + mu_b
    S_z  = mu_a^2 @ S_w + S_a @ (mu_w^2 + S_w) + S_b
Backward (deltas stored, applied by ``update``, or by the backward pass itself within
``update_in_backward``):
    delta_mw = S_w * (mu_a^T @ delta_mz)        delta_mb = S_b * sum delta_mz
    delta_Sw = S_w^2 * ((mu_a^2)^T @ delta_Sz)  delta_Sb = S_b^2 * sum delta_Sz
    delta_ma = delta_mz @ mu_w^T,  delta_Sa = delta_Sz @ (mu_w^2)^T

The parameters may be column views of a wider buffer (the projections of a
MultiheadAttentionV2 are); the kernels read and update a dense copy of such a view and
the update writes the result back into it, so a lone projection steps like any Linear.
"""

from __future__ import annotations

import contextlib

import torch
from torch import Tensor

from .. import _overlap
from ..base import LearnableLayer
from ..kernels.common import (fused_backward_delta, linear_forward, linear_param_deltas, linear_param_deltas_update,
                              linear_relu_forward)
from ..param_init import init_weight_bias_linear
from ..update import in_backward
from ..update.parameters import update_parameters


def _dense(t):
    return t if t is None or t.is_contiguous() else t.contiguous()


class Linear(LearnableLayer):
    """Fully connected layer with Gaussian weights; mw, Sw are (in, out), mb, Sb (1, out)."""

    def __init__(self, in_features: int, out_features: int, device: str = "cuda", init_method: str = "He",
                 gain_w: float = 1.0, gain_b: float = 1.0, bias: bool = True) -> None:
        self.in_features = in_features
        self.out_features = out_features
        self.device = torch.device(device)
        self.has_bias = bias
        self.mw, self.Sw, self.mb, self.Sb = init_weight_bias_linear(
            in_features, out_features, init_method=init_method, gain_w=gain_w, gain_b=gain_b, bias=bias,
            device=self.device,
        )
        self.ma_in = None
        self.delta_mw = self.delta_Sw = self.delta_mb = self.delta_Sb = None

    def _forward_input(self, ma: Tensor, Sa: Tensor | None):
        self._input_shape = ma.shape
        ma_flat = ma.reshape(-1, self.in_features).contiguous()
        # Sa None: a deterministic input (zero variance), which the kernel takes as such
        Sa_flat = None if Sa is None else Sa.reshape(-1, self.in_features).contiguous()
        self.ma_in = ma_flat
        return ma_flat, Sa_flat, (*self._input_shape[:-1], self.out_features)

    def forward(self, ma: Tensor, Sa: Tensor) -> tuple[Tensor, Tensor]:
        ma_flat, Sa_flat, out_shape = self._forward_input(ma, Sa)
        mz, Sz = linear_forward(ma_flat, Sa_flat, _dense(self.mw), _dense(self.Sw), _dense(self.mb),
                                _dense(self.Sb))
        return mz.reshape(out_shape), Sz.reshape(out_shape)

    def forward_relu(self, ma: Tensor, Sa: Tensor, relu) -> tuple[Tensor, Tensor]:
        """``forward`` followed by ``relu.forward`` in one launch: the ReLU's moments are
        formed in the product's epilogue and its Jacobian stored on ``relu`` as its own
        forward stores it; z itself is never written."""
        ma_flat, Sa_flat, out_shape = self._forward_input(ma, Sa)
        am, aS, J = linear_relu_forward(ma_flat, Sa_flat, _dense(self.mw), _dense(self.Sw), _dense(self.mb),
                                        _dense(self.Sb))
        relu.J = J.reshape(out_shape)
        return am.reshape(out_shape), aS.reshape(out_shape)

    def backward(self, delta_mz: Tensor, delta_Sz: Tensor) -> tuple[Tensor, Tensor]:
        return self._backward(delta_mz, delta_Sz, True)

    def backward_jacobian(self, delta_mz: Tensor, delta_Sz: Tensor, J: Tensor) -> tuple[Tensor, Tensor]:
        """``backward`` with the Jacobian ``J`` of the elementwise layer in front (a ReLU)
        applied in the input-delta product's epilogue: returns the deltas at that layer's
        input, as ``backward`` followed by its backward would."""
        return self._backward(delta_mz, delta_Sz, True, jacobian=J)

    def backward_param_deltas(self, delta_mz: Tensor, delta_Sz: Tensor) -> None:
        """The parameter deltas of ``backward`` without forming the input deltas."""
        self._backward(delta_mz, delta_Sz, False)

    def _backward(self, delta_mz: Tensor, delta_Sz: Tensor, input_deltas: bool, add=None, jacobian=None):
        """Parameter deltas, and the input deltas when ``input_deltas``; with ``add`` (a pair
        of contiguous tensors shaped like the input deltas) those are added to it in place
        and ``add`` is returned; with ``jacobian`` (shaped like the input) the input deltas
        are multiplied by it (variances by its square). Within ``update_in_backward`` the kernel that forms the
        parameter deltas also applies the capped update (after the input deltas, which read
        the weight means, are queued), unless that kernel goes to the side stream."""
        dmz = delta_mz.reshape(-1, self.out_features).contiguous()
        dSz = delta_Sz.reshape(-1, self.out_features).contiguous()
        ctx = _overlap.active()
        big = dmz.shape[0] * self.in_features * self.out_features >= _overlap.MIN_MACS_LINEAR
        # a parameter-delta product bound for the side stream would have to wait for the
        # input deltas before updating in place, losing its overlap (transformer block
        # -1.7%): such layers keep the update for after the backward pass
        upd = in_backward.active() if (ctx is None or not big) and self._dense_params() else None
        out = None
        if upd is not None and input_deltas:
            out = self._input_deltas(dmz, dSz, add, jacobian)
        side = ctx.fork(dmz.device, self.ma_in, dmz, dSz) if ctx is not None and big else None
        bias = (_dense(self.mb), _dense(self.Sb)) if self.has_bias else (None, None)
        with torch.cuda.stream(side) if side is not None else contextlib.nullcontext():
            if upd is not None:
                dmw, dSw, dmb, dSb = linear_param_deltas_update(self.ma_in, dmz, dSz, self.mw, self.Sw, *bias,
                                                                upd.cap_factor, upd.keep_deltas)
            else:
                dmw, dSw, dmb, dSb = linear_param_deltas(self.ma_in, dmz, dSz, _dense(self.Sw), bias[1])
        self._updated_in_backward = upd is not None
        self.delta_mw, self.delta_Sw = dmw, dSw
        if self.has_bias:
            self.delta_mb, self.delta_Sb = dmb, dSb
        if not input_deltas or upd is not None:
            return out
        return self._input_deltas(dmz, dSz, add, jacobian)

    def _input_deltas(self, dmz: Tensor, dSz: Tensor, add, jacobian=None):
        if add is not None:
            fused_backward_delta(dmz, dSz, _dense(self.mw), add=(add[0].view(-1, self.in_features),
                                                         add[1].view(-1, self.in_features)))
            return add
        J = None if jacobian is None else jacobian.reshape(-1, self.in_features).contiguous()
        dma, dSa = fused_backward_delta(dmz, dSz, _dense(self.mw), jacobian=J)
        in_shape = (*self._input_shape[:-1], self.in_features)
        return dma.reshape(in_shape), dSa.reshape(in_shape)

    def _update_items(self):
        items = [(self.mw, self.Sw, self.delta_mw, self.delta_Sw)]
        if self.has_bias:
            items.append((self.mb, self.Sb, self.delta_mb, self.delta_Sb))
        return items

    def update(self, cap_factor: float) -> None:
        if self._updated_in_backward:  # the backward pass applied it (update_in_backward)
            self._updated_in_backward = False
            return
        for m, S, dm, dS in self._update_items():
            if m.is_contiguous() and S.is_contiguous():
                update_parameters(m, S, _dense(dm), _dense(dS), cap_factor)
            else:
                mc, Sc = m.contiguous(), S.contiguous()
                update_parameters(mc, Sc, _dense(dm), _dense(dS), cap_factor)
                m.copy_(mc)
                S.copy_(Sc)

    def _dense_params(self) -> bool:
        return all(t is None or t.is_contiguous() for t in (self.mw, self.Sw, self.mb, self.Sb))

    @property
    def num_parameters(self) -> int:
        n = self.mw.numel() + (self.mb.numel() if self.has_bias else 0)
        return 2 * n

    def __repr__(self):
        return f"Linear(in={self.in_features}, out={self.out_features}, bias={self.has_bias})"
