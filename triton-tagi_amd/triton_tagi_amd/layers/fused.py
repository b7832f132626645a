"""Fused passes over consecutive layers of the step.

Running a layer list through ``forward_chain`` / ``backward_chain`` gives the same
results as calling every layer's own ``forward`` / ``backward`` in turn. It differs only
in how often activations cross HBM:

* ReLU followed by a training-mode BatchNorm2D (relu.py:135-140, batchnorm2d.py:360-431)
  runs as two passes over the ReLU input: the first forms the batch statistics of the
  rectified moments (and the ReLU Jacobian), the second recomputes the rectified moments
  and normalises them. The ReLU output is never written.
* When a Conv2D produces that ReLU input, the first pass is the convolution's own GEMM
  epilogue (conv2d.py:254-309): the output moments are not read back for the statistics.
* The residual add that closes a block (resblock.py:380) is folded into that second pass.
* Backward through BatchNorm2D and the ReLU in front of it (batchnorm2d.py:465-513,
  relu.py:152-169) is one pass; within ``Sequential.step``, where a stride-1 Conv2D
  follows the pair, that pass is the epilogue of the Conv2D's input-delta GEMM.
* The merge of the shortcut deltas into the main branch (resblock.py:421-423) is folded
  into the input-delta GEMM of the block's first convolution.
* Within ``Sequential.step``, when that convolution has stride 1, the same GEMM also runs
  the BatchNorm2D -> ReLU backward of the layers in front of the block (the previous
  block's closing pair, or the stem's): the block's input deltas are still stored (the
  previous block's shortcut reads them) and the previous block's backward starts at its
  second convolution.
* ReLU followed by AvgPool2D (relu.py:94-122, avgpool2d.py:38-90) is one pass that writes
  the ReLU Jacobian and the pooled moments, not the ReLU output; backward, the pooling's
  deltas and the Jacobian are one pass as well (when H and W are multiples of the window).
  Before a Flatten the pooled moments are written row-major (N, C, H, W), so the Flatten
  is a view each way instead of two layout copies.

Every layer still ends up holding the state its own ``backward`` reads (ReLU.J,
BatchNorm2D.m_hat and its normalisation variance, Conv2D.ma_in), so per-layer calls keep
working after a fused pass.
"""

from __future__ import annotations

import torch
from torch import Tensor

from .. import _lib
from ._bn_pending import active as _active_defer
from ._bn_pending import defer_bn_parameter_deltas  # noqa: F401  (re-exported)
from .avgpool2d import AvgPool2D
from .batchnorm2d import BatchNorm2D
from .conv2d import Conv2D
from .flatten import Flatten
from .linear import Linear
from .relu import ReLU
from .resblock import ResBlock


def _add_in_place(src_m: Tensor, src_S: Tensor, dst_m: Tensor, dst_S: Tensor) -> None:
    from .resblock import add_shortcut

    add_shortcut(src_m, src_S, dst_m, dst_S)


def _stats_args(bn: BatchNorm2D, C: int, dev) -> tuple[Tensor, Tensor, tuple]:
    """Batch-statistic outputs and the running-stat arguments shared by the first passes."""
    if not bn.training:
        raise ValueError("relu_bn_forward: the BatchNorm2D must be in training mode")
    if C != bn.num_features:
        raise ValueError(f"BatchNorm2D: expected {bn.num_features} channels, got {C}")
    bmean = torch.empty(C, device=dev, dtype=torch.float32)
    bvar = torch.empty(C, device=dev, dtype=torch.float32)
    tail = (_lib.check(bn.running_mean, "running_mean").data_ptr(),
            _lib.check(bn.running_var, "running_var").data_ptr(), _lib.check(bn.mw, "mw").data_ptr())
    return bmean, bvar, tail


def relu_bn_forward(relu: ReLU, bn: BatchNorm2D, mz: Tensor, Sz: Tensor,
                    add: tuple[Tensor, Tensor] | None = None) -> tuple[Tensor, Tensor]:
    """BatchNorm2D(ReLU(mz, Sz)) in training mode, plus ``add`` when given."""
    mz = _lib.check(_lib.channels_last(mz), "mz")
    Sz = _lib.check(_lib.channels_last(Sz), "Sz")
    if mz.dim() != 4 or Sz.shape != mz.shape:
        raise ValueError(f"relu_bn_forward: expected matching (N, C, H, W) moments, got {tuple(mz.shape)}")
    N, C, H, W = mz.shape
    dev = mz.device
    bmean, bvar, tail = _stats_args(bn, C, dev)
    J = torch.empty_like(mz)
    first = not bn._is_initialized
    ws = _lib.workspace(_lib.query("tagi_bn_stats_ws_bytes", N, C, H * W), dev)
    wp, wb = _lib.ws_args(ws)
    _lib.call("tagi_relu_bn_stats", mz.data_ptr(), Sz.data_ptr(), J.data_ptr(), bmean.data_ptr(), bvar.data_ptr(),
              *tail, N, C, H * W, float(bn.momentum), float(bn.eps), int(first), int(bn.preserve_var), wp, wb,
              _lib.stream_of(mz))
    return _relu_bn_apply(relu, bn, mz, Sz, J, bmean, bvar, add)


def conv_relu_bn_forward(conv: Conv2D, relu: ReLU, bn: BatchNorm2D, ma: Tensor, Sa: Tensor,
                         add: tuple[Tensor, Tensor] | None = None) -> tuple[Tensor, Tensor]:
    """BatchNorm2D(ReLU(Conv2D(ma, Sa))) in training mode, plus ``add`` when given."""
    ma, Sa, mz, Sz, geom = conv._forward_prepare(ma, Sa)
    N, C, H, W = mz.shape
    dev = mz.device
    bmean, bvar, tail = _stats_args(bn, C, dev)
    J = torch.empty_like(mz)
    first = not bn._is_initialized
    ws = _lib.workspace(_lib.query("tagi_conv2d_fwd_relu_bn_stats_ws_bytes", geom), dev)
    wp, wb = _lib.ws_args(ws)
    _lib.call("tagi_conv2d_fwd_relu_bn_stats", ma.data_ptr(), _lib.ptr(Sa), conv.mw.data_ptr(),
              conv.Sw.data_ptr(), conv.mb.data_ptr(), conv.Sb.data_ptr(), mz.data_ptr(), Sz.data_ptr(), geom,
              J.data_ptr(), bmean.data_ptr(), bvar.data_ptr(), *tail, float(bn.momentum), float(bn.eps), int(first),
              int(bn.preserve_var), wp, wb, _lib.stream_of(mz))
    return _relu_bn_apply(relu, bn, mz, Sz, J, bmean, bvar, add)


def _relu_bn_apply(relu: ReLU, bn: BatchNorm2D, mz: Tensor, Sz: Tensor, J: Tensor, bmean: Tensor, bvar: Tensor,
                   add: tuple[Tensor, Tensor] | None) -> tuple[Tensor, Tensor]:
    """Second pass: normalise the rectified moments (batch statistics already formed)."""
    N, C, H, W = mz.shape
    HW = H * W
    st = _lib.stream_of(mz)
    bn._is_initialized = True
    relu.J = J
    am = aS = None
    if add is not None:
        am = _lib.check(_lib.like(add[0], mz), "add_m")
        aS = _lib.check(_lib.like(add[1], mz), "add_S")
        if am.shape != mz.shape or aS.shape != mz.shape:
            raise ValueError(f"relu_bn_forward: addend {tuple(am.shape)} vs output {tuple(mz.shape)}")
    ma, Sa, mhat = torch.empty_like(mz), torch.empty_like(mz), torch.empty_like(mz)
    _lib.call("tagi_relu_bn_fwd", mz.data_ptr(), Sz.data_ptr(), bmean.data_ptr(), bvar.data_ptr(), bn.mw.data_ptr(),
              _lib.check(bn.Sw, "Sw").data_ptr(), _lib.check(bn.mb, "mb").data_ptr(),
              _lib.check(bn.Sb, "Sb").data_ptr(), _lib.ptr(am), _lib.ptr(aS), ma.data_ptr(), Sa.data_ptr(),
              mhat.data_ptr(), N, C, HW, float(bn.eps), st)
    bn.input_shape = mz.shape
    bn._norm_var = bvar
    bn.m_hat = mhat
    return ma, Sa


def bn_relu_backward(bn: BatchNorm2D, relu: ReLU, delta_ma: Tensor, delta_Sa: Tensor,
                     conv: Conv2D | None = None) -> tuple[Tensor, Tensor]:
    """relu.backward(*bn.backward(delta_ma, delta_Sa)) in one pass; stores the BN deltas.

    Within ``defer_bn_parameter_deltas``, ``conv`` (the Conv2D whose output the ReLU
    takes) gets its bias deltas from the same pass: the column sums of the returned
    deltas are formed with the BN sums (conv2d.py:341-354), and the conv's parameter-delta
    GEMM then runs without its bias row."""
    dma = _lib.check(_lib.channels_last(delta_ma.reshape(bn.input_shape)), "delta_ma")
    dSa = _lib.check(_lib.channels_last(delta_Sa.reshape(bn.input_shape)), "delta_Sa")
    J = _lib.check(_lib.like(relu.J, dma), "J")
    if J.shape != dma.shape:
        raise ValueError(f"bn_relu_backward: stored Jacobian {tuple(J.shape)} vs delta {tuple(dma.shape)}")
    N, C, H, W = bn.input_shape
    HW = H * W
    dev = dma.device
    dmz, dSz = torch.empty_like(dma), torch.empty_like(dSa)
    bn.delta_mw = torch.empty(C, device=dev, dtype=torch.float32)
    bn.delta_Sw = torch.empty_like(bn.delta_mw)
    bn.delta_mb = torch.empty_like(bn.delta_mw)
    bn.delta_Sb = torch.empty_like(bn.delta_mw)
    ws = _lib.workspace(_lib.query("tagi_bn_bwd_ws_bytes", N, C, HW), dev)
    wp, wb = _lib.ws_args(ws)
    ctx = _active_defer()
    if ctx is not None and conv is not None and conv.C_out == C and conv.mb is not None:
        conv.delta_mb = torch.empty(1, C, device=dev, dtype=torch.float32)
        conv.delta_Sb = torch.empty_like(conv.delta_mb)
        ws = _lib.workspace(_lib.query("tagi_bn_relu_bwd_bias_ws_bytes", N, C, HW), dev)
        wp, wb = _lib.ws_args(ws)
        _lib.call("tagi_bn_relu_bwd_partials_bias", dma.data_ptr(), dSa.data_ptr(), bn.m_hat.data_ptr(),
                  J.data_ptr(), bn._norm_var.data_ptr(), bn.mw.data_ptr(), dmz.data_ptr(), dSz.data_ptr(), N, C, HW,
                  float(bn.eps), wp, wb, _lib.stream_of(dma))
        ctx.add(bn, ws, N, C, HW, conv=conv)
        return dmz, dSz
    if ctx is not None:
        _lib.call("tagi_bn_relu_bwd_partials", dma.data_ptr(), dSa.data_ptr(), bn.m_hat.data_ptr(), J.data_ptr(),
                  bn._norm_var.data_ptr(), bn.mw.data_ptr(), dmz.data_ptr(), dSz.data_ptr(), N, C, HW,
                  float(bn.eps), wp, wb, _lib.stream_of(dma))
        ctx.add(bn, ws, N, C, HW)
        return dmz, dSz
    _lib.call("tagi_bn_relu_bwd", dma.data_ptr(), dSa.data_ptr(), bn.m_hat.data_ptr(), J.data_ptr(),
              bn._norm_var.data_ptr(), bn.mw.data_ptr(), bn.Sw.data_ptr(), bn.Sb.data_ptr(), dmz.data_ptr(),
              dSz.data_ptr(), bn.delta_mw.data_ptr(), bn.delta_Sw.data_ptr(), bn.delta_mb.data_ptr(),
              bn.delta_Sb.data_ptr(), N, C, HW, float(bn.eps), wp, wb, _lib.stream_of(dma))
    return dmz, dSz


def conv_bn_relu_backward(conv: Conv2D, bn: BatchNorm2D, relu: ReLU, conv_prev: Conv2D, delta_ma: Tensor,
                          delta_Sa: Tensor) -> tuple[Tensor, Tensor] | None:
    """``conv.backward`` followed by ``bn_relu_backward(bn, relu, ..., conv_prev)`` for the
    layer order conv_prev -> relu -> bn -> conv, with the BatchNorm2D -> ReLU backward
    folded into the epilogue of conv's input-delta GEMM: the deltas at the BatchNorm2D
    output are never written. Within ``defer_bn_parameter_deltas`` only (the pass leaves
    its partial sums pending, conv_prev's bias sums among them); returns None, having done
    nothing, where the fold does not apply (then the caller runs the two steps)."""
    ctx = _active_defer()
    if ctx is None or conv_prev.mb is None or bn.m_hat is None or relu.J is None:
        return None
    N, C, H, W = conv.input_shape
    if (conv_prev.C_out != C or tuple(bn.input_shape) != (N, C, H, W) or tuple(bn.m_hat.shape) != (N, C, H, W)
            or tuple(relu.J.shape) != (N, C, H, W)):
        return None
    g = conv._geom(N, C, H, W)
    part_bytes = _lib.query("tagi_conv2d_bwd_delta_bn_relu_part_bytes", g)
    if part_bytes <= 0:
        return None
    g, dmz, dSz = conv._output_deltas(delta_ma, delta_Sa)
    if any(t.data_ptr() % 16 for t in (dmz, dSz, conv.mw)):
        return None  # the fold reads the deltas and weights as float4
    conv._param_deltas(g, dmz, dSz)
    dev = dmz.device
    d_ma = _lib.empty_cl(N, C, H, W, dev)
    d_Sa = _lib.empty_cl(N, C, H, W, dev)
    mhat = _lib.check(_lib.like(bn.m_hat, d_ma), "m_hat")
    J = _lib.check(_lib.like(relu.J, d_ma), "J")
    bn.delta_mw = torch.empty(C, device=dev, dtype=torch.float32)
    bn.delta_Sw = torch.empty_like(bn.delta_mw)
    bn.delta_mb = torch.empty_like(bn.delta_mw)
    bn.delta_Sb = torch.empty_like(bn.delta_mw)
    conv_prev.delta_mb = torch.empty(1, C, device=dev, dtype=torch.float32)
    conv_prev.delta_Sb = torch.empty_like(conv_prev.delta_mb)
    part = _lib.workspace(part_bytes, dev)
    ws = _lib.workspace(_lib.query("tagi_conv2d_bwd_delta_ws_bytes", g), dev)
    wp, wb = _lib.ws_args(ws)
    _lib.call("tagi_conv2d_bwd_delta_bn_relu", dmz.data_ptr(), dSz.data_ptr(), conv.mw.data_ptr(), mhat.data_ptr(),
              J.data_ptr(), _lib.check(bn._norm_var, "norm_var").data_ptr(), _lib.check(bn.mw, "mw").data_ptr(),
              float(bn.eps), d_ma.data_ptr(), d_Sa.data_ptr(), part.data_ptr(), part_bytes, g, wp, wb,
              _lib.stream_of(dmz))
    ctx.add(bn, part, N, C, H * W, conv=conv_prev, nblk=part_bytes // (24 * C))
    return d_ma, d_Sa


def conv_add_bn_relu_backward(conv: Conv2D, delta_ma: Tensor, delta_Sa: Tensor, add: tuple[Tensor, Tensor],
                              bn: BatchNorm2D, relu: ReLU, conv_prev: Conv2D):
    """``conv._backward(delta, True, add=add)`` (a residual block's first convolution, the
    shortcut's deltas added) followed by ``bn_relu_backward(bn, relu, ..., conv_prev)`` for
    the layers conv_prev -> relu -> bn in front of the block, in one input-delta GEMM whose
    epilogue stores both. Returns ((d_ma, d_Sa), (d_mz, d_Sz)): the deltas at the block's
    input and at conv_prev's output; or None, having done nothing, where the fold does not
    apply (outside ``defer_bn_parameter_deltas``, stride 2, split plans). The BatchNorm2D
    parameter deltas and conv_prev's bias deltas are left pending, as in
    ``conv_bn_relu_backward``."""
    ctx = _active_defer()
    if ctx is None or conv_prev.mb is None or bn.m_hat is None or relu.J is None:
        return None
    N, C, H, W = conv.input_shape
    if (conv_prev.C_out != C or tuple(bn.input_shape) != (N, C, H, W) or tuple(bn.m_hat.shape) != (N, C, H, W)
            or tuple(relu.J.shape) != (N, C, H, W)):
        return None
    g = conv._geom(N, C, H, W)
    part_bytes = _lib.query("tagi_conv2d_bwd_delta_bn_relu_part_bytes", g)
    if part_bytes <= 0:
        return None
    g, dmz, dSz = conv._output_deltas(delta_ma, delta_Sa)
    if any(t.data_ptr() % 16 for t in (dmz, dSz, conv.mw)):
        return None  # the fold reads the deltas and weights as float4
    conv._param_deltas(g, dmz, dSz)
    dev = dmz.device
    d_ma = _lib.empty_cl(N, C, H, W, dev)
    d_Sa = _lib.empty_cl(N, C, H, W, dev)
    am = _lib.check(_lib.like(add[0].reshape(N, C, H, W), d_ma), "add_m")
    aS = _lib.check(_lib.like(add[1].reshape(N, C, H, W), d_ma), "add_S")
    d_mz = _lib.empty_cl(N, C, H, W, dev)
    d_Sz = _lib.empty_cl(N, C, H, W, dev)
    mhat = _lib.check(_lib.like(bn.m_hat, d_ma), "m_hat")
    J = _lib.check(_lib.like(relu.J, d_ma), "J")
    bn.delta_mw = torch.empty(C, device=dev, dtype=torch.float32)
    bn.delta_Sw = torch.empty_like(bn.delta_mw)
    bn.delta_mb = torch.empty_like(bn.delta_mw)
    bn.delta_Sb = torch.empty_like(bn.delta_mw)
    conv_prev.delta_mb = torch.empty(1, C, device=dev, dtype=torch.float32)
    conv_prev.delta_Sb = torch.empty_like(conv_prev.delta_mb)
    part = _lib.workspace(part_bytes, dev)
    ws = _lib.workspace(_lib.query("tagi_conv2d_bwd_delta_ws_bytes", g), dev)
    wp, wb = _lib.ws_args(ws)
    _lib.call("tagi_conv2d_bwd_delta_add_bn_relu", dmz.data_ptr(), dSz.data_ptr(), conv.mw.data_ptr(),
              am.data_ptr(), aS.data_ptr(), d_ma.data_ptr(), d_Sa.data_ptr(), mhat.data_ptr(), J.data_ptr(),
              _lib.check(bn._norm_var, "norm_var").data_ptr(), _lib.check(bn.mw, "mw").data_ptr(), float(bn.eps),
              d_mz.data_ptr(), d_Sz.data_ptr(), part.data_ptr(), part_bytes, g, wp, wb, _lib.stream_of(dmz))
    ctx.add(bn, part, N, C, H * W, conv=conv_prev, nblk=part_bytes // (24 * C))
    return (d_ma, d_Sa), (d_mz, d_Sz)


class _Fold:
    """The layers conv -> relu -> bn in front of a residual block, whose backward the
    block's first input-delta GEMM may take over; ``out`` receives the deltas at conv's
    output when it does."""

    __slots__ = ("conv", "relu", "bn", "out")

    def __init__(self, conv: Conv2D, relu: ReLU, bn: BatchNorm2D) -> None:
        self.conv, self.relu, self.bn = conv, relu, bn
        self.out = None


def _fold_in_front(layers, i: int):
    """A _Fold for the layers in front of the ResBlock ``layers[i]`` (the previous block's
    closing conv2 -> relu2 -> bn2, or three such layers of the list), or None."""
    if _active_defer() is None or i < 1:
        return None
    prev = layers[i - 1]
    if isinstance(prev, ResBlock):
        tail = prev._main_layers[3:6]
    elif i >= 3:
        tail = layers[i - 3:i]
    else:
        return None
    conv, relu, bn = tail
    if isinstance(conv, Conv2D) and _fusable_backward(bn, relu):
        return _Fold(conv, relu, bn)
    return None


def resblock_backward(block: ResBlock, delta_mu: Tensor, delta_var: Tensor, start=None, fold: _Fold | None = None):
    """Deltas at the block's input (resblock.py:387-430). ``start``: the deltas at conv2's
    output, when the next block's first input-delta GEMM already ran this block's closing
    BatchNorm2D -> ReLU backward; ``fold``: the layers in front of this block, whose
    backward this block's first input-delta GEMM then runs (``fold.out`` is set if it did)."""
    if block._proj_layers:
        d_skip = backward_chain(block._proj_layers, delta_mu, delta_var)
    else:
        d_skip = (delta_mu, delta_var)
    if start is None:
        return backward_chain(block._main_layers, delta_mu, delta_var, add=d_skip, fold=fold)
    return backward_chain(block._main_layers[:4], start[0], start[1], add=d_skip, fold=fold)


def relu_avgpool_forward(relu: ReLU, pool: AvgPool2D, mz: Tensor, Sz: Tensor,
                         nchw: bool = False) -> tuple[Tensor, Tensor]:
    """pool.forward(*relu.forward(mz, Sz)) in one pass; stores relu.J and the pool's input
    shape, as the two calls do. With ``nchw`` the pooled moments are row-major (N, C, H, W)
    tensors, which a following Flatten reshapes without a copy; channels-last otherwise."""
    mz = _lib.check(_lib.channels_last(mz), "mz")
    Sz = _lib.check(_lib.like(Sz, mz), "Sz")
    N, C, H, W = mz.shape
    k = pool.k
    J = torch.empty_like(mz)
    if nchw:
        mo = torch.empty((N, C, H // k, W // k), device=mz.device, dtype=torch.float32)
        So = torch.empty_like(mo)
    else:
        mo = _lib.empty_cl(N, C, H // k, W // k, mz.device)
        So = _lib.empty_cl(N, C, H // k, W // k, mz.device)
    _lib.call("tagi_relu_avgpool2d_fwd", mz.data_ptr(), Sz.data_ptr(), J.data_ptr(), mo.data_ptr(), So.data_ptr(),
              N, C, H, W, k, pool._var_scale(), int(nchw), _lib.stream_of(mz))
    relu.J = J
    pool.input_shape = mz.shape
    return mo, So


def avgpool_relu_backward(pool: AvgPool2D, relu: ReLU, delta_m: Tensor, delta_S: Tensor) -> tuple[Tensor, Tensor]:
    """relu.backward(*pool.backward(delta_m, delta_S)) in one pass. Row-major pooled deltas
    (what Flatten passes back) are read in place; any other layout goes through a
    channels-last copy."""
    N, C, H, W = pool.input_shape
    k = pool.k
    dm = delta_m.reshape(N, C, H // k, W // k)
    dS = delta_S.reshape(N, C, H // k, W // k)
    nchw = dm.is_contiguous() and dS.is_contiguous()
    if not nchw:
        dm, dS = _lib.channels_last(dm), _lib.channels_last(dS)
    dm, dS = _lib.check(dm, "delta_m"), _lib.check(dS, "delta_S")
    J = _lib.check(_lib.channels_last(relu.J), "J")
    om = _lib.empty_cl(N, C, H, W, dm.device)
    oS = _lib.empty_cl(N, C, H, W, dm.device)
    _lib.call("tagi_avgpool2d_relu_bwd", dm.data_ptr(), dS.data_ptr(), J.data_ptr(), om.data_ptr(), oS.data_ptr(),
              N, C, H, W, k, pool._var_scale(), int(nchw), _lib.stream_of(dm))
    return om, oS


def _fusable_relu_pool(layer, nxt, mu: Tensor) -> bool:
    return (isinstance(layer, ReLU) and isinstance(nxt, AvgPool2D) and mu.dim() == 4
            and mu.shape[2] % nxt.k == 0 and mu.shape[3] % nxt.k == 0)


def _fusable_pool_relu_backward(layer, prev) -> bool:
    if not (isinstance(layer, AvgPool2D) and isinstance(prev, ReLU) and prev.J is not None
            and layer.input_shape is not None):
        return False
    N, C, H, W = layer.input_shape
    return tuple(prev.J.shape) == (N, C, H, W) and H % layer.k == 0 and W % layer.k == 0


def _fusable_forward(layer, nxt, mu: Tensor) -> bool:
    return isinstance(layer, ReLU) and isinstance(nxt, BatchNorm2D) and nxt.training and mu.dim() == 4


def _fusable_conv_forward(layers, i: int, mu: Tensor) -> bool:
    return (i + 2 < len(layers) and isinstance(layers[i], Conv2D) and mu.dim() == 4
            and _fusable_forward(layers[i + 1], layers[i + 2], mu))


def _fusable_backward(layer, prev) -> bool:
    return (isinstance(layer, BatchNorm2D) and isinstance(prev, ReLU) and prev.J is not None
            and layer.m_hat is not None and tuple(prev.J.shape) == tuple(layer.m_hat.shape))


def forward_chain(layers, mu: Tensor, var: Tensor,
                  add: tuple[Tensor, Tensor] | None = None) -> tuple[Tensor, Tensor]:
    """Forward through ``layers`` in order; ``add`` is added to the final output."""
    i, n = 0, len(layers)
    while i < n:
        layer = layers[i]
        nxt = layers[i + 1] if i + 1 < n else None
        if _fusable_conv_forward(layers, i, mu):
            last = i + 3 == n
            mu, var = conv_relu_bn_forward(layer, nxt, layers[i + 2], mu, var, add if last else None)
            if last:
                add = None
            i += 3
        elif _fusable_forward(layer, nxt, mu):
            last = i + 2 == n
            mu, var = relu_bn_forward(layer, nxt, mu, var, add if last else None)
            if last:
                add = None
            i += 2
        elif isinstance(layer, Linear) and isinstance(nxt, ReLU) and mu.is_cuda:
            # the ReLU's moments formed in the Linear product's epilogue
            mu, var = layer.forward_relu(mu, var, nxt)
            i += 2
        elif _fusable_relu_pool(layer, nxt, mu):
            # pooled moments in the row-major layout a following Flatten views as is
            mu, var = relu_avgpool_forward(layer, nxt, mu, var, nchw=i + 2 < n and isinstance(layers[i + 2], Flatten))
            i += 2
        else:
            mu, var = layer.forward(mu, var)
            i += 1
    if add is not None:
        _add_in_place(add[0], add[1], mu, var)
    return mu, var


def backward_chain(layers, delta_mu: Tensor, delta_var: Tensor, add: tuple[Tensor, Tensor] | None = None,
                   first_params_only: bool = False, fold: _Fold | None = None):
    """Backward through ``layers`` in reverse; ``add`` is added to the returned deltas.

    With ``first_params_only`` the first layer forms only its parameter deltas (when it
    can) and None is returned. ``fold`` (with ``add``, the first layer a Conv2D): the
    layers in front, whose backward that Conv2D's input-delta GEMM runs where it can.
    """
    i = len(layers) - 1
    start = None  # conv2 output deltas of the ResBlock at i, formed by the block after it
    while i >= 0:
        layer = layers[i]
        prev = layers[i - 1] if i >= 1 else None
        if isinstance(layer, ResBlock):
            f = _fold_in_front(layers, i)
            delta_mu, delta_var = resblock_backward(layer, delta_mu, delta_var, start=start, fold=f)
            start = None
            if f is not None and f.out is not None:
                if isinstance(prev, ResBlock):
                    start = f.out
                    i -= 1
                else:
                    delta_mu, delta_var = f.out  # on to the conv in front of the ReLU
                    i -= 3
                continue
            i -= 1
            continue
        if (isinstance(layer, Conv2D) and i >= 3 and _fusable_backward(prev, layers[i - 2])
                and isinstance(layers[i - 3], Conv2D)):
            out = conv_bn_relu_backward(layer, prev, layers[i - 2], layers[i - 3], delta_mu, delta_var)
            if out is not None:
                delta_mu, delta_var = out
                i -= 3
                continue
        if _fusable_backward(layer, prev):
            conv = layers[i - 2] if i >= 2 and isinstance(layers[i - 2], Conv2D) else None
            delta_mu, delta_var = bn_relu_backward(layer, prev, delta_mu, delta_var, conv)
            i -= 2
            continue
        if _fusable_pool_relu_backward(layer, prev):
            delta_mu, delta_var = avgpool_relu_backward(layer, prev, delta_mu, delta_var)
            i -= 2
            continue
        if (isinstance(layer, Linear) and isinstance(prev, ReLU) and prev.J is not None
                and layer.ma_in is not None and prev.J.numel() == layer.ma_in.numel() and delta_mu.is_cuda):
            # the ReLU's Jacobian applied in the Linear input-delta product's epilogue
            delta_mu, delta_var = layer.backward_jacobian(delta_mu, delta_var, prev.J)
            i -= 2
            continue
        if i == 0:
            if first_params_only and hasattr(layer, "backward_param_deltas"):
                layer.backward_param_deltas(delta_mu, delta_var)
                return None
            if add is not None and isinstance(layer, Conv2D):
                if fold is not None:
                    out = conv_add_bn_relu_backward(layer, delta_mu, delta_var, add, fold.bn, fold.relu, fold.conv)
                    if out is not None:
                        fold.out = out[1]
                        return out[0]
                return layer._backward(delta_mu, delta_var, True, add=add)
        delta_mu, delta_var = layer.backward(delta_mu, delta_var)
        i -= 1
    if add is not None:
        _add_in_place(add[0], add[1], delta_mu, delta_var)
    return delta_mu, delta_var
