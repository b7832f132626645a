"""Linear moment GEMMs (mirrors triton_tagi/kernels/common.py).

    forward:  mz = ma @ mw + mb,  Sz = ma^2 @ Sw + Sa @ (mw^2 + Sw) + Sb
    backward: dma = dmz @ mw^T,   dSa = dSz @ (mw^2)^T
    deltas:   gmw = ma^T @ dmz,   gSw = (ma^2)^T @ dSz

Each is one fp32-MFMA kernel launch (two accumulators) behind the C ABI; the
``triton_*`` names of the reference are kept as aliases.
"""

from __future__ import annotations

import torch

from .. import _lib


def _2d(t, name):
    _lib.check(t, name)
    if t.dim() != 2:
        raise ValueError(f"{name}: expected a 2-D tensor, got shape {tuple(t.shape)}")
    return t


def linear_forward(ma, Sa, mw, Sw, mb=None, Sb=None, need_mean=True):
    """Fused mean and variance of z = a W + b (linear.py:99-100). Sa None: a deterministic
    input (the network's), the same values as zeros with one product fewer."""
    _2d(ma, "ma"), _2d(mw, "mw"), _2d(Sw, "Sw")
    if Sa is not None:
        _2d(Sa, "Sa")
    M, K = ma.shape
    K2, N = mw.shape
    if K2 != K or (Sa is not None and Sa.shape != ma.shape) or Sw.shape != mw.shape:
        raise ValueError(f"linear_forward: shapes ma {tuple(ma.shape)} mw {tuple(mw.shape)} disagree")
    for t, n in ((mb, "mb"), (Sb, "Sb")):
        if t is not None:
            _lib.check(t, n)
            if t.numel() != N:
                raise ValueError(f"{n}: expected {N} elements, got {t.numel()}")
    mz = torch.empty(M, N, device=ma.device, dtype=torch.float32) if need_mean else None
    Sz = torch.empty(M, N, device=ma.device, dtype=torch.float32)
    ws = _lib.workspace(_lib.query("tagi_linear_fwd_ws_bytes", M, K, N), ma.device)
    wp, wb = _lib.ws_args(ws)
    _lib.call("tagi_linear_fwd", ma.data_ptr(), _lib.ptr(Sa), mw.data_ptr(), Sw.data_ptr(), _lib.ptr(mb),
              _lib.ptr(Sb), _lib.ptr(mz), Sz.data_ptr(), M, K, N, wp, wb, _lib.stream_of(ma))
    return mz, Sz


def linear_relu_forward(ma, Sa, mw, Sw, mb=None, Sb=None):
    """(mu_a, S_a, J) of ReLU(a W + b) in one launch: the Linear forward (linear.py:99-100)
    whose epilogue applies the ReLU moments (relu.py:94-122) in place of storing z; the same
    bits as linear_forward followed by bayesian_relu. Sa None as in linear_forward."""
    _2d(ma, "ma"), _2d(mw, "mw"), _2d(Sw, "Sw")
    if Sa is not None:
        _2d(Sa, "Sa")
    M, K = ma.shape
    K2, N = mw.shape
    if K2 != K or (Sa is not None and Sa.shape != ma.shape) or Sw.shape != mw.shape:
        raise ValueError(f"linear_relu_forward: shapes ma {tuple(ma.shape)} mw {tuple(mw.shape)} disagree")
    for t, n in ((mb, "mb"), (Sb, "Sb")):
        if t is not None:
            _lib.check(t, n)
            if t.numel() != N:
                raise ValueError(f"{n}: expected {N} elements, got {t.numel()}")
    am, aS, J = (torch.empty(M, N, device=ma.device, dtype=torch.float32) for _ in range(3))
    ws = _lib.workspace(_lib.query("tagi_linear_fwd_ws_bytes", M, K, N), ma.device)
    wp, wb = _lib.ws_args(ws)
    _lib.call("tagi_linear_fwd_relu", ma.data_ptr(), _lib.ptr(Sa), mw.data_ptr(), Sw.data_ptr(), _lib.ptr(mb),
              _lib.ptr(Sb), am.data_ptr(), aS.data_ptr(), J.data_ptr(), M, K, N, wp, wb, _lib.stream_of(ma))
    return am, aS, J


def fused_var_forward(ma, Sa, mw, Sw, Sb):
    """Sz = ma^2 @ Sw + Sa @ (mw^2 + Sw) + Sb (common.py:170-210)."""
    return linear_forward(ma, Sa, mw, Sw, None, Sb, need_mean=False)[1]


def fused_backward_delta(dmz, dSz, mw, add=None, jacobian=None):
    """(dmz @ mw^T, dSz @ (mw^2)^T) (common.py:287-327).

    With ``add = (am, aS)`` (contiguous (M, K) tensors) the products are added to them in
    place, in the GEMM epilogue, and ``add`` is returned. With ``jacobian`` (a contiguous
    (M, K) tensor, the Jacobian of the elementwise layer in front, such as a ReLU's J) the
    epilogue returns (dmz @ mw^T) * J and (dSz @ (mw^2)^T) * J^2 instead: the deltas at that
    layer's input (relu.py:152-169).
    """
    _2d(dmz, "dmz"), _2d(dSz, "dSz"), _2d(mw, "mw")
    M, N = dmz.shape
    K = mw.shape[0]
    if mw.shape[1] != N or dSz.shape != dmz.shape:
        raise ValueError(f"fused_backward_delta: dmz {tuple(dmz.shape)} vs mw {tuple(mw.shape)}")
    if add is not None and jacobian is not None:
        raise ValueError("fused_backward_delta: an addend and a Jacobian cannot both be applied")
    ws = _lib.workspace(_lib.query("tagi_linear_bwd_delta_ws_bytes", M, K, N), dmz.device)
    wp, wb = _lib.ws_args(ws)
    if add is not None:
        dma, dSa = (_lib.check(t, n) for t, n in zip(add, ("add_m", "add_S")))
        if tuple(dma.shape) != (M, K) or tuple(dSa.shape) != (M, K) or not (dma.is_contiguous() and dSa.is_contiguous()):
            raise ValueError(f"fused_backward_delta: addend {tuple(dma.shape)} is not a contiguous ({M}, {K}) tensor")
        _lib.call("tagi_linear_bwd_delta_add", dmz.data_ptr(), dSz.data_ptr(), mw.data_ptr(), dma.data_ptr(),
                  dSa.data_ptr(), dma.data_ptr(), dSa.data_ptr(), M, K, N, wp, wb, _lib.stream_of(dmz))
        return dma, dSa
    dma = torch.empty(M, K, device=dmz.device, dtype=torch.float32)
    dSa = torch.empty(M, K, device=dmz.device, dtype=torch.float32)
    if jacobian is not None:
        J = _lib.check(jacobian, "jacobian")
        if tuple(J.shape) != (M, K) or not J.is_contiguous():
            raise ValueError(f"fused_backward_delta: Jacobian {tuple(J.shape)} is not a contiguous ({M}, {K}) tensor")
        _lib.call("tagi_linear_bwd_delta_jacobian", dmz.data_ptr(), dSz.data_ptr(), mw.data_ptr(), J.data_ptr(),
                  dma.data_ptr(), dSa.data_ptr(), M, K, N, wp, wb, _lib.stream_of(dmz))
        return dma, dSa
    _lib.call("tagi_linear_bwd_delta", dmz.data_ptr(), dSz.data_ptr(), mw.data_ptr(), dma.data_ptr(),
              dSa.data_ptr(), M, K, N, wp, wb, _lib.stream_of(dmz))
    return dma, dSa


def _wgrad(a, dmz, dSz, Sw, Sb, bias):
    _2d(a, "a"), _2d(dmz, "dmz"), _2d(dSz, "dSz")
    M, K = a.shape
    M2, N = dmz.shape
    if M2 != M or dSz.shape != dmz.shape:
        raise ValueError(f"weight deltas: a {tuple(a.shape)} vs dmz {tuple(dmz.shape)}")
    dev = a.device
    dmw = torch.empty(K, N, device=dev, dtype=torch.float32)
    dSw = torch.empty(K, N, device=dev, dtype=torch.float32)
    dmb = torch.empty(1, N, device=dev, dtype=torch.float32) if bias else None
    dSb = torch.empty(1, N, device=dev, dtype=torch.float32) if bias else None
    ws = _lib.workspace(_lib.query("tagi_linear_wgrad_ws_bytes", M, K, N), dev)
    wp, wb = _lib.ws_args(ws)
    _lib.call("tagi_linear_wgrad", a.data_ptr(), dmz.data_ptr(), dSz.data_ptr(), _lib.ptr(Sw), _lib.ptr(Sb),
              dmw.data_ptr(), dSw.data_ptr(), _lib.ptr(dmb), _lib.ptr(dSb), M, K, N, wp, wb, _lib.stream_of(a))
    return dmw, dSw, dmb, dSb


def linear_param_deltas_update(ma_in, dmz, dSz, mw, Sw, mb, Sb, cap_factor, keep_deltas=True):
    """``linear_param_deltas`` followed by the capped update of mw, Sw (and mb, Sb when
    given) with ``cap_factor`` (parameters.py:58-96), applied in place by the kernel that
    forms the deltas; returns the deltas (four Nones with ``keep_deltas=False``: applied,
    not stored). mw must not be read by work still queued (the layer's input-delta product
    reads it: queue that first)."""
    for t, n in ((mw, "mw"), (Sw, "Sw")):
        _lib.check(t, n)
    if mb is not None:
        _lib.check(mb, "mb"), _lib.check(Sb, "Sb")
    _2d(ma_in, "a"), _2d(dmz, "dmz"), _2d(dSz, "dSz")
    M, K = ma_in.shape
    M2, N = dmz.shape
    if M2 != M or dSz.shape != dmz.shape or tuple(mw.shape) != (K, N) or tuple(Sw.shape) != (K, N):
        raise ValueError(f"weight deltas: a {tuple(ma_in.shape)} vs dmz {tuple(dmz.shape)}, mw {tuple(mw.shape)}")
    if mb is not None and (mb.numel() != N or Sb.numel() != N):
        raise ValueError(f"weight deltas: bias of {mb.numel()} for {N} outputs")
    bias = mb is not None and keep_deltas
    dev = ma_in.device
    dmw = torch.empty(K, N, device=dev, dtype=torch.float32) if keep_deltas else None
    dSw = torch.empty(K, N, device=dev, dtype=torch.float32) if keep_deltas else None
    dmb = torch.empty(1, N, device=dev, dtype=torch.float32) if bias else None
    dSb = torch.empty(1, N, device=dev, dtype=torch.float32) if bias else None
    ws = _lib.workspace(_lib.query("tagi_linear_wgrad_ws_bytes", M, K, N), dev)
    wp, wb = _lib.ws_args(ws)
    _lib.call("tagi_linear_wgrad_update", ma_in.data_ptr(), dmz.data_ptr(), dSz.data_ptr(), mw.data_ptr(),
              Sw.data_ptr(), _lib.ptr(mb), _lib.ptr(Sb), _lib.ptr(dmw), _lib.ptr(dSw), _lib.ptr(dmb),
              _lib.ptr(dSb), float(cap_factor), M, K, N, wp, wb, _lib.stream_of(ma_in))
    return dmw, dSw, dmb, dSb


def fused_weight_grad(a, dmz, dSz):
    """Raw (a^T @ dmz, (a^2)^T @ dSz) (common.py:410-451)."""
    dmw, dSw, _, _ = _wgrad(a, dmz, dSz, None, None, False)
    return dmw, dSw


def linear_param_deltas(ma_in, dmz, dSz, Sw, Sb=None):
    """Parameter deltas of a Linear layer (linear.py:138-151):
    (Sw*gmw, Sw^2*gSw, Sb*gmb, Sb^2*gSb); the bias pair is None when Sb is None."""
    _lib.check(Sw, "Sw")
    if Sb is not None:
        _lib.check(Sb, "Sb")
    return _wgrad(ma_in, dmz, dSz, Sw, Sb, Sb is not None)


triton_fused_var_forward = fused_var_forward
triton_fused_backward_delta = fused_backward_delta
triton_fused_weight_grad = fused_weight_grad
