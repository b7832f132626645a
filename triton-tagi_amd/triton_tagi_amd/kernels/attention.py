"""Batched TAGI products of the attention layer (mirrors triton_tagi/kernels/attention.py).

    bmm_tagi:         mean = s a_mu @ b_mu,  var = s^2 [a_var @ (b_mu^2 + b_var) + a_mu^2 @ b_var]
    bmm_shared_right: mean = s a_mean @ b,   var = s^2 a_var @ b^2
    bmm_shared_left:  mean = s a @ b_mean,   var = s^2 a^2 @ b_var

Operands are strided views: transposed views and (B, H, ...) batch dims are read in
place, no copies. One fp32-MFMA launch produces mean and variance together.
"""

from __future__ import annotations

import torch

from .. import _lib


def _view_of(t: torch.Tensor, name: str) -> tuple[_lib.TagiView, int, tuple]:
    """tagi_view of a (..., I, J) tensor with at most two batch dims of any stride."""
    _lib.check(t, name, contiguous=False)
    if t.dim() < 2:
        raise ValueError(f"{name}: need at least 2 dims")
    batch = tuple(t.shape[:-2])
    si, sj = t.stride(-2), t.stride(-1)
    if len(batch) == 0:
        return _lib.view(1, 0, 0, si, sj), 1, batch
    if len(batch) == 1:
        return _lib.view(1, t.stride(0), 0, si, sj), batch[0], batch
    if len(batch) == 2:
        return _lib.view(batch[1], t.stride(0), t.stride(1), si, sj), batch[0] * batch[1], batch
    # more batch dims: they must flatten into one stride (the reference's packed layout)
    flat = t.reshape(-1, t.shape[-2], t.shape[-1])
    if flat.data_ptr() != t.data_ptr():
        raise ValueError(f"{name}: leading dims must be packed")
    return _lib.view(1, flat.stride(0), 0, si, sj), flat.shape[0], batch


def _out(batch, M, L, like):
    return torch.empty((*batch, M, L), device=like.device, dtype=torch.float32)


def bmm_tagi(mu_a, var_a, mu_b, var_b, scale=1.0, need_mean=True):
    """Mean and variance of the TAGI product of two Gaussian batched matrices."""
    va, n, batch = _view_of(mu_a, "mu_a")
    vb, nb, _ = _view_of(mu_b, "mu_b")
    if var_a.shape != mu_a.shape or var_a.stride() != mu_a.stride():
        raise ValueError("var_a must share mu_a's shape and strides")
    if var_b.shape != mu_b.shape or var_b.stride() != mu_b.stride():
        raise ValueError("var_b must share mu_b's shape and strides")
    M, K = mu_a.shape[-2], mu_a.shape[-1]
    Kb, L = mu_b.shape[-2], mu_b.shape[-1]
    if K != Kb:
        raise ValueError(f"Reduction dims disagree: a has {K}, b has {Kb}")
    if nb != n:
        raise ValueError("batch dims of a and b disagree")
    mean = _out(batch, M, L, mu_a) if need_mean else None
    var = _out(batch, M, L, mu_a)
    vo = _lib.view(1, M * L, 0, L, 1)
    s = float(scale)
    _lib.call("tagi_bmm_tagi", mu_a.data_ptr(), var_a.data_ptr(), mu_b.data_ptr(), var_b.data_ptr(),
              _lib.ptr(mean), var.data_ptr(), n, M, K, L, va, vb, vo, s, s * s, _lib.stream_of(mu_a))
    return mean, var


def bmm_tagi_var(mu_a, var_a, mu_b, var_b, scale_sq: float = 1.0):
    """var = scale_sq * sum_k (var_a (mu_b^2 + var_b) + mu_a^2 var_b) (attention.py:149-201)."""
    va, n, batch = _view_of(mu_a, "mu_a")
    vb, nb, _ = _view_of(mu_b, "mu_b")
    M, K = mu_a.shape[-2], mu_a.shape[-1]
    Kb, L = mu_b.shape[-2], mu_b.shape[-1]
    if K != Kb:
        raise ValueError(f"Reduction dims disagree: a has {K}, b has {Kb}")
    if var_a.stride() != mu_a.stride() or var_b.stride() != mu_b.stride():
        raise ValueError("variance tensors must share the mean tensors' strides")
    var = _out(batch, M, L, mu_a)
    vo = _lib.view(1, M * L, 0, L, 1)
    _lib.call("tagi_bmm_tagi", mu_a.data_ptr(), var_a.data_ptr(), mu_b.data_ptr(), var_b.data_ptr(), None,
              var.data_ptr(), n, M, K, L, va, vb, vo, 1.0, float(scale_sq), _lib.stream_of(mu_a))
    return var


def bmm_shared_right(a_mean, a_var, b, scale: float = 1.0, jacobian=None):
    """(s a_mean @ b, s^2 a_var @ b^2) (attention.py:286-336).

    With ``jacobian`` (a contiguous tensor shaped like the output) the results are
    multiplied by it and its square in the product's epilogue (the Remax Jacobian applied
    to the score deltas, multihead_attention.py:239-243).
    """
    va, n, batch = _view_of(a_mean, "a_mean")
    vb, nb, _ = _view_of(b, "b")
    if a_var.stride() != a_mean.stride() or a_var.shape != a_mean.shape:
        raise ValueError("a_var must share a_mean's shape and strides")
    M, K = a_mean.shape[-2], a_mean.shape[-1]
    Kb, L = b.shape[-2], b.shape[-1]
    if K != Kb:
        raise ValueError(f"Reduction dims disagree: a has {K}, b has {Kb}")
    mean, var = _out(batch, M, L, a_mean), _out(batch, M, L, a_mean)
    vo = _lib.view(1, M * L, 0, L, 1)
    s = float(scale)
    if jacobian is not None:
        J = _lib.check(jacobian, "jacobian")
        if tuple(J.shape) != tuple(mean.shape) or not J.is_contiguous():
            raise ValueError(f"jacobian must be a contiguous {tuple(mean.shape)} tensor, got {tuple(J.shape)}")
        _lib.call("tagi_bmm_shared_jacobian", a_mean.data_ptr(), a_var.data_ptr(), b.data_ptr(), J.data_ptr(),
                  mean.data_ptr(), var.data_ptr(), n, M, K, L, va, vb, vo, s, s * s, 0, _lib.stream_of(a_mean))
        return mean, var
    _lib.call("tagi_bmm_shared", a_mean.data_ptr(), a_var.data_ptr(), b.data_ptr(), mean.data_ptr(),
              var.data_ptr(), n, M, K, L, va, vb, vo, s, s * s, 0, _lib.stream_of(a_mean))
    return mean, var


def bmm_shared_left(a, b_mean, b_var, scale: float = 1.0):
    """(s a @ b_mean, s^2 a^2 @ b_var) (attention.py:339-374)."""
    va, n, batch = _view_of(a, "a")
    vb, nb, _ = _view_of(b_mean, "b_mean")
    if b_var.stride() != b_mean.stride() or b_var.shape != b_mean.shape:
        raise ValueError("b_var must share b_mean's shape and strides")
    M, K = a.shape[-2], a.shape[-1]
    Kb, L = b_mean.shape[-2], b_mean.shape[-1]
    if K != Kb:
        raise ValueError(f"Reduction dims disagree: a has {K}, b has {Kb}")
    mean, var = _out(batch, M, L, a), _out(batch, M, L, a)
    vo = _lib.view(1, M * L, 0, L, 1)
    s = float(scale)
    _lib.call("tagi_bmm_shared", b_mean.data_ptr(), b_var.data_ptr(), a.data_ptr(), mean.data_ptr(),
              var.data_ptr(), n, M, K, L, va, vb, vo, s, s * s, 1, _lib.stream_of(a))
    return mean, var
