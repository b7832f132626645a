"""Capped Bayesian parameter update (mirrors triton_tagi/update/parameters.py:30-128).

    bar  = sqrt(max(S, 1e-10)) / cap_factor          (pre-update S, both caps)
    m   += sign(dm) * min(|dm|, bar)
    S'   = S + sign(dS) * min(|dS|, bar);  S = 1e-5 if S' <= 0 else S'

The arithmetic runs in the HIP kernel behind ``tagi_capped_update``.
"""

from __future__ import annotations

import ctypes

import torch

from .. import _lib


def get_cap_factor(batch_size: int) -> float:
    """0.1 for a single sample, 2.0 below 256, 3.0 from 256 on (parameters.py:30-50)."""
    if batch_size == 1:
        return 0.1
    if batch_size < 256:
        return 2.0
    return 3.0


def update_parameters(m, S, delta_m, delta_S, cap_factor) -> None:
    """In-place capped update of (m, S) by (delta_m, delta_S) (parameters.py:104-128)."""
    for t, n in ((m, "m"), (S, "S"), (delta_m, "delta_m"), (delta_S, "delta_S")):
        _lib.check(t, n)
    n = m.numel()
    if S.numel() != n or delta_m.numel() != n or delta_S.numel() != n:
        raise ValueError("update_parameters: m, S, delta_m, delta_S must have the same number of elements")
    _lib.call("tagi_capped_update", m.data_ptr(), S.data_ptr(), delta_m.data_ptr(), delta_S.data_ptr(),
              float(cap_factor), n, _lib.stream_of(m))


def update_parameters_multi(items, cap_factor) -> None:
    """Apply ``update_parameters`` to many (m, S, delta_m, delta_S) groups in one launch."""
    items = [it for it in items if it[0].numel() > 0]
    if not items:
        return
    for m, S, dm, dS in items:
        for t, n in ((m, "m"), (S, "S"), (dm, "delta_m"), (dS, "delta_S")):
            _lib.check(t, n)
        if not (S.numel() == dm.numel() == dS.numel() == m.numel()):
            raise ValueError("update_parameters_multi: size mismatch within a group")
    k = len(items)
    arr = lambda vals, ty: (ty * k)(*vals)  # noqa: E731
    pm = arr([it[0].data_ptr() for it in items], ctypes.c_void_p)
    pS = arr([it[1].data_ptr() for it in items], ctypes.c_void_p)
    pdm = arr([it[2].data_ptr() for it in items], ctypes.c_void_p)
    pdS = arr([it[3].data_ptr() for it in items], ctypes.c_void_p)
    pn = arr([it[0].numel() for it in items], ctypes.c_int64)
    _lib.call("tagi_capped_update_multi", ctypes.addressof(pm), ctypes.addressof(pS), ctypes.addressof(pdm),
              ctypes.addressof(pdS), ctypes.addressof(pn), k, float(cap_factor), _lib.stream_of(items[0][0]))
