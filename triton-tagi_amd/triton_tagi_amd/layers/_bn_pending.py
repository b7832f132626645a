"""BatchNorm2D parameter deltas left pending over a backward pass.

Within ``defer_bn_parameter_deltas`` the fused BatchNorm2D -> ReLU backward passes
leave their per-channel partial sums pending, and leaving the context forms the
parameter deltas of all of them in one launch (``Sequential.step`` wraps its backward
pass in it). The same partial sums can hold the bias deltas of the Conv2D in front of
the ReLU; the context records which convolutions those are, so that their
parameter-delta GEMM runs without its bias row. That record belongs to the context
alone: when the context is left, normally or by an exception, nothing of it remains on
the layers, and a later step starts with every bias row in place.
"""

from __future__ import annotations

import threading

import torch
from torch import Tensor

from .. import _lib

_scope = threading.local()


def active():
    """The innermost ``defer_bn_parameter_deltas`` of this thread, or None."""
    return getattr(_scope, "ctx", None)


def bias_deltas_formed(conv) -> bool:
    """True (once) if a pending BatchNorm pass of the active context forms ``conv``'s bias
    deltas; the caller then leaves them out of its parameter-delta product."""
    ctx = active()
    return ctx is not None and ctx._take_bias(conv)


class defer_bn_parameter_deltas:
    """The layers' ``delta_*`` tensors are complete once the context has exited."""

    def __enter__(self):
        self.items = []
        self._keep = []
        self._bias_convs: set[int] = set()
        self._outer = active()
        _scope.ctx = self
        return self

    def add(self, bn, ws: Tensor, N: int, C: int, HW: int, conv=None, nblk: int = 0) -> None:
        """``conv``: the Conv2D in front of the ReLU, whose bias sums ``ws`` also holds;
        ``nblk``: partial sums per channel and quantity (0: the BatchNorm pass's own count)."""
        self._keep.append(ws)  # the partial sums must outlive the launch below
        cb = (None, None, None) if conv is None else (conv.Sb.data_ptr(), conv.delta_mb.data_ptr(),
                                                      conv.delta_Sb.data_ptr())
        self.items.append(_lib.BnPending(ws.data_ptr(), bn.Sw.data_ptr(), bn.Sb.data_ptr(), bn.delta_mw.data_ptr(),
                                         bn.delta_Sw.data_ptr(), bn.delta_mb.data_ptr(), bn.delta_Sb.data_ptr(),
                                         N, C, HW, *cb, nblk))
        if conv is not None:
            self._bias_convs.add(id(conv))

    def _take_bias(self, conv) -> bool:
        key = id(conv)
        if key in self._bias_convs:
            self._bias_convs.discard(key)
            return True
        return False

    def __exit__(self, exc_type, exc, tb):
        _scope.ctx = self._outer
        self._bias_convs.clear()
        if exc_type is None and self.items:
            # on the stream current at exit (every pending layer's partial sums are ordered
            # before it: side-stream work has been joined by then)
            arr = (_lib.BnPending * len(self.items))(*self.items)
            _lib.call("tagi_bn_bwd_finalize_multi", arr, len(self.items),
                      torch.cuda.current_stream(self._keep[0].device).cuda_stream)
        return False
