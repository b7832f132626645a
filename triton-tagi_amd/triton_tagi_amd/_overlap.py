"""Parameter-delta GEMMs of large Conv2D and Linear layers on a second stream during a step's backward pass.

In the backward pass only the input deltas are on the critical path (each layer waits for
the next one's); a layer's parameter deltas are first read by the update at the end of the
step. Within ``overlap_param_deltas`` such a layer queues its parameter-delta GEMM on a
side stream (default priority) that first waits for everything queued so far on the
current stream, so it runs beside the input-delta GEMMs and BatchNorm passes that follow
and fills the CUs their tail rounds leave idle. Leaving the context makes the current
stream wait for the side stream. Both waits go through tagi_stream_wait, whose event
carries no system-scope fence (a torch event's fence holds the recording stream for
about 5 us each time). The tensors the side stream reads (the layer input and
the output deltas) are kept alive until then, so the caching allocator cannot hand their
memory to later work on the current stream while the side stream still reads it.
Running a ResBlock's projection branch on the side stream as well (beside the main
branch's first convolution, joined where the main branch consumes it) was measured slower
(ResNet-18 b128: 11,523 against 11,871 samples/s): its kernels compete with the main
branch's for the same CUs and delay the parameter-delta GEMMs queued behind them.
Results are the same as on one stream: every kernel computes the same values whichever
order the streams interleave in.
"""

from __future__ import annotations

import threading

import torch

from . import _lib

# Products smaller than these (multiply-adds of one moment product) stay on the step's
# stream. Measured on MI355X: the side stream gains 5% on ResNet-18 b128 (convs of 1-5 G
# multiply-adds) and on the transformer block (projections of 0.27-1.1 G) and loses 11%
# on the small CNN (convs of 0.3-0.8 G), where the two streams' kernels only split the
# CUs between them.
MIN_MACS_CONV = 1 << 30
MIN_MACS_LINEAR = 1 << 28

_tls = threading.local()
_side: dict[int, torch.cuda.Stream] = {}


def active():
    return getattr(_tls, "ctx", None)


def _index(device) -> int:
    device = torch.device(device)
    return device.index if device.index is not None else torch.cuda.current_device()


def side_stream(device) -> torch.cuda.Stream:
    """The side stream of ``device`` (created once, default priority)."""
    idx = _index(device)
    side = _side.get(idx)
    if side is None:
        side = torch.cuda.Stream(device=idx)
        _side[idx] = side
    return side


def fork(device) -> torch.cuda.Stream:
    """The side stream, ordered after the work queued so far on the current stream (when
    the current stream is the side stream already, nothing is added)."""
    idx = _index(device)
    side = side_stream(idx)
    cur = torch.cuda.current_stream(idx)
    if cur != side:
        _lib.stream_wait(side, cur)
    return side


class overlap_param_deltas:
    def __enter__(self):
        self._outer = active()
        _tls.ctx = self
        self._keep: list = []
        self._main: dict[int, torch.cuda.Stream] = {}
        return self

    def fork(self, device: torch.device, *keep) -> torch.cuda.Stream:
        """``fork(device)``; ``keep`` stays referenced until the join at exit, which makes
        the stream current at the first fork wait for the side stream."""
        idx = _index(device)
        cur = torch.cuda.current_stream(idx)
        side = fork(idx)
        if cur != side:
            self._main.setdefault(idx, cur)
        self._keep.extend(keep)
        return side

    def __exit__(self, exc_type, exc, tb):
        _tls.ctx = self._outer
        for idx, main in self._main.items():
            _lib.stream_wait(main, side_stream(idx))
        self._keep.clear()
        return False
