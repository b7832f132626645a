"""Parameter-delta GEMMs of large Conv2D and Linear layers on a second stream during a step's backward pass.

In the backward pass only the input deltas are on the critical path (each layer waits for
the next one's); a layer's parameter deltas are first read by the update at the end of the
step. Within ``overlap_param_deltas`` such a layer queues its parameter-delta GEMM on a
side stream (default priority) that first waits for everything queued so far on the
current stream, so it runs beside the input-delta GEMMs and BatchNorm passes that follow
and fills the CUs their tail rounds leave idle. Leaving the context makes the current
stream wait for the side stream. The tensors the side stream reads (the layer input and
the output deltas) are kept alive until then, so the caching allocator cannot hand their
memory to later work on the current stream while the side stream still reads it.
Results are the same as on one stream: every kernel computes the same values whichever
order the streams interleave in.
"""

from __future__ import annotations

import threading

import torch

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


class overlap_param_deltas:
    def __enter__(self):
        self._outer = active()
        _tls.ctx = self
        self._keep: list = []
        self._used: dict[int, tuple[torch.cuda.Stream, torch.cuda.Stream]] = {}
        return self

    def fork(self, device: torch.device, *keep) -> torch.cuda.Stream:
        """The side stream of ``device``, ordered after the work queued so far on the current
        stream; ``keep`` stays referenced until the join."""
        idx = device.index if device.index is not None else torch.cuda.current_device()
        side = _side.get(idx)
        if side is None:
            side = torch.cuda.Stream(device=idx)
            _side[idx] = side
        main = torch.cuda.current_stream(idx)
        side.wait_stream(main)
        self._used[idx] = (main, side)
        self._keep.extend(keep)
        return side

    def __exit__(self, exc_type, exc, tb):
        _tls.ctx = self._outer
        for main, side in self._used.values():
            main.wait_stream(side)
        self._keep.clear()
        return False
