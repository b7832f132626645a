"""Parameter-delta GEMMs of Conv2D layers on a second stream during a step's backward pass.

In the backward pass only the input deltas are on the critical path (each layer waits for
the next one's); a layer's parameter deltas are first read by the update at the end of the
step. Within ``overlap_param_deltas`` a Conv2D layer queues its parameter-delta GEMM on a
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
