"""The capped update applied by the kernels that form the parameter deltas.

The reference's step runs the whole backward pass, which stores every layer's deltas,
and then the capped update of every layer (network.py:142-150, parameters.py:58-96).
Within ``update_in_backward(cap_factor)`` a Linear layer's backward does both for its
own parameters in one kernel: the epilogue that forms each delta also applies the capped
update to that parameter in place, with the same arithmetic as the update kernel
(``capped`` in the kernel library), so the result is the same to the bit. The deltas are
still stored on the layer, as the reference's backward leaves them (linear.py:146-151).
What changes is the traffic: the parameters and their deltas cross HBM once instead of
being written, read back and written again (the Linear layer of 4096 x 11008 moves 540 MB
less per step). With ``keep_deltas=False`` the deltas are applied without being stored
(the layer's delta attributes are None afterwards), for callers that only want the
updated parameters: another 360 MB less for that layer.

A layer's own input deltas read its weight means, so that product is queued before the
update; no other layer reads them during the backward pass. A layer whose
parameter-delta product runs on the side stream (``overlap_param_deltas``) is left to
the update after the backward pass: there the product starts beside the input deltas,
and waiting for them to update in place costs more than the traffic it saves.

A layer updated this way is flagged (``_updated_in_backward``); its next ``update()``,
or that of the Sequential holding it, leaves it out once and clears the flag, so every
layer is updated exactly once per step.
"""

from __future__ import annotations

import threading

_tls = threading.local()


def active():
    """The innermost ``update_in_backward`` of this thread, or None."""
    return getattr(_tls, "ctx", None)


class update_in_backward:
    """Context: Linear backward passes inside it also apply the capped update."""

    def __init__(self, cap_factor: float, keep_deltas: bool = True):
        if not cap_factor > 0.0:
            raise ValueError(f"update_in_backward: cap_factor must be positive, got {cap_factor}")
        self.cap_factor = float(cap_factor)
        self.keep_deltas = bool(keep_deltas)

    def __enter__(self):
        self._outer = active()
        _tls.ctx = self
        return self

    def __exit__(self, *exc):
        _tls.ctx = self._outer
        return False
