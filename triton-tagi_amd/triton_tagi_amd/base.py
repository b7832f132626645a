"""Layer contracts of the TAGI step (mirrors triton_tagi/base.py:21-67).

``Layer``: forward(ma, Sa) -> (ma, Sa) and backward(delta_ma, delta_Sa) -> deltas.
``LearnableLayer``: adds update(cap_factor) applying deltas stored by backward, and
the num_parameters property. ``Sequential`` dispatches on these two classes.
"""

from __future__ import annotations

from abc import ABC, abstractmethod

from torch import Tensor


class Layer(ABC):
    """Base class for all TAGI layers."""

    @abstractmethod
    def forward(self, ma: Tensor, Sa: Tensor) -> tuple[Tensor, Tensor]:
        """Propagate Gaussian moments (means, variances) forward."""

    @abstractmethod
    def backward(self, delta_ma: Tensor, delta_Sa: Tensor) -> tuple[Tensor, Tensor]:
        """Propagate innovation deltas backward; return the deltas for the previous layer."""

    def sublayers(self) -> tuple:
        """Layers held inside this one (a residual block's branches, an attention layer's
        projections); containers walk them to place or visit every parameter tensor."""
        return ()


class LearnableLayer(Layer):
    """Base class for layers with parameters updated by the capped TAGI rule."""

    # True after a backward pass that applied the layer's capped update itself (within
    # update_in_backward); the next update() of the layer, or of the Sequential holding
    # it, leaves the layer out once and clears it.
    _updated_in_backward = False

    @abstractmethod
    def update(self, cap_factor: float) -> None:
        """Apply the parameter deltas stored by ``backward``."""

    @property
    @abstractmethod
    def num_parameters(self) -> int:
        """Total number of learnable scalars (means + variances)."""

    def _update_items(self):
        """(m, S, delta_m, delta_S) quadruples of the layer's parameter groups, in order.

        ``Sequential.step`` uses these to apply every layer's update in one launch; a
        layer that returns None is updated through its own ``update`` instead.
        """
        return None

    def _update_groups(self):
        """The contiguous (m, S, delta_m, delta_S) groups the update applies: those of
        ``_update_items`` unless the layer keeps its parameters in larger buffers (the
        attention layer's projections live side by side)."""
        return self._update_items()
