"""Sequential container and the TAGI step (mirrors triton_tagi/network.py:40-267).

``step(x, y, sigma_v)``: forward moments -> output innovation -> reversed backward
(deltas stored on the layers) -> capped update of every learnable layer with the cap
factor of the batch size. The updates of all layers that expose their parameter groups
go out as one multi-tensor launch; the arithmetic is the per-layer rule. Consecutive
ReLU -> BatchNorm2D pairs run as fused passes (same results as the layers one by one).
"""

from __future__ import annotations

import contextlib

import torch
from torch import Tensor

from . import _overlap
from .base import Layer, LearnableLayer
from .layers.conv2d import Conv2D
from .layers.embedding import Embedding
from .layers.linear import Linear
from .layers.fused import backward_chain, defer_bn_parameter_deltas, forward_chain
from .layers.multihead_attention import MultiheadAttentionV2
from .update.observation import compute_innovation, hrc_innovation
from .update.in_backward import update_in_backward
from .update.parameters import get_cap_factor, update_parameters_multi


# Per-layer state that lives on the network's device: parameters, BatchNorm running
# statistics, the positional-encoding table. Anything else a layer holds is formed on
# the device of the tensors it is given.
_PLACED_STATE = ("mw", "Sw", "mb", "Sb", "running_mean", "running_var", "pe_cache")


def _all_layers(layers):
    """Every layer of the list, each followed by the layers nested inside it."""
    for layer in layers:
        yield layer
        nested = getattr(layer, "sublayers", None)
        if nested is not None:
            yield from _all_layers(nested())


class Sequential:
    overlap_param_deltas = True  # Conv2D parameter-delta GEMMs on a side stream within step()

    def __init__(self, layers: list, device: str = "cuda") -> None:
        """Holds ``layers`` in order and places every state tensor they (and the layers
        nested in them) hold on ``device``; layers that record a device are told it."""
        self.device = torch.device(device)
        self.layers = layers
        for layer in _all_layers(layers):
            if hasattr(layer, "device"):
                layer.device = self.device
            if isinstance(layer, Layer) and layer.sublayers():
                continue  # a container's parameters are its nested layers' (ResBlock only aliases them)
            for name in _PLACED_STATE:
                t = getattr(layer, name, None)
                if isinstance(t, torch.Tensor):
                    setattr(layer, name, t.to(self.device))

    def forward(self, x: Tensor) -> tuple[Tensor, Tensor]:
        """Layer-by-layer moment propagation from a deterministic input (S_a = 0)."""
        for layer in self.layers:
            if not isinstance(layer, Layer):
                raise TypeError(f"Unknown layer type: {type(layer)}")
        first = self.layers[0] if self.layers else None
        if x.dim() == 4 and isinstance(first, Conv2D):
            # the conv path keeps activations channels-last
            x = x.contiguous(memory_format=torch.channels_last)
        if isinstance(first, (Conv2D, Linear, Embedding)):
            # the input's variance is zero: a Conv2D or Linear first layer then forms the
            # variance of its output from the weight variances alone (the same values),
            # and the Embedding reads token ids
            Sa = None
        else:
            Sa = torch.zeros_like(x)
        return forward_chain(self.layers, x, Sa)

    def backward(self, delta_mu: Tensor, delta_var: Tensor) -> tuple[Tensor, Tensor]:
        return backward_chain(self.layers, delta_mu, delta_var)

    def update(self, cap_factor: float) -> None:
        """Capped update of every learnable layer (one launch for all exposed groups)."""
        items = []
        for layer in self.layers:
            if not isinstance(layer, LearnableLayer):
                continue
            if layer._updated_in_backward:  # the backward pass applied it (update_in_backward)
                layer._updated_in_backward = False
                continue
            got = layer._update_groups()
            if got is None:
                if items:
                    update_parameters_multi(items, cap_factor)
                    items = []
                layer.update(cap_factor)
            else:
                items.extend(got)
        if items:
            update_parameters_multi(items, cap_factor)

    def step(self, x_batch: Tensor, y_batch: Tensor, sigma_v: float) -> tuple[Tensor, Tensor]:
        """forward -> innovation -> backward -> capped update (network.py:119-152).

        The deltas the first layer would pass back to the network input reach no one, so
        a first layer that can skip them (Linear, Conv2D) only forms its parameter deltas.
        """
        batch_size = x_batch.shape[0]
        y_pred_mu, y_pred_var = self.forward(x_batch)
        delta_mu, delta_var = compute_innovation(y_batch, y_pred_mu, y_pred_var, sigma_v)
        cap = get_cap_factor(batch_size)
        with self._backward_scope(cap):
            backward_chain(self.layers, delta_mu, delta_var, first_params_only=True)
        self.update(cap)
        return y_pred_mu, y_pred_var

    def _backward_scope(self, cap_factor: float):
        """One launch forms every BatchNorm2D's parameter deltas at the end of the backward
        pass; with ``overlap_param_deltas`` the Conv2D parameter-delta GEMMs run on a side
        stream beside the input-delta chain (joined before the update); Linear layers apply
        their capped update in the kernel that forms their parameter deltas
        (``update_in_backward``), and the update after the backward pass does the rest."""
        stack = contextlib.ExitStack()
        stack.enter_context(defer_bn_parameter_deltas())
        if self.overlap_param_deltas:  # exits first: the side stream is joined before the BN finalize
            stack.enter_context(_overlap.overlap_param_deltas())
        stack.enter_context(update_in_backward(cap_factor))
        return stack

    def step_hrc(self, x_batch: Tensor, labels: Tensor, hrc, sigma_v: float) -> tuple[Tensor, Tensor]:
        """forward -> sparse HRC innovation -> backward -> capped update (network.py:157-224).

        The output layer is ``hrc.len`` wide; only the ``hrc.n_obs`` tree nodes on each
        label's path receive innovation. Sequence outputs (B, S, len) take B*S labels.
        """
        batch_size = x_batch.shape[0]
        y_pred_mu, y_pred_var = self.forward(x_batch)
        shape = y_pred_mu.shape
        width = shape[-1]
        delta_mu, delta_var = hrc_innovation(y_pred_mu.reshape(-1, width), y_pred_var.reshape(-1, width), labels,
                                             hrc, sigma_v)
        cap = get_cap_factor(batch_size)
        with self._backward_scope(cap):
            backward_chain(self.layers, delta_mu.reshape(shape), delta_var.reshape(shape), first_params_only=True)
        self.update(cap)
        return y_pred_mu, y_pred_var

    def capture_step(self, x_batch: Tensor, y_batch: Tensor, sigma_v: float) -> "StepGraph":
        """Record one ``step`` into a HIP graph for replay without host launch overhead.

        Runs one eager ``step`` first (so that first-call behaviour, such as BatchNorm2D's
        gamma re-initialisation, is not recorded), then records the next step. Each
        ``replay()`` of the returned graph is one more training step on the tensors that
        were passed here: copy new data into ``x_batch`` / ``y_batch`` in place before a
        replay. Replays give the same results as eager steps (the kernels and their order
        are the same, and every reduction is deterministic).
        """
        if not x_batch.is_cuda:
            raise ValueError("capture_step: the batch must be on a GPU")
        return self._capture(lambda: self.step(x_batch, y_batch, sigma_v), x_batch.device)

    def capture_step_hrc(self, x_batch: Tensor, labels: Tensor, hrc, sigma_v: float) -> "StepGraph":
        """``capture_step`` for ``step_hrc``: replays read ``x_batch`` and ``labels`` in place
        (both must be on the GPU; copy the next batch and labels into them before a replay)."""
        if not x_batch.is_cuda or not labels.is_cuda or labels.device != x_batch.device:
            raise ValueError("capture_step_hrc: the batch and the labels must be on the same GPU")
        return self._capture(lambda: self.step_hrc(x_batch, labels, hrc, sigma_v), x_batch.device)

    def _capture(self, step, device) -> "StepGraph":
        step()
        torch.cuda.synchronize(device)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            mu, var = step()
        return StepGraph(graph, mu, var)

    def train(self) -> None:
        for layer in self.layers:
            if hasattr(layer, "training"):
                layer.train()

    def eval(self) -> None:
        for layer in self.layers:
            if hasattr(layer, "training"):
                layer.eval()

    def __repr__(self):
        lines = ["Sequential("]
        for i, layer in enumerate(self.layers):
            lines.append(f"  ({i}): {layer}")
        lines.append(")")
        return "\n".join(lines)

    def num_parameters(self) -> int:
        return sum(layer.num_parameters for layer in self.layers if isinstance(layer, LearnableLayer))

    def get_attention_scores(self) -> dict[int, tuple[Tensor, Tensor]]:
        out: dict[int, tuple[Tensor, Tensor]] = {}
        for i, layer in enumerate(self.layers):
            if isinstance(layer, MultiheadAttentionV2):
                out[i] = layer.get_attention_scores()
        if not out:
            raise RuntimeError("No attention layers in this Sequential.")
        return out


class StepGraph:
    """A recorded training step (``Sequential.capture_step``): ``replay()`` runs it and
    returns the predicted moments (tensors reused by every replay)."""

    def __init__(self, graph, mu: Tensor, var: Tensor) -> None:
        self.graph = graph
        self.mu = mu
        self.var = var

    def replay(self) -> tuple[Tensor, Tensor]:
        self.graph.replay()
        return self.mu, self.var
