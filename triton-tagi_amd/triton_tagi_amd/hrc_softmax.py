"""Hierarchical softmax (HRC) output head (mirrors triton_tagi/hrc_softmax.py:1-231).

A class r is the leaf reached by the L = ceil(log2(n_classes)) bits of r (MSB first) in
a binary tree whose inner nodes are the outputs of the network. Bit c of class r is
observed at the tree node that the first c bits lead to, as +1 (bit 0, left) or -1
(bit 1, right). Nodes are numbered 1.. level by level; level d holds the distinct
d-bit prefixes, ceil(n_classes / 2^(L-d)) of them, so the tree has ``len`` nodes (11
for 10 classes) and the output layer is that wide.

Training uses the sparse innovation on the L nodes of each sample's class path
(``Sequential.step_hrc``); inference multiplies the node probabilities
Phi(mu / sqrt(1/alpha^2 + S)) along each class's path. Both run as HIP kernels; the
tree tables are built once on the host and kept on each device that uses them.
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field

import torch
from torch import Tensor

from . import _lib


@dataclass
class HierarchicalSoftmax:
    """Binary-tree encoding of the classes.

    obs:   (n_classes, n_obs) float32, +1 / -1 per bit.
    idx:   (n_classes, n_obs) int32, 1-indexed tree node of each bit.
    n_obs: bits per class, ceil(log2(n_classes)).
    len:   number of tree nodes (the output layer's width).
    """

    obs: Tensor
    idx: Tensor
    n_obs: int
    len: int
    _on_device: dict = field(default_factory=dict, repr=False, compare=False)

    def tables(self, device: torch.device) -> tuple[Tensor, Tensor]:
        """(obs, idx) on ``device``, copied once per device and then reused."""
        key = str(torch.device(device))
        got = self._on_device.get(key)
        if got is None or got[0] is not self.obs or got[1] is not self.idx:
            got = (self.obs, self.idx,
                   self.obs.to(device=device, dtype=torch.float32).contiguous(),
                   self.idx.to(device=device, dtype=torch.int32).contiguous())
            self._on_device[key] = got
        return got[2], got[3]


def _levels(n_classes: int, L: int) -> list[int]:
    """Number of tree nodes at depth d = 0..L (depth L: the leaves, one per class)."""
    width = [0] * (L + 1)
    width[L] = n_classes
    for d in range(L - 1, -1, -1):
        width[d] = -(-width[d + 1] // 2)
    return width


def class_to_obs(n_classes: int) -> HierarchicalSoftmax:
    """Tree tables for ``n_classes`` classes (hrc_softmax.py:73-128, cuTAGI's class_to_obs)."""
    if n_classes < 2:
        raise ValueError("class_to_obs: need at least 2 classes")
    L = math.ceil(math.log2(n_classes))
    width = _levels(n_classes, L)
    first = [1] * L  # number of the first node at each depth
    for d in range(1, L):
        first[d] = first[d - 1] + width[d - 1]
    obs = torch.empty(n_classes, L, dtype=torch.float32)
    idx = torch.empty(n_classes, L, dtype=torch.int32)
    for r in range(n_classes):
        for c in range(L):
            bit = (r >> (L - 1 - c)) & 1
            prefix = r >> (L - c)  # the c leading bits
            obs[r, c] = -1.0 if bit else 1.0
            idx[r, c] = first[c] + prefix
    return HierarchicalSoftmax(obs=obs, idx=idx, n_obs=L, len=int(idx.max()))


def labels_to_hrc(labels: Tensor, hrc: HierarchicalSoftmax) -> tuple[Tensor, Tensor]:
    """(y_obs, y_idx) of integer labels: rows of the class tables (hrc_softmax.py:131-150)."""
    obs, idx = hrc.tables(labels.device) if labels.is_cuda else (hrc.obs, hrc.idx)
    lab = labels.long()
    return obs[lab], idx[lab]


def _class_probs(ma: Tensor, Sa: Tensor, hrc: HierarchicalSoftmax, alpha: float, want_labels: bool):
    ma = _lib.check(_lib.dense(ma), "ma")
    Sa = _lib.check(_lib.like(Sa, ma), "Sa")
    if ma.dim() != 2 or ma.shape != Sa.shape:
        raise ValueError(f"HRC class probabilities: expected (B, len) moments, got {tuple(ma.shape)}")
    if ma.shape[1] < hrc.len:
        raise ValueError(f"HRC class probabilities: output width {ma.shape[1]} < tree size {hrc.len}")
    obs, idx = hrc.tables(ma.device)
    B, n_classes = ma.shape[0], obs.shape[0]
    probs = torch.empty(B, n_classes, device=ma.device, dtype=torch.float32)
    pred = torch.empty(B, device=ma.device, dtype=torch.int64) if want_labels else None
    _lib.call("tagi_hrc_class_probs", ma.data_ptr(), Sa.data_ptr(), obs.data_ptr(), idx.data_ptr(), float(alpha),
              probs.data_ptr(), _lib.ptr(pred), B, ma.shape[1], hrc.n_obs, n_classes, _lib.stream_of(ma))
    return probs, pred


def obs_to_class_probs(ma: Tensor, Sa: Tensor, hrc: HierarchicalSoftmax, alpha: float = 3.0) -> Tensor:
    """(B, n_classes) unnormalised class probabilities (hrc_softmax.py:164-208)."""
    return _class_probs(ma, Sa, hrc, alpha, False)[0]


def get_predicted_labels(ma: Tensor, Sa: Tensor, hrc: HierarchicalSoftmax, alpha: float = 3.0) -> Tensor:
    """(B,) int64 index of the most probable class (hrc_softmax.py:211-231)."""
    return _class_probs(ma, Sa, hrc, alpha, True)[1]
