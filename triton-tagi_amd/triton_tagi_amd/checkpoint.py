"""Run directories, checkpoints and metrics logging (mirrors triton_tagi/checkpoint.py:30-214).

A checkpoint is ``torch.save({"epoch", "config", "net_state"})`` with ``net_state``
keyed by the layer's position in ``net.layers``: a dict of CPU tensors
{mw, Sw, mb, Sb, running_mean, running_var} (those the layer has) for a learnable
layer, or a list of such dicts for a layer made of learnable sub-layers (ResBlock's
``_learnable``; MultiheadAttentionV2's q/k/v projections). Files written by the
reference load here and the other way round, for the layer types both save.

Differences from the reference: attributes that are None (Embedding's and RMSNorm's
absent bias) are skipped instead of failing, attention projections are saved, and files
are read with ``torch.load(weights_only=True)``, which executes nothing from the file
(a checkpoint whose config holds objects other than plain containers, numbers and
strings is refused with the loader's message).
"""

from __future__ import annotations

import csv
import json
from datetime import datetime
from pathlib import Path
from typing import Any, Callable

import torch

from .base import LearnableLayer

_PARAM_ATTRS = ("mw", "Sw", "mb", "Sb")
_STAT_ATTRS = ("running_mean", "running_var")


class RunDir:
    """``{base}/{dataset}_{arch}_{optimizer}_{YYYYmmdd-HHMMSS}/`` with ``checkpoints/``,
    ``figures/``, ``config.json`` and ``metrics.csv`` (checkpoint.py:30-115)."""

    def __init__(self, dataset: str, arch: str, optimizer: str, base: str = "runs") -> None:
        stamp = datetime.now().strftime("%Y%m%d-%H%M%S")
        self.path = Path(base) / f"{dataset}_{arch}_{optimizer}_{stamp}"
        self.checkpoints = self.path / "checkpoints"
        self.figures = self.path / "figures"
        self.config_json = self.path / "config.json"
        self.metrics_csv = self.path / "metrics.csv"
        self.path.mkdir(parents=True, exist_ok=True)
        self.checkpoints.mkdir()
        self.figures.mkdir()

    def save_config(self, config: dict[str, Any]) -> None:
        with open(self.config_json, "w") as f:
            json.dump(config, f, indent=2)

    def save_checkpoint(self, net, epoch: int, config: dict[str, Any]) -> Path:
        path = self.checkpoints / f"epoch_{epoch:04d}.pt"
        torch.save({"epoch": epoch, "config": config, "net_state": _extract_net_state(net)}, path)
        return path

    def load_checkpoint(self, net, path: str | Path | None = None) -> int:
        """Restore ``net`` from ``path`` (default: the latest ``epoch_*.pt``); returns the epoch."""
        if path is None:
            found = sorted(self.checkpoints.glob("epoch_*.pt"))
            if not found:
                raise FileNotFoundError(f"No checkpoints found in {self.checkpoints}")
            path = found[-1]
        ck = _load(path, net.device)
        _restore_net_state(net, ck["net_state"])
        return ck["epoch"]

    def append_metrics(self, epoch: int, **kwargs: float) -> None:
        """One CSV row; the header comes from the first call's keys."""
        row = {"epoch": epoch, **kwargs}
        new = not self.metrics_csv.exists()
        with open(self.metrics_csv, "a", newline="") as f:
            w = csv.DictWriter(f, fieldnames=list(row))
            if new:
                w.writeheader()
            w.writerow({k: f"{v:.6g}" if isinstance(v, float) else v for k, v in row.items()})

    def __repr__(self) -> str:
        return f"RunDir({self.path})"


def load_model(path: str | Path, build: Callable[[dict[str, Any]], Any], device: str | torch.device = "cuda"):
    """(net, config, epoch): ``build(config)`` makes the topology, the saved tensors fill it
    (checkpoint.py:118-162)."""
    device = torch.device(device)
    ck = _load(path, device)
    config = ck["config"]
    net = build(config)
    if hasattr(net, "to"):
        net = net.to(device)
    _restore_net_state(net, ck["net_state"])
    return net, config, ck["epoch"]


def _load(path, device):
    return torch.load(path, map_location=device, weights_only=True)


def _parts(layer) -> list | None:
    """Learnable sub-layers of a composite layer, or None for a plain layer."""
    if hasattr(layer, "_learnable"):
        return list(layer._learnable)
    if all(hasattr(layer, a) for a in ("q_proj", "k_proj", "v_proj")):
        return [layer.q_proj, layer.k_proj, layer.v_proj]
    return None


def _layer_state(layer) -> dict[str, torch.Tensor]:
    out = {}
    for attr in _PARAM_ATTRS + _STAT_ATTRS:
        t = getattr(layer, attr, None)
        if isinstance(t, torch.Tensor):
            out[attr] = t.detach().cpu().clone()
    return out


def _extract_net_state(net) -> dict[int, Any]:
    state: dict[int, Any] = {}
    for i, layer in enumerate(net.layers):
        parts = _parts(layer)
        if parts is not None:
            subs = [_layer_state(p) for p in parts]
            if any(subs):
                state[i] = subs
        elif isinstance(layer, LearnableLayer):
            s = _layer_state(layer)
            if s:
                state[i] = s
    return state


def _restore_layer(layer, d: dict[str, torch.Tensor], device) -> None:
    for attr in _PARAM_ATTRS + _STAT_ATTRS:
        if attr not in d:
            continue
        t = getattr(layer, attr, None)
        if not isinstance(t, torch.Tensor):
            continue
        src = d[attr]
        if tuple(src.shape) != tuple(t.shape):
            raise ValueError(f"checkpoint: {type(layer).__name__}.{attr} has shape {tuple(src.shape)}, "
                             f"the network expects {tuple(t.shape)}")
        t.data.copy_(src.to(device=t.device, dtype=t.dtype))  # in place: tensor identity is kept


def _restore_net_state(net, state: dict[int, Any]) -> None:
    device = getattr(net, "device", None)
    for i, layer in enumerate(net.layers):
        if i not in state:
            continue
        s = state[i]
        if isinstance(s, list):
            parts = _parts(layer)
            if parts is None:
                raise ValueError(f"checkpoint: entry {i} holds sub-layers but {type(layer).__name__} has none")
            for sub, sub_state in zip(parts, s):
                _restore_layer(sub, sub_state, device)
        else:
            _restore_layer(layer, s, device)
