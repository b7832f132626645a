"""The five TAGI step workloads, with seeded synthetic data.

Architectures follow the reference's example networks (examples/mnist_mlp.py,
examples/cifar10_cnn.py, examples/cifar10_resnet18.py:271-296,
examples/reverse_predictor.py:74-86). Priors are drawn on the CPU from torch's global
generator seeded with ``seed`` (layer order, weights before bias), so a network built on
any device holds the same priors; inputs use a generator seeded ``seed + 1`` and targets
``seed + 2``.

    mlp          784-256-128-10, ReLU, Remax head, batch 256, x ~ U[0,1], sigma_v 0.05
    cnn          3 x (Conv 5x5 pad 2, ReLU, AvgPool 2), Linear 1024-256-10, Remax, batch 128
    resnet18     BasicBlock stages 64/128/256/512, BN, Add, AvgPool 4, Linear 512-10, Remax,
                 gain 0.1, batch 128, x ~ N(0,1) 3x32x32
    transformer  Embedding(64, 256) + PE + MHA-V2 (8 heads) + RMSNorm + Linear 256-64,
                 batch 64, sequence 256, target = one-hot of the reversed sequence
    mlp_hrc      784-128-11 with a hierarchical-softmax head (10 classes), batch 512,
                 trained with step_hrc (tests/validation/test_mnist_hrc_10epochs.py)
    resnet18_hrc resnet18 with the head Linear 512-11 and step_hrc
                 (examples/cifar10_resnet18_hrc.py), batch 128
and the Linear microbenchmark shapes (batch, in, out).
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from .hrc_softmax import HierarchicalSoftmax, class_to_obs

from .layers import (
    AvgPool2D,
    BatchNorm2D,
    Conv2D,
    Embedding,
    Flatten,
    Linear,
    MultiheadAttentionV2,
    PositionalEncoding,
    ReLU,
    Remax,
    ResBlock,
    RMSNorm,
)
from .network import Sequential

LINEAR_SHAPES = [(4096, 4096, 4096), (8192, 1024, 4096), (256, 4096, 11008)]


@dataclass
class Workload:
    name: str
    net: Sequential
    x: torch.Tensor
    y: torch.Tensor  # one-hot targets, or integer labels for an HRC head
    sigma_v: float
    batch: int
    hrc: HierarchicalSoftmax | None = None

    def step(self):
        """One training step of the workload (step_hrc for an HRC head)."""
        if self.hrc is not None:
            return self.net.step_hrc(self.x, self.y, self.hrc, self.sigma_v)
        return self.net.step(self.x, self.y, self.sigma_v)


def _onehot(labels: torch.Tensor, classes: int) -> torch.Tensor:
    return torch.nn.functional.one_hot(labels, classes).to(torch.float32)


def mlp_layers():
    return [Linear(784, 256, device="cpu"), ReLU(), Linear(256, 128, device="cpu"), ReLU(),
            Linear(128, 10, device="cpu"), Remax()]


def cnn_layers():
    kw = dict(device="cpu")
    return [
        Conv2D(3, 32, 5, padding=2, **kw), ReLU(), AvgPool2D(2),
        Conv2D(32, 32, 5, padding=2, **kw), ReLU(), AvgPool2D(2),
        Conv2D(32, 64, 5, padding=2, **kw), ReLU(), AvgPool2D(2),
        Flatten(),
        Linear(1024, 256, **kw), ReLU(),
        Linear(256, 10, **kw), Remax(),
    ]


def mlp_hrc_layers(hrc_len: int = 11):
    return [Linear(784, 128, device="cpu"), ReLU(), Linear(128, hrc_len, device="cpu")]


def resnet18_layers(gain: float = 0.1, width: int = 64, hrc_len: int | None = None):
    kw = dict(device="cpu", gain_w=gain, gain_b=gain)
    w = width
    return [
        Conv2D(3, w, 3, stride=1, padding=1, **kw), ReLU(), BatchNorm2D(w, **kw),
        ResBlock(w, w, 1, **kw), ResBlock(w, w, 1, **kw),
        ResBlock(w, 2 * w, 2, **kw), ResBlock(2 * w, 2 * w, 1, **kw),
        ResBlock(2 * w, 4 * w, 2, **kw), ResBlock(4 * w, 4 * w, 1, **kw),
        ResBlock(4 * w, 8 * w, 2, **kw), ResBlock(8 * w, 8 * w, 1, **kw),
        AvgPool2D(4), Flatten(),
        *([Linear(8 * w, 10, **kw), Remax()] if hrc_len is None else [Linear(8 * w, hrc_len, **kw)]),
    ]


def transformer_layers(vocab: int = 64, embed: int = 256, heads: int = 8, seq: int = 256):
    return [
        Embedding(vocab, embed, input_size=seq, scale=0.25, device="cpu"),
        PositionalEncoding(embed, device="cpu"),
        MultiheadAttentionV2(embed, heads, seq, bias=False, gain_weight=0.25, gain_bias=0.5, init_method="He",
                             device="cpu"),
        RMSNorm([embed], device="cpu"),
        Linear(embed, vocab, device="cpu"),
    ]


def build(name: str, device: str = "cuda", seed: int = 0, batch: int | None = None, **kw) -> Workload:
    """Network with seeded priors on ``device`` plus seeded inputs/targets of one batch."""
    torch.manual_seed(seed)
    gx = torch.Generator().manual_seed(seed + 1)
    gy = torch.Generator().manual_seed(seed + 2)
    hrc = None
    if name == "mlp_hrc":
        B = batch or 512
        hrc = class_to_obs(10)
        layers = mlp_hrc_layers(hrc.len)
        x = torch.rand(B, 784, generator=gx)
        y = torch.randint(0, 10, (B,), generator=gy)
        sv = 0.05
    elif name == "resnet18_hrc":
        B = batch or 128
        hrc = class_to_obs(10)
        layers = resnet18_layers(hrc_len=hrc.len, **kw)
        x = torch.randn(B, 3, 32, 32, generator=gx)
        y = torch.randint(0, 10, (B,), generator=gy)
        sv = 0.05
    elif name == "mlp":
        B = batch or 256
        layers = mlp_layers()
        x = torch.rand(B, 784, generator=gx)
        y = _onehot(torch.randint(0, 10, (B,), generator=gy), 10)
        sv = 0.05
    elif name == "cnn":
        B = batch or 128
        layers = cnn_layers()
        x = torch.randn(B, 3, 32, 32, generator=gx)
        y = _onehot(torch.randint(0, 10, (B,), generator=gy), 10)
        sv = 0.05
    elif name == "resnet18":
        B = batch or 128
        layers = resnet18_layers(**kw)
        x = torch.randn(B, 3, 32, 32, generator=gx)
        y = _onehot(torch.randint(0, 10, (B,), generator=gy), 10)
        sv = 0.05
    elif name == "transformer":
        B = batch or 64
        S = kw.pop("seq", 256)
        V = kw.pop("vocab", 64)
        layers = transformer_layers(vocab=V, seq=S, **kw)
        tok = torch.randint(0, V, (B, S), generator=gx)
        x = tok.to(torch.float32)
        y = _onehot(tok.flip(1), V)
        sv = 4.5
    else:
        raise ValueError(f"unknown workload {name!r}")
    net = Sequential(layers, device=device)
    return Workload(name, net, x.to(device), y.to(device), sv, B, hrc)


def linear_microbench(batch: int, fan_in: int, fan_out: int, device: str = "cuda", seed: int = 0):
    """Linear layer + moments for the microbenchmark: mu_a ~ N(0,1), S_a ~ U[0.01, 0.1],
    He means, S_w = 1/in, mu_b = 0, S_b = 1e-3; delta_mu ~ N(0, 1e-2) (std 0.1),
    delta_S ~ -U[0, 1e-2]."""
    torch.manual_seed(seed)
    layer = Linear(fan_in, fan_out, device="cpu")
    layer.mb.zero_()
    layer.Sb.fill_(1e-3)
    g = torch.Generator().manual_seed(seed + 1)
    ma = torch.randn(batch, fan_in, generator=g)
    Sa = 0.01 + 0.09 * torch.rand(batch, fan_in, generator=g)
    dmz = 0.1 * torch.randn(batch, fan_out, generator=g)
    dSz = -1e-2 * torch.rand(batch, fan_out, generator=g)
    for attr in ("mw", "Sw", "mb", "Sb"):
        setattr(layer, attr, getattr(layer, attr).to(device))
    layer.device = torch.device(device)
    return layer, ma.to(device), Sa.to(device), dmz.to(device), dSz.to(device)
