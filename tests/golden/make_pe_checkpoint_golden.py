"""Write golden fixtures of the reference's sinusoidal table and checkpoint format.

Two formats on the path have no numeric test in the reference suite, so they are pinned
by files the reference itself writes: this script imports the reference checkout (pure
torch code, run on the CPU) and stores

* pe_golden.npz: the reference's PositionalEncoding cache (layers/positional_encoding.py:
  45-52, computed in float32 as the reference does) for the transformer block's table
  (embed_dim 256, max_seq_len 2048: every 5th of the first 256 positions and the last
  position) and for a small table (max_seq_len 7, embed_dim 6) in full;
* checkpoint_golden.pt: a checkpoint written by the reference's RunDir.save_checkpoint
  (checkpoint.py:63-77,169-195) for a small network with every layer type both
  implementations save (Conv2D, BatchNorm2D, ResBlock with a projection, Linear), with
  parameters moved off their priors and running statistics set, so that every tensor is
  distinct.

It runs only where the reference source is present; the committed fixtures are what the
tests read (the checkpoint with torch.load(weights_only=True)).

    python tests/golden/make_pe_checkpoint_golden.py [/root/reference]
"""

from __future__ import annotations

import shutil
import sys
import tempfile
from pathlib import Path

import numpy as np

REF = Path(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
OUT = Path(__file__).resolve().parent


def main():
    import torch

    sys.path.insert(0, str(REF))
    from triton_tagi.checkpoint import RunDir  # reference implementation
    from triton_tagi.layers.avgpool2d import AvgPool2D
    from triton_tagi.layers.batchnorm2d import BatchNorm2D
    from triton_tagi.layers.conv2d import Conv2D
    from triton_tagi.layers.flatten import Flatten
    from triton_tagi.layers.linear import Linear
    from triton_tagi.layers.positional_encoding import PositionalEncoding
    from triton_tagi.layers.relu import ReLU
    from triton_tagi.layers.resblock import ResBlock
    from triton_tagi.network import Sequential

    big = PositionalEncoding(256, 2048, device="cpu").pe_cache
    rows = np.array(list(range(0, 256, 5)) + [2047])
    small = PositionalEncoding(6, 7, device="cpu").pe_cache
    np.savez_compressed(OUT / "pe_golden.npz", e256_rows=rows, e256=big[rows].numpy(), e6_s7=small.numpy())

    torch.manual_seed(3)
    layers = [Conv2D(3, 4, 3, padding=1, device="cpu"), ReLU(), BatchNorm2D(4, device="cpu"),
              ResBlock(4, 8, 2, device="cpu"), AvgPool2D(2), Flatten(), Linear(8 * 2 * 2, 5, device="cpu")]
    net = Sequential(layers, device="cpu")
    g = torch.Generator().manual_seed(4)
    subs = [layers[0], layers[2], *layers[3]._learnable, layers[6]]
    for layer in subs:
        for a in ("mw", "Sw", "mb", "Sb", "running_mean", "running_var"):
            t = getattr(layer, a, None)
            if isinstance(t, torch.Tensor):
                step = 0.1 * torch.rand(t.shape, generator=g)
                t.copy_(t + step if a in ("Sw", "Sb", "running_var") else t + torch.randn(t.shape, generator=g))
    tmp = Path(tempfile.mkdtemp())
    try:
        run = RunDir("synthetic", "smallcnn", "tagi", base=str(tmp))
        path = run.save_checkpoint(net, 12, {"arch": "smallcnn", "batch": 4, "sigma_v": 0.05})
        shutil.copy(path, OUT / "checkpoint_golden.pt")
    finally:
        shutil.rmtree(tmp)
    for f in ("pe_golden.npz", "checkpoint_golden.pt"):
        print(f"wrote {OUT / f} ({(OUT / f).stat().st_size} bytes)")


if __name__ == "__main__":
    main()
