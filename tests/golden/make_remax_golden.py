"""Write golden input/output vectors of the reference Remax kernel.

Remax (triton_tagi/layers/remax.py:33-159) has no numeric test in the reference suite,
so its values are pinned by running the reference implementation itself: this script
imports ``triton_remax`` from the reference checkout and executes its Triton kernel on
the CPU through Triton's interpreter (TRITON_INTERPRET=1), on seeded inputs, and stores
inputs and outputs as a small .npz fixture. It runs only where the reference source is
present; the committed fixture is what the tests read.

    TRITON_INTERPRET=1 python tests/golden/make_remax_golden.py [/root/reference]
"""

from __future__ import annotations

import os
import sys
from pathlib import Path

import numpy as np

os.environ.setdefault("TRITON_INTERPRET", "1")
REF = Path(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
OUT = Path(__file__).resolve().parent / "remax_golden.npz"


def main():
    import torch

    sys.path.insert(0, str(REF))
    from triton_tagi.layers.remax import triton_remax  # reference implementation

    cases = {}
    g = torch.Generator().manual_seed(2024)
    specs = [("b16_k10", 16, 10, 1.0, 1.0), ("b8_k64", 8, 64, 2.0, 0.5), ("b4_k256", 4, 256, 1.0, 0.05),
             ("b6_k3_wide", 6, 3, 3.0, 4.0), ("b5_k10_tight", 5, 10, 0.5, 1e-3)]
    for name, B, K, mscale, vscale in specs:
        mu = (mscale * torch.randn(B, K, generator=g)).float()
        var = (vscale * (0.05 + torch.rand(B, K, generator=g))).float()
        ma, Sa, J = triton_remax(mu.clone(), var.clone())
        cases[f"{name}_mu_z"] = mu.numpy()
        cases[f"{name}_var_z"] = var.numpy()
        cases[f"{name}_mu_a"] = ma.numpy()
        cases[f"{name}_var_a"] = Sa.numpy()
        cases[f"{name}_J"] = J.numpy()
    np.savez_compressed(OUT, **cases)
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes, {len(specs)} cases)")


if __name__ == "__main__":
    main()
