"""Shared test setup: import paths, the ``gpu`` marker and comparison helpers."""

from __future__ import annotations

import sys
from pathlib import Path

import pytest
import torch

ROOT = Path(__file__).resolve().parent.parent
for p in (ROOT, ROOT / "triton-tagi_amd"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built libtagi_hip.so")


def assert_scaled_close(got, ref, scale=None, rtol=1e-4, atol=1e-6, what=""):
    """|got - ref| <= atol + rtol * scale elementwise.

    ``scale`` defaults to |ref|. For a sum of products with cancellation (GEMM means)
    pass the sum of the absolute terms, the quantity fp32 rounding error is relative to.
    """
    got = got.detach().to("cpu", torch.float64)
    ref = ref.detach().to("cpu", torch.float64)
    assert got.shape == ref.shape, f"{what}: shape {tuple(got.shape)} vs {tuple(ref.shape)}"
    sc = ref.abs() if scale is None else scale.detach().to("cpu", torch.float64).abs()
    err = (got - ref).abs()
    bound = atol + rtol * sc
    bad = err > bound
    if bad.any():
        i = int(torch.argmax((err - bound).reshape(-1)))
        raise AssertionError(
            f"{what}: {int(bad.sum())}/{bad.numel()} elements out of tolerance (rtol={rtol}, atol={atol}); "
            f"worst at flat {i}: got {got.reshape(-1)[i].item():.9g} ref {ref.reshape(-1)[i].item():.9g} "
            f"scale {sc.reshape(-1)[i].item():.3g}"
        )


@pytest.fixture(scope="session")
def dev():
    if not torch.cuda.is_available():
        pytest.fail("GPU test selected but no GPU is visible (run with -m 'not gpu' on a CPU host)")
    return torch.device("cuda:0")
