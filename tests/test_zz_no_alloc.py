"""tagi_linear_fwd_noalloc against tagi_linear_fwd, through the C ABI.

The no-allocation entry point runs the plan tagi_linear_fwd runs with its full
workspace, with the split-K partials in the library's fixed per-GPU scratch array, so
its outputs must equal the workspace entry point's bit for bit. Two calls in a row, the
second smaller (the scratch keeps the first call's partials), both with shapes whose
plans split the reduction so the scratch is used; a shape needing more scratch than the
fixed size must be refused before anything is launched.
"""

from __future__ import annotations

import ctypes

import pytest
import torch

from conftest import assert_scaled_close
from oracle import tagi_oracle as O

pytestmark = pytest.mark.gpu

SCRATCH_BYTES = 128 << 20


def _inputs(M, K, N, seed):
    r = torch.Generator().manual_seed(seed)
    ma, Sa = torch.randn(M, K, generator=r), 0.01 + 0.09 * torch.rand(M, K, generator=r)
    mw, Sw = torch.randn(K, N, generator=r) / K**0.5, torch.rand(K, N, generator=r) / K
    mb, Sb = torch.randn(1, N, generator=r), 1e-3 * torch.rand(1, N, generator=r)
    return ma, Sa, mw, Sw, mb, Sb


def _call(name, dev, tensors, M, K, N, ws=None):
    from triton_tagi_amd import _lib

    mz = torch.full((M, N), float("nan"), device=dev)
    Sz = torch.full((M, N), float("nan"), device=dev)
    ptrs = [t.data_ptr() for t in tensors] + [mz.data_ptr(), Sz.data_ptr()]
    st = torch.cuda.current_stream(dev).cuda_stream
    if ws is None:
        _lib.call(name, *ptrs, M, K, N, st)
    else:
        _lib.call(name, *ptrs, M, K, N, ws.data_ptr(), ws.numel() * 4, st)
    return mz, Sz


def test_noalloc_linear_forward_equals_workspace_entry_point(dev):
    from triton_tagi_amd import _lib

    torch.cuda.synchronize()
    for M, K, N, seed in ((256, 16384, 4096, 1), (256, 784, 256, 2)):
        need = _lib.query("tagi_linear_fwd_ws_bytes", M, K, N)
        assert 0 < need <= SCRATCH_BYTES, f"({M},{K},{N}) should split into the scratch, needs {need}"
        host = _inputs(M, K, N, seed)
        t = [x.to(dev) for x in host]
        ws = torch.empty(need // 4, device=dev)
        ref_m, ref_S = _call("tagi_linear_fwd", dev, t, M, K, N, ws)
        got_m, got_S = _call("tagi_linear_fwd_noalloc", dev, t, M, K, N)
        torch.cuda.synchronize()
        assert torch.equal(got_m, ref_m) and torch.equal(got_S, ref_S), f"({M},{K},{N}) differs"
        rows = torch.arange(0, M, max(1, M // 64))
        cols = torch.arange(0, N, max(1, N // 64))
        a, S, mw, Sw, mb, Sb = (x.double() for x in host)
        rm, rS = O.linear_moments(a[rows], S[rows], mw[:, cols], Sw[:, cols], mb[:, cols], Sb[:, cols])
        assert_scaled_close(got_m[rows][:, cols], rm, a[rows].abs() @ mw[:, cols].abs() + mb[:, cols].abs(),
                            1e-4, 1e-6, "noalloc mz sample")
        assert_scaled_close(got_S[rows][:, cols], rS, None, 1e-4, 1e-6, "noalloc Sz sample")


def test_noalloc_refuses_shapes_beyond_the_scratch(dev):
    from triton_tagi_amd import _lib

    M, K, N = 768, 8192, 11008
    need = _lib.query("tagi_linear_fwd_ws_bytes", M, K, N)
    assert need > SCRATCH_BYTES
    lib = _lib.load()
    fake = 256  # never dereferenced: the call must fail on the host before any launch
    rc = lib.tagi_linear_fwd_noalloc(*([fake] * 8), M, K, N, torch.cuda.current_stream(dev).cuda_stream)
    assert rc == _lib.TAGI_ERR_ARG if hasattr(_lib, "TAGI_ERR_ARG") else rc == 1
    assert "scratch" in _lib.last_error()
