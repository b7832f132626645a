"""The C-ABI library loads and exports every entry point declared in include/tagi_hip.h.

CPU-only: loads the shared object and resolves symbols; no kernel is launched.
"""

from __future__ import annotations

import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
HEADER = ROOT / "include" / "tagi_hip.h"


def declared_functions():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    names = re.findall(r"^\s*(?:const\s+)?(?:int|int64_t|char\s*\*|const\s+char\s*\*)\s*\**\s*(tagi_\w+)\s*\(",
                       text, flags=re.M)
    return sorted(set(names))


def test_header_declares_entry_points():
    names = declared_functions()
    assert "tagi_linear_fwd" in names and "tagi_conv2d_fwd" in names and "tagi_bmm_tagi" in names
    assert len(names) >= 30


def test_library_exports_every_declared_symbol():
    from triton_tagi_amd import _lib

    lib = _lib.load()
    missing = [n for n in declared_functions() if not hasattr(lib, n)]
    assert not missing, f"symbols declared but not exported: {missing}"


def test_binding_table_matches_header():
    from triton_tagi_amd import _lib

    assert sorted(_lib.EXPORTED) == declared_functions()


def test_abi_version_and_error_channel():
    from triton_tagi_amd import _lib

    lib = _lib.load()
    assert lib.tagi_abi_version() == 5
    # argument errors are reported without touching the GPU
    rc = lib.tagi_linear_fwd(None, None, None, None, None, None, None, None, 1, 1, 1, None, 0, None)
    assert rc == 1
    assert "null pointer" in _lib.last_error()
    rc = lib.tagi_capped_update(None, None, None, None, 2.0, -1, None)
    assert rc == 1 and "n < 0" in _lib.last_error()


def test_product_path_refuses_cpu_tensors():
    import torch

    from triton_tagi_amd.update.parameters import update_parameters

    t = torch.zeros(4)
    with pytest.raises(ValueError, match="GPU only"):
        update_parameters(t, t.clone(), t.clone(), t.clone(), 2.0)


def test_new_entry_points_validate_arguments_without_a_gpu():
    from triton_tagi_amd import _lib

    lib = _lib.load()
    # MaxPool2D: padding above half the window
    rc = lib.tagi_maxpool2d_fwd(None, None, None, None, None, 1, 1, 4, 4, 2, 2, 2, 0, None)
    assert rc == 1 and "pad" in _lib.last_error()
    # HRC class probabilities: alpha must be positive
    rc = lib.tagi_hrc_class_probs(None, None, None, None, 0.0, None, None, 1, 11, 4, 10, None)
    assert rc == 1 and "alpha" in _lib.last_error()
    # LayerNorm backward: workspace too small
    rc = lib.tagi_layernorm_bwd(*([1] * 14), 64, 256, 1e-5, 1, 0, None)
    assert rc == 1 and "workspace" in _lib.last_error()
    assert lib.tagi_layernorm_bwd_ws_bytes(64, 256) == 2 * 4 * 256 * 4
    # empty inputs are no-ops
    assert lib.tagi_innovation_heteros(None, None, None, None, None, 0, None) == 0
    assert lib.tagi_even_softplus_fwd(None, None, None, None, None, 0, None) == 0
    assert lib.tagi_innovation_indexed(None, None, None, None, None, None, None, 0, 11, 4, None) == 0
    rc = lib.tagi_hrc_innovation(None, None, None, None, None, 0.1, None, None, 3, 11, 4, 10, None)
    assert rc == 1 and "null pointer" in _lib.last_error()


def test_heads_refuse_cpu_tensors():
    import torch

    import triton_tagi_amd as tt
    from triton_tagi_amd.update.observation import compute_innovation_with_indices

    h = tt.class_to_obs(10)
    t = torch.zeros(2, h.len)
    with pytest.raises(ValueError, match="GPU only"):
        tt.obs_to_class_probs(t, t, h)
    with pytest.raises(ValueError, match="GPU only"):
        compute_innovation_with_indices(t, t, torch.zeros(2, 4), torch.zeros(2, 4), torch.ones(2, 4, dtype=torch.int32))
    with pytest.raises(ValueError, match="GPU only"):
        tt.MaxPool2D(2).forward(torch.zeros(1, 1, 4, 4), torch.zeros(1, 1, 4, 4))


def test_size_queries_and_their_cache():
    """Workspace sizes come from the plan choice, on the host. The parameter deltas of a
    76 x 32 output reduced over 131072 pixels (a 5 x 5 conv on a 3-channel input, with its
    bias row, at batch 128 on 32 x 32) split 512 ways, each split writing both moments; and
    the Python side's cache answers integer-only queries exactly as the library does."""
    from triton_tagi_amd import _lib

    lib = _lib.load()
    assert lib.tagi_linear_wgrad_ws_bytes(131072, 75, 32) == 512 * 2 * 76 * 32 * 4
    for args in ((256, 784, 256), (300, 70, 45), (131072, 75, 32)):
        for name in ("tagi_linear_fwd_ws_bytes", "tagi_linear_bwd_delta_ws_bytes", "tagi_linear_wgrad_ws_bytes"):
            direct = getattr(lib, name)(*args)
            assert _lib.query(name, *args) == direct
            assert (name, *args) in _lib._queries
            assert _lib.query(name, *args) == direct
