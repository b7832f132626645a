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
    assert lib.tagi_abi_version() == 1
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
