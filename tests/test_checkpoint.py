"""Checkpoint format and run directories (CPU only: no kernel runs).

The format is the reference's (checkpoint.py:63-214): ``{epoch, config, net_state}``,
``net_state[i]`` a dict of CPU tensors for learnable layer i or a list of such dicts for
a composite layer. Files are read with ``torch.load(weights_only=True)``.
"""

from __future__ import annotations

import csv
import datetime
import json
import pickle

import pytest
import torch

import triton_tagi_amd as tt
from triton_tagi_amd.checkpoint import _extract_net_state


def build(cfg=None):
    torch.manual_seed(0 if cfg is None else cfg.get("seed", 0))
    return tt.Sequential([
        tt.Embedding(16, 8, device="cpu"),
        tt.MultiheadAttentionV2(8, 2, 4, device="cpu"),
        tt.RMSNorm(8, device="cpu"),
        tt.LayerNorm(8, device="cpu"),
        tt.Linear(8, 6, device="cpu"),
        tt.ReLU(),
        tt.ResBlock(2, 4, stride=2, device="cpu"),
        tt.BatchNorm2D(4, device="cpu"),
        tt.Conv2D(4, 3, 3, padding=1, device="cpu"),
    ], device="cpu")


def leaves(net):
    out = []
    for layer in net.layers:
        if hasattr(layer, "_learnable"):
            out.extend(layer._learnable)
        elif hasattr(layer, "q_proj"):
            out.extend([layer.q_proj, layer.k_proj, layer.v_proj])
        else:
            out.append(layer)
    return out


ATTRS = ("mw", "Sw", "mb", "Sb", "running_mean", "running_var")


def test_round_trip_restores_every_tensor_in_place(tmp_path):
    src = build({"seed": 1})
    for layer in leaves(src):
        for a in ATTRS:
            t = getattr(layer, a, None)
            if isinstance(t, torch.Tensor):
                t.add_(torch.randn_like(t))  # move away from the prior
    run = tt.RunDir("synthetic", "mixed", "tagi", base=str(tmp_path))
    path = run.save_checkpoint(src, 7, {"seed": 1, "lr": 0.1})
    assert path.name == "epoch_0007.pt"
    dst = build({"seed": 2})
    before = {(i, a): getattr(l, a) for i, l in enumerate(leaves(dst)) for a in ATTRS
              if isinstance(getattr(l, a, None), torch.Tensor)}
    assert run.load_checkpoint(dst) == 7
    n = 0
    for i, (ls, ld) in enumerate(zip(leaves(src), leaves(dst))):
        for a in ATTRS:
            ts = getattr(ls, a, None)
            if isinstance(ts, torch.Tensor):
                td = getattr(ld, a)
                assert td is before[(i, a)], "restore must copy in place"
                assert torch.equal(td, ts), (type(ls).__name__, a)
                n += 1
    assert n >= 30
    net, cfg, ep = tt.load_model(path, build, device="cpu")
    assert ep == 7 and cfg == {"seed": 1, "lr": 0.1}
    assert torch.equal(leaves(net)[0].mw, leaves(src)[0].mw)


def test_state_layout_matches_reference_format():
    net = build()
    st = _extract_net_state(net)
    assert set(st) == {0, 1, 2, 3, 4, 6, 7, 8}  # ReLU (5) has nothing
    assert isinstance(st[1], list) and len(st[1]) == 3  # q, k, v projections
    assert isinstance(st[6], list) and len(st[6]) == 6  # conv, bn, conv, bn, proj conv, proj bn
    assert set(st[0]) == {"mw", "Sw"} and set(st[2]) == {"mw", "Sw"}  # no bias: skipped, not a crash
    assert set(st[7]) == {"mw", "Sw", "mb", "Sb", "running_mean", "running_var"}
    assert all(t.device.type == "cpu" for t in st[8].values())


def test_reference_written_file_loads(tmp_path):
    # a file laid out as the reference writes it, for the layer types it saves
    net = build()
    ref_state = {4: {"mw": torch.full((8, 6), 0.5), "Sw": torch.full((8, 6), 0.25), "mb": torch.ones(1, 6),
                     "Sb": torch.full((1, 6), 0.125)},
                 7: {"mw": torch.full((4,), 2.0), "Sw": torch.full((4,), 0.5), "mb": torch.zeros(4),
                     "Sb": torch.ones(4), "running_mean": torch.arange(4.0), "running_var": torch.ones(4)}}
    p = tmp_path / "epoch_0003.pt"
    torch.save({"epoch": 3, "config": {"arch": "x", "widths": [1, 2]}, "net_state": ref_state}, p)
    got, cfg, ep = tt.load_model(p, lambda c: net, device="cpu")
    assert ep == 3 and cfg["widths"] == [1, 2]
    assert torch.all(got.layers[4].mw == 0.5) and torch.equal(got.layers[7].running_mean, torch.arange(4.0))


def golden_net():
    """The topology of tests/golden/checkpoint_golden.pt (written by the reference's
    RunDir.save_checkpoint, tests/golden/make_pe_checkpoint_golden.py)."""
    torch.manual_seed(0)
    return tt.Sequential([tt.Conv2D(3, 4, 3, padding=1, device="cpu"), tt.ReLU(), tt.BatchNorm2D(4, device="cpu"),
                          tt.ResBlock(4, 8, 2, device="cpu"), tt.AvgPool2D(2), tt.Flatten(),
                          tt.Linear(8 * 2 * 2, 5, device="cpu")], device="cpu")


def test_file_written_by_the_reference_loads_and_resaves_identically(tmp_path):
    from pathlib import Path

    golden = Path(__file__).resolve().parent / "golden" / "checkpoint_golden.pt"
    ref = torch.load(golden, weights_only=True)  # executes nothing from the file
    net, cfg, ep = tt.load_model(golden, lambda c: golden_net(), device="cpu")
    assert ep == 12 and cfg == {"arch": "smallcnn", "batch": 4, "sigma_v": 0.05}
    # every tensor the reference saved is now in the engine's layer, at the same index
    ls = net.layers
    targets = {0: ls[0], 2: ls[2], 3: ls[3]._learnable, 6: ls[6]}
    n = 0
    for i, st in ref["net_state"].items():
        layers = targets[i] if isinstance(st, list) else [targets[i]]
        sts = st if isinstance(st, list) else [st]
        assert len(layers) == len(sts)
        for layer, d in zip(layers, sts):
            for a, t in d.items():
                assert torch.equal(getattr(layer, a), t), (i, type(layer).__name__, a)
                n += 1
    assert n == 4 + 6 + 3 * 4 + 3 * 6 + 4
    # and the engine writes the same layout back: keys, nesting, shapes, values
    run = tt.RunDir("synthetic", "smallcnn", "tagi", base=str(tmp_path))
    mine = torch.load(run.save_checkpoint(net, 12, cfg), weights_only=True)
    assert mine["epoch"] == ref["epoch"] and mine["config"] == ref["config"]
    assert set(mine["net_state"]) == set(ref["net_state"])
    for i, st in ref["net_state"].items():
        got = mine["net_state"][i]
        assert type(got) is type(st)
        for dg, dr in zip(got if isinstance(got, list) else [got], st if isinstance(st, list) else [st]):
            assert set(dg) == set(dr)
            assert all(torch.equal(dg[a], dr[a]) for a in dr)


def test_shape_mismatch_and_unsafe_files_are_refused(tmp_path):
    net = build()
    p = tmp_path / "bad.pt"
    torch.save({"epoch": 0, "config": {}, "net_state": {4: {"mw": torch.zeros(3, 3)}}}, p)
    with pytest.raises(ValueError, match="shape"):
        tt.load_model(p, lambda c: net, device="cpu")

    q = tmp_path / "custom.pt"
    torch.save({"epoch": 0, "config": {"when": datetime.date(2020, 1, 1)}, "net_state": {}}, q)
    with pytest.raises(pickle.UnpicklingError):
        tt.load_model(q, lambda c: net, device="cpu")


def test_run_dir_layout_and_metrics(tmp_path):
    run = tt.RunDir("cifar10", "resnet18", "tagi", base=str(tmp_path))
    assert run.path.parent == tmp_path and run.path.name.startswith("cifar10_resnet18_tagi_")
    assert run.checkpoints.is_dir() and run.figures.is_dir()
    run.save_config({"batch": 128})
    assert json.loads(run.config_json.read_text()) == {"batch": 128}
    run.append_metrics(1, loss=0.5, acc=0.123456789)
    run.append_metrics(2, loss=0.25, acc=0.5)
    rows = list(csv.DictReader(open(run.metrics_csv)))
    assert rows[0] == {"epoch": "1", "loss": "0.5", "acc": "0.123457"} and rows[1]["epoch"] == "2"
    with pytest.raises(FileNotFoundError):
        tt.RunDir("a", "b", "c", base=str(tmp_path / "other")).load_checkpoint(build())
