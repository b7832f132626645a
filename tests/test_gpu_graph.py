"""HIP-graph replay of the TAGI step against eager steps.

``Sequential.capture_step`` records one training step; each replay must give exactly
the eager step's results (same kernels, same order, deterministic reductions). Every
replay is checked, with eager work and synchronisations between replays.
"""

from __future__ import annotations

import pytest
import torch

pytestmark = pytest.mark.gpu


def _params(net):
    out = []
    for layer in net.layers:
        items = layer._update_items() if hasattr(layer, "_update_items") else None
        for m, S, _, _ in items or []:
            out += [m, S]
    for layer in net.layers:
        for name in ("running_mean", "running_var"):
            if hasattr(layer, name):
                out.append(getattr(layer, name))
    return out


@pytest.mark.parametrize("name,batch", [("mlp", 256), ("resnet18", 16), ("transformer", 4)])
def test_graph_replays_match_eager_steps(dev, name, batch):
    from triton_tagi_amd import workloads

    eager = workloads.build(name, device="cuda:0", batch=batch)
    graphed = workloads.build(name, device="cuda:0", batch=batch)
    for a, b in zip(_params(eager.net), _params(graphed.net)):
        assert torch.equal(a, b)
    g = graphed.net.capture_step(graphed.x, graphed.y, graphed.sigma_v)  # runs one eager step
    eager.net.step(eager.x, eager.y, eager.sigma_v)
    torch.cuda.synchronize()
    for r in range(3):
        mu, var = g.replay()
        emu, evar = eager.net.step(eager.x, eager.y, eager.sigma_v)
        torch.cuda.synchronize()
        assert torch.equal(mu, emu) and torch.equal(var, evar), f"replay {r}: predictions differ"
        for i, (a, b) in enumerate(zip(_params(eager.net), _params(graphed.net))):
            assert torch.equal(a, b), f"replay {r}: parameter tensor {i} differs"
        # eager work on the same stream between replays
        torch.cuda.synchronize()
    assert bool(torch.isfinite(mu).all())


@pytest.mark.parametrize("name,batch", [("mlp_hrc", 512), ("resnet18_hrc", 16)])
def test_graph_replays_match_eager_hrc_steps(dev, name, batch):
    from triton_tagi_amd import workloads

    eager = workloads.build(name, device="cuda:0", batch=batch)
    graphed = workloads.build(name, device="cuda:0", batch=batch)
    g = graphed.net.capture_step_hrc(graphed.x, graphed.y, graphed.hrc, graphed.sigma_v)
    eager.step()
    torch.cuda.synchronize()
    gen = torch.Generator().manual_seed(11)
    for r in range(3):
        mu, var = g.replay()
        emu, evar = eager.step()
        torch.cuda.synchronize()
        assert torch.equal(mu, emu) and torch.equal(var, evar), f"replay {r}: predictions differ"
        for i, (a, b) in enumerate(zip(_params(eager.net), _params(graphed.net))):
            assert torch.equal(a, b), f"replay {r}: parameter tensor {i} differs"
        # new labels copied in place are seen by the next replay and the next eager step
        new = torch.randint(0, 10, (batch,), generator=gen).to(dev)
        graphed.y.copy_(new)
        eager.y.copy_(new)
        torch.cuda.synchronize()


@pytest.mark.parametrize("name", ["resnet18", "transformer"])
def test_graph_replays_with_the_side_stream(dev, name):
    """Capture of the benchmarked steps (ResNet-18 batch 128, transformer block batch 64 x
    sequence 256), where the parameter-delta products run on the side stream: the capture
    must record the fork and the join, and every replay must equal an eager overlapped
    step bit for bit (network.py:119-152)."""
    from triton_tagi_amd import _overlap, workloads

    eager = workloads.build(name, device="cuda:0")
    graphed = workloads.build(name, device="cuda:0")
    assert eager.net.overlap_param_deltas and graphed.net.overlap_param_deltas
    forks = [0]
    orig = _overlap.overlap_param_deltas.fork

    def counting_fork(self, *a):
        forks[0] += 1
        return orig(self, *a)

    _overlap.overlap_param_deltas.fork = counting_fork
    try:
        g = graphed.net.capture_step(graphed.x, graphed.y, graphed.sigma_v)  # one eager step, then the capture
    finally:
        _overlap.overlap_param_deltas.fork = orig
    assert forks[0] >= 2, "the side stream was not used during the capture: the test would not cover it"
    eager.net.step(eager.x, eager.y, eager.sigma_v)
    torch.cuda.synchronize()
    for r in range(3):
        mu, var = g.replay()
        emu, evar = eager.net.step(eager.x, eager.y, eager.sigma_v)
        torch.cuda.synchronize()
        assert torch.equal(mu, emu) and torch.equal(var, evar), f"replay {r}: predictions differ"
        for i, (a, b) in enumerate(zip(_params(eager.net), _params(graphed.net))):
            assert torch.equal(a, b), f"replay {r}: parameter tensor {i} differs"
    assert bool(torch.isfinite(mu).all())
