"""One full TAGI step per workload, HIP engine vs the float64 CPU oracle, layer by layer.

For each workload the engine and the oracle start from identical priors and inputs and
run forward -> innovation -> backward -> capped update. Compared after the step:
  * every top-level layer's forward output (mu, S) and backward delta (delta_mu, delta_S);
  * every learnable parameter (mean and variance) after the update;
  * the argmax of the predicted means (must be identical).
Tolerance |gpu - oracle| <= 1e-6 + 1e-4 * scale. Variances are compared elementwise
(scale = |oracle|). Means and mean-deltas are sums with cancellation, so their scale is
|oracle| plus the tensor's mean absolute value (a norm-wise bound; fp32 rounding is
relative to the magnitude of the terms, not to a near-zero result).

Workload sizes: the MLP, CNN and transformer block run at their full benchmark shapes;
ResNet-18 runs at batch 16 here (the oracle takes minutes at batch 128 in float64) and
the full batch-128 step is covered by test_resnet18_full_batch_properties.
"""

from __future__ import annotations

import pytest
import torch

from conftest import assert_scaled_close
from oracle import tagi_oracle as O

pytestmark = pytest.mark.gpu

RTOL, ATOL = 1e-4, 1e-6


def run_traced(net, x, y, sv):
    from triton_tagi_amd.update.observation import compute_innovation
    from triton_tagi_amd.update.parameters import get_cap_factor

    ma, Sa = x, torch.zeros_like(x)
    fwd = []
    for layer in net.layers:
        ma, Sa = layer.forward(ma, Sa)
        fwd.append((ma.clone(), Sa.clone()))
    mu, var = ma.clone(), Sa.clone()
    dm, dS = compute_innovation(y, ma, Sa, sv)
    bwd = []
    for layer in reversed(net.layers):
        dm, dS = layer.backward(dm, dS)
        bwd.append((dm.clone(), dS.clone()))
    net.update(get_cap_factor(x.shape[0]))
    torch.cuda.synchronize()
    return mu, var, fwd, bwd


def gpu_params(net):
    out = []
    for layer in net.layers:
        items = layer._update_items() if hasattr(layer, "_update_items") else None
        for m, S, _, _ in items or []:
            out.append((m, S))
    return out


def oracle_params(onet):
    out = []
    for layer in onet.layers:
        for obj, m, S, _, _ in layer.param_groups():
            out.append((getattr(obj, m), getattr(obj, S)))
    return out


def mean_scale(ref):
    return ref.abs() + ref.abs().mean()


def check_step(w, names):
    """Compare everything, then report every mismatching tensor at once."""
    failures = []

    def chk(*a):
        try:
            assert_scaled_close(*a)
        except AssertionError as e:
            failures.append(str(e))

    _check_step(w, names, chk)
    assert not failures, "\n".join(failures)


def _check_step(w, names, assert_scaled_close):
    onet = O.mirror_net(w.net)
    mu, var, fwd, bwd = run_traced(w.net, w.x, w.y, w.sigma_v)
    rmu, rvar = onet.step(w.x.cpu().double(), w.y.cpu().double(), w.sigma_v, record=True)
    for i, ((gm, gS), (rm, rS)) in enumerate(zip(fwd, onet.trace)):
        tag = f"{w.name} fwd layer {i} {names[i]}"
        assert_scaled_close(gm, rm, mean_scale(rm), RTOL, ATOL, tag + " mu")
        assert_scaled_close(gS, rS, None, RTOL, ATOL, tag + " S")
    for i, ((gm, gS), (rm, rS)) in enumerate(zip(bwd, onet.bwd_trace)):
        tag = f"{w.name} bwd layer {len(names) - 1 - i} {names[len(names) - 1 - i]}"
        assert_scaled_close(gm, rm, mean_scale(rm), RTOL, ATOL, tag + " delta_mu")
        assert_scaled_close(gS, rS, mean_scale(rS), RTOL, ATOL, tag + " delta_S")
    gp, rp = gpu_params(w.net), oracle_params(onet)
    assert len(gp) == len(rp)
    for j, ((gm, gS), (rm, rS)) in enumerate(zip(gp, rp)):
        assert_scaled_close(gm, rm, mean_scale(rm), RTOL, ATOL, f"{w.name} param group {j} mean")
        assert_scaled_close(gS, rS, None, RTOL, ATOL, f"{w.name} param group {j} variance")
    pred, rpred = mu.reshape(-1, mu.shape[-1]).argmax(-1).cpu(), rmu.reshape(-1, rmu.shape[-1]).argmax(-1)
    assert torch.equal(pred, rpred), f"{w.name}: argmax differs on {(pred != rpred).sum().item()} rows"


@pytest.mark.parametrize("name,batch", [("mlp", None), ("cnn", None), ("resnet18", 16), ("transformer", None),
                                        ("mlp", 1), ("mlp", 257), ("cnn", 3), ("transformer", 1)])
def test_step_matches_oracle(dev, name, batch):
    """Full-size workloads, plus edge batches: 1 (cap factor 0.1, one-row GEMMs), 257 (the
    first batch with cap factor 3.0, ragged tiles), 3 (ragged conv tiles)."""
    from triton_tagi_amd import workloads

    w = workloads.build(name, device="cuda:0", batch=batch)
    names = [type(layer).__name__ for layer in w.net.layers]
    check_step(w, names)


def test_two_steps_bn_running_stats(dev):
    """Second step exercises the BatchNorm EMA branch and the updated parameters."""
    from triton_tagi_amd import workloads

    w = workloads.build("resnet18", device="cuda:0", batch=8)
    onet = O.mirror_net(w.net)
    for _ in range(2):
        w.net.step(w.x, w.y, w.sigma_v)
        onet.step(w.x.cpu().double(), w.y.cpu().double(), w.sigma_v)
    torch.cuda.synchronize()
    bn_g, bn_o = w.net.layers[2], onet.layers[2]
    assert_scaled_close(bn_g.running_mean, bn_o.running_mean, mean_scale(bn_o.running_mean), RTOL, ATOL, "running mean")
    assert_scaled_close(bn_g.running_var, bn_o.running_var, None, RTOL, ATOL, "running var")
    for j, ((gm, gS), (rm, rS)) in enumerate(zip(gpu_params(w.net), oracle_params(onet))):
        assert_scaled_close(gm, rm, mean_scale(rm), RTOL, ATOL, f"param group {j} mean after 2 steps")
        assert_scaled_close(gS, rS, None, RTOL, ATOL, f"param group {j} variance after 2 steps")


def test_resnet18_full_batch_properties(dev):
    """Batch-128 ResNet-18 step: finite moments, Remax means sum to one, positive
    variances, and bit-identical results when the same step is repeated from the same state."""
    from triton_tagi_amd import workloads

    outs = []
    for _ in range(2):
        w = workloads.build("resnet18", device="cuda:0")
        mu, var = w.net.step(w.x, w.y, w.sigma_v)
        torch.cuda.synchronize()
        outs.append((mu.cpu(), var.cpu(), w.net.layers[-2].mw.cpu(), w.net.layers[0].Sw.cpu()))
    mu, var = outs[0][0], outs[0][1]
    assert torch.isfinite(mu).all() and torch.isfinite(var).all()
    assert (var > 0).all()
    assert torch.allclose(mu.double().sum(-1), torch.ones(mu.shape[0], dtype=torch.float64), atol=1e-5)
    for a, b in zip(outs[0], outs[1]):
        assert torch.equal(a, b), "step is not deterministic"


@pytest.mark.parametrize("batch,fan_in,fan_out", [(4096, 4096, 4096), (8192, 1024, 4096), (256, 4096, 11008)])
def test_linear_microbench_shapes(dev, batch, fan_in, fan_out):
    """Full-size Linear microbenchmark shapes: a sampled block of rows/cols against the
    float64 oracle, plus the capped update of the sampled weights."""
    from triton_tagi_amd import workloads
    from triton_tagi_amd.update.parameters import get_cap_factor

    layer, ma, Sa, dmz, dSz = workloads.linear_microbench(batch, fan_in, fan_out)
    mw0, Sw0 = layer.mw.cpu().double(), layer.Sw.cpu().double()
    mz, Sz = layer.forward(ma, Sa)
    dma, dSa = layer.backward(dmz, dSz)
    torch.cuda.synchronize()
    r = torch.Generator().manual_seed(0)
    rows = torch.randint(0, batch, (64,), generator=r)
    cols = torch.randint(0, fan_out, (64,), generator=r)
    kin = torch.randint(0, fan_in, (64,), generator=r)
    a64, S64 = ma.cpu().double()[rows], Sa.cpu().double()[rows]
    rm, rS = O.linear_moments(a64, S64, mw0[:, cols], Sw0[:, cols], layer.mb.cpu().double()[:, cols],
                              layer.Sb.cpu().double()[:, cols])
    assert_scaled_close(mz[rows][:, cols], rm, a64.abs() @ mw0[:, cols].abs(), RTOL, ATOL, "mz sample")
    assert_scaled_close(Sz[rows][:, cols], rS, None, RTOL, ATOL, "Sz sample")
    dm64, dS64 = dmz.cpu().double()[rows], dSz.cpu().double()[rows]
    qm, qS = O.linear_backward_delta(dm64, dS64, mw0[kin])
    assert_scaled_close(dma[rows][:, kin], qm, dm64.abs() @ mw0[kin].abs().T, RTOL, ATOL, "dma sample")
    assert_scaled_close(dSa[rows][:, kin], qS, None, RTOL, ATOL, "dSa sample")
    A, D, DS = ma.cpu().double()[:, kin], dmz.cpu().double()[:, cols], dSz.cpu().double()[:, cols]
    Sws = Sw0[kin][:, cols]
    assert_scaled_close(layer.delta_mw[kin][:, cols], Sws * (A.T @ D), Sws * (A.abs().T @ D.abs()), RTOL, ATOL,
                        "delta_mw sample")
    assert_scaled_close(layer.delta_Sw[kin][:, cols], Sws * Sws * ((A * A).T @ DS), None, RTOL, ATOL,
                        "delta_Sw sample")
    dmw_s, dSw_s = layer.delta_mw[kin][:, cols].cpu().double(), layer.delta_Sw[kin][:, cols].cpu().double()
    layer.update(get_cap_factor(batch))
    torch.cuda.synchronize()
    um, uS = O.capped_update(mw0[kin][:, cols], Sws, dmw_s, dSw_s, get_cap_factor(batch))
    assert_scaled_close(layer.mw[kin][:, cols], um, None, RTOL, ATOL, "updated mw sample")
    assert_scaled_close(layer.Sw[kin][:, cols], uS, None, RTOL, ATOL, "updated Sw sample")


@pytest.mark.parametrize("batch,fan_in,fan_out", [(256, 4096, 11008), (4096, 4096, 4096), (300, 70, 45)])
def test_linear_update_in_backward_equals_backward_then_update(dev, batch, fan_in, fan_out):
    """The microbenchmark step as bench.py times it (the capped update applied by the
    parameter-delta kernel, ``update_in_backward``, without storing the deltas) and the
    same with the deltas stored, against backward followed by ``update`` from the same
    state: the same input deltas, parameter deltas (where stored) and updated parameters,
    bit for bit, and the layer's update() afterwards changes nothing. The shapes take the
    update in the GEMM epilogue (vector and scalar loaders) and in the split-K reduction."""
    from triton_tagi_amd import workloads
    from triton_tagi_amd.update.in_backward import update_in_backward
    from triton_tagi_amd.update.parameters import get_cap_factor

    cap = get_cap_factor(batch)
    res = []
    for fused in (False, True, "applied"):
        layer, ma, Sa, dmz, dSz = workloads.linear_microbench(batch, fan_in, fan_out)
        layer.forward(ma, Sa)
        if fused:
            with update_in_backward(cap, keep_deltas=fused is True):
                dma, dSa = layer.backward(dmz, dSz)
            assert layer._updated_in_backward
            before = [t.clone() for t in (layer.mw, layer.Sw, layer.mb, layer.Sb)]
            layer.update(cap)
            assert not layer._updated_in_backward
            torch.cuda.synchronize()
            assert all(torch.equal(x, y) for x, y in zip(before, (layer.mw, layer.Sw, layer.mb, layer.Sb)))
        else:
            dma, dSa = layer.backward(dmz, dSz)
            layer.update(cap)
        torch.cuda.synchronize()
        res.append([dma, dSa, layer.delta_mw, layer.delta_Sw, layer.delta_mb, layer.delta_Sb, layer.mw, layer.Sw,
                    layer.mb, layer.Sb])
    names = ("dma", "dSa", "delta_mw", "delta_Sw", "delta_mb", "delta_Sb", "mw", "Sw", "mb", "Sb")
    for n, x, y, z in zip(names, *res):
        assert torch.equal(x, y), f"{n} differs between the fused and the separate update"
        if n.startswith("delta"):
            assert z is None, f"{n} stored although the deltas were only applied"
        else:
            assert torch.equal(x, z), f"{n} differs between the applied-only and the separate update"


@pytest.mark.parametrize("name,overlap", [("mlp", True), ("cnn", True), ("transformer", False), ("transformer", True)])
def test_step_update_in_backward_equals_update_after(dev, name, overlap, monkeypatch):
    """Sequential.step (Linear layers updated by their parameter-delta kernels) against the
    same step with that switched off (every layer updated after the backward pass): every
    parameter and prediction equal, bit for bit, over two steps. With the side stream on,
    the transformer's head (a product big enough for it) keeps the separate update."""
    from triton_tagi_amd import workloads
    from triton_tagi_amd.layers import linear as linear_mod
    from triton_tagi_amd.update import in_backward

    fused_calls = []
    real = linear_mod.linear_param_deltas_update

    def counting(*a, **k):
        fused_calls.append(1)
        return real(*a, **k)

    monkeypatch.setattr(linear_mod, "linear_param_deltas_update", counting)
    outs = []
    for fused in (True, False):
        if not fused:
            monkeypatch.setattr(in_backward, "active", lambda: None)
        w = workloads.build(name, device="cuda:0")
        w.net.overlap_param_deltas = overlap
        mu, var = w.net.step(w.x, w.y, w.sigma_v)
        mu2, var2 = w.net.step(w.x, w.y, w.sigma_v)  # a second step from the updated state
        torch.cuda.synchronize()
        outs.append([mu, var, mu2, var2] + [t for m, S in gpu_params(w.net) for t in (m, S)])
        assert not any(getattr(layer, "_updated_in_backward", False) for layer in w.net.layers)
        if fused:
            n_fused = len(fused_calls)
            n_linear = sum(isinstance(layer, linear_mod.Linear) for layer in w.net.layers)
    assert n_fused == (0 if (name, overlap) == ("transformer", True) else 2 * n_linear)
    assert len(fused_calls) == n_fused  # none with the switch off
    assert len(outs[0]) == len(outs[1])
    for j, (x, y) in enumerate(zip(*outs)):
        assert torch.equal(x, y), f"{name}: tensor {j} differs"


def test_attention_projection_views_step_like_linear(dev):
    """After its first forward a MultiheadAttentionV2's projections hold column views of
    the side-by-side (E, 3E) parameters. Each projection must still work as a Linear on its
    own: updating the three one by one gives the layer's joint update, bit for bit, and a
    lone projection's forward, backward (within update_in_backward too) and update give
    what a Linear holding dense copies of its parameters gives."""
    from triton_tagi_amd.layers import Linear, MultiheadAttentionV2
    from triton_tagi_amd.update.in_backward import update_in_backward

    B, S, E, H = 2, 16, 64, 4
    cap = 2.0
    params = []
    for joint in (True, False):
        torch.manual_seed(7)
        att = MultiheadAttentionV2(E, H, S, bias=True, gain_weight=0.25, gain_bias=0.5, device=dev)
        r = torch.Generator().manual_seed(8)
        ma, Sa = torch.randn(B, S, E, generator=r).to(dev), 0.1 * torch.rand(B, S, E, generator=r).to(dev)
        dm, dS = 0.1 * torch.randn(B, S, E, generator=r).to(dev), -1e-2 * torch.rand(B, S, E, generator=r).to(dev)
        att.forward(ma, Sa)
        att.backward(dm, dS)
        assert not att.q_proj.mw.is_contiguous()
        if joint:
            att.update(cap)
        else:
            for p in (att.q_proj, att.k_proj, att.v_proj):
                p.update(cap)
        torch.cuda.synchronize()
        params.append([getattr(p, a).clone() for p in (att.q_proj, att.k_proj, att.v_proj)
                       for a in ("mw", "Sw", "mb", "Sb")])
    for j, (x, y) in enumerate(zip(*params)):
        assert torch.equal(x, y), f"parameter {j}: projection-by-projection update differs from the joint one"

    # the v projection on its own, against a Linear with dense copies of its parameters
    proj = att.v_proj
    lin = Linear(E, E, device=dev)
    lin.mw, lin.Sw, lin.mb, lin.Sb = (getattr(proj, a).clone() for a in ("mw", "Sw", "mb", "Sb"))
    r = torch.Generator().manual_seed(9)
    x, Sx = torch.randn(B * S, E, generator=r).to(dev), 0.1 * torch.rand(B * S, E, generator=r).to(dev)
    dz, dSz = 0.1 * torch.randn(B * S, E, generator=r).to(dev), -1e-2 * torch.rand(B * S, E, generator=r).to(dev)
    res = []
    for layer in (proj, lin):
        mz, Sz = layer.forward(x, Sx)
        with update_in_backward(cap):
            dma, dSa = layer.backward(dz, dSz)
        layer.update(cap)  # applies it for the view, skips it for the dense layer
        mz2, Sz2 = layer.forward(x, Sx)
        dma2, dSa2 = layer.backward(dz, dSz)
        layer.update(cap)
        torch.cuda.synchronize()
        res.append([mz, Sz, dma, dSa, mz2, Sz2, dma2, dSa2, layer.mw, layer.Sw, layer.mb, layer.Sb])
    assert proj.mw.data_ptr() == att._qkv["mw"].data_ptr() + 2 * E * 4  # still a view of the buffer
    for j, (x1, y1) in enumerate(zip(*res)):
        assert torch.equal(x1, y1), f"tensor {j}: the projection view differs from a dense Linear"
