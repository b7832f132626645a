"""GPU parity of the output heads and further layers against the float64 CPU oracle.

HRC sparse innovation and class probabilities, heteroscedastic innovation, EvenSoftplus,
MaxPool2D and LayerNorm, each at kernel level (including the edge cases the reference's
tests hold: 2 classes, repeated labels, ties in a pooling window, overlapping and padded
windows, rows of one element), then a full step of a small network per head
(step_hrc; the heteroscedastic step; a CNN with MaxPool2D and LayerNorm).
Tolerance |gpu - oracle| <= 1e-6 + 1e-4 * scale (scale = |oracle|, plus the mean
absolute value for means, which are sums with cancellation). Selections (pool indices,
node routing, zero patterns) must match exactly.
"""

from __future__ import annotations

import pytest
import torch

from conftest import assert_scaled_close
from oracle import tagi_oracle as O

pytestmark = pytest.mark.gpu

RTOL, ATOL = 1e-4, 1e-6


def g(seed):
    return torch.Generator().manual_seed(seed)


def d64(t):
    return t.detach().to("cpu", torch.float64)


def mscale(ref):
    return ref.abs() + ref.abs().mean()


# -------------------------------------------------------------------- HRC kernels
# fewer than 32 outputs: one thread per row in 256-row blocks ((28, 700): 31 outputs, three
# blocks, the last partial); wider outputs: one thread per output element
@pytest.mark.parametrize("n_classes,B", [(2, 5), (10, 256), (28, 700), (100, 33), (1000, 64)])
def test_innovation_indexed_and_labels(dev, n_classes, B):
    from triton_tagi_amd.hrc_softmax import class_to_obs, labels_to_hrc
    from triton_tagi_amd.update.observation import compute_innovation_with_indices, hrc_innovation

    h = class_to_obs(n_classes)
    r = g(n_classes + B)
    width = h.len + 3  # wider than the tree: extra outputs get no innovation
    ma = torch.randn(B, width, generator=r)
    Sa = 0.1 * torch.rand(B, width, generator=r) + 1e-3
    labels = torch.randint(0, n_classes, (B,), generator=r)
    labels[: min(B, 3)] = labels[0]  # repeated labels
    y_obs, y_idx = labels_to_hrc(labels, h)
    var_obs = torch.full_like(y_obs, 0.05**2)
    dm, dS = compute_innovation_with_indices(ma.to(dev), Sa.to(dev), y_obs.to(dev), var_obs.to(dev), y_idx.to(dev))
    rm, rS = O.innovation_indexed(d64(ma), d64(Sa), d64(y_obs), d64(var_obs), y_idx.long())
    assert torch.equal(dm.cpu() != 0, rm != 0) and torch.equal(dS.cpu() != 0, rS != 0)
    assert_scaled_close(dm, rm, None, RTOL, ATOL, "delta_mu")
    assert_scaled_close(dS, rS, None, RTOL, ATOL, "delta_S")
    lm, lS = hrc_innovation(ma.to(dev), Sa.to(dev), labels.to(dev), h, 0.05)
    assert torch.equal(lm.cpu(), dm.cpu()) and torch.equal(lS.cpu(), dS.cpu())


def test_innovation_indexed_repeated_and_out_of_range_nodes(dev):
    from triton_tagi_amd.update.observation import compute_innovation_with_indices, hrc_innovation
    from triton_tagi_amd.hrc_softmax import class_to_obs

    r = g(3)
    ma, Sa = torch.randn(2, 6, generator=r), torch.rand(2, 6, generator=r) + 0.1
    idx = torch.tensor([[3, 3, 0, 7], [6, 1, 2, -4]], dtype=torch.int32)
    y = torch.tensor([[1.0, -1.0, 1.0, 1.0], [-1.0, 1.0, 1.0, 1.0]])
    v = torch.tensor([[0.1, 0.2, 0.1, 0.1], [0.3, 0.1, 0.2, 0.1]])
    dm, dS = compute_innovation_with_indices(ma.to(dev), Sa.to(dev), y.to(dev), v.to(dev), idx.to(dev))
    rm, rS = O.innovation_indexed(d64(ma), d64(Sa), d64(y), d64(v), idx.long())
    assert_scaled_close(dm, rm, None, RTOL, ATOL, "delta_mu")
    assert_scaled_close(dS, rS, None, RTOL, ATOL, "delta_S")
    assert int((dm.cpu() != 0).sum()) == 4
    # a label outside the classes marks its row instead of reading out of the tables
    h = class_to_obs(4)
    lm, lS = hrc_innovation(ma.to(dev), Sa.to(dev), torch.tensor([1, 4]).to(dev), h, 0.1)
    assert torch.isnan(lm[1]).all() and torch.isnan(lS[1]).all() and not torch.isnan(lm[0]).any()


# (10, 600) and (30, 300): several 256-row blocks of the row-per-thread kernel, the last
# partial; 40 classes: the one-wavefront-per-row kernel; 100 and more: one block per row;
# 10000 classes: a tree wider than that kernel's LDS table
@pytest.mark.parametrize("n_classes,B", [(2, 4), (10, 128), (10, 600), (30, 300), (40, 70), (100, 16), (1000, 8),
                                         (10000, 3)])
def test_class_probs_and_predicted_labels(dev, n_classes, B):
    from triton_tagi_amd.hrc_softmax import class_to_obs, get_predicted_labels, obs_to_class_probs

    h = class_to_obs(n_classes)
    r = g(n_classes * 7 + B)
    ma = 0.8 * torch.randn(B, h.len, generator=r)
    Sa = 0.2 * torch.rand(B, h.len, generator=r)
    P = obs_to_class_probs(ma.to(dev), Sa.to(dev), h)
    R = O.hrc_class_probs(d64(ma), d64(Sa), d64(h.obs), h.idx.long(), 3.0)
    assert_scaled_close(P, R, None, RTOL, ATOL, "class probabilities")
    pred = get_predicted_labels(ma.to(dev), Sa.to(dev), h)
    assert pred.dtype == torch.int64 and torch.equal(pred.cpu(), P.cpu().argmax(1))
    top2 = R.topk(2, dim=1).values
    clear = (top2[:, 0] - top2[:, 1]) > 1e-3 * top2[:, 0]
    assert torch.equal(pred.cpu()[clear], R.argmax(1)[clear])
    # strongly positive nodes: class 0 (all bits 0) wins
    assert get_predicted_labels(torch.full((1, h.len), 10.0, device=dev), torch.zeros(1, h.len, device=dev), h).item() == 0
    # a NaN node moment: the classes whose path uses it are NaN, and NaN is the largest
    # value for the argmax, as in torch.argmax
    ma[B // 2, h.len - 1] = float("nan")
    P = obs_to_class_probs(ma.to(dev), Sa.to(dev), h).cpu()
    assert P[B // 2].isnan().any() and not P[:B // 2].isnan().any()
    assert torch.equal(get_predicted_labels(ma.to(dev), Sa.to(dev), h).cpu(), P.argmax(1))


def test_class_probs_in_the_far_tails(dev):
    """Node moments with |mu| / sqrt(1/alpha^2 + S) from 6 to 40: the node probability
    Phi is formed as Q(-x) = erfc(-x/sqrt 2)/2 here, so the far-tail class probabilities
    are the tiny positive values of exact arithmetic (the float64 oracle, torch's ndtr),
    held to the 1e-4 bar; the reference's float32 0.5*(1+erf(x/sqrt 2)) rounds them to
    exactly 0 below x ~ -5.9 (hrc_softmax.py:164-208). Either way they are far below the
    absolute tolerance and the predicted labels are the oracle's."""
    from triton_tagi_amd.hrc_softmax import class_to_obs, get_predicted_labels, obs_to_class_probs

    h = class_to_obs(10)
    r = g(77)
    B = 64
    sign = torch.where(torch.rand(B, h.len, generator=r) < 0.5, -1.0, 1.0)
    ma = sign * (6.0 + 34.0 * torch.rand(B, h.len, generator=r)) * (1.0 / 3.0)
    Sa = torch.zeros(B, h.len)
    P = obs_to_class_probs(ma.to(dev), Sa.to(dev), h)
    R = O.hrc_class_probs(d64(ma), d64(Sa), d64(h.obs), h.idx.long(), 3.0)
    assert_scaled_close(P, R, None, RTOL, ATOL, "far-tail class probabilities")
    # the reference's float32 form of the same products (zeros in the far tails) sits within
    # the same tolerance of the oracle
    x = ma / torch.sqrt(torch.tensor(1.0 / 9.0) + Sa)
    node = (0.5 * (1.0 + torch.erf(x * 0.7071067811865476)))[:, h.idx.long() - 1]
    ref32 = torch.where(h.obs > 0, node, 1.0 - node).prod(dim=2)
    assert_scaled_close(ref32, R, None, RTOL, ATOL, "reference float32 form")
    # labels where some class keeps a probability float32 can hold; in rows where every
    # class path crosses a node far in its tail all products are below 1e-30 and the label
    # is decided by rounding in every implementation
    pred = get_predicted_labels(ma.to(dev), Sa.to(dev), h).cpu()
    ok = R.max(1).values > 1e-30
    assert ok.sum() > B // 2
    assert torch.equal(pred[ok], R.argmax(1)[ok])


# ---------------------------------------------------------- heteroscedastic head
@pytest.mark.parametrize("shape,offset", [((4, 10), 0), ((128, 1), 0), ((3, 7), 1), ((64, 256, 8), 0)])
def test_heteros_innovation(dev, shape, offset):
    from triton_tagi_amd.update.observation import compute_innovation

    r = g(sum(shape) + offset)
    y = torch.randn(*shape, generator=r)
    pshape = (*shape[:-1], 2 * shape[-1])
    n = torch.Size(pshape).numel()
    mu = torch.randn(n + offset, generator=r)
    var = 0.05 + torch.rand(n + offset, generator=r)
    mu_v = mu[offset:].view(pshape)
    mu_v[..., 1::2] = 0.1 + torch.rand(*shape, generator=r)  # noise-variance means are positive
    var_v = var[offset:].view(pshape)
    # the offset view is 4-byte aligned only: the scalar path
    mg, vg = mu.to(dev)[offset:].view(pshape), var.to(dev)[offset:].view(pshape)
    dm, dS = compute_innovation(y.to(dev), mg, vg, 0.05)
    rm, rS = O.heteros_innovation(d64(y), d64(mu_v), d64(var_v))
    assert dm.shape == pshape
    assert_scaled_close(dm, rm, mscale(rm), RTOL, ATOL, "delta_mu")
    assert_scaled_close(dS, rS, mscale(rS), RTOL, ATOL, "delta_S")


@pytest.mark.parametrize("n,offset", [(20, 0), (4096 * 10, 0), (13, 0), (40, 1)])
def test_even_softplus(dev, n, offset):
    from triton_tagi_amd.layers.even_softplus import EvenSoftplus

    r = g(n + offset)
    mz = torch.cat([torch.linspace(-30, 40, n // 2 + 1), 3 * torch.randn(n - n // 2 - 1 + offset, generator=r)])
    Sz = torch.rand(n + offset, generator=r)
    layer = EvenSoftplus(n // 2)
    ma, Sa = layer.forward(mz.to(dev)[offset:], Sz.to(dev)[offset:])
    rm, rS, rJ = O.even_softplus(d64(mz[offset:]), d64(Sz[offset:]))
    assert_scaled_close(ma, rm, None, RTOL, ATOL, "mu_a")
    assert_scaled_close(Sa, rS, None, RTOL, ATOL, "S_a")
    assert_scaled_close(layer.J, rJ, None, RTOL, ATOL, "J")
    dm, dS = torch.randn(n, generator=r), -torch.rand(n, generator=r)
    om, oS = layer.backward(dm.to(dev), dS.to(dev))
    assert_scaled_close(om, d64(dm) * rJ, None, RTOL, ATOL, "delta_mu")
    assert_scaled_close(oS, d64(dS) * rJ * rJ, None, RTOL, ATOL, "delta_S")


# -------------------------------------------------------------------- MaxPool2D
POOLS = [(2, 2, 0), (3, 2, 1), (3, 1, 1), (2, 1, 0), (4, 4, 2), (3, 3, 0)]


@pytest.mark.parametrize("k,s,p", POOLS)
@pytest.mark.parametrize("channels_last,C", [(False, 5), (True, 5), (True, 8)])
def test_maxpool(dev, k, s, p, channels_last, C):
    """C = 8 channels-last takes the float4 path, C = 5 the per-element one."""
    import torch.nn.functional as F

    from triton_tagi_amd.layers.maxpool2d import MaxPool2D

    r = g(k * 100 + s * 10 + p + int(channels_last) + C)
    N, H, W = 3, 11, 9
    ma = torch.randn(N, C, H, W, generator=r)
    ma[0, 0, :2, :2] = 1.5  # ties inside one window
    Sa = torch.rand(N, C, H, W, generator=r)
    fmt = torch.channels_last if channels_last else torch.contiguous_format
    layer = MaxPool2D(k, s, p)
    mz, Sz = layer.forward(ma.to(dev).contiguous(memory_format=fmt), Sa.to(dev).contiguous(memory_format=fmt))
    ref, ridx = F.max_pool2d_with_indices(ma, k, stride=s, padding=p)
    assert mz.shape == ref.shape and mz.is_contiguous(memory_format=fmt)
    assert torch.equal(layer.pool_idx.cpu().long(), ridx)
    assert torch.equal(mz.cpu(), ref)
    assert torch.equal(Sz.cpu(), Sa.reshape(N, C, -1).gather(2, ridx.reshape(N, C, -1)).reshape(ref.shape))
    o = O.OMaxPool2D(k, s, p)
    o.forward(d64(ma), d64(Sa))
    dm, dS = torch.randn(*ref.shape, generator=r), -torch.rand(*ref.shape, generator=r)
    om, oS = layer.backward(dm.to(dev), dS.to(dev))
    rm, rS = o.backward(d64(dm), d64(dS))
    assert torch.equal(om.cpu() != 0, rm != 0)
    assert_scaled_close(om, rm, mscale(rm), RTOL, ATOL, "delta_mu")
    assert_scaled_close(oS, rS, mscale(rS), RTOL, ATOL, "delta_S")


# -------------------------------------------------------------------- LayerNorm
@pytest.mark.parametrize("rows,D", [(1, 3), (7, 16), (300, 256), (33, 100), (5, 1024), (9, 1500), (64, 4096)])
def test_layernorm(dev, rows, D):
    from triton_tagi_amd.layers.layernorm import LayerNorm

    r = g(rows * 13 + D)
    layer = LayerNorm(D, device=dev)
    mw, Sw = 1 + 0.1 * torch.randn(D, generator=r), 0.05 * torch.rand(D, generator=r)
    mb, Sb = 0.1 * torch.randn(D, generator=r), 0.02 * torch.rand(D, generator=r)
    layer.mw, layer.Sw, layer.mb, layer.Sb = (t.to(dev) for t in (mw, Sw, mb, Sb))
    ma, Sa = 2 * torch.randn(rows, D, generator=r) + 0.5, 0.3 * torch.rand(rows, D, generator=r)
    mz, Sz = layer.forward(ma.to(dev), Sa.to(dev))
    o = O.OLayerNorm(d64(mw), d64(Sw), d64(mb), d64(Sb), 1e-5)
    rm, rS = o.forward(d64(ma), d64(Sa))
    assert layer.mu_ra.shape == (rows, 1) and layer.var_ra.shape == (rows, 1)
    assert_scaled_close(layer.mu_ra, o.mu_ra, mscale(d64(ma)).mean(1, keepdim=True), RTOL, ATOL, "mu_ra")
    assert_scaled_close(layer.var_ra, o.var_ra, None, RTOL, ATOL, "var_ra")
    assert_scaled_close(mz, rm, mscale(rm), RTOL, ATOL, "mu_z")
    assert_scaled_close(Sz, rS, None, RTOL, ATOL, "S_z")
    dmz, dSz = torch.randn(rows, D, generator=r), -torch.rand(rows, D, generator=r)
    dma, dSa = layer.backward(dmz.to(dev), dSz.to(dev))
    em, eS = o.backward(d64(dmz), d64(dSz))
    assert_scaled_close(dma, em, mscale(em), RTOL, ATOL, "delta_ma")
    assert_scaled_close(dSa, eS, None, RTOL, ATOL, "delta_Sa")
    for name, scale in (("delta_mw", True), ("delta_Sw", False), ("delta_mb", True), ("delta_Sb", False)):
        ref = getattr(o, name)
        # parameter deltas are sums over rows: relative to the sum of absolute terms
        sc = ref.abs() + ref.abs().mean() if scale else None
        assert_scaled_close(getattr(layer, name), ref, sc, RTOL, ATOL, name)


# ------------------------------------------------------------ network-level steps
def gpu_params(net):
    out = []
    for layer in net.layers:
        for m, S, _, _ in (layer._update_items() or []) if hasattr(layer, "_update_items") else []:
            out.append((m, S))
    return out


def oracle_params(onet):
    return [(getattr(o, m), getattr(o, S)) for layer in onet.layers for o, m, S, _, _ in layer.param_groups()]


def compare_params(net, onet):
    gp, op = gpu_params(net), oracle_params(onet)
    assert len(gp) == len(op) and gp
    for i, ((m, S), (rm, rS)) in enumerate(zip(gp, op)):
        assert_scaled_close(m.reshape(rm.shape), rm, mscale(rm), RTOL, ATOL, f"param {i} mean")
        assert_scaled_close(S.reshape(rS.shape), rS, None, RTOL, ATOL, f"param {i} variance")


def test_step_hrc_mlp(dev):
    import triton_tagi_amd as tt

    torch.manual_seed(0)
    h = tt.class_to_obs(10)
    net = tt.Sequential([tt.Linear(64, 128, device="cpu"), tt.ReLU(), tt.LayerNorm(128, device="cpu"),
                         tt.Linear(128, h.len, device="cpu")], device=dev)
    onet = O.mirror_net(net)
    r = g(42)
    for step in range(2):
        x = torch.rand(256, 64, generator=r)
        labels = torch.randint(0, 10, (256,), generator=r)
        mu, var = net.step_hrc(x.to(dev), labels.to(dev), h, 0.05)
        rmu, rvar = onet.step_hrc(d64(x), labels, 10, 0.05)
        torch.cuda.synchronize()
        assert_scaled_close(mu, rmu, mscale(rmu), RTOL, ATOL, f"step {step} mu")
        assert_scaled_close(var, rvar, None, RTOL, ATOL, f"step {step} var")
        compare_params(net, onet)


def test_step_hrc_sequence_output(dev):
    import triton_tagi_amd as tt

    torch.manual_seed(1)
    h = tt.class_to_obs(16)
    net = tt.Sequential([tt.Linear(8, 32, device="cpu"), tt.ReLU(), tt.Linear(32, h.len, device="cpu")], device=dev)
    onet = O.mirror_net(net)
    r = g(7)
    x = torch.randn(4, 5, 8, generator=r)
    labels = torch.randint(0, 16, (4, 5), generator=r)
    mu, var = net.step_hrc(x.to(dev), labels.to(dev), h, 0.1)
    rmu, rvar = onet.step_hrc(d64(x), labels, 16, 0.1)
    torch.cuda.synchronize()
    assert mu.shape == (4, 5, h.len)
    assert_scaled_close(mu, rmu, mscale(rmu), RTOL, ATOL, "mu")
    compare_params(net, onet)


def test_heteroscedastic_step(dev):
    import triton_tagi_amd as tt

    torch.manual_seed(2)
    K = 3
    net = tt.Sequential([tt.Linear(16, 64, device="cpu"), tt.ReLU(), tt.Linear(64, 2 * K, device="cpu"),
                         tt.EvenSoftplus(K)], device=dev)
    onet = O.mirror_net(net)
    r = g(5)
    for step in range(2):
        x = torch.randn(128, 16, generator=r)
        y = torch.randn(128, K, generator=r)
        mu, var = net.step(x.to(dev), y.to(dev), 0.0)
        rmu, rvar = onet.step_heteros(d64(x), d64(y))
        torch.cuda.synchronize()
        assert_scaled_close(mu, rmu, mscale(rmu), RTOL, ATOL, f"step {step} mu")
        assert_scaled_close(var, rvar, None, RTOL, ATOL, f"step {step} var")
        compare_params(net, onet)


def test_cnn_maxpool_step(dev):
    import triton_tagi_amd as tt

    torch.manual_seed(3)
    net = tt.Sequential([
        tt.Conv2D(3, 16, 3, padding=1, device="cpu"), tt.ReLU(), tt.MaxPool2D(2),
        tt.Conv2D(16, 16, 3, padding=1, device="cpu"), tt.ReLU(), tt.BatchNorm2D(16, device="cpu"),
        tt.MaxPool2D(3, 2, 1), tt.Flatten(), tt.Linear(16 * 4 * 4, 32, device="cpu"), tt.ReLU(),
        tt.LayerNorm(32, device="cpu"), tt.Linear(32, 10, device="cpu"), tt.Remax(),
    ], device=dev)
    onet = O.mirror_net(net)
    r = g(9)
    x = torch.randn(32, 3, 16, 16, generator=r)
    y = torch.nn.functional.one_hot(torch.randint(0, 10, (32,), generator=r), 10).float()
    mu, var = net.step(x.to(dev), y.to(dev), 0.05)
    rmu, rvar = onet.step(d64(x), d64(y), 0.05)
    torch.cuda.synchronize()
    assert_scaled_close(mu, rmu, mscale(rmu), RTOL, ATOL, "mu")
    assert_scaled_close(var, rvar, None, RTOL, ATOL, "var")
    compare_params(net, onet)


def test_checkpoint_round_trip_on_gpu(dev, tmp_path):
    import triton_tagi_amd as tt

    def build(cfg):
        torch.manual_seed(cfg["seed"])
        return tt.Sequential([tt.Linear(8, 16, device="cpu"), tt.ReLU(), tt.LayerNorm(16, device="cpu"),
                              tt.Linear(16, 4, device="cpu")], device=dev)

    net = build({"seed": 0})
    x, y = torch.randn(32, 8, device=dev), torch.randn(32, 4, device=dev)
    net.step(x, y, 0.1)
    run = tt.RunDir("synthetic", "mlp", "tagi", base=str(tmp_path))
    path = run.save_checkpoint(net, 1, {"seed": 5})
    other, cfg, ep = tt.load_model(path, build, device=dev)
    assert ep == 1 and other.layers[0].mw.device.type == "cuda"
    a, _ = net.step(x, y, 0.1)
    b, _ = other.step(x, y, 0.1)
    torch.cuda.synchronize()
    assert torch.equal(a.cpu(), b.cpu())


def test_resnet18_hrc_workload_step(dev):
    from triton_tagi_amd import workloads

    w = workloads.build("resnet18_hrc", device=dev, batch=4)
    onet = O.mirror_net(w.net)
    mu, var = w.step()
    rmu, rvar = onet.step_hrc(d64(w.x), w.y.cpu(), 10, w.sigma_v)
    torch.cuda.synchronize()
    assert mu.shape == (4, 11)
    assert_scaled_close(mu, rmu, mscale(rmu), RTOL, ATOL, "mu")
    assert_scaled_close(var, rvar, None, RTOL, ATOL, "var")
    compare_params(w.net, onet)


# ------------------------------------------------------------ eval-mode forward
def test_eval_forward_uses_running_statistics(dev):
    """Inference after training (batchnorm2d.py:393-395): BatchNorm2D normalises with its
    running statistics, the fused ReLU->BatchNorm2D passes step aside, and train() restores
    the batch-statistics path."""
    from triton_tagi_amd import workloads

    w = workloads.build("resnet18", device=dev, batch=8)
    for _ in range(2):
        w.step()
    w.net.eval()
    r = g(77)
    x = torch.randn(8, 3, 32, 32, generator=r)
    mu, var = w.net.forward(x.to(dev))
    onet = O.mirror_net(w.net)
    rmu, rvar = onet.forward(d64(x))
    torch.cuda.synchronize()
    assert_scaled_close(mu, rmu, mscale(rmu), RTOL, ATOL, "eval mu")
    assert_scaled_close(var, rvar, None, RTOL, ATOL, "eval var")
    assert torch.equal(mu.cpu().argmax(1), rmu.argmax(1))
    # the prediction of one sample does not depend on the rest of the batch in eval mode
    mu1, _ = w.net.forward(x[:1].to(dev))
    assert_scaled_close(mu1, rmu[:1], mscale(rmu[:1]), RTOL, ATOL, "eval mu, batch of one")
    w.net.train()
    mu_t, _ = w.net.forward(x.to(dev))
    assert not torch.allclose(mu_t.cpu(), mu.cpu())


def test_eval_hrc_predicted_labels(dev):
    import triton_tagi_amd as tt

    torch.manual_seed(4)
    h = tt.class_to_obs(10)
    net = tt.Sequential([
        tt.Conv2D(3, 16, 3, padding=1, device="cpu"), tt.ReLU(), tt.BatchNorm2D(16, device="cpu"),
        tt.AvgPool2D(2), tt.Flatten(), tt.Linear(16 * 8 * 8, 64, device="cpu"), tt.ReLU(),
        tt.Linear(64, h.len, device="cpu"),
    ], device=dev)
    r = g(8)
    for _ in range(3):
        x = torch.randn(64, 3, 16, 16, generator=r)
        net.step_hrc(x.to(dev), torch.randint(0, 10, (64,), generator=r).to(dev), h, 0.05)
    net.eval()
    x = torch.randn(32, 3, 16, 16, generator=r)
    mu, var = net.forward(x.to(dev))
    pred = tt.get_predicted_labels(mu, var, h)
    onet = O.mirror_net(net)
    rmu, rvar = onet.forward(d64(x))
    R = O.hrc_class_probs(rmu, rvar, d64(h.obs), h.idx.long())
    top2 = R.topk(2, dim=1).values
    clear = (top2[:, 0] - top2[:, 1]) > 1e-3 * top2[:, 0]
    assert clear.sum() >= 16
    assert torch.equal(pred.cpu()[clear], R.argmax(1)[clear])


def test_layernorm_sequence_input_and_no_bias(dev):
    """(B, S, D) input (rows = B*S) and bias=False (zero beta that is never updated)."""
    import triton_tagi_amd as tt

    torch.manual_seed(6)
    layer = tt.LayerNorm(48, bias=False, device="cpu")
    net = tt.Sequential([tt.Linear(16, 48, device="cpu"), tt.ReLU(), layer, tt.Linear(48, 8, device="cpu")],
                        device=dev)
    onet = O.mirror_net(net)
    r = g(12)
    x, y = torch.randn(4, 9, 16, generator=r), torch.randn(4, 9, 8, generator=r)
    mu, var = net.step(x.to(dev), y.to(dev), 0.3)
    rmu, rvar = onet.step(d64(x), d64(y), 0.3)
    torch.cuda.synchronize()
    assert mu.shape == (4, 9, 8) and layer.mu_ra.shape == (36, 1)
    assert_scaled_close(mu, rmu, mscale(rmu), RTOL, ATOL, "mu")
    assert_scaled_close(var, rvar, None, RTOL, ATOL, "var")
    compare_params(net, onet)
    assert torch.all(layer.mb == 0) and torch.all(layer.Sb == 0) and layer.num_parameters == 2 * 48
