"""Fused multi-layer passes against the float64 oracle and against the unfused layers.

The fused passes (Conv2D -> ReLU -> BatchNorm2D and ReLU -> BatchNorm2D forward with an
optional residual add, BatchNorm2D -> ReLU backward, conv input deltas with the shortcut
deltas added in the epilogue) must give the reference's results: checked against the oracle's layer-by-layer chain at the
engine's bar (|gpu - oracle| <= 1e-6 + 1e-4 * scale), and against the engine's own
unfused kernels (same fp32 formulas, so they agree to a few ulps).
"""

from __future__ import annotations

import copy
import ctypes

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


def close_unfused(a, b, what):
    a, b = a.detach().cpu().double(), b.detach().cpu().double()
    err = (a - b).abs().max().item()
    lim = 1e-6 * (b.abs().max().item() + 1e-30) + 1e-12
    assert err <= lim, f"{what}: fused vs unfused max err {err:.3e} > {lim:.3e}"


def make_bn(C, first, preserve, seed, dev):
    from triton_tagi_amd.layers.batchnorm2d import BatchNorm2D

    torch.manual_seed(seed)
    bn = BatchNorm2D(C, device="cpu", gain_w=0.3, gain_b=0.2, preserve_var=preserve)
    r = g(seed)
    bn.mw = 1.0 + 0.1 * torch.randn(C, generator=r)
    if not first:
        bn._is_initialized = True
        bn.running_mean = torch.randn(C, generator=r)
        bn.running_var = torch.rand(C, generator=r) + 0.5
    ref = O.mirror(bn)
    for a in ("mw", "Sw", "mb", "Sb", "running_mean", "running_var"):
        setattr(bn, a, getattr(bn, a).to(dev))
    return bn, ref


FUSED_CASES = [
    # shape, first call, preserve_var, residual add
    ((16, 64, 8, 8), True, False, True),
    ((16, 64, 8, 8), False, False, False),
    ((8, 128, 4, 4), True, True, True),
    ((3, 6, 5, 5), True, True, True),      # channel count off the float4 path
    ((128, 16, 4, 4), False, True, False),
    ((2, 512, 2, 2), True, False, True),
]


@pytest.mark.parametrize("shape,first,preserve,add", FUSED_CASES, ids=[str(c) for c in FUSED_CASES])
def test_relu_bn_fused(dev, shape, first, preserve, add):
    from triton_tagi_amd.layers.fused import bn_relu_backward, relu_bn_forward
    from triton_tagi_amd.layers.relu import ReLU

    N, C, H, W = shape
    seed = N * 7 + C
    bn, rbn = make_bn(C, first, preserve, seed, dev)
    bn_u = copy.deepcopy(bn)
    relu, relu_u, rrelu = ReLU(), ReLU(), O.OReLU()
    r = g(seed + 1)
    mz, Sz = torch.randn(shape, generator=r), 0.05 + torch.rand(shape, generator=r)
    mz[0, 0, 0, 0] = -40.0  # deep in the asymptotic branch of the ReLU
    am, aS = torch.randn(shape, generator=r), torch.rand(shape, generator=r)
    addend = (am.to(dev), aS.to(dev)) if add else None

    ma, Sa = relu_bn_forward(relu, bn, mz.to(dev), Sz.to(dev), addend)
    # oracle: ReLU, BN, then the add
    qa, qS = rrelu.forward(d64(mz), d64(Sz))
    rm, rS = rbn.forward(qa, qS)
    if add:
        rm, rS = rm + d64(am), rS + d64(aS)
    assert_scaled_close(ma, rm, rm.abs() + 1.0, RTOL, ATOL, "fused mean")
    assert_scaled_close(Sa, rS, None, RTOL, ATOL, "fused var")
    assert_scaled_close(bn.running_mean, rbn.running_mean, rbn.running_mean.abs() + 1.0, RTOL, ATOL, "running mean")
    assert_scaled_close(bn.running_var, rbn.running_var, None, RTOL, ATOL, "running var")
    assert_scaled_close(bn.mw, rbn.mw, None, RTOL, ATOL, "gamma")
    assert_scaled_close(relu.J, rrelu.J, None, RTOL, ATOL, "ReLU Jacobian")

    # the engine's unfused layers on the same inputs
    um, uS = relu_u.forward(mz.to(dev), Sz.to(dev))
    um, uS = bn_u.forward(um, uS)
    if add:
        um, uS = um + addend[0], uS + addend[1]
    close_unfused(ma, um, "mean")
    close_unfused(Sa, uS, "var")
    close_unfused(bn.m_hat, bn_u.m_hat, "mhat")

    dma, dSa = torch.randn(shape, generator=r), -torch.rand(shape, generator=r)
    om, oS = bn_relu_backward(bn, relu, dma.to(dev), dSa.to(dev))
    qm, qS = rbn.backward(d64(dma), d64(dSa))
    qm, qS = rrelu.backward(qm, qS)
    assert_scaled_close(om, qm, None, RTOL, ATOL, "fused bwd mean")
    assert_scaled_close(oS, qS, None, RTOL, ATOL, "fused bwd var")
    mh = rbn.m_hat
    assert_scaled_close(bn.delta_mw, rbn.delta_mw, rbn.Sw * (d64(dma) * mh).abs().sum((0, 2, 3)), RTOL, ATOL,
                        "delta gamma")
    assert_scaled_close(bn.delta_Sw, rbn.delta_Sw, None, RTOL, ATOL, "delta Sgamma")
    assert_scaled_close(bn.delta_mb, rbn.delta_mb, rbn.Sb * d64(dma).abs().sum((0, 2, 3)), RTOL, ATOL, "delta beta")
    assert_scaled_close(bn.delta_Sb, rbn.delta_Sb, None, RTOL, ATOL, "delta Sbeta")

    vm, vS = bn_u.backward(dma.to(dev), dSa.to(dev))
    vm, vS = relu_u.backward(vm, vS)
    close_unfused(om, vm, "bwd mean")
    close_unfused(oS, vS, "bwd var")
    close_unfused(bn.delta_mw, bn_u.delta_mw, "delta gamma")


CONV_BN_CASES = [
    # N, C, H, W, Cout, k, stride, padding, padding_type, first call, preserve_var, residual add
    (16, 16, 16, 16, 64, 3, 1, 1, 1, True, True, True),
    (4, 3, 32, 32, 64, 3, 1, 1, 1, True, True, False),     # stem: 3 input channels
    (8, 64, 16, 16, 128, 3, 2, 1, 2, False, False, True),  # stride 2, right/bottom padding
    (3, 5, 7, 9, 6, 3, 2, 1, 2, True, False, True),        # 6 channels, rows not a tile multiple
    (32, 512, 4, 4, 512, 3, 1, 1, 1, False, False, True),  # long reduction: split-K launch
    (16, 256, 8, 8, 512, 2, 2, 0, 1, True, False, False),  # 2x2 projection
]


@pytest.mark.parametrize("case", CONV_BN_CASES, ids=[str(c) for c in CONV_BN_CASES])
def test_conv_relu_bn_fused(dev, case):
    """Conv2D -> ReLU -> BatchNorm2D with the statistics formed in the conv epilogue."""
    from triton_tagi_amd.layers.conv2d import Conv2D
    from triton_tagi_amd.layers.fused import conv_relu_bn_forward, relu_bn_forward
    from triton_tagi_amd.layers.relu import ReLU

    N, C, H, W, Cout, k, s, p, pt, first, preserve, add = case
    seed = N * 13 + C + Cout
    torch.manual_seed(seed)
    conv = Conv2D(C, Cout, k, stride=s, padding=p, padding_type=pt, device="cpu")
    rconv = O.mirror(conv)
    for a in ("mw", "Sw", "mb", "Sb"):
        setattr(conv, a, getattr(conv, a).to(dev))
    conv_u = copy.deepcopy(conv)
    bn, rbn = make_bn(Cout, first, preserve, seed, dev)
    bn_u = copy.deepcopy(bn)
    relu, relu_u, rrelu = ReLU(), ReLU(), O.OReLU()
    r = g(seed + 1)
    ma, Sa = torch.randn(N, C, H, W, generator=r), 0.1 * torch.rand(N, C, H, W, generator=r)
    qz, qSz = rconv.forward(d64(ma), d64(Sa))
    am, aS = torch.randn(qz.shape, generator=r), torch.rand(qz.shape, generator=r)
    addend = (am.to(dev), aS.to(dev)) if add else None

    om, oS = conv_relu_bn_forward(conv, relu, bn, ma.to(dev), Sa.to(dev), addend)
    qa, qS = rrelu.forward(qz, qSz)
    rm, rS = rbn.forward(qa, qS)
    if add:
        rm, rS = rm + d64(am), rS + d64(aS)
    assert_scaled_close(om, rm, rm.abs() + 1.0, RTOL, ATOL, "mean")
    assert_scaled_close(oS, rS, None, RTOL, ATOL, "var")
    assert_scaled_close(relu.J, rrelu.J, None, RTOL, ATOL, "ReLU Jacobian")
    assert_scaled_close(bn.running_mean, rbn.running_mean, rbn.running_mean.abs() + 1.0, RTOL, ATOL, "running mean")
    assert_scaled_close(bn.running_var, rbn.running_var, None, RTOL, ATOL, "running var")
    assert_scaled_close(bn.mw, rbn.mw, None, RTOL, ATOL, "gamma")
    assert conv.ma_in.shape == (N, C, H, W) and conv.spatial == tuple(qz.shape[2:])

    # the engine's separate passes: conv forward, then the ReLU -> BatchNorm2D statistics pass
    uz, uSz = conv_u.forward(ma.to(dev), Sa.to(dev))
    um, uS = relu_bn_forward(relu_u, bn_u, uz, uSz, addend)
    close_unfused(om, um, "mean vs separate passes")
    close_unfused(oS, uS, "var vs separate passes")
    close_unfused(relu.J, relu_u.J, "Jacobian vs separate passes")
    close_unfused(bn.running_var, bn_u.running_var, "running var vs separate passes")


ADD_CASES = [
    # N, C, H, W, Cout, k, stride, padding, padding_type
    (4, 16, 8, 8, 16, 3, 1, 1, 1),
    (4, 16, 8, 8, 32, 3, 2, 1, 2),
    (2, 8, 10, 7, 12, 2, 3, 1, 1),   # stride phases without taps
    (8, 64, 16, 16, 128, 3, 2, 1, 2),
]


@pytest.mark.parametrize("case", ADD_CASES, ids=[str(c) for c in ADD_CASES])
def test_conv_bwd_delta_with_addend(dev, case):
    from triton_tagi_amd.layers.conv2d import Conv2D

    N, C, H, W, Cout, k, s, p, pt = case
    torch.manual_seed(sum(case))
    layer = Conv2D(C, Cout, k, stride=s, padding=p, padding_type=pt, device="cpu")
    ref = O.mirror(layer)
    for a in ("mw", "Sw", "mb", "Sb"):
        setattr(layer, a, getattr(layer, a).to(dev))
    r = g(sum(case) + 5)
    ma, Sa = torch.randn(N, C, H, W, generator=r), torch.rand(N, C, H, W, generator=r)
    mz, _ = layer.forward(ma.to(dev), Sa.to(dev))
    ref.forward(d64(ma), d64(Sa))
    dm, dS = torch.randn(mz.shape, generator=r), -torch.rand(mz.shape, generator=r)
    am, aS = torch.randn(N, C, H, W, generator=r), torch.rand(N, C, H, W, generator=r)
    om, oS = layer._backward(dm.to(dev), dS.to(dev), True, add=(am.to(dev), aS.to(dev)))
    qm, qS = ref.backward(d64(dm), d64(dS))
    scale_m = (O.col2im(d64(dm).permute(0, 2, 3, 1).reshape(-1, Cout).abs() @ ref.mw.abs().T, N, C, H, W, k, s, p,
                        pt)) + d64(am).abs()
    assert_scaled_close(om, qm + d64(am), scale_m, RTOL, ATOL, "dma + addend")
    assert_scaled_close(oS, qS + d64(aS), None, RTOL, ATOL, "dSa + addend")
    um, uS = layer.backward(dm.to(dev), dS.to(dev))
    close_unfused(om, um + am.to(dev), "dma")
    close_unfused(oS, uS + aS.to(dev), "dSa")


FOLD_CASES = [
    # N, C_in (the BatchNorm2D channels), H, W, C_out, k: shapes whose input-delta plan
    # is unsplit with one tile per wave (the fold's condition)
    (16, 64, 32, 32, 64, 3),  # ResNet-18 stage 1 at batch 16
    (16, 6, 16, 16, 8, 3),    # C_in off the float4 path
    (8, 12, 12, 10, 16, 3),   # C_out below the tile-aligned loaders' 16
    (8, 32, 8, 8, 16, 1),
]


@pytest.mark.parametrize("case", FOLD_CASES, ids=[str(c) for c in FOLD_CASES])
def test_conv_bwd_delta_bn_relu_fold(dev, case):
    """tagi_conv2d_bwd_delta_bn_relu (the BatchNorm2D -> ReLU backward in the input-delta
    GEMM's epilogue) against tagi_conv2d_bwd_delta followed by
    tagi_bn_relu_bwd_partials_bias: the propagated deltas bit for bit (same fp32 operations
    on the same products), the parameter and bias deltas after tagi_bn_bwd_finalize_multi
    to 1e-5 (the per-channel sums are grouped by GEMM tile instead of by row block)."""
    from triton_tagi_amd import _lib
    from triton_tagi_amd.layers.conv2d import Conv2D

    N, C, H, W, Cout, k = case
    torch.manual_seed(sum(case))
    conv = Conv2D(C, Cout, k, stride=1, padding=k // 2, device="cpu")
    for a in ("mw", "Sw", "mb", "Sb"):
        setattr(conv, a, getattr(conv, a).to(dev))
    r = g(sum(case) + 11)
    cl = lambda t: t.to(dev).contiguous(memory_format=torch.channels_last)
    dmz, dSz = cl(torch.randn(N, Cout, H, W, generator=r)), cl(-torch.rand(N, Cout, H, W, generator=r))
    mhat, J = cl(torch.randn(N, C, H, W, generator=r)), cl(torch.rand(N, C, H, W, generator=r))
    var = (torch.rand(C, generator=r) + 0.5).to(dev)
    mg = (1 + 0.1 * torch.randn(C, generator=r)).to(dev)
    Sg, Sb, cSb = ((torch.rand(C, generator=r) * 0.1 + 0.01).to(dev) for _ in range(3))
    eps = 1e-5
    conv.input_shape = (N, C, H, W)
    geo = conv._geom(N, C, H, W)
    st = _lib.stream_of(dmz)
    ws = _lib.workspace(_lib.query("tagi_conv2d_bwd_delta_ws_bytes", geo), dev)
    wp, wb = _lib.ws_args(ws)
    part_bytes = _lib.query("tagi_conv2d_bwd_delta_bn_relu_part_bytes", geo)
    assert part_bytes > 0
    part = _lib.workspace(part_bytes, dev)
    fm, fS = _lib.empty_cl(N, C, H, W, dev), _lib.empty_cl(N, C, H, W, dev)
    _lib.call("tagi_conv2d_bwd_delta_bn_relu", dmz.data_ptr(), dSz.data_ptr(), conv.mw.data_ptr(), mhat.data_ptr(),
              J.data_ptr(), var.data_ptr(), mg.data_ptr(), eps, fm.data_ptr(), fS.data_ptr(), part.data_ptr(),
              part_bytes, geo, wp, wb, st)
    # the two calls
    dma, dSa = _lib.empty_cl(N, C, H, W, dev), _lib.empty_cl(N, C, H, W, dev)
    _lib.call("tagi_conv2d_bwd_delta", dmz.data_ptr(), dSz.data_ptr(), conv.mw.data_ptr(), dma.data_ptr(),
              dSa.data_ptr(), geo, wp, wb, st)
    um, uS = _lib.empty_cl(N, C, H, W, dev), _lib.empty_cl(N, C, H, W, dev)
    ws2 = _lib.workspace(_lib.query("tagi_bn_relu_bwd_bias_ws_bytes", N, C, H * W), dev)
    w2p, w2b = _lib.ws_args(ws2)
    _lib.call("tagi_bn_relu_bwd_partials_bias", dma.data_ptr(), dSa.data_ptr(), mhat.data_ptr(), J.data_ptr(),
              var.data_ptr(), mg.data_ptr(), um.data_ptr(), uS.data_ptr(), N, C, H * W, eps, w2p, w2b, st)
    assert torch.equal(fm, um) and torch.equal(fS, uS), "folded deltas differ from the two calls"
    outs = []
    for wsx, nblk in ((part, part_bytes // (24 * C)), (ws2, 0)):
        o = [torch.empty(C, device=dev) for _ in range(6)]
        item = _lib.BnPending(wsx.data_ptr(), Sg.data_ptr(), Sb.data_ptr(), *(t.data_ptr() for t in o[:4]), N, C,
                              H * W, cSb.data_ptr(), o[4].data_ptr(), o[5].data_ptr(), nblk)
        _lib.call("tagi_bn_bwd_finalize_multi", ctypes.byref(item), 1, st)
        outs.append(o)
    names = ("delta gamma", "delta Sgamma", "delta beta", "delta Sbeta", "conv bias delta", "conv bias Sdelta")
    for name, a, b in zip(names, *outs):
        close_unfused_rel(a, b, 1e-5, name)


@pytest.mark.parametrize("case", FOLD_CASES, ids=[str(c) for c in FOLD_CASES])
def test_conv_bwd_delta_add_bn_relu_fold(dev, case):
    """tagi_conv2d_bwd_delta_add_bn_relu (the input deltas plus the shortcut's, then the
    BatchNorm2D -> ReLU backward of the layers in front, in one GEMM epilogue) against
    tagi_conv2d_bwd_delta_add followed by tagi_bn_relu_bwd_partials_bias: the stored sum and
    the propagated deltas bit for bit, the parameter and bias deltas after
    tagi_bn_bwd_finalize_multi to 1e-5 (per-channel sums grouped by GEMM tile)."""
    from triton_tagi_amd import _lib
    from triton_tagi_amd.layers.conv2d import Conv2D

    N, C, H, W, Cout, k = case
    torch.manual_seed(sum(case) + 1)
    conv = Conv2D(C, Cout, k, stride=1, padding=k // 2, device="cpu")
    for a in ("mw", "Sw", "mb", "Sb"):
        setattr(conv, a, getattr(conv, a).to(dev))
    r = g(sum(case) + 13)
    cl = lambda t: t.to(dev).contiguous(memory_format=torch.channels_last)
    dmz, dSz = cl(torch.randn(N, Cout, H, W, generator=r)), cl(-torch.rand(N, Cout, H, W, generator=r))
    am, aS = cl(torch.randn(N, C, H, W, generator=r)), cl(-torch.rand(N, C, H, W, generator=r))
    mhat, J = cl(torch.randn(N, C, H, W, generator=r)), cl(torch.rand(N, C, H, W, generator=r))
    var = (torch.rand(C, generator=r) + 0.5).to(dev)
    mg = (1 + 0.1 * torch.randn(C, generator=r)).to(dev)
    Sg, Sb, cSb = ((torch.rand(C, generator=r) * 0.1 + 0.01).to(dev) for _ in range(3))
    eps = 1e-5
    conv.input_shape = (N, C, H, W)
    geo = conv._geom(N, C, H, W)
    st = _lib.stream_of(dmz)
    ws = _lib.workspace(_lib.query("tagi_conv2d_bwd_delta_ws_bytes", geo), dev)
    wp, wb = _lib.ws_args(ws)
    part_bytes = _lib.query("tagi_conv2d_bwd_delta_bn_relu_part_bytes", geo)
    assert part_bytes > 0
    part = _lib.workspace(part_bytes, dev)
    sm, sS = _lib.empty_cl(N, C, H, W, dev), _lib.empty_cl(N, C, H, W, dev)
    fm, fS = _lib.empty_cl(N, C, H, W, dev), _lib.empty_cl(N, C, H, W, dev)
    _lib.call("tagi_conv2d_bwd_delta_add_bn_relu", dmz.data_ptr(), dSz.data_ptr(), conv.mw.data_ptr(),
              am.data_ptr(), aS.data_ptr(), sm.data_ptr(), sS.data_ptr(), mhat.data_ptr(), J.data_ptr(),
              var.data_ptr(), mg.data_ptr(), eps, fm.data_ptr(), fS.data_ptr(), part.data_ptr(), part_bytes, geo, wp,
              wb, st)
    # the two calls
    dma, dSa = _lib.empty_cl(N, C, H, W, dev), _lib.empty_cl(N, C, H, W, dev)
    _lib.call("tagi_conv2d_bwd_delta_add", dmz.data_ptr(), dSz.data_ptr(), conv.mw.data_ptr(), am.data_ptr(),
              aS.data_ptr(), dma.data_ptr(), dSa.data_ptr(), geo, wp, wb, st)
    um, uS = _lib.empty_cl(N, C, H, W, dev), _lib.empty_cl(N, C, H, W, dev)
    ws2 = _lib.workspace(_lib.query("tagi_bn_relu_bwd_bias_ws_bytes", N, C, H * W), dev)
    w2p, w2b = _lib.ws_args(ws2)
    _lib.call("tagi_bn_relu_bwd_partials_bias", dma.data_ptr(), dSa.data_ptr(), mhat.data_ptr(), J.data_ptr(),
              var.data_ptr(), mg.data_ptr(), um.data_ptr(), uS.data_ptr(), N, C, H * W, eps, w2p, w2b, st)
    assert torch.equal(sm, dma) and torch.equal(sS, dSa), "stored product + addend differs from the add call"
    assert torch.equal(fm, um) and torch.equal(fS, uS), "folded deltas differ from the two calls"
    outs = []
    for wsx, nblk in ((part, part_bytes // (24 * C)), (ws2, 0)):
        o = [torch.empty(C, device=dev) for _ in range(6)]
        item = _lib.BnPending(wsx.data_ptr(), Sg.data_ptr(), Sb.data_ptr(), *(t.data_ptr() for t in o[:4]), N, C,
                              H * W, cSb.data_ptr(), o[4].data_ptr(), o[5].data_ptr(), nblk)
        _lib.call("tagi_bn_bwd_finalize_multi", ctypes.byref(item), 1, st)
        outs.append(o)
    names = ("delta gamma", "delta Sgamma", "delta beta", "delta Sbeta", "conv bias delta", "conv bias Sdelta")
    for name, a, b in zip(names, *outs):
        close_unfused_rel(a, b, 1e-5, name)


def test_conv_bwd_delta_bn_relu_fold_refuses_stride2(dev):
    from triton_tagi_amd import _lib
    from triton_tagi_amd.layers.conv2d import Conv2D

    conv = Conv2D(16, 16, 3, stride=2, padding=1, device="cpu")
    assert _lib.query("tagi_conv2d_bwd_delta_bn_relu_part_bytes", conv._geom(2, 16, 8, 8)) == 0


def close_unfused_rel(a, b, rtol, what):
    a, b = a.detach().cpu().double(), b.detach().cpu().double()
    err = (a - b).abs().max().item()
    lim = rtol * (b.abs().max().item() + 1e-30) + 1e-12
    assert err <= lim, f"{what}: folded vs two-call max err {err:.3e} > {lim:.3e}"


def test_bn_fold_taken_in_step(dev, monkeypatch):
    """Within Sequential.step on ResNet-18 (batch 16) the BatchNorm2D -> ReLU backward of
    each stage-1 block's first BatchNorm2D runs inside the second conv's input-delta GEMM
    (the fold applies there: stride 1, unsplit plan), so the step exercises that path."""
    from triton_tagi_amd import workloads
    from triton_tagi_amd.layers import fused

    taken = []
    orig = fused.conv_bn_relu_backward

    def counting(*a, **k):
        out = orig(*a, **k)
        taken.append(out is not None)
        return out

    monkeypatch.setattr(fused, "conv_bn_relu_backward", counting)
    across = []
    orig_x = fused.conv_add_bn_relu_backward

    def counting_x(*a, **k):
        out = orig_x(*a, **k)
        across.append(out is not None)
        return out

    monkeypatch.setattr(fused, "conv_add_bn_relu_backward", counting_x)
    w = workloads.build("resnet18", device="cuda:0", batch=16)
    w.net.step(w.x, w.y, w.sigma_v)
    torch.cuda.synchronize()
    assert len(taken) == 8 and sum(taken) >= 2, taken
    # across block boundaries: tried by all 8 blocks' first convolutions, last block first
    # (each previous block's closing pair in front of blocks 8..2, the stem's in front of
    # block 1), taken at least by the two stride-1 stage-1 blocks; never by the stride-2
    # first blocks of stages 2-4 (blocks 7, 5, 3: entries 1, 3, 5)
    assert len(across) == 8 and across[-1] and across[-2], across
    assert not any(across[j] for j in (1, 3, 5)), across


def test_fused_step_matches_oracle(dev):
    """Sequential.step (fused passes) on ResNet-18 at batch 16 against the oracle's step:
    predictions, every updated parameter and the BN running statistics."""
    from triton_tagi_amd import workloads

    w = workloads.build("resnet18", device="cuda:0", batch=16)
    onet = O.mirror_net(w.net)
    mu, var = w.net.step(w.x, w.y, w.sigma_v)
    torch.cuda.synchronize()
    rmu, rvar = onet.step(w.x.cpu().double(), w.y.cpu().double(), w.sigma_v)
    failures = []

    def chk(*a):
        try:
            assert_scaled_close(*a)
        except AssertionError as e:
            failures.append(str(e))

    chk(mu, rmu, rmu.abs() + rmu.abs().mean(), RTOL, ATOL, "predicted mean")
    chk(var, rvar, None, RTOL, ATOL, "predicted var")
    gp = []
    for layer in w.net.layers:
        items = layer._update_items() if hasattr(layer, "_update_items") else None
        gp.extend((m, S) for m, S, _, _ in items or [])
    rp = []
    for layer in onet.layers:
        rp.extend((getattr(o, m), getattr(o, S)) for o, m, S, _, _ in layer.param_groups())
    assert len(gp) == len(rp)
    for j, ((gm, gS), (rm, rS)) in enumerate(zip(gp, rp)):
        chk(gm, rm, rm.abs() + rm.abs().mean(), RTOL, ATOL, f"param group {j} mean")
        chk(gS, rS, None, RTOL, ATOL, f"param group {j} variance")
    bn, rbn = w.net.layers[2], onet.layers[2]
    chk(bn.running_mean, rbn.running_mean, rbn.running_mean.abs() + 1.0, RTOL, ATOL, "stem BN running mean")
    chk(bn.running_var, rbn.running_var, None, RTOL, ATOL, "stem BN running var")
    assert not failures, "\n".join(failures)
    assert torch.equal(mu.argmax(-1).cpu(), rmu.argmax(-1))


@pytest.mark.parametrize("B,H,M,K,L", [(2, 3, 33, 20, 45), (4, 8, 64, 32, 64)])
def test_bmm_shared_with_jacobian(dev, B, H, M, K, L):
    """Score deltas times the Remax Jacobian in the product's epilogue, against the oracle's
    product followed by the elementwise Jacobian (multihead_attention.py:239-243)."""
    from triton_tagi_amd.kernels.attention import bmm_shared_right

    r = g(B * H + M)
    am, av = torch.randn(B, H, M, K, generator=r), torch.rand(B, H, M, K, generator=r)
    b = torch.randn(B, H, K, L, generator=r)
    J = torch.rand(B, H, M, L, generator=r)
    m, v = bmm_shared_right(am.to(dev), av.to(dev), b.to(dev), jacobian=J.to(dev))
    rm, rv = O.bmm_shared_right(d64(am), d64(av), d64(b), 1.0)
    J64 = d64(J)
    assert_scaled_close(m, rm * J64, (d64(am).abs() @ d64(b).abs()) * J64, RTOL, ATOL, "mean * J")
    assert_scaled_close(v, rv * J64 * J64, None, RTOL, ATOL, "var * J^2")


@pytest.mark.parametrize("M,K,N", [(300, 70, 45), (16384, 256, 256), (256, 4096, 1024)])
def test_linear_bwd_delta_with_addend(dev, M, K, N):
    """Input deltas added in place to an existing pair in the GEMM epilogue (the sum of the
    attention projections' input deltas), against the oracle plus the addend."""
    from triton_tagi_amd.kernels.common import fused_backward_delta

    r = g(M + K + N)
    dmz, dSz = 0.1 * torch.randn(M, N, generator=r), -1e-2 * torch.rand(M, N, generator=r)
    mw = torch.randn(K, N, generator=r) / N ** 0.5
    am, aS = torch.randn(M, K, generator=r), torch.rand(M, K, generator=r)
    gm, gS = am.to(dev), aS.to(dev)
    om, oS = fused_backward_delta(dmz.to(dev), dSz.to(dev), mw.to(dev), add=(gm, gS))
    assert om.data_ptr() == gm.data_ptr() and oS.data_ptr() == gS.data_ptr()
    rm, rS = O.linear_backward_delta(d64(dmz), d64(dSz), d64(mw))
    assert_scaled_close(om, rm + d64(am), d64(dmz).abs() @ d64(mw).abs().T + d64(am).abs(), RTOL, ATOL,
                        "dma + addend")
    assert_scaled_close(oS, rS + d64(aS), None, RTOL, ATOL, "dSa + addend")


@pytest.mark.parametrize("nchw", [False, True])
@pytest.mark.parametrize("N,C,H,W,k,sc", [(4, 32, 32, 32, 2, False), (3, 5, 12, 12, 3, True), (2, 64, 8, 8, 4, False),
                                          (128, 32, 16, 16, 2, False)])
def test_relu_avgpool_fused(dev, N, C, H, W, k, sc, nchw):
    """ReLU -> AvgPool2D as one pass each way (tagi_relu_avgpool2d_fwd, tagi_avgpool2d_relu_bwd)
    against the two layers' own calls, bit for bit, and against the float64 oracle; C % 4 != 0
    takes the scalar path. ``nchw``: the pooled side row-major (as before a Flatten) instead
    of channels-last, in both directions."""
    from triton_tagi_amd.layers.avgpool2d import AvgPool2D
    from triton_tagi_amd.layers.fused import avgpool_relu_backward, relu_avgpool_forward
    from triton_tagi_amd.layers.relu import ReLU

    r = g(N + C + H + k)
    mz = (2 * torch.randn(N, C, H, W, generator=r)).contiguous(memory_format=torch.channels_last).to(dev)
    Sz = (0.05 + torch.rand(N, C, H, W, generator=r)).contiguous(memory_format=torch.channels_last).to(dev)
    mz[0, 0, 0, :4] = torch.tensor([-30.0, -6.0, 0.0, 40.0], device=dev)  # both tails of the rectified moments
    relu, pool = ReLU(), AvgPool2D(k, spatial_correlation=sc)
    mo, So = relu_avgpool_forward(relu, pool, mz, Sz, nchw=nchw)
    assert mo.is_contiguous() == nchw or mo.shape[2] * mo.shape[3] == 1
    relu_u, pool_u = ReLU(), AvgPool2D(k, spatial_correlation=sc)
    uo, uSo = pool_u.forward(*relu_u.forward(mz, Sz))
    assert torch.equal(mo, uo) and torch.equal(So, uSo), "pooled moments differ from the separate passes"
    assert torch.equal(relu.J, relu_u.J), "ReLU Jacobian differs from the separate pass"
    orelu, opool = O.OReLU(), O.OAvgPool2D(k, sc)
    rm, rS = opool.forward(*orelu.forward(d64(mz), d64(Sz)))
    assert_scaled_close(mo, rm, rm.abs() + 1.0, RTOL, ATOL, "pooled mean vs oracle")
    assert_scaled_close(So, rS, None, RTOL, ATOL, "pooled var vs oracle")
    dm = torch.randn(mo.shape, generator=r).to(dev)
    dS = -torch.rand(mo.shape, generator=r).to(dev)
    if not nchw:  # channels-last deltas, read as they are
        dm = dm.contiguous(memory_format=torch.channels_last)
        dS = dS.contiguous(memory_format=torch.channels_last)
    om, oS = avgpool_relu_backward(pool, relu, dm, dS)
    um, uS = relu_u.backward(*pool_u.backward(dm, dS))
    assert torch.equal(om, um) and torch.equal(oS, uS), "input deltas differ from the separate passes"
    qm, qS = orelu.backward(*opool.backward(d64(dm), d64(dS)))
    assert_scaled_close(om, qm, None, RTOL, ATOL, "input delta mean vs oracle")
    assert_scaled_close(oS, qS, None, RTOL, ATOL, "input delta var vs oracle")


LIN_RELU_CASES = [(256, 784, 256), (256, 256, 128), (300, 70, 45), (33, 2000, 45), (4096, 1024, 1024),
                  (1024, 512, 513)]


@pytest.mark.parametrize("zero_var", [False, True])
@pytest.mark.parametrize("M,K,N", LIN_RELU_CASES, ids=[str(c) for c in LIN_RELU_CASES])
def test_linear_relu_forward_fused(dev, M, K, N, zero_var):
    """Linear -> ReLU as one launch (tagi_linear_fwd_relu) against the two layers' own calls,
    bit for bit, and against the float64 oracle. The shapes take unsplit plans (vector and
    scalar loaders) and split-K plans whose reduction applies the ReLU (vector and scalar
    reduction paths); ``zero_var``: the deterministic-input product (Sa NULL)."""
    from triton_tagi_amd.kernels.common import linear_forward, linear_relu_forward
    from triton_tagi_amd.layers.relu import bayesian_relu

    r = g(M + K + N + zero_var)
    ma = torch.randn(M, K, generator=r)
    Sa = None if zero_var else 0.5 * torch.rand(M, K, generator=r)
    mw = torch.randn(K, N, generator=r) / K ** 0.5
    Sw = torch.rand(K, N, generator=r) / K
    mb, Sb = 0.1 * torch.randn(N, generator=r), 0.01 * torch.rand(N, generator=r)
    mb[:3] = torch.tensor([-40.0, 25.0, 0.0])  # both tails of the rectified moments
    on = lambda t: None if t is None else t.to(dev)  # noqa: E731
    args = (ma.to(dev), on(Sa), mw.to(dev), Sw.to(dev), mb.to(dev), Sb.to(dev))
    am, aS, J = linear_relu_forward(*args)
    um, uS, uJ = bayesian_relu(*linear_forward(*args))
    assert torch.equal(am, um) and torch.equal(aS, uS) and torch.equal(J, uJ), "differs from the separate passes"
    Sa64 = torch.zeros(M, K, dtype=torch.float64) if zero_var else d64(Sa)
    rmz, rSz = O.linear_moments(d64(ma), Sa64, d64(mw), d64(Sw), d64(mb), d64(Sb))
    orelu = O.OReLU()
    rm, rS = orelu.forward(rmz, rSz)
    # first-order error of the product's mean (relative to its absolute terms T) carried
    # through the ReLU: d mu_a / d mu_z = J <= 1, d S_a / d mu_z = 2 mu_a (1 - J)
    T = d64(ma).abs() @ d64(mw).abs() + d64(mb).abs()
    assert_scaled_close(am, rm, T + rm.abs(), RTOL, ATOL, "ReLU mean vs oracle")
    assert_scaled_close(aS, rS, rS + 2 * rm.abs() * T, RTOL, ATOL, "ReLU var vs oracle")
    assert_scaled_close(J, orelu.J, None, RTOL, ATOL, "ReLU Jacobian vs oracle")


LIN_JAC_CASES = [(256, 784, 256), (300, 70, 45), (1024, 512, 513), (4096, 1024, 1024), (128, 1024, 256)]


@pytest.mark.parametrize("M,K,N", LIN_JAC_CASES, ids=[str(c) for c in LIN_JAC_CASES])
def test_linear_bwd_delta_jacobian(dev, M, K, N):
    """Input deltas times the ReLU Jacobian in the product's epilogue
    (tagi_linear_bwd_delta_jacobian) against the product followed by tagi_jacobian_bwd (the
    variance within one rounding of J^2) and against the float64 oracle."""
    from triton_tagi_amd.kernels.common import fused_backward_delta
    from triton_tagi_amd.layers.relu import jacobian_backward

    r = g(M + 2 * K + N)
    dmz, dSz = 0.1 * torch.randn(M, N, generator=r), -1e-2 * torch.rand(M, N, generator=r)
    mw = torch.randn(K, N, generator=r) / N ** 0.5
    J = torch.rand(M, K, generator=r)
    J[0, :3] = torch.tensor([0.0, 1.0, 1e-20])
    om, oS = fused_backward_delta(dmz.to(dev), dSz.to(dev), mw.to(dev), jacobian=J.to(dev))
    um, uS = jacobian_backward(*fused_backward_delta(dmz.to(dev), dSz.to(dev), mw.to(dev)), J.to(dev))
    assert torch.equal(om, um), "mean differs from the separate passes"
    close_unfused(oS, uS, "variance")
    orelu = O.OReLU()
    orelu.J = d64(J)
    rm, rS = orelu.backward(*O.linear_backward_delta(d64(dmz), d64(dSz), d64(mw)))
    assert_scaled_close(om, rm, (d64(dmz).abs() @ d64(mw).abs().T) * d64(J), RTOL, ATOL, "dma * J vs oracle")
    assert_scaled_close(oS, rS, None, RTOL, ATOL, "dSa * J^2 vs oracle")


def test_linear_relu_folds_taken_in_step(dev, monkeypatch):
    """In the MLP step (784-256-128-10) both Linear -> ReLU pairs run as one forward launch
    and one input-delta launch each; no ReLU runs its own passes, and the step still
    matches the oracle's."""
    from triton_tagi_amd import workloads
    from triton_tagi_amd.layers.linear import Linear
    from triton_tagi_amd.layers.relu import ReLU

    w = workloads.build("mlp", device="cuda:0", batch=64)
    onet = O.mirror_net(w.net)
    calls = {"fwd": 0, "bwd": 0}
    fr, bj = Linear.forward_relu, Linear.backward_jacobian

    def fwd(self, *a, **k):
        calls["fwd"] += 1
        return fr(self, *a, **k)

    def bwd(self, *a, **k):
        calls["bwd"] += 1
        return bj(self, *a, **k)

    def forbid(*a, **k):
        raise AssertionError("a ReLU ran its own pass")

    monkeypatch.setattr(Linear, "forward_relu", fwd)
    monkeypatch.setattr(Linear, "backward_jacobian", bwd)
    monkeypatch.setattr(ReLU, "forward", forbid)
    monkeypatch.setattr(ReLU, "backward", forbid)
    mu, var = w.net.step(w.x, w.y, w.sigma_v)
    torch.cuda.synchronize()
    assert calls == {"fwd": 2, "bwd": 2}
    rmu, rvar = onet.step(w.x.cpu().double(), w.y.cpu().double(), w.sigma_v)
    assert_scaled_close(mu, rmu, rmu.abs() + rmu.abs().mean(), RTOL, ATOL, "predicted mean")
    assert_scaled_close(var, rvar, None, RTOL, ATOL, "predicted var")
    for layer, olayer in zip(w.net.layers, onet.layers):
        if isinstance(layer, Linear):
            for (m, S, _, _), (o, mn, Sn, _, _) in zip(layer._update_items(), olayer.param_groups()):
                rm_, rS_ = getattr(o, mn), getattr(o, Sn)
                assert_scaled_close(m, rm_, rm_.abs() + rm_.abs().mean(), RTOL, ATOL, "updated mean")
                assert_scaled_close(S, rS_, None, RTOL, ATOL, "updated variance")
