"""Kernel-level parity: every HIP entry point against the float64 CPU oracle.

Inputs are seeded fp32 tensors; the oracle evaluates the reference's equations on the
same values in float64. Tolerance (the engine's bar): |gpu - oracle| <= 1e-6 + 1e-4 *
scale, where scale is |oracle| for variances and elementwise results, and the sum of
absolute products for GEMM means (fp32 rounding is relative to that sum when terms
cancel).
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


LINEAR_SHAPES = [(1, 3, 2), (37, 29, 13), (128, 512, 10), (256, 784, 256), (64, 2048, 96), (300, 64, 700),
                 (16, 4096, 64)]


@pytest.mark.parametrize("M,K,N", LINEAR_SHAPES)
def test_linear_forward(dev, M, K, N):
    from triton_tagi_amd.kernels.common import fused_var_forward, linear_forward

    r = g(M * 131 + K * 7 + N)
    ma, Sa = torch.randn(M, K, generator=r), 0.01 + 0.09 * torch.rand(M, K, generator=r)
    mw, Sw = torch.randn(K, N, generator=r) / K**0.5, torch.rand(K, N, generator=r) / K
    mb, Sb = torch.randn(1, N, generator=r), 1e-3 * torch.rand(1, N, generator=r)
    mz, Sz = linear_forward(*(t.to(dev) for t in (ma, Sa, mw, Sw, mb, Sb)))
    rm, rS = O.linear_moments(*(d64(t) for t in (ma, Sa, mw, Sw, mb, Sb)))
    scale = d64(ma).abs() @ d64(mw).abs() + d64(mb).abs()
    assert_scaled_close(mz, rm, scale, RTOL, ATOL, "mz")
    assert_scaled_close(Sz, rS, None, RTOL, ATOL, "Sz")
    Sz2 = fused_var_forward(*(t.to(dev) for t in (ma, Sa, mw, Sw, Sb)))
    assert torch.equal(Sz2.cpu(), Sz.cpu())


@pytest.mark.parametrize("M,K,N", LINEAR_SHAPES)
def test_linear_backward_delta(dev, M, K, N):
    from triton_tagi_amd.kernels.common import fused_backward_delta

    r = g(M + 17 * K + 3 * N)
    dmz, dSz = torch.randn(M, N, generator=r), -torch.rand(M, N, generator=r)
    mw = torch.randn(K, N, generator=r) / K**0.5
    dma, dSa = fused_backward_delta(dmz.to(dev), dSz.to(dev), mw.to(dev))
    rm, rS = O.linear_backward_delta(d64(dmz), d64(dSz), d64(mw))
    assert_scaled_close(dma, rm, d64(dmz).abs() @ d64(mw).abs().T, RTOL, ATOL, "dma")
    assert_scaled_close(dSa, rS, None, RTOL, ATOL, "dSa")


@pytest.mark.parametrize("M,K,N", LINEAR_SHAPES + [(8192, 64, 32), (65536, 27, 16)])
def test_linear_param_deltas(dev, M, K, N):
    from triton_tagi_amd.kernels.common import fused_weight_grad, linear_param_deltas

    r = g(5 * M + K + 11 * N)
    a = torch.randn(M, K, generator=r)
    dmz, dSz = 0.1 * torch.randn(M, N, generator=r), -1e-2 * torch.rand(M, N, generator=r)
    Sw, Sb = torch.rand(K, N, generator=r) / K, torch.rand(1, N, generator=r) / K
    dmw, dSw, dmb, dSb = linear_param_deltas(a.to(dev), dmz.to(dev), dSz.to(dev), Sw.to(dev), Sb.to(dev))
    gmw, gmb, gSw, gSb = O.linear_param_grads(d64(a), d64(dmz), d64(dSz))
    S64, Sb64 = d64(Sw), d64(Sb)
    assert_scaled_close(dmw, S64 * gmw, S64 * (d64(a).abs().T @ d64(dmz).abs()), RTOL, ATOL, "delta_mw")
    assert_scaled_close(dSw, S64 * S64 * gSw, None, RTOL, ATOL, "delta_Sw")
    assert_scaled_close(dmb, Sb64 * gmb, Sb64 * d64(dmz).abs().sum(0, keepdim=True), RTOL, ATOL, "delta_mb")
    assert_scaled_close(dSb, Sb64 * Sb64 * gSb, None, RTOL, ATOL, "delta_Sb")
    raw_m, raw_S = fused_weight_grad(a.to(dev), dmz.to(dev), dSz.to(dev))
    assert_scaled_close(raw_m, gmw, d64(a).abs().T @ d64(dmz).abs(), RTOL, ATOL, "raw grad mw")
    assert_scaled_close(raw_S, gSw, None, RTOL, ATOL, "raw grad Sw")


@pytest.mark.parametrize("M,K,N,bias,offset", [(256, 4096, 1100, True, 0), (64, 96, 80, True, 0), (8192, 64, 32, False, 0),
                                                (300, 77, 45, True, 1), (5, 3, 7, False, 0)])
def test_linear_param_deltas_update(dev, M, K, N, bias, offset):
    """tagi_linear_wgrad_update (the capped update applied by the kernel that forms the
    parameter deltas) against tagi_linear_wgrad followed by tagi_capped_update: the same
    deltas and the same updated parameters, bit for bit. Split-K (a long reduction) and
    unsplit plans, with and without the bias, and an input offset by one float (scalar
    loaders)."""
    from triton_tagi_amd.kernels.common import linear_param_deltas, linear_param_deltas_update
    from triton_tagi_amd.update.parameters import update_parameters

    r = g(3 * M + 7 * K + N + offset)
    a_buf = torch.randn(M * K + offset, generator=r)
    a = a_buf[offset:].view(M, K)
    dmz, dSz = 0.1 * torch.randn(M, N, generator=r), -1e-2 * torch.rand(M, N, generator=r)
    mw, Sw = torch.randn(K, N, generator=r) / K ** 0.5, torch.rand(K, N, generator=r) / K
    mb, Sb = torch.randn(1, N, generator=r) * 0.1, torch.rand(1, N, generator=r) * 1e-3
    Sw[0, :4] = torch.tensor([1e-12, 1e-6, 2.0, 0.0])  # caps at the 1e-10 floor and wide ones
    a_d = a_buf.to(dev)[offset:].view(M, K)  # offset 1: not 16-byte aligned on the device
    dmz_d, dSz_d = dmz.to(dev), dSz.to(dev)
    cap = 2.0
    ref = [t.to(dev) for t in (mw, Sw, mb, Sb)]
    rdmw, rdSw, rdmb, rdSb = linear_param_deltas(a_d, dmz_d, dSz_d, ref[1], ref[3] if bias else None)
    update_parameters(ref[0], ref[1], rdmw, rdSw, cap)
    if bias:
        update_parameters(ref[2], ref[3], rdmb, rdSb, cap)
    got = [t.to(dev) for t in (mw, Sw, mb, Sb)]
    dmw, dSw, dmb, dSb = linear_param_deltas_update(a_d, dmz_d, dSz_d, got[0], got[1], got[2] if bias else None,
                                                    got[3] if bias else None, cap)
    torch.cuda.synchronize()
    assert torch.equal(dmw, rdmw) and torch.equal(dSw, rdSw), "weight deltas differ"
    assert torch.equal(got[0], ref[0]) and torch.equal(got[1], ref[1]), "updated weights differ"
    if bias:
        assert torch.equal(dmb, rdmb) and torch.equal(dSb, rdSb), "bias deltas differ"
        assert torch.equal(got[2], ref[2]) and torch.equal(got[3], ref[3]), "updated bias differs"
    else:
        assert dmb is None and torch.equal(got[2], mb.to(dev)) and torch.equal(got[3], Sb.to(dev))
    # the update itself against the oracle's capped rule on the deltas
    um, uS = O.capped_update(d64(mw), d64(Sw), d64(dmw), d64(dSw), cap)
    assert_scaled_close(got[0], um, None, RTOL, ATOL, "updated mw")
    assert_scaled_close(got[1], uS, None, RTOL, ATOL, "updated Sw")


def test_relu(dev):
    from triton_tagi_amd.layers.relu import bayesian_relu

    r = g(3)
    mz = 3 * torch.randn(1000, 37, generator=r)
    Sz = torch.rand(1000, 37, generator=r) * 2 + 1e-4
    mz[0, :8] = torch.tensor([-20.0, -6.0, -5.01, -4.99, 0.0, 5.0, 40.0, -1e-3])
    Sz[0, :8] = torch.tensor([1.0, 1.0, 1.0, 1.0, 1e-8, 1e-6, 1.0, 1e-2])
    ma, Sa, J = bayesian_relu(mz.to(dev), Sz.to(dev))
    rm, rS, rJ = O.relu_moments(d64(mz), d64(Sz))
    assert_scaled_close(ma, rm, None, RTOL, ATOL, "relu mean")
    assert_scaled_close(Sa, rS, None, RTOL, ATOL, "relu var")
    assert_scaled_close(J, rJ, None, RTOL, ATOL, "relu J")


@pytest.mark.parametrize("B,K", [(128, 10), (7, 1), (4096, 64), (300, 77), (512, 256), (3, 1000)])
def test_remax(dev, B, K):
    from triton_tagi_amd.layers.remax import remax

    r = g(B * 7 + K)
    mz = torch.randn(B, K, generator=r)
    Sz = 0.05 + torch.rand(B, K, generator=r)
    ma, Sa, J = remax(mz.to(dev), Sz.to(dev))
    rm, rS, rJ = O.remax_moments(d64(mz), d64(Sz))
    assert_scaled_close(ma, rm, None, RTOL, ATOL, "remax mean")
    assert_scaled_close(Sa, rS, None, RTOL, ATOL, "remax var")
    assert_scaled_close(J, rJ, None, RTOL, ATOL, "remax J")


@pytest.mark.parametrize("B,K", [(256, 256), (64, 10)])
def test_remax_wide_range(dev, B, K):
    """Remax where the rectified means span the normal tails: |mz|/sqrt(Sz) up to about
    60, variances over four decades (both sides of the 1e-6 floors)."""
    from triton_tagi_amd.layers.remax import remax

    r = g(B + 3 * K)
    mz = 6.0 * torch.randn(B, K, generator=r)
    Sz = 10.0 ** (4.0 * torch.rand(B, K, generator=r) - 3.0)
    mz[0, :6] = torch.tensor([-30.0, -8.0, -4.0, 0.0, 4.0, 30.0])
    ma, Sa, J = remax(mz.to(dev), Sz.to(dev))
    rm, rS, rJ = O.remax_moments(d64(mz), d64(Sz))
    assert_scaled_close(ma, rm, None, RTOL, ATOL, "remax mean")
    assert_scaled_close(Sa, rS, None, RTOL, ATOL, "remax var")
    assert_scaled_close(J, rJ, None, RTOL, ATOL, "remax J")


@pytest.mark.parametrize("B,K", [(64, 256), (512, 10)])
def test_remax_negative_scores_near_the_variance_floor(dev, B, K):
    """Remax where most scores sit at mz / sqrt(Sz) between about -5 and -2.5 (attention
    rows far below their maximum): there the mixture moments' two terms cancel (the mean
    by ~x^2, the variance by ~x^4 at x = -alpha), and their rectified variances sit just
    above the 1e-6 floor, so the Jacobian is as sensitive as the fp32 evaluation gets.
    Seeded rows of this kind took the Jacobian to 2x the bound when the density and the
    tail were rounded independently; the mixture moments are now formed from the Mills
    ratio (remax.py:59-109; the cancellation-free forms are in tagi_moments.h)."""
    from triton_tagi_amd.layers.remax import remax

    r = g(5 + B + K)
    mz = -1.5 + 0.35 * torch.randn(B, K, generator=r)
    Sz = 0.08 + 0.14 * torch.rand(B, K, generator=r)
    mz[:, 0] += 3.0  # one larger score per row
    ma, Sa, J = remax(mz.to(dev), Sz.to(dev))
    rm, rS, rJ = O.remax_moments(d64(mz), d64(Sz))
    assert_scaled_close(ma, rm, None, RTOL, ATOL, "remax mean")
    assert_scaled_close(Sa, rS, None, RTOL, ATOL, "remax var")
    assert_scaled_close(J, rJ, None, RTOL, ATOL, "remax J")


def test_remax_on_reference_golden_inputs(dev):
    """HIP Remax on the inputs of the reference-generated fixture: within 1e-4 of the
    float64 oracle, and within the reference's own fp32 rounding of its stored outputs."""
    from pathlib import Path

    import numpy as np

    from triton_tagi_amd.layers.remax import remax

    d = np.load(Path(__file__).resolve().parent / "golden" / "remax_golden.npz")
    names = sorted({k[: -len("_mu_z")] for k in d.files if k.endswith("_mu_z")})
    for n in names:
        mu, var = torch.tensor(d[n + "_mu_z"]), torch.tensor(d[n + "_var_z"])
        got = remax(mu.to(dev), var.to(dev))
        ref64 = O.remax_moments(d64(mu), d64(var))
        for key, gt, rt in zip(("mu_a", "var_a", "J"), got, ref64):
            assert_scaled_close(gt, rt, None, RTOL, ATOL, f"remax {n} {key} vs oracle")
            stored = torch.tensor(d[f"{n}_{key}"], dtype=torch.float64)
            rel = ((gt.cpu().double() - stored).norm() / stored.norm()).item()
            # the oracle itself sits 1.2e-6 (mean) and 2.4e-4 / 3.0e-4 (variance, J) from these
            # outputs in the 2-norm (the reference's fp32 rounding)
            assert rel < (1e-5 if key == "mu_a" else 1e-3), f"remax {n} {key}: {rel:.2e} from the reference output"


def update_multi_many_groups_with_empty_ones(dev, r):
    """The C entry point directly (the Python wrapper drops empty groups): 50 groups, more
    than one launch holds, with empty groups first and in between. Every non-empty group
    must be updated exactly once (a second application would move it twice)."""
    import ctypes

    from triton_tagi_amd import _lib

    sizes = [0] + [int(n) for n in torch.randint(1, 9000, (49,), generator=r)]
    sizes[7] = sizes[30] = 0
    groups, refs = [], []
    for n in sizes:
        m, S = torch.randn(n, generator=r), 1e-3 + torch.rand(n, generator=r) * 1e-2
        ddm, ddS = torch.randn(n, generator=r) * 0.05, torch.randn(n, generator=r) * 1e-2
        groups.append(tuple(t.to(dev) for t in (m, S, ddm, ddS)))
        refs.append(O.capped_update(d64(m), d64(S), d64(ddm), d64(ddS), 2.0))
    k = len(groups)
    tab = [(ctypes.c_void_p * k)(*[grp[j].data_ptr() for grp in groups]) for j in range(4)]
    pn = (ctypes.c_int64 * k)(*sizes)
    _lib.call("tagi_capped_update_multi", *(ctypes.addressof(t) for t in tab), ctypes.addressof(pn), k, 2.0,
              torch.cuda.current_stream(dev).cuda_stream)
    for j, ((mg, Sg, _, _), (rm, rS)) in enumerate(zip(groups, refs)):
        assert_scaled_close(mg, rm, None, RTOL, ATOL, f"50-group update m, group {j} (n={sizes[j]})")
        assert_scaled_close(Sg, rS, None, RTOL, ATOL, f"50-group update S, group {j} (n={sizes[j]})")


def test_innovation_update_add_jacobian(dev):
    from triton_tagi_amd.layers.relu import jacobian_backward
    from triton_tagi_amd.layers.resblock import add_shortcut
    from triton_tagi_amd.update.observation import compute_innovation
    from triton_tagi_amd.update.parameters import update_parameters, update_parameters_multi

    r = g(9)
    y, mu, var = torch.randn(257, 13, generator=r), torch.randn(257, 13, generator=r), torch.rand(257, 13, generator=r)
    dm, dS = compute_innovation(y.to(dev), mu.to(dev), var.to(dev), 0.05)
    rdm, rdS = O.innovation(d64(y), d64(mu), d64(var), 0.05)
    assert_scaled_close(dm, rdm, None, RTOL, ATOL, "innovation dm")
    assert_scaled_close(dS, rdS, None, RTOL, ATOL, "innovation dS")

    for n in (1, 5, 4096, 100003):
        m, S = torch.randn(n, generator=r), torch.rand(n, generator=r) * 1e-2
        S[: min(n, 3)] = torch.tensor([1e-12, 1e-4, 0.5])[: min(n, 3)]
        ddm = torch.randn(n, generator=r) * 0.1
        ddS = torch.randn(n, generator=r) * 1e-2
        ddm[0], ddS[0] = 0.0, -1.0  # zero mean delta, variance pushed below zero
        mg, Sg = m.to(dev), S.to(dev)
        update_parameters(mg, Sg, ddm.to(dev), ddS.to(dev), 2.0)
        rm, rS = O.capped_update(d64(m), d64(S), d64(ddm), d64(ddS), 2.0)
        assert_scaled_close(mg, rm, None, RTOL, ATOL, f"update m n={n}")
        assert_scaled_close(Sg, rS, None, RTOL, ATOL, f"update S n={n}")

    groups, refs = [], []
    for n, offset in ((3, 0), (4096 * 3 + 1, 0), (17, 0), (70000, 0), (9001, 1), (4099, 2)):
        # offset > 0: the tensors are views starting off a 16-byte boundary (scalar path)
        m, S = torch.randn(n, generator=r), 1e-3 + torch.rand(n, generator=r) * 1e-2
        ddm, ddS = torch.randn(n, generator=r) * 0.05, torch.randn(n, generator=r) * 1e-2
        groups.append(tuple(torch.cat([torch.zeros(offset), t]).to(dev)[offset:] for t in (m, S, ddm, ddS)))
        refs.append(O.capped_update(d64(m), d64(S), d64(ddm), d64(ddS), 3.0))
    update_parameters_multi(groups, 3.0)
    for (mg, Sg, _, _), (rm, rS) in zip(groups, refs):
        assert_scaled_close(mg, rm, None, RTOL, ATOL, "multi update m")
        assert_scaled_close(Sg, rS, None, RTOL, ATOL, "multi update S")

    update_multi_many_groups_with_empty_ones(dev, r)

    a, b, c, d = (torch.randn(1001, generator=r) for _ in range(4))
    ag, bg = a.to(dev), b.to(dev)
    add_shortcut(c.to(dev), d.to(dev), ag, bg)
    assert torch.equal(ag.cpu(), a + c) and torch.equal(bg.cpu(), b + d)

    J = torch.rand(333, generator=r)
    om, oS = jacobian_backward(a[:333].to(dev), b[:333].to(dev), J.to(dev))
    assert_scaled_close(om, d64(a[:333]) * d64(J), None, RTOL, ATOL, "jacobian mean")
    assert_scaled_close(oS, d64(b[:333]) * d64(J) ** 2, None, RTOL, ATOL, "jacobian var")


# C = 8: float4 along the channels; 13 x 13 with k = 2 or 3: a partial last window row
# and column, whose input positions receive zero deltas
@pytest.mark.parametrize("k,sc,C,HW", [(2, False, 5, 12), (4, False, 5, 12), (2, True, 5, 12), (3, False, 5, 12),
                                       (2, False, 8, 12), (2, True, 8, 13), (3, False, 8, 13), (3, False, 5, 13)])
def test_avgpool(dev, k, sc, C, HW):
    from triton_tagi_amd.layers.avgpool2d import AvgPool2D

    r = g(k + C + HW)
    ma, Sa = torch.randn(3, C, HW, HW, generator=r), torch.rand(3, C, HW, HW, generator=r)
    layer, ref = AvgPool2D(k, sc), O.OAvgPool2D(k, sc)
    mo, So = layer.forward(ma.to(dev), Sa.to(dev))
    rm, rS = ref.forward(d64(ma), d64(Sa))
    assert_scaled_close(mo, rm, d64(ma).abs().mean() * torch.ones_like(rm), RTOL, ATOL, "pool mean")
    assert_scaled_close(So, rS, None, RTOL, ATOL, "pool var")
    dm, dS = torch.randn(rm.shape, generator=r), torch.rand(rm.shape, generator=r)
    om, oS = layer.backward(dm.to(dev), dS.to(dev))
    qm, qS = ref.backward(d64(dm), d64(dS))
    assert_scaled_close(om, qm, None, RTOL, ATOL, "pool bwd mean")
    assert_scaled_close(oS, qS, None, RTOL, ATOL, "pool bwd var")


CONV_CASES = [
    # N, C, H, W, Cout, k, stride, padding, padding_type
    (2, 3, 8, 8, 5, 3, 1, 1, 1),
    (2, 3, 32, 32, 32, 5, 1, 2, 1),
    (3, 4, 9, 7, 6, 3, 2, 1, 2),
    (2, 8, 16, 16, 16, 3, 2, 1, 2),
    (2, 8, 16, 16, 16, 2, 2, 0, 1),
    (1, 16, 8, 8, 32, 3, 1, 1, 1),
    (4, 64, 8, 8, 128, 3, 2, 1, 2),
    (2, 5, 11, 11, 7, 4, 3, 2, 1),
    (2, 4, 9, 9, 8, 1, 2, 0, 1),      # 1x1 stride 2: odd pixels get no taps
    (2, 8, 10, 7, 12, 2, 3, 1, 1),    # kernel smaller than the stride, uneven sizes
    (128, 3, 32, 32, 64, 3, 1, 1, 1),  # ResNet-18 stem at full batch
    (2, 1, 9, 9, 6, 3, 1, 1, 1),      # one and two input channels
    (3, 2, 10, 10, 5, 5, 2, 2, 1),
]


@pytest.mark.parametrize("case", CONV_CASES, ids=[str(c) for c in CONV_CASES])
def test_conv2d_forward_backward(dev, case):
    from triton_tagi_amd.layers.conv2d import Conv2D

    N, C, H, W, Cout, k, s, p, pt = case
    torch.manual_seed(sum(case))
    layer = Conv2D(C, Cout, k, stride=s, padding=p, padding_type=pt, device="cpu")
    ref = O.mirror(layer)
    for a in ("mw", "Sw", "mb", "Sb"):
        setattr(layer, a, getattr(layer, a).to(dev))
    r = g(sum(case) + 1)
    ma, Sa = torch.randn(N, C, H, W, generator=r), torch.rand(N, C, H, W, generator=r)
    mz, Sz = layer.forward(ma.to(dev), Sa.to(dev))
    rm, rS = ref.forward(d64(ma), d64(Sa))
    P = ref.patches
    scale = (P.abs() @ ref.mw.abs() + ref.mb.abs()).view(N, *ref.spatial, Cout).permute(0, 3, 1, 2)
    assert_scaled_close(mz, rm, scale, RTOL, ATOL, "conv mz")
    assert_scaled_close(Sz, rS, None, RTOL, ATOL, "conv Sz")
    dmz, dSz = 0.1 * torch.randn(rm.shape, generator=r), -1e-2 * torch.rand(rm.shape, generator=r)
    dma, dSa = layer.backward(dmz.to(dev), dSz.to(dev))
    qm, qS = ref.backward(d64(dmz), d64(dSz))
    dm_rows = d64(dmz).permute(0, 2, 3, 1).reshape(-1, Cout)
    sc_in = O.col2im(dm_rows.abs() @ ref.mw.abs().T, N, C, H, W, k, s, p, pt)
    assert_scaled_close(dma, qm, sc_in, RTOL, ATOL, "conv delta ma")
    assert_scaled_close(dSa, qS, None, RTOL, ATOL, "conv delta Sa")
    sc_w = ref.Sw * (P.abs().T @ dm_rows.abs())
    assert_scaled_close(layer.delta_mw, ref.delta_mw, sc_w, RTOL, ATOL, "conv delta mw")
    assert_scaled_close(layer.delta_Sw, ref.delta_Sw, None, RTOL, ATOL, "conv delta Sw")
    assert_scaled_close(layer.delta_mb, ref.delta_mb, ref.Sb * dm_rows.abs().sum(0, keepdim=True), RTOL, ATOL,
                        "conv delta mb")
    assert_scaled_close(layer.delta_Sb, ref.delta_Sb, None, RTOL, ATOL, "conv delta Sb")


@pytest.mark.parametrize("shape,first,preserve", [((4, 6, 5, 5), True, True), ((8, 64, 8, 8), True, False),
                                                  ((3, 5, 4, 4), False, False), ((128, 16, 4, 4), True, True)])
def test_batchnorm(dev, shape, first, preserve):
    from triton_tagi_amd.layers.batchnorm2d import BatchNorm2D

    N, C, H, W = shape
    torch.manual_seed(N + C)
    layer = BatchNorm2D(C, device="cpu", gain_w=0.3, gain_b=0.2, preserve_var=preserve)
    r = g(C)
    layer.mw = 1.0 + 0.1 * torch.randn(C, generator=r)
    if not first:
        layer._is_initialized = True
        layer.running_mean = torch.randn(C, generator=r)
        layer.running_var = torch.rand(C, generator=r) + 0.5
    ref = O.mirror(layer)
    for a in ("mw", "Sw", "mb", "Sb", "running_mean", "running_var"):
        setattr(layer, a, getattr(layer, a).to(dev))
    mz, Sz = 2 + torch.randn(shape, generator=r), torch.rand(shape, generator=r)
    ma, Sa = layer.forward(mz.to(dev), Sz.to(dev))
    rm, rS = ref.forward(d64(mz), d64(Sz))
    assert_scaled_close(layer.running_mean, ref.running_mean, None, RTOL, ATOL, "running mean")
    assert_scaled_close(layer.running_var, ref.running_var, None, RTOL, ATOL, "running var")
    assert_scaled_close(layer.mw, ref.mw, None, RTOL, ATOL, "gamma after first call")
    assert_scaled_close(ma, rm, rm.abs() + 1.0, RTOL, ATOL, "bn mean")
    assert_scaled_close(Sa, rS, None, RTOL, ATOL, "bn var")
    dma, dSa = torch.randn(shape, generator=r), -torch.rand(shape, generator=r)
    om, oS = layer.backward(dma.to(dev), dSa.to(dev))
    qm, qS = ref.backward(d64(dma), d64(dSa))
    assert_scaled_close(om, qm, None, RTOL, ATOL, "bn bwd mean")
    assert_scaled_close(oS, qS, None, RTOL, ATOL, "bn bwd var")
    mh = ref.m_hat
    assert_scaled_close(layer.delta_mw, ref.delta_mw, ref.Sw * (d64(dma) * mh).abs().sum((0, 2, 3)), RTOL, ATOL,
                        "bn delta gamma")
    assert_scaled_close(layer.delta_Sw, ref.delta_Sw, None, RTOL, ATOL, "bn delta Sgamma")
    assert_scaled_close(layer.delta_mb, ref.delta_mb, ref.Sb * d64(dma).abs().sum((0, 2, 3)), RTOL, ATOL,
                        "bn delta beta")
    assert_scaled_close(layer.delta_Sb, ref.delta_Sb, None, RTOL, ATOL, "bn delta Sbeta")


def test_rmsnorm_embedding_pe(dev):
    from triton_tagi_amd.layers import Embedding, PositionalEncoding, RMSNorm

    torch.manual_seed(4)
    r = g(4)
    rms = RMSNorm([96], device="cpu")
    rms.mw = 1 + 0.1 * torch.randn(96, generator=r)
    ref = O.mirror(rms)
    rms.mw, rms.Sw = rms.mw.to(dev), rms.Sw.to(dev)
    ma, Sa = torch.randn(5, 33, 96, generator=r), torch.rand(5, 33, 96, generator=r)
    mz, Sz = rms.forward(ma.to(dev), Sa.to(dev))
    rm, rS = ref.forward(d64(ma), d64(Sa))
    assert_scaled_close(mz, rm, None, RTOL, ATOL, "rms mean")
    assert_scaled_close(Sz, rS, None, RTOL, ATOL, "rms var")
    dm, dS = torch.randn(5, 33, 96, generator=r), -torch.rand(5, 33, 96, generator=r)
    om, oS = rms.backward(dm.to(dev), dS.to(dev))
    qm, qS = ref.backward(d64(dm), d64(dS))
    assert_scaled_close(om, qm, None, RTOL, ATOL, "rms bwd mean")
    assert_scaled_close(oS, qS, None, RTOL, ATOL, "rms bwd var")
    sc = (ref.inv * ref.m_in * d64(dm).reshape(-1, 96)).abs().sum(0) * ref.Sw
    assert_scaled_close(rms.delta_mw, ref.delta_mw, sc, RTOL, ATOL, "rms delta gamma")
    assert_scaled_close(rms.delta_Sw, ref.delta_Sw, None, RTOL, ATOL, "rms delta Sgamma")

    # (6, 300) tokens: one 16384-token window; (3, 6000): two windows; V = 64, D = 256: the
    # transformer block's table; D = 30: the scalar loads; D = 300: two 256-column groups
    for V, D, pad, T in ((17, 40, -1, (6, 300)), (17, 40, 3, (6, 300)), (64, 256, -1, (6, 300)),
                         (64, 256, 5, (6, 300)), (300, 24, 7, (6, 300)), (1100, 30, -1, (6, 300)),
                         (5, 300, 2, (6, 300)), (40, 64, 1, (3, 6000))):
        emb = Embedding(V, D, scale=0.25, padding_idx=pad, device="cpu")
        eref = O.mirror(emb)
        emb.mw, emb.Sw = emb.mw.to(dev), emb.Sw.to(dev)
        tok = torch.randint(0, V, T, generator=r).to(torch.float32)
        mz, Sz = emb.forward(tok.to(dev), torch.zeros_like(tok).to(dev))
        rm, rS = eref.forward(d64(tok), d64(tok) * 0)
        assert torch.equal(mz.cpu().double(), rm) and torch.equal(Sz.cpu().double(), rS)
        dm, dS = torch.randn(*T, D, generator=r), -torch.rand(*T, D, generator=r)
        zm, zS = emb.backward(dm.to(dev), dS.to(dev))
        eref.backward(d64(dm), d64(dS))
        assert float(zm.abs().sum()) == 0.0 and tuple(zm.shape) == T
        sc = torch.zeros(V, D, dtype=torch.float64).index_add_(
            0, tok.long().reshape(-1), (d64(dm).reshape(-1, D) * eref.Sw[tok.long().reshape(-1)]).abs())
        assert_scaled_close(emb.delta_mw, eref.delta_mw, sc, RTOL, ATOL, "emb delta mw")
        assert_scaled_close(emb.delta_Sw, eref.delta_Sw, None, RTOL, ATOL, "emb delta Sw")

    pe = PositionalEncoding(64, max_seq_len=512, device="cpu")
    pref = O.OPositionalEncoding(O.sinusoidal_table(512, 64))
    pe.pe_cache = pe.pe_cache.to(dev)
    ma = torch.randn(3, 200, 64, generator=r)
    out, _ = pe.forward(ma.to(dev), ma.to(dev))
    ro, _ = pref.forward(d64(ma), d64(ma))
    assert_scaled_close(out, ro, d64(ma).abs() + pref.pe[:200].abs(), RTOL, ATOL, "pe add")

    # the transformer block's table, built on the GPU, against the table the reference wrote
    from pathlib import Path

    import numpy as np

    gold = np.load(Path(__file__).resolve().parent / "golden" / "pe_golden.npz")
    pe_dev = PositionalEncoding(256, max_seq_len=2048, device=dev)
    rows = torch.tensor(gold["e256_rows"])
    assert_scaled_close(pe_dev.pe_cache[rows.to(dev)], torch.tensor(gold["e256"], dtype=torch.float64), None,
                        RTOL, ATOL, "PE table (GPU) vs the reference's")
    z = torch.zeros(2, 256, 256, device=dev)
    out, _ = pe_dev.forward(z, z)
    assert torch.equal(out[1].cpu(), pe_dev.pe_cache[:256].cpu())


@pytest.mark.parametrize("B,S,E,H", [(2, 16, 32, 2), (3, 40, 64, 8), (2, 256, 256, 8)])
def test_attention_layer(dev, B, S, E, H, monkeypatch):
    """MultiheadAttentionV2 forward and backward (fused kernels for head dimensions 16 and
    32, the two-call path for 8): every stage against the float64 oracle, teacher forced, at
    the per-element bar (teacher_forcing.check_attention); then the layer's outputs against
    the oracle's whole attention from the same input (a chain of stages: the Remax carries
    the score product's fp32 rounding into the outputs, held to 1e-3, the scores themselves
    to 1e-4; the worst ratio at the 1e-4 bar is printed)."""
    from teacher_forcing import Report, check_attention

    from triton_tagi_amd.layers import MultiheadAttentionV2
    from triton_tagi_amd.layers import multihead_attention as mha_mod

    torch.manual_seed(B + S)
    att = MultiheadAttentionV2(E, H, S, gain_weight=0.25, gain_bias=0.5, device="cpu")
    ref = O.mirror(att)
    for lin in (att.q_proj, att.k_proj, att.v_proj):
        for a in ("mw", "Sw", "mb", "Sb"):
            setattr(lin, a, getattr(lin, a).to(dev))
    seen = {}
    orig_fwd, orig_bd = mha_mod.linear_forward, mha_mod.fused_backward_delta

    def lf(*a, **k):
        out = orig_fwd(*a, **k)
        seen["qkv"] = (out[0].clone(), out[1].clone())
        return out

    def bd(dmz, dSz, mw, add=None):
        seen["dqkv"] = (dmz.clone(), dSz.clone())
        return orig_bd(dmz, dSz, mw, add)

    monkeypatch.setattr(mha_mod, "linear_forward", lf)
    monkeypatch.setattr(mha_mod, "fused_backward_delta", bd)
    r = g(S)
    ma, Sa = torch.randn(B, S, E, generator=r), 0.1 * torch.rand(B, S, E, generator=r)
    mo, So = att.forward(ma.to(dev), Sa.to(dev))
    msc, vsc = att.get_attention_scores()
    jcb = att._cache["jcb"]
    dm, dS = 0.1 * torch.randn(B, S, E, generator=r), -1e-2 * torch.rand(B, S, E, generator=r)
    om, oS = att.backward(dm.to(dev), dS.to(dev))
    torch.cuda.synchronize()
    monkeypatch.undo()
    projs = (ref.q, ref.k, ref.v)
    rep = Report()
    check_attention(rep, f"B{B} S{S} E{E} H{H}", dict(
        H=H, ma=ma, Sa=Sa, w_m=torch.cat([p.mw for p in projs], 1), w_S=torch.cat([p.Sw for p in projs], 1),
        qkv_m=seen["qkv"][0], qkv_S=seen["qkv"][1], mu_a=msc, var_a=vsc, J=jcb, out_m=mo, out_S=So, d_m=dm, d_S=dS,
        dqkv_m=seen["dqkv"][0], dqkv_S=seen["dqkv"][1], dma=om, dSa=oS,
        pd=[(p.delta_mw, p.delta_Sw) for p in (att.q_proj, att.k_proj, att.v_proj)], Sw_qkv=[p.Sw for p in projs]))
    rep.finish()
    # the chain, end to end
    rm, rS = ref.forward(d64(ma), d64(Sa))
    qm, qS = ref.backward(d64(dm), d64(dS))
    chain = Report()
    chain.check("scores mean", msc, ref.attn[0])
    chain.check("scores var", vsc, ref.attn[1])
    chain.check("out mean", mo, rm, rm.abs() + rm.abs().mean())
    chain.check("out var", So, rS)
    chain.check("bwd mean", om, qm, qm.abs() + qm.abs().mean())
    chain.check("bwd var", oS, qS, qS.abs() + qS.abs().mean())
    for name in ("q_proj", "k_proj", "v_proj"):
        gl, rl = getattr(att, name), getattr(ref, name[0])
        chain.check(f"{name} delta mw", gl.delta_mw, rl.delta_mw, rl.delta_mw.abs() + rl.delta_mw.abs().mean())
        chain.check(f"{name} delta Sw", gl.delta_Sw, rl.delta_Sw, rl.delta_Sw.abs() + rl.delta_Sw.abs().mean())
    print("\nend to end, ratio to the 1e-4 bar (the chain is held to 1e-3, i.e. ratio <= 10):")
    for tag, worst, *_ in chain.rows:
        print(f"  {tag:<18} {worst:9.3e}")
    # the scores are one product of the inputs' projections: they keep the 1e-4 bar
    bad = [t for t in chain.rows if t[1] > (1.0 if t[0].startswith("scores") else 10.0)]
    assert not bad, f"end-to-end attention out of tolerance: {[(t[0], t[1]) for t in bad]}"


@pytest.mark.parametrize("B,H,S,D", [(2, 8, 256, 32), (1, 2, 40, 16), (2, 2, 100, 64), (1, 3, 1, 32)])
def test_attention_scores_remax_fused_equals_two_calls(dev, B, H, S, D):
    """tagi_attn_scores_remax (scores and Remax in one kernel) gives the outputs of
    tagi_bmm_tagi followed by tagi_remax_fwd bit for bit (same product order, same row
    math); the oracle comparison of both paths is test_attention_layer's."""
    import math

    from triton_tagi_amd import _lib
    from triton_tagi_amd.layers.remax import remax

    r = g(B * S + D)
    E = H * D
    mq, mk = (torch.randn(B, S, E, generator=r).to(dev) for _ in range(2))
    vq, vk = (0.1 * torch.rand(B, S, E, generator=r).to(dev) for _ in range(2))
    sc = 1.0 / math.sqrt(D)
    st = _lib.stream_of(mq)
    mu_qk, var_qk = torch.empty(B, H, S, S, device=dev), torch.empty(B, H, S, S, device=dev)
    _lib.call("tagi_bmm_tagi", mq.data_ptr(), vq.data_ptr(), mk.data_ptr(), vk.data_ptr(), mu_qk.data_ptr(),
              var_qk.data_ptr(), B * H, S, D, S, _lib.view(H, S * E, D, E, 1), _lib.view(H, S * E, D, 1, E),
              _lib.view(1, S * S, 0, S, 1), sc, sc * sc, st)
    ra, rv, rj = remax(mu_qk.view(-1, S), var_qk.view(-1, S))
    fa, fv, fj = (torch.empty(B, H, S, S, device=dev) for _ in range(3))
    _lib.call("tagi_attn_scores_remax", mq.data_ptr(), vq.data_ptr(), mk.data_ptr(), vk.data_ptr(), E,
              fa.data_ptr(), fv.data_ptr(), fj.data_ptr(), B, H, S, D, sc, sc * sc, st)
    for name, got, ref in (("mu_a", fa, ra), ("var_a", fv, rv), ("J", fj, rj)):
        assert torch.equal(got.view(-1, S), ref), f"{name}: fused differs from the two calls"


@pytest.mark.parametrize("B,H,S,D", [(2, 8, 256, 32), (1, 2, 40, 16), (2, 2, 100, 32), (1, 3, 1, 32),
                                     (1, 4, 250, 16)])
def test_attention_fwd_fused(dev, B, H, S, D):
    """tagi_attn_fwd (scores, Remax and score @ V in one kernel) on Q/K/V read from one
    (B*S, 3E) buffer: mu_a, var_a and J equal tagi_attn_scores_remax's bit for bit, with or
    without var_a requested; the output equals tagi_bmm_tagi's score @ V on those scores to
    1e-5 of the sum of its terms' magnitudes (the sum over keys runs per 32-key stretch, then
    over the stretches)."""
    import math

    from triton_tagi_amd import _lib

    r = g(11 * S + D + H)
    E = H * D
    L = 3 * E
    qkv_m = torch.randn(B * S, L, generator=r).to(dev)
    qkv_S = (0.1 * torch.rand(B * S, L, generator=r) + 0.01).to(dev)
    q_m, q_S = qkv_m.data_ptr(), qkv_S.data_ptr()
    k_m, k_S, v_m, v_S = q_m + 4 * E, q_S + 4 * E, q_m + 8 * E, q_S + 8 * E
    sc = 1.0 / math.sqrt(D)
    st = _lib.stream_of(qkv_m)
    ra, rv, rj = (torch.empty(B, H, S, S, device=dev) for _ in range(3))
    _lib.call("tagi_attn_scores_remax", q_m, q_S, k_m, k_S, L, ra.data_ptr(), rv.data_ptr(), rj.data_ptr(), B, H, S,
              D, sc, sc * sc, st)
    rm, rS = torch.empty(B, S, E, device=dev), torch.empty(B, S, E, device=dev)
    hL = _lib.view(H, S * L, D, L, 1)
    _lib.call("tagi_bmm_tagi", ra.data_ptr(), rv.data_ptr(), v_m, v_S, rm.data_ptr(), rS.data_ptr(), B * H, S, S, D,
              _lib.view(1, S * S, 0, S, 1), hL, _lib.view(H, S * E, D, E, 1), 1.0, 1.0, st)
    outs = []
    for keep_var in (True, False):
        fa, fv, fj = (torch.full((B, H, S, S), 7.0, device=dev) for _ in range(3))
        fm, fS = torch.empty(B, S, E, device=dev), torch.empty(B, S, E, device=dev)
        _lib.call("tagi_attn_fwd", q_m, q_S, k_m, k_S, v_m, v_S, L, fa.data_ptr(), fv.data_ptr() if keep_var else None,
                  fj.data_ptr(), fm.data_ptr(), fS.data_ptr(), E, B, H, S, D, sc, sc * sc, st)
        assert torch.equal(fa, ra) and torch.equal(fj, rj), "mu_a / J differ from tagi_attn_scores_remax"
        if keep_var:
            assert torch.equal(fv, rv), "var_a differs from tagi_attn_scores_remax"
        else:
            assert bool((fv == 7.0).all()), "var_a written although not requested"
        outs.append((fm, fS))
    assert torch.equal(outs[0][0], outs[1][0]) and torch.equal(outs[0][1], outs[1][1])
    fm, fS = outs[0]
    vm = qkv_m[:, 2 * E:].reshape(B, S, H, D).permute(0, 2, 1, 3).contiguous()
    tm = torch.matmul(ra.abs(), vm.abs()).permute(0, 2, 1, 3).reshape(B, S, E)
    assert_scaled_close(fm, rm, tm, 1e-5, 1e-7, "out mean")
    assert_scaled_close(fS, rS, rS, 1e-5, 1e-7, "out var")


def test_attention_scores_rebuilt_after_fused_forward(dev):
    """The fused attention forward keeps only the score means; get_attention_scores rebuilds
    the variances with tagi_attn_scores_remax from the kept projections. Both halves must be
    the values that kernel forms from those projections, bit for bit."""
    import math

    from triton_tagi_amd import _lib
    from triton_tagi_amd.layers import MultiheadAttentionV2

    torch.manual_seed(3)
    B, S, E, H = 2, 256, 256, 8
    att = MultiheadAttentionV2(E, H, S, device=dev)
    r = g(3)
    ma, Sa = torch.randn(B, S, E, generator=r).to(dev), (0.1 * torch.rand(B, S, E, generator=r)).to(dev)
    att.forward(ma, Sa)
    qkv_m, qkv_S, _, _ = att._attn_src
    msc, vsc = att.get_attention_scores()
    D = E // H
    sc = 1.0 / math.sqrt(D)
    rm, rv, rj = (torch.empty(B, H, S, S, device=dev) for _ in range(3))
    q_m, q_S = qkv_m.data_ptr(), qkv_S.data_ptr()
    _lib.call("tagi_attn_scores_remax", q_m, q_S, q_m + 4 * E, q_S + 4 * E, 3 * E, rm.data_ptr(), rv.data_ptr(),
              rj.data_ptr(), B, H, S, D, sc, sc * sc, _lib.stream_of(qkv_m))
    assert torch.equal(msc, rm) and torch.equal(vsc, rv)
    assert torch.equal(att._cache["jcb"], rj)


@pytest.mark.parametrize("B,H,S,D", [(2, 8, 256, 32), (1, 2, 40, 16), (2, 2, 100, 32), (1, 3, 1, 32)])
def test_attention_score_deltas_qk_fused(dev, B, H, S, D):
    """tagi_attn_score_deltas_qk (the Jacobian-scaled score deltas formed per block in LDS,
    then the dQ / dK product) against tagi_bmm_shared_jacobian followed by tagi_bmm_shared
    on the materialised scaled deltas: the same terms summed in a different grouping (the
    reduction over the S scores is split over 8 waves), so each output is held to 1e-5 of
    the sum of its terms' magnitudes."""
    import math

    from triton_tagi_amd import _lib

    r = g(7 * S + D + H)
    E = H * D
    dmu, mv, mq, mk = (torch.randn(B, S, E, generator=r).to(dev) for _ in range(4))
    dvar = -torch.rand(B, S, E, generator=r).to(dev)
    J = torch.rand(B, H, S, S, generator=r).to(dev)
    sc = 1.0 / math.sqrt(D)
    st = _lib.stream_of(dmu)
    hv, hvt = _lib.view(H, S * E, D, E, 1), _lib.view(H, S * E, D, 1, E)
    sv, svt = _lib.view(1, S * S, 0, S, 1), _lib.view(1, S * S, 0, 1, S)
    smu, svar = torch.empty(B, H, S, S, device=dev), torch.empty(B, H, S, S, device=dev)
    _lib.call("tagi_bmm_shared_jacobian", dmu.data_ptr(), dvar.data_ptr(), mv.data_ptr(), J.data_ptr(),
              smu.data_ptr(), svar.data_ptr(), B * H, S, D, S, hv, hvt, sv, 1.0, 1.0, 0, st)
    for x, view, tr, name in ((mk, sv, 0, "dQ"), (mq, svt, 1, "dK")):
        rm, rS = torch.empty(B, S, E, device=dev), torch.empty(B, S, E, device=dev)
        _lib.call("tagi_bmm_shared", smu.data_ptr(), svar.data_ptr(), x.data_ptr(), rm.data_ptr(), rS.data_ptr(),
                  B * H, S, S, D, view, hv, hv, sc, sc * sc, 0, st)
        fm, fS = torch.empty(B, S, E, device=dev), torch.empty(B, S, E, device=dev)
        _lib.call("tagi_attn_score_deltas_qk", dmu.data_ptr(), dvar.data_ptr(), E, mv.data_ptr(), x.data_ptr(), E,
                  J.data_ptr(), fm.data_ptr(), fS.data_ptr(), E, B, H, S, D, sc, sc * sc, tr, st)
        # term magnitudes: |scaled| @ |x| per head (the scaled deltas as the two-call path holds them)
        a_m, a_S = smu.abs(), svar.abs()
        if tr:
            a_m, a_S = a_m.transpose(-1, -2), a_S.transpose(-1, -2)
        xh = x.view(B, S, H, D).permute(0, 2, 1, 3).contiguous()
        tm = sc * torch.matmul(a_m.contiguous(), xh.abs()).permute(0, 2, 1, 3).reshape(B, S, E)
        tS = sc * sc * torch.matmul(a_S.contiguous(), xh * xh).permute(0, 2, 1, 3).reshape(B, S, E)
        assert_scaled_close(fm, rm, tm, 1e-5, 1e-7, f"{name} mean")
        assert_scaled_close(fS, rS, tS, 1e-5, 1e-7, f"{name} var")


@pytest.mark.parametrize("B,H,S,D", [(2, 8, 256, 32), (1, 2, 40, 16), (1, 4, 250, 16), (2, 2, 100, 32),
                                     (1, 3, 1, 32), (3, 1, 33, 16)])
def test_attention_score_deltas_qk_joint(dev, B, H, S, D):
    """tagi_attn_score_deltas_qk_joint (one block per head: the scaled score deltas formed
    once per query block, feeding the query deltas and register-held key deltas) against
    tagi_attn_score_deltas_qk called twice. The query deltas are summed in the same order,
    so they are the same bits; the key deltas sum the query rows 32 at a time instead of 8
    waves' strided shares, so they are held to 1e-5 of the sum of their terms' magnitudes.
    The inputs sit in one (B*S, 3E) buffer, as the layer holds them, so the rows past S of
    the last head are the edge of the allocation."""
    import math

    from triton_tagi_amd import _lib

    r = g(11 * S + D + 5 * H)
    E = H * D
    L = 3 * E
    qkv = torch.randn(B * S, L, generator=r).to(dev)
    q, k, v = (qkv[:, i * E:(i + 1) * E] for i in range(3))
    dmu = torch.randn(B, S, E, generator=r).to(dev)
    dvar = -torch.rand(B, S, E, generator=r).to(dev)
    J = torch.rand(B, H, S, S, generator=r).to(dev)
    sc = 1.0 / math.sqrt(D)
    st = _lib.stream_of(dmu)
    ref = {}
    for x, tr, name in ((k, 0, "dQ"), (q, 1, "dK")):
        rm, rS = torch.empty(B, S, E, device=dev), torch.empty(B, S, E, device=dev)
        _lib.call("tagi_attn_score_deltas_qk", dmu.data_ptr(), dvar.data_ptr(), E, v.data_ptr(), x.data_ptr(), L,
                  J.data_ptr(), rm.data_ptr(), rS.data_ptr(), E, B, H, S, D, sc, sc * sc, tr, st)
        ref[name] = (rm, rS)
    # outputs in a strided (B*S, 3E) buffer too, with NaN canaries in the untouched columns
    out = torch.full((B * S, 2 * E + 8), float("nan"), device=dev)
    outS = torch.full_like(out, float("nan"))
    ld = out.shape[1]
    _lib.call("tagi_attn_score_deltas_qk_joint", dmu.data_ptr(), dvar.data_ptr(), E, v.data_ptr(), q.data_ptr(),
              k.data_ptr(), L, J.data_ptr(), out.data_ptr(), outS.data_ptr(), out[:, E:].data_ptr(),
              outS[:, E:].data_ptr(), ld, B, H, S, D, sc, sc * sc, st)
    torch.cuda.synchronize()
    assert torch.isnan(out[:, 2 * E:]).all() and torch.isnan(outS[:, 2 * E:]).all(), "wrote past the outputs"
    qm, qS = out[:, :E].reshape(B, S, E), outS[:, :E].reshape(B, S, E)
    km, kS = out[:, E:2 * E].reshape(B, S, E), outS[:, E:2 * E].reshape(B, S, E)
    assert torch.equal(qm, ref["dQ"][0]) and torch.equal(qS, ref["dQ"][1]), "query deltas differ from the dQ kernel"
    # key-delta term magnitudes: |scaled|^T @ |q| per head, from the materialised scaled deltas
    hv, hvt = _lib.view(H, S * E, D, E, 1), _lib.view(H, S * E, D, 1, E)
    sv = _lib.view(1, S * S, 0, S, 1)
    vc = v.contiguous()
    smu, svar = torch.empty(B, H, S, S, device=dev), torch.empty(B, H, S, S, device=dev)
    _lib.call("tagi_bmm_shared_jacobian", dmu.data_ptr(), dvar.data_ptr(), vc.data_ptr(), J.data_ptr(),
              smu.data_ptr(), svar.data_ptr(), B * H, S, D, S, hv, hvt, sv, 1.0, 1.0, 0, st)
    qh = q.reshape(B, S, H, D).permute(0, 2, 1, 3).contiguous()
    tm = sc * torch.matmul(smu.abs().transpose(-1, -2).contiguous(), qh.abs()).permute(0, 2, 1, 3).reshape(B, S, E)
    tS = sc * sc * torch.matmul(svar.abs().transpose(-1, -2).contiguous(), qh * qh).permute(0, 2, 1, 3).reshape(
        B, S, E)
    assert_scaled_close(km, ref["dK"][0], tm, 1e-5, 1e-7, "dK mean")
    assert_scaled_close(kS, ref["dK"][1], tS, 1e-5, 1e-7, "dK var")


@pytest.mark.parametrize("transpose_a,transpose_b", [(False, False), (True, False), (False, True), (True, True)])
def test_bmm_wrappers_strided(dev, transpose_a, transpose_b):
    from triton_tagi_amd.kernels.attention import bmm_shared_left, bmm_shared_right, bmm_tagi, bmm_tagi_var

    r = g(int(transpose_a) * 2 + int(transpose_b))
    B, H, M, K, L = 2, 3, 33, 20, 45

    def mk(shape, t):
        x = torch.randn(*shape, generator=r)
        return x.transpose(-1, -2).contiguous().transpose(-1, -2) if t else x

    ma, va = mk((B, H, M, K), transpose_a), mk((B, H, M, K), transpose_a).abs()
    mb, vb = mk((B, H, K, L), transpose_b), mk((B, H, K, L), transpose_b).abs()
    if transpose_a:
        va = va.transpose(-1, -2).contiguous().transpose(-1, -2)
    if transpose_b:
        vb = vb.transpose(-1, -2).contiguous().transpose(-1, -2)
    mean, var = bmm_tagi(ma.to(dev), va.to(dev), mb.to(dev), vb.to(dev), scale=0.7)
    rm, rv = O.bmm_tagi(d64(ma), d64(va), d64(mb), d64(vb), 0.7)
    assert_scaled_close(mean, rm, 0.7 * d64(ma).abs() @ d64(mb).abs(), RTOL, ATOL, "bmm mean")
    assert_scaled_close(var, rv, None, RTOL, ATOL, "bmm var")
    v2 = bmm_tagi_var(ma.to(dev), va.to(dev), mb.to(dev), vb.to(dev), scale_sq=0.49)
    assert_scaled_close(v2, rv, None, RTOL, ATOL, "bmm_tagi_var")
    m3, v3 = bmm_shared_right(ma.to(dev), va.to(dev), mb.to(dev), scale=0.5)
    rm3, rv3 = O.bmm_shared_right(d64(ma), d64(va), d64(mb), 0.5)
    assert_scaled_close(m3, rm3, 0.5 * d64(ma).abs() @ d64(mb).abs(), RTOL, ATOL, "shared right mean")
    assert_scaled_close(v3, rv3, None, RTOL, ATOL, "shared right var")
    m4, v4 = bmm_shared_left(ma.to(dev), mb.to(dev), vb.to(dev), scale=2.0)
    rm4, rv4 = O.bmm_shared_left(d64(ma), d64(mb), d64(vb), 2.0)
    assert_scaled_close(m4, rm4, 2.0 * d64(ma).abs() @ d64(mb).abs(), RTOL, ATOL, "shared left mean")
    assert_scaled_close(v4, rv4, None, RTOL, ATOL, "shared left var")


@pytest.mark.parametrize("M,K,N", [(256, 784, 256), (128, 256, 10), (33, 70, 19), (4096, 512, 1024)])
def test_linear_forward_zero_variance_input(dev, M, K, N):
    """A deterministic input (Sa None, as Sequential passes the network input): the
    two-product kernel against the float64 oracle with zero input variance, and against
    the three-product kernel given explicit zeros (same terms; the plans may split the
    reduction differently, so within fp32 rounding)."""
    from triton_tagi_amd.kernels.common import linear_forward

    r = g(M + K + N)
    ma = torch.randn(M, K, generator=r)
    mw, Sw = torch.randn(K, N, generator=r) / K**0.5, torch.rand(K, N, generator=r) / K
    mb, Sb = torch.randn(1, N, generator=r), 1e-3 * torch.rand(1, N, generator=r)
    mz, Sz = linear_forward(ma.to(dev), None, *(t.to(dev) for t in (mw, Sw, mb, Sb)))
    rm, rS = O.linear_moments(d64(ma), torch.zeros(M, K, dtype=torch.float64), *(d64(t) for t in (mw, Sw, mb, Sb)))
    assert_scaled_close(mz, rm, d64(ma).abs() @ d64(mw).abs() + d64(mb).abs(), RTOL, ATOL, "mz")
    assert_scaled_close(Sz, rS, None, RTOL, ATOL, "Sz")
    zm, zS = linear_forward(ma.to(dev), torch.zeros(M, K, device=dev), *(t.to(dev) for t in (mw, Sw, mb, Sb)))
    assert_scaled_close(mz, d64(zm), d64(zm).abs() + 1.0, 1e-6, 1e-9, "mz vs explicit zeros")
    assert_scaled_close(Sz, d64(zS), None, 1e-6, 1e-12, "Sz vs explicit zeros")


@pytest.mark.parametrize("case", [(8, 3, 32, 32, 64, 3, 1, 1, 1), (4, 16, 12, 12, 32, 3, 1, 1, 1),
                                  (4, 8, 9, 9, 16, 5, 2, 2, 1), (128, 3, 32, 32, 64, 3, 1, 1, 1)])
def test_conv2d_forward_zero_variance_input(dev, case):
    """Conv2D forward on a deterministic input (Sa None): against the oracle with zero input
    variance and against the three-product kernel given explicit zeros; and the stem form
    that also forms the ReLU -> BatchNorm2D statistics (fused.conv_relu_bn_forward)."""
    from triton_tagi_amd.layers.batchnorm2d import BatchNorm2D
    from triton_tagi_amd.layers.conv2d import Conv2D
    from triton_tagi_amd.layers.fused import conv_relu_bn_forward
    from triton_tagi_amd.layers.relu import ReLU

    N, C, H, W, Cout, k, s, p, pt = case
    torch.manual_seed(sum(case) + 3)
    layer = Conv2D(C, Cout, k, stride=s, padding=p, padding_type=pt, device="cpu")
    ref = O.mirror(layer)
    for a in ("mw", "Sw", "mb", "Sb"):
        setattr(layer, a, getattr(layer, a).to(dev))
    ma = torch.randn(N, C, H, W, generator=g(sum(case)))
    mz, Sz = layer.forward(ma.to(dev), None)
    rm, rS = ref.forward(d64(ma), torch.zeros(N, C, H, W, dtype=torch.float64))
    scale = (ref.patches.abs() @ ref.mw.abs() + ref.mb.abs()).view(N, *ref.spatial, Cout).permute(0, 3, 1, 2)
    assert_scaled_close(mz, rm, scale, RTOL, ATOL, "conv mz")
    assert_scaled_close(Sz, rS, None, RTOL, ATOL, "conv Sz")
    zm, zS = layer.forward(ma.to(dev), torch.zeros(N, C, H, W, device=dev))
    assert_scaled_close(mz, d64(zm), d64(zm).abs() + 1.0, 1e-6, 1e-9, "mz vs explicit zeros")
    assert_scaled_close(Sz, d64(zS), None, 1e-6, 1e-12, "Sz vs explicit zeros")
    if s == 1:
        outs = []
        for Sa in (None, torch.zeros(N, C, H, W, device=dev)):
            bn = BatchNorm2D(Cout, device=dev)
            outs.append(conv_relu_bn_forward(layer, ReLU(), bn, ma.to(dev), Sa) + (bn.running_mean.clone(),))
        for j, (x, y) in enumerate(zip(*outs)):
            assert_scaled_close(x, d64(y), d64(y).abs() + 1.0, 1e-5, 1e-9, f"stem form output {j}")
