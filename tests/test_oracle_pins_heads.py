"""Pins of the oracle's output heads and further layers (CPU only).

Each function is checked against something that does not restate its formula:
  * HRC tree: the reference's own known answers (test_hrc_softmax.py), heap numbering for
    power-of-two class counts and a table worked out by hand for 10 classes;
  * sparse innovation: the (pinned) dense innovation at the selected nodes;
  * HRC class probabilities: Monte Carlo descent of the tree with noisy node signs, and
    the reference's known answers;
  * heteroscedastic innovation: numerical quadrature of the conditional V | Y = y and of
    V^2, Monte Carlo of Var[V^2], exact Gaussian conditioning for the gain step, and the
    reduction to the dense innovation for the mean outputs;
  * EvenSoftplus: second-order Taylor moments from autograd derivatives of softplus;
  * MaxPool2D: torch's max_pool2d_with_indices and brute-force delta routing;
  * LayerNorm: torch.var, Monte Carlo moments and the autograd delta rule;
  * engine host logic (tree tables, checkpoint format) against the same references.
Planted mistakes at the end confirm that the pins catch them.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F
from scipy import integrate

from oracle import tagi_oracle as O

D = torch.float64


def gen(seed):
    return torch.Generator().manual_seed(seed)


# ---------------------------------------------------------------------- HRC tree
HAND_10 = [[1, 2, 4, 7], [1, 2, 4, 7], [1, 2, 4, 8], [1, 2, 4, 8], [1, 2, 5, 9], [1, 2, 5, 9], [1, 2, 5, 10],
           [1, 2, 5, 10], [1, 3, 6, 11], [1, 3, 6, 11]]


def test_hrc_tree_known_answers():
    obs, idx, L, n = O.hrc_tree(10)
    assert (L, n) == (4, 11)  # cuTAGI's Linear(hidden, 11) for 10 classes
    assert idx.tolist() == HAND_10
    assert torch.all(obs[0] == 1) and obs[1].tolist() == [1, 1, 1, -1]
    assert O.hrc_tree(2)[2:] == (1, 1)
    for nc in [2, 4, 8, 10, 16, 100]:
        obs, idx, L, n = O.hrc_tree(nc)
        assert L == math.ceil(math.log2(nc)) and int(idx.max()) == n and torch.all(idx[:, 0] == 1)
        assert torch.all((obs == 1) | (obs == -1))


@pytest.mark.parametrize("nc", [2, 4, 8, 32])
def test_hrc_tree_power_of_two_is_heap_numbering(nc):
    obs, idx, L, n = O.hrc_tree(nc)
    assert n == nc - 1
    for r in range(nc):
        node = 1
        for c in range(L):
            assert idx[r, c] == node
            bit = (r >> (L - 1 - c)) & 1
            assert obs[r, c] == (1.0 if bit == 0 else -1.0)
            node = 2 * node + bit


@pytest.mark.parametrize("nc", [2, 3, 5, 10, 16, 100, 1000])
def test_engine_tree_tables_match_oracle(nc):
    from triton_tagi_amd.hrc_softmax import class_to_obs

    h = class_to_obs(nc)
    obs, idx, L, n = O.hrc_tree(nc)
    assert h.n_obs == L and h.len == n
    assert h.obs.dtype == torch.float32 and h.idx.dtype == torch.int32
    assert torch.equal(h.obs.double(), obs) and torch.equal(h.idx.long(), idx)


def test_engine_labels_to_hrc_on_cpu():
    from triton_tagi_amd.hrc_softmax import class_to_obs, labels_to_hrc

    h = class_to_obs(10)
    y_obs, y_idx = labels_to_hrc(torch.tensor([3, 0, 0, 9]), h)
    assert torch.equal(y_obs[0], h.obs[3]) and torch.equal(y_idx[3], h.idx[9]) and torch.equal(y_obs[1], y_obs[2])


# --------------------------------------------------------------- sparse innovation
def test_innovation_indexed_reduces_to_dense_rule():
    r = gen(1)
    B, n_out, L = 6, 11, 4
    ma, Sa = torch.randn(B, n_out, generator=r, dtype=D), 0.1 * torch.rand(B, n_out, generator=r, dtype=D) + 1e-3
    obs, idx, _, _ = O.hrc_tree(10)
    lab = torch.randint(0, 10, (B,), generator=r)
    y, ii = obs[lab], idx[lab]
    v = torch.full_like(y, 0.05**2)
    dm, dS = O.innovation_indexed(ma, Sa, y, v, ii)
    sel = torch.zeros(B, n_out, dtype=torch.bool)
    for b in range(B):
        g = ii[b] - 1
        rm, rS = O.innovation(y[b], ma[b, g], Sa[b, g], 0.05)
        assert torch.allclose(dm[b, g], rm, rtol=1e-14, atol=0) and torch.allclose(dS[b, g], rS, rtol=1e-14, atol=0)
        sel[b, g] = True
    assert torch.all(dm[~sel] == 0) and torch.all(dS[~sel] == 0) and torch.all(dS <= 0)
    # a node selected twice receives both terms; out-of-range nodes receive nothing
    ii2 = torch.tensor([[3, 3, 0, 12]])
    y2, v2 = torch.tensor([[1.0, -1.0, 1.0, 1.0]], dtype=D), torch.tensor([[0.1, 0.2, 0.1, 0.1]], dtype=D)
    dm2, dS2 = O.innovation_indexed(ma[:1], Sa[:1], y2, v2, ii2)
    a = O.innovation(y2[0, :2], ma[0, 2].expand(2), Sa[0, 2].expand(2), 0.0)
    e1 = ((y2[0, 0] - ma[0, 2]) / (Sa[0, 2] + 0.1)) + ((y2[0, 1] - ma[0, 2]) / (Sa[0, 2] + 0.2))
    assert torch.isclose(dm2[0, 2], e1) and (dm2[0] != 0).sum() == 1 and a[0].numel() == 2


# ----------------------------------------------------------- HRC class probabilities
@pytest.mark.parametrize("nc", [8, 10])
def test_hrc_class_probs_monte_carlo(nc):
    obs, idx, L, n = O.hrc_tree(nc)
    r = gen(nc)
    B = 3
    ma, Sa = 0.7 * torch.randn(B, n, generator=r, dtype=D), 0.3 * torch.rand(B, n, generator=r, dtype=D)
    alpha = 3.0
    P = O.hrc_class_probs(ma, Sa, obs, idx, alpha)
    # a sample z_node ~ N(mu, S) + N(0, 1/alpha^2) per node; class r is taken when the sign
    # of every node on its path matches its bit (+1: z > 0)
    T = 400_000
    z = ma[None] + Sa.sqrt()[None] * torch.randn(T, B, n, generator=r, dtype=D) + (1 / alpha) * torch.randn(
        T, B, n, generator=r, dtype=D)
    s = torch.where(z > 0, 1.0, -1.0)
    for c in range(nc):
        hit = (s[:, :, idx[c] - 1] == obs[c]).all(dim=2).double().mean(0)
        se = torch.sqrt(P[:, c] * (1 - P[:, c]) / T)
        assert torch.all((hit - P[:, c]).abs() <= 5 * se + 1e-4), (c, hit, P[:, c])
    if nc == 8:  # a full tree: the classes partition the outcomes
        assert torch.allclose(P.sum(1), torch.ones(B, dtype=D), atol=1e-12)


def test_hrc_class_probs_known_answers():
    obs, idx, L, n = O.hrc_tree(10)
    P = O.hrc_class_probs(torch.full((1, n), 10.0, dtype=D), torch.zeros(1, n, dtype=D), obs, idx)
    assert P.argmax(1).item() == 0
    P0 = O.hrc_class_probs(torch.zeros(1, n, dtype=D), torch.zeros(1, n, dtype=D), obs, idx)
    assert P0.sum() <= 1 + 1e-12 and torch.all(P0 >= 0)


# ------------------------------------------------------- heteroscedastic innovation
def _cond_moments(y, mu_a, var_a, mu_v2, power):
    """E[V^power | Y = y] by quadrature, Y = A + V, V ~ N(0, mu_v2), A ~ N(mu_a, var_a)."""
    sv = math.sqrt(mu_v2)

    def w(v):
        return math.exp(-0.5 * v * v / mu_v2) * math.exp(-0.5 * (y - v - mu_a) ** 2 / var_a)

    lo, hi = -12 * sv, 12 * sv
    Z = integrate.quad(w, lo, hi, epsabs=0, epsrel=1e-12, limit=200)[0]
    return integrate.quad(lambda v: v**power * w(v), lo, hi, epsabs=0, epsrel=1e-12, limit=200)[0] / Z


@pytest.mark.parametrize("y,mu_a,var_a,mu_v2", [(0.3, -0.2, 0.5, 0.8), (2.0, 0.1, 0.05, 0.3), (-1.0, 0.4, 1.5, 2.0)])
def test_hetero_posterior_by_quadrature(y, mu_a, var_a, mu_v2):
    m, v = O.hetero_v_posterior(torch.tensor(y, dtype=D), mu_a, var_a, mu_v2)
    e1, e2, e3, e4 = (_cond_moments(y, mu_a, var_a, mu_v2, p) for p in (1, 2, 3, 4))
    assert abs(float(m) - e1) < 1e-8 and abs(float(v) - (e2 - e1 * e1)) < 1e-8
    m2, v2 = O.gaussian_square_moments(m, v)
    assert abs(float(m2) - e2) < 1e-8 and abs(float(v2) - (e4 - e2 * e2)) < 1e-7


def test_hetero_noise_prior_monte_carlo():
    r = gen(5)
    mu, var = 2.0, 0.09  # V2b stays positive
    T = 2_000_000
    v2b = mu + math.sqrt(var) * torch.randn(T, generator=r, dtype=D)
    v = torch.sqrt(v2b) * torch.randn(T, generator=r, dtype=D)
    e, s = O.hetero_noise_prior(torch.tensor(mu, dtype=D), torch.tensor(var, dtype=D))
    sq = v * v
    assert abs(sq.mean().item() - e.item()) < 5 * sq.std().item() / math.sqrt(T)
    assert abs(sq.var().item() - s.item()) / s.item() < 0.01


def test_rts_gain_step_equals_exact_conditioning():
    # X ~ N(mu, sx2); W = X + E, E ~ N(0, t2); observe Z = W + N(0, r2) = z
    mu, sx2, t2, r2, z = 0.4, 0.7, 0.3, 0.2, 1.3
    Sigma = np.array([[sx2, sx2], [sx2, sx2 + t2]])  # cov of (X, W)
    sz = sx2 + t2 + r2
    ex_m = mu + sx2 / sz * (z - mu)
    ex_v = sx2 - sx2 * sx2 / sz
    w_post_m = mu + Sigma[1, 1] / sz * (z - mu)
    w_post_v = Sigma[1, 1] - Sigma[1, 1] ** 2 / sz
    m, v = O.rts_update(mu, sx2, Sigma[0, 1], mu, Sigma[1, 1], w_post_m, w_post_v)
    assert abs(m - ex_m) < 1e-14 and abs(v - ex_v) < 1e-14


def test_heteros_innovation_mean_outputs_are_dense_rule():
    r = gen(9)
    y = torch.randn(4, 5, generator=r, dtype=D)
    mu = torch.randn(4, 10, generator=r, dtype=D)
    mu[:, 1::2] = 0.2 + torch.rand(4, 5, generator=r, dtype=D)
    var = 0.1 + torch.rand(4, 10, generator=r, dtype=D)
    dm, dS = O.heteros_innovation(y, mu, var)
    Sy = var[:, 0::2] + mu[:, 1::2]
    assert torch.allclose(dm[:, 0::2], (y - mu[:, 0::2]) / Sy, rtol=1e-14, atol=0)
    assert torch.allclose(dS[:, 0::2], -1.0 / Sy, rtol=1e-14, atol=0)
    # the noise outputs follow the pinned steps
    mv, vv = O.hetero_v_posterior(y, mu[:, 0::2], var[:, 0::2], mu[:, 1::2])
    m2, v2 = O.gaussian_square_moments(mv, vv)
    pm, pv = O.hetero_noise_prior(mu[:, 1::2], var[:, 1::2])
    k = var[:, 1::2] / pv
    assert torch.allclose(dm[:, 1::2], k * (m2 - pm), rtol=1e-10, atol=1e-14)
    assert torch.allclose(dS[:, 1::2], k * k * (v2 - pv), rtol=1e-10, atol=1e-14)


# ------------------------------------------------------------------- EvenSoftplus
def test_even_softplus_second_order_moments():
    r = gen(11)
    mz = torch.linspace(-8, 25, 64, dtype=D)
    Sz = 0.5 * torch.rand(64, generator=r, dtype=D)
    ma, Sa, J = O.even_softplus(mz, Sz)
    x = mz.clone().requires_grad_(True)
    f = torch.log1p(torch.exp(x))
    (d1,) = torch.autograd.grad(f.sum(), x, create_graph=True)
    (d2,) = torch.autograd.grad(d1.sum(), x)
    odd = torch.arange(64) % 2 == 1
    exp_m = torch.clamp(f.detach() + 0.5 * d2 * Sz, min=1e-9)
    exp_S = torch.clamp(d1.detach() ** 2 * Sz, min=1e-9)
    # above 20 the rule takes softplus(mu) = mu (a 2e-9 difference, even_softplus.py:70)
    tol = torch.where(mz > 20, torch.full_like(mz, 1e-8), 1e-12 * exp_m.abs() + 1e-15)
    assert torch.all(((ma - exp_m).abs() <= tol)[odd])
    assert torch.allclose(Sa[odd], exp_S[odd], rtol=1e-12, atol=1e-15)
    assert torch.allclose(J[odd], d1.detach()[odd], rtol=1e-12, atol=0)
    assert torch.equal(ma[~odd], mz[~odd]) and torch.equal(Sa[~odd], Sz[~odd]) and torch.all(J[~odd] == 1)


# ---------------------------------------------------------------------- MaxPool2D
@pytest.mark.parametrize("k,s,p", [(2, 2, 0), (3, 2, 1), (3, 1, 1), (2, 1, 0), (4, 4, 2), (3, 3, 0)])
def test_maxpool_against_library_and_loops(k, s, p):
    r = gen(k * 10 + s + p)
    N, C, H, W = 2, 3, 9, 7
    ma = torch.randn(N, C, H, W, generator=r, dtype=D)
    Sa = torch.rand(N, C, H, W, generator=r, dtype=D)
    layer = O.OMaxPool2D(k, s, p)
    mz, Sz = layer.forward(ma, Sa)
    ref, ridx = F.max_pool2d_with_indices(ma, k, stride=s, padding=p)
    assert torch.equal(mz, ref) and torch.equal(layer.idx, ridx)
    assert torch.equal(Sz, Sa.reshape(N, C, -1).gather(2, ridx.reshape(N, C, -1)).reshape(ref.shape))
    dm, dS = torch.randn(*ref.shape, generator=r, dtype=D), -torch.rand(*ref.shape, generator=r, dtype=D)
    om, oS = layer.backward(dm, dS)
    em, eS = torch.zeros_like(ma), torch.zeros_like(ma)
    for n in range(N):
        for c in range(C):
            for ho in range(ref.shape[2]):
                for wo in range(ref.shape[3]):
                    j = int(ridx[n, c, ho, wo])
                    em[n, c, j // W, j % W] += dm[n, c, ho, wo]
                    eS[n, c, j // W, j % W] += dS[n, c, ho, wo]
    assert torch.allclose(om, em, rtol=1e-14, atol=1e-15) and torch.allclose(oS, eS, rtol=1e-14, atol=1e-15)


def test_maxpool_ties_pick_the_first_position():
    ma = torch.zeros(1, 1, 4, 4, dtype=D)
    ma[0, 0, 1, 1] = ma[0, 0, 1, 0] = 1.0
    layer = O.OMaxPool2D(2, 2, 0)
    layer.forward(ma, torch.ones_like(ma))
    _, ridx = F.max_pool2d_with_indices(ma, 2, stride=2)
    assert torch.equal(layer.idx, ridx) and layer.idx[0, 0, 0, 0] == 4


# ---------------------------------------------------------------------- LayerNorm
def test_layernorm_stats_against_torch_var():
    r = gen(21)
    ma, Sa = torch.randn(5, 37, generator=r, dtype=D), torch.rand(5, 37, generator=r, dtype=D)
    mu, var = O.layernorm_stats(ma, Sa)
    assert torch.allclose(mu[:, 0], ma.mean(1)) and torch.allclose(var[:, 0], ma.var(1) + Sa.sum(1) / 36)


def test_layernorm_moments_monte_carlo_and_delta_rule():
    r = gen(22)
    B, Dm = 3, 6
    ma, Sa = torch.randn(B, Dm, generator=r, dtype=D), 0.2 * torch.rand(B, Dm, generator=r, dtype=D)
    mw, Sw = 1 + 0.1 * torch.randn(Dm, generator=r, dtype=D), 0.05 * torch.rand(Dm, generator=r, dtype=D)
    mb, Sb = 0.1 * torch.randn(Dm, generator=r, dtype=D), 0.02 * torch.rand(Dm, generator=r, dtype=D)
    layer = O.OLayerNorm(mw, Sw, mb, Sb, 1e-5)
    mz, Sz = layer.forward(ma, Sa)
    # statistics are deterministic functions of the means; the rest is a product of
    # independent Gaussians a, g plus b
    inv = 1 / torch.sqrt(layer.var_ra + 1e-5)
    T = 400_000
    a = ma + Sa.sqrt() * torch.randn(T, B, Dm, generator=r, dtype=D)
    g = mw + Sw.sqrt() * torch.randn(T, 1, Dm, generator=r, dtype=D)
    bb = mb + Sb.sqrt() * torch.randn(T, 1, Dm, generator=r, dtype=D)
    z = inv * (a - layer.mu_ra) * g + bb
    assert torch.all((z.mean(0) - mz).abs() <= 5 * z.std(0) / math.sqrt(T))
    assert torch.all(((z.var(0) - Sz) / Sz).abs() < 0.02)
    # delta rule with autograd Jacobians of the mean map (statistics held fixed)
    dmz, dSz = torch.randn(B, Dm, generator=r, dtype=D), -torch.rand(B, Dm, generator=r, dtype=D)
    dma, dSa = layer.backward(dmz, dSz)
    x, gw, gb = ma.clone().requires_grad_(True), mw.clone().requires_grad_(True), mb.clone().requires_grad_(True)
    f = inv * (x - layer.mu_ra) * gw + gb
    Jx = torch.autograd.functional.jacobian(lambda t: (inv * (t - layer.mu_ra) * mw + mb), ma)  # (B,D,B,D)
    Jx = Jx.reshape(B * Dm, B * Dm)
    assert torch.allclose(dma.reshape(-1), Jx.T @ dmz.reshape(-1)) and torch.allclose(
        dSa.reshape(-1), (Jx**2).T @ dSz.reshape(-1))
    Jw = torch.autograd.functional.jacobian(lambda t: (inv * (ma - layer.mu_ra) * t + mb), mw).reshape(B * Dm, Dm)
    Jb = torch.autograd.functional.jacobian(lambda t: (inv * (ma - layer.mu_ra) * mw + t), mb).reshape(B * Dm, Dm)
    assert torch.allclose(layer.delta_mw, Sw * (Jw.T @ dmz.reshape(-1)))
    assert torch.allclose(layer.delta_Sw, Sw * Sw * ((Jw**2).T @ dSz.reshape(-1)))
    assert torch.allclose(layer.delta_mb, Sb * (Jb.T @ dmz.reshape(-1)))
    assert torch.allclose(layer.delta_Sb, Sb * Sb * ((Jb**2).T @ dSz.reshape(-1)))
    del f, x, gw, gb


# ----------------------------------------------------------------- planted mistakes
def test_head_pins_catch_planted_mistakes(monkeypatch):
    # class probabilities with the bit orientation swapped
    good = O.hrc_class_probs

    def swapped(ma, Sa, obs, idx, alpha=3.0):
        return good(ma, Sa, -obs, idx, alpha)

    monkeypatch.setattr(O, "hrc_class_probs", swapped)
    with pytest.raises(AssertionError):
        test_hrc_class_probs_monte_carlo(10)
    monkeypatch.setattr(O, "hrc_class_probs", good)
    # node numbering off by one level offset
    tree = O.hrc_tree

    def shifted(nc):
        obs, idx, L, n = tree(nc)
        idx = idx.clone()
        idx[:, -1] += 1
        return obs, idx, L, n + 1

    monkeypatch.setattr(O, "hrc_tree", shifted)
    with pytest.raises(AssertionError):
        test_hrc_tree_known_answers()
    monkeypatch.setattr(O, "hrc_tree", tree)
    # V posterior variance with the wrong sign of the correction
    post = O.hetero_v_posterior
    monkeypatch.setattr(O, "hetero_v_posterior",
                        lambda y, ma, va, mv: (post(y, ma, va, mv)[0], 2 * mv - post(y, ma, va, mv)[1]))
    with pytest.raises(AssertionError):
        test_hetero_posterior_by_quadrature(0.3, -0.2, 0.5, 0.8)
    monkeypatch.setattr(O, "hetero_v_posterior", post)
    # Var[V^2] without the 2 mu^2 term
    monkeypatch.setattr(O, "hetero_noise_prior", lambda m, v: (m, 3.0 * v))
    with pytest.raises(AssertionError):
        test_hetero_noise_prior_monte_carlo()
    # LayerNorm variance without Bessel's correction
    st = O.layernorm_stats
    monkeypatch.setattr(O, "layernorm_stats", lambda m, S: (st(m, S)[0], st(m, S)[1] * (m.shape[-1] - 1) / m.shape[-1]))
    with pytest.raises(AssertionError):
        test_layernorm_stats_against_torch_var()
