"""CPU oracle of the TAGI step: a restatement of triton-tagi's moment equations.

TEST INFRASTRUCTURE ONLY. The HIP engine is tested against this oracle; only tests/,
``__graft_entry__.smoke()`` and the CPU-baseline leg of ``bench.py`` may import it. The
engine (package ``triton_tagi_amd``) never imports it and has no CPU path.

Everything runs in torch on the CPU, in float64 by default (``dtype`` selects float32
for the CPU-baseline timing). Each function cites the reference file:line it restates
(paths relative to the miquelflorensa/triton-tagi source tree). How each function is
pinned (closed forms, autograd Jacobians, Monte Carlo, quadrature, brute-force
convolution, reference-generated golden vectors) is listed in tests/test_oracle_pins.py.

The oracle layers mirror the engine's layers by duck typing: ``mirror(layer)`` copies a
layer's hyper-parameters and parameter tensors (moved to CPU in ``dtype``).
"""

from __future__ import annotations

import math

import torch
import torch.nn.functional as F

DT = torch.float64
INV_SQRT_2PI = 0.3989422804014327
INV_SQRT_2 = 0.7071067811865476


def _c(t, dtype=DT):
    return None if t is None else t.detach().to("cpu", dtype).clone()


# ===================================================================== update rules
def get_cap_factor(batch_size: int) -> float:
    """update/parameters.py:30-50."""
    if batch_size == 1:
        return 0.1
    if batch_size < 256:
        return 2.0
    return 3.0


def capped_update(m, S, dm, dS, cap):
    """update/parameters.py:58-96 (returns new tensors; both caps use the pre-update S)."""
    bar = torch.sqrt(torch.clamp(S, min=1e-10)) / cap
    m_new = m + torch.sign(dm) * torch.minimum(dm.abs(), bar)
    S_raw = S + torch.sign(dS) * torch.minimum(dS.abs(), bar)
    S_new = torch.where(S_raw <= 0, torch.full_like(S_raw, 1e-5), S_raw)
    return m_new, S_new


def innovation(y, mu, var, sigma_v):
    """update/observation.py:24-46: (y-mu)/(var+sv^2), -1/(var+sv^2)."""
    Sy = var + sigma_v**2
    return (y - mu) / Sy, -1.0 / Sy


# ======================================================================= primitives
def linear_moments(ma, Sa, mw, Sw, mb, Sb):
    """layers/linear.py:99-100, kernels/common.py:148-151,159-164."""
    mz = ma @ mw + mb
    Sz = (ma * ma) @ Sw + Sa @ (mw * mw + Sw) + Sb
    return mz, Sz


def linear_backward_delta(dmz, dSz, mw):
    """kernels/common.py:266-267: dmz @ mw^T, dSz @ (mw^2)^T."""
    return dmz @ mw.T, dSz @ (mw * mw).T


def linear_param_grads(a, dmz, dSz):
    """layers/linear.py:138-141: a^T dmz, sum dmz, (a^2)^T dSz, sum dSz."""
    return a.T @ dmz, dmz.sum(0, keepdim=True), (a * a).T @ dSz, dSz.sum(0, keepdim=True)


def relu_moments(mz, Sz):
    """layers/relu.py:55-84 (incl. the alpha < -5 asymptotic Phi and the variance floor)."""
    Ss = torch.clamp(Sz, min=1e-30)
    sig = torch.sqrt(Ss)
    alpha = mz / sig
    pdf = torch.exp(-0.5 * alpha * alpha) * INV_SQRT_2PI
    cdf_erf = 0.5 * (1.0 + torch.erf(alpha * INV_SQRT_2))
    cdf = torch.where(alpha < -5.0, pdf / (-alpha), cdf_erf)
    mu = sig * pdf + mz * cdf
    var = -mu * mu + 2.0 * mu * mz - mz * sig * pdf + (Ss - mz * mz) * cdf
    return mu, torch.clamp(var, min=0.0), cdf


def remax_moments(mu_z, var_z):
    """layers/remax.py:59-109, rows over the last dim."""
    EPS = 1e-6
    std_z = torch.sqrt(var_z)
    alpha = mu_z / std_z
    pdf = INV_SQRT_2PI * torch.exp(-0.5 * alpha * alpha)
    cdf = 0.5 + 0.5 * torch.erf(alpha * INV_SQRT_2)
    mu_m = torch.clamp(mu_z * cdf + std_z * pdf, min=EPS)
    var_m = torch.clamp(-mu_m * mu_m + 2.0 * mu_m * mu_z - mu_z * std_z * pdf + (var_z - mu_z * mu_z) * cdf, min=EPS)
    mu_mt = torch.clamp(mu_m.sum(-1, keepdim=True), min=EPS)
    var_mt = torch.clamp(var_m.sum(-1, keepdim=True), min=EPS)
    var_log_m = torch.log(1.0 + var_m / (mu_m * mu_m))
    mu_log_m = torch.log(mu_m) - 0.5 * var_log_m
    var_log_mt = torch.log(1.0 + var_mt / (mu_mt * mu_mt))
    mu_log_mt = torch.log(mu_mt) - 0.5 * var_log_mt
    cov_log_m_mt = torch.log(1.0 + var_m / (mu_m * mu_mt))
    mu_log_a = mu_log_m - mu_log_mt
    var_log_a = torch.clamp(var_log_m + var_log_mt - 2.0 * cov_log_m_mt, min=0.0)
    mu_a_raw = torch.clamp(torch.exp(mu_log_a + 0.5 * var_log_a), min=EPS)
    sum_a = torch.clamp(mu_a_raw.sum(-1, keepdim=True), min=EPS)
    mu_a = mu_a_raw / sum_a
    var_a = (torch.exp(var_log_a) - 1.0) * mu_a * mu_a
    cov_a_m = (torch.exp(var_log_m - cov_log_m_mt) - 1.0) * mu_a * mu_m
    cov_a_z = torch.minimum(torch.sqrt(var_a * var_z), cov_a_m / torch.clamp(cdf, min=EPS))
    return mu_a, var_a, cov_a_z / var_z


def conv_pads(H, W, k, s, p, padding_type):
    """layers/conv2d.py:280-291: (pad_top/left, Ho, Wo)."""
    if padding_type == 2 and p > 0:
        return 0, (H + p - k) // s + 1, (W + p - k) // s + 1
    return p, (H + 2 * p - k) // s + 1, (W + 2 * p - k) // s + 1


def im2col(x, k, s, p, padding_type):
    """layers/conv2d.py:40-77,278-297 via F.unfold: rows (n, oh, ow), cols (c, kh, kw)."""
    N = x.shape[0]
    if padding_type == 2 and p > 0:
        x = F.pad(x, (0, p, 0, p))
        pad = 0
    else:
        pad = p
    cols = F.unfold(x, kernel_size=k, padding=pad, stride=s)  # (N, K, L)
    return cols.permute(0, 2, 1).reshape(-1, cols.shape[1])


def col2im(cols, N, C, H, W, k, s, p, padding_type):
    """layers/conv2d.py:85-132,359-370 via F.fold, with the padding_type-2 crop."""
    K = cols.shape[1]
    if padding_type == 2 and p > 0:
        Hp, Wp = H + p, W + p
        Ho, Wo = (Hp - k) // s + 1, (Wp - k) // s + 1
        t = cols.view(N, Ho * Wo, K).permute(0, 2, 1)
        img = F.fold(t, output_size=(Hp, Wp), kernel_size=k, stride=s)
        return img[:, :, :H, :W].contiguous()
    Ho, Wo = (H + 2 * p - k) // s + 1, (W + 2 * p - k) // s + 1
    t = cols.view(N, Ho * Wo, K).permute(0, 2, 1)
    return F.fold(t, output_size=(H, W), kernel_size=k, stride=s, padding=p)


def bn_batch_stats(mz, Sz):
    """layers/batchnorm2d.py:321-339 (Bessel-corrected variance of the Gaussian inputs)."""
    N, C, H, W = mz.shape
    n = N * H * W
    mean = mz.mean(dim=(0, 2, 3))
    mean_S = Sz.mean(dim=(0, 2, 3))
    mean_sq = (mz * mz).mean(dim=(0, 2, 3))
    return mean, (mean_S + mean_sq - mean * mean) * (n / (n - 1))


def bmm_tagi(mu_a, var_a, mu_b, var_b, scale=1.0):
    """kernels/attention.py:66-131 plus the mean matmul (multihead_attention.py:180,192)."""
    mean = scale * (mu_a @ mu_b)
    var = (scale * scale) * (var_a @ (mu_b * mu_b + var_b) + (mu_a * mu_a) @ var_b)
    return mean, var


def bmm_shared_right(a_mean, a_var, b, scale=1.0):
    """kernels/attention.py:215-336."""
    return scale * (a_mean @ b), (scale * scale) * (a_var @ (b * b))


def bmm_shared_left(a, b_mean, b_var, scale=1.0):
    """kernels/attention.py:339-374."""
    return scale * (a @ b_mean), (scale * scale) * ((a * a) @ b_var)


def sinusoidal_table(max_seq_len, embed_dim):
    """layers/positional_encoding.py:45-52 (frequency exponent d/E with d as a float).

    The table is a constant of the layer that the reference builds in float32 (angle =
    t * freq rounded to float32 before sin/cos); it is built the same way here and then
    widened, so it holds the reference's values rather than the float64 ones (they differ
    by the float32 rounding of the angle, up to ~1e-4 at t = 2047)."""
    f32 = torch.float32
    d = torch.arange(embed_dim, dtype=f32)
    pos = torch.arange(max_seq_len, dtype=f32)
    freq = 1.0 / torch.pow(10000.0, d / embed_dim)
    angle = pos.unsqueeze(1) * freq.unsqueeze(0)
    even = (torch.arange(embed_dim) % 2 == 0).unsqueeze(0)
    return torch.where(even, torch.sin(angle), torch.cos(angle)).to(DT)


# =========================================================================== layers
class OLayer:
    learnable = False

    def param_groups(self):
        return []

    def update(self, cap):
        for obj, m, S, dm, dS in self.param_groups():
            nm, nS = capped_update(getattr(obj, m), getattr(obj, S), getattr(obj, dm), getattr(obj, dS), cap)
            setattr(obj, m, nm)
            setattr(obj, S, nS)


class OLinear(OLayer):
    """layers/linear.py:83-172."""

    learnable = True

    def __init__(self, mw, Sw, mb, Sb, has_bias=True):
        self.mw, self.Sw, self.mb, self.Sb, self.has_bias = mw, Sw, mb, Sb, has_bias

    def forward(self, ma, Sa):
        self.shape = ma.shape
        K = self.mw.shape[0]
        a = ma.reshape(-1, K)
        self.ma_in = a
        mz, Sz = linear_moments(a, Sa.reshape(-1, K), self.mw, self.Sw, self.mb, self.Sb)
        out = (*self.shape[:-1], self.mw.shape[1])
        return mz.reshape(out), Sz.reshape(out)

    def backward(self, dmz, dSz):
        N = self.mw.shape[1]
        dm, dS = dmz.reshape(-1, N), dSz.reshape(-1, N)
        gmw, gmb, gSw, gSb = linear_param_grads(self.ma_in, dm, dS)
        self.delta_mw, self.delta_Sw = self.Sw * gmw, self.Sw * self.Sw * gSw
        if self.has_bias:
            self.delta_mb, self.delta_Sb = self.Sb * gmb, self.Sb * self.Sb * gSb
        dma, dSa = linear_backward_delta(dm, dS, self.mw)
        inn = (*self.shape[:-1], self.mw.shape[0])
        return dma.reshape(inn), dSa.reshape(inn)

    def param_groups(self):
        g = [(self, "mw", "Sw", "delta_mw", "delta_Sw")]
        if self.has_bias:
            g.append((self, "mb", "Sb", "delta_mb", "delta_Sb"))
        return g


class OConv2D(OLayer):
    """layers/conv2d.py:254-379 (im2col + Linear on patches + col2im)."""

    learnable = True

    def __init__(self, mw, Sw, mb, Sb, C_out, k, stride, padding, padding_type):
        self.mw, self.Sw, self.mb, self.Sb = mw, Sw, mb, Sb
        self.C_out, self.k, self.stride, self.padding, self.padding_type = C_out, k, stride, padding, padding_type

    def forward(self, ma, Sa):
        N, C, H, W = ma.shape
        self.input_shape = (N, C, H, W)
        _, Ho, Wo = conv_pads(H, W, self.k, self.stride, self.padding, self.padding_type)
        self.spatial = (Ho, Wo)
        P = im2col(ma, self.k, self.stride, self.padding, self.padding_type)
        PS = im2col(Sa, self.k, self.stride, self.padding, self.padding_type)
        self.patches = P
        mz, Sz = linear_moments(P, PS, self.mw, self.Sw, self.mb, self.Sb)
        mz = mz.view(N, Ho, Wo, self.C_out).permute(0, 3, 1, 2).contiguous()
        Sz = Sz.view(N, Ho, Wo, self.C_out).permute(0, 3, 1, 2).contiguous()
        return mz, Sz

    def backward(self, dmz, dSz):
        N, C, H, W = self.input_shape
        dm = dmz.permute(0, 2, 3, 1).reshape(-1, self.C_out)
        dS = dSz.permute(0, 2, 3, 1).reshape(-1, self.C_out)
        gmw, gmb, gSw, gSb = linear_param_grads(self.patches, dm, dS)
        self.delta_mw, self.delta_Sw = self.Sw * gmw, self.Sw * self.Sw * gSw
        self.delta_mb, self.delta_Sb = self.Sb * gmb, self.Sb * self.Sb * gSb
        dpm, dpS = linear_backward_delta(dm, dS, self.mw)
        a = (N, C, H, W, self.k, self.stride, self.padding, self.padding_type)
        return col2im(dpm, *a), col2im(dpS, *a)

    def param_groups(self):
        return [(self, "mw", "Sw", "delta_mw", "delta_Sw"), (self, "mb", "Sb", "delta_mb", "delta_Sb")]


class OBatchNorm2D(OLayer):
    """layers/batchnorm2d.py:307-527 (training: batch statistics, running-stat EMA,
    first-call gamma := sqrt(var + eps) when preserve_var)."""

    learnable = True

    def __init__(self, mw, Sw, mb, Sb, running_mean, running_var, momentum, eps, preserve_var, initialized,
                 training=True):
        self.mw, self.Sw, self.mb, self.Sb = mw, Sw, mb, Sb
        self.running_mean, self.running_var = running_mean, running_var
        self.momentum, self.eps, self.preserve_var = momentum, eps, preserve_var
        self._is_initialized = initialized
        self.training = training

    def forward(self, mz, Sz):
        self.input_shape = mz.shape
        if self.training:
            bmean, bvar = bn_batch_stats(mz, Sz)
            if not self._is_initialized:
                self.running_mean, self.running_var = bmean.clone(), bvar.clone()
                if self.preserve_var:
                    self.mw = torch.sqrt(self.running_var + self.eps)
                self._is_initialized = True
            else:
                a = self.momentum
                self.running_mean = (1 - a) * self.running_mean + a * bmean
                self.running_var = (1 - a) * self.running_var + a * bvar
            mean, var = bmean, bvar
        else:
            mean, var = self.running_mean, self.running_var
        self.norm_var = var
        v = lambda t: t.view(1, -1, 1, 1)  # noqa: E731
        mhat = (mz - v(mean)) / torch.sqrt(v(var) + self.eps)
        Shat = Sz / (v(var) + self.eps)
        self.m_hat = mhat
        g, Sg, b, Sb = v(self.mw), v(self.Sw), v(self.mb), v(self.Sb)
        return g * mhat + b, g * g * Shat + Sg * mhat * mhat + Sg * Shat + Sb

    def backward(self, dma, dSa):
        v = lambda t: t.view(1, -1, 1, 1)  # noqa: E731
        mh = self.m_hat
        self.delta_mw = self.Sw * (dma * mh).sum(dim=(0, 2, 3))
        self.delta_Sw = self.Sw * self.Sw * (dSa * mh * mh).sum(dim=(0, 2, 3))
        self.delta_mb = self.Sb * dma.sum(dim=(0, 2, 3))
        self.delta_Sb = self.Sb * self.Sb * dSa.sum(dim=(0, 2, 3))
        g = v(self.mw)
        var = v(self.norm_var) + self.eps
        return dma * g / torch.sqrt(var), dSa * g * g / var

    def param_groups(self):
        return [(self, "mw", "Sw", "delta_mw", "delta_Sw"), (self, "mb", "Sb", "delta_mb", "delta_Sb")]


class OReLU(OLayer):
    """layers/relu.py:135-169."""

    def forward(self, mz, Sz):
        ma, Sa, self.J = relu_moments(mz, Sz)
        return ma, Sa

    def backward(self, dm, dS):
        return dm * self.J, dS * self.J * self.J


class ORemax(OLayer):
    """layers/remax.py:180-188."""

    def forward(self, mz, Sz):
        ma, Sa, self.J = remax_moments(mz, Sz)
        return ma, Sa

    def backward(self, dm, dS):
        return dm * self.J, dS * self.J * self.J


class OAvgPool2D(OLayer):
    """layers/avgpool2d.py:349-430."""

    def __init__(self, k, spatial_correlation=False):
        self.k, self.sc = k, spatial_correlation

    def _vs(self):
        i = 1.0 / (self.k * self.k)
        return i if self.sc else i * i

    def forward(self, ma, Sa):
        self.input_shape = ma.shape
        N, C, H, W = ma.shape
        k = self.k
        Ho, Wo = H // k, W // k
        t = lambda x: x[:, :, : Ho * k, : Wo * k].reshape(N, C, Ho, k, Wo, k).sum(dim=(3, 5))  # noqa: E731
        return t(ma) / (k * k), t(Sa) * self._vs()

    def backward(self, dm, dS):
        N, C, H, W = self.input_shape
        k = self.k
        up = lambda x: x.repeat_interleave(k, 2).repeat_interleave(k, 3)  # noqa: E731
        om = torch.zeros(N, C, H, W, dtype=dm.dtype)
        oS = torch.zeros(N, C, H, W, dtype=dm.dtype)
        Ho, Wo = H // k, W // k
        om[:, :, : Ho * k, : Wo * k] = up(dm) / (k * k)
        oS[:, :, : Ho * k, : Wo * k] = up(dS) * self._vs()
        return om, oS


class OFlatten(OLayer):
    """layers/flatten.py:25-53."""

    def forward(self, ma, Sa):
        self.shape = ma.shape
        return ma.reshape(ma.shape[0], -1), Sa.reshape(Sa.shape[0], -1)

    def backward(self, dm, dS):
        return dm.reshape(self.shape), dS.reshape(self.shape)


class OResBlock(OLayer):
    """layers/resblock.py:354-438."""

    learnable = True

    def __init__(self, main, proj):
        self.main, self.proj = main, proj

    def forward(self, mu, var):
        mz, Sz = mu, var
        for layer in self.main:
            mz, Sz = layer.forward(mz, Sz)
        mx, Sx = mu, var
        for layer in self.proj:
            mx, Sx = layer.forward(mx, Sx)
        return mz + mx, Sz + Sx

    def backward(self, dm, dS):
        am, aS = dm, dS
        for layer in reversed(self.main):
            am, aS = layer.backward(am, aS)
        bm, bS = dm, dS
        for layer in reversed(self.proj):
            bm, bS = layer.backward(bm, bS)
        return am + bm, aS + bS

    def param_groups(self):
        return [g for layer in self.main + self.proj for g in layer.param_groups()]


class OMultiheadAttentionV2(OLayer):
    """layers/multihead_attention.py:154-276."""

    learnable = True

    def __init__(self, q, k, v, num_heads):
        self.q, self.k, self.v, self.H = q, k, v, num_heads

    def forward(self, ma, Sa):
        B, S, E = ma.shape
        H = self.H
        D = E // H
        s = 1.0 / math.sqrt(D)
        heads = lambda t: t.reshape(B, S, H, D).transpose(1, 2)  # noqa: E731
        mq, vq = (heads(t) for t in self.q.forward(ma, Sa))
        mk, vk = (heads(t) for t in self.k.forward(ma, Sa))
        mv, vv = (heads(t) for t in self.v.forward(ma, Sa))
        mu_qk, var_qk = bmm_tagi(mq, vq, mk.transpose(-1, -2), vk.transpose(-1, -2), s)
        msc, vsc, J = remax_moments(mu_qk, var_qk)
        mo, vo = bmm_tagi(msc, vsc, mv, vv, 1.0)
        self.cache = dict(B=B, S=S, H=H, D=D, s=s, mq=mq, mk=mk, mv=mv, msc=msc, J=J)
        self.attn = (msc, vsc)
        unh = lambda t: t.transpose(1, 2).reshape(B, S, E)  # noqa: E731
        return unh(mo), unh(vo)

    def backward(self, dmz, dSz):
        c = self.cache
        B, S, H, D, s = c["B"], c["S"], c["H"], c["D"], c["s"]
        E = H * D
        heads = lambda t: t.reshape(B, S, H, D).transpose(1, 2)  # noqa: E731
        unh = lambda t: t.transpose(1, 2).reshape(B, S, E)  # noqa: E731
        dm, dv_ = heads(dmz), heads(dSz)
        dV, dSV = bmm_shared_left(c["msc"].transpose(-1, -2), dm, dv_)
        dsc, dSsc = bmm_shared_right(dm, dv_, c["mv"].transpose(-1, -2))
        sm, sv = dsc * c["J"], dSsc * c["J"] * c["J"]
        dQ, dSQ = bmm_shared_right(sm, sv, c["mk"], s)
        dK, dSK = bmm_shared_right(sm.transpose(-1, -2), sv.transpose(-1, -2), c["mq"], s)
        a1, b1 = self.q.backward(unh(dQ), unh(dSQ))
        a2, b2 = self.k.backward(unh(dK), unh(dSK))
        a3, b3 = self.v.backward(unh(dV), unh(dSV))
        return a1 + a2 + a3, b1 + b2 + b3

    def param_groups(self):
        return self.q.param_groups() + self.k.param_groups() + self.v.param_groups()


class ORMSNorm(OLayer):
    """layers/rms_norm.py:93-140."""

    learnable = True

    def __init__(self, mw, Sw, eps):
        self.mw, self.Sw, self.eps = mw, Sw, eps

    def forward(self, ma, Sa):
        self.shape = ma.shape
        D = self.mw.shape[0]
        m, S = ma.reshape(-1, D), Sa.reshape(-1, D)
        rms = (m * m + S).mean(dim=1, keepdim=True)
        inv = 1.0 / torch.sqrt(rms + self.eps)
        self.m_in, self.inv = m, inv
        mz = inv * m * self.mw
        Sz = inv * inv * (S * (self.mw * self.mw + self.Sw) + self.Sw * m * m)
        return mz.reshape(self.shape), Sz.reshape(self.shape)

    def backward(self, dmz, dSz):
        D = self.mw.shape[0]
        dm, dS = dmz.reshape(-1, D), dSz.reshape(-1, D)
        t = self.inv * self.mw
        self.delta_mw = (self.inv * self.m_in * dm).sum(0) * self.Sw
        self.delta_Sw = (self.inv * self.inv * self.m_in * self.m_in * dS).sum(0) * self.Sw * self.Sw
        return (t * dm).reshape(dmz.shape), (t * t * dS).reshape(dSz.shape)

    def param_groups(self):
        return [(self, "mw", "Sw", "delta_mw", "delta_Sw")]


class OEmbedding(OLayer):
    """layers/embedding.py:88-150."""

    learnable = True

    def __init__(self, mw, Sw, padding_idx=-1):
        self.mw, self.Sw, self.padding_idx = mw, Sw, padding_idx

    def forward(self, ma, Sa):
        if ma.dim() == 3 and ma.shape[-1] == 1:
            ma = ma.squeeze(-1)
        cat = ma.long()
        self.cat = cat
        mz, Sz = self.mw[cat], self.Sw[cat]
        if self.padding_idx >= 0:
            mask = (cat == self.padding_idx).unsqueeze(-1)
            mz, Sz = mz.masked_fill(mask, 0.0), Sz.masked_fill(mask, 0.0)
        return mz, Sz

    def backward(self, dmz, dSz):
        cat = self.cat.reshape(-1)
        D = self.mw.shape[1]
        sw = self.Sw[cat]
        dm, dS = dmz.reshape(-1, D) * sw, dSz.reshape(-1, D) * sw * sw
        if self.padding_idx >= 0:
            keep = (cat != self.padding_idx).unsqueeze(-1).to(dm.dtype)
            dm, dS = dm * keep, dS * keep
        idx = cat.unsqueeze(-1).expand(-1, D)
        self.delta_mw = torch.zeros_like(self.mw).scatter_add_(0, idx, dm)
        self.delta_Sw = torch.zeros_like(self.Sw).scatter_add_(0, idx, dS)
        z = torch.zeros(self.cat.shape, dtype=dmz.dtype)
        return z, z.clone()

    def param_groups(self):
        return [(self, "mw", "Sw", "delta_mw", "delta_Sw")]


class OPositionalEncoding(OLayer):
    """layers/positional_encoding.py:59-68."""

    def __init__(self, pe):
        self.pe = pe

    def forward(self, ma, Sa):
        return ma + self.pe[: ma.shape[-2]], Sa

    def backward(self, dm, dS):
        return dm, dS


class ONet:
    """network.py:92-152: forward, step (innovation, reversed backward, capped update)."""

    def __init__(self, layers):
        self.layers = layers

    def forward(self, x, record=False):
        ma, Sa = x, torch.zeros_like(x)
        self.trace = []
        for layer in self.layers:
            ma, Sa = layer.forward(ma, Sa)
            if record:
                self.trace.append((ma.clone(), Sa.clone()))
        return ma, Sa

    def step(self, x, y, sigma_v, record=False):
        mu, var = self.forward(x, record=record)
        dm, dS = innovation(y, mu, var, sigma_v)
        self.bwd_trace = []
        for layer in reversed(self.layers):
            dm, dS = layer.backward(dm, dS)
            if record:
                self.bwd_trace.append((dm.clone(), dS.clone()))
        cap = get_cap_factor(x.shape[0])
        for layer in self.layers:
            if layer.learnable:
                layer.update(cap)
        return mu, var

    def step_hrc(self, x, labels, n_classes, sigma_v):
        """network.py:157-224: sparse innovation on each label's tree path."""
        mu, var = self.forward(x)
        obs, idx, L, _ = hrc_tree(n_classes)
        width = mu.shape[-1]
        lab = labels.reshape(-1).long()
        y_obs, y_idx = obs[lab], idx[lab]
        dm, dS = innovation_indexed(mu.reshape(-1, width), var.reshape(-1, width), y_obs,
                                    torch.full_like(y_obs, sigma_v**2), y_idx)
        dm, dS = dm.reshape(mu.shape), dS.reshape(mu.shape)
        for layer in reversed(self.layers):
            dm, dS = layer.backward(dm, dS)
        cap = get_cap_factor(x.shape[0])
        for layer in self.layers:
            if layer.learnable:
                layer.update(cap)
        return mu, var

    def step_heteros(self, x, y):
        """network.py:119-152 with the heteroscedastic innovation (observation.py:137)."""
        mu, var = self.forward(x)
        dm, dS = heteros_innovation(y, mu, var)
        for layer in reversed(self.layers):
            dm, dS = layer.backward(dm, dS)
        cap = get_cap_factor(x.shape[0])
        for layer in self.layers:
            if layer.learnable:
                layer.update(cap)
        return mu, var


# ================================================================ output heads (HRC)
def hrc_tree(n_classes):
    """hrc_softmax.py:73-128 (cuTAGI class_to_obs): (obs, idx, n_obs, len).

    Bits of class r are its binary code, MSB first; bit c is observed as (-1)^bit at the
    node numbered 1 + (nodes on the levels above) + (value of the c leading bits).
    """
    L = math.ceil(math.log2(n_classes))
    per_level = [n_classes]
    for _ in range(L):
        per_level.insert(0, math.ceil(per_level[0] / 2))
    offset = [1]
    for d in range(1, L):
        offset.append(offset[-1] + per_level[d - 1])
    obs = [[0.0] * L for _ in range(n_classes)]
    idx = [[0] * L for _ in range(n_classes)]
    for r in range(n_classes):
        code = format(r, f"0{L}b")
        for c in range(L):
            obs[r][c] = 1.0 if code[c] == "0" else -1.0
            idx[r][c] = offset[c] + (int(code[:c], 2) if c else 0)
    return torch.tensor(obs, dtype=DT), torch.tensor(idx, dtype=torch.int64), L, max(max(row) for row in idx)


def innovation_indexed(ma, Sa, y_obs, var_obs, idx):
    """update/observation.py:171-224: dense rule at node idx-1 of each row, zeros elsewhere
    (index_add, so a node selected twice receives both terms)."""
    dm, dS = torch.zeros_like(ma), torch.zeros_like(Sa)
    for b in range(ma.shape[0]):
        for c in range(idx.shape[1]):
            j = int(idx[b, c]) - 1
            if j < 0 or j >= ma.shape[1]:
                continue
            den = Sa[b, j] + var_obs[b, c]
            dm[b, j] += (y_obs[b, c] - ma[b, j]) / den
            dS[b, j] += -1.0 / den
    return dm, dS


def hrc_class_probs(ma, Sa, obs, idx, alpha=3.0):
    """hrc_softmax.py:164-208: product along each class path of Phi(mu/sqrt(1/alpha^2+S))
    (bit +1) or its complement (bit -1)."""
    P = torch.special.ndtr(ma / torch.sqrt((1.0 / alpha) ** 2 + Sa))
    node = P[:, idx - 1]  # (B, n_classes, L)
    f = torch.where(obs > 0, node, 1.0 - node)
    return f.prod(dim=2)


# ===================================================== heteroscedastic output (TAGI-V)
def hetero_noise_prior(mu_v2b, var_v2b):
    """observation.py:82-86: moments of V^2 for V ~ N(0, V2b), V2b ~ N(mu, var):
    E[V^2] = mu, Var[V^2] = 3 var + 2 mu^2."""
    return mu_v2b, 3.0 * var_v2b + 2.0 * mu_v2b * mu_v2b


def hetero_v_posterior(y, mu_a, var_a, mu_v2):
    """observation.py:88-98: Y = A + V, A ~ N(mu_a, var_a), V ~ N(0, mu_v2); moments of
    V | Y = y (and the innovation of the mean output)."""
    var_sum = var_a + mu_v2
    m = mu_v2 / var_sum * (y - mu_a)
    v = mu_v2 - mu_v2 / var_sum * mu_v2
    return m, v


def gaussian_square_moments(m, v):
    """observation.py:100-102: E[X^2], Var[X^2] of X ~ N(m, v)."""
    return m * m + v, 2.0 * v * v + 4.0 * v * m * m


def rts_update(mu_x, var_x, cov_xw, mu_w, var_w, mu_w_post, var_w_post):
    """observation.py:104-107: move X by the change of the linked W (gain cov/var_w)."""
    k = cov_xw / var_w
    return mu_x + k * (mu_w_post - mu_w), var_x + k * k * (var_w_post - var_w)


def heteros_innovation(y, mu, var):
    """observation.py:49-111: interleaved (mean, noise) output pairs; returns deltas
    shaped like mu."""
    mu_a, mu_v2b = mu[..., 0::2], mu[..., 1::2]
    var_a, var_v2b = var[..., 0::2], var[..., 1::2]
    mu_v2, var_v2 = hetero_noise_prior(mu_v2b, var_v2b)
    var_sum = var_a + mu_v2
    d_mu, d_var = (y - mu_a) / var_sum, -1.0 / var_sum
    mv, vv = hetero_v_posterior(y, mu_a, var_a, mu_v2)
    m2, v2 = gaussian_square_moments(mv, vv)
    mb_post, vb_post = rts_update(mu_v2b, var_v2b, var_v2b, mu_v2, var_v2, m2, v2)
    dm, dS = torch.empty_like(mu), torch.empty_like(var)
    dm[..., 0::2], dS[..., 0::2] = d_mu, d_var
    dm[..., 1::2], dS[..., 1::2] = mb_post - mu_v2b, vb_post - var_v2b
    return dm, dS


def even_softplus(mz, Sz):
    """layers/even_softplus.py:38-90: second-order softplus moments at odd flat positions."""
    m, S = mz.reshape(-1), Sz.reshape(-1)
    sig = torch.sigmoid(m)
    sp = F.softplus(m)
    mu = torch.clamp(sp + 0.5 * S * sig * (1.0 - sig), min=1e-9)
    var = torch.clamp(sig * sig * S, min=1e-9)
    odd = (torch.arange(m.numel()) % 2) == 1
    ma = torch.where(odd, mu, m)
    Sa = torch.where(odd, var, S)
    J = torch.where(odd, sig, torch.ones_like(m))
    return ma.reshape(mz.shape), Sa.reshape(mz.shape), J.reshape(mz.shape)


class OEvenSoftplus(OLayer):
    """layers/even_softplus.py:157-190."""

    def forward(self, mz, Sz):
        ma, Sa, self.J = even_softplus(mz, Sz)
        return ma, Sa

    def backward(self, dm, dS):
        return dm * self.J, dS * self.J * self.J


class OMaxPool2D(OLayer):
    """layers/maxpool2d.py:62-126: window loops; first largest mean wins, a NaN replaces
    the pick; backward adds each delta at its pick."""

    def __init__(self, k, stride, padding):
        self.k, self.s, self.p = k, stride, padding

    def forward(self, ma, Sa):
        N, C, H, W = ma.shape
        k, s, p = self.k, self.s, self.p
        Ho, Wo = (H + 2 * p - k) // s + 1, (W + 2 * p - k) // s + 1
        self.shape = (N, C, H, W)
        flat_m, flat_S = ma.reshape(N, C, H * W), Sa.reshape(N, C, H * W)
        idx = torch.empty(N, C, Ho, Wo, dtype=torch.int64)
        for ho in range(Ho):
            for wo in range(Wo):
                h0, w0 = ho * s - p, wo * s - p
                cand = [(h, w) for h in range(max(h0, 0), min(h0 + k, H)) for w in range(max(w0, 0), min(w0 + k, W))]
                best = torch.full((N, C), -math.inf, dtype=ma.dtype)
                pick = torch.full((N, C), cand[0][0] * W + cand[0][1], dtype=torch.int64)
                for h, w in cand:
                    v = ma[:, :, h, w]
                    take = (v > best) | torch.isnan(v)
                    best = torch.where(take, v, best)
                    pick = torch.where(take, torch.full_like(pick, h * W + w), pick)
                idx[:, :, ho, wo] = pick
        self.idx = idx
        g = idx.reshape(N, C, -1)
        return flat_m.gather(2, g).reshape(N, C, Ho, Wo), flat_S.gather(2, g).reshape(N, C, Ho, Wo)

    def backward(self, dm, dS):
        N, C, H, W = self.shape
        g = self.idx.reshape(N, C, -1)
        om = torch.zeros(N, C, H * W, dtype=dm.dtype).scatter_add_(2, g, dm.reshape(N, C, -1))
        oS = torch.zeros(N, C, H * W, dtype=dS.dtype).scatter_add_(2, g, dS.reshape(N, C, -1))
        return om.reshape(N, C, H, W), oS.reshape(N, C, H, W)


def layernorm_stats(ma, Sa):
    """layers/layernorm.py:117-121: per-row mean, (sum of squared deviations + sum S)/(D-1)."""
    D = ma.shape[-1]
    mu = ma.mean(dim=-1, keepdim=True)
    var = (((ma - mu) ** 2).sum(dim=-1, keepdim=True) + Sa.sum(dim=-1, keepdim=True)) / (D - 1)
    return mu, var


class OLayerNorm(OLayer):
    """layers/layernorm.py:101-175."""

    learnable = True

    def __init__(self, mw, Sw, mb, Sb, eps, has_bias=True):
        self.mw, self.Sw, self.mb, self.Sb, self.eps, self.has_bias = mw, Sw, mb, Sb, eps, has_bias

    def forward(self, ma, Sa):
        D = self.mw.shape[0]
        self.shape = ma.shape
        m, S = ma.reshape(-1, D), Sa.reshape(-1, D)
        self.mu_ra, self.var_ra = layernorm_stats(m, S)
        inv = 1.0 / torch.sqrt(self.var_ra + self.eps)
        d = m - self.mu_ra
        self.m_in, self.inv = m, inv
        mz = inv * d * self.mw + self.mb
        Sz = inv * inv * (S * (self.mw * self.mw + self.Sw) + self.Sw * d * d) + self.Sb
        return mz.reshape(self.shape), Sz.reshape(self.shape)

    def backward(self, dmz, dSz):
        D = self.mw.shape[0]
        dm, dS = dmz.reshape(-1, D), dSz.reshape(-1, D)
        J = self.inv * self.mw
        h = self.inv * (self.m_in - self.mu_ra)
        self.delta_mw = self.Sw * (h * dm).sum(0)
        self.delta_Sw = self.Sw * self.Sw * (h * h * dS).sum(0)
        self.delta_mb = self.Sb * dm.sum(0)
        self.delta_Sb = self.Sb * self.Sb * dS.sum(0)
        return (J * dm).reshape(dmz.shape), (J * J * dS).reshape(dSz.shape)

    def param_groups(self):
        g = [(self, "mw", "Sw", "delta_mw", "delta_Sw")]
        if self.has_bias:
            g.append((self, "mb", "Sb", "delta_mb", "delta_Sb"))
        return g


# ========================================================================== mirror
def mirror(layer, dtype=DT):
    """Oracle copy of an engine (or reference-API) layer, parameters copied to CPU."""
    name = type(layer).__name__
    c = lambda t: _c(t, dtype)  # noqa: E731
    if name == "Linear":
        return OLinear(c(layer.mw), c(layer.Sw), c(layer.mb), c(layer.Sb), layer.has_bias)
    if name == "Conv2D":
        return OConv2D(c(layer.mw), c(layer.Sw), c(layer.mb), c(layer.Sb), layer.C_out, layer.kH, layer.stride,
                       layer.padding, layer.padding_type)
    if name == "BatchNorm2D":
        return OBatchNorm2D(c(layer.mw), c(layer.Sw), c(layer.mb), c(layer.Sb), c(layer.running_mean),
                            c(layer.running_var), layer.momentum, layer.eps, layer.preserve_var,
                            layer._is_initialized, layer.training)
    if name == "ReLU":
        return OReLU()
    if name == "Remax":
        return ORemax()
    if name == "AvgPool2D":
        return OAvgPool2D(layer.k, layer.spatial_correlation)
    if name == "Flatten":
        return OFlatten()
    if name == "ResBlock":
        return OResBlock([mirror(x, dtype) for x in layer._main_layers], [mirror(x, dtype) for x in layer._proj_layers])
    if name == "MultiheadAttentionV2":
        return OMultiheadAttentionV2(mirror(layer.q_proj, dtype), mirror(layer.k_proj, dtype),
                                     mirror(layer.v_proj, dtype), layer.num_heads)
    if name == "RMSNorm":
        return ORMSNorm(c(layer.mw), c(layer.Sw), layer.eps)
    if name == "Embedding":
        return OEmbedding(c(layer.mw), c(layer.Sw), layer.padding_idx)
    if name == "PositionalEncoding":
        return OPositionalEncoding(c(layer.pe_cache))
    if name == "MaxPool2D":
        return OMaxPool2D(layer.kernel_size, layer.stride, layer.padding)
    if name == "LayerNorm":
        return OLayerNorm(c(layer.mw), c(layer.Sw), c(layer.mb), c(layer.Sb), layer.eps, layer.has_bias)
    if name == "EvenSoftplus":
        return OEvenSoftplus()
    raise TypeError(f"no oracle for layer type {name}")


def mirror_net(net, dtype=DT):
    return ONet([mirror(layer, dtype) for layer in net.layers])
