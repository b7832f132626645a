"""Parity of the exact configurations bench.py times.

1. Side stream vs one stream. ``Sequential.step`` runs the large parameter-delta GEMMs on
   a second stream (``overlap_param_deltas``). ResNet-18 at batch 128 and the transformer
   block at batch 64 x sequence 256 are built twice from the same seed and stepped twice
   with the side stream on and off: predictions, every parameter and the BatchNorm
   running statistics must be bit-identical. For the transformer, the one-stream step must
   also equal, bit for bit, the layer-by-layer path that test_gpu_step.py compares with
   the oracle.

2. Teacher-forced oracle comparison of ResNet-18 at batch 128 through ``Sequential.step``
   with the side stream on (network.py:119-152, resblock.py:354-438). Every pass of the
   step is recorded as it runs (the fused conv -> ReLU -> BatchNorm2D passes, the
   BatchNorm2D -> ReLU backward passes, each Conv2D backward, the conv input-delta
   products that carry the BatchNorm2D -> ReLU backward in their epilogue, the head
   layers, the innovation) and counted by kind, so a pass that goes unrecorded fails the
   test; the float64 oracle then recomputes each pass from the GPU's own input to
   that pass, so no error is carried from one layer to the next, and the result is held
   elementwise to |gpu - oracle| <= 1e-6 + 1e-4 * scale, where scale is the sum of the
   absolute values of the terms the oracle adds for that element:
     * products (conv, linear): sum_k |a_k w_k| (+ |bias|, + |addend|);
     * BatchNorm2D outputs: |gamma| (|mu_a| + |mean|) / sigma + |beta| (+ |addend|) for the
       mean; |S_out| + S_gamma ((|mu_a| + |mean|) / sigma)^2 for the variance (the
       normalised mean is a difference of two terms);
     * per-channel / per-weight sums: sum of |terms|; sums of same-sign terms (every
       variance delta is <= 0) and elementwise maps: |oracle|.
   Conv forward and input-delta passes are checked on three whole images of the batch
   (each output depends only on its own image); BatchNorm2D, ReLU, pooling, the head and
   the innovation on the full batch (the folded passes too: their BatchNorm parameter
   deltas sum over every image, so the oracle forms the transposed product of the whole
   batch); Conv2D parameter deltas over the full batch for up to
   96 sampled weight rows (all columns); the capped update of every parameter tensor in
   full. The worst err/bound of every pass is printed.
"""

from __future__ import annotations

import pytest
import torch

from oracle import tagi_oracle as O
from teacher_forcing import ATOL, RTOL, Report, check_attention, d64  # noqa: F401

pytestmark = pytest.mark.gpu

IMAGES = [0, 63, 127]
MAX_ROWS = 96


# ---------------------------------------------------------------------------- part 1
def _state(net, outs):
    """Every tensor a step leaves behind: predictions, parameters, BN running stats."""
    got = []
    for mu, var in outs:
        got += [mu, var]
    for layer in net.layers:
        subs = layer._learnable if hasattr(layer, "_learnable") else [layer]
        for sub in subs:
            if hasattr(sub, "q_proj"):
                subs2 = [sub.q_proj, sub.k_proj, sub.v_proj]
            else:
                subs2 = [sub]
            for s in subs2:
                for name in ("mw", "Sw", "mb", "Sb", "running_mean", "running_var"):
                    t = getattr(s, name, None)
                    if isinstance(t, torch.Tensor):
                        got.append(t)
    return [t.detach().cpu().clone() for t in got]


def _run(name, overlap, steps=2):
    from triton_tagi_amd import _overlap, workloads

    w = workloads.build(name, device="cuda:0")
    w.net.overlap_param_deltas = overlap
    forks = [0]
    orig = _overlap.overlap_param_deltas.fork

    def counting_fork(self, *a):
        forks[0] += 1
        return orig(self, *a)

    _overlap.overlap_param_deltas.fork = counting_fork
    try:
        outs = []
        for _ in range(steps):
            mu, var = w.net.step(w.x, w.y, w.sigma_v)
            outs.append((mu.clone(), var.clone()))
        torch.cuda.synchronize()
    finally:
        _overlap.overlap_param_deltas.fork = orig
    return _state(w.net, outs), forks[0]


@pytest.mark.parametrize("name", ["resnet18", "transformer"])
def test_side_stream_step_equals_one_stream_step(dev, name):
    a, forks_a = _run(name, True)
    b, forks_b = _run(name, False)
    assert forks_a > 0, "the side stream was never used: the test would not cover it"
    assert forks_b == 0
    assert len(a) == len(b)
    bad = [i for i, (x, y) in enumerate(zip(a, b)) if not torch.equal(x, y)]
    assert not bad, f"{name}: {len(bad)} of {len(a)} tensors differ between the two-stream and one-stream steps"


def test_transformer_step_equals_layer_by_layer_path(dev):
    """Sequential.step (one stream) == the per-layer path the oracle step test compares."""
    from test_gpu_step import run_traced

    from triton_tagi_amd import workloads

    w1 = workloads.build("transformer", device="cuda:0")
    w1.net.overlap_param_deltas = False
    mu1, var1 = w1.net.step(w1.x, w1.y, w1.sigma_v)
    torch.cuda.synchronize()
    s1 = _state(w1.net, [(mu1, var1)])
    w2 = workloads.build("transformer", device="cuda:0")
    mu2, var2, _, _ = run_traced(w2.net, w2.x, w2.y, w2.sigma_v)
    s2 = _state(w2.net, [(mu2, var2)])
    bad = [i for i, (x, y) in enumerate(zip(s1, s2)) if not torch.equal(x, y)]
    assert not bad, f"{len(bad)} of {len(s1)} tensors differ between Sequential.step and the per-layer path"


# ---------------------------------------------------------------------------- part 2
def _pads(conv, H, W):
    return O.conv_pads(H, W, conv.kH, conv.stride, conv.padding, conv.padding_type)


def _padded(conv, x):
    p = conv.padding
    if conv.padding_type == 2 and p > 0:
        return torch.nn.functional.pad(x, (0, p, 0, p))
    return torch.nn.functional.pad(x, (p, p, p, p))


def _patch_columns(conv, x, rows):
    """Columns ``rows`` of the patch matrix (pixel rows (n, oh, ow), weight rows (c, kh, kw))
    of the whole batch, taken straight from the padded input."""
    N, C, H, W = x.shape
    k, s = conv.kH, conv.stride
    _, Ho, Wo = _pads(conv, H, W)
    xp = _padded(conv, x)
    cols = []
    for r in rows:
        c, rem = divmod(int(r), k * k)
        kh, kw = divmod(rem, k)
        cols.append(xp[:, c, kh: kh + s * (Ho - 1) + 1: s, kw: kw + s * (Wo - 1) + 1: s].reshape(-1))
    return torch.stack(cols, 1)


def _conv_args(conv, x):
    N, C, H, W = x.shape
    return N, C, H, W, conv.kH, conv.stride, conv.padding, conv.padding_type


def _nchw_rows(t):
    """(N, C, H, W) -> (N*H*W, C), rows (n, h, w)."""
    return t.permute(0, 2, 3, 1).reshape(-1, t.shape[1])


def _rows_nchw(t, N, H, W):
    return t.reshape(N, H, W, -1).permute(0, 3, 1, 2)


def _install(monkeypatch, rec):
    from triton_tagi_amd import network
    from triton_tagi_amd.layers import AvgPool2D, Conv2D, Flatten, Linear, Remax, fused

    cl = lambda t: None if t is None else t.detach().clone()  # noqa: E731
    orig_prep = Conv2D._forward_prepare
    conv_out = {}

    def prep(self, ma, Sa):
        out = orig_prep(self, ma, Sa)
        conv_out[id(self)] = (out[2], out[3])
        return out

    monkeypatch.setattr(Conv2D, "_forward_prepare", prep)

    orig_crb = fused.conv_relu_bn_forward

    def crb(conv, relu, bn, ma, Sa, add=None):
        first = not bn._is_initialized
        out = orig_crb(conv, relu, bn, ma, Sa, add)
        mz, Sz = conv_out[id(conv)]
        rec.append(dict(kind="crb", conv=conv, bn=bn, first=first, ma=cl(ma), Sa=cl(Sa), mz=cl(mz), Sz=cl(Sz),
                        add=None if add is None else (cl(add[0]), cl(add[1])), out=(cl(out[0]), cl(out[1])),
                        J=cl(relu.J), mhat=cl(bn.m_hat), gamma=cl(bn.mw), rmean=cl(bn.running_mean),
                        rvar=cl(bn.running_var)))
        return out

    monkeypatch.setattr(fused, "conv_relu_bn_forward", crb)

    def forbid(*a, **k):
        raise AssertionError("unexpected pass in the ResNet-18 step")

    monkeypatch.setattr(fused, "relu_bn_forward", forbid)

    orig_brb = fused.bn_relu_backward

    def brb(bn, relu, dma, dSa, conv=None):
        out = orig_brb(bn, relu, dma, dSa, conv)
        rec.append(dict(kind="brb", bn=bn, dma=cl(dma), dSa=cl(dSa), out=(cl(out[0]), cl(out[1]))))
        return out

    monkeypatch.setattr(fused, "bn_relu_backward", brb)

    orig_fold = fused.conv_bn_relu_backward

    def fold(conv, bn, relu, conv_prev, dma, dSa):
        out = orig_fold(conv, bn, relu, conv_prev, dma, dSa)
        if out is not None:  # None: the fold declined and the two-step path (recorded above) runs
            rec.append(dict(kind="fold", conv=conv, bn=bn, conv_prev=conv_prev, dmz=cl(dma), dSz=cl(dSa),
                            out=(cl(out[0]), cl(out[1]))))
        return out

    monkeypatch.setattr(fused, "conv_bn_relu_backward", fold)

    orig_xfold = fused.conv_add_bn_relu_backward

    def xfold(conv, dma, dSa, add, bn, relu, conv_prev):
        out = orig_xfold(conv, dma, dSa, add, bn, relu, conv_prev)
        if out is not None:  # None: declined, the block's own passes (recorded above) run
            rec.append(dict(kind="xfold", conv=conv, bn=bn, dmz=cl(dma), dSz=cl(dSa), add=(cl(add[0]), cl(add[1])),
                            out=(cl(out[0][0]), cl(out[0][1])), fout=(cl(out[1][0]), cl(out[1][1]))))
        return out

    monkeypatch.setattr(fused, "conv_add_bn_relu_backward", xfold)

    orig_cb = Conv2D._backward

    def cb(self, dmz, dSz, input_deltas, add=None):
        out = orig_cb(self, dmz, dSz, input_deltas, add)
        rec.append(dict(kind="conv_bwd", conv=self, dmz=cl(dmz), dSz=cl(dSz),
                        add=None if add is None else (cl(add[0]), cl(add[1])),
                        out=None if out is None else (cl(out[0]), cl(out[1]))))
        return out

    monkeypatch.setattr(Conv2D, "_backward", cb)

    for cls in (AvgPool2D, Flatten, Linear, Remax):
        for meth in ("forward", "backward"):
            orig = getattr(cls, meth)

            def wrap(self, a, b, _orig=orig, _meth=meth):
                out = _orig(self, a, b)
                rec.append(dict(kind=_meth, layer=self, a=cl(a), b=cl(b), out=(cl(out[0]), cl(out[1]))))
                return out

            monkeypatch.setattr(cls, meth, wrap)

    orig_inn = network.compute_innovation

    def inn(y, mu, var, sv):
        out = orig_inn(y, mu, var, sv)
        rec.append(dict(kind="innovation", y=cl(y), mu=cl(mu), var=cl(var), sv=sv, out=(cl(out[0]), cl(out[1]))))
        return out

    monkeypatch.setattr(network, "compute_innovation", inn)


def _transposed_product(conv, d, w):
    """The input deltas sum_co d[n, co, oh, ow] * w[(c, kh, kw), co] folded back onto the
    input pixels, over the whole batch: the transposed convolution of ``d`` (NCHW) with the
    weights read as (C_out, C_in, k, k). Stride-1 padding-type-1 convolutions only."""
    assert conv.stride == 1 and conv.padding_type == 1
    k = conv.kH
    wt = w.T.reshape(conv.C_out, conv.C_in, k, k).contiguous()
    return torch.nn.functional.conv_transpose2d(d, wt, stride=1, padding=conv.padding)


def _check_conv_param_deltas(rep, tag, conv, oc, x, dm, dS):
    """delta_mw / delta_Sw on up to MAX_ROWS sampled weight rows (every column) and the bias
    deltas, from the recorded input ``x`` and output deltas (full batch, float64)."""
    Cout = conv.C_out
    K = oc.mw.shape[0]
    gr = torch.Generator().manual_seed(K * 7 + Cout)
    rows = torch.arange(K) if K <= MAX_ROWS else torch.randperm(K, generator=gr)[:MAX_ROWS].sort().values
    Pc = _patch_columns(conv, x, rows)
    dmr, dSr = _nchw_rows(dm), _nchw_rows(dS)
    Sw = oc.Sw[rows]
    rep.check(f"{tag} delta_mw", d64(conv.delta_mw)[rows], Sw * (Pc.T @ dmr), Sw * (Pc.abs().T @ dmr.abs()))
    rep.check(f"{tag} delta_Sw", d64(conv.delta_Sw)[rows], Sw * Sw * ((Pc * Pc).T @ dSr))
    rep.check(f"{tag} delta_mb", conv.delta_mb, oc.Sb * dmr.sum(0, keepdim=True),
              oc.Sb * dmr.abs().sum(0, keepdim=True))
    rep.check(f"{tag} delta_Sb", conv.delta_Sb, oc.Sb ** 2 * dSr.sum(0, keepdim=True))


def _oracle_map(net, onet):
    """id(engine layer) -> oracle mirror (pre-step parameters), through the ResBlocks."""
    m = {}
    for g, o in zip(net.layers, onet.layers):
        m[id(g)] = o
        if hasattr(g, "_main_layers"):
            for gs, os_ in zip(g._main_layers + g._proj_layers, o.main + o.proj):
                m[id(gs)] = os_
    return m


@pytest.mark.timeout(900)
def test_resnet18_b128_step_teacher_forced(dev, monkeypatch):
    from triton_tagi_amd import workloads
    from triton_tagi_amd.layers import BatchNorm2D, Conv2D, Linear

    w = workloads.build("resnet18", device="cuda:0")
    assert w.batch == 128 and w.net.overlap_param_deltas
    onet = O.mirror_net(w.net)
    omap = _oracle_map(w.net, onet)
    rec = []
    _install(monkeypatch, rec)
    mu_pred, var_pred = w.net.step(w.x, w.y, w.sigma_v)
    torch.cuda.synchronize()
    monkeypatch.undo()

    rep = Report()
    cap = O.get_cap_factor(w.batch)
    bn_state = {}  # id(bn) -> oracle forward state (J, sigma, gamma, mhat, |mu_a| + |mean|)
    conv_in = {}  # id(conv) -> recorded input mean (float64, NCHW)
    learn = []  # (tag, engine layer) in order, for the update check
    nconv = nbn = 0
    n_indelta = n_param = n_bnbwd = n_fold = n_xfold = 0  # backward passes by kind
    for r in rec:
        if r["kind"] == "crb":
            conv, bn = r["conv"], r["bn"]
            oc, ob = omap[id(conv)], omap[id(bn)]
            tag = f"conv{nconv} {tuple(r['ma'].shape[1:])}->{conv.C_out}"
            nconv += 1
            learn.append((tag, conv))
            x = d64(r["ma"])
            # the network input reaches the stem without a variance tensor (zero variance)
            assert (r["Sa"] is None) == (nconv == 1), "only the stem takes the zero-variance input"
            xS = torch.zeros_like(x) if r["Sa"] is None else d64(r["Sa"])
            conv_in[id(conv)] = x
            # conv forward on whole images
            xi, xSi = x[IMAGES], xS[IMAGES]
            a = _conv_args(conv, xi)
            P, PS = O.im2col(xi, *a[4:]), O.im2col(xSi, *a[4:])
            rm = P @ oc.mw + oc.mb
            rS = (P * P) @ oc.Sw + PS @ (oc.mw * oc.mw + oc.Sw) + oc.Sb
            sm = P.abs() @ oc.mw.abs() + oc.mb.abs()
            _, Ho, Wo = _pads(conv, x.shape[2], x.shape[3])
            n = len(IMAGES)
            rep.check(f"{tag} fwd mu", d64(r["mz"])[IMAGES], _rows_nchw(rm, n, Ho, Wo), _rows_nchw(sm, n, Ho, Wo))
            rep.check(f"{tag} fwd S", d64(r["Sz"])[IMAGES], _rows_nchw(rS, n, Ho, Wo))
            # ReLU -> BatchNorm2D (+ shortcut) on the full batch, from the GPU's conv output
            mz, Sz = d64(r["mz"]), d64(r["Sz"])
            ra, rSa, rJ = O.relu_moments(mz, Sz)
            mean, var = O.bn_batch_stats(ra, rSa)
            v = lambda t: t.view(1, -1, 1, 1)  # noqa: E731
            nb = mz.shape[0] * mz.shape[2] * mz.shape[3]
            gamma = torch.sqrt(var + ob.eps) if (r["first"] and ob.preserve_var) else ob.mw
            sig = torch.sqrt(v(var) + ob.eps)
            mhat = (ra - v(mean)) / sig
            Shat = rSa / (v(var) + ob.eps)
            mag = (ra.abs() + v(mean).abs()) / sig
            om = v(gamma) * mhat + v(ob.mb)
            oS = v(gamma) ** 2 * Shat + v(ob.Sw) * (mhat * mhat + Shat) + v(ob.Sb)
            sm = v(gamma).abs() * mag + v(ob.mb).abs()
            if r["add"] is not None:
                am, aS = d64(r["add"][0]), d64(r["add"][1])
                om, oS, sm = om + am, oS + aS, sm + am.abs()
            btag = f"bn{nbn} C={mz.shape[1]}"
            nbn += 1
            learn.append((btag, bn))
            rep.check(f"{btag} relu J", r["J"], rJ)
            rep.check(f"{btag} m_hat", r["mhat"], mhat, mag)
            rep.check(f"{btag} out mu" + (" +shortcut" if r["add"] is not None else ""), r["out"][0], om, sm)
            rep.check(f"{btag} out S", r["out"][1], oS, oS.abs() + v(ob.Sw) * mag * mag)
            if r["first"]:
                mean_sq = (ra * ra).mean(dim=(0, 2, 3))
                rep.check(f"{btag} running mean", r["rmean"], mean)
                rep.check(f"{btag} running var", r["rvar"], var,
                          (rSa.mean(dim=(0, 2, 3)) + mean_sq + mean * mean) * (nb / (nb - 1)))
                if ob.preserve_var:
                    rep.check(f"{btag} gamma re-init", r["gamma"], gamma)
            bn_state[id(bn)] = dict(J=rJ, sig=sig, gamma=d64(r["gamma"]), mhat=mhat, mag=mag, ob=ob)
        elif r["kind"] == "brb":
            bn = r["bn"]
            st = bn_state[id(bn)]
            btag = [t for t, lay in learn if lay is bn][0]
            dma, dSa = d64(r["dma"]), d64(r["dSa"])
            v = lambda t: t.view(1, -1, 1, 1)  # noqa: E731
            g = v(st["gamma"])
            rep.check(f"{btag} bwd delta_mu", r["out"][0], dma * g / st["sig"] * st["J"])
            rep.check(f"{btag} bwd delta_S", r["out"][1], dSa * g * g / (st["sig"] ** 2) * st["J"] ** 2)
            ob = st["ob"]
            mh = st["mhat"]
            dims = (0, 2, 3)
            rep.check(f"{btag} delta_gamma", bn.delta_mw, ob.Sw * (dma * mh).sum(dims), ob.Sw * (dma * mh).abs().sum(dims))
            rep.check(f"{btag} delta_S_gamma", bn.delta_Sw, ob.Sw ** 2 * (dSa * mh * mh).sum(dims),
                      ob.Sw ** 2 * (dSa.abs() * st["mag"] ** 2).sum(dims))
            rep.check(f"{btag} delta_beta", bn.delta_mb, ob.Sb * dma.sum(dims), ob.Sb * dma.abs().sum(dims))
            rep.check(f"{btag} delta_S_beta", bn.delta_Sb, ob.Sb ** 2 * dSa.sum(dims))
            n_bnbwd += 1
        elif r["kind"] == "conv_bwd":
            conv = r["conv"]
            oc = omap[id(conv)]
            tag = [t for t, lay in learn if lay is conv][0]
            x = conv_in[id(conv)]
            dm, dS = d64(r["dmz"]), d64(r["dSz"])
            if r["out"] is not None:
                a = _conv_args(conv, x[IMAGES])
                dmi, dSi = _nchw_rows(dm[IMAGES]), _nchw_rows(dS[IMAGES])
                qm = O.col2im(dmi @ oc.mw.T, *a)
                qS = O.col2im(dSi @ (oc.mw * oc.mw).T, *a)
                sm = O.col2im(dmi.abs() @ oc.mw.abs().T, *a)
                if r["add"] is not None:
                    am, aS = d64(r["add"][0])[IMAGES], d64(r["add"][1])[IMAGES]
                    qm, qS, sm = qm + am, qS + aS, sm + am.abs()
                sfx = " +shortcut" if r["add"] is not None else ""
                rep.check(f"{tag} bwd delta_mu{sfx}", d64(r["out"][0])[IMAGES], qm, sm)
                rep.check(f"{tag} bwd delta_S{sfx}", d64(r["out"][1])[IMAGES], qS)
            _check_conv_param_deltas(rep, tag, conv, oc, x, dm, dS)
            n_param += 1
            n_indelta += r["out"] is not None
        elif r["kind"] == "fold":
            # conv's input-delta product with the BatchNorm2D -> ReLU backward of the pair in
            # front of it in the epilogue: the deltas at the BatchNorm output exist only in
            # registers, so the oracle forms them from the GPU's deltas at conv's output, over
            # the whole batch (the BatchNorm parameter deltas sum over every image)
            conv, bn = r["conv"], r["bn"]
            oc = omap[id(conv)]
            tag = [t for t, lay in learn if lay is conv][0]
            btag = [t for t, lay in learn if lay is bn][0]
            st = bn_state[id(bn)]
            x = conv_in[id(conv)]
            dm, dS = d64(r["dmz"]), d64(r["dSz"])
            q = _transposed_product(conv, dm, oc.mw)
            qS = _transposed_product(conv, dS, oc.mw * oc.mw)
            sq = _transposed_product(conv, dm.abs(), oc.mw.abs())
            # the transposed convolution is the oracle's patch product folded back (col2im)
            a = _conv_args(conv, x[IMAGES])
            ref_i = O.col2im(_nchw_rows(dm[IMAGES]) @ oc.mw.T, *a)
            assert torch.allclose(q[IMAGES], ref_i, rtol=1e-12, atol=1e-15), "transposed product != col2im"
            v = lambda t: t.view(1, -1, 1, 1)  # noqa: E731
            g = v(st["gamma"])
            fm, fS = g / st["sig"] * st["J"], (g / st["sig"]) ** 2 * st["J"] ** 2
            rep.check(f"{tag}+{btag} folded bwd delta_mu", r["out"][0], q * fm, sq * fm.abs())
            rep.check(f"{tag}+{btag} folded bwd delta_S", r["out"][1], qS * fS)
            ob, mh, dims = st["ob"], st["mhat"], (0, 2, 3)
            rep.check(f"{btag} (folded) delta_gamma", bn.delta_mw, ob.Sw * (q * mh).sum(dims),
                      ob.Sw * (sq * st["mag"]).sum(dims))
            rep.check(f"{btag} (folded) delta_S_gamma", bn.delta_Sw, ob.Sw ** 2 * (qS * mh * mh).sum(dims),
                      ob.Sw ** 2 * (qS.abs() * st["mag"] ** 2).sum(dims))
            rep.check(f"{btag} (folded) delta_beta", bn.delta_mb, ob.Sb * q.sum(dims), ob.Sb * sq.sum(dims))
            rep.check(f"{btag} (folded) delta_S_beta", bn.delta_Sb, ob.Sb ** 2 * qS.sum(dims))
            _check_conv_param_deltas(rep, f"{tag} (folded)", conv, oc, x, dm, dS)
            n_fold += 1
            n_param += 1
            n_indelta += 1
            n_bnbwd += 1
        elif r["kind"] == "xfold":
            # a block's first convolution: its input deltas plus the shortcut's (stored: the
            # block in front reads them through its own shortcut), then, in the same
            # epilogue, the BatchNorm2D -> ReLU backward of the pair in front of the block
            # (the previous block's closing pair, or the stem's), over the whole batch
            conv, bn = r["conv"], r["bn"]
            oc = omap[id(conv)]
            tag = [t for t, lay in learn if lay is conv][0]
            btag = [t for t, lay in learn if lay is bn][0]
            st = bn_state[id(bn)]
            x = conv_in[id(conv)]
            dm, dS = d64(r["dmz"]), d64(r["dSz"])
            am, aS = d64(r["add"][0]), d64(r["add"][1])
            q = _transposed_product(conv, dm, oc.mw) + am
            qS = _transposed_product(conv, dS, oc.mw * oc.mw) + aS
            sq = _transposed_product(conv, dm.abs(), oc.mw.abs()) + am.abs()
            rep.check(f"{tag} bwd delta_mu +shortcut (stored by the fold)", r["out"][0], q, sq)
            rep.check(f"{tag} bwd delta_S +shortcut (stored by the fold)", r["out"][1], qS)
            v = lambda t: t.view(1, -1, 1, 1)  # noqa: E731
            g = v(st["gamma"])
            fm, fS = g / st["sig"] * st["J"], (g / st["sig"]) ** 2 * st["J"] ** 2
            rep.check(f"{tag}+{btag} folded bwd delta_mu", r["fout"][0], q * fm, sq * fm.abs())
            rep.check(f"{tag}+{btag} folded bwd delta_S", r["fout"][1], qS * fS)
            ob, mh, dims = st["ob"], st["mhat"], (0, 2, 3)
            rep.check(f"{btag} (folded) delta_gamma", bn.delta_mw, ob.Sw * (q * mh).sum(dims),
                      ob.Sw * (sq * st["mag"]).sum(dims))
            rep.check(f"{btag} (folded) delta_S_gamma", bn.delta_Sw, ob.Sw ** 2 * (qS * mh * mh).sum(dims),
                      ob.Sw ** 2 * (qS.abs() * st["mag"] ** 2).sum(dims))
            rep.check(f"{btag} (folded) delta_beta", bn.delta_mb, ob.Sb * q.sum(dims), ob.Sb * sq.sum(dims))
            rep.check(f"{btag} (folded) delta_S_beta", bn.delta_Sb, ob.Sb ** 2 * qS.sum(dims))
            _check_conv_param_deltas(rep, f"{tag} (folded)", conv, oc, x, dm, dS)
            n_xfold += 1
            n_param += 1
            n_indelta += 1
            n_bnbwd += 1
        elif r["kind"] in ("forward", "backward"):
            layer = r["layer"]
            name = type(layer).__name__
            a, b = d64(r["a"]), d64(r["b"])
            tag = f"{name} {r['kind']}"
            if name == "Flatten":
                assert torch.equal(d64(r["out"][0]), a.reshape(r["out"][0].shape))
                assert torch.equal(d64(r["out"][1]), b.reshape(r["out"][1].shape))
            elif name == "AvgPool2D":
                op = O.OAvgPool2D(layer.k, layer.spatial_correlation)
                if r["kind"] == "forward":
                    rm, rS = op.forward(a, b)
                    sm, _ = op.forward(a.abs(), b)
                    rep.check(f"{tag} mu", r["out"][0], rm, sm)
                    rep.check(f"{tag} S", r["out"][1], rS)
                else:
                    op.input_shape = layer.input_shape
                    rm, rS = op.backward(a, b)
                    rep.check(f"{tag} delta_mu", r["out"][0], rm)
                    rep.check(f"{tag} delta_S", r["out"][1], rS)
            elif name == "Linear":
                ol = omap[id(layer)]
                if r["kind"] == "forward":
                    learn.append(("fc", layer))
                    ol.a_in = a
                    rm, rS = O.linear_moments(a, b, ol.mw, ol.Sw, ol.mb, ol.Sb)
                    rep.check(f"{tag} mu", r["out"][0], rm, a.abs() @ ol.mw.abs() + ol.mb.abs())
                    rep.check(f"{tag} S", r["out"][1], rS)
                else:
                    qm, qS = O.linear_backward_delta(a, b, ol.mw)
                    rep.check(f"{tag} delta_mu", r["out"][0], qm, a.abs() @ ol.mw.abs().T)
                    rep.check(f"{tag} delta_S", r["out"][1], qS)
                    x = ol.a_in
                    rep.check("fc delta_mw", layer.delta_mw, ol.Sw * (x.T @ a), ol.Sw * (x.abs().T @ a.abs()))
                    rep.check("fc delta_Sw", layer.delta_Sw, ol.Sw ** 2 * ((x * x).T @ b))
                    rep.check("fc delta_mb", layer.delta_mb, ol.Sb * a.sum(0, keepdim=True),
                              ol.Sb * a.abs().sum(0, keepdim=True))
                    rep.check("fc delta_Sb", layer.delta_Sb, ol.Sb ** 2 * b.sum(0, keepdim=True))
            elif name == "Remax":
                if r["kind"] == "forward":
                    rm, rS, rJ = O.remax_moments(a, b)
                    remax_J = rJ
                    rep.check(f"{tag} mu", r["out"][0], rm)
                    rep.check(f"{tag} S", r["out"][1], rS)
                    rep.check(f"{tag} J", layer.J, rJ)
                    assert torch.equal(r["out"][0].cpu(), mu_pred.cpu())
                    assert torch.equal(r["out"][0].argmax(-1).cpu(), rm.argmax(-1))
                else:
                    rep.check(f"{tag} delta_mu", r["out"][0], a * remax_J)
                    rep.check(f"{tag} delta_S", r["out"][1], b * remax_J ** 2)
        elif r["kind"] == "innovation":
            y, mu, var = d64(r["y"]), d64(r["mu"]), d64(r["var"])
            qm, qS = O.innovation(y, mu, var, r["sv"])
            rep.check("innovation delta_mu", r["out"][0], qm, (y.abs() + mu.abs()) / (var + r["sv"] ** 2))
            rep.check("innovation delta_S", r["out"][1], qS)
    # every pass of the step was recorded and checked: 20 convolutions and 20 BatchNorm2D
    # layers forward; backward, every conv's parameter deltas, the input deltas of all but
    # the stem (the first layer forms none), every BatchNorm2D backward (two-step or folded)
    print(f"\npasses: {nconv} conv forward, {nbn} BatchNorm2D forward, {n_param} conv parameter-delta, "
          f"{n_indelta} conv input-delta ({n_fold} with the BatchNorm2D -> ReLU backward folded in, {n_xfold} "
          f"with the shortcut added and the previous block's or the stem's folded in), "
          f"{n_bnbwd} BatchNorm2D backward")
    assert nconv == 20 and nbn == 20
    assert n_param == 20 and n_indelta == 19 and n_bnbwd == 20
    assert n_fold > 0, "the folded BatchNorm2D backward never ran: the test would not cover it"
    assert n_xfold > 0, "the fold across a block boundary never ran: the test would not cover it"

    # capped update of every parameter tensor from its pre-step value and the GPU's deltas
    for tag, layer in learn:
        ol = omap[id(layer)]
        pre_m = {"mw": ol.mw, "mb": ol.mb}
        if isinstance(layer, BatchNorm2D):
            pre_m["mw"] = bn_state[id(layer)]["gamma"]
        for mname, Sname, dmn, dSn in (("mw", "Sw", "delta_mw", "delta_Sw"), ("mb", "Sb", "delta_mb", "delta_Sb")):
            m0 = pre_m[mname].reshape(getattr(layer, mname).shape)
            S0 = getattr(ol, Sname).reshape(m0.shape)
            dmv, dSv = d64(getattr(layer, dmn)).reshape(m0.shape), d64(getattr(layer, dSn)).reshape(m0.shape)
            um, uS = O.capped_update(m0, S0, dmv, dSv, cap)
            rep.check(f"{tag} updated {mname}", getattr(layer, mname), um, m0.abs() + (um - m0).abs())
            rep.check(f"{tag} updated {Sname}", getattr(layer, Sname), uS, S0.abs() + (uS - S0).abs())
    assert isinstance(w.net.layers[0], Conv2D) and isinstance(w.net.layers[-2], Linear)
    rep.finish()


# ---------------------------------------------------------------------------- part 3
def _install_transformer(monkeypatch, rec):
    from triton_tagi_amd import network
    from triton_tagi_amd.layers import Embedding, Linear, MultiheadAttentionV2, PositionalEncoding, RMSNorm
    from triton_tagi_amd.layers import multihead_attention as mha_mod

    cl = lambda t: None if t is None else t.detach().clone()  # noqa: E731
    for cls in (Embedding, PositionalEncoding, RMSNorm, Linear):
        for meth in ("forward", "backward"):
            orig = getattr(cls, meth)

            def wrap(self, a, b, _orig=orig, _meth=meth):
                out = _orig(self, a, b)
                rec.append(dict(kind=_meth, layer=self, a=cl(a), b=cl(b), out=(cl(out[0]), cl(out[1]))))
                return out

            monkeypatch.setattr(cls, meth, wrap)
    # the step's first layer forms only its parameter deltas (the token ids take none)
    orig_pd = Embedding.backward_param_deltas

    def emb_param_deltas(self, a, b):
        out = orig_pd(self, a, b)
        rec.append(dict(kind="backward_param_deltas", layer=self, a=cl(a), b=cl(b), out=None))
        return out

    monkeypatch.setattr(Embedding, "backward_param_deltas", emb_param_deltas)

    orig_f = MultiheadAttentionV2.forward

    def mha_forward(self, ma, Sa):
        out = orig_f(self, ma, Sa)
        src = self._attn_src
        assert src is not None, "the fused attention forward did not run at the benchmarked shape"
        rec.append(dict(kind="mha_forward", layer=self, ma=cl(ma), Sa=cl(Sa), qkv_m=cl(src[0]), qkv_S=cl(src[1]),
                        mu_a=cl(self._cache["mu_score"]), J=cl(self._cache["jcb"]), out=(cl(out[0]), cl(out[1]))))
        return out

    monkeypatch.setattr(MultiheadAttentionV2, "forward", mha_forward)

    seen = {}
    orig_delta = mha_mod.fused_backward_delta

    def delta(dmz, dSz, mw, add=None):  # the summed input deltas of the three projections
        seen["dqkv"] = (cl(dmz), cl(dSz))
        return orig_delta(dmz, dSz, mw, add)

    monkeypatch.setattr(mha_mod, "fused_backward_delta", delta)
    orig_b = MultiheadAttentionV2.backward

    def mha_backward(self, dm, dS):
        seen.clear()
        out = orig_b(self, dm, dS)
        rec.append(dict(kind="mha_backward", layer=self, d_m=cl(dm), d_S=cl(dS), dqkv=seen["dqkv"],
                        out=(cl(out[0]), cl(out[1]))))
        return out

    monkeypatch.setattr(MultiheadAttentionV2, "backward", mha_backward)

    orig_inn = network.compute_innovation

    def inn(y, mu, var, sv):
        out = orig_inn(y, mu, var, sv)
        rec.append(dict(kind="innovation", y=cl(y), mu=cl(mu), var=cl(var), sv=sv, out=(cl(out[0]), cl(out[1]))))
        return out

    monkeypatch.setattr(network, "compute_innovation", inn)


@pytest.mark.timeout(900)
def test_transformer_b64_s256_step_teacher_forced(dev, monkeypatch):
    """The transformer block (Embedding -> PositionalEncoding -> MultiheadAttentionV2 ->
    RMSNorm -> Linear) at batch 64 x sequence 256 through ``Sequential.step`` with the side
    stream on, teacher forced: every pass recorded, recomputed by the float64 oracle from
    the GPU's own input to it and held to the per-element bar (teacher_forcing.py)."""
    from triton_tagi_amd import _overlap, workloads
    from triton_tagi_amd.layers import Embedding, Linear, MultiheadAttentionV2, PositionalEncoding, RMSNorm

    w = workloads.build("transformer", device="cuda:0")
    assert w.batch == 64 and w.net.overlap_param_deltas
    emb, pe, att, rms, head = w.net.layers
    assert (isinstance(emb, Embedding) and isinstance(pe, PositionalEncoding) and isinstance(att, MultiheadAttentionV2)
            and isinstance(rms, RMSNorm) and isinstance(head, Linear))
    onet = O.mirror_net(w.net)
    oemb, ope, oatt, orms, ohead = onet.layers
    rec = []
    forks = [0]
    orig_fork = _overlap.overlap_param_deltas.fork

    def counting_fork(self, *a):
        forks[0] += 1
        return orig_fork(self, *a)

    _install_transformer(monkeypatch, rec)
    monkeypatch.setattr(_overlap.overlap_param_deltas, "fork", counting_fork)
    w.net.step(w.x, w.y, w.sigma_v)
    torch.cuda.synchronize()
    monkeypatch.undo()
    assert forks[0] > 0, "the side stream was never used: the test would not cover the overlapped step"
    var_a = att.get_attention_scores()[1]  # rebuilt from the recorded projections (the fused kernel's values)
    torch.cuda.synchronize()

    rep = Report()
    kinds = [(r["kind"], type(r.get("layer")).__name__) for r in rec]
    expect = [("forward", "Embedding"), ("forward", "PositionalEncoding"), ("mha_forward", "MultiheadAttentionV2"),
              ("forward", "RMSNorm"), ("forward", "Linear"), ("innovation", "NoneType"), ("backward", "Linear"),
              ("backward", "RMSNorm"), ("mha_backward", "MultiheadAttentionV2"), ("backward", "PositionalEncoding"),
              ("backward_param_deltas", "Embedding")]
    assert kinds == expect, f"passes of the step: {kinds}"
    f_emb, f_pe, f_att, f_rms, f_head, r_inn, b_head, b_rms, b_att, b_pe, b_emb = rec
    D = emb.embedding_dim

    # Embedding forward: a gather (embedding.py:88-106)
    cat = d64(f_emb["a"]).long()
    assert torch.equal(d64(f_emb["out"][0]), oemb.mw[cat]) and torch.equal(d64(f_emb["out"][1]), oemb.Sw[cat])
    # PositionalEncoding forward (positional_encoding.py:59-63)
    a = d64(f_pe["a"])
    pe_rows = ope.pe[: a.shape[-2]]
    rep.check("PositionalEncoding fwd mu", f_pe["out"][0], a + pe_rows, a.abs() + pe_rows.abs())
    assert torch.equal(f_pe["out"][1], f_pe["b"])
    # attention, stage by stage
    projs = (oatt.q, oatt.k, oatt.v)
    check_attention(rep, "attention", dict(
        H=att.num_heads, ma=f_att["ma"], Sa=f_att["Sa"], w_m=torch.cat([p.mw for p in projs], 1),
        w_S=torch.cat([p.Sw for p in projs], 1), qkv_m=f_att["qkv_m"], qkv_S=f_att["qkv_S"], mu_a=f_att["mu_a"],
        var_a=var_a, J=f_att["J"], out_m=f_att["out"][0], out_S=f_att["out"][1], d_m=b_att["d_m"], d_S=b_att["d_S"],
        dqkv_m=b_att["dqkv"][0], dqkv_S=b_att["dqkv"][1], dma=b_att["out"][0], dSa=b_att["out"][1],
        pd=[(p.delta_mw, p.delta_Sw) for p in (att.q_proj, att.k_proj, att.v_proj)], Sw_qkv=[p.Sw for p in projs]))
    # RMSNorm forward (rms_norm.py:93-110): products of same-sign factors, no cancellation
    a, b = d64(f_rms["a"]).reshape(-1, D), d64(f_rms["b"]).reshape(-1, D)
    inv = 1.0 / torch.sqrt((a * a + b).mean(1, keepdim=True) + orms.eps)
    g, Sg = orms.mw, orms.Sw
    rep.check("RMSNorm fwd mu", f_rms["out"][0].reshape(-1, D), inv * a * g)
    rep.check("RMSNorm fwd S", f_rms["out"][1].reshape(-1, D), inv * inv * (b * (g * g + Sg) + Sg * a * a))
    # head Linear forward (linear.py:83-103)
    a, b = d64(f_head["a"]).reshape(-1, D), d64(f_head["b"]).reshape(-1, D)
    rm, rS = O.linear_moments(a, b, ohead.mw, ohead.Sw, ohead.mb, ohead.Sb)
    rep.check("head Linear fwd mu", f_head["out"][0].reshape(rm.shape), rm, a.abs() @ ohead.mw.abs() + ohead.mb.abs())
    rep.check("head Linear fwd S", f_head["out"][1].reshape(rS.shape), rS)
    x_head = a
    # innovation (observation.py:24-46)
    y, mu, var = d64(r_inn["y"]), d64(r_inn["mu"]), d64(r_inn["var"])
    qm, qS = O.innovation(y, mu, var, r_inn["sv"])
    rep.check("innovation delta_mu", r_inn["out"][0], qm, (y.abs() + mu.abs()) / (var + r_inn["sv"] ** 2))
    rep.check("innovation delta_S", r_inn["out"][1], qS)
    # head Linear backward (linear.py:108-156)
    N = ohead.mw.shape[1]
    dm, dS = d64(b_head["a"]).reshape(-1, N), d64(b_head["b"]).reshape(-1, N)
    qm, qS = O.linear_backward_delta(dm, dS, ohead.mw)
    rep.check("head Linear bwd delta_mu", b_head["out"][0].reshape(qm.shape), qm, dm.abs() @ ohead.mw.abs().T)
    rep.check("head Linear bwd delta_S", b_head["out"][1].reshape(qS.shape), qS)
    rep.check("head delta_mw", head.delta_mw, ohead.Sw * (x_head.T @ dm), ohead.Sw * (x_head.abs().T @ dm.abs()))
    rep.check("head delta_Sw", head.delta_Sw, ohead.Sw ** 2 * ((x_head * x_head).T @ dS))
    rep.check("head delta_mb", head.delta_mb, ohead.Sb * dm.sum(0, keepdim=True),
              ohead.Sb * dm.abs().sum(0, keepdim=True))
    rep.check("head delta_Sb", head.delta_Sb, ohead.Sb ** 2 * dS.sum(0, keepdim=True))
    # RMSNorm backward (rms_norm.py:112-140), from the forward's input
    a = d64(f_rms["a"]).reshape(-1, D)
    dm, dS = d64(b_rms["a"]).reshape(-1, D), d64(b_rms["b"]).reshape(-1, D)
    t = inv * g
    rep.check("RMSNorm bwd delta_mu", b_rms["out"][0].reshape(-1, D), t * dm)
    rep.check("RMSNorm bwd delta_S", b_rms["out"][1].reshape(-1, D), t * t * dS)
    rep.check("RMSNorm delta_mw", rms.delta_mw, Sg * (inv * a * dm).sum(0), Sg * (inv * a * dm).abs().sum(0))
    rep.check("RMSNorm delta_Sw", rms.delta_Sw, Sg * Sg * (inv * inv * a * a * dS).sum(0))
    # PositionalEncoding backward: identity (positional_encoding.py:65-68)
    assert torch.equal(b_pe["out"][0], b_pe["a"]) and torch.equal(b_pe["out"][1], b_pe["b"])
    # Embedding backward (embedding.py:108-157): per category, Sw-weighted sums of the deltas
    dm, dS = d64(b_emb["a"]).reshape(-1, D), d64(b_emb["b"]).reshape(-1, D)
    flat = cat.reshape(-1)
    V = oemb.mw.shape[0]
    sum_m = torch.zeros(V, D, dtype=torch.float64).index_add_(0, flat, dm)
    sum_abs = torch.zeros(V, D, dtype=torch.float64).index_add_(0, flat, dm.abs())
    sum_S = torch.zeros(V, D, dtype=torch.float64).index_add_(0, flat, dS)
    rep.check("Embedding delta_mw", emb.delta_mw, oemb.Sw * sum_m, oemb.Sw * sum_abs)
    rep.check("Embedding delta_Sw", emb.delta_Sw, oemb.Sw ** 2 * sum_S)
    assert b_emb["out"] is None  # no deltas for the token ids

    # capped update of every parameter tensor from its pre-step value and the GPU's deltas
    cap = O.get_cap_factor(w.batch)
    groups = [("Embedding", emb, oemb, ("mw",)), ("q_proj", att.q_proj, oatt.q, ("mw",)),
              ("k_proj", att.k_proj, oatt.k, ("mw",)), ("v_proj", att.v_proj, oatt.v, ("mw",)),
              ("RMSNorm", rms, orms, ("mw",)), ("head", head, ohead, ("mw", "mb"))]
    for tag, layer, ol, means in groups:
        for mname in means:
            Sname, dmn, dSn = "S" + mname[1:], "delta_" + mname, "delta_S" + mname[1:]
            m0, S0 = getattr(ol, mname), getattr(ol, Sname)
            dmv, dSv = d64(getattr(layer, dmn)).reshape(m0.shape), d64(getattr(layer, dSn)).reshape(m0.shape)
            um, uS = O.capped_update(m0, S0, dmv, dSv, cap)
            rep.check(f"{tag} updated {mname}", getattr(layer, mname), um, m0.abs() + (um - m0).abs())
            rep.check(f"{tag} updated {Sname}", getattr(layer, Sname), uS, S0.abs() + (uS - S0).abs())
    rep.finish()
