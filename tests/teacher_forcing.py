"""Teacher-forced comparison against the float64 oracle: shared by the step-level tests.

A step is recorded as it runs on the GPU; the oracle then recomputes every pass from the
GPU's own input to that pass, so no error is carried from one pass to the next, and each
result is held elementwise to |gpu - oracle| <= 1e-6 + 1e-4 * scale. ``scale`` is the sum
of the absolute values of the terms the oracle adds for that element where the terms
can cancel (products, per-column sums, normalised means), and |oracle| for sums of
same-sign terms and elementwise maps: fp32 rounding is relative to the terms, not to a
result that cancels towards zero.

``check_attention`` does this for MultiheadAttentionV2 (multihead_attention.py:154-268)
stage by stage: the Q/K/V product, the score product, the Remax, the score @ V product,
the value, query and key deltas, the summed input deltas and the projections' parameter
deltas. Where the engine runs several stages in one kernel (scores, Remax and score @ V
in ``tagi_attn_fwd``; score deltas and the query / key product in
``tagi_attn_score_deltas_qk``) the intermediate is not in memory: the scores the Remax
reads are re-formed on the GPU by the two-call product, and the test asserts that the
Remax of those scores is the fused kernel's output bit for bit (so they are the values
the fused kernel read); the score deltas exist only as a term of the oracle's query /
key products, which are compared with the fused kernel's outputs.
"""

from __future__ import annotations

import math

import torch

from oracle import tagi_oracle as O

RTOL, ATOL = 1e-4, 1e-6


def d64(t):
    return t.detach().to("cpu", torch.float64).contiguous()


class Report:
    """Collects (pass, worst err/bound) rows; ``finish`` prints the table and fails on any
    element out of tolerance."""

    def __init__(self):
        self.rows = []

    def check(self, tag, got, ref, scale=None):
        got = d64(got)
        ref = ref.to(torch.float64)
        assert got.shape == ref.shape, f"{tag}: shape {tuple(got.shape)} vs {tuple(ref.shape)}"
        sc = ref.abs() if scale is None else scale.abs()
        bound = ATOL + RTOL * sc
        r = ((got - ref).abs() / bound).reshape(-1)
        r = torch.nan_to_num(r, nan=math.inf)
        i = int(torch.argmax(r))
        self.rows.append((tag, float(r[i]), int((r > 1).sum()), r.numel(), float(got.reshape(-1)[i]),
                          float(ref.reshape(-1)[i]), float(sc.reshape(-1)[i])))

    def merge(self, tag, parts):
        """One row for a pass checked in chunks: ``parts`` are (worst, over, n, got, ref, sc)."""
        worst = max(parts, key=lambda p: p[0])
        self.rows.append((tag, worst[0], sum(p[1] for p in parts), sum(p[2] for p in parts), *worst[3:]))

    def finish(self):
        w = max(len(t[0]) for t in self.rows)
        print(f"\n{'pass':<{w}}  worst err/bound   over  elements")
        for tag, worst, over, n, *_ in self.rows:
            print(f"{tag:<{w}}  {worst:15.3e}  {over:5d}  {n:9d}")
        bad = [t for t in self.rows if t[1] > 1.0]
        assert not bad, "out of tolerance:\n" + "\n".join(
            f"{t[0]}: {t[2]}/{t[3]} elements, worst err/bound {t[1]:.3g} (got {t[4]:.9g} ref {t[5]:.9g} "
            f"scale {t[6]:.3g})" for t in bad)


class _Chunked:
    """Accumulates the rows of one pass over several chunks into a single report row."""

    def __init__(self, rep):
        self.rep = rep
        self.parts: dict[str, list] = {}

    def check(self, tag, got, ref, scale=None):
        sub = Report()
        sub.check(tag, got, ref, scale)
        self.parts.setdefault(tag, []).append(sub.rows[0][1:])

    def flush(self):
        for tag, parts in self.parts.items():
            self.rep.merge(tag, parts)


def gpu_scores(qkv_m, qkv_S, B, H, S, D):
    """The fp32 score moments of every head, formed on the GPU by the two-call product
    (``tagi_bmm_tagi``, the fused forward kernel's product order): (B, H, S, S) each."""
    from triton_tagi_amd import _lib

    E = H * D
    L = 3 * E
    dev = qkv_m.device
    s = 1.0 / math.sqrt(D)
    mu = torch.empty(B, H, S, S, device=dev)
    var = torch.empty_like(mu)
    q_m, q_S = qkv_m.data_ptr(), qkv_S.data_ptr()
    _lib.call("tagi_bmm_tagi", q_m, q_S, q_m + 4 * E, q_S + 4 * E, mu.data_ptr(), var.data_ptr(), B * H, S, D, S,
              _lib.view(H, S * L, D, L, 1), _lib.view(H, S * L, D, 1, L), _lib.view(1, S * S, 0, S, 1), s, s * s,
              _lib.stream_of(qkv_m))
    return mu, var


def check_attention(rep, tag, a):
    """Stage-by-stage oracle check of one MultiheadAttentionV2 forward and backward.

    ``a`` holds, as recorded on the GPU (B batch, S sequence, E = H D model width):
      ma, Sa (B, S, E) input; w_m, w_S (E, 3E) float64 pre-step q | k | v weights (no bias);
      qkv_m, qkv_S (B S, 3E) projections; mu_a, var_a, J (B, H, S, S) Remax outputs (var_a
      from get_attention_scores); out_m, out_S (B, S, E); d_m, d_S (B, S, E) output deltas;
      dqkv_m, dqkv_S (B S, 3E) projection output deltas; dma, dSa (B, S, E) input deltas;
      pd: [(delta_mw, delta_Sw)] of the q, k, v projections; Sw_qkv: [Sw] float64 pre-step.
    """
    B, S, E = a["ma"].shape
    H = a["H"]
    D = E // H
    s = 1.0 / math.sqrt(D)
    L = 3 * E
    x, xS = d64(a["ma"]).reshape(B * S, E), d64(a["Sa"]).reshape(B * S, E)
    w_m, w_S = a["w_m"], a["w_S"]
    # Q/K/V product (multihead_attention.py:160-172; linear.py:99-100)
    rm, rS = O.linear_moments(x, xS, w_m, w_S, 0.0, 0.0)
    rep.check(f"{tag} q|k|v product mu", a["qkv_m"], rm, x.abs() @ w_m.abs())
    rep.check(f"{tag} q|k|v product S", a["qkv_S"], rS)
    # the scores the fused kernel read: the two-call product's, bit for bit (their Remax is
    # the fused output bit for bit); checked against the oracle's product of the GPU's q, k
    z_m, z_S = gpu_scores(a["qkv_m"], a["qkv_S"], B, H, S, D)
    from triton_tagi_amd.layers.remax import remax

    tm, tS, tJ = remax(z_m.view(-1, S), z_S.view(-1, S))
    assert torch.equal(tm.view(B, H, S, S), a["mu_a"]), "Remax of the two-call scores != fused forward mu_a"
    assert torch.equal(tJ.view(B, H, S, S), a["J"]), "Remax of the two-call scores != fused forward J"
    assert torch.equal(tS.view(B, H, S, S), a["var_a"]), "Remax of the two-call scores != rebuilt var_a"
    del tm, tS, tJ
    qkv, qkvS = d64(a["qkv_m"]), d64(a["qkv_S"])

    def heads(t, j, nb):  # block j (q, k, v) of (nb S, 3E) rows as (nb, H, S, D)
        return t[:, j * E:(j + 1) * E].reshape(nb, S, H, D).transpose(1, 2)

    dmo, dSo = d64(a["d_m"]), d64(a["d_S"])
    dq_all = d64(a["dqkv_m"])
    dqS_all = d64(a["dqkv_S"])
    ck = _Chunked(rep)
    step = max(1, 8 * 8 * 256 * 256 // (H * S * S))  # batches per chunk: bounded float64 memory
    for b0 in range(0, B, step):
        sl = slice(b0, min(B, b0 + step))
        nb = sl.stop - sl.start
        rows = slice(sl.start * S, sl.stop * S)
        mq, mk, mv = (heads(qkv[rows], j, nb) for j in range(3))
        vq, vk, vv = (heads(qkvS[rows], j, nb) for j in range(3))
        # scores (multihead_attention.py:176-183, attention.py:66-131)
        om, oS = O.bmm_tagi(mq, vq, mk.transpose(-1, -2), vk.transpose(-1, -2), s)
        ck.check(f"{tag} scores mu", z_m[sl], om, s * (mq.abs() @ mk.abs().transpose(-1, -2)))
        ck.check(f"{tag} scores S", z_S[sl], oS)
        # Remax of the scores the kernel read (remax.py:59-109)
        ra, rSa, rJ = O.remax_moments(d64(z_m[sl]), d64(z_S[sl]))
        ck.check(f"{tag} Remax mu_a", a["mu_a"][sl], ra)
        ck.check(f"{tag} Remax S_a", a["var_a"][sl], rSa)
        ck.check(f"{tag} Remax J", a["J"][sl], rJ)
        del om, oS, ra, rSa, rJ
        # score @ V from the GPU's Remax outputs (multihead_attention.py:188-196)
        pa, pSa, pJ = d64(a["mu_a"][sl]), d64(a["var_a"][sl]), d64(a["J"][sl])
        om, oS = O.bmm_tagi(pa, pSa, mv, vv, 1.0)
        unh = lambda t: t.transpose(1, 2).reshape(nb, S, E)  # noqa: E731
        ck.check(f"{tag} out mu", a["out_m"][sl], unh(om), unh(pa @ mv.abs()))
        ck.check(f"{tag} out S", a["out_S"][sl], unh(oS))
        # backward (multihead_attention.py:233-260, attention.py:215-374)
        hd = lambda t: t.reshape(nb, S, H, D).transpose(1, 2)  # noqa: E731
        dm, dS = hd(dmo[sl]), hd(dSo[sl])
        gV, gSV = O.bmm_shared_left(pa.transpose(-1, -2), dm, dS)
        ck.check(f"{tag} delta V mu", heads(dq_all[rows], 2, nb), gV, pa.transpose(-1, -2) @ dm.abs())
        ck.check(f"{tag} delta V S", heads(dqS_all[rows], 2, nb), gSV)
        dsc, dSsc = O.bmm_shared_right(dm, dS, mv.transpose(-1, -2))
        tsc = dm.abs() @ mv.abs().transpose(-1, -2)  # terms of the score deltas
        sm, sv, st = dsc * pJ, dSsc * pJ * pJ, tsc * pJ.abs()
        gQ, gSQ = O.bmm_shared_right(sm, sv, mk, s)
        gK, gSK = O.bmm_shared_right(sm.transpose(-1, -2), sv.transpose(-1, -2), mq, s)
        ck.check(f"{tag} delta Q mu", heads(dq_all[rows], 0, nb), gQ, s * (st @ mk.abs()))
        ck.check(f"{tag} delta Q S", heads(dqS_all[rows], 0, nb), gSQ)
        ck.check(f"{tag} delta K mu", heads(dq_all[rows], 1, nb), gK, s * (st.transpose(-1, -2) @ mq.abs()))
        ck.check(f"{tag} delta K S", heads(dqS_all[rows], 1, nb), gSK)
        del pa, pSa, pJ, dsc, dSsc, tsc, sm, sv, st
    ck.flush()
    # the three projections' input deltas summed, as one product over the 3E deltas
    # (multihead_attention.py:262-267, common.py:266-267)
    rm, rS = O.linear_backward_delta(dq_all, dqS_all, w_m)
    rep.check(f"{tag} input delta mu", a["dma"].reshape(B * S, E), rm, dq_all.abs() @ w_m.abs().T)
    rep.check(f"{tag} input delta S", a["dSa"].reshape(B * S, E), rS)
    # parameter deltas of q, k and v (linear.py:138-151)
    for j, name in enumerate("qkv"):
        Sw = a["Sw_qkv"][j]
        dj, dSj = dq_all[:, j * E:(j + 1) * E], dqS_all[:, j * E:(j + 1) * E]
        rep.check(f"{tag} {name}_proj delta_mw", a["pd"][j][0], Sw * (x.T @ dj), Sw * (x.abs().T @ dj.abs()))
        rep.check(f"{tag} {name}_proj delta_Sw", a["pd"][j][1], Sw * Sw * ((x * x).T @ dSj))
    assert L == w_m.shape[1]
