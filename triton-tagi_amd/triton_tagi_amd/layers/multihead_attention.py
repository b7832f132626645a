"""Bayesian multi-head self-attention V2 (mirrors triton_tagi/layers/multihead_attention.py:64-294).

Separate Q/K/V Linear projections (three Linear layers holding the parameters), run as
one product with their weights side by side: the (B*S, 3E) output holds Q, K and V, and
heads are read in place from it through strided views (no head transposes are
materialised):
    mu_qk  = s mu_q mu_k^T,  var_qk = s^2 sum (S_q (mu_k^2 + S_k) + mu_q^2 S_k),  s = 1/sqrt(D)
    scores = Remax over the last dim of (mu_qk, var_qk)       -> mu_score, var_score, J
    out    = TAGI product score @ V, written straight into (B, S, E)
Backward (deterministic operand shared per product):
    dV     = score^T @ d_out          (var: score^2)
    dscore = d_out @ mu_v^T           (var: mu_v^2), then * J and * J^2
    dQ     = s dscore @ mu_k,  dK = s dscore^T @ mu_q   (var: s^2, squared operand)
and the three projection backwards are summed: one input-delta product over the (B*S, 3E)
deltas of Q, K and V, one parameter-delta product whose (E, 3E) result holds the three
layers' deltas side by side. The projections' parameters live side by side as well (each
Linear's tensors are column views of (E, 3E) / (1, 3E) buffers), so neither direction
concatenates or splits tensors.
"""

from __future__ import annotations

import contextlib
import math

import torch
from torch import Tensor

from .. import _lib, _overlap
from ..base import LearnableLayer
from ..kernels.common import fused_backward_delta, linear_forward, linear_param_deltas
from ..update.parameters import update_parameters_multi
from .linear import Linear
from .remax import remax


class MultiheadAttentionV2(LearnableLayer):
    def __init__(self, embed_dim: int, num_heads: int, seq_len: int, num_kv_heads: int | None = None,
                 bias: bool = False, gain_weight: float = 1.0, gain_bias: float = 1.0, init_method: str = "He",
                 pos_emb: str = "", use_causal_mask: bool = False, device: str = "cuda") -> None:
        if pos_emb != "":
            raise NotImplementedError(f"MultiheadAttentionV2 only supports pos_emb='' (got {pos_emb!r})")
        if use_causal_mask:
            raise NotImplementedError("MultiheadAttentionV2 does not support causal masking")
        if num_kv_heads is None:
            num_kv_heads = num_heads
        if num_kv_heads != num_heads:
            raise NotImplementedError("Grouped-query attention (num_kv_heads != num_heads) is not implemented")
        if embed_dim % num_heads != 0:
            raise ValueError(f"embed_dim ({embed_dim}) must be divisible by num_heads ({num_heads})")
        self.embed_dim = embed_dim
        self.num_heads = num_heads
        self.num_kv_heads = num_kv_heads
        self.seq_len = seq_len
        self.has_bias = bias
        self.init_method = init_method
        self.gain_weight = gain_weight
        self.gain_bias = gain_bias
        self.device = torch.device(device)
        self.head_dim = embed_dim // num_heads
        self.q_output_size = num_heads * self.head_dim
        self.k_output_size = num_kv_heads * self.head_dim
        self.v_output_size = num_kv_heads * self.head_dim
        kw = dict(device=device, init_method=init_method, gain_w=gain_weight, gain_b=gain_bias, bias=bias)
        self.q_proj = Linear(embed_dim, self.q_output_size, **kw)
        self.k_proj = Linear(embed_dim, self.k_output_size, **kw)
        self.v_proj = Linear(embed_dim, self.v_output_size, **kw)
        self._scale = 1.0 / math.sqrt(self.head_dim)
        self._cache: dict | None = None
        self._attn_mu: Tensor | None = None
        self._attn_var: Tensor | None = None
        self._attn_src: tuple | None = None  # (qkv_m, qkv_S, B, S) when the variances were not kept

    # views of a (B, S, ld) tensor as (B*H, S, D) heads (row stride ld; the Q/K/V
    # projections live side by side in one (B*S, 3E) buffer), and of (B, H, S, S) scores
    def _head_view(self, S: int, transpose: bool = False, ld: int | None = None):
        D, H = self.head_dim, self.num_heads
        ld = self.embed_dim if ld is None else ld
        return _lib.view(H, S * ld, D, 1, ld) if transpose else _lib.view(H, S * ld, D, ld, 1)

    @staticmethod
    def _score_view(S: int, transpose: bool = False):
        return _lib.view(1, S * S, 0, 1, S) if transpose else _lib.view(1, S * S, 0, S, 1)

    def _projections(self):
        return (self.q_proj, self.k_proj, self.v_proj)

    _QKV_ATTRS = ("mw", "Sw", "mb", "Sb")

    def _qkv_params(self) -> dict:
        """The three projections' parameters side by side: (E, 3E) weights and (1, 3E)
        biases, which the fused projection product and the update read directly. Each
        projection's mw, Sw, mb, Sb are column views of them, so in-place changes to either
        are seen by both (checkpoint restore copies in place). Built at the first forward;
        rebuilt from the projections' tensors if any of them was replaced since."""
        projs = self._projections()
        bufs = getattr(self, "_qkv", None)
        if bufs is not None and self._qkv_intact(bufs):
            return bufs
        bufs = {}
        for attr in self._QKV_ATTRS:
            parts = [getattr(p, attr) for p in projs]
            if parts[0] is None:
                continue
            buf = torch.cat(parts, 1)
            n = parts[0].shape[1]
            for i, p in enumerate(projs):
                setattr(p, attr, buf[:, i * n:(i + 1) * n])
            bufs[attr] = buf
        self._qkv = bufs
        return bufs

    def _qkv_intact(self, bufs: dict) -> bool:
        for attr, buf in bufs.items():
            n = buf.shape[1] // 3
            for i, p in enumerate(self._projections()):
                t = getattr(p, attr, None)
                if not (isinstance(t, Tensor) and t.device == buf.device and t.dtype == buf.dtype
                        and tuple(t.shape) == (buf.shape[0], n) and t.stride() == buf.stride()
                        and t.data_ptr() == buf.data_ptr() + i * n * buf.element_size()):
                    return False
        return True

    def sublayers(self) -> tuple:
        return self._projections()

    def forward(self, ma: Tensor, Sa: Tensor) -> tuple[Tensor, Tensor]:
        B, S, E = ma.shape
        if E != self.embed_dim:
            raise ValueError(f"Expected last dim {self.embed_dim}, got {E}")
        H, D = self.num_heads, self.head_dim
        # Q, K and V (multihead_attention.py:160-172) as one product with the three weight
        # matrices side by side: the same values as three projections, one pass over the input
        ma_flat = ma.reshape(-1, E).contiguous()
        Sa_flat = Sa.reshape(-1, E).contiguous()
        projs = self._projections()
        qkv = self._qkv_params()
        w_m, w_S, b_m, b_S = (qkv.get(a) for a in self._QKV_ATTRS)
        qkv_m, qkv_S = linear_forward(ma_flat, Sa_flat, w_m, w_S, b_m, b_S)
        for p in projs:
            p.ma_in, p._input_shape = ma_flat, ma.shape
        L = 3 * E
        f4 = 4  # bytes per float
        q_m, q_S = qkv_m.data_ptr(), qkv_S.data_ptr()
        k_m, k_S = q_m + E * f4, q_S + E * f4
        v_m, v_S = q_m + 2 * E * f4, q_S + 2 * E * f4
        dev = ma.device
        st = _lib.stream_of(qkv_m)
        s = self._scale
        aligned = B * H < 65536 and L % 4 == 0 and q_m % 16 == 0 and q_S % 16 == 0
        self._attn_src = None
        if S <= 256 and D in (16, 32) and aligned:
            # scores, Remax and score @ V in one kernel (the scores and Remax are the values
            # of the calls below, bit for bit); the score variances are not kept: the
            # backward does not read them and get_attention_scores rebuilds them on request
            mu_score = torch.empty(B, H, S, S, device=dev, dtype=torch.float32)
            jcb = torch.empty_like(mu_score)
            mu_out = torch.empty(B, S, E, device=dev, dtype=torch.float32)
            var_out = torch.empty_like(mu_out)
            _lib.call("tagi_attn_fwd", q_m, q_S, k_m, k_S, v_m, v_S, L, mu_score.data_ptr(), None, jcb.data_ptr(),
                      mu_out.data_ptr(), var_out.data_ptr(), E, B, H, S, D, s, s * s, st)
            self._cache = dict(B=B, S=S, H=H, D=D, qkv_m=qkv_m, ma_in=ma_flat, w_m=w_m, w_S=w_S, b_S=b_S,
                               mu_score=mu_score, jcb=jcb)
            self._attn_mu, self._attn_var = mu_score, None
            self._attn_src = (qkv_m, qkv_S, B, S)
            return mu_out, var_out
        if S <= 256 and D in (16, 32, 64) and aligned:
            # scores and Remax in one kernel; the same values as the two calls below
            mu_score = torch.empty(B, H, S, S, device=dev, dtype=torch.float32)
            var_score, jcb = torch.empty_like(mu_score), torch.empty_like(mu_score)
            _lib.call("tagi_attn_scores_remax", q_m, q_S, k_m, k_S, L, mu_score.data_ptr(), var_score.data_ptr(),
                      jcb.data_ptr(), B, H, S, D, s, s * s, st)
        else:
            mu_qk = torch.empty(B, H, S, S, device=dev, dtype=torch.float32)
            var_qk = torch.empty_like(mu_qk)
            _lib.call("tagi_bmm_tagi", q_m, q_S, k_m, k_S, mu_qk.data_ptr(), var_qk.data_ptr(), B * H, S, D, S,
                      self._head_view(S, ld=L), self._head_view(S, transpose=True, ld=L), self._score_view(S), s,
                      s * s, st)
            mu_score, var_score, jcb = remax(mu_qk.view(B * H * S, S), var_qk.view(B * H * S, S))
            mu_score = mu_score.view(B, H, S, S)
            var_score = var_score.view(B, H, S, S)
            jcb = jcb.view(B, H, S, S)
        mu_out = torch.empty(B, S, E, device=dev, dtype=torch.float32)
        var_out = torch.empty_like(mu_out)
        _lib.call("tagi_bmm_tagi", mu_score.data_ptr(), var_score.data_ptr(), v_m, v_S, mu_out.data_ptr(),
                  var_out.data_ptr(), B * H, S, S, D, self._score_view(S), self._head_view(S, ld=L),
                  self._head_view(S), 1.0, 1.0, st)
        self._cache = dict(B=B, S=S, H=H, D=D, qkv_m=qkv_m, ma_in=ma_flat, w_m=w_m, w_S=w_S, b_S=b_S,
                           mu_score=mu_score, jcb=jcb)
        self._attn_mu = mu_score
        self._attn_var = var_score
        return mu_out, var_out

    def backward(self, delta_mz: Tensor, delta_Sz: Tensor) -> tuple[Tensor, Tensor]:
        c = self._cache
        B, S, H, D = c["B"], c["S"], c["H"], c["D"]
        E = self.embed_dim
        L = 3 * E
        f4 = 4
        s = self._scale
        d_mu = _lib.check(delta_mz.reshape(B, S, E).contiguous(), "delta_mz")
        d_var = _lib.check(delta_Sz.reshape(B, S, E).contiguous(), "delta_Sz")
        dev = d_mu.device
        st = _lib.stream_of(d_mu)
        hv, sv, svt = self._head_view(S), self._score_view(S), self._score_view(S, True)
        hL, hLt = self._head_view(S, ld=L), self._head_view(S, True, ld=L)
        qkv = c["qkv_m"]
        q_m, k_m, v_m = qkv.data_ptr(), qkv.data_ptr() + E * f4, qkv.data_ptr() + 2 * E * f4
        # the deltas of Q, K and V side by side, (B*S, 3E), for one projection backward
        dqkv_m = torch.empty(B * S, L, device=dev)
        dqkv_S = torch.empty(B * S, L, device=dev)
        dq_m, dq_S = dqkv_m.data_ptr(), dqkv_S.data_ptr()
        dk_m, dk_S = dq_m + E * f4, dq_S + E * f4
        dv_m, dv_S = dq_m + 2 * E * f4, dq_S + 2 * E * f4
        # dV = score^T @ d_out (score shared on the left)
        _lib.call("tagi_bmm_shared", d_mu.data_ptr(), d_var.data_ptr(), c["mu_score"].data_ptr(), dv_m, dv_S,
                  B * H, S, S, D, svt, hv, hL, 1.0, 1.0, 1, st)
        # dscore = d_out @ mu_v^T (mu_v shared on the right), times the Remax Jacobian
        # (multihead_attention.py:239-243); dQ = s scaled @ mu_k ; dK = s scaled^T @ mu_q
        jcb = _lib.check(c["jcb"], "jcb")
        if tuple(jcb.shape) != (B, H, S, S):
            raise ValueError(f"MultiheadAttentionV2: stored Remax Jacobian {tuple(jcb.shape)} vs {(B, H, S, S)}")
        if S <= 256 and D in (16, 32) and B * H < 65536 and all(
                t.data_ptr() % 16 == 0 for t in (d_mu, d_var, qkv)):
            # the scaled score deltas are formed once per head in LDS, never in memory, and
            # feed both the query and the key deltas
            _lib.call("tagi_attn_score_deltas_qk_joint", d_mu.data_ptr(), d_var.data_ptr(), E, v_m, q_m, k_m, L,
                      jcb.data_ptr(), dq_m, dq_S, dk_m, dk_S, L, B, H, S, D, s, s * s, st)
        else:
            scaled_mu = torch.empty(B, H, S, S, device=dev)
            scaled_var = torch.empty_like(scaled_mu)
            _lib.call("tagi_bmm_shared_jacobian", d_mu.data_ptr(), d_var.data_ptr(), v_m, jcb.data_ptr(),
                      scaled_mu.data_ptr(), scaled_var.data_ptr(), B * H, S, D, S, hv, hLt, sv, 1.0, 1.0, 0, st)
            _lib.call("tagi_bmm_shared", scaled_mu.data_ptr(), scaled_var.data_ptr(), k_m, dq_m, dq_S, B * H, S, S,
                      D, sv, hL, hL, s, s * s, 0, st)
            _lib.call("tagi_bmm_shared", scaled_mu.data_ptr(), scaled_var.data_ptr(), q_m, dk_m, dk_S, B * H, S, S,
                      D, svt, hL, hL, s, s * s, 0, st)
        # the three projections' parameter deltas in one product (on the side stream within
        # a step when large), their input deltas in one product over the 3E deltas
        # (the sum of the three projections' input deltas, multihead_attention.py:262-267)
        projs = self._projections()
        ma_in = c["ma_in"]
        ctx = _overlap.active()
        big = ma_in.shape[0] * E * L >= _overlap.MIN_MACS_LINEAR
        side = ctx.fork(dev, ma_in, dqkv_m, dqkv_S, c["w_S"], c["b_S"]) if ctx is not None and big else None
        with torch.cuda.stream(side) if side is not None else contextlib.nullcontext():
            dmw, dSw, dmb, dSb = linear_param_deltas(ma_in, dqkv_m, dqkv_S, c["w_S"], c["b_S"])
        # each projection's deltas are column views of the (E, 3E) ones, as its parameters
        # are of the side-by-side buffers the update applies them to
        self._qkv_deltas = (dmw, dSw, dmb, dSb)
        for i, p in enumerate(projs):
            cols = slice(i * E, (i + 1) * E)
            p.delta_mw, p.delta_Sw = dmw[:, cols], dSw[:, cols]
            if self.has_bias:
                p.delta_mb, p.delta_Sb = dmb[:, cols], dSb[:, cols]
        dma, dSa = fused_backward_delta(dqkv_m, dqkv_S, c["w_m"])
        return dma.reshape(B, S, E), dSa.reshape(B, S, E)

    def _update_items(self):
        return self.q_proj._update_items() + self.k_proj._update_items() + self.v_proj._update_items()

    def _update_groups(self):
        """The update over the side-by-side buffers: two groups (weights, biases) instead
        of six, the same values element by element."""
        bufs = getattr(self, "_qkv", None)
        deltas = getattr(self, "_qkv_deltas", None)
        if bufs is None or deltas is None or not self._qkv_intact(bufs):
            return self._update_items()
        dmw, dSw, dmb, dSb = deltas
        groups = [(bufs["mw"], bufs["Sw"], dmw, dSw)]
        if self.has_bias:
            groups.append((bufs["mb"], bufs["Sb"], dmb, dSb))
        return groups

    def update(self, cap_factor: float) -> None:
        update_parameters_multi(self._update_groups(), cap_factor)

    @property
    def num_parameters(self) -> int:
        return self.q_proj.num_parameters + self.k_proj.num_parameters + self.v_proj.num_parameters

    def get_attention_scores(self) -> tuple[Tensor, Tensor]:
        if self._attn_mu is None:
            raise RuntimeError("No attention scores yet; call forward first.")
        if self._attn_var is None and self._attn_src is not None:
            # the fused forward kept only the means: form the scores and their Remax again
            # from the stored projections (the same kernel math, so the same values)
            qkv_m, qkv_S, B, S = self._attn_src
            E, H, D, s = self.embed_dim, self.num_heads, self.head_dim, self._scale
            mu = torch.empty_like(self._attn_mu)
            var, jcb = torch.empty_like(mu), torch.empty_like(mu)
            q_m, q_S = qkv_m.data_ptr(), qkv_S.data_ptr()
            _lib.call("tagi_attn_scores_remax", q_m, q_S, q_m + 4 * E, q_S + 4 * E, 3 * E, mu.data_ptr(),
                      var.data_ptr(), jcb.data_ptr(), B, H, S, D, s, s * s, _lib.stream_of(qkv_m))
            self._attn_var = var
        return self._attn_mu, self._attn_var

    def __repr__(self) -> str:
        return (f"MultiheadAttentionV2(embed_dim={self.embed_dim}, num_heads={self.num_heads}, "
                f"seq_len={self.seq_len}, bias={self.has_bias})")
