"""Bayesian multi-head self-attention V2 (mirrors triton_tagi/layers/multihead_attention.py:64-294).

Separate Q/K/V Linear projections; heads are read in place from the (B, S, E)
projection outputs through strided views (no head transposes are materialised):
    mu_qk  = s mu_q mu_k^T,  var_qk = s^2 sum (S_q (mu_k^2 + S_k) + mu_q^2 S_k),  s = 1/sqrt(D)
    scores = Remax over the last dim of (mu_qk, var_qk)       -> mu_score, var_score, J
    out    = TAGI product score @ V, written straight into (B, S, E)
Backward (deterministic operand shared per product):
    dV     = score^T @ d_out          (var: score^2)
    dscore = d_out @ mu_v^T           (var: mu_v^2), then * J and * J^2
    dQ     = s dscore @ mu_k,  dK = s dscore^T @ mu_q   (var: s^2, squared operand)
and the three projection backwards are summed.
"""

from __future__ import annotations

import math

import torch
from torch import Tensor

from .. import _lib
from ..base import LearnableLayer
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

    # views of a (B, S, E) tensor as (B*H, S, D) heads, and of (B, H, S, S) scores
    def _head_view(self, S: int, transpose: bool = False):
        E, D, H = self.embed_dim, self.head_dim, self.num_heads
        return _lib.view(H, S * E, D, 1, E) if transpose else _lib.view(H, S * E, D, E, 1)

    @staticmethod
    def _score_view(S: int, transpose: bool = False):
        return _lib.view(1, S * S, 0, 1, S) if transpose else _lib.view(1, S * S, 0, S, 1)

    def forward(self, ma: Tensor, Sa: Tensor) -> tuple[Tensor, Tensor]:
        B, S, E = ma.shape
        if E != self.embed_dim:
            raise ValueError(f"Expected last dim {self.embed_dim}, got {E}")
        H, D = self.num_heads, self.head_dim
        mu_q, var_q = self.q_proj.forward(ma, Sa)
        mu_k, var_k = self.k_proj.forward(ma, Sa)
        mu_v, var_v = self.v_proj.forward(ma, Sa)
        dev = ma.device
        st = _lib.stream_of(mu_q)
        s = self._scale
        if S <= 256 and D in (16, 32, 64) and B * H < 65536 and all(
                t.data_ptr() % 16 == 0 for t in (mu_q, var_q, mu_k, var_k)):
            # scores and Remax in one kernel; the same values as the two calls below
            mu_score = torch.empty(B, H, S, S, device=dev, dtype=torch.float32)
            var_score, jcb = torch.empty_like(mu_score), torch.empty_like(mu_score)
            _lib.call("tagi_attn_scores_remax", mu_q.data_ptr(), var_q.data_ptr(), mu_k.data_ptr(),
                      var_k.data_ptr(), mu_score.data_ptr(), var_score.data_ptr(), jcb.data_ptr(), B, H, S, D,
                      s, s * s, st)
        else:
            mu_qk = torch.empty(B, H, S, S, device=dev, dtype=torch.float32)
            var_qk = torch.empty_like(mu_qk)
            _lib.call("tagi_bmm_tagi", mu_q.data_ptr(), var_q.data_ptr(), mu_k.data_ptr(), var_k.data_ptr(),
                      mu_qk.data_ptr(), var_qk.data_ptr(), B * H, S, D, S, self._head_view(S),
                      self._head_view(S, transpose=True), self._score_view(S), s, s * s, st)
            mu_score, var_score, jcb = remax(mu_qk.view(B * H * S, S), var_qk.view(B * H * S, S))
            mu_score = mu_score.view(B, H, S, S)
            var_score = var_score.view(B, H, S, S)
            jcb = jcb.view(B, H, S, S)
        mu_out = torch.empty(B, S, E, device=dev, dtype=torch.float32)
        var_out = torch.empty_like(mu_out)
        _lib.call("tagi_bmm_tagi", mu_score.data_ptr(), var_score.data_ptr(), mu_v.data_ptr(), var_v.data_ptr(),
                  mu_out.data_ptr(), var_out.data_ptr(), B * H, S, S, D, self._score_view(S), self._head_view(S),
                  self._head_view(S), 1.0, 1.0, st)
        self._cache = dict(B=B, S=S, H=H, D=D, mu_q=mu_q, mu_k=mu_k, mu_v=mu_v, mu_score=mu_score, jcb=jcb)
        self._attn_mu = mu_score
        self._attn_var = var_score
        return mu_out, var_out

    def backward(self, delta_mz: Tensor, delta_Sz: Tensor) -> tuple[Tensor, Tensor]:
        c = self._cache
        B, S, H, D = c["B"], c["S"], c["H"], c["D"]
        E = self.embed_dim
        s = self._scale
        d_mu = _lib.check(delta_mz.reshape(B, S, E).contiguous(), "delta_mz")
        d_var = _lib.check(delta_Sz.reshape(B, S, E).contiguous(), "delta_Sz")
        dev = d_mu.device
        st = _lib.stream_of(d_mu)
        hv, hvt, sv, svt = self._head_view(S), self._head_view(S, True), self._score_view(S), self._score_view(S, True)
        # dV = score^T @ d_out (score shared on the left)
        dv, dSv = torch.empty(B, S, E, device=dev), torch.empty(B, S, E, device=dev)
        _lib.call("tagi_bmm_shared", d_mu.data_ptr(), d_var.data_ptr(), c["mu_score"].data_ptr(), dv.data_ptr(),
                  dSv.data_ptr(), B * H, S, S, D, svt, hv, hv, 1.0, 1.0, 1, st)
        # dscore = d_out @ mu_v^T (mu_v shared on the right), times the Remax Jacobian
        # (multihead_attention.py:239-243); dQ = s scaled @ mu_k ; dK = s scaled^T @ mu_q
        jcb = _lib.check(c["jcb"], "jcb")
        if tuple(jcb.shape) != (B, H, S, S):
            raise ValueError(f"MultiheadAttentionV2: stored Remax Jacobian {tuple(jcb.shape)} vs {(B, H, S, S)}")
        dq, dSq = torch.empty(B, S, E, device=dev), torch.empty(B, S, E, device=dev)
        dk, dSk = torch.empty(B, S, E, device=dev), torch.empty(B, S, E, device=dev)
        mu_v = c["mu_v"]
        if S <= 256 and D in (16, 32) and B * H < 65536 and all(t.data_ptr() % 16 == 0 for t in (d_mu, d_var, mu_v)):
            # the scaled score deltas are formed per block in LDS, never in memory
            for x, om, oS, tr in ((c["mu_k"], dq, dSq, 0), (c["mu_q"], dk, dSk, 1)):
                _lib.call("tagi_attn_score_deltas_qk", d_mu.data_ptr(), d_var.data_ptr(), mu_v.data_ptr(),
                          jcb.data_ptr(), _lib.check(x, "mu_x").data_ptr(), om.data_ptr(), oS.data_ptr(), B, H, S, D,
                          s, s * s, tr, st)
        else:
            scaled_mu = torch.empty(B, H, S, S, device=dev)
            scaled_var = torch.empty_like(scaled_mu)
            _lib.call("tagi_bmm_shared_jacobian", d_mu.data_ptr(), d_var.data_ptr(), mu_v.data_ptr(),
                      jcb.data_ptr(), scaled_mu.data_ptr(), scaled_var.data_ptr(), B * H, S, D, S, hv, hvt, sv, 1.0,
                      1.0, 0, st)
            _lib.call("tagi_bmm_shared", scaled_mu.data_ptr(), scaled_var.data_ptr(), c["mu_k"].data_ptr(),
                      dq.data_ptr(), dSq.data_ptr(), B * H, S, S, D, sv, hv, hv, s, s * s, 0, st)
            _lib.call("tagi_bmm_shared", scaled_mu.data_ptr(), scaled_var.data_ptr(), c["mu_q"].data_ptr(),
                      dk.data_ptr(), dSk.data_ptr(), B * H, S, S, D, svt, hv, hv, s, s * s, 0, st)
        # the projections' input deltas summed in the GEMM epilogues: (q + k) + v
        d_ma_q, d_Sa_q = self.q_proj.backward(dq, dSq)
        self.k_proj._backward(dk, dSk, True, add=(d_ma_q, d_Sa_q))
        self.v_proj._backward(dv, dSv, True, add=(d_ma_q, d_Sa_q))
        return d_ma_q, d_Sa_q

    def _update_items(self):
        return self.q_proj._update_items() + self.k_proj._update_items() + self.v_proj._update_items()

    def update(self, cap_factor: float) -> None:
        self.q_proj.update(cap_factor)
        self.k_proj.update(cap_factor)
        self.v_proj.update(cap_factor)

    @property
    def num_parameters(self) -> int:
        return self.q_proj.num_parameters + self.k_proj.num_parameters + self.v_proj.num_parameters

    def get_attention_scores(self) -> tuple[Tensor, Tensor]:
        if self._attn_mu is None:
            raise RuntimeError("No attention scores yet; call forward first.")
        return self._attn_mu, self._attn_var

    def __repr__(self) -> str:
        return (f"MultiheadAttentionV2(embed_dim={self.embed_dim}, num_heads={self.num_heads}, "
                f"seq_len={self.seq_len}, bias={self.has_bias})")
