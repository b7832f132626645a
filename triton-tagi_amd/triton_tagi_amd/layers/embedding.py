"""Bayesian Embedding (mirrors triton_tagi/layers/embedding.py:39-168).

Forward: (mu, S) = (mw[cat], Sw[cat]) for the integer ids carried in ``ma`` (cast toward
zero, like ``.long()``); ids equal to padding_idx give zeros. Backward accumulates
delta_mw[cat] += delta_mu * Sw[cat], delta_Sw[cat] += delta_S * Sw[cat]^2 and returns
zero input deltas (the index is discrete).
"""

from __future__ import annotations

import torch
from torch import Tensor

from .. import _lib
from ..base import LearnableLayer
from ..param_init import gaussian_param_init
from ..update.parameters import update_parameters


class Embedding(LearnableLayer):
    def __init__(self, num_embeddings: int, embedding_dim: int, input_size: int = 0, scale: float = 1.0,
                 padding_idx: int = -1, device: str = "cuda") -> None:
        self.num_embeddings = num_embeddings
        self.embedding_dim = embedding_dim
        self.input_size = input_size
        self.scale = scale
        self.padding_idx = padding_idx
        self.device = torch.device(device)
        self.has_bias = False
        self.mw, self.Sw = gaussian_param_init(scale, 1.0, (num_embeddings, embedding_dim), device=self.device)
        self.mb = self.Sb = None
        self.cat_idx: Tensor | None = None  # float token ids as given
        self.delta_mw = self.delta_Sw = self.delta_mb = self.delta_Sb = None

    def forward(self, ma: Tensor, Sa: Tensor) -> tuple[Tensor, Tensor]:
        if ma.dim() == 3 and ma.shape[-1] == 1:
            ma = ma.squeeze(-1)
        tokens = _lib.check(ma.contiguous(), "ma")
        self.cat_idx = tokens
        D = self.embedding_dim
        mz = torch.empty(*tokens.shape, D, device=tokens.device, dtype=torch.float32)
        Sz = torch.empty_like(mz)
        _lib.call("tagi_embedding_fwd", tokens.data_ptr(), self.mw.data_ptr(), self.Sw.data_ptr(), mz.data_ptr(),
                  Sz.data_ptr(), tokens.numel(), self.num_embeddings, D, int(self.padding_idx),
                  _lib.stream_of(tokens))
        return mz, Sz

    def backward(self, delta_mz: Tensor, delta_Sz: Tensor) -> tuple[Tensor, Tensor]:
        tokens = self.backward_param_deltas(delta_mz, delta_Sz)
        zeros = torch.zeros(tokens.shape, device=tokens.device, dtype=delta_mz.dtype)
        return zeros, zeros.clone()

    def backward_param_deltas(self, delta_mz: Tensor, delta_Sz: Tensor):
        """The parameter deltas of ``backward`` without the (zero) deltas of the token ids;
        returns the ids."""
        tokens = self.cat_idx
        D = self.embedding_dim
        dm = _lib.check(delta_mz.reshape(-1, D).contiguous(), "delta_mz")
        dS = _lib.check(delta_Sz.reshape(-1, D).contiguous(), "delta_Sz")
        n = tokens.numel()
        self.delta_mw = torch.empty_like(self.mw)
        self.delta_Sw = torch.empty_like(self.Sw)
        ws = _lib.workspace(_lib.query("tagi_embedding_bwd_ws_bytes", n, self.num_embeddings, D), dm.device)
        wp, wb = _lib.ws_args(ws)
        _lib.call("tagi_embedding_bwd", tokens.data_ptr(), dm.data_ptr(), dS.data_ptr(), self.Sw.data_ptr(),
                  self.delta_mw.data_ptr(), self.delta_Sw.data_ptr(), n, self.num_embeddings, D,
                  int(self.padding_idx), wp, wb, _lib.stream_of(dm))
        return tokens

    def _update_items(self):
        return [(self.mw, self.Sw, self.delta_mw, self.delta_Sw)]

    def update(self, cap_factor: float) -> None:
        update_parameters(self.mw, self.Sw, self.delta_mw, self.delta_Sw, cap_factor)

    @property
    def num_parameters(self) -> int:
        return 2 * self.mw.numel()

    def __repr__(self) -> str:
        return (f"Embedding(num_embeddings={self.num_embeddings}, embedding_dim={self.embedding_dim}, "
                f"padding_idx={self.padding_idx}, scale={self.scale})")
