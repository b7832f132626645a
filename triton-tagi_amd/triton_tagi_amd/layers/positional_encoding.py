"""Sinusoidal positional encoding (mirrors triton_tagi/layers/positional_encoding.py:25-71).

pe[t, d] = sin(t / 10000^(d/E)) for even d, cos(...) for odd d (d as a float, not
rounded to pairs). Forward adds pe[:S] to the means; variances and deltas pass through.
"""

from __future__ import annotations

import torch
from torch import Tensor

from .. import _lib
from ..base import Layer


def sinusoidal_table(max_seq_len: int, embed_dim: int, device="cpu") -> Tensor:
    d = torch.arange(embed_dim, dtype=torch.float32, device=device)
    pos = torch.arange(max_seq_len, dtype=torch.float32, device=device)
    freq = 1.0 / torch.pow(10000.0, d / embed_dim)
    angle = pos.unsqueeze(1) * freq.unsqueeze(0)
    even = (torch.arange(embed_dim, device=device) % 2 == 0).unsqueeze(0)
    return torch.where(even, torch.sin(angle), torch.cos(angle)).contiguous()


class PositionalEncoding(Layer):
    def __init__(self, embed_dim: int, max_seq_len: int = 2048, device: str = "cuda") -> None:
        self.embed_dim = embed_dim
        self.max_seq_len = max_seq_len
        self.device = torch.device(device)
        # built on the CPU whatever the device: the float32 angles t * freq reach ~2000 rad, so
        # a one-ulp difference between two devices' pow() moves an entry by up to ~1e-4; the
        # CPU table is the same on every machine (and equal to the reference's CPU table)
        self.pe_cache = sinusoidal_table(max_seq_len, embed_dim, device="cpu").to(self.device)

    def forward(self, ma: Tensor, Sa: Tensor) -> tuple[Tensor, Tensor]:
        S, E = ma.shape[-2], ma.shape[-1]
        if E != self.embed_dim or S > self.max_seq_len:
            raise ValueError(f"PositionalEncoding: got (..., {S}, {E}) for table ({self.max_seq_len}, {self.embed_dim})")
        ma = _lib.check(ma.contiguous(), "ma")
        pe = _lib.check(self.pe_cache, "pe_cache")
        out = torch.empty_like(ma)
        _lib.call("tagi_pe_add", ma.data_ptr(), pe.data_ptr(), out.data_ptr(), ma.numel() // (S * E), S, E,
                  _lib.stream_of(ma))
        return out, Sa

    def backward(self, delta_ma: Tensor, delta_Sa: Tensor) -> tuple[Tensor, Tensor]:
        return delta_ma, delta_Sa

    def __repr__(self) -> str:
        return f"PositionalEncoding(embed_dim={self.embed_dim}, max_seq_len={self.max_seq_len})"
