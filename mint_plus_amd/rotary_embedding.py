"""Rotary position embedding, with the interface of
``mint_plus/models/rotary_embedding.py:16-55``.

The fused attention kernels apply RoPE themselves while loading Q and K (from
device cos/sin tables, ``_lib.rope_tables``); this module serves the eager
attention paths of the modules (``MultiHeadAttention.forward`` and the
materialised multimer pipeline).

Layout: half split, dim ``d`` pairs with ``d + D/2``; positions are the global
token index ``0..T-1``; ``inv_freq = 1 / 10000**(arange(0, D, 2) / D)``.
Difference from the reference: the angle table is always evaluated in fp32
from ``inv_freq`` recomputed in fp32, so a module cast to bf16 keeps exact
positions (the reference's bf16 ``inv_freq`` buffer quantises the angles,
rotary_embedding.py:44-49). The ``inv_freq`` buffer is kept for state-dict
compatibility.
"""
import torch


def rotate_half(x):
    """cat(-x2, x1) over the two halves of the last dim (rotary_embedding.py:16-18)."""
    h = x.shape[-1] // 2
    return torch.cat((-x[..., h:], x[..., :h]), dim=-1)


def apply_rotary_pos_emb(x, cos, sin):
    """x * cos + rotate_half(x) * sin over the first T rows of the tables
    (rotary_embedding.py:21-24)."""
    T = x.shape[-2]
    return x * cos[:, :T, :] + rotate_half(x) * sin[:, :T, :]


def _inv_freq(dim, device=None):
    """fp32 rounding of 10000^(-2i/dim), formed in fp64 (the same table the
    kernels' RoPE uses)."""
    e = torch.arange(0, dim, 2, device=device, dtype=torch.float64) / dim
    return (1.0 / 10000.0 ** e).to(torch.float32)


class RotaryEmbedding(torch.nn.Module):
    """RoPE over the last dim of (..., T, D) inputs (rotary_embedding.py:27-55)."""

    def __init__(self, dim: int, *_, **__):
        super().__init__()
        self.dim = dim
        self.register_buffer("inv_freq", _inv_freq(dim))
        self._cache = {}

    def tables(self, seq_len, device, dtype=torch.float32):
        """(1, T, D) cos and sin of emb = cat(t * inv_freq, t * inv_freq); the
        angle is an fp32 product, cos/sin are evaluated in ``dtype`` (fp32 or
        fp64). One table per (device, dtype) is kept, at the largest length
        seen (rounded up to 256 positions); shorter lengths read its first T
        positions, so variable-length inputs do not grow the cache."""
        key = (device, dtype)
        hit = self._cache.get(key)
        if hit is None or hit[0].shape[1] < seq_len:
            n = (int(seq_len) + 255) // 256 * 256
            t = torch.arange(n, device=device, dtype=torch.float32)
            freqs = (t[:, None] * _inv_freq(self.dim, device)[None, :]).to(dtype)
            emb = torch.cat((freqs, freqs), dim=-1)
            hit = (emb.cos()[None], emb.sin()[None])
            self._cache[key] = hit
        return hit[0][:, :seq_len], hit[1][:, :seq_len]

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        """Rotate x (..., T, D); computed in fp32 (fp64 for fp64 inputs) and
        returned in x's dtype."""
        ct = torch.float64 if x.dtype == torch.float64 else torch.float32
        cos, sin = self.tables(x.shape[-2], x.device, ct)
        return apply_rotary_pos_emb(x.to(ct), cos, sin).to(x.dtype)
