"""Attention modules with the interface of ``mint_plus/models/attention.py``.

``MultiHeadAttention`` (attention.py:32-270) and ``MultimerAttention``
(attention.py:273-371) keep the reference's constructor arguments, parameter
names (so state dicts load unchanged), initialisation and methods. Both gain
``project_qkv(x)``, which returns the projection outputs in the (T, B, .)
layout that the fused multi-pathway op reads through strides (no head-major
copies): one (T, B, 3E) tensor for a fused projection, or q, k, v as three
(T, B, E) tensors.

The eager methods (``forward``, ``forward_before_softmax``) are torch
compositions kept for the reference's non-fused paths; the multi-pathway
computation itself runs in the HIP kernels (``mint_plus_amd.kernels``).
Differences from the reference's eager arithmetic: the softmax runs in fp32,
RoPE tables are fp32 (see ``rotary_embedding``), and the key operand of every
logit ``bmm`` is made contiguous first (bf16 ``bmm`` with a transposed right
operand is avoided on ROCm).
"""
import uuid
from typing import Dict, Optional, Tuple

import torch
import torch.nn.functional as F
from torch import Tensor, nn

from .rotary_embedding import RotaryEmbedding


class IncrementalStateMixin:
    """Per-module key/value cache keyed by a module id (attention.py:12-29)."""

    def __init__(self, *args, **kwargs):
        super().__init__(*args, **kwargs)
        self._incremental_state_id = str(uuid.uuid4())

    def _get_full_key(self, key: str) -> str:
        return f"{self._incremental_state_id}.{key}"

    def get_incremental_state(self, incremental_state: Optional[Dict], key: str):
        if incremental_state is None:
            return None
        return incremental_state.get(self._get_full_key(key))

    def set_incremental_state(self, incremental_state: Optional[Dict], key: str, value):
        if incremental_state is not None:
            incremental_state[self._get_full_key(key)] = value
        return incremental_state


def _to_heads(t: Tensor, H: int) -> Tensor:
    """(T, B, E) -> contiguous (B*H, T, D)."""
    T, B, E = t.shape
    return t.reshape(T, B * H, E // H).transpose(0, 1).contiguous()


def _logits(q: Tensor, k: Tensor) -> Tensor:
    """q (N, T, D) @ k (N, S, D)^T -> (N, T, S) with a contiguous right operand."""
    return torch.bmm(q, k.transpose(1, 2).contiguous())


def _mask_padding(logits: Tensor, key_padding_mask: Optional[Tensor], B: int, H: int) -> Tensor:
    if key_padding_mask is None:
        return logits
    N, T, S = logits.shape
    return logits.view(B, H, T, S).masked_fill(
        key_padding_mask.to(torch.bool)[:, None, None, :], float("-inf")).view(N, T, S)


class MultiHeadAttention(IncrementalStateMixin, nn.Module):
    """Multi-head self-attention with optional RoPE and fused QKV
    (attention.py:32-270)."""

    def __init__(self, embed_dim: int, num_heads: int, dropout: float = 0.0, bias: bool = True,
                 use_rotary_embeddings: bool = False, no_proj: bool = False,
                 use_fused_qkv: bool = False):
        super().__init__()
        self.embed_dim = embed_dim
        self.num_heads = num_heads
        self.head_dim = embed_dim // num_heads
        assert self.head_dim * num_heads == embed_dim, "embed_dim must be divisible by num_heads"
        self.scaling = self.head_dim ** -0.5
        self.dropout = dropout
        self.use_fused_qkv = use_fused_qkv
        if use_fused_qkv:
            self.fused_qkv = nn.Linear(embed_dim, 3 * embed_dim, bias=bias)
            self.q_proj = self.k_proj = self.v_proj = None
        else:
            self.q_proj = nn.Linear(embed_dim, embed_dim, bias=bias)
            self.k_proj = nn.Linear(embed_dim, embed_dim, bias=bias)
            self.v_proj = nn.Linear(embed_dim, embed_dim, bias=bias)
        self.out_proj = None if no_proj else nn.Linear(embed_dim, embed_dim, bias=bias)
        self.rot_emb = RotaryEmbedding(dim=self.head_dim) if use_rotary_embeddings else None
        self._init_parameters()

    def _init_parameters(self):
        """xavier_uniform(gain 2^-1/2) on the projections, zero fused bias;
        xavier_uniform out_proj with zero bias (attention.py:73-85)."""
        g = 2 ** -0.5
        if self.use_fused_qkv:
            nn.init.xavier_uniform_(self.fused_qkv.weight, gain=g)
            if self.fused_qkv.bias is not None:
                nn.init.zeros_(self.fused_qkv.bias)
        else:
            for proj in (self.q_proj, self.k_proj, self.v_proj):
                nn.init.xavier_uniform_(proj.weight, gain=g)
        if self.out_proj is not None:
            nn.init.xavier_uniform_(self.out_proj.weight)
            if self.out_proj.bias is not None:
                nn.init.zeros_(self.out_proj.bias)

    def _project_qkv(self, x: Tensor) -> Tuple[Tensor, Tensor, Tensor]:
        """q, k, v as (T, B, E) (attention.py:87-95)."""
        if self.use_fused_qkv:
            return tuple(t.contiguous() for t in self.fused_qkv(x).chunk(3, dim=-1))
        return self.q_proj(x), self.k_proj(x), self.v_proj(x)

    def project_qkv(self, x: Tensor):
        """The projections in the (T, B, .) layout the fused kernels read by
        strides: the (T, B, 3E) output [q | k | v] of the fused projection, or
        the three (T, B, E) outputs q, k, v of separate projections (three
        GEMMs; no weight concatenation, so nothing is cached across calls)."""
        if self.use_fused_qkv:
            return self.fused_qkv(x)
        return self.q_proj(x), self.k_proj(x), self.v_proj(x)

    def project_qkv_4d(self, x: Tensor) -> Tuple[Tensor, Tensor, Tensor]:
        """q, k, v as contiguous (B, H, T, D); scale and RoPE are left to the
        caller (attention.py:97-117)."""
        T, B, _ = x.shape
        H, D = self.num_heads, self.head_dim
        return tuple(t.reshape(T, B, H, D).permute(1, 2, 0, 3).contiguous()
                     for t in self._project_qkv(x))

    def forward_before_softmax(self, x: Tensor, key_padding_mask: Optional[Tensor] = None
                               ) -> Tuple[Tensor, Tensor]:
        """(B, H, T, T) scaled (and RoPE'd) logits with padded keys at -inf,
        and (B, H, T, D) values (attention.py:119-164)."""
        T, B, _ = x.shape
        H, D = self.num_heads, self.head_dim
        q, k, v = self._project_qkv(x)
        q, k, v = _to_heads(q * self.scaling, H), _to_heads(k, H), _to_heads(v, H)
        if self.rot_emb is not None:
            q, k = self.rot_emb(q), self.rot_emb(k)
        logits = _mask_padding(_logits(q, k), key_padding_mask, B, H)
        return logits.view(B, H, T, T), v.view(B, H, T, D)

    def forward(self, x: Tensor, key_padding_mask: Optional[Tensor] = None,
                attn_mask: Optional[Tensor] = None, incremental_state: Optional[Dict] = None,
                need_weights: bool = False, need_head_weights: bool = False,
                before_softmax: bool = False):
        """Eager attention (attention.py:172-270): returns ``(out (T, B, E),
        weights)``, or ``(logits (B, H, T, S), v (B, H, S, D))`` when
        ``before_softmax``."""
        T, B, E = x.shape
        assert E == self.embed_dim
        H, D = self.num_heads, self.head_dim
        q, k, v = self._project_qkv(x)
        q = _to_heads(q * self.scaling, H)
        k, v = _to_heads(k, H), _to_heads(v, H)
        if incremental_state is not None:
            saved = self.get_incremental_state(incremental_state, "attn_state")
            if saved is not None:
                k = torch.cat([saved["prev_key"].reshape(B * H, -1, D), k], dim=1)
                v = torch.cat([saved["prev_value"].reshape(B * H, -1, D), v], dim=1)
            self.set_incremental_state(incremental_state, "attn_state", {
                "prev_key": k.view(B, H, -1, D), "prev_value": v.view(B, H, -1, D)})
        if self.rot_emb is not None:
            q, k = self.rot_emb(q), self.rot_emb(k)
        logits = _logits(q, k)
        if attn_mask is not None:
            logits = logits + attn_mask
        logits = _mask_padding(logits, key_padding_mask, B, H)
        S = logits.shape[-1]
        if before_softmax:
            return logits.view(B, H, T, S), v.view(B, H, S, D)
        sd = torch.float64 if logits.dtype == torch.float64 else torch.float32
        probs = F.softmax(logits, dim=-1, dtype=sd).to(v.dtype)
        probs = F.dropout(probs, p=self.dropout, training=self.training)
        out = torch.bmm(probs, v).transpose(0, 1).reshape(T, B, E)
        if self.out_proj is not None:
            out = self.out_proj(out)
        weights = None
        if need_weights:
            weights = probs.view(B, H, T, S)
            if not need_head_weights:
                weights = weights.mean(dim=1)
        return out, weights


class MultimerAttention(nn.Module):
    """Cross-chain pathway: fused QKV, no RoPE, no output projection; always
    returns pre-softmax ``(logits, v_heads)`` (attention.py:273-371)."""

    def __init__(self, embed_dim: int, num_heads: int, dropout: float = 0.0, bias: bool = True):
        super().__init__()
        self.embed_dim = embed_dim
        self.num_heads = num_heads
        self.head_dim = embed_dim // num_heads
        assert self.head_dim * num_heads == embed_dim
        self.scaling = self.head_dim ** -0.5
        self.dropout = dropout
        self.fused_qkv = nn.Linear(embed_dim, 3 * embed_dim, bias=bias)
        self._init_parameters()

    def _init_parameters(self):
        nn.init.xavier_uniform_(self.fused_qkv.weight, gain=2 ** -0.5)
        if self.fused_qkv.bias is not None:
            nn.init.zeros_(self.fused_qkv.bias)

    def project_qkv(self, x: Tensor) -> Tensor:
        """(T, B, 3E) fused projection output [q | k | v]."""
        return self.fused_qkv(x)

    def project_qkv_4d(self, x: Tensor) -> Tuple[Tensor, Tensor, Tensor]:
        """q, k, v as contiguous (B, H, T, D) (attention.py:304-323)."""
        T, B, _ = x.shape
        H, D = self.num_heads, self.head_dim
        return tuple(t.reshape(T, B, H, D).permute(1, 2, 0, 3).contiguous()
                     for t in self.fused_qkv(x).chunk(3, dim=-1))

    def forward(self, x: Tensor, key_padding_mask: Optional[Tensor] = None,
                before_softmax: Optional[bool] = None, **kwargs) -> Tuple[Tensor, Tensor]:
        """(B, H, T, T) scaled logits with padded keys at -inf and (B, H, T, D)
        values (attention.py:325-371); ``before_softmax`` is ignored."""
        T, B, _ = x.shape
        H, D = self.num_heads, self.head_dim
        q, k, v = self.fused_qkv(x).chunk(3, dim=-1)
        q, k, v = _to_heads(q * self.scaling, H), _to_heads(k, H), _to_heads(v, H)
        logits = _mask_padding(_logits(q, k), key_padding_mask, B, H)
        return logits.view(B, H, T, T), v.view(B, H, T, D)
