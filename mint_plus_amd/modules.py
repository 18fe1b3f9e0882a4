"""Transformer layer of MINT with the interface of
``mint_plus/models/modules.py``.

``TransformerLayer_MINT`` keeps the reference's constructor, parameter names
and dispatch (modules.py:26-320):

* ``use_multimer=False``: standard self-attention (eager torch).
* ``use_multimer=True``: the multi-pathway attention. With
  ``_use_fused_multi_pathway`` set (``enable_fused_multi_pathway``), the HIP
  kernel reads Q/K/V of both pathways straight from the projection outputs,
  applies scale and RoPE itself, takes ``chain_ids`` and the key padding mask,
  and writes O ready for ``out_proj``
  (``kernels.multi_pathway_attention_from_qkv``); forward and backward run on
  the GPU. Without the flag, the materialised pipeline runs: (B, H, T, T)
  logits of both pathways, then ``fused_multimer_combine`` (with autograd:
  ``differentiable_multimer_combine``).

Behaviour that differs from the reference on purpose:

* The fused path applies the key padding mask (the reference's fused path
  ignores it, modules.py:251-320), so fused, materialised and eager paths all
  compute the eager semantics (modules.py:94-154).
* The chain selection uses ``chain_ids`` when the caller passes them (the
  model does, esm2.py:130); a (B, T, T) ``chain_mask`` alone also works.
* The eager combine (``_multimer_attention``) runs its softmax in fp32; the
  reference's bf16 softmax fails for fp32 models (modules.py:135).
"""
import math
from typing import Optional

import torch
import torch.nn as nn
import torch.nn.functional as F
from torch.nn import LayerNorm as ESM1bLayerNorm

from .attention import MultiHeadAttention
from .kernels import (differentiable_multimer_combine, fused_multimer_combine,
                      multi_pathway_attention_from_qkv)


def gelu_erf(x):
    """x * Phi(x) with the exact erf form (modules.py:16-23)."""
    return x * 0.5 * (1.0 + torch.erf(x / math.sqrt(2.0)))


class VanillaFeedForward(nn.Module):
    """fc1 -> GELU (erf) -> fc2 (modules.py:323-336)."""

    def __init__(self, embed_dim, ffn_embed_dim, use_erf_gelu: bool = False):
        super().__init__()
        self.fc1 = nn.Linear(embed_dim, ffn_embed_dim)
        self.fc2 = nn.Linear(ffn_embed_dim, embed_dim)
        self.use_erf_gelu = use_erf_gelu

    def forward(self, x):
        h = self.fc1(x)
        return self.fc2(gelu_erf(h) if self.use_erf_gelu else F.gelu(h))


class RobertaLMHead(nn.Module):
    """dense -> GELU -> LayerNorm -> tied output projection + bias
    (modules.py:339-369)."""

    def __init__(self, embed_dim: int, output_dim: int, weight: torch.Tensor):
        super().__init__()
        self.dense = nn.Linear(embed_dim, embed_dim)
        self.layer_norm = ESM1bLayerNorm(embed_dim)
        self.weight = weight
        self.bias = nn.Parameter(torch.zeros(output_dim))

    def forward(self, features):
        x = self.layer_norm(F.gelu(self.dense(features)))
        return F.linear(x, self.weight) + self.bias


def compute_per_chain_positions(chain_ids: torch.Tensor) -> torch.Tensor:
    """Position of each token inside its chain run: [0,0,0,1,1] -> [0,1,2,0,1]
    (modules.py:372-395)."""
    T = chain_ids.shape[1]
    pos = torch.arange(T, device=chain_ids.device).expand_as(chain_ids)
    start = torch.ones_like(chain_ids, dtype=torch.bool)
    start[:, 1:] = chain_ids[:, 1:] != chain_ids[:, :-1]
    run_start = torch.where(start, pos, torch.zeros_like(pos)).cummax(dim=1).values
    return pos - run_start


def chain_ids_from_mask(chain_mask: torch.Tensor) -> torch.Tensor:
    """(B, T) labels of a (B, T, T) "different chain" mask: the label of key j
    is the first query i on j's chain, min{i : not mask[b, i, j]}."""
    T = chain_mask.shape[-1]
    same = ~chain_mask.to(torch.bool)
    idx = torch.arange(T, device=chain_mask.device)[None, :, None].expand_as(same)
    return torch.where(same, idx, torch.full_like(idx, T)).amin(dim=1).to(torch.int32)


def _needs_grad(*modules):
    return torch.is_grad_enabled() and any(p.requires_grad for m in modules
                                           for p in m.parameters())


class TransformerLayer_MINT(nn.Module):
    """Pre-norm transformer layer with optional multimer pathway
    (modules.py:26-320)."""

    def __init__(self, embed_dim, ffn_embed_dim, attention_heads,
                 use_rotary_embeddings: bool = True, use_multimer: bool = False,
                 use_rmsnorm: bool = False, use_erf_gelu: bool = False):
        super().__init__()
        self.embed_dim = embed_dim
        self.ffn_embed_dim = ffn_embed_dim
        self.attention_heads = attention_heads
        self.use_rotary_embeddings = use_rotary_embeddings
        self.use_multimer = use_multimer
        self.use_rmsnorm = use_rmsnorm
        self.use_erf_gelu = use_erf_gelu
        self._use_fused_multi_pathway = False
        self.self_attn = MultiHeadAttention(embed_dim, attention_heads,
                                            use_rotary_embeddings=use_rotary_embeddings)
        if use_multimer:
            self.multimer_attn = self._make_multimer_attn(embed_dim, attention_heads)
        self.feed_forward = VanillaFeedForward(embed_dim, ffn_embed_dim, use_erf_gelu=use_erf_gelu)
        self.self_attn_layer_norm = self._make_norm(embed_dim, use_rmsnorm)
        self.final_layer_norm = self._make_norm(embed_dim, use_rmsnorm)

    @staticmethod
    def _make_multimer_attn(embed_dim, heads):
        # separate q/k/v projections, no RoPE, no output projection (modules.py:54-60)
        return MultiHeadAttention(embed_dim, heads, use_rotary_embeddings=False, no_proj=True)

    @staticmethod
    def _make_norm(embed_dim, use_rmsnorm):
        # the reference's base layer always uses LayerNorm (modules.py:63-64)
        return ESM1bLayerNorm(embed_dim)

    # -- attention paths ---------------------------------------------------

    def _standard_attention(self, x, attn_mask, padding_mask):
        return self.self_attn(x=x, key_padding_mask=padding_mask, attn_mask=attn_mask)

    def _selection(self, chain_mask, chain_ids, x):
        """chain_ids (preferred) or the (B, T, T) mask; none = one chain."""
        if chain_ids is not None:
            return chain_ids, None
        if chain_mask is not None:
            return None, chain_mask
        T, B, _ = x.shape
        return torch.zeros((B, T), dtype=torch.int32, device=x.device), None

    def _multimer_attention(self, x, chain_mask, padding_mask, chain_ids=None):
        """Eager combine over materialised logits (modules.py:94-154), fp32
        softmax."""
        T, B, E = x.shape
        if chain_mask is None:
            cid, _ = self._selection(None, chain_ids, x)
            chain_mask = cid[:, :, None] != cid[:, None, :]
        intra_logits, intra_v = self.self_attn(x=x, key_padding_mask=padding_mask,
                                               before_softmax=True)
        inter_logits, inter_v = self.multimer_attn(x=x, key_padding_mask=padding_mask,
                                                   before_softmax=True)
        cross = chain_mask.to(torch.bool).unsqueeze(1)
        s = torch.where(cross, inter_logits, intra_logits)
        probs = F.softmax(s, dim=-1, dtype=torch.float64 if s.dtype == torch.float64
                          else torch.float32)
        probs = torch.nan_to_num(probs, nan=0.0)  # rows whose keys are all padded
        probs = F.dropout(probs, p=self.self_attn.dropout, training=self.training)
        out = torch.matmul(probs.masked_fill(cross, 0.0).to(intra_v.dtype), intra_v) + \
            torch.matmul(probs.masked_fill(~cross, 0.0).to(inter_v.dtype), inter_v)
        out = out.transpose(1, 2).reshape(B, T, E)
        return self.self_attn.out_proj(out).transpose(0, 1).contiguous(), None

    def _multimer_attention_reference_arith(self, x, chain_mask, padding_mask, chain_ids=None):
        """The eager combine with the reference's own arithmetic
        (modules_plus.py:182-194, modules.py:135-147): softmax returned in
        bf16 (``dtype=torch.bfloat16``), no ``nan_to_num``, the pathway masks
        applied to the bf16 probabilities. Kept as the timing baseline of
        bf16 models; a row whose keys are all padded gives NaN, as in the
        reference."""
        T, B, E = x.shape
        if chain_mask is None:
            cid, _ = self._selection(None, chain_ids, x)
            chain_mask = cid[:, :, None] != cid[:, None, :]
        intra_logits, intra_v = self.self_attn(x=x, key_padding_mask=padding_mask, before_softmax=True)
        inter_logits, inter_v = self.multimer_attn(x=x, key_padding_mask=padding_mask, before_softmax=True)
        cross = chain_mask.to(torch.bool).unsqueeze(1)
        probs = F.softmax(torch.where(cross, inter_logits, intra_logits), dim=-1, dtype=torch.bfloat16)
        probs = F.dropout(probs, p=self.self_attn.dropout, training=self.training)
        out = torch.matmul(probs.masked_fill(cross, 0.0), intra_v) + \
            torch.matmul(probs.masked_fill(~cross, 0.0), inter_v)
        out = out.transpose(1, 2).reshape(B, T, E)
        return self.self_attn.out_proj(out).transpose(0, 1).contiguous(), None

    def _multimer_attention_plus(self, x, chain_mask, padding_mask, chain_ids=None):
        """Dispatch (modules.py:200-249): fused multi-pathway kernel when the
        flag is set (every dtype and mode), else the materialised pipeline
        with the combine kernel."""
        if self._use_fused_multi_pathway:
            return self._multimer_attention_superfused(x, chain_mask, padding_mask, chain_ids)
        eager = getattr(self, "_use_eager_multimer", False)
        if eager == "reference":
            return self._multimer_attention_reference_arith(x, chain_mask, padding_mask, chain_ids)
        if eager:
            return self._multimer_attention(x, chain_mask, padding_mask, chain_ids)
        T, B, E = x.shape
        sa, ma = self.self_attn, self.multimer_attn
        if chain_mask is None:
            cid, _ = self._selection(None, chain_ids, x)
            chain_mask = cid[:, :, None] != cid[:, None, :]
        intra_logits, intra_v = sa(x=x, key_padding_mask=padding_mask, before_softmax=True)
        inter_logits, inter_v = ma(x=x, key_padding_mask=padding_mask, before_softmax=True)
        p = sa.dropout if self.training else 0.0
        combine = differentiable_multimer_combine if _needs_grad(sa, ma) else fused_multimer_combine
        out = combine(intra_logits, inter_logits, chain_mask.to(torch.bool), intra_v, inter_v,
                      dropout_p=p)
        out = out.transpose(1, 2).reshape(B, T, E)
        return sa.out_proj(out).transpose(0, 1).contiguous(), None

    def _multimer_attention_superfused(self, x, chain_mask, padding_mask, chain_ids=None):
        """Fused multi-pathway attention, no (B, H, T, T) tensor
        (modules.py:251-320): projections -> kernel -> out_proj, all in the
        (T, B, E) layout."""
        sa, ma = self.self_attn, self.multimer_attn
        cid, cmask = self._selection(chain_mask, chain_ids, x)
        out = multi_pathway_attention_from_qkv(
            sa.project_qkv(x), ma.project_qkv(x), self.attention_heads, chain_mask=cmask,
            dropout_p=sa.dropout if self.training else 0.0, training=self.training,
            chain_ids=cid, key_padding_mask=padding_mask, rope=sa.rot_emb is not None,
            scale=sa.scaling)
        return sa.out_proj(out), None

    def forward(self, x: torch.Tensor, self_attn_mask: torch.Tensor = None,
                self_attn_padding_mask: torch.Tensor = None, chain_ids=None):
        """x (T, B, E) -> (x, None) (modules.py:156-197). In multimer mode
        ``self_attn_mask`` is the (B, T, T) different-chain mask."""
        residual = x
        x = self.self_attn_layer_norm(x)
        if self.use_multimer:
            x, attn = self._multimer_attention_plus(x, self_attn_mask, self_attn_padding_mask,
                                                    chain_ids)
        else:
            x, attn = self._standard_attention(x, self_attn_mask, self_attn_padding_mask)
        x = residual + x
        residual = x
        x = residual + self.feed_forward(self.final_layer_norm(x))
        return x, attn


def enable_fused_multi_pathway(model: nn.Module, enabled: bool = True):
    """Set ``_use_fused_multi_pathway`` on every layer of ``model.layers``,
    including layers wrapped in a block that holds ``.layers``
    (modules.py:398-417)."""
    for layer in model.layers:
        for sub in (layer.layers if hasattr(layer, "layers") else (layer,)):
            sub._use_fused_multi_pathway = enabled


def use_eager_multimer(model: nn.Module, enabled=True):
    """Route every layer's non-fused multimer attention through the eager
    torch combine instead of the combine kernel: the baselines the fused
    path is measured against. ``True``: ``_multimer_attention`` (fp32
    softmax, modules.py:94-154); ``"reference"``: the reference's bf16
    arithmetic (``_multimer_attention_reference_arith``); ``False``: off."""
    if enabled not in (True, False, "reference"):
        raise ValueError(f"enabled must be True, False or 'reference' (got {enabled!r})")
    for layer in model.layers:
        for sub in (layer.layers if hasattr(layer, "layers") else (layer,)):
            sub._use_eager_multimer = enabled
