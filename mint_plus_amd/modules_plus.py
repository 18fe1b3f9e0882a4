"""``TransformerLayer_MINT_plus`` and ``build_mint_plus`` with the interface of
``mint_plus/models/modules_plus.py``.

The _plus layer has fused QKV projections on both pathways (a
``MultimerAttention`` for the cross-chain pathway) and optional RMSNorm
(modules_plus.py:20-63). It dispatches like ``TransformerLayer_MINT``; unlike
the reference, which runs the eager combine while training
(modules_plus.py:217-224), the HIP path serves training too, because its
backward is exact.
"""
import torch
import torch.nn as nn

from .attention import MultiHeadAttention, MultimerAttention
from .modules import ESM1bLayerNorm, TransformerLayer_MINT


class TransformerLayer_MINT_plus(TransformerLayer_MINT):
    """Same constructor as ``TransformerLayer_MINT`` (modules_plus.py:28-63)."""

    @staticmethod
    def _make_multimer_attn(embed_dim, heads):
        return MultimerAttention(embed_dim, heads)

    @staticmethod
    def _make_norm(embed_dim, use_rmsnorm):
        return nn.RMSNorm(embed_dim) if use_rmsnorm else ESM1bLayerNorm(embed_dim)


def _cat_qkv(dst: nn.Linear, q: nn.Linear, k: nn.Linear, v: nn.Linear):
    with torch.no_grad():
        dst.weight.copy_(torch.cat([q.weight, k.weight, v.weight], 0))
        if q.bias is not None:
            dst.bias.copy_(torch.cat([q.bias, k.bias, v.bias], 0))


def build_mint_plus(model: nn.Module) -> nn.Module:
    """Replace every ``TransformerLayer_MINT`` of ``model.layers`` by the _plus
    layer, concatenating the q/k/v weights of both pathways into their fused
    projections; out_proj, RoPE, feed-forward and norms move over as they are
    (modules_plus.py:240-305). New parameters take the old layer's device and
    dtype, and the fused-path flag is kept."""
    for i, old in enumerate(model.layers):
        ref = next(old.parameters())
        new = TransformerLayer_MINT_plus(
            old.embed_dim, old.ffn_embed_dim, old.attention_heads,
            use_rotary_embeddings=old.use_rotary_embeddings, use_multimer=old.use_multimer,
            use_rmsnorm=getattr(old, "use_rmsnorm", False),
            use_erf_gelu=getattr(old, "use_erf_gelu", False)).to(device=ref.device,
                                                                 dtype=ref.dtype)
        new._use_fused_multi_pathway = getattr(old, "_use_fused_multi_pathway", False)
        osa = old.self_attn
        if osa.use_fused_qkv:
            sa = osa
        else:
            sa = MultiHeadAttention(new.embed_dim, new.attention_heads,
                                    use_rotary_embeddings=osa.rot_emb is not None,
                                    bias=osa.q_proj.bias is not None,
                                    use_fused_qkv=True).to(device=ref.device, dtype=ref.dtype)
            _cat_qkv(sa.fused_qkv, osa.q_proj, osa.k_proj, osa.v_proj)
            sa.out_proj = osa.out_proj
            sa.rot_emb = osa.rot_emb
            sa.dropout = osa.dropout
        new.self_attn = sa
        if hasattr(old, "multimer_attn"):
            oma = old.multimer_attn
            if isinstance(oma, MultimerAttention):
                new.multimer_attn = oma
            else:
                _cat_qkv(new.multimer_attn.fused_qkv, oma.q_proj, oma.k_proj, oma.v_proj)
        new.feed_forward = old.feed_forward
        new.self_attn_layer_norm = old.self_attn_layer_norm
        new.final_layer_norm = old.final_layer_norm
        model.layers[i] = new
    return model
