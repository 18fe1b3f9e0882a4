"""Autograd wrappers (drop-in for
``mint_plus/models/kernels/differentiable_attention.py:14-140``).

Forward and backward both run in the gfx950 kernels; the forward saves the
output and its log-sum-exp so the backward needs no statistics pass.
"""
import torch
from torch.autograd import Function

from .. import _lib
from .multi_pathway_attention import _check_inputs, _resolve_dropout


class _MultiPathwayAttentionFn(Function):
    @staticmethod
    def forward(ctx, q_self, k_self, v_self, q_multi, k_multi, v_multi, chain_mask, chain_ids,
                key_padding_mask, rope, scale, sqrt_softmax, dropout_p, dropout_seed):
        # The backward regenerates the dropout mask from (dropout_p, seed).
        sel = dict(chain_ids=chain_ids, chain_mask=None if chain_ids is not None else chain_mask,
                   key_padding_mask=key_padding_mask, rope=rope, scale=scale,
                   sqrt_softmax=sqrt_softmax, dropout_p=dropout_p, dropout_seed=dropout_seed)
        out, lse = _lib.mpattn_fwd(q_self, k_self, v_self, q_multi, k_multi, v_multi,
                                   need_lse=True, **sel)
        ctx.save_for_backward(q_self, k_self, v_self, q_multi, k_multi, v_multi, out, lse)
        ctx.sel = sel
        ctx.sel_tensors = (chain_mask, chain_ids, key_padding_mask)
        return out

    @staticmethod
    def backward(ctx, grad_output):
        q_self, k_self, v_self, q_multi, k_multi, v_multi, out, lse = ctx.saved_tensors
        with torch.no_grad():
            grads = _lib.mpattn_bwd(q_self, k_self, v_self, q_multi, k_multi, v_multi, out, lse,
                                    grad_output, **ctx.sel)
        return (*grads, None, None, None, None, None, None, None, None)


def differentiable_multi_pathway_attention(q_self, k_self, v_self, q_multi, k_multi, v_multi,
                                           chain_mask=None, dropout_p=0.0, training=True, qpp=8,
                                           sqrt_softmax=False, *, chain_ids=None,
                                           key_padding_mask=None, rope=False, scale=None,
                                           dropout_seed=None):
    """Same interface as ``fused_multi_pathway_attention``, with autograd."""
    B, H, T, D = _check_inputs(q_self, k_self, v_self, q_multi, k_multi, v_multi,
                               chain_mask, chain_ids)
    p, seed = _resolve_dropout(dropout_p, training, dropout_seed)
    if scale is None:
        scale = D ** -0.5 if rope else 1.0
    return _MultiPathwayAttentionFn.apply(q_self, k_self, v_self, q_multi, k_multi, v_multi,
                                          chain_mask, chain_ids, key_padding_mask, bool(rope),
                                          float(scale), bool(sqrt_softmax), p, seed)
