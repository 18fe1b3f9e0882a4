"""Backward of multi-pathway attention on gfx950.

Drop-in for ``mint_plus/models/kernels/multi_pathway_attention_bwd.py:15-59``
(``fused_multi_pathway_attention_bwd``). Unlike the reference's Triton
phase-1/phase-2 kernels, the gradients are exact (full-row softmax backward,
one logit scale) and deterministic (no atomics).
"""
from .. import _lib
from .multi_pathway_attention import _check_inputs


def fused_multi_pathway_attention_bwd(q_self, k_self, v_self, q_multi, k_multi, v_multi,
                                      chain_mask, grad_output, BLOCK_TQ=8, BLOCK_TK=None, QPP=8,
                                      sqrt_softmax=False, *, chain_ids=None,
                                      key_padding_mask=None, rope=False, scale=None,
                                      dropout_p=0.0, dropout_seed=0):
    """Gradients ``(dq_self, dk_self, dv_self, dq_multi, dk_multi, dv_multi)``.

    Recomputes the forward (output and log-sum-exp) and runs the backward
    kernels. Tiling arguments of the reference are accepted and ignored.
    ``dropout_p`` / ``dropout_seed`` (additions) select the forward's dropout
    mask; the reference's backward has no dropout.
    """
    B, H, T, D = _check_inputs(q_self, k_self, v_self, q_multi, k_multi, v_multi,
                               chain_mask, chain_ids)
    if scale is None:
        scale = D ** -0.5 if rope else 1.0
    sel = dict(chain_ids=chain_ids, chain_mask=None if chain_ids is not None else chain_mask,
               key_padding_mask=key_padding_mask, rope=rope, scale=scale,
               sqrt_softmax=sqrt_softmax, dropout_p=float(dropout_p), dropout_seed=int(dropout_seed))
    out, lse = _lib.mpattn_fwd(q_self, k_self, v_self, q_multi, k_multi, v_multi,
                               need_lse=True, **sel)
    return _lib.mpattn_bwd(q_self, k_self, v_self, q_multi, k_multi, v_multi, out, lse,
                           grad_output, **sel)
