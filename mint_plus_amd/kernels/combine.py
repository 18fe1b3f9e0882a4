"""Materialised-logit combine on gfx950 (drop-in for
``mint_plus/models/kernels/__init__.py:179-286`` and
``mint_plus/models/kernels/differentiable_attention.py:88-140``).

For callers that already hold the two (B, H, T, T) pre-softmax logit tensors:
``where(chain_mask, inter, intra)`` -> one fp32 softmax over keys -> split by
pathway -> ``P_intra @ V_self + P_inter @ V_multi``. The kernels behind
``mpattn_combine_fwd`` / ``mpattn_combine_bwd`` accept any T (no power-of-2
limit) and bf16, fp16 or fp32 inputs; a row whose keys are all -inf gives 0.
"""
import torch
from torch.autograd import Function

from .. import _lib
from .multi_pathway_attention import _resolve_dropout


def _check_mask(chain_mask):
    if chain_mask.dtype != torch.bool:
        raise AssertionError("chain_mask must be bool")


def fused_multimer_combine(intra_logits, inter_logits, chain_mask, intra_values, inter_values,
                           dropout_p=0.0, *, dropout_seed=None):
    """(B, H, T, D) combined output, ready for ``out_proj``
    (kernels/__init__.py:179-242). With ``dropout_p`` > 0 each element of P
    is dropped by the fused op's hash mask for ``dropout_seed`` (default:
    drawn from torch's CPU generator, as the reference draws its seed,
    kernels/__init__.py:211) and the kept ones scaled by 1 / (1 - p)."""
    _check_mask(chain_mask)
    p, seed = _resolve_dropout(dropout_p, True, dropout_seed)
    return _lib.mpattn_combine_fwd(intra_logits, inter_logits, chain_mask, intra_values,
                                   inter_values, dropout_p=p, dropout_seed=seed)


def fused_multimer_combine_bwd(intra_logits, inter_logits, chain_mask, intra_values,
                               inter_values, grad_output, dropout_p=0.0, *, dropout_seed=0,
                               lse=None, output=None):
    """(d_intra_logits, d_inter_logits, d_intra_values, d_inter_values) of the
    combine (kernels/__init__.py:247-286), in the inputs' dtype; with dropout,
    ``dropout_seed`` must be the forward's. ``lse`` / ``output``: the
    forward's log-sum-exp and output (both or neither); given, the row
    statistics come from them instead of a pass over both logit tensors."""
    _check_mask(chain_mask)
    return _lib.mpattn_combine_bwd(intra_logits, inter_logits, chain_mask, intra_values,
                                   inter_values, grad_output, dropout_p=dropout_p,
                                   dropout_seed=dropout_seed, lse=lse, out=output)


class _MultimerCombineFn(Function):
    @staticmethod
    def forward(ctx, intra_logits, inter_logits, chain_mask, intra_values, inter_values,
                dropout_p, dropout_seed):
        # The forward's LSE and output go to the backward, which then needs
        # no statistics pass over the two logit tensors.
        out, lse = _lib.mpattn_combine_fwd(intra_logits, inter_logits, chain_mask, intra_values,
                                           inter_values, dropout_p=dropout_p,
                                           dropout_seed=dropout_seed, need_lse=True)
        ctx.save_for_backward(intra_logits, inter_logits, chain_mask, intra_values, inter_values,
                              out, lse)
        ctx.dropout_p, ctx.dropout_seed = dropout_p, dropout_seed
        return out

    @staticmethod
    def backward(ctx, grad_output):
        il, el, cm, vs, vm, out, lse = ctx.saved_tensors
        with torch.no_grad():
            d_il, d_el, d_vs, d_vm = fused_multimer_combine_bwd(
                il, el, cm, vs, vm, grad_output.contiguous(), dropout_p=ctx.dropout_p,
                dropout_seed=ctx.dropout_seed, lse=lse, output=out)
        return d_il, d_el, None, d_vs, d_vm, None, None


def differentiable_multimer_combine(intra_logits, inter_logits, chain_mask, intra_values,
                                    inter_values, dropout_p=0.0, *, dropout_seed=None):
    """``fused_multimer_combine`` with autograd
    (differentiable_attention.py:127-140); the backward reuses the forward's
    dropout seed."""
    _check_mask(chain_mask)
    p, seed = _resolve_dropout(dropout_p, True, dropout_seed)
    return _MultimerCombineFn.apply(intra_logits, inter_logits, chain_mask, intra_values,
                                    inter_values, p, seed)
