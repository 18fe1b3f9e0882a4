"""Multi-pathway attention read straight from the QKV projection outputs.

The fused-layer path of the reference (``_multimer_attention_superfused``,
mint_plus/models/modules.py:251-320) makes three copies around the op:
``project_qkv_4d``'s ``permute(1, 2, 0, 3).contiguous()`` of every Q/K/V
(attention.py:97-117), the Q scaling and RoPE passes with their own
``.contiguous()`` (modules.py:270-287) and the ``transpose(1, 2).contiguous()``
of the output before ``out_proj`` (modules.py:317-318). Here the kernel reads
the six (B, H, T, D) operands as strided views of the two (T, B, 3E) fused
projection outputs, applies the scale and RoPE while loading them, and writes
O in the (T, B, E) layout that ``out_proj`` consumes, so none of those copies
exist. The backward writes dQ/dK/dV of a pathway into one (T, B, 3E)
gradient buffer, the layout the fused projection's weight gradient reads.
"""
import torch
from torch.autograd import Function

from .. import _lib
from .multi_pathway_attention import _resolve_dropout


def _heads(t, E, H):
    """(T, B, k*E) projection output -> k strided (B, H, T, D) head views."""
    T, B, W = t.shape
    k, D = W // E, E // H
    v = t.view(T, B, k, H, D)
    return [v[:, :, i].permute(1, 2, 0, 3) for i in range(k)]


class _FromQKVFn(Function):
    @staticmethod
    def forward(ctx, qkv_self, qkv_multi, num_heads, chain_ids, chain_mask, key_padding_mask, rope,
                scale, sqrt_softmax, dropout_p, dropout_seed):
        T, B, E3 = qkv_self.shape
        E = E3 // 3
        ins = _heads(qkv_self, E, num_heads) + _heads(qkv_multi, E, num_heads)
        out = torch.empty((T, B, E), dtype=qkv_self.dtype, device=qkv_self.device)
        sel = dict(chain_ids=chain_ids, chain_mask=None if chain_ids is not None else chain_mask,
                   key_padding_mask=key_padding_mask, rope=rope, scale=scale,
                   sqrt_softmax=sqrt_softmax, dropout_p=dropout_p, dropout_seed=dropout_seed)
        _, lse = _lib.mpattn_fwd(*ins, out=_heads(out, E, num_heads)[0], need_lse=True, **sel)
        ctx.save_for_backward(qkv_self, qkv_multi, out, lse)
        ctx.sel = sel
        ctx.num_heads = num_heads
        return out

    @staticmethod
    def backward(ctx, grad_out):
        qkv_self, qkv_multi, out, lse = ctx.saved_tensors
        H = ctx.num_heads
        E = out.shape[2]
        if not grad_out.is_contiguous():
            grad_out = grad_out.contiguous()
        g_self = torch.empty_like(qkv_self)
        g_multi = torch.empty_like(qkv_multi)
        with torch.no_grad():
            _lib.mpattn_bwd(*_heads(qkv_self, E, H), *_heads(qkv_multi, E, H),
                            _heads(out, E, H)[0], lse, _heads(grad_out, E, H)[0],
                            grads=_heads(g_self, E, H) + _heads(g_multi, E, H), **ctx.sel)
        return g_self, g_multi, None, None, None, None, None, None, None, None, None


def multi_pathway_attention_from_qkv(qkv_self, qkv_multi, num_heads, chain_mask=None,
                                     dropout_p=0.0, training=True, sqrt_softmax=False, *,
                                     chain_ids=None, key_padding_mask=None, rope=True,
                                     scale=None, dropout_seed=None):
    """Multi-pathway attention on the (T, B, 3E) outputs of the two fused QKV
    projections (self pathway first); returns O as (T, B, E). Differentiable
    w.r.t. both projection outputs.

    ``rope`` applies RoPE (global positions, half-split layout) to the self
    pathway's Q and K; ``scale`` defaults to ``head_dim ** -0.5``. Chain
    selection by ``chain_ids`` (B, T) or ``chain_mask`` (B, T, T), True =
    different chains; ``key_padding_mask`` (B, T), True = padded key.
    ``dropout_p`` applies in training only (per-element mask from
    ``dropout_seed``, default drawn from torch's CPU generator).
    """
    if qkv_self.dim() != 3 or qkv_self.shape != qkv_multi.shape:
        raise AssertionError("qkv_self / qkv_multi must both be (T, B, 3E)")
    T, B, E3 = qkv_self.shape
    if E3 % (3 * num_heads):
        raise AssertionError(f"3E={E3} is not divisible by 3 * num_heads={3 * num_heads}")
    D = E3 // (3 * num_heads)
    p, seed = _resolve_dropout(dropout_p, training, dropout_seed)
    if chain_ids is None and (chain_mask is None or tuple(chain_mask.shape) != (B, T, T)):
        raise AssertionError(f"chain_ids (B, T) or chain_mask (B, T, T) = {(B, T, T)} required")
    if scale is None:
        scale = D ** -0.5
    qkv_self = qkv_self if qkv_self.is_contiguous() else qkv_self.contiguous()
    qkv_multi = qkv_multi if qkv_multi.is_contiguous() else qkv_multi.contiguous()
    return _FromQKVFn.apply(qkv_self, qkv_multi, int(num_heads), chain_ids, chain_mask,
                            key_padding_mask, bool(rope), float(scale), bool(sqrt_softmax), p, seed)
