"""Multi-pathway attention read straight from the QKV projection outputs.

The fused-layer path of the reference (``_multimer_attention_superfused``,
mint_plus/models/modules.py:251-320) makes three copies around the op:
``project_qkv_4d``'s ``permute(1, 2, 0, 3).contiguous()`` of every Q/K/V
(attention.py:97-117), the Q scaling and RoPE passes with their own
``.contiguous()`` (modules.py:270-287) and the ``transpose(1, 2).contiguous()``
of the output before ``out_proj`` (modules.py:317-318). Here the kernel reads
the six (B, H, T, D) operands as strided views of the projection outputs
(one (T, B, 3E) tensor for a fused projection, three (T, B, E) tensors for
separate q/k/v projections), applies the scale and RoPE while loading them,
and writes O in the (T, B, E) layout that ``out_proj`` consumes, so none of
those copies exist. The backward writes dQ/dK/dV in the same layouts (one
(T, B, 3E) gradient buffer for a fused projection), the layouts the
projections' weight gradients read.
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


def _part_heads(parts, E, H):
    """One pathway's projection tensors -> its three (B, H, T, D) views."""
    if len(parts) == 1:
        return _heads(parts[0], E, H)
    return [_heads(t, E, H)[0] for t in parts]


class _FromQKVFn(Function):
    """Inputs: the self pathway's projection tensors (one (T, B, 3E) or three
    (T, B, E)) followed by the multimer pathway's; ``nself`` says how many are
    the self pathway's."""

    @staticmethod
    def forward(ctx, meta, *parts):
        num_heads, nself, sel = meta
        p_self, p_multi = parts[:nself], parts[nself:]
        T, B, _ = parts[0].shape
        E = p_multi[0].shape[2] // 3 if len(p_multi) == 1 else p_multi[0].shape[2]
        ins = _part_heads(p_self, E, num_heads) + _part_heads(p_multi, E, num_heads)
        out = torch.empty((T, B, E), dtype=parts[0].dtype, device=parts[0].device)
        _, lse = _lib.mpattn_fwd(*ins, out=_heads(out, E, num_heads)[0], need_lse=True, **sel)
        ctx.save_for_backward(*parts, out, lse)
        ctx.meta = (num_heads, nself, sel)
        return out

    @staticmethod
    def backward(ctx, grad_out):
        *parts, out, lse = ctx.saved_tensors
        H, nself, sel = ctx.meta
        E = out.shape[2]
        if not grad_out.is_contiguous():
            grad_out = grad_out.contiguous()
        grads = [torch.empty_like(t) for t in parts]
        p_self, p_multi = parts[:nself], parts[nself:]
        g_self, g_multi = grads[:nself], grads[nself:]
        with torch.no_grad():
            _lib.mpattn_bwd(*_part_heads(p_self, E, H), *_part_heads(p_multi, E, H),
                            _heads(out, E, H)[0], lse, _heads(grad_out, E, H)[0],
                            grads=_part_heads(g_self, E, H) + _part_heads(g_multi, E, H), **sel)
        return (None, *grads)


def _as_parts(x, name):
    """A pathway's projections as a tuple of contiguous (T, B, .) tensors."""
    parts = tuple(x) if isinstance(x, (tuple, list)) else (x,)
    if len(parts) not in (1, 3) or any(t.dim() != 3 for t in parts):
        raise AssertionError(f"{name} must be one (T, B, 3E) tensor or three (T, B, E) tensors")
    return tuple(t if t.is_contiguous() else t.contiguous() for t in parts)


def multi_pathway_attention_from_qkv(qkv_self, qkv_multi, num_heads, chain_mask=None,
                                     dropout_p=0.0, training=True, sqrt_softmax=False, *,
                                     chain_ids=None, key_padding_mask=None, rope=True,
                                     scale=None, dropout_seed=None):
    """Multi-pathway attention on the projection outputs of the two pathways
    (self pathway first); returns O as (T, B, E). Each pathway is given as the
    (T, B, 3E) output of a fused QKV projection or as its (q, k, v) outputs,
    three (T, B, E) tensors. Differentiable w.r.t. every projection output.

    ``rope`` applies RoPE (global positions, half-split layout) to the self
    pathway's Q and K; ``scale`` defaults to ``head_dim ** -0.5``. Chain
    selection by ``chain_ids`` (B, T) or ``chain_mask`` (B, T, T), True =
    different chains; ``key_padding_mask`` (B, T), True = padded key.
    ``dropout_p`` applies in training only (per-element mask from
    ``dropout_seed``, default drawn from torch's CPU generator).
    """
    p_self, p_multi = _as_parts(qkv_self, "qkv_self"), _as_parts(qkv_multi, "qkv_multi")
    T, B = p_self[0].shape[:2]
    E = [t.shape[2] // (3 if len(p) == 1 else 1) for p in (p_self, p_multi) for t in p]
    if len(set(E)) != 1 or any(t.shape[:2] != (T, B) for t in p_self + p_multi):
        raise AssertionError("qkv_self / qkv_multi: mismatched (T, B, E) shapes")
    E = E[0]
    if len(p_self) == 1 and p_self[0].shape[2] != 3 * E or len(p_multi) == 1 and p_multi[0].shape[2] != 3 * E:
        raise AssertionError("a fused projection output must be (T, B, 3E)")
    if E % num_heads:
        raise AssertionError(f"E={E} is not divisible by num_heads={num_heads}")
    D = E // num_heads
    p, seed = _resolve_dropout(dropout_p, training, dropout_seed)
    if chain_ids is None and (chain_mask is None or tuple(chain_mask.shape) != (B, T, T)):
        raise AssertionError(f"chain_ids (B, T) or chain_mask (B, T, T) = {(B, T, T)} required")
    if scale is None:
        scale = D ** -0.5
    sel = dict(chain_ids=chain_ids, chain_mask=None if chain_ids is not None else chain_mask,
               key_padding_mask=key_padding_mask, rope=bool(rope), scale=float(scale),
               sqrt_softmax=bool(sqrt_softmax), dropout_p=p, dropout_seed=seed)
    return _FromQKVFn.apply((int(num_heads), len(p_self), sel), *p_self, *p_multi)
