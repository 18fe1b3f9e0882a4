"""Fused multi-pathway attention forward on gfx950.

Drop-in for ``mint_plus/models/kernels/multi_pathway_attention.py:184-279``
(``fused_multi_pathway_attention``) and its fp16 twin
``mint_plus/models/kernels/multi_pathway_attention_fp16.py:148-198``. The
computation runs in the HIP kernel behind ``libmpattn.so`` (``mpattn_fwd``).
"""
import torch

from .. import _lib


def _check_inputs(q_self, k_self, v_self, q_multi, k_multi, v_multi, chain_mask, chain_ids):
    """The reference's asserts (multi_pathway_attention.py:224-226)."""
    B, H, T, D = q_self.shape
    if not all(t.shape == q_self.shape for t in (k_self, v_self, q_multi, k_multi, v_multi)):
        raise AssertionError("q/k/v of both pathways must share one (B, H, T, D) shape")
    if chain_ids is None:
        if chain_mask is None or tuple(chain_mask.shape) != (B, T, T):
            raise AssertionError(f"chain_mask must be (B, T, T) = {(B, T, T)}")
    elif tuple(chain_ids.shape) != (B, T):
        raise AssertionError(f"chain_ids must be (B, T) = {(B, T)}")
    return B, H, T, D


def _resolve_dropout(dropout_p, training, dropout_seed=None):
    """Effective (p, seed): p is 0 outside training; a missing seed is drawn
    from torch's default CPU generator (so ``torch.manual_seed`` fixes it), as
    the reference draws its per-call seed (multi_pathway_attention_fp16.py:187).
    """
    p = float(dropout_p) if training else 0.0
    if not 0.0 <= p < 1.0:
        raise ValueError(f"dropout_p must be in [0, 1), got {p}")
    if p == 0.0:
        return 0.0, 0
    if dropout_seed is None:
        dropout_seed = int(torch.randint(0, 2**62, (1,), dtype=torch.int64).item())
    return p, int(dropout_seed) & 0xFFFFFFFFFFFFFFFF


def fused_multi_pathway_attention(q_self, k_self, v_self, q_multi, k_multi, v_multi,
                                  chain_mask=None, dropout_p=0.0, training=True, qpp=None,
                                  sqrt_softmax=False, *, chain_ids=None, key_padding_mask=None,
                                  rope=False, scale=None, dropout_seed=None):
    """Multi-pathway attention, no (B, H, T, T) logits materialised.

    Same contract as the reference: q/k/v of both pathways are (B, H, T, D);
    ``chain_mask`` (B, T, T) bool, True = different chains. By default the
    caller has already applied the scale to q and RoPE to q_self/k_self.

    Additions (keyword-only, all optional):
      chain_ids:        (B, T) int chain labels; replaces ``chain_mask`` and
                        enables per-tile pathway skipping.
      key_padding_mask: (B, T) bool, True = padded key (masked to -inf).
      rope:             apply RoPE (global positions) to q_self/k_self in the
                        kernel; q/k are then the raw projections.
      scale:            logit scale; default 1 (pre-scaled q) or D^-1/2 when
                        ``rope`` is set.
      dropout_seed:     64-bit seed of the dropout mask (default: drawn from
                        torch's CPU generator). With ``dropout_p`` > 0 in
                        training, each element of P is dropped independently
                        (a hash of seed, b*H+h, query, key) and the kept ones
                        scaled by 1 / (1 - p); 16-bit inputs only.
    ``qpp`` is a Triton tuning hint and is ignored.

    Returns a new (B, H, T, D) tensor in the input dtype.
    """
    B, H, T, D = _check_inputs(q_self, k_self, v_self, q_multi, k_multi, v_multi,
                               chain_mask, chain_ids)
    p, seed = _resolve_dropout(dropout_p, training, dropout_seed)
    if scale is None:
        scale = D ** -0.5 if rope else 1.0
    return _lib.mpattn_fwd(q_self, k_self, v_self, q_multi, k_multi, v_multi,
                           chain_ids=chain_ids, chain_mask=None if chain_ids is not None else chain_mask,
                           key_padding_mask=key_padding_mask, rope=rope, scale=scale,
                           sqrt_softmax=sqrt_softmax, dropout_p=p, dropout_seed=seed)


def fused_multi_pathway_attention_fp16(q_self, k_self, v_self, q_multi, k_multi, v_multi,
                                       chain_mask=None, dropout_p=0.0, training=True, qpp=None,
                                       **kwargs):
    """fp16 entry point of the reference (multi_pathway_attention_fp16.py:148).
    The same kernel family serves fp16 inputs."""
    if q_self.dtype != torch.float16:
        raise AssertionError("fused_multi_pathway_attention_fp16 expects float16 inputs")
    return fused_multi_pathway_attention(q_self, k_self, v_self, q_multi, k_multi, v_multi,
                                         chain_mask, dropout_p, training, qpp, **kwargs)
