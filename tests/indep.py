"""Checkers that share no code with the oracle -- TEST INFRASTRUCTURE ONLY.

``rope_complex`` restates RoPE as complex multiplication and ``sdpa_concat``
computes the op with torch's ``scaled_dot_product_attention`` (a library
routine) on concatenated features. ``tests/test_oracle.py`` checks the oracle
against them and ``tests/golden/make_golden.py`` writes the golden fixtures
with them.
"""
import numpy as np
import torch
import torch.nn.functional as F

from oracle import mpattn_oracle as orc


# ---------------------------------------------------------------------------
def rope_complex(x, positions):
    """RoPE as complex multiplication: pair (d, d + D/2) is the complex number
    x_d + i x_{d+D/2}, rotated by exp(i * p * theta_d), theta_d =
    fp32(10000^(-2d/D)) and the angle one fp32 product (the reference forms
    both in fp32)."""
    D = x.shape[-1]
    h = D // 2
    theta = (10000.0 ** (-(2.0 * np.arange(h)) / D)).astype(np.float32)
    ang = (np.asarray(positions, np.float32)[:, None] * theta[None, :]).astype(np.float64)
    z = (x[..., :h] + 1j * x[..., h:]) * np.exp(1j * ang)
    return np.concatenate([z.real, z.imag], axis=-1)


def sdpa_concat(qs, ks, vs, qm, km, vm, cid, key_pad, rope, scale, requires_grad=False):
    """The op through torch SDPA. For queries on chain c every key j gets the
    feature k'_j = [R k_self_j, 0] if chain_j == c else [0, k_multi_j] and
    value v_self_j / v_multi_j; the query feature is [R q_self_i, q_multi_i].
    Then q'.k'_j is exactly the selected logit and one SDPA call per chain
    computes the op. Returns (out, logits) as torch float64."""
    t = lambda a: torch.as_tensor(np.asarray(a, np.float64))
    B, H, L, D = qs.shape
    leaves = [t(a).requires_grad_(requires_grad) for a in (qs, ks, vs, qm, km, vm)]
    qs_t, ks_t, vs_t, qm_t, km_t, vm_t = leaves
    if rope:
        cos, sin = (t(a) for a in orc.rope_tables(L, D))  # tables pinned separately below
        h = D // 2
        rot = lambda x: torch.cat([x[..., :h] * cos - x[..., h:] * sin,
                                   x[..., h:] * cos + x[..., :h] * sin], dim=-1)
        qs_r, ks_r = rot(qs_t), rot(ks_t)
    else:
        qs_r, ks_r = qs_t, ks_t
    out = torch.zeros(B, H, L, D, dtype=torch.float64)
    logits = torch.zeros(B, H, L, L, dtype=torch.float64)
    zero = torch.zeros(H, L, D, dtype=torch.float64)
    for b in range(B):
        valid = ~torch.as_tensor(np.asarray(key_pad[b], bool))
        for c in np.unique(cid[b]):
            qi = torch.as_tensor(np.nonzero(cid[b] == c)[0])
            same = torch.as_tensor(cid[b] == c)[None, :, None]
            kfeat = torch.cat([torch.where(same, ks_r[b], zero), torch.where(same, zero, km_t[b])], -1)
            vfeat = torch.where(same, vs_t[b], vm_t[b])
            qfeat = torch.cat([qs_r[b][:, qi], qm_t[b][:, qi]], -1)
            mask = valid[None, None, :].expand(H, len(qi), L)
            o = F.scaled_dot_product_attention(qfeat, kfeat, vfeat, attn_mask=mask, scale=scale)
            out[b][:, qi] = o
            logits[b][:, qi] = scale * qfeat @ kfeat.transpose(-1, -2)
    return out, logits, leaves
