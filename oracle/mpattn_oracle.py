"""CPU oracle for multi-pathway attention -- TEST INFRASTRUCTURE ONLY.

This module is the checker, never the product: only ``tests/``,
``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may import
it. The HIP library (``mint_plus_amd``) never calls into it.

It restates, in float64 numpy, the math of the reference's eager path:

* RoPE -- ``mint_plus/models/rotary_embedding.py:16-55``: half-split layout,
  ``inv_freq = 1 / 10000**(arange(0, D, 2) / D)``, global positions
  ``t = arange(L)``, ``emb = cat(freqs, freqs)``,
  ``x*cos + rotate_half(x)*sin`` with ``rotate_half = cat(-x2, x1)``.
* Logits -- ``mint_plus/models/attention.py:186-236`` (self pathway: scale,
  RoPE, bmm, key padding -> -inf) and ``:343-365`` (multimer pathway: scale,
  bmm, key padding, no RoPE).
* Combine -- ``mint_plus/models/modules_plus.py:178-194``:
  ``where(chain_mask, inter, intra)``, one softmax over all keys, split by
  pathway, ``P_intra @ V_self + P_inter @ V_multi``. The softmax runs in high
  precision as in ``mint_plus/models/mu_scaling/layer.py:159`` and
  ``profiles/test_sqrt_softmax.py:77-94`` (the eager bf16 softmax of
  ``modules_plus.py:185`` is a reference quirk, not a target).
* A row whose keys are all padded gives 0, the ``d == 0`` guard of
  ``mint_plus/models/kernels/multi_pathway_attention.py:163-167``.
* ``sqrt_softmax``: ``O = sum_j sqrt(P_ij) V_j``
  (``multi_pathway_attention.py:138-152,164-165``).
* Dropout: per element of P, ``keep = rand > p`` and ``P / (1 - p)``, as the
  reference's kernels apply it (``kernels/__init__.py:118-122``,
  ``profiles/bench_optimizations.py:798-803``), with the row sum over the
  undropped P. The reference draws one Triton ``tl.rand`` value per program;
  this build's mask is a counter-based hash of (seed, b*H+h, query, key)
  (the definition in ``include/mpattn.h``), restated by ``dropout_keep``.

Gradients are analytic (softmax backward ``dS = P * (dP - rowsum(P*dP))``
and the transpose of the RoPE rotation). The reference's Triton backward
(``multi_pathway_attention_bwd.py``) is not followed: it is mathematically
wrong (see the module tests, which pin these gradients by central finite
differences instead).

How each function is pinned (``tests/test_oracle.py``):

* ``rope_tables`` / ``apply_rope``: identity at position 0, norm
  preservation, the relative-position identity
  ``<R_i q, R_j k> = <q, R_{j-i} k>``, and a hand-computed half-split vector.
* ``mpattn_forward``: reduction to ``torch.nn.functional.scaled_dot_product_attention``
  on concatenated features (one call per query chain), all-same-chain
  reduction to plain SDPA with RoPE, invariants (chain-label permutation,
  appended padded keys, constant V, zero Q), L = 1, and a pure-Python
  triple loop on tiny inputs.
* ``mpattn_backward``: central finite differences of ``mpattn_forward``
  (also with dropout: the mask is fixed by the seed).
* ``fmix32``: MurmurHash3_x86_32 known answers (the finaliser is the whole
  hash of the empty string, and inside the hash of longer ones).
* ``dropout_keep``: p = 0 keeps everything, the kept fraction is 1 - p within
  binomial bounds, rows / keys / heads / seeds give uncorrelated masks, and
  a pure-Python restatement of the formula on a few elements.
* ``combine_forward``: equals ``mpattn_forward`` when fed the logits of the
  two pathways computed by torch (bmm, scale, -inf padding); all-same-chain
  reduces to ``torch.softmax(intra) @ Vs``.
* ``combine_backward``: torch autograd of an independent torch expression
  and central finite differences of ``combine_forward``.
"""
import numpy as np

ROPE_BASE = 10000.0


def rope_tables(L, D):
    """cos/sin tables (L, D/2) of the angle ``t * inv_freq[i]``.

    Follows ``rotary_embedding.py:44,49-53``: ``inv_freq`` and the angle
    ``t * inv_freq`` are fp32 quantities in the reference, so they are formed
    here in fp32 (inv_freq = fp32 rounding of the exact value, angle = one
    fp32 product); cos/sin are then evaluated in fp64.
    """
    inv = (1.0 / ROPE_BASE ** (np.arange(0, D, 2, dtype=np.float64) / D)).astype(np.float32)
    t = np.arange(L, dtype=np.float32)
    ang = (t[:, None] * inv[None, :]).astype(np.float64)  # fp32 product, exact in fp64
    return np.cos(ang), np.sin(ang)


def apply_rope(x, cos, sin):
    """``x * cos + rotate_half(x) * sin`` on (..., L, D), positions 0..L-1
    (``rotary_embedding.py:16-24``)."""
    h = x.shape[-1] // 2
    x1, x2 = x[..., :h], x[..., h:]
    return np.concatenate([x1 * cos - x2 * sin, x2 * cos + x1 * sin], axis=-1)


def apply_rope_transpose(g, cos, sin):
    """Transpose of ``apply_rope`` (rotation by the negative angle)."""
    h = g.shape[-1] // 2
    g1, g2 = g[..., :h], g[..., h:]
    return np.concatenate([g1 * cos + g2 * sin, g2 * cos - g1 * sin], axis=-1)


def cross_mask(chain_ids=None, chain_mask=None):
    """(B, L, L) bool, True where query and key are on different chains
    (``esm2.py:89``: ``~eq(chain_ids[:, :, None], chain_ids[:, None, :])``)."""
    if chain_mask is not None:
        return np.asarray(chain_mask, dtype=bool)
    c = np.asarray(chain_ids)
    return c[:, :, None] != c[:, None, :]


def _tr(x):
    """Swap the last two axes."""
    return np.swapaxes(x, -1, -2)


def _mm(a, b):
    """Batched float64 matrix product over the leading axes (numpy's matmul,
    BLAS per (b, h) slice)."""
    return np.matmul(np.ascontiguousarray(a), np.ascontiguousarray(b))


def _prepare(qs, ks, qm, km, rope, scale):
    qs, ks, qm, km = (np.asarray(a, dtype=np.float64) for a in (qs, ks, qm, km))
    L, D = qs.shape[-2], qs.shape[-1]
    if rope:
        cos, sin = rope_tables(L, D)
        qs_r, ks_r = apply_rope(qs, cos, sin), apply_rope(ks, cos, sin)
    else:
        cos = sin = None
        qs_r, ks_r = qs, ks
    s_self = scale * _mm(qs_r, _tr(ks_r))
    s_multi = scale * _mm(qm, _tr(km))
    return qs_r, ks_r, s_self, s_multi, cos, sin


def _probs(s_self, s_multi, cross, key_pad):
    s = np.where(cross[:, None], s_multi, s_self)
    if key_pad is not None:
        s = np.where(np.asarray(key_pad, dtype=bool)[:, None, None, :], -np.inf, s)
    m = s.max(axis=-1, keepdims=True)
    dead = ~np.isfinite(m)  # every key padded
    m = np.where(dead, 0.0, m)
    e = np.exp(s - m)
    l = e.sum(axis=-1, keepdims=True)
    p = np.where(l > 0, e / np.where(l > 0, l, 1.0), 0.0)
    lse = np.where(l[..., 0] > 0, m[..., 0] + np.log(np.where(l[..., 0] > 0, l[..., 0], 1.0)), -np.inf)
    return p, lse


def fmix32(x):
    """MurmurHash3's 32-bit finaliser, elementwise on uint32 arrays."""
    x = np.asarray(x, dtype=np.uint32).copy()
    x ^= x >> np.uint32(16)
    x *= np.uint32(0x85EBCA6B)
    x ^= x >> np.uint32(13)
    x *= np.uint32(0xC2B2AE35)
    x ^= x >> np.uint32(16)
    return x


def dropout_threshold(p):
    """round(p * 2^24): an element is kept when the top 24 bits of its hash
    are >= this."""
    return int(np.floor(np.float64(np.float32(p)) * 16777216.0 + 0.5))


def dropout_keep(B, H, L, p, seed):
    """(B, H, L, L) bool keep mask of attention dropout (the definition in
    ``include/mpattn.h``): element (b, h, i, j) is kept when
    ``fmix32(row ^ (j * 0x85EBCA77 + hi)) >> 8 >= round(p * 2^24)`` with
    ``row = fmix32(lo ^ (b*H + h) * 0xC2B2AE3D ^ i * 0x9E3779B1)``, lo / hi
    the low / high 32 bits of ``seed``; all arithmetic modulo 2^32."""
    seed = int(seed) & 0xFFFFFFFFFFFFFFFF
    lo, hi = np.uint32(seed & 0xFFFFFFFF), np.uint32(seed >> 32)
    with np.errstate(over="ignore"):
        bh = np.arange(B * H, dtype=np.uint32)[:, None]
        i = np.arange(L, dtype=np.uint32)[None, :]
        row = fmix32(lo ^ (bh * np.uint32(0xC2B2AE3D)) ^ (i * np.uint32(0x9E3779B1)))  # (BH, L)
        col = np.arange(L, dtype=np.uint32) * np.uint32(0x85EBCA77) + hi               # (L,)
        r = fmix32(row[:, :, None] ^ col[None, None, :])
    keep = (r >> np.uint32(8)) >= np.uint32(dropout_threshold(p))
    return keep.reshape(B, H, L, L)


def _dropout_factor(shape, dropout_p, dropout_seed):
    """Z / (1 - p) as float64 (B, H, L, L), or None without dropout."""
    if not dropout_p:
        return None
    B, H, L = shape[0], shape[1], shape[2]
    return dropout_keep(B, H, L, dropout_p, dropout_seed) / (1.0 - np.float64(np.float32(dropout_p)))


def mpattn_forward(qs, ks, vs, qm, km, vm, chain_ids=None, chain_mask=None, key_pad=None,
                   rope=False, scale=1.0, sqrt_softmax=False, dropout_p=0.0, dropout_seed=0):
    """Multi-pathway attention forward in float64.

    Inputs (B, H, L, D); ``chain_ids`` (B, L) or ``chain_mask`` (B, L, L)
    (True = different chains); ``key_pad`` (B, L) bool (True = padded key).
    ``rope`` applies RoPE to q_self/k_self; ``scale`` multiplies both logits.
    ``dropout_p`` > 0 multiplies P by ``dropout_keep(...) / (1 - p)`` after
    the softmax (the LSE stays that of the undropped softmax).
    Returns ``(out (B,H,L,D), lse (B,H,L))``; lse is in natural-log units.
    """
    cross = cross_mask(chain_ids, chain_mask)
    _, _, s_self, s_multi, _, _ = _prepare(qs, ks, qm, km, rope, scale)
    p, lse = _probs(s_self, s_multi, cross, key_pad)
    w = np.sqrt(p) if sqrt_softmax else p
    z = _dropout_factor(np.shape(qs), dropout_p, dropout_seed)
    if z is not None:
        w = w * z
    c = cross[:, None]
    vs, vm = np.asarray(vs, np.float64), np.asarray(vm, np.float64)
    out = _mm(np.where(c, 0.0, w), vs) + _mm(np.where(c, w, 0.0), vm)
    return out, lse


def mpattn_backward(qs, ks, vs, qm, km, vm, grad_out, chain_ids=None, chain_mask=None,
                    key_pad=None, rope=False, scale=1.0, sqrt_softmax=False, dropout_p=0.0,
                    dropout_seed=0):
    """Gradients (dq_s, dk_s, dv_s, dq_m, dk_m, dv_m) of
    ``sum(grad_out * mpattn_forward(...)[0])`` in float64."""
    cross = cross_mask(chain_ids, chain_mask)
    qs_r, ks_r, s_self, s_multi, cos, sin = _prepare(qs, ks, qm, km, rope, scale)
    qm, km = np.asarray(qm, np.float64), np.asarray(km, np.float64)
    vs, vm = np.asarray(vs, np.float64), np.asarray(vm, np.float64)
    g = np.asarray(grad_out, np.float64)
    p, _ = _probs(s_self, s_multi, cross, key_pad)
    c = cross[:, None]
    w = np.sqrt(p) if sqrt_softmax else p
    z = _dropout_factor(np.shape(qs), dropout_p, dropout_seed)
    wz = w if z is None else w * z  # the weights that multiply V
    w_s, w_m = np.where(c, 0.0, wz), np.where(c, wz, 0.0)
    dv_s = _mm(_tr(w_s), g)
    dv_m = _mm(_tr(w_m), g)
    # dW_ij = dO_i . V_sel(ij), j, through the dropout factor
    dw = np.where(c, _mm(g, _tr(vm)), _mm(g, _tr(vs)))
    if z is not None:
        dw = dw * z
    if sqrt_softmax:
        # W = sqrt(P): P * dP = W * dW / 2
        pdp = 0.5 * w * dw
    else:
        pdp = p * dw
    ds = pdp - p * pdp.sum(axis=-1, keepdims=True)
    ds_s, ds_m = np.where(c, 0.0, ds), np.where(c, ds, 0.0)
    dq_s = scale * _mm(ds_s, ks_r)
    dk_s = scale * _mm(_tr(ds_s), qs_r)
    dq_m = scale * _mm(ds_m, km)
    dk_m = scale * _mm(_tr(ds_m), qm)
    if rope:
        dq_s = apply_rope_transpose(dq_s, cos, sin)
        dk_s = apply_rope_transpose(dk_s, cos, sin)
    return dq_s, dk_s, dv_s, dq_m, dk_m, dv_m


def combine_forward(intra_logits, inter_logits, chain_mask, vs, vm, dropout_p=0.0,
                    dropout_seed=0):
    """Materialised-logit combine in float64: ``where(chain_mask, inter,
    intra)`` -> one softmax over keys -> split by pathway -> ``P_intra @ Vs +
    P_inter @ Vm`` (the contract of ``fused_multimer_combine``,
    ``mint_plus/models/kernels/__init__.py:93-176``, and of the eager
    ``modules_plus.py:178-194``). Logits already carry the scale and -inf at
    padded keys; an all -inf row gives 0. Dropout as in ``mpattn_forward``.
    Returns ``(out, lse)``."""
    cross = np.asarray(chain_mask, dtype=bool)
    il, el = np.asarray(intra_logits, np.float64), np.asarray(inter_logits, np.float64)
    p, lse = _probs(il, el, cross, None)
    z = _dropout_factor(np.shape(il), dropout_p, dropout_seed)
    if z is not None:
        p = p * z
    c = cross[:, None]
    vs, vm = np.asarray(vs, np.float64), np.asarray(vm, np.float64)
    out = np.einsum("bhij,bhjd->bhid", np.where(c, 0.0, p), vs) + \
        np.einsum("bhij,bhjd->bhid", np.where(c, p, 0.0), vm)
    return out, lse


def combine_backward(intra_logits, inter_logits, chain_mask, vs, vm, grad_out, dropout_p=0.0,
                     dropout_seed=0):
    """Gradients (d_intra_logits, d_inter_logits, d_vs, d_vm) of
    ``sum(grad_out * combine_forward(...)[0])`` in float64 (the contract of
    ``fused_multimer_combine_bwd``, ``kernels/__init__.py:247-286``)."""
    cross = np.asarray(chain_mask, dtype=bool)
    il, el = np.asarray(intra_logits, np.float64), np.asarray(inter_logits, np.float64)
    vs, vm = np.asarray(vs, np.float64), np.asarray(vm, np.float64)
    g = np.asarray(grad_out, np.float64)
    p, _ = _probs(il, el, cross, None)
    c = cross[:, None]
    z = _dropout_factor(np.shape(il), dropout_p, dropout_seed)
    pz = p if z is None else p * z
    d_vs = np.einsum("bhij,bhid->bhjd", np.where(c, 0.0, pz), g)
    d_vm = np.einsum("bhij,bhid->bhjd", np.where(c, pz, 0.0), g)
    dw = np.where(c, _mm(g, _tr(vm)), _mm(g, _tr(vs)))
    if z is not None:
        dw = dw * z
    pdp = p * dw
    ds = pdp - p * pdp.sum(axis=-1, keepdims=True)
    return np.where(c, 0.0, ds), np.where(c, ds, 0.0), d_vs, d_vm


def mpattn_forward_loops(qs, ks, vs, qm, km, vm, chain_ids, key_pad=None, rope=False, scale=1.0):
    """Pure-Python triple loop of the same forward, for tiny inputs only.

    Written element by element from the definition (rotation of each pair
    (d, d + D/2), logit selection per (i, j), max-subtracted softmax), as an
    independent cross-check of the vectorised ``mpattn_forward``.
    """
    import math
    B, H, L, D = len(qs), len(qs[0]), len(qs[0][0]), len(qs[0][0][0])
    half = D // 2

    def rot(x, pos):
        if not rope:
            return list(x)
        y = [0.0] * D
        for i in range(half):
            inv = float(np.float32(1.0 / ROPE_BASE ** (2 * i / D)))
            a = float(np.float32(np.float32(pos) * np.float32(inv)))
            y[i] = x[i] * math.cos(a) - x[i + half] * math.sin(a)
            y[i + half] = x[i + half] * math.cos(a) + x[i] * math.sin(a)
        return y

    out = [[[[0.0] * D for _ in range(L)] for _ in range(H)] for _ in range(B)]
    for b in range(B):
        for h in range(H):
            kr = [rot(ks[b][h][j], j) for j in range(L)]
            for i in range(L):
                qr = rot(qs[b][h][i], i)
                logits, vals = [], []
                for j in range(L):
                    if key_pad is not None and key_pad[b][j]:
                        continue
                    if chain_ids[b][i] == chain_ids[b][j]:
                        s = scale * sum(qr[d] * kr[j][d] for d in range(D))
                        v = vs[b][h][j]
                    else:
                        s = scale * sum(qm[b][h][i][d] * km[b][h][j][d] for d in range(D))
                        v = vm[b][h][j]
                    logits.append(s)
                    vals.append(v)
                if not logits:
                    continue
                mx = max(logits)
                e = [math.exp(s - mx) for s in logits]
                tot = sum(e)
                for d in range(D):
                    out[b][h][i][d] = sum(e[j] * vals[j][d] for j in range(len(e))) / tot
    return np.array(out)
