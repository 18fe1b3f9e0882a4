"""Inputs and comparisons shared by the GPU parity tests and by the CPU test
that plants mistakes in oracle outputs (``tests/test_parity_power.py``).

Why the inputs look the way they do. With the benchmark distribution
(Q, K, V ~ N(0, 1/D)) the softmax is almost uniform: O, dQ and dK are then a
few hundredths or less, below the 2e-2 absolute bound, and an all-zero
result would pass. The generators here keep the Q/K distribution (so the
logits, and every kernel path they select, are the benchmark's) and scale
what enters linearly:

* V entries ~ N(0, V_STD^2) (O is linear in V), so |O| is O(0.1-1);
* dO by sqrt(L) (every gradient is linear in dO), so dQ, dK, dV are O(1).

Each comparison holds two bounds, both of which must pass:

* elementwise ``|got - ref| <= 2e-2 + 1e-2 |ref|`` (the task's bf16 bound);
* per tensor ``||got - ref||_F <= 1e-2 ||ref||_F`` (catches a result that is
  uniformly a little wrong, e.g. a dropped scale, that the elementwise bound
  can let through where |ref| is small).

``tests/test_parity_power.py`` runs every GPU case's generator and
comparison on oracle outputs with planted mistakes (zeroed output or
gradients, dQ and dK swapped, pathways swapped, RoPE dropped, one 256-query
block zeroed) and asserts that each is rejected, and that the oracle on the
operands rounded the way the kernels round them is accepted.
"""
import numpy as np
import torch

from conftest import multi_chain_ids, tail_padding, two_chain_ids

ATOL16, RTOL16, RELF16 = 2e-2, 1e-2, 1e-2
V_STD = 4.0  # std of V entries in the discriminating inputs


def chains(rng, B, L, nchains):
    if nchains == "3b":
        return three_chain_ids(rng, B, L)
    return two_chain_ids(rng, B, L) if nchains == 2 else multi_chain_ids(rng, B, L, nchains)


def three_chain_ids(rng, B, L, lo=200, hi=800, limit=2048):
    """The 3B configuration's layout: three contiguous chains of ~U[lo, hi]
    tokens, resampled until their total is <= min(L, limit); the rest of the
    row is the padding tail (chain id 2, key padding set by ``pad_after``)."""
    cid = np.full((B, L), 2, dtype=np.int32)
    for b in range(B):
        while True:
            n = rng.integers(lo, hi + 1, size=3)
            if n.sum() <= min(L, limit):
                break
        cid[b, :n[0]] = 0
        cid[b, n[0]:n[0] + n[1]] = 1
        cid[b, n.sum():] = -1  # marks the tail for pad_after
    return cid


def pad_after(cid):
    """Key padding of a ``three_chain_ids`` layout (tail marked -1), with the
    tail's chain id reset to the last chain's."""
    kp = cid < 0
    cid[kp] = 2
    return kp


def fwd_inputs(B, H, L, D, dtype, seed, sigma=None, nchains=2, pad=True, v_std=V_STD):
    """Six (B, H, L, D) tensors in ``dtype`` plus chain ids and key padding.

    Q and K are N(0, sigma^2) with sigma = D^-1/2 by default (the benchmark
    distribution); V entries are N(0, v_std^2)."""
    rng = np.random.default_rng(seed)
    sigma = D ** -0.5 if sigma is None else sigma
    z = [rng.standard_normal((B, H, L, D)).astype(np.float32) for _ in range(6)]
    mul = [sigma, sigma, v_std, sigma, sigma, v_std]
    xs = [torch.from_numpy(x * m).to(dtype) for x, m in zip(z, mul)]
    cid = chains(rng, B, L, nchains)
    if nchains == "3b":
        kp = pad_after(cid)
    else:
        kp = tail_padding(rng, B, L) if pad else np.zeros((B, L), dtype=bool)
    return xs, cid, kp


def bwd_inputs(B, H, L, D, dtype, seed, sigma=None, nchains=2, pad=True, v_std=V_STD, go_log2=0):
    """``fwd_inputs`` plus an upstream gradient dO with entries of std
    sqrt(L) * 2^go_log2.

    ``go_log2`` is each case's calibration (``tests/test_parity_power.py``
    checks it): the largest power of two, at most the one that brings the
    largest gradient RMS to 1, for which the backward's rounding model
    (``emulate_bwd16``) stays within half the bound. Sharper softmaxes give
    larger gradients per unit dO and a larger share of rounding error from
    Delta = rowsum(round(O) dO), so they take smaller dO."""
    xs, cid, kp = fwd_inputs(B, H, L, D, dtype, seed, sigma, nchains, pad, v_std)
    rng = np.random.default_rng(seed + 7919)
    mul = L ** 0.5 * 2.0 ** go_log2
    go = torch.from_numpy(rng.standard_normal((B, H, L, D)).astype(np.float32) * mul).to(dtype)
    return xs, go, cid, kp


def shifted_logit_inputs(B, H, L, D, dtype, seed, shift, spread, nchains=2, v_std=V_STD):
    """Caller-side (pre-scaled, pre-rotated) operands whose logits are
    ``shift + N(0, spread^2)`` on both pathways: Q = q' + a e0, K = k' + b e0
    with q', k' orthogonal to e0 and a * b = shift, so <Q, K> = <q', k'> + shift.
    Used with rope=False, scale=1 (the reference's contract)."""
    rng = np.random.default_rng(seed)
    a = 3.5 if shift >= 0 else -3.5
    bcoef = shift / a
    sig = (spread ** 2 / (D - 1)) ** 0.25
    out = []
    for pw in range(2):
        q = rng.standard_normal((B, H, L, D)) * sig
        k = rng.standard_normal((B, H, L, D)) * sig
        q[..., 0] = a
        k[..., 0] = bcoef
        v = rng.standard_normal((B, H, L, D)) * v_std
        out += [q, k, v]
    xs = [torch.from_numpy(t.astype(np.float32)).to(dtype) for t in
          (out[0], out[1], out[2], out[3], out[4], out[5])]
    cid = chains(rng, B, L, nchains)
    kp = tail_padding(rng, B, L)
    return xs, cid, kp


def _as_np(x):
    if isinstance(x, torch.Tensor):
        return x.detach().double().cpu().numpy()
    return np.asarray(x, dtype=np.float64)


def compare16(got, ref):
    """Both bounds for one tensor; returns None if they hold, else a message."""
    g, r = _as_np(got), _as_np(ref)
    if g.shape != r.shape:
        return f"shape {g.shape} != {r.shape}"
    if not np.isfinite(g).all():
        return f"{int((~np.isfinite(g)).sum())} non-finite elements"
    err = np.abs(g - r)
    bound = ATOL16 + RTOL16 * np.abs(r)
    nbad = int((err > bound).sum())
    nr = float(np.linalg.norm(r))
    rel = float(np.linalg.norm(g - r)) / nr if nr > 0 else float(np.linalg.norm(g))
    msgs = []
    if nbad:
        msgs.append(f"{nbad} elements out of tolerance (max err {err.max():.4g}, "
                    f"worst excess {(err - bound).max():.4g})")
    if rel > RELF16:
        msgs.append(f"relative Frobenius error {rel:.4g} > {RELF16}")
    return "; ".join(msgs) if msgs else None


def compare16_torch(got, ref):
    """compare16 for large device tensors (evaluated in fp32/fp64 on device)."""
    g = got.double()
    r = ref.double()
    if not bool(torch.isfinite(g).all()):
        return "non-finite elements"
    err = (g - r).abs()
    bound = ATOL16 + RTOL16 * r.abs()
    nbad = int((err > bound).sum().item())
    nr = float(torch.linalg.vector_norm(r).item())
    rel = float(torch.linalg.vector_norm(g - r).item()) / nr if nr > 0 else float(
        torch.linalg.vector_norm(g).item())
    msgs = []
    if nbad:
        msgs.append(f"{nbad} elements out of tolerance (max err {err.max().item():.4g})")
    if rel > RELF16:
        msgs.append(f"relative Frobenius error {rel:.4g} > {RELF16}")
    return "; ".join(msgs) if msgs else None


def assert16(got, ref, what):
    msg = compare16(got, ref)
    assert msg is None, f"{what}: {msg}"


def assert16_torch(got, ref, what):
    msg = compare16_torch(got, ref)
    assert msg is None, f"{what}: {msg}"


GRAD_NAMES = ("dq_self", "dk_self", "dv_self", "dq_multi", "dk_multi", "dv_multi")


def compare_grads16(got, ref):
    """compare16 over the six gradients; returns the failures (name, msg)."""
    out = []
    for n, g, r in zip(GRAD_NAMES, got, ref):
        m = compare16(g, r)
        if m:
            out.append((n, m))
    return out


def assert_grads16(got, ref, what):
    bad = compare_grads16(got, ref)
    assert not bad, f"{what}: " + "; ".join(f"{n}: {m}" for n, m in bad)


# fp32 bound (the task's fp32 tolerance): max |gpu - ref| <= 1e-4 and
# ||gpu - ref||_F <= 1e-4 ||ref||_F per tensor.
ATOL32, RELF32 = 1e-4, 1e-4


def compare32(got, ref):
    """Both fp32 bounds for one tensor; returns None if they hold, else a message."""
    g, r = _as_np(got), _as_np(ref)
    if g.shape != r.shape:
        return f"shape {g.shape} != {r.shape}"
    if not np.isfinite(g).all():
        return f"{int((~np.isfinite(g)).sum())} non-finite elements"
    err = float(np.abs(g - r).max()) if g.size else 0.0
    nr = float(np.linalg.norm(r))
    rel = float(np.linalg.norm(g - r)) / nr if nr > 0 else float(np.linalg.norm(g))
    msgs = []
    if err > ATOL32:
        msgs.append(f"max err {err:.3g} > {ATOL32}")
    if rel > RELF32:
        msgs.append(f"relative Frobenius error {rel:.3g} > {RELF32}")
    return "; ".join(msgs) or None


def compare_grads32(got, ref):
    out = []
    for n, g, r in zip(GRAD_NAMES, got, ref):
        m = compare32(g, r)
        if m:
            out.append((n, m))
    return out


def assert_grads32(got, ref, what):
    bad = compare_grads32(got, ref)
    assert not bad, f"{what}: " + "; ".join(f"{n}: {m}" for n, m in bad)


def bwd32_inputs(B, H, L, D, seed, scale, rope=True, sigma=1.0, nchains=2, pad=True,
                 sqrt_softmax=False, dense=False):
    """fp32 backward case: Q/K entries N(0, sigma^2), V N(0, 1) (logit std
    about sigma^2 * sqrt(D) * scale), chain ids and key padding, and an
    upstream gradient N(0, 1) times the power of two that brings the largest
    oracle gradient RMS into [0.7, 1.4] (gradients are linear in dO, so the
    oracle's gradients are scaled by the same exact factor).

    Returns (xs, go, cid, kp, ref) with float32 numpy inputs and the float64
    oracle gradients."""
    from oracle import mpattn_oracle as orc
    rng = np.random.default_rng(seed)
    z = [rng.standard_normal((B, H, L, D)).astype(np.float32) for _ in range(6)]
    mul = [sigma, sigma, 1.0, sigma, sigma, 1.0]
    xs = [(x * np.float32(m)).astype(np.float32) for x, m in zip(z, mul)]
    cid = chains(rng, B, L, nchains)
    kp = tail_padding(rng, B, L) if pad else np.zeros((B, L), dtype=bool)
    go = rng.standard_normal((B, H, L, D)).astype(np.float32)
    sel = dict(chain_mask=(cid[:, :, None] != cid[:, None, :])) if dense else dict(chain_ids=cid)
    ref = orc.mpattn_backward(*[x.astype(np.float64) for x in xs], go.astype(np.float64), key_pad=kp,
                              rope=rope, scale=scale, sqrt_softmax=sqrt_softmax, **sel)
    rms = max(float(np.sqrt(np.mean(r ** 2))) for r in ref)
    f = 2.0 ** -round(np.log2(rms)) if rms > 0 else 1.0
    go = (go * np.float32(f)).astype(np.float32)
    ref = [r * f for r in ref]
    return xs, go, cid, kp, ref


def round_operands(xs, D, scale, rope, dtype):
    """The operands the 16-bit kernels feed their MFMAs: with fused RoPE, Q
    is rotated and multiplied by scale*log2(e) in fp32 and rounded once
    (the kernel divides the log2(e) back out through exp2), K_self is
    rotated in fp32 and rounded; without it they are the inputs as given.
    Returns float64 arrays and the scale to apply to their logits."""
    from oracle import mpattn_oracle as orc
    a = [_as_np(x) for x in xs]
    if not rope:
        return a, scale
    L = a[0].shape[2]
    cos, sin = orc.rope_tables(L, D)
    lg2e = np.float32(1.4426950408889634)
    f = np.float32(scale) * lg2e

    def rnd(v):
        return torch.from_numpy(v.astype(np.float32)).to(dtype).double().numpy()

    qs = rnd(orc.apply_rope(a[0], cos, sin).astype(np.float32) * f) / float(lg2e)
    ks = rnd(orc.apply_rope(a[1], cos, sin))
    qm = rnd(a[3].astype(np.float32) * f) / float(lg2e)
    return [qs, ks, a[2], qm, a[4], a[5]], 1.0


def ref_forward(xs, cid, kp, rope, scale, swap_v=False):
    """Oracle forward (``oracle/torch_ref.py`` in float64 on the CPU); swap_v
    exchanges the two V pathways (a planted mistake)."""
    from oracle import torch_ref
    a = [x.double() for x in xs]
    if swap_v:
        a[2], a[5] = a[5], a[2]
    out, _ = torch_ref.forward(*a, chain_ids=torch.from_numpy(cid), key_pad=torch.from_numpy(kp),
                               rope=rope, scale=scale, dtype=torch.float64, chunk=1)
    return out.numpy()


def round_st(x, dtype):
    """Rounding to dtype in the forward, identity for the gradient."""
    return x + (x.to(dtype).double() - x).detach()


def ref_grads(xs, go, cid, kp, rope, scale, swap_v=False, round_dtype=None):
    """Gradients of sum(out * go) w.r.t. the six inputs (torch autograd in
    float64). With round_dtype and rope, the logits are taken over the
    operands the 16-bit kernels feed their MFMAs with fused RoPE (both
    passes): R(q_self) * f, q_multi * f (f = scale * log2 e, fp32) and
    R(k_self), each rounded once to round_dtype; the rounding is the identity
    for the gradient."""
    from oracle import torch_ref
    leaves = [x.double().requires_grad_(True) for x in xs]
    a = list(leaves)
    if swap_v:
        a[2], a[5] = a[5], a[2]
    L, D = xs[0].shape[2], xs[0].shape[3]
    if round_dtype is not None and rope:
        cos, sin = torch_ref.rope_tables(L, D, "cpu")
        f = float(np.float32(scale) * np.float32(1.4426950408889634))
        a[0] = round_st(torch_ref.apply_rope(a[0], cos, sin) * f, round_dtype) / f
        a[1] = round_st(torch_ref.apply_rope(a[1], cos, sin), round_dtype)
        a[3] = round_st(a[3] * f, round_dtype) / f
        rope = False
    out, _ = torch_ref.forward(*a, chain_ids=torch.from_numpy(cid), key_pad=torch.from_numpy(kp),
                               rope=rope, scale=scale, dtype=torch.float64, chunk=1)
    (out * go.double()).sum().backward()
    g = [leaf.grad.numpy() for leaf in leaves]
    if swap_v:
        g[2], g[5] = g[5], g[2]
    return g


def _rnd(x, dtype):
    return x.to(dtype).to(torch.float64)


def emulate_bwd16(xs, go, cid, kp, rope, scale, dtype, sqrt_softmax=False, cross=None):
    """The six gradients computed the way the 16-bit backward kernels round
    (a model of their arithmetic, for calibrating the tests, not an oracle):
    with fused RoPE the logits come from the forward's folded, rounded
    operands (``ref_grads``); P from the exact
    LSE; dV = round(P)^T dO; dS = P (dP - Delta) (sqrt-softmax:
    W (dW - W Delta) / 2) rounded to ``dtype`` before dQ = scale dS K and
    dK = scale dS^T Q; Delta = rowsum(round(O) * dO); RoPE's transpose applied
    to dQ_self/dK_self in fp32; every gradient rounded to ``dtype``.
    Accumulations are exact (float64)."""
    from oracle import torch_ref
    a = [x.to(torch.float64) for x in xs]
    g = go.to(torch.float64)
    B, H, L, D = a[0].shape
    qs, ks, qm = a[0], a[1], a[3]
    if rope:  # the forward's folded, rounded operands (see ref_grads)
        cos, sin = torch_ref.rope_tables(L, D, "cpu")
        f = float(np.float32(scale) * np.float32(1.4426950408889634)) * (0.5 if sqrt_softmax else 1.0)
        qs = _rnd(torch_ref.apply_rope(qs, cos, sin).float().double() * f, dtype) / f
        ks = _rnd(torch_ref.apply_rope(ks, cos, sin).float().double(), dtype)
        qm = _rnd(qm * f, dtype) / f
    if cross is None:  # (or a given (B, L, L) "different chain" mask)
        c = torch.from_numpy(cid)
        cross = c[:, :, None] != c[:, None, :]
    cross = torch.as_tensor(cross)[:, None]
    pad = torch.from_numpy(kp)[:, None, None, :]
    s = torch.where(cross, scale * qm @ a[4].transpose(-1, -2), scale * qs @ ks.transpose(-1, -2))
    s = s.masked_fill(pad, float("-inf"))
    m = s.amax(-1, keepdim=True)
    m = torch.where(torch.isfinite(m), m, torch.zeros_like(m))
    e = torch.exp(s - m)
    lsum = e.sum(-1, keepdim=True)
    p = torch.where(lsum > 0, e / torch.where(lsum > 0, lsum, torch.ones_like(lsum)), torch.zeros_like(e))
    w = p.sqrt() if sqrt_softmax else p
    vsel_s, vsel_m = a[2], a[5]
    out = (w.masked_fill(cross, 0) @ vsel_s) + (w.masked_fill(~cross, 0) @ vsel_m)
    delta = (_rnd(out, dtype) * g).sum(-1, keepdim=True)
    dw = torch.where(cross, g @ vsel_m.transpose(-1, -2), g @ vsel_s.transpose(-1, -2))
    ds = 0.5 * w * (dw - w * delta) if sqrt_softmax else p * (dw - delta)
    ds16 = _rnd(ds, dtype)
    w16 = _rnd(w, dtype)
    ds_s, ds_m = ds16.masked_fill(cross, 0), ds16.masked_fill(~cross, 0)
    dv_s = w16.masked_fill(cross, 0).transpose(-1, -2) @ g
    dv_m = w16.masked_fill(~cross, 0).transpose(-1, -2) @ g
    dq_s, dk_s = scale * ds_s @ ks, scale * ds_s.transpose(-1, -2) @ qs
    dq_m, dk_m = scale * ds_m @ a[4], scale * ds_m.transpose(-1, -2) @ qm
    if rope:
        cos, sin = torch_ref.rope_tables(L, D, "cpu")
        h = D // 2

        def rot_t(x):  # transpose of x*cos + rotate_half(x)*sin
            x1, x2 = x[..., :h], x[..., h:]
            return torch.cat([x1 * cos + x2 * sin, x2 * cos - x1 * sin], -1)
        dq_s, dk_s = rot_t(dq_s), rot_t(dk_s)
    return [_rnd(t, dtype).numpy() for t in (dq_s, dk_s, dv_s, dq_m, dk_m, dv_m)]


def upstream_scale(grads, target=1.0):
    """Power of two 2^k such that the largest RMS over the gradient tensors
    times 2^k lies in (target/2, target]. Every gradient is linear in dO, so
    scaling dO by 2^k scales them exactly (also after rounding to bf16/fp16),
    and the 2e-2 absolute bound stays a few percent of their typical size."""
    import math
    rms = max(float(np.sqrt(np.mean(np.square(np.asarray(g, dtype=np.float64))))) for g in grads)
    if rms == 0:
        return 1.0
    return 2.0 ** math.floor(math.log2(target / rms))
