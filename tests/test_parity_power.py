"""The GPU parity comparisons can fail (CPU only).

For the forward and backward GPU parity cases of ``tests/test_fwd_gpu.py``
and ``tests/test_bwd_gpu.py``, this runs the case's own input generator and
the same comparison (``tests/parity.py``) on CPU oracle results and checks:

* planted mistakes are rejected: zeroed or halved output, swapped V
  pathways, one 256-query block zeroed, dropped RoPE (cases whose logits
  RoPE moves by O(1)); for the backward, each of dQ/dK of either pathway
  zeroed, dQ and dK swapped, dQ and dK halved, swapped pathways, one
  256-query block of dQ_self zeroed, dropped RoPE; the same for the fp32
  backward cases of ``tests/test_bwd32_gpu.py`` at the fp32 bound;
* the comparison accepts the oracle evaluated on the operands rounded as
  the kernels round them (fused RoPE: rotated Q and K rounded to the input
  dtype), so a correct kernel is not rejected by the rounding of its
  operands.

The oracle here is ``oracle/torch_ref.py`` in float64 (pinned to the numpy
oracle in ``tests/test_oracle.py``), with torch autograd for gradients. For
the full-size shapes the check runs on a slice of the same inputs (sample 0,
and heads 0-3 at the 3B shape): samples and heads are independent and
identically distributed, and a mistake that every element shares is
rejected on any slice.
"""
import numpy as np
import pytest
import torch

import parity as P
import test_bwd32_gpu as BW32
import test_bwd_gpu as BW
import test_fwd_gpu as FW
from oracle import mpattn_oracle as orc
from oracle import torch_ref


def _block(B, H, L):
    """(b, h, query slice) of the 256-query block a planted mistake zeroes."""
    q0 = 256 if L >= 512 else 0
    return B - 1, H - 1, slice(q0, min(L, q0 + 256))


def check_fwd_case(xs, cid, kp, rope, scale, dtype=torch.bfloat16, rope_matters=False,
                   rounded_ref=False):
    """rounded_ref: the GPU test compares against the oracle on the rounded
    operands (``parity.round_operands``), so that is the reference here."""
    B, H, L, D = xs[0].shape
    exact = P.ref_forward(xs, cid, kp, rope, scale)
    # a correct kernel's operand rounding passes
    em, sc = P.round_operands(xs, D, scale, rope, dtype)
    emo = P.ref_forward([torch.from_numpy(e) for e in em], cid, kp, False, sc)
    if rounded_ref:
        ref = emo
        rel = np.linalg.norm(emo - exact) / np.linalg.norm(exact)
        assert rel < 2e-2, rel   # the rounding is a small perturbation of the exact result
    else:
        ref = exact
        assert P.compare16(emo, ref) is None, P.compare16(emo, ref)
    bad = {"zero": ref * 0, "half": ref * 0.5}
    blk = ref.copy()
    b, h, qs = _block(B, H, L)
    blk[b, h, qs] = 0
    bad["block"] = blk
    bad["swap_v"] = P.ref_forward(xs, cid, kp, rope, scale, swap_v=True)
    if rope_matters:
        bad["no_rope"] = P.ref_forward(xs, cid, kp, False, scale)
    passed = [k for k, v in bad.items() if P.compare16(v, ref) is None]
    assert not passed, f"planted mistakes not rejected: {passed}"


def _worst_ratio(got, ref):
    """Largest |got - ref| / (atol + rtol |ref|) over the gradient tensors."""
    return max(float((np.abs(g - r) / (P.ATOL16 + P.RTOL16 * np.abs(r))).max()) for g, r in zip(got, ref))


def check_bwd_case(xs, go, cid, kp, rope, scale, dtype=torch.bfloat16, rope_matters=False,
                   rounded_ref=False, sqrt=False, mistakes=True):
    """rounded_ref: the GPU test's reference is autograd with the rotated
    Q_self/K_self rounded to dtype (``parity.ref_grads``). The backward's
    rounding model (``parity.emulate_bwd16``) must stay within half the
    bound of the reference (the calibration of each case's dO scale)."""
    B, H, L, D = xs[0].shape
    if sqrt:
        a = [x.double().numpy() for x in xs]
        ref = orc.mpattn_backward(*a, go.double().numpy(), chain_ids=cid, key_pad=kp, rope=rope,
                                  scale=scale, sqrt_softmax=True)
    else:
        ref = P.ref_grads(xs, go, cid, kp, rope, scale, round_dtype=dtype if rounded_ref else None)
    em = P.emulate_bwd16(xs, go, cid, kp, rope, scale, dtype, sqrt_softmax=sqrt)
    ratio = _worst_ratio(em, ref)
    assert ratio <= 0.5, f"rounding model uses {ratio:.2f} of the bound"
    if rounded_ref:
        exact = P.ref_grads(xs, go, cid, kp, rope, scale)
        for r, x in zip(ref, exact):
            rel = np.linalg.norm(r - x) / np.linalg.norm(x)
            assert rel < 2e-2, rel   # operand rounding: a small perturbation
    if not mistakes:
        return
    names = P.GRAD_NAMES
    cands = {}
    for i in (0, 1, 3, 4):
        g = list(ref)
        g[i] = g[i] * 0
        cands[f"zero_{names[i]}"] = g
    g = list(ref)
    g[0], g[1], g[3], g[4] = ref[1], ref[0], ref[4], ref[3]
    cands["swap_dq_dk"] = g
    g = list(ref)
    for i in (0, 1, 3, 4):
        g[i] = g[i] * 0.5
    cands["half_dq_dk"] = g
    g = list(ref)
    blk = ref[0].copy()
    b, h, qs = _block(B, H, L)
    blk[b, h, qs] = 0
    g[0] = blk
    cands["block_dq_self"] = g
    cands["swap_pathways"] = P.ref_grads(xs, go, cid, kp, rope, scale, swap_v=True)
    if rope_matters:
        cands["no_rope"] = P.ref_grads(xs, go, cid, kp, False, scale)
    passed = [k for k, v in cands.items() if not P.compare_grads16(v, ref)]
    assert not passed, f"planted mistakes not rejected: {passed}"


# ---------------------------------------------------------------- forward

@pytest.mark.parametrize("D,L", FW.SMALL)
def test_power_fwd_small(D, L):
    xs, cid, kp = FW.small_case(D, L)
    check_fwd_case(xs, cid, kp, True, D ** -0.5)


@pytest.mark.parametrize("n", FW.CHAIN_COUNTS)
def test_power_fwd_chains(n):
    xs, cid, kp = FW.chain_case(n)
    check_fwd_case(xs, cid, kp, True, 32 ** -0.5)


@pytest.mark.parametrize("B,H,L,D,nchains,dense", FW.DISPATCH)
def test_power_fwd_dispatch(B, H, L, D, nchains, dense):
    xs, cid, kp = FW.dispatch_case(B, H, L, D, nchains)
    check_fwd_case(xs, cid, kp, True, D ** -0.5)


@pytest.mark.parametrize("D", FW.ROPE_SHARP)
def test_power_fwd_rope_sharp(D):
    xs, cid, kp = FW.rope_sharp_case(D)
    check_fwd_case(xs, cid, kp, True, D ** -0.5, rope_matters=True, rounded_ref=True)


def test_power_fwd_headline():
    xs, cid, kp = FW.headline_case()
    D = xs[0].shape[3]
    check_fwd_case([x[:1] for x in xs], cid[:1], kp[:1], True, D ** -0.5)


@pytest.mark.parametrize("L,D", FW.DENSE_NP[:3])
def test_power_fwd_dense_not_partition(L, D):
    xs, cm, kp = FW.dense_np_case(L, D)
    a = [x.double().numpy() for x in xs]
    ref, _ = orc.mpattn_forward(*a, chain_mask=cm.numpy(), key_pad=kp, rope=True, scale=D ** -0.5)
    # a correct kernel's operand rounding passes
    em, sc = P.round_operands(xs, D, D ** -0.5, True, torch.bfloat16)
    emo, _ = orc.mpattn_forward(*em, chain_mask=cm.numpy(), key_pad=kp, rope=False, scale=sc)
    assert P.compare16(emo, ref) is None, P.compare16(emo, ref)
    # rows 1 and 2 run as if their masks were partitions (labels of the rows)
    lab = torch.where(~cm, torch.arange(L)[None, None, :], L).amin(dim=2)
    as_part, _ = orc.mpattn_forward(*a, chain_mask=(lab[:, :, None] != lab[:, None, :]).numpy(),
                                    key_pad=kp, rope=True, scale=D ** -0.5)
    bad = {"zero": ref * 0, "half": ref * 0.5, "as_partition": as_part,
           "swap_v": orc.mpattn_forward(a[0], a[1], a[5], a[3], a[4], a[2], chain_mask=cm.numpy(),
                                        key_pad=kp, rope=True, scale=D ** -0.5)[0]}
    passed = [k for k, v in bad.items() if P.compare16(v, ref) is None]
    assert not passed, f"planted mistakes not rejected: {passed}"


@pytest.mark.parametrize("B,H,L,D", FW.CFG3B)
def test_power_fwd_3b(B, H, L, D):
    xs, cid, kp = FW.case3b(B, H, L, D)
    check_fwd_case([x[:1, :4] for x in xs], cid[:1], kp[:1], True, D ** -0.5)


# ---------------------------------------------------------------- backward

@pytest.mark.parametrize("D,L", BW.SMALL)
def test_power_bwd_small(D, L):
    xs, go, cid, kp = BW.small_case(D, L)
    check_bwd_case(xs, go, cid, kp, True, D ** -0.5)


@pytest.mark.parametrize("n", [3, 5])
def test_power_bwd_chains(n):
    xs, go, cid, kp = BW.chain_case(n)
    check_bwd_case(xs, go, cid, kp, True, 32 ** -0.5)


@pytest.mark.parametrize("B,H,L,D,nchains,dense", BW.DISPATCH)
def test_power_bwd_dispatch(B, H, L, D, nchains, dense):
    xs, go, cid, kp = BW.dispatch_case(B, H, L, D, nchains)
    check_bwd_case(xs, go, cid, kp, True, D ** -0.5)


@pytest.mark.parametrize("D", BW.ROPE_SHARP)
def test_power_bwd_rope_sharp(D):
    xs, go, cid, kp = BW.rope_sharp_case(D)
    check_bwd_case(xs, go, cid, kp, True, D ** -0.5, rope_matters=True, rounded_ref=True)


def test_power_bwd_autograd():
    xs, go, cid, kp = BW.autograd_case()
    check_bwd_case(xs, go, cid, kp, True, 32 ** -0.5)


def test_power_bwd_headline():
    xs, go, cid, kp = BW.headline_case()
    D = xs[0].shape[3]
    b = BW.HEADLINE_SAMPLES[0]
    sl = slice(b, b + 1)
    check_bwd_case([x[sl] for x in xs], go[sl], cid[sl], kp[sl], True, D ** -0.5)


@pytest.mark.parametrize("B,H,L,D", BW.CFG3B)
def test_power_bwd_3b(B, H, L, D):
    xs, go, cid, kp = BW.case3b(B, H, L, D)
    check_bwd_case([x[:1, :4] for x in xs], go[:1, :4], cid[:1], kp[:1], True, D ** -0.5)


@pytest.mark.parametrize("n", [1])
def test_power_bwd_one_chain(n):
    xs, go, cid, kp = BW.chain_case(n)
    check_bwd_case(xs, go, cid, kp, True, 32 ** -0.5, mistakes=False)


@pytest.mark.parametrize("D", [32, 64])
def test_power_bwd_dense_norope(D):
    xs, go, cid, kp = BW.dense_norope_case(D)
    check_bwd_case(xs, go, cid, kp, False, 1.0)


@pytest.mark.parametrize("D", [16, 32, 64])
def test_power_bwd_sqrt(D):
    xs, go, cid, kp = BW.sqrt_case(D)
    check_bwd_case(xs, go, cid, kp, True, D ** -0.5, sqrt=True, mistakes=False)


@pytest.mark.parametrize("dtype,shift,spread,go_std", BW.RANGE)
def test_power_bwd_range_calibration(dtype, shift, spread, go_std):
    xs, go, cid, kp = BW.range_case(dtype, shift, spread, go_std)
    check_bwd_case(xs, go, cid, kp, False, 1.0, dtype=dtype, mistakes=False)


@pytest.mark.parametrize("L,D", [(256, 32), (200, 32), (1000, 32), (136, 64)])
def test_power_bwd_dense_tiles(L, D):
    xs, go, cid, kp = P.bwd_inputs(2, 2, L, D, torch.bfloat16, seed=41 + L + D, nchains=3)
    check_bwd_case(xs, go, cid, kp, True, D ** -0.5)


def test_power_bwd_all_padded_sample():
    xs, go, cid, kp = P.bwd_inputs(2, 2, 96, 32, torch.bfloat16, seed=19, pad=False)
    kp[1, :] = True
    check_bwd_case(xs, go, cid, kp, True, 32 ** -0.5, mistakes=False)


def test_power_bwd_fp16():
    xs, go, cid, kp = P.bwd_inputs(2, 3, 190, 32, torch.float16, seed=17)
    check_bwd_case(xs, go, cid, kp, True, 32 ** -0.5, dtype=torch.float16)


@pytest.mark.parametrize("L,D", BW.DENSE_NP)
def test_power_bwd_dense_not_partition(L, D):
    xs, go, cm, kp = BW.dense_np_case(L, D)
    a = [x.double().numpy() for x in xs]
    ref = orc.mpattn_backward(*a, go.double().numpy(), chain_mask=cm.numpy(), key_pad=kp, rope=True,
                              scale=D ** -0.5)
    em = P.emulate_bwd16(xs, go, None, kp, True, D ** -0.5, torch.bfloat16, cross=cm)
    ratio = _worst_ratio(em, ref)
    assert ratio <= 0.5, f"rounding model uses {ratio:.2f} of the bound"
    lab = torch.where(~cm, torch.arange(L)[None, None, :], L).amin(dim=2)
    as_part = orc.mpattn_backward(*a, go.double().numpy(), chain_mask=(lab[:, :, None] != lab[:, None, :]).numpy(),
                                  key_pad=kp, rope=True, scale=D ** -0.5)
    names = P.GRAD_NAMES
    cands = {"as_partition": list(as_part)}
    for i in (0, 1, 3, 4):
        g = list(ref)
        g[i] = g[i] * 0
        cands[f"zero_{names[i]}"] = g
    g = list(ref)
    g[0], g[1], g[3], g[4] = ref[1], ref[0], ref[4], ref[3]
    cands["swap_dq_dk"] = g
    passed = [k for k, v in cands.items() if not P.compare_grads16(v, ref)]
    assert not passed, f"planted mistakes not rejected: {passed}"


def test_power_detects_planted_oracle_rope_mistake():
    """A mistake planted in the oracle itself (RoPE sign flipped: the
    rotation by -theta) is rejected by the fused-RoPE comparison."""
    xs, cid, kp = FW.rope_sharp_case(32)
    ref = P.ref_forward(xs, cid, kp, True, 32 ** -0.5)
    L, D = xs[0].shape[2], 32
    cos, sin = torch_ref.rope_tables(L, D, "cpu")
    a = [x.double() for x in xs]
    a[0] = torch_ref.apply_rope(a[0], cos, -sin)
    a[1] = torch_ref.apply_rope(a[1], cos, -sin)
    bad = P.ref_forward(a, cid, kp, False, 32 ** -0.5)
    assert P.compare16(bad, ref) is not None
    assert np.isfinite(ref).all()


# ---------------------------------------------------------------- fp32 backward

def _grads32_autograd(xs, go, cid, kp, rope, scale, sqrt_softmax, dense, dtype):
    """Gradients of sum(out * go) by torch autograd through ``torch_ref`` in
    ``dtype`` (float32: a correct fp32 implementation's arithmetic)."""
    leaves = [torch.from_numpy(x).to(dtype).requires_grad_(True) for x in xs]
    sel = {}
    if dense:
        c = torch.from_numpy(cid)
        sel["chain_mask"] = c[:, :, None] != c[:, None, :]
    else:
        sel["chain_ids"] = torch.from_numpy(cid)
    if sqrt_softmax:
        # sqrt(P) as exp((s - LSE) / 2): autograd through sqrt would give
        # 0 * inf at the padded keys (torch_ref is a forward reference)
        qs, ks, vs, qm, km, vm = leaves
        if rope:
            cos, sin = torch_ref.rope_tables(xs[0].shape[2], xs[0].shape[3], "cpu", dtype)
            qs, ks = torch_ref.apply_rope(qs, cos, sin), torch_ref.apply_rope(ks, cos, sin)
        c = sel.get("chain_mask")
        if c is None:
            ci = sel["chain_ids"]
            c = ci[:, :, None] != ci[:, None, :]
        c = c[:, None]
        sc = torch.where(c, scale * qm @ km.transpose(-1, -2), scale * qs @ ks.transpose(-1, -2))
        sc = sc.masked_fill(torch.from_numpy(kp)[:, None, None, :], float("-inf"))
        w = torch.exp(0.5 * (sc - torch.logsumexp(sc, dim=-1, keepdim=True)))
        out = w.masked_fill(c, 0.0) @ vs + w.masked_fill(~c, 0.0) @ vm
    else:
        out, _ = torch_ref.forward(*leaves, key_pad=torch.from_numpy(kp), rope=rope, scale=scale,
                                   dtype=dtype, chunk=1, **sel)
    (out * torch.from_numpy(go).to(dtype)).sum().backward()
    return [leaf.grad.double().numpy() for leaf in leaves]


def check_bwd32_case(case, rope, scale, sqrt_softmax=False, dense=False):
    """The fp32 GPU comparison (``parity.compare_grads32``) accepts fp32
    autograd of the reference forward with margin (at most 1/4 of each
    bound) and rejects the planted mistakes."""
    xs, go, cid, kp, ref = case
    B, H, L, D = xs[0].shape
    f32 = _grads32_autograd(xs, go, cid, kp, rope, scale, sqrt_softmax, dense, torch.float32)
    for n, g, r in zip(P.GRAD_NAMES, f32, ref):
        err = float(np.abs(g - r).max())
        nr = float(np.linalg.norm(r))
        rel = float(np.linalg.norm(g - r)) / nr if nr > 0 else float(np.linalg.norm(g))
        assert err <= P.ATOL32 / 4 and rel <= P.RELF32 / 4, (n, err, rel)
    names = P.GRAD_NAMES
    cands = {}
    for i in (0, 1, 3, 4):
        if np.any(ref[i] != 0):
            g = list(ref)
            g[i] = g[i] * 0
            cands[f"zero_{names[i]}"] = g
    g = list(ref)
    g[0], g[1], g[3], g[4] = ref[1], ref[0], ref[4], ref[3]
    cands["swap_dq_dk"] = g
    g = list(ref)
    for i in (0, 1, 3, 4):
        g[i] = g[i] * 0.5
    cands["half_dq_dk"] = g
    g = list(ref)
    g[0], g[1], g[2], g[3], g[4], g[5] = ref[3], ref[4], ref[5], ref[0], ref[1], ref[2]
    cands["swap_pathways"] = g
    g = list(ref)
    blk = ref[0].copy()
    b, h, qs = _block(B, H, L)
    blk[b, h, qs] = 0
    g[0] = blk
    cands["block_dq_self"] = g
    if rope:
        sel = dict(chain_mask=(cid[:, :, None] != cid[:, None, :])) if dense else dict(chain_ids=cid)
        cands["no_rope"] = orc.mpattn_backward(*[x.astype(np.float64) for x in xs], go.astype(np.float64),
                                               key_pad=kp, rope=False, scale=scale,
                                               sqrt_softmax=sqrt_softmax, **sel)
    passed = [k for k, v in cands.items() if not P.compare_grads32(v, ref)]
    assert not passed, f"planted mistakes not rejected: {passed}"


@pytest.mark.parametrize("D,L", BW32.SMALL)
def test_power_bwd32_small(D, L):
    check_bwd32_case(BW32.small_case(D, L), True, D ** -0.5)


@pytest.mark.parametrize("n", BW32.CHAIN_COUNTS)
def test_power_bwd32_chains(n):
    check_bwd32_case(BW32.chain_case(n), True, 0.25)


@pytest.mark.parametrize("D", [32, 64])
def test_power_bwd32_dense(D):
    check_bwd32_case(BW32.dense_case(D), False, 1.0, dense=True)


@pytest.mark.parametrize("D", [16, 32])
def test_power_bwd32_sqrt(D):
    check_bwd32_case(BW32.sqrt_case(D), True, D ** -0.5, sqrt_softmax=True)


def test_power_bwd32_long_rows():
    B, H, L, D, n = BW32.LARGE[2]
    check_bwd32_case(BW32.large_case(B, H, L, D, n), True, D ** -0.5)
