"""Parity of the materialised-logit combine kernels (mpattn_combine_fwd /
mpattn_combine_bwd through the C ABI) with the float64 oracle
(``oracle.mpattn_oracle.combine_forward`` / ``combine_backward``).

Tolerances: bf16 / fp16 |gpu - ref| <= 2e-2 + 1e-2 |ref|; fp32 max-abs 1e-4.
Gradients of the logits are small (about P), so they are also held to a
relative Frobenius error (2e-2 for 16-bit, 1e-5 for fp32), which a wrong
term would exceed.
"""
import numpy as np
import pytest
import torch

from conftest import multi_chain_ids, tail_padding
from oracle import mpattn_oracle as orc

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _m():
    import mint_plus_amd
    return mint_plus_amd


def make(B, H, L, D, dtype, seed, sigma=2.0, nchains=3):
    rng = np.random.default_rng(seed)
    il, el = (rng.standard_normal((B, H, L, L)) * sigma for _ in range(2))
    kp = tail_padding(rng, B, L, 0.15)
    il = np.where(kp[:, None, None, :], -np.inf, il)
    el = np.where(kp[:, None, None, :], -np.inf, el)
    vs, vm, go = (rng.standard_normal((B, H, L, D)) for _ in range(3))
    cid = multi_chain_ids(rng, B, L, nchains)
    cm = cid[:, :, None] != cid[:, None, :]
    # round through the dtype so the oracle sees the kernel's inputs
    r = lambda a: torch.from_numpy(a.astype(np.float32)).to(dtype)
    t = [r(a) for a in (il, el, vs, vm, go)]
    return t, cm


def tol(dtype):
    return (1e-4, 0.0) if dtype == torch.float32 else (2e-2, 1e-2)


def check(got, ref, dtype, what, rel_fro=None):
    atol, rtol = tol(dtype)
    got = got.double().cpu().numpy()
    err = np.abs(got - ref)
    bad = err > atol + rtol * np.abs(ref)
    assert not bad.any(), f"{what}: {bad.sum()} out of tolerance, max err {err.max():.3g}"
    if rel_fro is not None:
        e = np.linalg.norm(got - ref) / max(np.linalg.norm(ref), 1e-30)
        assert e <= rel_fro, f"{what}: relative Frobenius error {e:.3g}"


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("D", [16, 24, 32, 64])
@pytest.mark.parametrize("L", [16, 64, 100, 208, 257])
def test_combine_fwd(dtype, D, L):
    """L = 16, 64, 208 (16-bit rows of 16-byte multiples): the copy-staged
    kernel, with a partial last key stage (16, 208) and query blocks past L;
    L = 100, 257: the register-load kernel."""
    print(f"[combine fwd] {dtype} D={D} L={L}", flush=True)
    t, cm = make(2, 3, L, D, dtype, seed=100 + D + L)
    out = _m().fused_multimer_combine(*[x.to(DEV) for x in t[:2]], torch.from_numpy(cm).to(DEV),
                                      *[x.to(DEV) for x in t[2:4]])
    torch.cuda.synchronize()
    ref, _ = orc.combine_forward(*[x.double().numpy() for x in t[:2]], cm,
                                 *[x.double().numpy() for x in t[2:4]])
    check(out, ref, dtype, f"out {dtype} D={D} L={L}")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("D", [16, 32, 64])
@pytest.mark.parametrize("L", [64, 129, 208])
def test_combine_bwd(dtype, D, L):
    print(f"[combine bwd] {dtype} D={D} L={L}", flush=True)
    t, cm = make(2, 2, L, D, dtype, seed=200 + D + L)
    g = [x.to(DEV) for x in t]
    grads = _m().fused_multimer_combine_bwd(g[0], g[1], torch.from_numpy(cm).to(DEV), g[2], g[3],
                                            g[4])
    torch.cuda.synchronize()
    ref = orc.combine_backward(*[x.double().numpy() for x in t[:2]], cm,
                               *[x.double().numpy() for x in t[2:]])
    fro = 1e-5 if dtype == torch.float32 else 2e-2
    for name, a, r in zip(("d_intra_logits", "d_inter_logits", "d_vs", "d_vm"), grads, ref):
        assert a.dtype == dtype
        check(a, r, dtype, f"{name} {dtype} D={D} L={L}", rel_fro=fro)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("D", [16, 32, 64])
@pytest.mark.parametrize("L", [64, 129, 208])
@pytest.mark.parametrize("p", [0.0, 0.25])
def test_combine_bwd_with_forward_stats(dtype, D, L, p):
    """The backward given the forward's LSE and output (Delta = dO . O from
    them, no statistics pass over the logits) against the oracle, and
    against the backward that recomputes the statistics (LSE comes from the
    same arithmetic; Delta differs by the rounding of the stored O)."""
    print(f"[combine bwd fwd-stats] {dtype} D={D} L={L} p={p}", flush=True)
    t, cm = make(2, 2, L, D, dtype, seed=300 + D + L)
    g = [x.to(DEV) for x in t]
    cmt = torch.from_numpy(cm).to(DEV)
    m = _m()
    out, lse = m._lib.mpattn_combine_fwd(g[0], g[1], cmt, g[2], g[3], dropout_p=p,
                                         dropout_seed=11, need_lse=True)
    fast = m.fused_multimer_combine_bwd(g[0], g[1], cmt, g[2], g[3], g[4], dropout_p=p,
                                        dropout_seed=11, lse=lse, output=out)
    slow = m.fused_multimer_combine_bwd(g[0], g[1], cmt, g[2], g[3], g[4], dropout_p=p,
                                        dropout_seed=11)
    torch.cuda.synchronize()
    ref = orc.combine_backward(*[x.double().numpy() for x in t[:2]], cm,
                               *[x.double().numpy() for x in t[2:]], dropout_p=p,
                               dropout_seed=11)
    fro = 1e-5 if dtype == torch.float32 else 2e-2
    for name, a, b, r in zip(("d_intra_logits", "d_inter_logits", "d_vs", "d_vm"), fast, slow, ref):
        assert a.dtype == dtype
        check(a, r, dtype, f"{name} {dtype} D={D} L={L} p={p}", rel_fro=fro)
        check(a, b.double().cpu().numpy(), dtype, f"{name} vs recomputed statistics")


def test_combine_bwd_stats_arguments():
    """lse without out (or out without lse) is refused before any launch."""
    t, cm = make(1, 2, 64, 32, torch.bfloat16, seed=1)
    g = [x.to(DEV) for x in t]
    cmt = torch.from_numpy(cm).to(DEV)
    lse = torch.zeros(1, 2, 64, dtype=torch.float32, device=DEV)
    with pytest.raises(ValueError):
        _m().fused_multimer_combine_bwd(g[0], g[1], cmt, g[2], g[3], g[4], lse=lse)
    with pytest.raises(ValueError):
        _m().fused_multimer_combine_bwd(g[0], g[1], cmt, g[2], g[3], g[4], lse=lse[:, :1],
                                        output=g[2])


def test_combine_all_padded_row_and_strided_logits():
    """A sample whose keys are all -inf gives zero output and gradients (the
    reference kernel would produce NaN); logits given as a strided slice of a
    wider buffer are read in place."""
    print("[combine padded+strided]", flush=True)
    dtype = torch.bfloat16
    t, cm = make(2, 2, 80, 32, dtype, seed=7)
    t[0][1] = float("-inf")
    t[1][1] = float("-inf")
    wide = torch.zeros(2, 2, 80, 96, dtype=dtype)
    wide[..., 8:88] = t[0]
    g = [x.to(DEV) for x in t]
    il = wide.to(DEV)[..., 8:88]
    out = _m().fused_multimer_combine(il, g[1], torch.from_numpy(cm).to(DEV), g[2], g[3])
    grads = _m().fused_multimer_combine_bwd(il, g[1], torch.from_numpy(cm).to(DEV), g[2], g[3],
                                            g[4])
    torch.cuda.synchronize()
    assert torch.all(out[1] == 0)
    for x in grads:
        assert torch.all(x[1] == 0)
    ref, _ = orc.combine_forward(*[x.double().numpy() for x in t[:2]], cm,
                                 *[x.double().numpy() for x in t[2:4]])
    check(out, ref, dtype, "strided out")


def test_differentiable_combine_autograd():
    print("[combine autograd]", flush=True)
    dtype = torch.float32
    t, cm = make(2, 2, 70, 16, dtype, seed=9)
    leaves = [x.to(DEV).requires_grad_(True) for x in t[:4]]
    out = _m().differentiable_multimer_combine(leaves[0], leaves[1],
                                               torch.from_numpy(cm).to(DEV), leaves[2], leaves[3])
    (out * t[4].to(DEV)).sum().backward()
    ref = orc.combine_backward(*[x.double().numpy() for x in t[:2]], cm,
                               *[x.double().numpy() for x in t[2:]])
    for leaf, r in zip(leaves, ref):
        check(leaf.grad, r, dtype, "autograd", rel_fro=1e-5)


def test_combine_150m_shape():
    """Two samples at L=1024, H=20, D=32 in bf16 against fp32 torch on the GPU."""
    print("[combine 150M shape]", flush=True)
    B, H, L, D = 2, 20, 1024, 32
    gen = torch.Generator(device=DEV).manual_seed(5)
    il = torch.randn(B, H, L, L, device=DEV, generator=gen).to(torch.bfloat16) * 2
    el = torch.randn(B, H, L, L, device=DEV, generator=gen).to(torch.bfloat16) * 2
    vs = torch.randn(B, H, L, D, device=DEV, generator=gen).to(torch.bfloat16)
    vm = torch.randn(B, H, L, D, device=DEV, generator=gen).to(torch.bfloat16)
    cid = torch.zeros(B, L, dtype=torch.int32, device=DEV)
    cid[0, 300:] = 1
    cid[1, 700:] = 1
    cm = cid[:, :, None] != cid[:, None, :]
    out = _m().fused_multimer_combine(il, el, cm, vs, vm)
    m = cm[:, None]
    p = torch.softmax(torch.where(m, el.float(), il.float()), -1)
    ref = torch.matmul(p.masked_fill(m, 0), vs.float()) + torch.matmul(p.masked_fill(~m, 0),
                                                                       vm.float())
    err = (out.float() - ref).abs()
    assert bool((err <= 2e-2 + 1e-2 * ref.abs()).all()), f"max err {err.max().item():.3g}"


# ---------------------------------------------------------------------------
# Dropout (the fused op's hash mask, include/mpattn.h)
# ---------------------------------------------------------------------------
def _code(L, D):
    """Row j: 2^(j // D) in column j % D (see tests/test_dropout_gpu.py)."""
    c = np.zeros((L, D))
    j = np.arange(L)
    c[j, j % D] = 2.0 ** (j // D)
    return c


@pytest.mark.parametrize("dtype,D,L", [(torch.bfloat16, 32, 128), (torch.float16, 32, 256),
                                       (torch.float32, 32, 256), (torch.bfloat16, 16, 50)])
def test_combine_dropout_exact_mask(dtype, D, L):
    """Zero logits (P = 1/n over valid keys) and one-hot coded V / dO: every
    output and dV element is an integer of keep bits times r / n, so a single
    mask element that differs from the oracle's moves it by r / n (allowed:
    r / (4n)). L = 50 takes the scalar-load path."""
    print(f"[combine dropout exact] {dtype} D={D} L={L}", flush=True)
    B, H, p, seed = 2, 3, 0.35, 0xDEADBEEF12345
    rng = np.random.default_rng(L + D)
    kp = tail_padding(rng, B, L, 0.15)
    z = np.where(kp[:, None, None, :], -np.inf, np.zeros((B, H, L, L)))
    cm = multi_chain_ids(rng, B, L, 2)
    cm = cm[:, :, None] != cm[:, None, :]
    code = np.broadcast_to(_code(L, D), (B, H, L, D)).copy()
    vrand = rng.standard_normal((B, H, L, D))
    r = lambda a: torch.from_numpy(a.astype(np.float32)).to(dtype).to(DEV)
    cmt = torch.from_numpy(cm).to(DEV)
    m = _m()
    out = m.fused_multimer_combine(r(z), r(z), cmt, r(code), r(code), dropout_p=p,
                                   dropout_seed=seed)
    grads = m.fused_multimer_combine_bwd(r(z), r(z), cmt, r(vrand), r(vrand), r(code),
                                         dropout_p=p, dropout_seed=seed)
    torch.cuda.synchronize()
    n = (~kp).sum(axis=1).astype(np.float64)
    step = (1.0 / (1.0 - np.float64(np.float32(p))) / n)[:, None, None, None]
    ref, _ = orc.combine_forward(z, z, cm, code, code, dropout_p=p, dropout_seed=seed)
    err = np.abs(out.double().cpu().numpy() - ref)
    assert (err <= 0.25 * step).all(), f"out: max err {err.max():.3g}"
    rg = orc.combine_backward(z, z, cm, vrand.astype(np.float32).astype(np.float64),
                              vrand.astype(np.float32).astype(np.float64), code, dropout_p=p,
                              dropout_seed=seed)
    for name, i in (("d_vs", 2), ("d_vm", 3)):
        err = np.abs(grads[i].double().cpu().numpy() - rg[i])
        assert (err <= 0.25 * step).all(), f"{name}: max err {err.max():.3g}"


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("L", [64, 100, 257])
def test_combine_dropout_random(dtype, L):
    print(f"[combine dropout random] {dtype} L={L}", flush=True)
    D, p, seed = 32, 0.2, 99 + L
    t, cm = make(2, 3, L, D, dtype, seed=300 + L)
    g = [x.to(DEV) for x in t]
    cmt = torch.from_numpy(cm).to(DEV)
    m = _m()
    out = m.fused_multimer_combine(g[0], g[1], cmt, g[2], g[3], dropout_p=p, dropout_seed=seed)
    grads = m.fused_multimer_combine_bwd(g[0], g[1], cmt, g[2], g[3], g[4], dropout_p=p,
                                         dropout_seed=seed)
    torch.cuda.synchronize()
    a = [x.double().numpy() for x in t]
    ref, _ = orc.combine_forward(a[0], a[1], cm, a[2], a[3], dropout_p=p, dropout_seed=seed)
    check(out, ref, dtype, "out")
    rg = orc.combine_backward(*a[:2], cm, *a[2:], dropout_p=p, dropout_seed=seed)
    fro = 1e-5 if dtype == torch.float32 else 2e-2
    for name, x, r in zip(("d_intra_logits", "d_inter_logits", "d_vs", "d_vm"), grads, rg):
        check(x, r, dtype, f"{name} dropout {dtype} L={L}", rel_fro=fro)


def test_combine_dropout_autograd_seed():
    """differentiable_multimer_combine keeps the forward's seed for the
    backward; a fixed seed reproduces bitwise; torch.manual_seed fixes the
    default seed."""
    print("[combine dropout autograd]", flush=True)
    D, L, p = 32, 96, 0.3
    t, cm = make(1, 2, L, D, torch.bfloat16, seed=5)
    cmt = torch.from_numpy(cm).to(DEV)
    m = _m()

    def run(**kw):
        leaves = [x.to(DEV).requires_grad_(True) for x in t[:4]]
        out = m.differentiable_multimer_combine(leaves[0], leaves[1], cmt, leaves[2], leaves[3],
                                                dropout_p=p, **kw)
        (out.float() * t[4].to(DEV).float()).sum().backward()
        return [out.detach()] + [x.grad for x in leaves]

    a = run(dropout_seed=17)
    b = run(dropout_seed=17)
    torch.manual_seed(3)
    c = run()
    torch.manual_seed(3)
    d = run()
    torch.cuda.synchronize()
    for x, y in zip(a, b):
        assert torch.equal(x, y)
    for x, y in zip(c, d):
        assert torch.equal(x, y)
    x = [v.double().numpy() for v in t]
    rg = orc.combine_backward(x[0], x[1], cm, x[2], x[3], x[4], dropout_p=p, dropout_seed=17)
    for name, g, r in zip(("d_intra_logits", "d_inter_logits", "d_vs", "d_vm"), a[1:], rg):
        check(g, r, torch.bfloat16, f"autograd {name}", rel_fro=2e-2)
