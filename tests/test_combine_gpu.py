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
@pytest.mark.parametrize("L", [64, 100, 257])
def test_combine_fwd(dtype, D, L):
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
@pytest.mark.parametrize("L", [64, 129])
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
