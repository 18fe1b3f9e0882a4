"""Backward parity of the HIP kernels (through the C ABI) against the oracle.

The oracle's gradients are the exact float64 gradients of the forward
(``oracle.mpattn_oracle.mpattn_backward``, pinned against finite differences
in ``tests/test_oracle.py``).

Tolerance (bf16 / fp16 inputs, gradients rounded to the input dtype):
  |gpu - ref| <= 2e-2 + 1e-2 * |ref|
"""
import numpy as np
import pytest
import torch

from conftest import multi_chain_ids, tail_padding, two_chain_ids
from oracle import mpattn_oracle as orc
from oracle import torch_ref

pytestmark = pytest.mark.gpu

ATOL16, RTOL16 = 2e-2, 1e-2
DEV = "cuda:0"
NAMES = ("dq_self", "dk_self", "dv_self", "dq_multi", "dk_multi", "dv_multi")


def _mpattn():
    import mint_plus_amd
    return mint_plus_amd


def make_inputs(B, H, L, D, dtype, seed, sigma=None, nchains=2, pad=True):
    rng = np.random.default_rng(seed)
    sigma = D ** -0.5 if sigma is None else sigma
    xs = [torch.from_numpy(rng.standard_normal((B, H, L, D)).astype(np.float32) * sigma).to(dtype)
          for _ in range(6)]
    go = torch.from_numpy(rng.standard_normal((B, H, L, D)).astype(np.float32)).to(dtype)
    cid = two_chain_ids(rng, B, L) if nchains == 2 else multi_chain_ids(rng, B, L, nchains)
    kp = tail_padding(rng, B, L) if pad else np.zeros((B, L), dtype=bool)
    return xs, go, cid, kp


def run_gpu(xs, go, cid, kp, rope, scale, dense=False):
    m = _mpattn()
    g = [x.to(DEV) for x in xs]
    kw = dict(key_padding_mask=torch.from_numpy(kp).to(DEV), rope=rope, scale=scale)
    if dense:
        c = torch.from_numpy(cid)
        cm = (c[:, :, None] != c[:, None, :]).to(DEV)
        grads = m.fused_multi_pathway_attention_bwd(*g, cm, go.to(DEV), **kw)
    else:
        grads = m.fused_multi_pathway_attention_bwd(*g, None, go.to(DEV),
                                                    chain_ids=torch.from_numpy(cid).to(DEV), **kw)
    torch.cuda.synchronize()
    return [t.float().cpu().numpy().astype(np.float64) for t in grads]


def oracle_grads(xs, go, cid, kp, rope, scale):
    a = [x.double().numpy() for x in xs]
    return orc.mpattn_backward(*a, go.double().numpy(), chain_ids=cid, key_pad=kp, rope=rope,
                               scale=scale)


def assert_grads(got, ref, what):
    for name, g, r in zip(NAMES, got, ref):
        err = np.abs(g - r)
        bound = ATOL16 + RTOL16 * np.abs(r)
        bad = err > bound
        assert not bad.any(), (f"{what} {name}: {bad.sum()} elements out of tolerance; "
                               f"max err {err.max():.4g} (max |ref| {np.abs(r).max():.4g})")


@pytest.mark.parametrize("D", [16, 24, 32, 64])
@pytest.mark.parametrize("L", [64, 100, 257])
def test_bwd_bf16_small(D, L):
    print(f"[bwd bf16] D={D} L={L}", flush=True)
    xs, go, cid, kp = make_inputs(2, 3, L, D, torch.bfloat16, seed=3000 + D + L)
    got = run_gpu(xs, go, cid, kp, rope=True, scale=D ** -0.5)
    ref = oracle_grads(xs, go, cid, kp, rope=True, scale=D ** -0.5)
    assert_grads(got, ref, f"bf16 D={D} L={L}")


@pytest.mark.parametrize("nchains", [1, 3, 5])
def test_bwd_chain_counts(nchains):
    """One chain: every pair is intra (pure self subtiles); more chains mix
    pure-multimer and general subtiles."""
    print(f"[bwd chains] n={nchains}", flush=True)
    xs, go, cid, kp = make_inputs(2, 2, 333, 32, torch.bfloat16, seed=70 + nchains,
                                  nchains=nchains)
    got = run_gpu(xs, go, cid, kp, rope=True, scale=32 ** -0.5)
    ref = oracle_grads(xs, go, cid, kp, rope=True, scale=32 ** -0.5)
    assert_grads(got, ref, f"nchains={nchains}")


@pytest.mark.parametrize("B,H,L,D,nchains,dense", [(2, 4, 1000, 32, 3, False), (2, 4, 512, 64, 2, False),
                                                   (2, 4, 1000, 32, 3, True)])
def test_bwd_heavy_first_dispatch(B, H, L, D, nchains, dense):
    """Grids that divide evenly over the 8 XCDs take the dispatch order with
    two-chain (and, for dK/dV, padded) blocks first (dense mask: the plain
    order inside each XCD's share): every block must still be computed
    exactly once."""
    print(f"[bwd dispatch] B={B} H={H} L={L} D={D} chains={nchains} dense={dense}", flush=True)
    xs, go, cid, kp = make_inputs(B, H, L, D, torch.bfloat16, seed=B * L + D, nchains=nchains)
    got = run_gpu(xs, go, cid, kp, rope=True, scale=D ** -0.5, dense=dense)
    ref = oracle_grads(xs, go, cid, kp, rope=True, scale=D ** -0.5)
    assert_grads(got, ref, f"dispatch B={B} H={H} L={L} D={D}")


@pytest.mark.parametrize("D", [32, 64])
def test_bwd_no_rope_dense_mask(D):
    """Reference contract: no fused RoPE, scale 1, dense (B, L, L) mask."""
    print(f"[bwd dense] D={D}", flush=True)
    xs, go, cid, kp = make_inputs(2, 2, 200, D, torch.bfloat16, seed=13 + D)
    got = run_gpu(xs, go, cid, kp, rope=False, scale=1.0, dense=True)
    ref = oracle_grads(xs, go, cid, kp, rope=False, scale=1.0)
    assert_grads(got, ref, f"dense D={D}")


@pytest.mark.parametrize("L,Lpad,D", [(256, 256, 32), (200, 208, 32), (1000, 1008, 32), (136, 144, 64)])
def test_bwd_dense_mask_tiles(L, Lpad, D):
    """Dense masks whose rows are 16-byte aligned: dK/dV copies the mask
    tiles into LDS. A padded row stride (Lpad > L) with L not a multiple of
    16 exercises the last key chunk copied from L - 16."""
    print(f"[bwd dense tiles] L={L} Lpad={Lpad} D={D}", flush=True)
    m = _mpattn()
    xs, go, cid, kp = make_inputs(2, 2, L, D, torch.bfloat16, seed=41 + L + D, nchains=3)
    g = [x.to(DEV) for x in xs]
    c = torch.from_numpy(cid)
    full = torch.zeros(2, L, Lpad, dtype=torch.bool)
    full[:, :, :L] = c[:, :, None] != c[:, None, :]
    cm = full.to(DEV)[:, :, :L]
    assert cm.stride(1) == Lpad
    grads = m.fused_multi_pathway_attention_bwd(*g, cm, go.to(DEV), key_padding_mask=torch.from_numpy(kp).to(DEV),
                                                rope=True, scale=D ** -0.5)
    torch.cuda.synchronize()
    got = [t.float().cpu().numpy().astype(np.float64) for t in grads]
    ref = oracle_grads(xs, go, cid, kp, rope=True, scale=D ** -0.5)
    assert_grads(got, ref, f"dense tiles L={L} Lpad={Lpad}")


def test_bwd_fp16():
    print("[bwd fp16]", flush=True)
    xs, go, cid, kp = make_inputs(2, 3, 190, 32, torch.float16, seed=17)
    got = run_gpu(xs, go, cid, kp, rope=True, scale=32 ** -0.5)
    ref = oracle_grads(xs, go, cid, kp, rope=True, scale=32 ** -0.5)
    assert_grads(got, ref, "fp16")


def test_bwd_all_keys_padded_sample():
    """A sample whose keys are all padded has zero output and zero gradients."""
    print("[bwd all padded]", flush=True)
    xs, go, cid, kp = make_inputs(2, 2, 96, 32, torch.bfloat16, seed=19, pad=False)
    kp[1, :] = True
    got = run_gpu(xs, go, cid, kp, rope=True, scale=32 ** -0.5)
    ref = oracle_grads(xs, go, cid, kp, rope=True, scale=32 ** -0.5)
    for g in got:
        assert np.all(g[1] == 0.0)
    assert_grads(got, ref, "all padded")


def test_bwd_deterministic():
    """No atomics: two runs give bitwise-identical gradients."""
    print("[bwd deterministic]", flush=True)
    xs, go, cid, kp = make_inputs(2, 4, 515, 32, torch.bfloat16, seed=23)
    a = run_gpu(xs, go, cid, kp, rope=True, scale=32 ** -0.5)
    b = run_gpu(xs, go, cid, kp, rope=True, scale=32 ** -0.5)
    for x, y in zip(a, b):
        assert np.array_equal(x, y)


def test_bwd_autograd_wrapper():
    """differentiable_multi_pathway_attention: autograd gradients equal the
    oracle's for a loss sum(out * G)."""
    print("[bwd autograd]", flush=True)
    m = _mpattn()
    D, L = 32, 150
    xs, go, cid, kp = make_inputs(2, 2, L, D, torch.bfloat16, seed=29)
    leaves = [x.to(DEV).requires_grad_(True) for x in xs]
    out = m.differentiable_multi_pathway_attention(
        *leaves, None, training=False, chain_ids=torch.from_numpy(cid).to(DEV),
        key_padding_mask=torch.from_numpy(kp).to(DEV), rope=True)
    (out.float() * go.to(DEV).float()).sum().backward()
    got = [t.grad.float().cpu().numpy().astype(np.float64) for t in leaves]
    ref = oracle_grads(xs, go, cid, kp, rope=True, scale=D ** -0.5)
    assert_grads(got, ref, "autograd")


def test_bwd_headline_shape():
    """150M shape (B=16, H=20, L=1024, D=32, bf16): the kernel runs on all 16
    samples; samples 0 and 9 are checked against fp32 autograd of the chunked
    torch reference (samples are independent)."""
    print("[bwd headline 16x20x1024x32]", flush=True)
    B, H, L, D = 16, 20, 1024, 32
    xs, go, cid, kp = make_inputs(B, H, L, D, torch.bfloat16, seed=2025)
    m = _mpattn()
    g = [x.to(DEV) for x in xs]
    cid_t = torch.from_numpy(cid).to(DEV)
    kp_t = torch.from_numpy(kp).to(DEV)
    go_d = go.to(DEV)
    grads = m.fused_multi_pathway_attention_bwd(*g, None, go_d, chain_ids=cid_t,
                                                key_padding_mask=kp_t, rope=True,
                                                scale=D ** -0.5)
    for b in (0, 9):
        sl = slice(b, b + 1)
        leaves = [x[sl].float().clone().requires_grad_(True) for x in g]
        ref_out, _ = torch_ref.forward(*leaves, chain_ids=cid_t[sl], key_pad=kp_t[sl], rope=True,
                                       scale=D ** -0.5, dtype=torch.float32, chunk=1)
        (ref_out * go_d[sl].float()).sum().backward()
        for name, gg, leaf in zip(NAMES, grads, leaves):
            r = leaf.grad
            err = (gg[sl].float() - r).abs()
            bound = ATOL16 + RTOL16 * r.abs()
            assert bool((err <= bound).all()), f"sample {b} {name}: max err {err.max().item():.4g}"


@pytest.mark.parametrize("D", [16, 32, 64])
def test_bwd_sqrt_softmax(D):
    """Gradients of the sqrt-softmax variant (dS = W (dW - W delta) / 2)."""
    print(f"[bwd sqrt] D={D}", flush=True)
    m = _mpattn()
    xs, go, cid, kp = make_inputs(2, 2, 140, D, torch.bfloat16, seed=60 + D)
    g = [x.to(DEV) for x in xs]
    grads = m.fused_multi_pathway_attention_bwd(*g, None, go.to(DEV),
                                                chain_ids=torch.from_numpy(cid).to(DEV),
                                                key_padding_mask=torch.from_numpy(kp).to(DEV),
                                                rope=True, scale=D ** -0.5, sqrt_softmax=True)
    torch.cuda.synchronize()
    got = [t.float().cpu().numpy().astype(np.float64) for t in grads]
    a = [x.double().numpy() for x in xs]
    ref = orc.mpattn_backward(*a, go.double().numpy(), chain_ids=cid, key_pad=kp, rope=True,
                              scale=D ** -0.5, sqrt_softmax=True)
    assert_grads(got, ref, f"sqrt D={D}")
