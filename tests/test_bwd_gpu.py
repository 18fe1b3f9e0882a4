"""Backward parity of the HIP kernels (through the C ABI) against the oracle.

The oracle's gradients are the exact float64 gradients of the forward
(``oracle.mpattn_oracle.mpattn_backward``, pinned against finite differences
in ``tests/test_oracle.py``).

Tolerance (bf16 / fp16 inputs, gradients rounded to the input dtype), per
gradient tensor:
  |gpu - ref| <= 2e-2 + 1e-2 * |ref| elementwise, and
  ||gpu - ref||_F <= 1e-2 ||ref||_F

Inputs come from ``tests/parity.py``: V entries ~N(0, 16) and dO entries of
std sqrt(L) times a per-case power of two, so every gradient's RMS is at
most ~1 and a correct kernel's rounding (modelled by
``parity.emulate_bwd16``) stays within half the bound.
``tests/test_parity_power.py`` checks that calibration on the CPU, and that
each comparison rejects zeroed dQ or dK, dQ and dK swapped, dQ and dK
halved, swapped pathways, one zeroed 256-query block and (RoPE cases)
dropped RoPE.
"""
import numpy as np
import pytest
import torch

import parity as P
from oracle import mpattn_oracle as orc
from oracle import torch_ref

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
NAMES = P.GRAD_NAMES

# Case lists (shared with tests/test_parity_power.py).
SMALL = [(D, L) for D in (16, 24, 32, 64) for L in (64, 100, 257)]       # B=2, H=3
CHAIN_COUNTS = [1, 3, 5]                                                  # (2, 2, 333, 32)
DISPATCH = [(2, 4, 1000, 32, 3, False), (2, 4, 512, 64, 2, False), (2, 4, 1000, 32, 3, True)]
ROPE_SHARP = [32, 64]            # fused RoPE, logit std 2, (2, 2, 300, D)
HEADLINE = (8, 20, 1024, 32)     # BASELINE configs[3] (training shape)
HEADLINE_SAMPLES = (0, 7)
CFG3B = [(1, 40, 2048, 64), (1, 40, 2304, 64)]   # configs[4]; 2304 moves the summary windows


def small_case(D, L):
    return P.bwd_inputs(2, 3, L, D, torch.bfloat16, seed=3000 + D + L)


def chain_case(n):
    return P.bwd_inputs(2, 2, 333, 32, torch.bfloat16, seed=70 + n, nchains=n, go_log2=-1 if n == 1 else 0)


def dispatch_case(B, H, L, D, nchains):
    return P.bwd_inputs(B, H, L, D, torch.bfloat16, seed=B * L + D, nchains=nchains)


def rope_sharp_case(D):
    return P.bwd_inputs(2, 2, 300, D, torch.bfloat16, seed=5500 + D, sigma=2.0 ** 0.5, nchains=3, go_log2=-6)


def autograd_case():
    return P.bwd_inputs(2, 2, 150, 32, torch.bfloat16, seed=29)


def headline_case():
    B, H, L, D = HEADLINE
    return P.bwd_inputs(B, H, L, D, torch.bfloat16, seed=2025)


def case3b(B, H, L, D):
    return P.bwd_inputs(B, H, L, D, torch.bfloat16, seed=3400 + L, nchains="3b", go_log2=-1 if L > 2048 else 0)


def dense_norope_case(D):
    return P.bwd_inputs(2, 2, 200, D, torch.bfloat16, seed=13 + D, go_log2=-2)


DENSE_NP = [(300, 32), (200, 64)]


def dense_np_case(L, D):
    """(B=3, H=2) inputs and a (3, L, L) bool mask: row 0 a chain partition,
    row 1 random (asymmetric), row 2 a partition with one entry flipped."""
    xs, go, cid, kp = P.bwd_inputs(3, 2, L, D, torch.bfloat16, seed=93 + L + D, nchains=3, go_log2=-2)
    c = torch.from_numpy(cid)
    cm = c[:, :, None] != c[:, None, :]
    g = torch.Generator().manual_seed(L + D + 1)
    cm[1] = torch.rand(L, L, generator=g) < 0.4
    cm[2, 5, L - 3] = ~cm[2, 5, L - 3]
    return xs, go, cm, kp


def sqrt_case(D):
    return P.bwd_inputs(2, 2, 140, D, torch.bfloat16, seed=60 + D, go_log2=-4)


# (dtype, logit shift, logit spread, dO std) of the softmax-range cases
RANGE = [(torch.bfloat16, 0.0, 20.0, 0.25 / 8), (torch.float16, 14.0, 2.0, 1.0),
         (torch.float16, -14.0, 0.6, 4.0)]


def range_case(dtype, shift, spread, go_std):
    D, L = 32, 300
    xs, cid, kp = P.shifted_logit_inputs(2, 3, L, D, dtype, seed=int(abs(shift) * 10 + spread * 100) + 1,
                                         shift=shift, spread=spread, v_std=1.0)
    rng = np.random.default_rng(int(spread * 7))
    go = torch.from_numpy(rng.standard_normal((2, 3, L, D)).astype(np.float32) * go_std).to(dtype)
    return xs, go, cid, kp


def _mpattn():
    import mint_plus_amd
    return mint_plus_amd


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


@pytest.mark.parametrize("D,L", SMALL)
def test_bwd_bf16_small(D, L):
    print(f"[bwd bf16] D={D} L={L}", flush=True)
    xs, go, cid, kp = small_case(D, L)
    got = run_gpu(xs, go, cid, kp, rope=True, scale=D ** -0.5)
    ref = oracle_grads(xs, go, cid, kp, rope=True, scale=D ** -0.5)
    P.assert_grads16(got, ref, f"bf16 D={D} L={L}")


@pytest.mark.parametrize("nchains", CHAIN_COUNTS)
def test_bwd_chain_counts(nchains):
    """One chain: every pair is intra (pure self subtiles); more chains mix
    pure-multimer and general subtiles."""
    print(f"[bwd chains] n={nchains}", flush=True)
    xs, go, cid, kp = chain_case(nchains)
    got = run_gpu(xs, go, cid, kp, rope=True, scale=32 ** -0.5)
    ref = oracle_grads(xs, go, cid, kp, rope=True, scale=32 ** -0.5)
    if nchains == 1:  # no cross-chain pair: the multimer gradients are exactly 0
        ref_m = [r for n, r in zip(NAMES, ref) if n.endswith("multi")]
        assert all(np.all(r == 0) for r in ref_m)
        assert all(np.all(g == 0) for n, g in zip(NAMES, got) if n.endswith("multi"))
        got = [g for n, g in zip(NAMES, got) if n.endswith("self")]
        ref = [r for n, r in zip(NAMES, ref) if n.endswith("self")]
        for n, g, r in zip(("dq_self", "dk_self", "dv_self"), got, ref):
            P.assert16(g, r, f"nchains=1 {n}")
        return
    P.assert_grads16(got, ref, f"nchains={nchains}")


@pytest.mark.parametrize("B,H,L,D,nchains,dense", DISPATCH)
def test_bwd_heavy_first_dispatch(B, H, L, D, nchains, dense):
    """Grids that divide evenly over the 8 XCDs take the dispatch order with
    two-chain (and, for dK/dV, padded) blocks first (dense mask: the plain
    order inside each XCD's share): every block must still be computed
    exactly once."""
    print(f"[bwd dispatch] B={B} H={H} L={L} D={D} chains={nchains} dense={dense}", flush=True)
    xs, go, cid, kp = dispatch_case(B, H, L, D, nchains)
    got = run_gpu(xs, go, cid, kp, rope=True, scale=D ** -0.5, dense=dense)
    ref = oracle_grads(xs, go, cid, kp, rope=True, scale=D ** -0.5)
    P.assert_grads16(got, ref, f"dispatch B={B} H={H} L={L} D={D}")


@pytest.mark.parametrize("D", ROPE_SHARP)
def test_bwd_fused_rope_sharp(D):
    """Fused RoPE with logit std ~2: gradients of Q/K_self depend on the
    rotation in the prologue (R) and the epilogue (R^T). The reference is
    float64 autograd with the rotated Q_self/K_self rounded to bf16 in the
    forward (the backward kernels' MFMA operands) and the exact rotation in
    the gradient (``parity.ref_grads``): at this logit size the operand
    rounding alone moves dQ_self by up to ~1."""
    print(f"[bwd rope sharp] D={D}", flush=True)
    xs, go, cid, kp = rope_sharp_case(D)
    got = run_gpu(xs, go, cid, kp, rope=True, scale=D ** -0.5)
    ref = P.ref_grads(xs, go, cid, kp, True, D ** -0.5, round_dtype=torch.bfloat16)
    P.assert_grads16(got, ref, f"rope sharp D={D}")


@pytest.mark.parametrize("D", [32, 64])
def test_bwd_no_rope_dense_mask(D):
    """Reference contract: no fused RoPE, scale 1, dense (B, L, L) mask."""
    print(f"[bwd dense] D={D}", flush=True)
    xs, go, cid, kp = dense_norope_case(D)
    got = run_gpu(xs, go, cid, kp, rope=False, scale=1.0, dense=True)
    ref = oracle_grads(xs, go, cid, kp, rope=False, scale=1.0)
    P.assert_grads16(got, ref, f"dense D={D}")


@pytest.mark.parametrize("L,Lpad,D", [(256, 256, 32), (200, 208, 32), (1000, 1008, 32), (136, 144, 64)])
def test_bwd_dense_mask_tiles(L, Lpad, D):
    """Dense masks whose rows are 16-byte aligned: dK/dV copies the mask
    tiles into LDS. A padded row stride (Lpad > L) with L not a multiple of
    16 exercises the last key chunk copied from L - 16."""
    print(f"[bwd dense tiles] L={L} Lpad={Lpad} D={D}", flush=True)
    m = _mpattn()
    xs, go, cid, kp = P.bwd_inputs(2, 2, L, D, torch.bfloat16, seed=41 + L + D, nchains=3)
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
    P.assert_grads16(got, ref, f"dense tiles L={L} Lpad={Lpad}")


@pytest.mark.parametrize("L,D", DENSE_NP)
def test_bwd_dense_mask_not_partition(L, D):
    """Chain-partition mask rows run the chain-id backward kernels on the
    mask's row labels, the others the dense-mask kernels, in one call."""
    print(f"[bwd dense non-partition] L={L} D={D}", flush=True)
    m = _mpattn()
    xs, go, cm, kp = dense_np_case(L, D)
    grads = m.fused_multi_pathway_attention_bwd(*[x.to(DEV) for x in xs], cm.to(DEV), go.to(DEV),
                                                key_padding_mask=torch.from_numpy(kp).to(DEV), rope=True,
                                                scale=D ** -0.5)
    torch.cuda.synchronize()
    got = [t.float().cpu().numpy().astype(np.float64) for t in grads]
    a = [x.double().numpy() for x in xs]
    ref = orc.mpattn_backward(*a, go.double().numpy(), chain_mask=cm.numpy(), key_pad=kp, rope=True,
                              scale=D ** -0.5)
    P.assert_grads16(got, ref, f"dense non-partition L={L} D={D}")


def test_bwd_fp16():
    print("[bwd fp16]", flush=True)
    xs, go, cid, kp = P.bwd_inputs(2, 3, 190, 32, torch.float16, seed=17)
    got = run_gpu(xs, go, cid, kp, rope=True, scale=32 ** -0.5)
    ref = oracle_grads(xs, go, cid, kp, rope=True, scale=32 ** -0.5)
    P.assert_grads16(got, ref, "fp16")


@pytest.mark.parametrize("dtype,shift,spread,go_std", RANGE)
def test_bwd_softmax_range(dtype, shift, spread, go_std):
    """Gradients where the forward leaves its unshifted range (logits up to
    ~100 in bf16, past the fp16 maximum, or all in the fp16 subnormal range);
    the backward's probabilities come from the forward's LSE. V ~ N(0, 1);
    dO is calibrated per case: with nearly one-hot rows, the kernels'
    Delta = rowsum(O * dO) taken from the bf16/fp16-rounded O is most of the
    dQ/dK error, so |dO| |O| |K| must stay small against the 2e-2 bound."""
    print(f"[bwd range] dtype={dtype} shift={shift} spread={spread}", flush=True)
    m = _mpattn()
    xs, go, cid, kp = range_case(dtype, shift, spread, go_std)
    g = [x.to(DEV) for x in xs]
    out, lse = m._lib.mpattn_fwd(*g, chain_ids=torch.from_numpy(cid).to(DEV),
                                 key_padding_mask=torch.from_numpy(kp).to(DEV), need_lse=True)
    grads = m._lib.mpattn_bwd(*g, out, lse, go.to(DEV), chain_ids=torch.from_numpy(cid).to(DEV),
                              key_padding_mask=torch.from_numpy(kp).to(DEV))
    torch.cuda.synchronize()
    got = [t.float().cpu().numpy().astype(np.float64) for t in grads]
    ref = oracle_grads(xs, go, cid, kp, rope=False, scale=1.0)
    P.assert_grads16(got, ref, f"range {dtype} shift={shift}")


def test_bwd_all_keys_padded_sample():
    """A sample whose keys are all padded has zero output and zero gradients."""
    print("[bwd all padded]", flush=True)
    xs, go, cid, kp = P.bwd_inputs(2, 2, 96, 32, torch.bfloat16, seed=19, pad=False)
    kp[1, :] = True
    got = run_gpu(xs, go, cid, kp, rope=True, scale=32 ** -0.5)
    ref = oracle_grads(xs, go, cid, kp, rope=True, scale=32 ** -0.5)
    for g in got:
        assert np.all(g[1] == 0.0)
    P.assert_grads16(got, ref, "all padded")


def test_bwd_deterministic():
    """No atomics: two runs give bitwise-identical gradients."""
    print("[bwd deterministic]", flush=True)
    xs, go, cid, kp = P.bwd_inputs(2, 4, 515, 32, torch.bfloat16, seed=23)
    a = run_gpu(xs, go, cid, kp, rope=True, scale=32 ** -0.5)
    b = run_gpu(xs, go, cid, kp, rope=True, scale=32 ** -0.5)
    for x, y in zip(a, b):
        assert np.array_equal(x, y)


def test_bwd_autograd_wrapper():
    """differentiable_multi_pathway_attention: autograd gradients equal the
    oracle's for a loss sum(out * G), in the argument order of the op."""
    print("[bwd autograd]", flush=True)
    m = _mpattn()
    D, L = 32, 150
    xs, go, cid, kp = autograd_case()
    leaves = [x.to(DEV).requires_grad_(True) for x in xs]
    out = m.differentiable_multi_pathway_attention(
        *leaves, None, training=False, chain_ids=torch.from_numpy(cid).to(DEV),
        key_padding_mask=torch.from_numpy(kp).to(DEV), rope=True)
    (out.float() * go.to(DEV).float()).sum().backward()
    got = [t.grad.float().cpu().numpy().astype(np.float64) for t in leaves]
    ref = oracle_grads(xs, go, cid, kp, rope=True, scale=D ** -0.5)
    P.assert_grads16(got, ref, "autograd")


def _torch_grads(g, go_d, cid_t, kp_t, sl, D):
    leaves = [x[sl].float().clone().requires_grad_(True) for x in g]
    ref_out, _ = torch_ref.forward(*leaves, chain_ids=cid_t[sl], key_pad=kp_t[sl], rope=True,
                                   scale=D ** -0.5, dtype=torch.float32, chunk=1)
    (ref_out * go_d[sl].float()).sum().backward()
    return [leaf.grad for leaf in leaves]


def test_bwd_headline_shape():
    """configs[3] training shape (B=8, H=20, L=1024, D=32, bf16): the kernels
    run on all 8 samples; samples 0 and 7 are checked against fp32 autograd
    of the chunked torch reference (samples are independent)."""
    print("[bwd headline 8x20x1024x32]", flush=True)
    B, H, L, D = HEADLINE
    xs, go, cid, kp = headline_case()
    m = _mpattn()
    g = [x.to(DEV) for x in xs]
    cid_t = torch.from_numpy(cid).to(DEV)
    kp_t = torch.from_numpy(kp).to(DEV)
    go_d = go.to(DEV)
    grads = m.fused_multi_pathway_attention_bwd(*g, None, go_d, chain_ids=cid_t,
                                                key_padding_mask=kp_t, rope=True,
                                                scale=D ** -0.5)
    for b in HEADLINE_SAMPLES:
        sl = slice(b, b + 1)
        for name, gg, r in zip(NAMES, grads, _torch_grads(g, go_d, cid_t, kp_t, sl, D)):
            P.assert16_torch(gg[sl], r, f"sample {b} {name}")


@pytest.mark.parametrize("B,H,L,D", CFG3B)
def test_bwd_3b_shape(B, H, L, D):
    """configs[4] attention shape (H=40, D=64, three chains, L=2048 and
    2304) against fp32 autograd of the chunked torch reference."""
    print(f"[bwd 3B] B={B} H={H} L={L} D={D}", flush=True)
    xs, go, cid, kp = case3b(B, H, L, D)
    m = _mpattn()
    g = [x.to(DEV) for x in xs]
    cid_t = torch.from_numpy(cid).to(DEV)
    kp_t = torch.from_numpy(kp).to(DEV)
    go_d = go.to(DEV)
    grads = m.fused_multi_pathway_attention_bwd(*g, None, go_d, chain_ids=cid_t,
                                                key_padding_mask=kp_t, rope=True,
                                                scale=D ** -0.5)
    for b in range(B):
        sl = slice(b, b + 1)
        for name, gg, r in zip(NAMES, grads, _torch_grads(g, go_d, cid_t, kp_t, sl, D)):
            P.assert16_torch(gg[sl], r, f"3B L={L} sample {b} {name}")


@pytest.mark.parametrize("D", [16, 32, 64])
def test_bwd_sqrt_softmax(D):
    """Gradients of the sqrt-softmax variant (dS = W (dW - W delta) / 2)."""
    print(f"[bwd sqrt] D={D}", flush=True)
    m = _mpattn()
    xs, go, cid, kp = sqrt_case(D)
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
    P.assert_grads16(got, ref, f"sqrt D={D}")
