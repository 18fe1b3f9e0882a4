"""Attention dropout of the fused op (16-bit and fp32 kernels, with and
without sqrt-softmax) against the oracle.

The keep mask is a function of (seed, b*H + h, query, key) (definition in
include/mpattn.h, restated by ``oracle.mpattn_oracle.dropout_keep``), so the
GPU result is compared with the oracle's for the same seed.

Two kinds of check:

* Exact-mask tests. With Q = 0 every logit is 0, so P = 1/n over the n valid
  keys of a row and the kernel's probabilities are exactly 1 before the
  normalisation. V (forward), dO (dV) or K (dQ) is then a one-hot code that
  gives key j (or query i) the weight 2^(j // D) in column j % D, so an
  output element holds the keep bits of up to G = L / D keys as an integer
  times r / n (r = 1 / (1 - p)). One element of the mask that differs from
  the oracle's moves an output by at least r / n; the tests allow a quarter
  of that. G is kept to 4 for bf16 outputs (8 mantissa bits) and 8 for fp16
  (11 bits), so output rounding stays far below r / (4n).
* Random inputs, with the op's tolerance |gpu - ref| <= 2e-2 + 1e-2 |ref|.
"""
import numpy as np
import pytest
import torch

from conftest import multi_chain_ids, tail_padding, two_chain_ids
from oracle import mpattn_oracle as orc

pytestmark = pytest.mark.gpu

ATOL16, RTOL16 = 2e-2, 1e-2
DEV = "cuda:0"
NAMES = ("dq_self", "dk_self", "dv_self", "dq_multi", "dk_multi", "dv_multi")


def _m():
    import mint_plus_amd
    return mint_plus_amd


def _code(L, D):
    """(L, D) one-hot code: row j has 2^(j // D) in column j % D."""
    c = np.zeros((L, D))
    j = np.arange(L)
    c[j, j % D] = 2.0 ** (j // D)
    return c


def _structured(B, H, L, D, seed):
    rng = np.random.default_rng(seed)
    cid = two_chain_ids(rng, B, L)
    kp = tail_padding(rng, B, L, 0.15)
    return rng, cid, kp


def _gpu_fwd(xs, cid, kp, p, seed, dtype, rope=False, scale=1.0):
    m = _m()
    g = [torch.as_tensor(x).to(dtype).to(DEV) for x in xs]
    out = m.fused_multi_pathway_attention(
        *g, None, dropout_p=p, training=True, chain_ids=torch.from_numpy(cid).to(DEV),
        key_padding_mask=torch.from_numpy(kp).to(DEV), rope=rope, scale=scale, dropout_seed=seed)
    torch.cuda.synchronize()
    return out.float().cpu().numpy().astype(np.float64)


def _gpu_bwd(xs, go, cid, kp, p, seed, dtype, rope=False, scale=1.0, dense=False):
    m = _m()
    g = [torch.as_tensor(x).to(dtype).to(DEV) for x in xs]
    kw = dict(key_padding_mask=torch.from_numpy(kp).to(DEV), rope=rope, scale=scale,
              dropout_p=p, dropout_seed=seed)
    gout = torch.as_tensor(go).to(dtype).to(DEV)
    if dense:
        c = torch.from_numpy(cid)
        grads = m.fused_multi_pathway_attention_bwd(
            *g, (c[:, :, None] != c[:, None, :]).to(DEV), gout, **kw)
    else:
        grads = m.fused_multi_pathway_attention_bwd(
            *g, None, gout, chain_ids=torch.from_numpy(cid).to(DEV), **kw)
    torch.cuda.synchronize()
    return [t.float().cpu().numpy().astype(np.float64) for t in grads]


def _rounded(xs, dtype):
    """The inputs as the kernel sees them (rounded to the 16-bit type)."""
    return [torch.as_tensor(x).to(dtype).double().numpy() for x in xs]


def _step(kp, p):
    """r / n per sample, shaped to broadcast over (B, H, L, D)."""
    n = (~kp).sum(axis=1).astype(np.float64)
    r = 1.0 / (1.0 - np.float64(np.float32(p)))
    return (r / n)[:, None, None, None]


EXACT_CASES = [  # (dtype, D, L): L / D groups, at most 4 (bf16), 8 (fp16) or 16 (fp32)
    (torch.bfloat16, 16, 64),
    (torch.bfloat16, 32, 128),
    (torch.bfloat16, 64, 256),
    (torch.float16, 32, 256),
    (torch.float16, 24, 190),
    (torch.float32, 16, 200),
    (torch.float32, 32, 256),
]


@pytest.mark.parametrize("dtype,D,L", EXACT_CASES)
@pytest.mark.parametrize("p", [0.1, 0.5])
def test_dropout_exact_mask_forward(dtype, D, L, p):
    print(f"[dropout exact fwd] {dtype} D={D} L={L} p={p}", flush=True)
    B, H = 2, 3
    rng, cid, kp = _structured(B, H, L, D, seed=D + L)
    q = np.zeros((B, H, L, D))
    k = rng.standard_normal((B, H, L, D))
    v = np.broadcast_to(_code(L, D), (B, H, L, D)).copy()
    xs = [q, k, v, q, k.copy(), v]
    seed = 0x1234_5678_0000_0000 + D * 131 + L
    got = _gpu_fwd(xs, cid, kp, p, seed, dtype)
    ref, _ = orc.mpattn_forward(*_rounded(xs, dtype), chain_ids=cid, key_pad=kp, dropout_p=p,
                                dropout_seed=seed)
    tol = 0.25 * _step(kp, p)
    err = np.abs(got - ref)
    assert (err <= tol).all(), f"max err {err.max():.4g} vs step/4 {tol.min():.4g}"
    # and the mask is not trivial: dropout changed the result
    ref0, _ = orc.mpattn_forward(*_rounded(xs, dtype), chain_ids=cid, key_pad=kp)
    assert np.abs(ref - ref0).max() > 4 * tol.max()


@pytest.mark.parametrize("dtype,D,L", EXACT_CASES)
def test_dropout_exact_mask_dv(dtype, D, L):
    """dV_j = r sum_i Z_ij P_ij dO_i with dO the query code: the key-stationary
    kernel's mask, element by element."""
    print(f"[dropout exact dV] {dtype} D={D} L={L}", flush=True)
    B, H, p = 2, 3, 0.3
    rng, cid, kp = _structured(B, H, L, D, seed=7 * D + L)
    q = np.zeros((B, H, L, D))
    k = rng.standard_normal((B, H, L, D))
    v = rng.standard_normal((B, H, L, D))
    go = np.broadcast_to(_code(L, D), (B, H, L, D)).copy()
    xs = [q, k, v, q, k.copy(), v.copy()]
    seed = 987654321 + D
    got = _gpu_bwd(xs, go, cid, kp, p, seed, dtype)
    ref = orc.mpattn_backward(*_rounded(xs, dtype), _rounded([go], dtype)[0], chain_ids=cid,
                              key_pad=kp, dropout_p=p, dropout_seed=seed)
    tol = 0.25 * _step(kp, p)
    for name in ("dv_self", "dv_multi"):
        i = NAMES.index(name)
        err = np.abs(got[i] - ref[i])
        assert (err <= tol).all(), f"{name}: max err {err.max():.4g} vs {tol.min():.4g}"


@pytest.mark.parametrize("dtype,D,L", [c for c in EXACT_CASES if c[0] != torch.float16])
def test_dropout_exact_mask_dq(dtype, D, L):
    """dQ_i = sum_j P_ij (r Z_ij - Delta_i) K_j with dO . V = 1 and K the key
    code: the query-stationary kernel's mask, element by element."""
    print(f"[dropout exact dQ] {dtype} D={D} L={L}", flush=True)
    B, H, p = 2, 3, 0.3
    rng, cid, kp = _structured(B, H, L, D, seed=11 * D + L)
    q = np.zeros((B, H, L, D))
    k = np.broadcast_to(_code(L, D), (B, H, L, D)).copy()
    e0 = np.zeros((B, H, L, D))
    e0[..., 0] = 1.0
    xs = [q, k, e0, q, k.copy(), e0.copy()]
    seed = 55 + D
    got = _gpu_bwd(xs, e0, cid, kp, p, seed, dtype)
    ref = orc.mpattn_backward(*_rounded(xs, dtype), e0, chain_ids=cid, key_pad=kp, dropout_p=p,
                              dropout_seed=seed)
    tol = 0.25 * _step(kp, p)
    for name in ("dq_self", "dq_multi"):
        i = NAMES.index(name)
        err = np.abs(got[i] - ref[i])
        assert (err <= tol).all(), f"{name}: max err {err.max():.4g} vs {tol.min():.4g}"


def _random(B, H, L, D, seed, nchains=2):
    rng = np.random.default_rng(seed)
    xs = [rng.standard_normal((B, H, L, D)) * D ** -0.5 for _ in range(6)]
    go = rng.standard_normal((B, H, L, D))
    cid = two_chain_ids(rng, B, L) if nchains == 2 else multi_chain_ids(rng, B, L, nchains)
    kp = tail_padding(rng, B, L)
    return xs, go, cid, kp


def _assert16(got, ref, what):
    err = np.abs(got - ref)
    bad = err > ATOL16 + RTOL16 * np.abs(ref)
    assert not bad.any(), f"{what}: {bad.sum()} out of tolerance, max err {err.max():.4g}"


@pytest.mark.parametrize("D,L,nchains,dense", [(32, 257, 2, False), (64, 300, 3, False),
                                               (16, 130, 1, False), (32, 200, 2, True)])
def test_dropout_random_inputs(D, L, nchains, dense):
    print(f"[dropout random] D={D} L={L} chains={nchains} dense={dense}", flush=True)
    B, H, p, seed = 2, 3, 0.2, 2024 + D
    xs, go, cid, kp = _random(B, H, L, D, seed=D * L, nchains=nchains)
    dt = torch.bfloat16
    xr = _rounded(xs, dt)
    ref_o, _ = orc.mpattn_forward(*xr, chain_ids=cid, key_pad=kp, rope=True, scale=D ** -0.5,
                                  dropout_p=p, dropout_seed=seed)
    if not dense:
        got_o = _gpu_fwd(xs, cid, kp, p, seed, dt, rope=True, scale=D ** -0.5)
        _assert16(got_o, ref_o, "out")
    got = _gpu_bwd(xs, go, cid, kp, p, seed, dt, rope=True, scale=D ** -0.5, dense=dense)
    ref = orc.mpattn_backward(*xr, _rounded([go], dt)[0], chain_ids=cid, key_pad=kp, rope=True,
                              scale=D ** -0.5, dropout_p=p, dropout_seed=seed)
    for name, g, r in zip(NAMES, got, ref):
        _assert16(g, r, name)


def test_dropout_seed_semantics():
    """Same seed: bitwise-identical output; another seed: a different one;
    training=False or p = 0: the no-dropout result; no seed: drawn from
    torch's CPU generator (so torch.manual_seed reproduces it)."""
    print("[dropout seeds]", flush=True)
    m = _m()
    xs, _, cid, kp = _random(2, 4, 300, 32, seed=5)
    g = [torch.as_tensor(x).to(torch.bfloat16).to(DEV) for x in xs]
    kw = dict(chain_ids=torch.from_numpy(cid).to(DEV), key_padding_mask=torch.from_numpy(kp).to(DEV),
              rope=True)
    f = lambda **k: m.fused_multi_pathway_attention(*g, None, **kw, **k)
    a = f(dropout_p=0.3, dropout_seed=1)
    b = f(dropout_p=0.3, dropout_seed=1)
    c = f(dropout_p=0.3, dropout_seed=2)
    d = f(dropout_p=0.3, dropout_seed=1 + (1 << 32))
    base = f()
    ev = f(dropout_p=0.3, training=False)
    torch.manual_seed(7)
    s1 = f(dropout_p=0.3)
    torch.manual_seed(7)
    s2 = f(dropout_p=0.3)
    torch.cuda.synchronize()
    assert torch.equal(a, b)
    assert not torch.equal(a, c) and not torch.equal(a, d)
    assert torch.equal(ev, base)
    assert torch.equal(s1, s2)
    assert not torch.equal(a, base)


def test_dropout_autograd_and_projected_path():
    """differentiable_multi_pathway_attention and multi_pathway_attention_from_qkv
    with dropout: the forward equals the oracle's and the backward uses the
    forward's mask (gradients equal the oracle's for the same seed)."""
    print("[dropout autograd]", flush=True)
    m = _m()
    B, H, L, D, p, seed = 2, 4, 180, 32, 0.25, 31337
    xs, go, cid, kp = _random(B, H, L, D, seed=77)
    dt = torch.bfloat16
    xr = _rounded(xs, dt)
    gr = _rounded([go], dt)[0]
    sel = dict(chain_ids=cid, key_pad=kp, rope=True, scale=D ** -0.5, dropout_p=p,
               dropout_seed=seed)
    ref_o, _ = orc.mpattn_forward(*xr, **sel)
    ref_g = orc.mpattn_backward(*xr, gr, **sel)
    cid_t, kp_t = torch.from_numpy(cid).to(DEV), torch.from_numpy(kp).to(DEV)

    leaves = [torch.as_tensor(x).to(dt).to(DEV).requires_grad_(True) for x in xs]
    out = m.differentiable_multi_pathway_attention(
        *leaves, None, dropout_p=p, training=True, chain_ids=cid_t, key_padding_mask=kp_t,
        rope=True, dropout_seed=seed)
    (out.float() * torch.as_tensor(gr).float().to(DEV)).sum().backward()
    _assert16(out.detach().float().cpu().double().numpy(), ref_o, "autograd out")
    for name, t, r in zip(NAMES, leaves, ref_g):
        _assert16(t.grad.float().cpu().double().numpy(), r, f"autograd {name}")

    # (T, B, 3E) projection outputs holding the same Q/K/V
    E = H * D

    def pack(qkv):
        return torch.cat([torch.as_tensor(x).to(dt).permute(2, 0, 1, 3).reshape(L, B, E)
                          for x in qkv], dim=-1).to(DEV).requires_grad_(True)

    qkv_s, qkv_m = pack(xs[:3]), pack(xs[3:])
    o = m.multi_pathway_attention_from_qkv(qkv_s, qkv_m, H, dropout_p=p, training=True,
                                           chain_ids=cid_t, key_padding_mask=kp_t, rope=True,
                                           dropout_seed=seed)
    go_tbe = torch.as_tensor(gr).float().permute(2, 0, 1, 3).reshape(L, B, E).to(DEV)
    (o.float() * go_tbe).sum().backward()
    o4 = o.detach().float().view(L, B, H, D).permute(1, 2, 0, 3).cpu().double().numpy()
    _assert16(o4, ref_o, "from_qkv out")
    assert torch.equal(o.detach().view(L, B, H, D).permute(1, 2, 0, 3), out.detach())

    def unpack(g):
        g = g.float().view(L, B, 3, H, D).permute(2, 1, 3, 0, 4).cpu().double().numpy()
        return [g[0], g[1], g[2]]

    got = unpack(qkv_s.grad) + unpack(qkv_m.grad)
    order = (0, 1, 2, 3, 4, 5)
    for i in order:
        _assert16(got[i], ref_g[i], f"from_qkv {NAMES[i]}")


def test_dropout_invalid_p_and_eval():
    """p outside [0, 1) is a ValueError; training=False turns dropout off."""
    print("[dropout p range]", flush=True)
    m = _m()
    x32 = torch.randn(1, 2, 64, 32, device=DEV)
    cid = torch.zeros(1, 64, dtype=torch.int32, device=DEV)
    xb = x32.to(torch.bfloat16)
    with pytest.raises(ValueError):
        m.fused_multi_pathway_attention(xb, xb, xb, xb, xb, xb, None, dropout_p=1.0,
                                        chain_ids=cid)
    a = m.fused_multi_pathway_attention(x32, x32, x32, x32, x32, x32, None, dropout_p=0.1,
                                        training=False, chain_ids=cid)
    b = m.fused_multi_pathway_attention(x32, x32, x32, x32, x32, x32, None, chain_ids=cid)
    torch.cuda.synchronize()
    assert torch.equal(a, b)


def _assert32(got, ref, what):
    err = np.abs(got - ref)
    rel = np.linalg.norm(got - ref) / max(np.linalg.norm(ref), 1e-30)
    assert err.max() <= 1e-4 and rel <= 1e-4, f"{what}: max err {err.max():.3g}, relative {rel:.3g}"


@pytest.mark.parametrize("D,L,sqrt", [(16, 200, False), (32, 257, False), (64, 150, False),
                                      (16, 180, True), (24, 130, True)])
def test_dropout_fp32(D, L, sqrt):
    """fp32 inputs with dropout (and with sqrt-softmax): forward and all six
    gradients against the oracle at the fp32 bound (1e-4 max-abs and
    relative Frobenius), Q/K N(0, 1) with scale D^-1/2 and dO scaled so the
    largest gradient RMS is ~1."""
    print(f"[dropout fp32] D={D} L={L} sqrt={sqrt}", flush=True)
    B, H, p, seed = 2, 3, 0.2, 99 + D + L
    rng = np.random.default_rng(D * 1000 + L)
    xs = [rng.standard_normal((B, H, L, D)).astype(np.float32) for _ in range(6)]
    cid = multi_chain_ids(rng, B, L, 3)
    kp = tail_padding(rng, B, L, 0.1)
    go = rng.standard_normal((B, H, L, D)).astype(np.float32)
    sel = dict(chain_ids=cid, key_pad=kp, rope=True, scale=D ** -0.5, sqrt_softmax=sqrt,
               dropout_p=p, dropout_seed=seed)
    x64 = [x.astype(np.float64) for x in xs]
    ref_o, _ = orc.mpattn_forward(*x64, **sel)
    ref = orc.mpattn_backward(*x64, go.astype(np.float64), **sel)
    f = 2.0 ** -round(np.log2(max(float(np.sqrt(np.mean(r ** 2))) for r in ref)))
    go = (go * np.float32(f)).astype(np.float32)
    ref = [r * f for r in ref]
    m = _m()
    g = [torch.from_numpy(x).to(DEV) for x in xs]
    kw = dict(chain_ids=torch.from_numpy(cid).to(DEV), key_padding_mask=torch.from_numpy(kp).to(DEV),
              rope=True, scale=D ** -0.5, sqrt_softmax=sqrt, dropout_p=p, dropout_seed=seed)
    out = m.fused_multi_pathway_attention(*g, None, training=True, **kw)
    grads = m.fused_multi_pathway_attention_bwd(*g, None, torch.from_numpy(go).to(DEV), **kw)
    torch.cuda.synchronize()
    _assert32(out.cpu().double().numpy(), ref_o, "out")
    ref0, _ = orc.mpattn_forward(*x64, **dict(sel, dropout_p=0.0))
    assert np.abs(ref_o - ref0).max() > 1e-2  # the mask changes the result
    for name, t, r in zip(NAMES, grads, ref):
        assert t.dtype == torch.float32
        _assert32(t.cpu().double().numpy(), r, name)


@pytest.mark.parametrize("dtype,D,L", [(torch.bfloat16, 32, 257), (torch.float16, 64, 200),
                                       (torch.bfloat16, 16, 140)])
def test_dropout_sqrt_softmax_16bit(dtype, D, L):
    """Dropout of the sqrt(P) weights (16-bit kernels): forward and
    gradients against the oracle at the 16-bit bound."""
    print(f"[dropout sqrt] {dtype} D={D} L={L}", flush=True)
    B, H, p, seed = 2, 3, 0.25, 7 + D
    xs, go, cid, kp = _random(B, H, L, D, seed=D + 3 * L)
    xr = _rounded(xs, dtype)
    sel = dict(chain_ids=cid, key_pad=kp, rope=True, scale=D ** -0.5, sqrt_softmax=True,
               dropout_p=p, dropout_seed=seed)
    ref_o, _ = orc.mpattn_forward(*xr, **sel)
    ref = orc.mpattn_backward(*xr, _rounded([go], dtype)[0], **sel)
    m = _m()
    g = [torch.as_tensor(x).to(dtype).to(DEV) for x in xs]
    kw = dict(chain_ids=torch.from_numpy(cid).to(DEV), key_padding_mask=torch.from_numpy(kp).to(DEV),
              rope=True, scale=D ** -0.5, sqrt_softmax=True, dropout_p=p, dropout_seed=seed)
    out = m.fused_multi_pathway_attention(*g, None, training=True, **kw)
    grads = m.fused_multi_pathway_attention_bwd(*g, None, torch.as_tensor(go).to(dtype).to(DEV), **kw)
    torch.cuda.synchronize()
    _assert16(out.float().cpu().double().numpy(), ref_o, "out")
    ref0, _ = orc.mpattn_forward(*xr, **dict(sel, dropout_p=0.0))
    assert np.abs(ref_o - ref0).max() > 0.1  # the mask changes the result
    for name, t, r in zip(NAMES, grads, ref):
        _assert16(t.float().cpu().double().numpy(), r, name)


def test_dropout_long_rows():
    """L = 1024 (the 150M sequence length), two heads: rows span 16 key
    stages, so every stage offset of the key index enters the mask."""
    print("[dropout L=1024]", flush=True)
    B, H, L, D, p, seed = 1, 2, 1024, 32, 0.1, 4
    xs, go, cid, kp = _random(B, H, L, D, seed=1024)
    dt = torch.bfloat16
    xr = _rounded(xs, dt)
    ref_o, _ = orc.mpattn_forward(*xr, chain_ids=cid, key_pad=kp, rope=True, scale=D ** -0.5,
                                  dropout_p=p, dropout_seed=seed)
    got_o = _gpu_fwd(xs, cid, kp, p, seed, dt, rope=True, scale=D ** -0.5)
    _assert16(got_o, ref_o, "out")
    got = _gpu_bwd(xs, go, cid, kp, p, seed, dt, rope=True, scale=D ** -0.5)
    ref = orc.mpattn_backward(*xr, _rounded([go], dt)[0], chain_ids=cid, key_pad=kp, rope=True,
                              scale=D ** -0.5, dropout_p=p, dropout_seed=seed)
    for name, g, r in zip(NAMES, got, ref):
        _assert16(g, r, name)


def test_dropout_layer_fused_equals_combine_path():
    """A multimer layer in training mode with attention dropout: the fused
    path and the materialised combine path draw the same seed from torch's
    CPU generator and use the same mask, so their outputs and input
    gradients agree to the bf16 tolerance; without the same seed they do
    not."""
    print("[dropout layer]", flush=True)
    from mint_plus_amd import modules as M
    torch.manual_seed(21)
    T, B, E, H = 160, 2, 640, 20
    layer = M.TransformerLayer_MINT(E, 4 * E, H, use_multimer=True).to(DEV, torch.bfloat16).train()
    layer.self_attn.dropout = 0.2
    rng = np.random.default_rng(3)
    x = torch.from_numpy(rng.standard_normal((T, B, E)).astype(np.float32)).to(torch.bfloat16)
    cid = torch.from_numpy(two_chain_ids(rng, B, T)).to(DEV)
    kp = torch.zeros(B, T, dtype=torch.bool, device=DEV)
    kp[1, T - 12:] = True
    go = torch.from_numpy(rng.standard_normal((T, B, E)).astype(np.float32)).to(DEV)

    def run(fused, seed):
        layer._use_fused_multi_pathway = fused
        xi = x.to(DEV).requires_grad_(True)
        torch.manual_seed(seed)
        y, _ = layer(xi, self_attn_padding_mask=kp, chain_ids=cid)
        (y.float() * go).sum().backward()
        return y.detach().float().cpu().double().numpy(), xi.grad.float().cpu().double().numpy()

    yf, gf = run(True, 100)
    yc, gc = run(False, 100)
    yo, _ = run(True, 101)
    torch.cuda.synchronize()
    valid = ~kp.cpu().numpy().T[:, :, None]  # (T, B, 1): outputs of unpadded tokens
    _assert16(np.where(valid, yf, 0), np.where(valid, yc, 0), "layer output fused vs combine")
    err = np.linalg.norm(gf - gc) / np.linalg.norm(gc)
    assert err < 2e-2, f"input gradient fused vs combine: relative error {err:.3g}"
    assert np.abs(yo - yf).max() > 0.05  # another seed, another mask
