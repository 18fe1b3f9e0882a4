"""Pins of the CPU oracle (runs without a GPU).

Each oracle function is checked against something it does not share code
with: closed forms and hand-computed vectors for RoPE, torch's
``scaled_dot_product_attention`` (a library routine) on concatenated
features for the forward, torch autograd of that construction and central
finite differences for the backward, invariants the op must satisfy, and the
pure-Python loop on tiny inputs. A plausible slip (a dropped term, a swapped
pathway, a wrong sign or rotation pairing, a transposed operand) fails at
least one of them.
"""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

from conftest import multi_chain_ids, tail_padding, two_chain_ids
from oracle import mpattn_oracle as orc
from oracle import torch_ref
from indep import rope_complex, sdpa_concat


def rand_inputs(rng, B, H, L, D, sigma=None):
    sigma = D ** -0.5 if sigma is None else sigma
    return [rng.standard_normal((B, H, L, D)) * sigma for _ in range(6)]


# ---------------------------------------------------------------------------
# RoPE
# ---------------------------------------------------------------------------
def test_rope_half_split_known_vector():
    """D = 4, position 1, x = e_0: half-split pairs (0, 2), so R x =
    [cos 1, 0, sin 1, 0] (an interleaved layout would give [cos 1, sin 1, 0, 0])."""
    cos, sin = orc.rope_tables(2, 4)
    x = np.zeros((2, 4))
    x[1, 0] = 1.0
    y = orc.apply_rope(x, cos, sin)
    np.testing.assert_allclose(y[1], [np.cos(1.0), 0.0, np.sin(1.0), 0.0], atol=1e-15)
    # second frequency: theta_1 = 10000^(-2/4) = 1/100
    x[1] = [0, 1, 0, 0]
    y = orc.apply_rope(x, cos, sin)
    a = float(np.float32(1.0) * np.float32(0.01))
    np.testing.assert_allclose(y[1], [0.0, np.cos(a), 0.0, np.sin(a)], atol=1e-15)


@pytest.mark.parametrize("D", [16, 24, 32, 64])
def test_rope_matches_complex_rotation(D):
    rng = np.random.default_rng(D)
    L = 300
    x = rng.standard_normal((3, L, D))
    cos, sin = orc.rope_tables(L, D)
    np.testing.assert_allclose(orc.apply_rope(x, cos, sin), rope_complex(x, np.arange(L)),
                               atol=1e-12)


def test_rope_identity_norm_and_transpose():
    rng = np.random.default_rng(1)
    L, D = 64, 32
    x = rng.standard_normal((2, L, D))
    g = rng.standard_normal((2, L, D))
    cos, sin = orc.rope_tables(L, D)
    y = orc.apply_rope(x, cos, sin)
    np.testing.assert_allclose(y[:, 0], x[:, 0], atol=0)  # position 0: identity
    np.testing.assert_allclose(np.linalg.norm(y, axis=-1), np.linalg.norm(x, axis=-1), rtol=1e-12)
    # <R x, g> == <x, R^T g>
    np.testing.assert_allclose((y * g).sum(), (x * orc.apply_rope_transpose(g, cos, sin)).sum(),
                               rtol=1e-12)
    np.testing.assert_allclose(orc.apply_rope_transpose(y, cos, sin), x, atol=1e-12)


def test_rope_relative_position():
    """<R_i q, R_j k> = <q, R_{j-i} k>: only the offset matters (up to the
    fp32 rounding of the angle, ~1e-5 rad at these positions)."""
    rng = np.random.default_rng(2)
    L, D = 200, 32
    cos, sin = orc.rope_tables(L, D)
    q, k = rng.standard_normal(D), rng.standard_normal(D)
    for i, j in [(0, 5), (17, 60), (100, 199), (42, 42)]:
        Q = np.zeros((L, D)); Q[i] = q
        K = np.zeros((L, D)); K[j] = k
        lhs = orc.apply_rope(Q, cos, sin)[i] @ orc.apply_rope(K, cos, sin)[j]
        K2 = np.zeros((L, D)); K2[j - i] = k
        rhs = q @ orc.apply_rope(K2, cos, sin)[j - i]
        assert abs(lhs - rhs) < 1e-4 * np.linalg.norm(q) * np.linalg.norm(k)


# ---------------------------------------------------------------------------
# Forward
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("rope", [False, True])
@pytest.mark.parametrize("nchains,L,D", [(1, 33, 16), (2, 64, 32), (3, 57, 24), (4, 40, 64)])
def test_forward_vs_sdpa_concat(rope, nchains, L, D):
    rng = np.random.default_rng(100 + L + D + nchains)
    B, H = 2, 3
    xs = rand_inputs(rng, B, H, L, D, sigma=0.7)
    cid = multi_chain_ids(rng, B, L, nchains) if nchains != 2 else two_chain_ids(rng, B, L)
    if nchains == 3:  # non-contiguous chains too
        cid = rng.integers(0, 3, size=(B, L)).astype(np.int32)
    kp = tail_padding(rng, B, L, 0.2)
    scale = D ** -0.5
    out, lse = orc.mpattn_forward(*xs, chain_ids=cid, key_pad=kp, rope=rope, scale=scale)
    ref, logits, _ = sdpa_concat(*xs, cid, kp, rope, scale)
    np.testing.assert_allclose(out, ref.numpy(), atol=1e-12, rtol=1e-10)
    # LSE: logsumexp over valid keys of the SDPA construction's logits
    lg = logits.numpy()
    lg = np.where(kp[:, None, None, :], -np.inf, lg)
    np.testing.assert_allclose(lse, np.logaddexp.reduce(lg, axis=-1), atol=1e-12)


def test_forward_single_chain_is_sdpa_with_rope():
    rng = np.random.default_rng(5)
    B, H, L, D = 2, 2, 50, 32
    xs = rand_inputs(rng, B, H, L, D)
    cid = np.zeros((B, L), np.int32)
    kp = tail_padding(rng, B, L, 0.2)
    out, _ = orc.mpattn_forward(*xs, chain_ids=cid, key_pad=kp, rope=True, scale=D ** -0.5)
    pos = np.arange(L)
    qr = torch.as_tensor(rope_complex(xs[0], pos))
    kr = torch.as_tensor(rope_complex(xs[1], pos))
    mask = torch.as_tensor(~kp)[:, None, None, :]
    ref = F.scaled_dot_product_attention(qr, kr, torch.as_tensor(xs[2]), attn_mask=mask)
    np.testing.assert_allclose(out, ref.numpy(), atol=1e-10)


def test_forward_all_cross_mask_is_sdpa_multi():
    """A dense mask that is True everywhere selects the multimer pathway only."""
    rng = np.random.default_rng(6)
    B, H, L, D = 2, 2, 45, 16
    xs = rand_inputs(rng, B, H, L, D)
    cm = np.ones((B, L, L), bool)
    out, _ = orc.mpattn_forward(*xs, chain_mask=cm, rope=True, scale=0.3)
    t = [torch.as_tensor(a) for a in xs]
    ref = F.scaled_dot_product_attention(t[3], t[4], t[5], scale=0.3)
    np.testing.assert_allclose(out, ref.numpy(), atol=1e-12)


@pytest.mark.parametrize("rope", [False, True])
@pytest.mark.parametrize("nchains", [1, 2, 3])
def test_forward_vs_python_loops(rope, nchains):
    rng = np.random.default_rng(7 + nchains)
    B, H, L, D = 2, 1, 37, 8
    xs = rand_inputs(rng, B, H, L, D, sigma=0.8)
    cid = rng.integers(0, nchains, size=(B, L)).astype(np.int32)
    kp = tail_padding(rng, B, L, 0.3)
    out, _ = orc.mpattn_forward(*xs, chain_ids=cid, key_pad=kp, rope=rope, scale=0.4)
    loops = orc.mpattn_forward_loops(*[a.tolist() for a in xs], cid.tolist(), kp.tolist(),
                                     rope=rope, scale=0.4)
    np.testing.assert_allclose(out, loops, atol=1e-12)


def test_forward_invariants():
    rng = np.random.default_rng(8)
    B, H, L, D = 2, 2, 40, 16
    xs = rand_inputs(rng, B, H, L, D)
    cid = rng.integers(0, 3, size=(B, L)).astype(np.int32)
    kp = tail_padding(rng, B, L, 0.2)
    kw = dict(key_pad=kp, rope=True, scale=0.25)
    out, _ = orc.mpattn_forward(*xs, chain_ids=cid, **kw)
    # relabelling chains changes nothing
    perm = np.array([7, -3, 11], np.int32)
    out2, _ = orc.mpattn_forward(*xs, chain_ids=perm[cid], **kw)
    np.testing.assert_allclose(out, out2, atol=0)
    # appended padded keys change nothing for the original queries
    ext = [np.concatenate([a, rng.standard_normal((B, H, 5, D))], axis=2) for a in xs]
    cid_e = np.concatenate([cid, rng.integers(0, 3, size=(B, 5)).astype(np.int32)], axis=1)
    kp_e = np.concatenate([kp, np.ones((B, 5), bool)], axis=1)
    out_e, _ = orc.mpattn_forward(*ext, chain_ids=cid_e, key_pad=kp_e, rope=True, scale=0.25)
    np.testing.assert_allclose(out_e[:, :, :L], out, atol=1e-14)
    # constant V: every row of a valid sample is that constant
    ones = np.ones((B, H, L, D))
    o1, _ = orc.mpattn_forward(xs[0], xs[1], ones, xs[3], xs[4], ones, chain_ids=cid, **kw)
    np.testing.assert_allclose(o1, 1.0, atol=1e-14)
    # zero queries: uniform weights -> mean over valid keys of the selected V
    z = np.zeros_like(xs[0])
    o0, _ = orc.mpattn_forward(z, xs[1], xs[2], z, xs[4], xs[5], chain_ids=cid, **kw)
    same = cid[:, :, None] == cid[:, None, :]
    w = (~kp)[:, None, :] / (~kp).sum(-1)[:, None, None]
    ref = np.einsum("bij,bhjd->bhid", np.where(same, w, 0), xs[2]) + \
        np.einsum("bij,bhjd->bhid", np.where(same, 0, w), xs[5])
    np.testing.assert_allclose(o0, ref, atol=1e-14)
    # L = 1: the only key is the query's own (same chain) -> v_self
    x1 = [a[:, :, :1] for a in xs]
    o_1, _ = orc.mpattn_forward(*x1, chain_ids=cid[:, :1], rope=True, scale=0.25)
    np.testing.assert_allclose(o_1, xs[2][:, :, :1], atol=0)


def test_forward_all_padded_sample():
    rng = np.random.default_rng(9)
    B, H, L, D = 2, 2, 20, 16
    xs = rand_inputs(rng, B, H, L, D)
    cid = two_chain_ids(rng, B, L)
    kp = np.zeros((B, L), bool)
    kp[1] = True
    out, lse = orc.mpattn_forward(*xs, chain_ids=cid, key_pad=kp, rope=True, scale=0.25)
    assert np.all(out[1] == 0) and np.all(np.isneginf(lse[1]))
    assert np.all(np.isfinite(out[0])) and np.all(np.isfinite(lse[0]))


def test_forward_sqrt_softmax_closed_form():
    """sqrt_softmax: O = sum_j sqrt(P_ij) V_sel, with P the softmax of the
    concatenated-feature logits over valid keys."""
    rng = np.random.default_rng(10)
    B, H, L, D = 1, 2, 30, 16
    xs = rand_inputs(rng, B, H, L, D)
    cid = two_chain_ids(rng, B, L)
    kp = tail_padding(rng, B, L, 0.2)
    out, _ = orc.mpattn_forward(*xs, chain_ids=cid, key_pad=kp, rope=True, scale=0.25,
                                sqrt_softmax=True)
    _, logits, _ = sdpa_concat(*xs, cid, kp, True, 0.25)
    lg = np.where(kp[:, None, None, :], -np.inf, logits.numpy())
    P = np.exp(lg - np.logaddexp.reduce(lg, axis=-1, keepdims=True))
    same = (cid[:, :, None] == cid[:, None, :])[:, None]
    ref = np.einsum("bhij,bhjd->bhid", np.where(same, np.sqrt(P), 0), xs[2]) + \
        np.einsum("bhij,bhjd->bhid", np.where(same, 0, np.sqrt(P)), xs[5])
    np.testing.assert_allclose(out, ref, atol=1e-12)


# ---------------------------------------------------------------------------
# Dropout mask
# ---------------------------------------------------------------------------
def _murmur3_x86_32(data, seed):
    """MurmurHash3_x86_32 (Appleby's published algorithm), body in Python
    ints, finalised by the oracle's fmix32."""
    c1, c2, m32 = 0xCC9E2D51, 0x1B873593, 0xFFFFFFFF
    rotl = lambda x, r: ((x << r) | (x >> (32 - r))) & m32
    h, n = seed, len(data)
    for i in range(0, n // 4 * 4, 4):
        k = int.from_bytes(data[i:i + 4], "little")
        k = (rotl((k * c1) & m32, 15) * c2) & m32
        h = (rotl(h ^ k, 13) * 5 + 0xE6546B64) & m32
    tail = data[n // 4 * 4:]
    if tail:
        k = int.from_bytes(tail, "little")
        h ^= (rotl((k * c1) & m32, 15) * c2) & m32
    return int(orc.fmix32(np.uint32(h ^ n)))


def test_fmix32_murmur3_known_answers():
    """Published MurmurHash3_x86_32 test vectors; for the empty string the
    hash is fmix32(seed)."""
    assert int(orc.fmix32(np.uint32(0))) == 0
    assert int(orc.fmix32(np.uint32(1))) == 0x514E28B7
    assert int(orc.fmix32(np.uint32(0xFFFFFFFF))) == 0x81F16F39
    assert _murmur3_x86_32(b"test", 0) == 0xBA6BD213
    assert _murmur3_x86_32(b"Hello, world!", 1234) == 0xFAF6CDB3
    # vectorised form == scalar form
    xs = np.array([0, 1, 0xFFFFFFFF, 12345, 0x80000000], dtype=np.uint32)
    assert [int(v) for v in orc.fmix32(xs)] == [int(orc.fmix32(np.uint32(v))) for v in xs]


def test_dropout_keep_scalar_restatement():
    """A few elements against the formula evaluated with Python ints: a
    transposed (i, j), a wrong head index or a swapped seed word fails."""
    B, H, L, p, seed = 2, 3, 40, 0.3, 0x1234_5678_9ABC_DEF0
    keep = orc.dropout_keep(B, H, L, p, seed)
    lo, hi, m32 = seed & 0xFFFFFFFF, seed >> 32, 0xFFFFFFFF
    f = lambda x: int(orc.fmix32(np.uint32(x & m32)))
    thr = int(p * 2**24 + 0.5)
    for b, h, i, j in [(0, 0, 0, 0), (1, 2, 39, 0), (0, 1, 3, 17), (1, 0, 20, 39), (1, 2, 7, 8)]:
        row = f(lo ^ ((b * H + h) * 0xC2B2AE3D) ^ (i * 0x9E3779B1))
        r = f(row ^ ((j * 0x85EBCA77 + hi) & m32))
        assert bool(keep[b, h, i, j]) == ((r >> 8) >= thr), (b, h, i, j)
    # asymmetric in (i, j), and the head index matters
    assert not np.array_equal(keep[0, 0], keep[0, 0].T)
    assert not np.array_equal(keep[0, 0], keep[0, 1])


def test_dropout_keep_statistics():
    B, H, L = 2, 3, 256
    n = B * H * L * L
    assert orc.dropout_keep(B, H, L, 0.0, 5).all()  # p = 0 keeps everything
    for p in (0.1, 0.5, 0.9):
        k = orc.dropout_keep(B, H, L, p, 77)
        sd = np.sqrt(p * (1 - p) / n)
        assert abs(k.mean() - (1 - p)) < 6 * sd, (p, k.mean())
        # neighbouring keys / queries and different heads are independent
        q = (1 - p) ** 2
        sd2 = np.sqrt(q * (1 - q) / n) * 2
        assert abs((k[..., 1:] & k[..., :-1]).mean() - q) < 6 * sd2
        assert abs((k[:, :, 1:] & k[:, :, :-1]).mean() - q) < 6 * sd2
        assert abs((k[:, 1:] & k[:, :-1]).mean() - q) < 6 * sd2
    # the seed (both words) changes the mask, independently
    a = orc.dropout_keep(1, 2, 128, 0.5, 1)
    for other in (2, 1 + (1 << 32)):
        b = orc.dropout_keep(1, 2, 128, 0.5, other)
        assert abs((a == b).mean() - 0.5) < 0.02


def test_forward_dropout_vs_torch_expression():
    """O = (softmax * Z / (1 - p)) split by pathway, with the softmax from
    torch over the concatenated-feature logits; LSE unchanged by dropout."""
    rng = np.random.default_rng(11)
    B, H, L, D, p = 2, 2, 33, 16, 0.25
    xs = rand_inputs(rng, B, H, L, D)
    cid = two_chain_ids(rng, B, L)
    kp = tail_padding(rng, B, L, 0.2)
    out, lse = orc.mpattn_forward(*xs, chain_ids=cid, key_pad=kp, rope=True, scale=0.3,
                                  dropout_p=p, dropout_seed=99)
    _, lse0 = orc.mpattn_forward(*xs, chain_ids=cid, key_pad=kp, rope=True, scale=0.3)
    np.testing.assert_array_equal(lse, lse0)
    _, logits, _ = sdpa_concat(*xs, cid, kp, True, 0.3)
    lg = logits.masked_fill(torch.as_tensor(kp)[:, None, None, :], float("-inf"))
    P = torch.softmax(lg, dim=-1)
    P = torch.nan_to_num(P, nan=0.0)
    Z = torch.as_tensor(orc.dropout_keep(B, H, L, p, 99)).double() / (1 - np.float32(p))
    same = torch.as_tensor(cid[:, :, None] == cid[:, None, :])[:, None]
    Pd = P * Z
    ref = torch.where(same, Pd, 0) @ torch.as_tensor(xs[2]) + \
        torch.where(same, 0, Pd) @ torch.as_tensor(xs[5])
    np.testing.assert_allclose(out, ref.numpy(), atol=1e-12)


# ---------------------------------------------------------------------------
# Backward
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("rope", [False, True])
def test_backward_vs_autograd_of_sdpa_concat(rope):
    rng = np.random.default_rng(20 + rope)
    B, H, L, D = 2, 2, 36, 16
    xs = rand_inputs(rng, B, H, L, D, sigma=0.6)
    cid = rng.integers(0, 3, size=(B, L)).astype(np.int32)
    kp = tail_padding(rng, B, L, 0.2)
    go = rng.standard_normal((B, H, L, D))
    grads = orc.mpattn_backward(*xs, go, chain_ids=cid, key_pad=kp, rope=rope, scale=0.3)
    out, _, leaves = sdpa_concat(*xs, cid, kp, rope, 0.3, requires_grad=True)
    (out * torch.as_tensor(go)).sum().backward()
    for g, leaf in zip(grads, leaves):
        np.testing.assert_allclose(g, leaf.grad.numpy(), atol=1e-11)


@pytest.mark.parametrize("sqrt_softmax,dropout_p", [(False, 0.0), (True, 0.0), (False, 0.3)])
def test_backward_finite_differences(sqrt_softmax, dropout_p):
    """Central differences; with dropout the mask is fixed by the seed."""
    rng = np.random.default_rng(30 + sqrt_softmax)
    B, H, L, D = 1, 2, 14, 8
    xs = rand_inputs(rng, B, H, L, D, sigma=0.7)
    cid = two_chain_ids(rng, B, L)
    kp = np.zeros((B, L), bool)
    kp[0, -3:] = True
    go = rng.standard_normal((B, H, L, D))
    kw = dict(chain_ids=cid, key_pad=kp, rope=True, scale=0.35, sqrt_softmax=sqrt_softmax,
              dropout_p=dropout_p, dropout_seed=4242)
    grads = orc.mpattn_backward(*xs, go, **kw)

    def f(args):
        return float((orc.mpattn_forward(*args, **kw)[0] * go).sum())

    eps = 1e-6
    for i in range(6):
        for trial in range(2):
            d = rng.standard_normal(xs[i].shape)
            plus = [a.copy() for a in xs]
            minus = [a.copy() for a in xs]
            plus[i] += eps * d
            minus[i] -= eps * d
            fd = (f(plus) - f(minus)) / (2 * eps)
            an = float((grads[i] * d).sum())
            assert abs(fd - an) <= 1e-6 * max(1.0, abs(an)), (i, trial, fd, an)


def test_backward_dense_mask_equals_chain_ids():
    rng = np.random.default_rng(40)
    B, H, L, D = 2, 2, 30, 16
    xs = rand_inputs(rng, B, H, L, D)
    cid = rng.integers(0, 2, size=(B, L)).astype(np.int32)
    go = rng.standard_normal((B, H, L, D))
    a = orc.mpattn_backward(*xs, go, chain_ids=cid, rope=False, scale=1.0)
    b = orc.mpattn_backward(*xs, go, chain_mask=cid[:, :, None] != cid[:, None, :], rope=False,
                            scale=1.0)
    for x, y in zip(a, b):
        np.testing.assert_array_equal(x, y)


# ---------------------------------------------------------------------------
# torch restatement used at the benchmark shape
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("dense", [False, True])
def test_torch_ref_matches_oracle(dense):
    rng = np.random.default_rng(50 + dense)
    B, H, L, D = 3, 2, 70, 32
    xs = rand_inputs(rng, B, H, L, D)
    cid = two_chain_ids(rng, B, L)
    kp = tail_padding(rng, B, L, 0.2)
    kp[2] = True
    out, lse = orc.mpattn_forward(*xs, chain_ids=cid, key_pad=kp, rope=True, scale=D ** -0.5)
    t = [torch.as_tensor(a) for a in xs]
    sel = dict(chain_mask=torch.as_tensor(cid[:, :, None] != cid[:, None, :])) if dense else \
        dict(chain_ids=torch.as_tensor(cid))
    o2, l2 = torch_ref.forward(*t, key_pad=torch.as_tensor(kp), rope=True, scale=D ** -0.5,
                               dtype=torch.float64, chunk=2, **sel)
    np.testing.assert_allclose(o2.numpy(), out, atol=1e-12)
    np.testing.assert_allclose(l2.numpy(), lse, atol=1e-12)


# ---------------------------------------------------------------------------
# Materialised combine
# ---------------------------------------------------------------------------
def _torch_logits(xs, cid, kp, scale):
    """Both pathways' logits with torch (RoPE by complex multiplication),
    padded keys at -inf: the inputs fused_multimer_combine receives."""
    qs, ks, _, qm, km, _ = xs
    L = qs.shape[2]
    qr, kr = rope_complex(qs, np.arange(L)), rope_complex(ks, np.arange(L))
    t = lambda a: torch.as_tensor(np.asarray(a, np.float64))
    il = scale * torch.matmul(t(qr), t(kr).transpose(-1, -2))
    el = scale * torch.matmul(t(qm), t(km).transpose(-1, -2))
    pad = torch.as_tensor(kp)[:, None, None, :]
    return il.masked_fill(pad, float("-inf")).numpy(), el.masked_fill(pad, float("-inf")).numpy()


def test_combine_equals_fused_op_on_torch_logits():
    rng = np.random.default_rng(60)
    B, H, L, D = 2, 3, 45, 16
    xs = rand_inputs(rng, B, H, L, D, sigma=0.8)
    cid = multi_chain_ids(rng, B, L, 3)
    kp = tail_padding(rng, B, L, 0.2)
    kp[1] = True
    il, el = _torch_logits(xs, cid, kp, 0.4)
    out, lse = orc.combine_forward(il, el, cid[:, :, None] != cid[:, None, :], xs[2], xs[5])
    ref, ref_lse = orc.mpattn_forward(*xs, chain_ids=cid, key_pad=kp, rope=True, scale=0.4)
    np.testing.assert_allclose(out, ref, atol=1e-12)
    np.testing.assert_allclose(lse, ref_lse, atol=1e-12)
    assert np.all(out[1] == 0.0)


def test_combine_single_chain_is_softmax_of_intra():
    rng = np.random.default_rng(61)
    B, H, L, D = 2, 2, 33, 8
    il, el = rng.standard_normal((2, B, H, L, L))
    vs, vm = rng.standard_normal((2, B, H, L, D))
    out, _ = orc.combine_forward(il, el, np.zeros((B, L, L), bool), vs, vm)
    ref = torch.softmax(torch.as_tensor(il), -1) @ torch.as_tensor(vs)
    np.testing.assert_allclose(out, ref.numpy(), atol=1e-12)
    out2, _ = orc.combine_forward(il, el, np.ones((B, L, L), bool), vs, vm)
    ref2 = torch.softmax(torch.as_tensor(el), -1) @ torch.as_tensor(vm)
    np.testing.assert_allclose(out2, ref2.numpy(), atol=1e-12)


def test_combine_backward_vs_autograd():
    rng = np.random.default_rng(62)
    B, H, L, D = 2, 2, 29, 8
    il, el = rng.standard_normal((2, B, H, L, L)) * 2
    il[:, :, :, -3:] = -np.inf
    el[:, :, :, -3:] = -np.inf
    vs, vm, go = rng.standard_normal((3, B, H, L, D))
    cm = rng.random((B, L, L)) < 0.4
    grads = orc.combine_backward(il, el, cm, vs, vm, go)
    leaves = [torch.as_tensor(a).requires_grad_(True) for a in (il, el, vs, vm)]
    m = torch.as_tensor(cm)[:, None]
    p = torch.softmax(torch.where(m, leaves[1], leaves[0]), -1)
    out = p.masked_fill(m, 0.0) @ leaves[2] + p.masked_fill(~m, 0.0) @ leaves[3]
    (out * torch.as_tensor(go)).sum().backward()
    for g, leaf in zip(grads, leaves):
        ref = torch.nan_to_num(leaf.grad, nan=0.0).numpy()
        np.testing.assert_allclose(np.nan_to_num(g), ref, atol=1e-12)


def test_combine_backward_finite_differences():
    rng = np.random.default_rng(63)
    B, H, L, D = 1, 2, 11, 4
    il, el = rng.standard_normal((2, B, H, L, L))
    vs, vm, go = rng.standard_normal((3, B, H, L, D))
    cm = rng.random((B, L, L)) < 0.5
    grads = orc.combine_backward(il, el, cm, vs, vm, go)
    args = [il, el, vs, vm]

    def f(a):
        return float((orc.combine_forward(a[0], a[1], cm, a[2], a[3])[0] * go).sum())

    eps = 1e-6
    for i in range(4):
        d = rng.standard_normal(args[i].shape)
        plus = [x.copy() for x in args]
        minus = [x.copy() for x in args]
        plus[i] += eps * d
        minus[i] -= eps * d
        fd = (f(plus) - f(minus)) / (2 * eps)
        an = float((grads[i] * d).sum())
        assert abs(fd - an) <= 1e-6 * max(1.0, abs(an)), (i, fd, an)


def test_combine_dropout_equals_fused_op_dropout():
    """Fed the two pathways' logits, the combine with dropout equals the fused
    op with the same seed (forward and every gradient through the chain
    rule of the logits), and its backward matches central differences."""
    rng = np.random.default_rng(62)
    B, H, L, D, p, seed = 2, 2, 20, 8, 0.3, 777
    xs = rand_inputs(rng, B, H, L, D)
    cid = two_chain_ids(rng, B, L)
    kp = tail_padding(rng, B, L, 0.2)
    il, el = _torch_logits(xs, cid, kp, 0.3)
    cm = cid[:, :, None] != cid[:, None, :]
    out_c, lse_c = orc.combine_forward(il, el, cm, xs[2], xs[5], dropout_p=p, dropout_seed=seed)
    out_f, lse_f = orc.mpattn_forward(*xs, chain_ids=cid, key_pad=kp, rope=True, scale=0.3,
                                      dropout_p=p, dropout_seed=seed)
    np.testing.assert_allclose(out_c, out_f, atol=1e-12)
    np.testing.assert_allclose(lse_c, lse_f, atol=1e-12)
    go = rng.standard_normal((B, H, L, D))
    d_il, d_el, d_vs, d_vm = orc.combine_backward(il, el, cm, xs[2], xs[5], go, dropout_p=p,
                                                  dropout_seed=seed)
    g = orc.mpattn_backward(*xs, go, chain_ids=cid, key_pad=kp, rope=True, scale=0.3,
                            dropout_p=p, dropout_seed=seed)
    np.testing.assert_allclose(d_vs, g[2], atol=1e-12)
    np.testing.assert_allclose(d_vm, g[5], atol=1e-12)
    # dQ_multi = scale * d_inter @ K_multi
    np.testing.assert_allclose(0.3 * np.einsum("bhij,bhjd->bhid", d_el, xs[4]), g[3], atol=1e-12)
    # finite differences in one logit tensor (finite entries only)
    fin = np.isfinite(il)
    d = np.where(fin, rng.standard_normal(il.shape), 0.0)
    eps = 1e-6
    f = lambda x: float((orc.combine_forward(x, el, cm, xs[2], xs[5], dropout_p=p,
                                             dropout_seed=seed)[0] * go).sum())
    fd = (f(np.where(fin, il + eps * d, il)) - f(np.where(fin, il - eps * d, il))) / (2 * eps)
    assert abs(fd - float((np.where(fin, d_il, 0) * d).sum())) < 1e-6 * max(1.0, abs(fd))
