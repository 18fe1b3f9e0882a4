"""fp32 forward parity of the HIP kernel (the ESM-2 8M configuration runs in
fp32) against the float64 oracle.

Tolerance (stated for fp32 by the task): max |gpu - ref| <= 1e-4.
"""
import numpy as np
import pytest
import torch

from conftest import multi_chain_ids, tail_padding, two_chain_ids
from oracle import mpattn_oracle as orc

pytestmark = pytest.mark.gpu

ATOL32 = 1e-4
DEV = "cuda:0"


def _mpattn():
    import mint_plus_amd
    return mint_plus_amd


def make_inputs(B, H, L, D, seed, sigma=None, nchains=2, pad=True):
    rng = np.random.default_rng(seed)
    sigma = D ** -0.5 if sigma is None else sigma
    xs = [rng.standard_normal((B, H, L, D)).astype(np.float32) * np.float32(sigma) for _ in range(6)]
    cid = two_chain_ids(rng, B, L) if nchains == 2 else multi_chain_ids(rng, B, L, nchains)
    kp = tail_padding(rng, B, L) if pad else np.zeros((B, L), dtype=bool)
    return xs, cid, kp


def run(xs, cid, kp, rope, scale, dense=False, sqrt_softmax=False, need_lse=False):
    m = _mpattn()
    g = [torch.from_numpy(x).to(DEV) for x in xs]
    kw = dict(key_padding_mask=torch.from_numpy(kp).to(DEV), rope=rope, scale=scale,
              sqrt_softmax=sqrt_softmax, need_lse=True)
    if dense:
        c = torch.from_numpy(cid)
        kw["chain_mask"] = (c[:, :, None] != c[:, None, :]).to(DEV)
    else:
        kw["chain_ids"] = torch.from_numpy(cid).to(DEV)
    out, lse = m._lib.mpattn_fwd(*g, **kw)
    torch.cuda.synchronize()
    return out.double().cpu().numpy(), (lse.double().cpu().numpy() if need_lse else None)


def oracle(xs, cid, kp, rope, scale, sqrt_softmax=False):
    return orc.mpattn_forward(*[x.astype(np.float64) for x in xs], chain_ids=cid, key_pad=kp,
                              rope=rope, scale=scale, sqrt_softmax=sqrt_softmax)


@pytest.mark.parametrize("D", [16, 24, 32, 64])
@pytest.mark.parametrize("L", [40, 130])
def test_fp32_fwd(D, L):
    print(f"[fp32] D={D} L={L}", flush=True)
    xs, cid, kp = make_inputs(2, 3, L, D, seed=500 + D + L)
    got, lse = run(xs, cid, kp, rope=True, scale=D ** -0.5, need_lse=True)
    ref, lse_ref = oracle(xs, cid, kp, rope=True, scale=D ** -0.5)
    assert np.abs(got - ref).max() <= ATOL32, np.abs(got - ref).max()
    assert np.abs(lse - lse_ref).max() <= ATOL32


@pytest.mark.parametrize("nchains", [1, 3])
def test_fp32_chains_sharp(nchains):
    """Sharper logits (sigma 1) and 1 or 3 chains."""
    print(f"[fp32 chains] n={nchains}", flush=True)
    xs, cid, kp = make_inputs(2, 2, 150, 16, seed=600 + nchains, sigma=1.0, nchains=nchains)
    got, _ = run(xs, cid, kp, rope=True, scale=0.25)
    ref, _ = oracle(xs, cid, kp, rope=True, scale=0.25)
    assert np.abs(got - ref).max() <= ATOL32, np.abs(got - ref).max()


def test_fp32_dense_no_rope():
    print("[fp32 dense]", flush=True)
    xs, cid, kp = make_inputs(2, 2, 100, 32, seed=610)
    got, _ = run(xs, cid, kp, rope=False, scale=1.0, dense=True)
    ref, _ = oracle(xs, cid, kp, rope=False, scale=1.0)
    assert np.abs(got - ref).max() <= ATOL32, np.abs(got - ref).max()


def test_fp32_sqrt_softmax():
    print("[fp32 sqrt]", flush=True)
    xs, cid, kp = make_inputs(2, 2, 120, 16, seed=620)
    got, lse = run(xs, cid, kp, rope=True, scale=0.25, sqrt_softmax=True, need_lse=True)
    ref, lse_ref = oracle(xs, cid, kp, rope=True, scale=0.25, sqrt_softmax=True)
    assert np.abs(got - ref).max() <= ATOL32, np.abs(got - ref).max()
    assert np.abs(lse - lse_ref).max() <= ATOL32


def test_fp32_all_padded_sample():
    print("[fp32 all padded]", flush=True)
    xs, cid, kp = make_inputs(2, 2, 64, 16, seed=630, pad=False)
    kp[0] = True
    got, _ = run(xs, cid, kp, rope=True, scale=0.25)
    ref, _ = oracle(xs, cid, kp, rope=True, scale=0.25)
    assert np.all(got[0] == 0.0)
    assert np.abs(got - ref).max() <= ATOL32


def test_fp32_8m_config_shape():
    """The 8M configuration's attention shape: B=4, H=20, D=16, two chains of
    U[60,200] + U[40,160] tokens plus <cls>/<eos> each, padded to the batch max."""
    print("[fp32 8M shape]", flush=True)
    rng = np.random.default_rng(8)
    la = rng.integers(60, 201, size=4) + 2
    lb = rng.integers(40, 161, size=4) + 2
    L = int((la + lb).max())
    cid = np.zeros((4, L), np.int32)
    kp = np.zeros((4, L), bool)
    for b in range(4):
        cid[b, la[b]:] = 1
        kp[b, la[b] + lb[b]:] = True
    xs = [rng.standard_normal((4, 20, L, 16)).astype(np.float32) * np.float32(0.5) for _ in range(6)]
    got, _ = run(xs, cid, kp, rope=True, scale=0.25)
    ref, _ = oracle(xs, cid, kp, rope=True, scale=0.25)
    assert np.abs(got - ref).max() <= ATOL32, np.abs(got - ref).max()
