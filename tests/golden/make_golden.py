"""Write the golden fixtures of multi-pathway attention.

Expected values come from ``tests/indep.py`` (torch SDPA on concatenated
features, float64, and its autograd), not from the oracle, so the fixtures
check the oracle as well as the kernels. Inputs are bf16-representable
float32 values, so a bf16 kernel run sees exactly the fixture's inputs;
expected values are stored as float32 (relative rounding 6e-8).

The reference's own tests hold no golden vectors for this path (they
cross-check two implementations on random tensors), so these fixtures are
this build's.

    python tests/golden/make_golden.py      # rewrites mpattn_cases.npz
"""
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))                   # tests/
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))  # repo root

from indep import sdpa_concat  # noqa: E402

# (name, B, H, L, D, chains, rope, scale, pad_frac, seed)
CASES = [
    ("d16_l40_3chains_noncontig", 2, 1, 40, 16, "random3", True, 0.25, 0.2, 1),
    ("d24_l33_2chains_norope", 2, 1, 33, 24, "split2", False, 1.0, 0.15, 2),
    ("d32_l67_2chains_rope", 1, 2, 67, 32, "split2", True, 32 ** -0.5, 0.1, 3),
    ("d64_l29_1chain_rope", 1, 1, 29, 64, "one", True, 0.125, 0.2, 4),
]


def bf16_exact(rng, shape, sigma):
    x = torch.from_numpy((rng.standard_normal(shape) * sigma).astype(np.float32))
    return x.to(torch.bfloat16).float().numpy()


def make_case(B, H, L, D, chains, rope, scale, pad_frac, seed):
    rng = np.random.default_rng(seed)
    xs = [bf16_exact(rng, (B, H, L, D), 0.8 * D ** -0.5 * 2) for _ in range(6)]
    go = bf16_exact(rng, (B, H, L, D), 1.0)
    if chains == "random3":
        cid = rng.integers(0, 3, size=(B, L)).astype(np.int32)
    elif chains == "split2":
        cid = np.zeros((B, L), np.int32)
        for b in range(B):
            cid[b, rng.integers(L // 4, 3 * L // 4):] = 1
    else:
        cid = np.zeros((B, L), np.int32)
    kp = np.zeros((B, L), bool)
    for b in range(B):
        n = int(rng.integers(0, int(pad_frac * L) + 1))
        if n:
            kp[b, L - n:] = True
    out, logits, leaves = sdpa_concat(*[x.astype(np.float64) for x in xs], cid, kp, rope, scale,
                                      requires_grad=True)
    (out * torch.from_numpy(go.astype(np.float64))).sum().backward()
    lg = np.where(kp[:, None, None, :], -np.inf, logits.detach().numpy())
    lse = np.logaddexp.reduce(lg, axis=-1)
    rec = dict(qs=xs[0], ks=xs[1], vs=xs[2], qm=xs[3], km=xs[4], vm=xs[5], go=go, chain_ids=cid,
               key_pad=kp, rope=np.array(rope), scale=np.array(scale, np.float64),
               out=out.detach().numpy().astype(np.float32), lse=lse.astype(np.float32))
    for n, leaf in zip(("dqs", "dks", "dvs", "dqm", "dkm", "dvm"), leaves):
        rec[n] = leaf.grad.numpy().astype(np.float32)
    return rec


def main():
    arrays = {}
    for name, *args in CASES:
        for k, v in make_case(*args).items():
            arrays[f"{name}/{k}"] = v
    path = os.path.join(HERE, "mpattn_cases.npz")
    np.savez_compressed(path, **arrays)
    print(f"wrote {path} ({os.path.getsize(path)} bytes, {len(CASES)} cases)")


if __name__ == "__main__":
    main()
