"""mpattn_fwd_noalloc (the forward with the library's static device scratch
instead of a caller workspace) against mpattn_fwd, through the C ABI.

Both run the same kernels, so the outputs and LSE must be bitwise equal.
Two calls in a row, the second smaller, check that the scratch's previous
contents do not leak into a later call.
"""
import pytest
import torch

import parity as P

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def _case(B, H, L, D, seed, nchains, dense):
    xs, cid, kp = P.fwd_inputs(B, H, L, D, torch.bfloat16, seed=seed, nchains=nchains)
    g = [x.to(DEV) for x in xs]
    kw = dict(key_padding_mask=torch.from_numpy(kp).to(DEV), rope=True, scale=D ** -0.5)
    if dense:
        c = torch.from_numpy(cid)
        kw["chain_mask"] = (c[:, :, None] != c[:, None, :]).to(DEV)
    else:
        kw["chain_ids"] = torch.from_numpy(cid).to(DEV)
    return g, kw


@pytest.mark.parametrize("first,second", [
    ((4, 8, 1000, 32, 11, 2, False), (2, 4, 300, 32, 12, 3, False)),
    ((2, 8, 777, 64, 13, 3, True), (1, 2, 130, 16, 14, 2, True)),
])
def test_fwd_noalloc_matches_fwd(first, second):
    from mint_plus_amd import _lib
    for case in (first, second):
        print(f"[noalloc] B,H,L,D={case[:4]} chains={case[5]} dense={case[6]}", flush=True)
        g, kw = _case(*case)
        B, H, L, D = g[0].shape
        ref, ref_lse = _lib.mpattn_fwd(*g, need_lse=True, **kw)
        out = torch.empty_like(g[0])
        lse = torch.empty((B, H, L), dtype=torch.float32, device=DEV)
        _lib.mpattn_fwd(*g, out=out, lse=lse, need_lse=True, noalloc=True, **kw)
        torch.cuda.synchronize()
        assert torch.equal(out, ref)
        assert torch.equal(lse, ref_lse)
