"""Golden fixtures (tests/golden/mpattn_cases.npz, written by
tests/golden/make_golden.py from the SDPA construction in tests/indep.py).

CPU: the oracle reproduces every fixture (forward, LSE and all six gradients)
to float32 storage precision. GPU: the kernels reproduce them within the bf16
tolerance 2e-2 abs + 1e-2 rel (the fixture inputs are bf16-exact)."""
import os

import numpy as np
import pytest
import torch

from oracle import mpattn_oracle as orc

PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "mpattn_cases.npz")
GRADS = ("dqs", "dks", "dvs", "dqm", "dkm", "dvm")


def load_cases():
    z = np.load(PATH)  # plain arrays only (allow_pickle stays False)
    cases = {}
    for key in z.files:
        name, field = key.split("/")
        cases.setdefault(name, {})[field] = z[key]
    return cases


CASES = load_cases()


def test_fixture_inventory():
    assert len(CASES) == 4
    for c in CASES.values():
        assert c["qs"].dtype == np.float32 and c["chain_ids"].dtype == np.int32
        bf = torch.from_numpy(c["qs"]).to(torch.bfloat16).float().numpy()
        assert np.array_equal(bf, c["qs"])  # inputs are bf16-exact


@pytest.mark.parametrize("name", sorted(CASES))
def test_oracle_reproduces_fixture(name):
    c = CASES[name]
    xs = [c[k].astype(np.float64) for k in ("qs", "ks", "vs", "qm", "km", "vm")]
    kw = dict(chain_ids=c["chain_ids"], key_pad=c["key_pad"], rope=bool(c["rope"]),
              scale=float(c["scale"]))
    out, lse = orc.mpattn_forward(*xs, **kw)
    np.testing.assert_allclose(out, c["out"], rtol=1e-6, atol=1e-7)
    np.testing.assert_allclose(lse, c["lse"], rtol=1e-6, atol=1e-6)
    grads = orc.mpattn_backward(*xs, c["go"].astype(np.float64), **kw)
    for n, g in zip(GRADS, grads):
        np.testing.assert_allclose(g, c[n], rtol=1e-6, atol=1e-7, err_msg=n)


@pytest.mark.gpu
@pytest.mark.parametrize("name", sorted(CASES))
def test_kernels_reproduce_fixture(name):
    import mint_plus_amd as m
    print(f"[golden gpu] {name}", flush=True)
    c = CASES[name]
    dev = "cuda:0"
    xs = [torch.from_numpy(c[k]).to(torch.bfloat16).to(dev)
          for k in ("qs", "ks", "vs", "qm", "km", "vm")]
    kw = dict(chain_ids=torch.from_numpy(c["chain_ids"]).to(dev),
              key_padding_mask=torch.from_numpy(c["key_pad"]).to(dev), rope=bool(c["rope"]),
              scale=float(c["scale"]))
    out = m.fused_multi_pathway_attention(*xs, None, training=False, **kw)
    grads = m.fused_multi_pathway_attention_bwd(*xs, None,
                                                torch.from_numpy(c["go"]).to(torch.bfloat16).to(dev),
                                                **kw)
    torch.cuda.synchronize()
    for n, got in zip(("out",) + GRADS, (out,) + tuple(grads)):
        g = got.float().cpu().numpy()
        ref = c[n]
        err = np.abs(g - ref)
        assert (err <= 2e-2 + 1e-2 * np.abs(ref)).all(), f"{name} {n}: max err {err.max():.4g}"
