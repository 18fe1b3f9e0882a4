"""Module- and model-level parity on the GPU: ``TransformerLayer_MINT(_plus)``
and ``MINT`` running the HIP paths (fused multi-pathway kernel, or the
materialised pipeline with the combine kernel) against the float64 layer /
model oracle (``oracle/model_oracle.py``) built from the same weights.

Tolerances: fp32 max-abs 1e-4; bf16 |gpu - ref| <= 2e-2 + 1e-2 |ref| (the
oracle sees the bf16-rounded weights and inputs, so the difference is the
bf16 arithmetic of the layer).
"""
import numpy as np
import pytest
import torch

from conftest import two_chain_ids
from oracle import model_oracle as mo

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _mods():
    from mint_plus_amd import modules, modules_plus, esm2
    return modules, modules_plus, esm2


def _inputs(T, B, E, seed, dtype, pad=True):
    rng = np.random.default_rng(seed)
    x = torch.from_numpy(rng.standard_normal((T, B, E)).astype(np.float32)).to(dtype)
    cid = torch.from_numpy(two_chain_ids(rng, B, T))
    kp = torch.zeros(B, T, dtype=torch.bool)
    if pad:
        kp[1, T - T // 8:] = True
    return x, cid, kp


def _oracle_layer(layer, x, cid, kp, H):
    sd = {"l." + k: v for k, v in layer.state_dict().items()}
    eps = torch.finfo(next(layer.parameters()).dtype).eps
    return mo.layer_forward(sd, "l", x.double(), cid.numpy(), kp.numpy(), H, norm_eps=eps)


def _check(got, ref, dtype, what, valid=None):
    got = got.double().cpu()
    if valid is not None:
        got, ref = got[valid], ref[valid]
    err = (got - ref).abs()
    if dtype == torch.float32:
        assert err.max().item() <= 1e-4, f"{what}: max err {err.max().item():.3g}"
    else:
        bad = err > 2e-2 + 1e-2 * ref.abs()
        assert not bad.any(), f"{what}: {int(bad.sum())} out of tolerance, max {err.max().item():.3g}"


@pytest.mark.parametrize("fused", [True, False])
@pytest.mark.parametrize("plus", [False, True])
def test_layer_fp32_8m_width(fused, plus):
    """E=320, H=20 (D=16), fp32: fused kernel path and materialised combine
    path, base and _plus layers."""
    print(f"[layer fp32] fused={fused} plus={plus}", flush=True)
    M, MP, _ = _mods()
    torch.manual_seed(11)
    T, B, E, H = 150, 2, 320, 20
    layer = M.TransformerLayer_MINT(E, 4 * E, H, use_multimer=True)
    if plus:
        holder = torch.nn.Module()
        holder.layers = torch.nn.ModuleList([layer])
        MP.build_mint_plus(holder)
        layer = holder.layers[0]
    layer = layer.to(DEV).eval()
    layer._use_fused_multi_pathway = fused
    x, cid, kp = _inputs(T, B, E, 12, torch.float32)
    with torch.no_grad():
        y, attn = layer(x.to(DEV), self_attn_padding_mask=kp.to(DEV), chain_ids=cid.to(DEV))
    torch.cuda.synchronize()
    assert attn is None
    _check(y, _oracle_layer(layer, x, cid, kp, H), torch.float32, f"fused={fused} plus={plus}")


@pytest.mark.parametrize("E,H", [(640, 20), (480, 20), (1280, 20)])
def test_layer_bf16_fused(E, H):
    """bf16 layers of the 150M (D=32), 35M (D=24) and 650M (D=64) widths,
    fused path, chain selection from the dense (B, T, T) mask."""
    print(f"[layer bf16] E={E} H={H}", flush=True)
    M, _, _ = _mods()
    torch.manual_seed(13)
    T, B = 200, 2
    layer = M.TransformerLayer_MINT(E, 4 * E, H, use_multimer=True).to(DEV, torch.bfloat16).eval()
    layer._use_fused_multi_pathway = True
    x, cid, kp = _inputs(T, B, E, 14, torch.bfloat16)
    mask = (cid[:, :, None] != cid[:, None, :]).to(DEV)
    with torch.no_grad():
        y, _ = layer(x.to(DEV), self_attn_mask=mask, self_attn_padding_mask=kp.to(DEV))
    torch.cuda.synchronize()
    _check(y, _oracle_layer(layer, x, cid, kp, H), torch.bfloat16, f"bf16 E={E}")


@pytest.mark.parametrize("fused,dtype", [(True, torch.bfloat16), (False, torch.float32),
                                         (True, torch.float32)])
def test_layer_backward_matches_eager(fused, dtype, monkeypatch):
    """Training step through the HIP path: input and parameter gradients of
    the GPU layer against torch autograd of the same layer's eager path in
    float64 on the CPU (itself pinned to the layer oracle on the CPU).
    bf16 layer (fused kernels): bound 2e-2 of each gradient's max; fp32
    layer (the 8M width; fused fp32 forward and backward, or the combine
    kernels): bound 1e-4 of each max. With the fused flag the combine
    kernels must not run."""
    print(f"[layer bwd] fused={fused} dtype={dtype}", flush=True)
    M, _, _ = _mods()
    if fused:
        def no_combine(*a, **k):
            raise AssertionError("combine kernels called on the fused path")
        monkeypatch.setattr(M, "differentiable_multimer_combine", no_combine)
        monkeypatch.setattr(M, "fused_multimer_combine", no_combine)
    torch.manual_seed(15)
    T, B, E, H = 130, 2, 320, 20
    ref_layer = M.TransformerLayer_MINT(E, 2 * E, H, use_multimer=True).double().train()
    gpu_layer = M.TransformerLayer_MINT(E, 2 * E, H, use_multimer=True).to(DEV, dtype).train()
    gpu_layer.load_state_dict(ref_layer.state_dict())
    ref_layer.load_state_dict(gpu_layer.state_dict())  # reference sees the rounded weights
    gpu_layer._use_fused_multi_pathway = fused
    x, cid, kp = _inputs(T, B, E, 16, dtype)
    g = torch.randn(T, B, E, generator=torch.Generator().manual_seed(1)).to(dtype)

    def run(layer, dev, path):
        layer.zero_grad(set_to_none=True)
        xi = x.to(dev, next(layer.parameters()).dtype).requires_grad_(True)
        c, k = cid.to(dev), kp.to(dev)
        h = layer.self_attn_layer_norm(xi)
        if path == "eager":
            a, _ = layer._multimer_attention(h, None, k, chain_ids=c)
        else:
            a, _ = layer._multimer_attention_plus(h, None, k, chain_ids=c)
        y = xi + a
        y = y + layer.feed_forward(layer.final_layer_norm(y))
        (y * g.to(dev, y.dtype)).sum().backward()
        out = {"x": xi.grad.double().cpu()}
        out.update({n: p.grad.double().cpu() for n, p in layer.named_parameters()
                    if p.grad is not None})
        return out

    got = run(gpu_layer, DEV, "hip")
    ref = run(ref_layer, "cpu", "eager")
    assert set(got) == set(ref)
    bound = 2e-2 if dtype == torch.bfloat16 else 1e-4
    for n in ref:
        scale = ref[n].abs().max().item()
        err = (got[n] - ref[n]).abs().max().item()
        assert err <= bound * max(scale, 1e-6), f"{n}: err {err:.3g} (scale {scale:.3g})"


def _config0_batch(seed=0, B=4):
    """The 8M configuration's input: two chains A ~ U[60,200], B ~ U[40,160]
    tokens over the 20 standard amino acids, each wrapped <cls> ... <eos>,
    laid out [A][B][pad] and padded to the batch max."""
    from mint_plus_amd.alphabet import Alphabet
    a = Alphabet.from_architecture("ESM-1b")
    rng = np.random.default_rng(seed)
    la = rng.integers(60, 201, size=B)
    lb = rng.integers(40, 161, size=B)
    L = int((la + lb).max()) + 4
    tok = np.full((B, L), a.padding_idx, np.int64)
    cid = np.ones((B, L), np.int64)
    for b in range(B):
        ca = [a.cls_idx] + list(rng.integers(4, 24, size=la[b])) + [a.eos_idx]
        cb = [a.cls_idx] + list(rng.integers(4, 24, size=lb[b])) + [a.eos_idx]
        tok[b, :len(ca) + len(cb)] = ca + cb
        cid[b, :len(ca)] = 0
    return torch.from_numpy(tok), torch.from_numpy(cid)


@pytest.mark.parametrize("fused", [True, False])
def test_mint_8m_embeddings_fp32(fused):
    """Config 0: the 8M MINT model in fp32 (random init from a seed), B=4
    two-chain complexes; per-residue embeddings (final LayerNorm output) at
    valid positions against the model oracle, max-abs 1e-4."""
    print(f"[8M model] fused={fused}", flush=True)
    M, _, E2 = _mods()
    torch.manual_seed(8)
    model = E2.MINT.from_config("8M").to(DEV).eval()
    if fused:
        M.enable_fused_multi_pathway(model)
    tok, cid = _config0_batch()
    with torch.no_grad():
        res = model(tok.to(DEV), chain_ids=cid.to(DEV), repr_layers=[6])
    torch.cuda.synchronize()
    emb = res["representations"][6]
    sd = {k: v for k, v in model.state_dict().items()}
    logits_ref, emb_ref = mo.mint_forward(sd, tok, cid, 6, 20)
    valid = tok != 1
    _check(emb, emb_ref, torch.float32, "8M embeddings", valid=valid)
    _check(res["logits"], logits_ref, torch.float32, "8M logits", valid=valid)


def test_mint_650m_width_bf16_two_layers():
    """Two bf16 layers of the 650M width (E=1280, H=20, D=64) inside the MINT
    trunk, fused path, against the model oracle."""
    print("[650M-width model]", flush=True)
    M, _, E2 = _mods()
    torch.manual_seed(65)
    model = E2.MINT(num_layers=2, embed_dim=1280, attention_heads=20).to(DEV, torch.bfloat16).eval()
    M.enable_fused_multi_pathway(model)
    tok, cid = _config0_batch(seed=3, B=2)
    with torch.no_grad():
        res = model(tok.to(DEV), chain_ids=cid.to(DEV), repr_layers=[2])
    torch.cuda.synchronize()
    sd = {k: v for k, v in model.state_dict().items()}
    _, emb_ref = mo.mint_forward(sd, tok, cid, 2, 20, norm_eps=torch.finfo(torch.bfloat16).eps)
    _check(res["representations"][2], emb_ref, torch.bfloat16, "650M-width", valid=tok != 1)


def test_650m_layers_bf16_long_rows():
    """Three bf16 TransformerLayer_MINT layers of the 650M width (E=1280,
    H=20, D=64, FFN 5120) at the benchmark's row length: B=2 two-chain
    complexes of 1006 and 951 tokens (chains >= 64), fused path. Each layer
    is checked on its own input (the previous GPU layer's output) against
    the layer oracle in float64 on the same bf16 weights, so bf16 errors of
    earlier layers do not compound: per element 2e-2 + 1e-2 |ref| at valid
    rows, and relative Frobenius error <= 1e-2."""
    print("[650M-width layers, L=1006]", flush=True)
    M, _, _ = _mods()
    torch.manual_seed(66)
    T, B, E, H = 1006, 2, 1280, 20
    rng = np.random.default_rng(1006)
    cid = torch.ones(B, T, dtype=torch.int32)
    kp = torch.zeros(B, T, dtype=torch.bool)
    for b, n in enumerate((1006, 951)):
        cid[b, :int(rng.integers(64, n - 64 + 1))] = 0
        kp[b, n:] = True
    x = torch.from_numpy(rng.standard_normal((T, B, E)).astype(np.float32)).to(torch.bfloat16)
    valid = ~kp.transpose(0, 1)  # (T, B)
    for i in range(3):
        layer = M.TransformerLayer_MINT(E, 4 * E, H, use_multimer=True).to(DEV, torch.bfloat16).eval()
        layer._use_fused_multi_pathway = True
        with torch.no_grad():
            y, _ = layer(x.to(DEV), self_attn_padding_mask=kp.to(DEV), chain_ids=cid.to(DEV))
        torch.cuda.synchronize()
        ref = _oracle_layer(layer, x, cid, kp, H)
        _check(y, ref, torch.bfloat16, f"650M-width layer {i} L=1006", valid=valid)
        g, r = y.double().cpu()[valid], ref[valid]
        rel = float((g - r).norm() / r.norm())
        assert rel <= 1e-2, (i, rel)
        x = y.cpu()
