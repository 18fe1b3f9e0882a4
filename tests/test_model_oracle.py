"""Pins of the layer / model oracle (``oracle/model_oracle.py``), CPU only."""
import numpy as np
import torch
import torch.nn.functional as F

from conftest import two_chain_ids
from oracle import model_oracle as mo


def _layer_sd(rng, E, F_, prefix="l", fused=False, multimer=True):
    sd = {}
    r = lambda *s: torch.from_numpy(rng.standard_normal(s) * 0.2)
    for p in (["self_attn"] + (["multimer_attn"] if multimer else [])):
        if fused:
            sd[f"{prefix}.{p}.fused_qkv.weight"] = r(3 * E, E)
            sd[f"{prefix}.{p}.fused_qkv.bias"] = r(3 * E)
        else:
            for n in "qkv":
                sd[f"{prefix}.{p}.{n}_proj.weight"] = r(E, E)
                sd[f"{prefix}.{p}.{n}_proj.bias"] = r(E)
    sd[f"{prefix}.self_attn.out_proj.weight"] = r(E, E)
    sd[f"{prefix}.self_attn.out_proj.bias"] = r(E)
    for n in ("self_attn_layer_norm", "final_layer_norm"):
        sd[f"{prefix}.{n}.weight"] = 1 + r(E)
        sd[f"{prefix}.{n}.bias"] = r(E)
    sd[f"{prefix}.feed_forward.fc1.weight"] = r(F_, E)
    sd[f"{prefix}.feed_forward.fc1.bias"] = r(F_)
    sd[f"{prefix}.feed_forward.fc2.weight"] = r(E, F_)
    sd[f"{prefix}.feed_forward.fc2.bias"] = r(E)
    return sd


def test_layer_identity_when_branches_zeroed():
    rng = np.random.default_rng(0)
    T, B, E, H = 20, 2, 32, 4
    sd = _layer_sd(rng, E, 64)
    for n in ("self_attn.out_proj", "feed_forward.fc2"):
        sd[f"l.{n}.weight"].zero_()
        sd[f"l.{n}.bias"].zero_()
    x = torch.from_numpy(rng.standard_normal((T, B, E)))
    y = mo.layer_forward(sd, "l", x, two_chain_ids(rng, B, T), None, H)
    torch.testing.assert_close(y, x, rtol=0, atol=0)


def test_one_chain_multimer_layer_equals_standard_layer():
    rng = np.random.default_rng(1)
    T, B, E, H = 24, 2, 32, 4
    sd = _layer_sd(rng, E, 64)
    x = torch.from_numpy(rng.standard_normal((T, B, E)))
    kp = np.zeros((B, T), bool)
    kp[1, -5:] = True
    a = mo.layer_forward(sd, "l", x, np.zeros((B, T), np.int32), kp, H, multimer=True)
    b = mo.layer_forward(sd, "l", x, None, kp, H, multimer=False)
    torch.testing.assert_close(a, b, rtol=0, atol=1e-12)


def test_attention_block_single_chain_is_sdpa():
    """One chain: the attention block is RoPE'd SDPA over the self pathway
    with padded keys masked, then out_proj."""
    rng = np.random.default_rng(2)
    T, B, E, H = 30, 2, 48, 3
    D = E // H
    sd = _layer_sd(rng, E, 64, fused=True)
    x = torch.from_numpy(rng.standard_normal((T, B, E)))
    kp = np.zeros((B, T), bool)
    kp[0, -7:] = True
    got = mo.attention_block(sd, "l", x, np.zeros((B, T), np.int32), kp, H)
    q, k, v = F.linear(x, sd["l.self_attn.fused_qkv.weight"],
                       sd["l.self_attn.fused_qkv.bias"]).chunk(3, -1)
    heads = lambda t: t.reshape(T, B, H, D).permute(1, 2, 0, 3)
    pos = torch.arange(T, dtype=torch.float32)
    inv = (1.0 / 10000 ** (torch.arange(0, D, 2, dtype=torch.float64) / D)).float()
    ang = (pos[:, None] * inv[None, :]).double()

    def rope(t):  # complex-multiplication form
        z = torch.complex(t[..., :D // 2], t[..., D // 2:]) * torch.polar(torch.ones_like(ang), ang)
        return torch.cat([z.real, z.imag], -1)

    mask = ~torch.as_tensor(kp)[:, None, None, :]
    o = F.scaled_dot_product_attention(rope(heads(q)), rope(heads(k)), heads(v), attn_mask=mask)
    ref = F.linear(o.permute(2, 0, 1, 3).reshape(T, B, E), sd["l.self_attn.out_proj.weight"],
                   sd["l.self_attn.out_proj.bias"])
    torch.testing.assert_close(got, ref, rtol=0, atol=1e-11)


def test_fused_and_separate_qkv_agree():
    rng = np.random.default_rng(3)
    T, B, E, H = 16, 2, 32, 4
    sd = _layer_sd(rng, E, 64, fused=False)
    fused = {k: v for k, v in sd.items() if "_proj" not in k or "out_proj" in k}
    for p in ("self_attn", "multimer_attn"):
        for s in ("weight", "bias"):
            fused[f"l.{p}.fused_qkv.{s}"] = torch.cat([sd[f"l.{p}.{n}_proj.{s}"] for n in "qkv"])
    x = torch.from_numpy(rng.standard_normal((T, B, E)))
    cid = two_chain_ids(rng, B, T)
    a = mo.layer_forward(sd, "l", x, cid, None, H)
    b = mo.layer_forward(fused, "l", x, cid, None, H)
    torch.testing.assert_close(a, b, rtol=0, atol=1e-12)


def test_model_padding_rows_do_not_affect_valid_positions():
    """Appending padded tokens leaves the embeddings of real tokens unchanged."""
    rng = np.random.default_rng(4)
    E, H, V, nl = 32, 4, 33, 2
    sd = {}
    for i in range(nl):
        sd.update(_layer_sd(rng, E, 64, prefix=f"layers.{i}"))
    sd["embed_tokens.weight"] = torch.from_numpy(rng.standard_normal((V, E)))
    for n in ("emb_layer_norm_after", "lm_head.layer_norm"):
        sd[f"{n}.weight"] = torch.ones(E, dtype=torch.float64)
        sd[f"{n}.bias"] = torch.zeros(E, dtype=torch.float64)
    sd["lm_head.dense.weight"] = torch.from_numpy(rng.standard_normal((E, E)) * 0.1)
    sd["lm_head.dense.bias"] = torch.zeros(E, dtype=torch.float64)
    sd["lm_head.bias"] = torch.zeros(V, dtype=torch.float64)
    tok = torch.from_numpy(rng.integers(4, 24, size=(1, 20)))
    cid = torch.zeros(1, 20, dtype=torch.int32)
    cid[0, 12:] = 1
    _, e1 = mo.mint_forward(sd, tok, cid, nl, H)
    tok2 = torch.cat([tok, torch.ones(1, 6, dtype=tok.dtype)], 1)
    cid2 = torch.cat([cid, torch.ones(1, 6, dtype=cid.dtype)], 1)
    _, e2 = mo.mint_forward(sd, tok2, cid2, nl, H)
    torch.testing.assert_close(e2[:, :20], e1, rtol=0, atol=1e-12)
