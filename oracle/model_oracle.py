"""CPU oracle of the MINT transformer layer and model -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s
``cpu_baseline`` leg may use it; the product (``mint_plus_amd``) never does.

Float64 torch on the CPU, from a state dict with the reference's parameter
names (either separate ``q_proj/k_proj/v_proj`` or ``fused_qkv``):

* ``layer_forward`` -- ``TransformerLayer_MINT(_plus).forward``
  (``mint_plus/models/modules.py:156-197``, ``modules_plus.py:203-237``):
  pre-norm residual attention block, then pre-norm residual feed-forward
  (``fc2(gelu(fc1(x)))``, ``modules.py:323-336``). The multimer attention is
  the eager combine of ``modules.py:94-154`` computed by
  ``mpattn_oracle.mpattn_forward`` on the projected Q/K/V (scale
  ``head_dim**-0.5``, RoPE on the self pathway, key padding), followed by
  ``self_attn.out_proj``. Without ``multimer`` it is plain self-attention
  (``attention.py:172-270``), i.e. the same op with one chain.
* ``mint_forward`` -- ``MINT.forward`` in eval (``esm2.py:77-145``):
  embedding, padded rows zeroed, the layers in (T, B, E), final LayerNorm
  (the per-residue embeddings), tied LM head (``modules.py:339-369``).

Pinned by (``tests/test_model_oracle.py``): the layer with zeroed
``out_proj`` and ``fc2`` is the identity; a one-chain multimer layer equals
the standard layer built from the self pathway; the attention block equals
``torch.nn.functional.scaled_dot_product_attention`` (a library routine) for
one chain; key padding and padded rows leave valid positions unchanged.
LayerNorm, Linear and GELU are torch library routines.
"""
import numpy as np
import torch
import torch.nn.functional as F

from . import mpattn_oracle as orc


def _t(x):
    return x.detach().to(device="cpu", dtype=torch.float64)


def _linear(sd, name, x):
    b = sd.get(name + ".bias")
    return F.linear(x, _t(sd[name + ".weight"]), None if b is None else _t(b))


def _norm(sd, name, x, eps):
    w = _t(sd[name + ".weight"])
    if name + ".bias" in sd:
        return F.layer_norm(x, (x.shape[-1],), w, _t(sd[name + ".bias"]), eps=1e-5)
    return F.rms_norm(x, (x.shape[-1],), w, eps=eps)


def _qkv(sd, prefix, x):
    if prefix + ".fused_qkv.weight" in sd:
        return _linear(sd, prefix + ".fused_qkv", x).chunk(3, dim=-1)
    return tuple(_linear(sd, f"{prefix}.{n}_proj", x) for n in ("q", "k", "v"))


def _heads(t, H):
    T, B, E = t.shape
    return t.reshape(T, B, H, E // H).permute(1, 2, 0, 3).numpy()


def attention_block(sd, prefix, x, chain_ids, key_pad, heads, multimer=True, rope=True):
    """Attention sub-block output (before the residual add), (T, B, E)."""
    T, B, E = x.shape
    D = E // heads
    qs, ks, vs = (_heads(t, heads) for t in _qkv(sd, prefix + ".self_attn", x))
    if multimer:
        qm, km, vm = (_heads(t, heads) for t in _qkv(sd, prefix + ".multimer_attn", x))
        cid = np.asarray(chain_ids)
    else:
        qm, km, vm = qs, ks, vs
        cid = np.zeros((B, T), np.int32)
    out, _ = orc.mpattn_forward(qs, ks, vs, qm, km, vm, chain_ids=cid, key_pad=key_pad,
                                rope=rope, scale=D ** -0.5)
    out = torch.from_numpy(out).permute(2, 0, 1, 3).reshape(T, B, E)
    return _linear(sd, prefix + ".self_attn.out_proj", out)


def layer_forward(sd, prefix, x, chain_ids, key_pad, heads, multimer=True, rope=True,
                  norm_eps=None):
    """One layer, x (T, B, E) float64 -> (T, B, E)."""
    x = _t(x)
    h = _norm(sd, prefix + ".self_attn_layer_norm", x, norm_eps)
    x = x + attention_block(sd, prefix, h, chain_ids, key_pad, heads, multimer, rope)
    h = _norm(sd, prefix + ".final_layer_norm", x, norm_eps)
    h = _linear(sd, prefix + ".feed_forward.fc2", F.gelu(_linear(sd, prefix + ".feed_forward.fc1", h)))
    return x + h


def mint_forward(sd, tokens, chain_ids, num_layers, heads, padding_idx=1, multimer=True,
                 norm_eps=None):
    """``MINT.forward`` in eval; returns (logits (B, T, V), embeddings (B, T, E))."""
    tokens = torch.as_tensor(tokens).cpu()
    pad = tokens.eq(padding_idx)
    x = _t(sd["embed_tokens.weight"])[tokens]
    x = x * (1 - pad.unsqueeze(-1).double())
    x = x.transpose(0, 1)
    cid = np.asarray(torch.as_tensor(chain_ids).cpu())
    kp = pad.numpy()
    for i in range(num_layers):
        x = layer_forward(sd, f"layers.{i}", x, cid, kp, heads, multimer=multimer,
                          norm_eps=norm_eps)
    emb = _norm(sd, "emb_layer_norm_after", x, norm_eps).transpose(0, 1)
    h = _norm(sd, "lm_head.layer_norm", F.gelu(_linear(sd, "lm_head.dense", emb)), norm_eps)
    logits = F.linear(h, _t(sd["embed_tokens.weight"])) + _t(sd["lm_head.bias"])
    return logits, emb
