"""MINT model (ESM-2 trunk with the multi-pathway attention), with the
interface of ``mint_plus/models/esm2.py:14-180``.

``MINT(num_layers, embed_dim, attention_heads, alphabet, token_dropout,
use_multimer, use_rmsnorm, use_erf_gelu)``; ``forward(tokens, chain_ids=None,
repr_layers=[])`` returns ``{"logits", "representations"}`` where
``representations[num_layers]`` is the final-LayerNorm output (the
per-residue embeddings). Parameter names follow the reference, so its state
dicts load unchanged (``load_pretrained_weights`` remaps HF-style keys as
esm2.py:214-256 does).

Differences from the reference on purpose: the (B, T, T) chain mask is not
built up front (layers take ``chain_ids`` and build it only for the
materialised pipeline); layers are checkpointed only while training with
autograd on; ``load_pretrained_weights`` loads with ``weights_only=True``.
"""
from typing import Dict, List, Optional, Union

import torch
import torch.nn as nn
from torch.utils.checkpoint import checkpoint

from .alphabet import Alphabet
from .modules import ESM1bLayerNorm, RobertaLMHead, TransformerLayer_MINT

# Model shapes of the ESM-2 family (the reference's registry,
# mint_plus/models/__init__.py:1-101), plus the 3B attention shape the
# benchmarks use (40 heads of 64).
MODEL_REGISTRY = {
    "8M": dict(num_layers=6, embed_dim=320, attention_heads=20),
    "35M": dict(num_layers=12, embed_dim=480, attention_heads=20),
    "150M": dict(num_layers=30, embed_dim=640, attention_heads=20),
    "650M": dict(num_layers=33, embed_dim=1280, attention_heads=20),
    "3B": dict(num_layers=36, embed_dim=1792, attention_heads=16),
    "15B": dict(num_layers=48, embed_dim=5120, attention_heads=20),
    "3B-shape": dict(num_layers=36, embed_dim=2560, attention_heads=40),
}


class MINT(nn.Module):
    def __init__(self, num_layers: int = 33, embed_dim: int = 1280, attention_heads: int = 20,
                 alphabet: Union[Alphabet, str] = "ESM-1b", token_dropout: bool = True,
                 use_multimer: bool = True, use_rmsnorm: bool = False,
                 use_erf_gelu: bool = False, fp8: bool = False):
        super().__init__()
        self.num_layers = num_layers
        self.embed_dim = embed_dim
        self.attention_heads = attention_heads
        if not isinstance(alphabet, Alphabet):
            alphabet = Alphabet.from_architecture(alphabet)
        self.alphabet = alphabet
        self.alphabet_size = len(alphabet)
        self.padding_idx = alphabet.padding_idx
        self.mask_idx = alphabet.mask_idx
        self.cls_idx = alphabet.cls_idx
        self.eos_idx = alphabet.eos_idx
        self.prepend_bos = alphabet.prepend_bos
        self.append_eos = alphabet.append_eos
        self.token_dropout = token_dropout
        self.use_multimer = use_multimer
        self.use_rmsnorm = use_rmsnorm
        self.use_erf_gelu = use_erf_gelu
        self._init_submodules()

    def _init_submodules(self):
        self.embed_tokens = nn.Embedding(self.alphabet_size, self.embed_dim,
                                         padding_idx=self.padding_idx)
        self.layers = nn.ModuleList([
            TransformerLayer_MINT(self.embed_dim, 4 * self.embed_dim, self.attention_heads,
                                  use_rotary_embeddings=True, use_multimer=self.use_multimer,
                                  use_rmsnorm=self.use_rmsnorm, use_erf_gelu=self.use_erf_gelu)
            for _ in range(self.num_layers)])
        self.emb_layer_norm_after = (nn.RMSNorm(self.embed_dim) if self.use_rmsnorm
                                     else ESM1bLayerNorm(self.embed_dim))
        self.lm_head = RobertaLMHead(self.embed_dim, self.alphabet_size, self.embed_tokens.weight)

    def forward(self, tokens: torch.Tensor, chain_ids: Optional[torch.Tensor] = None,
                repr_layers: List[int] = []) -> Dict[str, torch.Tensor]:
        """esm2.py:77-145: embed (token dropout while training), zero padded
        rows, run the layers in (T, B, E), final norm, LM head."""
        assert tokens.ndim == 2
        padding_mask = tokens.eq(self.padding_idx)
        if chain_ids is None:
            chain_ids = torch.zeros_like(tokens)
        x = self.embed_tokens(tokens)
        if self.token_dropout and self.training:
            masked = tokens == self.mask_idx
            x = x.masked_fill(masked.unsqueeze(-1), 0.0)
            ratio_train = 0.15 * 0.8
            lengths = (~padding_mask).sum(-1)
            ratio_obs = masked.sum(-1).to(x.dtype) / lengths
            x = x * (1 - ratio_train) / (1 - ratio_obs)[:, None, None]
        x = x * (1 - padding_mask.unsqueeze(-1).type_as(x))
        repr_layers = set(repr_layers)
        hidden = {}
        if 0 in repr_layers:
            hidden[0] = x
        x = x.transpose(0, 1)
        ckpt = self.training and torch.is_grad_enabled()
        if ckpt and not x.requires_grad:
            x.requires_grad_(True)
        for i, layer in enumerate(self.layers):
            kw = dict(self_attn_padding_mask=padding_mask, self_attn_mask=None, chain_ids=chain_ids)
            if ckpt:
                x, _ = checkpoint(layer, x, use_reentrant=False, **kw)
            else:
                x, _ = layer(x, **kw)
            if (i + 1) in repr_layers:
                hidden[i + 1] = x.transpose(0, 1)
        x = self.emb_layer_norm_after(x).transpose(0, 1)
        if self.num_layers in repr_layers:
            hidden[self.num_layers] = x
        return {"logits": self.lm_head(x), "representations": hidden}

    @classmethod
    def from_config(cls, model_size: str, fp8: bool = False, use_erf_gelu: bool = False):
        """Model of a registry size (esm2.py:147-170)."""
        if model_size not in MODEL_REGISTRY:
            raise ValueError(f"Unknown model size: {model_size}. Available: {list(MODEL_REGISTRY)}")
        return cls(**MODEL_REGISTRY[model_size], fp8=fp8, use_erf_gelu=use_erf_gelu)

    def load_pretrained_weights(self, checkpoint_path: str, strict: bool = False,
                                dtype: torch.dtype = torch.float32, alternating: bool = False):
        """Load a local checkpoint (esm2.py:172-211); tensors only."""
        ckpt = torch.load(checkpoint_path, map_location="cpu", weights_only=True)
        sd = ckpt.get("model", ckpt.get("state_dict", ckpt)) if isinstance(ckpt, dict) else ckpt
        sd = self._upgrade_state_dict(sd)
        if dtype != torch.float32:
            sd = {k: v.to(dtype=dtype) for k, v in sd.items()}
        if "lm_head.decoder.weight" in sd and "lm_head.weight" not in sd:
            sd["lm_head.weight"] = sd["lm_head.decoder.weight"]
        return self.load_state_dict(sd, strict=strict)

    # HF-style names -> this module's names (esm2.py:214-256).
    _LAYER_KEYS = (("attention.self.query", "self_attn.q_proj"),
                   ("attention.self.key", "self_attn.k_proj"),
                   ("attention.self.value", "self_attn.v_proj"),
                   ("attention.output.dense", "self_attn.out_proj"),
                   ("attention.Layer", "self_attn_layer_norm"),
                   ("LayerNorm", "final_layer_norm"),
                   ("intermediate", "feed_forward.fc1"),
                   ("output", "feed_forward.fc2"))

    def _upgrade_state_dict(self, state_dict: Dict[str, torch.Tensor]) -> Dict[str, torch.Tensor]:
        out = {}
        for key, value in state_dict.items():
            k = key
            for prefix in ("esm.", "encoder."):
                if k.startswith(prefix):
                    k = k[len(prefix):]
            parts = k.split(".")
            if len(parts) > 1 and parts[0] in ("layer", "layers") and parts[1].isdigit():
                for pat, name in self._LAYER_KEYS:
                    if pat in k:
                        k = f"layers.{parts[1]}.{name}.{parts[-1]}"
                        break
            elif "word_embeddings.weight" in k:
                k = "embed_tokens.weight"
            elif "lm_head.decoder.weight" in k:
                k = "lm_head.weight"
            out[k] = value
        return out
