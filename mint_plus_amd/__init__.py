"""MI355X (gfx950) multi-pathway attention for MINT+.

The op behind ``mint_plus/models/kernels`` and ``MultimerAttention`` /
``TransformerLayer_MINT(_plus)``: per (query, key) pair it takes the RoPE
self-attention logit on the same chain and the multimer logit across chains,
applies key padding and one softmax over all keys, and returns
``P_intra V_self + P_inter V_multi``. Hand-written HIP kernels behind a C ABI
(include/mpattn.h, libmpattn.so) do the work.
"""
from . import _lib
from ._lib import MpattnError, MpattnUnsupported, load_library, rope_tables
from .kernels import (differentiable_multi_pathway_attention, differentiable_multimer_combine,
                      fused_multi_pathway_attention, fused_multi_pathway_attention_bwd,
                      fused_multi_pathway_attention_fp16, fused_multimer_combine,
                      fused_multimer_combine_bwd, multi_pathway_attention_from_qkv)

__all__ = [
    "MpattnError", "MpattnUnsupported", "load_library", "rope_tables",
    "fused_multi_pathway_attention", "fused_multi_pathway_attention_fp16",
    "fused_multi_pathway_attention_bwd", "differentiable_multi_pathway_attention",
    "fused_multimer_combine", "fused_multimer_combine_bwd", "differentiable_multimer_combine",
    "multi_pathway_attention_from_qkv",
]
