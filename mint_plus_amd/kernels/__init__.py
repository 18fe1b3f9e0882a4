"""gfx950 kernels of the multi-pathway attention op, with the reference's
Python entry points (``mint_plus/models/kernels/__init__.py``,
``multi_pathway_attention.py``, ``multi_pathway_attention_bwd.py``,
``multi_pathway_attention_fp16.py``, ``differentiable_attention.py``)."""
from .multi_pathway_attention import (fused_multi_pathway_attention,
                                      fused_multi_pathway_attention_fp16)
from .multi_pathway_attention_bwd import fused_multi_pathway_attention_bwd
from .differentiable_attention import differentiable_multi_pathway_attention
from .combine import (differentiable_multimer_combine, fused_multimer_combine,
                      fused_multimer_combine_bwd)
from .projected import multi_pathway_attention_from_qkv

__all__ = [
    "fused_multi_pathway_attention",
    "fused_multi_pathway_attention_fp16",
    "fused_multi_pathway_attention_bwd",
    "differentiable_multi_pathway_attention",
    "fused_multimer_combine",
    "fused_multimer_combine_bwd",
    "differentiable_multimer_combine",
    "multi_pathway_attention_from_qkv",
]
