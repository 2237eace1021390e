"""MI355X-native Gated Sparse Attention (GSA) forward.

Drop-in for the GSA layer of nirmalpratheep/GSA_GDN_BenchmarkStudy
(``gsa_triton/gsa_opt.py``): the same module API, backed by hand-written gfx950
HIP kernels in ``libgsa_hip.so`` (C ABI: ``include/gsa_hip.h``).
"""

from .gsa import (  # noqa: F401
    AdaptiveTopKSelector,
    GatedLightningIndexer,
    GatedSparseAttention,
    OutputGate,
    RotaryEmbedding,
    ValueGate,
    apply_rotary_pos_emb,
    fused_gated_indexer,
    fused_sparse_attention,
)

__all__ = [
    "AdaptiveTopKSelector", "GatedLightningIndexer", "GatedSparseAttention", "OutputGate",
    "RotaryEmbedding", "ValueGate", "apply_rotary_pos_emb", "fused_gated_indexer",
    "fused_sparse_attention",
]
