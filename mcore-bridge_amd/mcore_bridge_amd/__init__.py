"""mcore_bridge_amd -- MI355X-native (gfx950) DSA sparse-attention hot path.

Kernel-native ops (packed THD layout) live in ``ops``; Megatron-compatible drop-ins
(``fused_qk_topk_naive``, ``sparse_mla_attention``, ``absorbed_mla_sparse_attention``,
``indexer_forward_before_topk``, ``indexer_kl_loss``, the ``DSAIndexer`` and ``DSAttention`` modules) in
``dsa``; the absorbed DSA ``MLASelfAttention`` and its layer-spec swap in ``mla``; the DeepSeek-V4 hybrid
attention (sliding window + compressed entries + sink) in ``v4``; ``patch.install()``
swaps ``fused_qk_topk_naive`` into Megatron-Core's DSA module when it is importable.  All arithmetic
runs in the HIP kernels of ``libdsa_amd.so`` (C ABI: include/dsa_abi.h); there is no CPU fallback.
"""
from . import _lib
from .dsa import (DSAIndexer, DSAttention, IndexerView, absorbed_mla_sparse_attention, fused_qk_topk_naive,
                  indexer_forward_before_topk, indexer_kl_loss, sparse_mla_attention, sparse_mla_with_indexer_loss)
from .mla import absorbed_mla_class, install_attention, uninstall_attention
from .v4 import DSv4HybridAttention, sink_attention
from .ops import (build_decode_rows, build_rows, bwd_workspace_bytes, decode_indexer_topk, decode_workspace_bytes,
                  indexer_kl_rows, indexer_kl_target, indexer_prologue, indexer_scores, indexer_scores_bwd,
                  indexer_selected_scores, indexer_topk, sparse_mla, sparse_mla_bwd, sparse_mla_decode,
                  sparse_mla_fwd, topk)

__all__ = [
    "DSAIndexer", "DSAttention", "DSv4HybridAttention", "IndexerView", "absorbed_mla_class", "absorbed_mla_sparse_attention",
    "build_decode_rows", "build_rows", "bwd_workspace_bytes", "decode_indexer_topk", "decode_workspace_bytes",
    "fused_qk_topk_naive", "indexer_forward_before_topk", "indexer_kl_loss", "indexer_kl_rows", "indexer_kl_target",
    "indexer_prologue", "indexer_scores", "indexer_scores_bwd", "indexer_selected_scores", "indexer_topk",
    "install_attention", "sparse_mla", "sparse_mla_attention", "sparse_mla_bwd", "sparse_mla_decode",
    "sink_attention", "sparse_mla_fwd", "sparse_mla_with_indexer_loss", "topk", "uninstall_attention",
]
__version__ = "0.2.0"
