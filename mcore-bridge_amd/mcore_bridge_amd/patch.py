"""Swap the DSA hot path of an installed Megatron-Core for the MI355X kernels.

Reference plugin point: DSAIndexer.forward_with_scores imports ``fused_qk_topk_naive`` from
``megatron.core.transformer.experimental_attention_variant.dsa`` *inside* the method at call time
(reference src/mcore_bridge/patcher.py:349), so reassigning that module attribute replaces the
scoring + top-k with no model-code change -- the same module-attribute mechanism mcore-bridge
itself uses to install its patched DSAIndexer (patcher.py:382).
"""
from __future__ import annotations

import importlib

from .dsa import fused_qk_topk_naive
# The whole DSA attention (indexer, top-k, absorbed sparse attention, indexer loss) goes in at the
# layer spec instead: install_attention(spec) swaps an absorbed MLASelfAttention subclass into every
# MLA layer spec, the mechanism of reference src/mcore_bridge/model/register.py:158-162.
from .mla import install_attention, uninstall_attention  # noqa: F401

DSA_MODULE = "megatron.core.transformer.experimental_attention_variant.dsa"

_saved = {}


def install() -> bool:
    """Point Megatron's ``fused_qk_topk_naive`` at the HIP implementation.  Returns False (and
    changes nothing) when Megatron-Core is not importable."""
    try:
        mod = importlib.import_module(DSA_MODULE)
    except ImportError:
        return False
    if "fused_qk_topk_naive" not in _saved:
        _saved["fused_qk_topk_naive"] = getattr(mod, "fused_qk_topk_naive", None)
    mod.fused_qk_topk_naive = fused_qk_topk_naive
    return True


def uninstall() -> None:
    """Restore what ``install()`` replaced."""
    if not _saved:
        return
    mod = importlib.import_module(DSA_MODULE)
    mod.fused_qk_topk_naive = _saved.pop("fused_qk_topk_naive")
