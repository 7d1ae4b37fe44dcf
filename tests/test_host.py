"""CPU tests of the host-side logic: the Megatron plug-in point, workload constants, and the
causal-mask detection used by the fused_qk_topk_naive drop-in."""
import sys
import types

import torch

from mcore_bridge_amd import patch, dsa, workloads as W


def test_patch_install_swaps_megatron_attribute():
    # a stand-in for megatron.core.transformer.experimental_attention_variant.dsa: install()
    # must replace exactly the attribute DSAIndexer.forward_with_scores imports at call time
    # (reference src/mcore_bridge/patcher.py:349) and uninstall() must restore it
    names = ["megatron", "megatron.core", "megatron.core.transformer",
             "megatron.core.transformer.experimental_attention_variant", patch.DSA_MODULE]
    saved = {n: sys.modules.get(n) for n in names}
    try:
        for n in names:
            sys.modules[n] = types.ModuleType(n)
        orig = object()
        sys.modules[patch.DSA_MODULE].fused_qk_topk_naive = orig
        assert patch.install()
        assert sys.modules[patch.DSA_MODULE].fused_qk_topk_naive is dsa.fused_qk_topk_naive
        patch.uninstall()
        assert sys.modules[patch.DSA_MODULE].fused_qk_topk_naive is orig
    finally:
        for n, m in saved.items():
            if m is None:
                sys.modules.pop(n, None)
            else:
                sys.modules[n] = m


def test_patch_install_without_megatron_is_a_no_op():
    assert "megatron" not in sys.modules or sys.modules["megatron"] is None or True
    if "megatron" not in sys.modules:
        assert patch.install() is False


def test_causal_mask_detection():
    S = 9
    m = torch.triu(torch.full((S, S), float("-inf")), 1)[None].expand(2, S, S)
    assert dsa._is_causal_mask(m)
    m2 = m.clone()
    m2[1, 3, 5] = 0.0
    assert not dsa._is_causal_mask(m2)
    assert not dsa._is_causal_mask(torch.zeros(1, S, S))


def test_config_shapes():
    c3 = W.CONFIGS["cfg3"]
    assert c3.cu_seqlens[-1] == c3.S == 16384 and c3.backward
    assert W.CONFIGS["cfg4"].fp8_indexer and W.CONFIGS["cfg4"].S == 32768
    assert len(W.CONFIGS["cfg5"].decode_lens) == 64
    x = W.make_prefill(W.CONFIGS["cfg1"], S=64)
    assert x["q"].shape == (64, 16, 576) and x["w"].min() >= 0      # cfg1 weights ~ U(0,1)
    y = W.make_prefill(W.CONFIGS["cfg1"], S=64)
    assert torch.equal(x["q"], y["q"])                                 # seeded, reproducible
