"""Pin the DeepSeek-V4 oracle (oracle/dsv4_oracle.py) against the third-party transformers
DeepseekV4Attention (eager, float64, no cache) for all three layer types -- sliding window, CSA
(4-token overlapped compression + lightning indexer top-k) and HCA (every compressed entry) --
and the core attention against a dense masked restatement with the sink as an extra logit."""
import math

import pytest
import torch

from oracle import dsv4_oracle as V

mod = pytest.importorskip("transformers.models.deepseek_v4.modeling_deepseek_v4")
cfg_mod = pytest.importorskip("transformers.models.deepseek_v4.configuration_deepseek_v4")

LAYER_TYPES = ["sliding_attention", "compressed_sparse_attention", "heavily_compressed_attention"]


def _hf_config():
    c = cfg_mod.DeepseekV4Config(
        hidden_size=64, num_attention_heads=4, head_dim=32, q_lora_rank=24, num_hidden_layers=3,
        layer_types=LAYER_TYPES, compress_rates={"compressed_sparse_attention": 2, "heavily_compressed_attention": 4},
        sliding_window=5, o_groups=2, o_lora_rank=8, index_n_heads=2, index_head_dim=16, index_topk=3,
        partial_rotary_factor=8 / 32, rope_theta=100.0, compress_rope_theta=400.0, rms_norm_eps=1e-6,
        vocab_size=32, n_routed_experts=4, num_experts_per_tok=2, moe_intermediate_size=16)
    c._attn_implementation = "eager"
    return c


def _params(attn, layer_type):
    p = {"wq_a": attn.q_a_proj.weight, "q_norm": attn.q_a_norm.weight, "wq_b": attn.q_b_proj.weight,
         "wkv": attn.kv_proj.weight, "kv_norm": attn.kv_norm.weight, "wo_a": attn.o_a_proj.weight,
         "wo_b": attn.o_b_proj.weight, "sinks": attn.sinks}
    if attn.compressor is not None:
        c = attn.compressor
        p.update(comp_wkv=c.kv_proj.weight, comp_wgate=c.gate_proj.weight, comp_ape=c.position_bias,
                 comp_norm=c.kv_norm.weight)
        if layer_type == "compressed_sparse_attention":
            ix = c.indexer
            p.update(idx_wq_b=ix.q_b_proj.weight, idx_weights_proj=ix.scorer.weights_proj.weight,
                     idx_comp_wkv=ix.kv_proj.weight, idx_comp_wgate=ix.gate_proj.weight,
                     idx_comp_ape=ix.position_bias, idx_comp_norm=ix.kv_norm.weight)
    return {k: v.detach() for k, v in p.items()}


@pytest.mark.parametrize("layer_idx", [0, 1, 2])
def test_v4_attention_layer_matches_transformers(layer_idx):
    torch.manual_seed(7 + layer_idx)
    c = _hf_config()
    lt = c.layer_types[layer_idx]
    attn = mod.DeepseekV4Attention(c, layer_idx).double().eval()
    with torch.no_grad():
        for n, prm in attn.named_parameters():
            prm.normal_(0.0, 0.3 if prm.dim() > 1 else 0.5)
        for n, prm in attn.named_parameters():
            if n.endswith("norm.weight"):
                prm.add_(1.0)
    S = 23
    x = torch.randn(1, S, 64, dtype=torch.float64)
    pos = torch.arange(S)[None]
    rot = mod.DeepseekV4RotaryEmbedding(c)
    pe = {k: rot(x, pos, layer_type=k) for k in ("main", "compress")}
    s = torch.arange(S)
    vis = (s[None] <= s[:, None]) & (s[None] > s[:, None] - c.sliding_window)
    mask = torch.where(vis, 0.0, float("-inf")).double()[None, None]
    with torch.no_grad():
        hf, _ = attn(x, pe, pos, mask)
    ocfg = {"heads": 4, "head_dim": 32, "window": c.sliding_window, "eps": c.rms_norm_eps, "o_groups": 2,
            "index_heads": 2, "index_head_dim": 16, "index_topk": 3,
            "rates": {"csa": 2, "hca": 4},
            "inv_freq": {"main": rot.main_inv_freq, "compress": rot.compress_inv_freq},
            "mscale": {"main": rot.main_attention_scaling, "compress": rot.compress_attention_scaling}}
    ref = V.attention_layer(x[0], _params(attn, lt), ocfg, lt)
    # transformers forms the RoPE angles in float32 even in a float64 module (positions x inv_freq
    # in fp32, ~1e-7 relative), the oracle in float64: the bar is that rounding, far below the
    # O(1) error of a wrong sign, pairing, window or mask
    torch.testing.assert_close(ref, hf[0], rtol=2e-5, atol=5e-6)


def test_v4_core_attention_equals_dense_masked_form_with_sink_logit():
    # the gather form (per-query key lists) against one dense [T, T + Nc] masked softmax with the
    # sink as an extra column, HCA and CSA, over two packed documents
    g = torch.Generator().manual_seed(3)
    cu = [0, 11, 26]
    T, H, D, W, rate = cu[-1], 3, 8, 4, 3
    q = torch.randn(T, H, D, generator=g, dtype=torch.float64)
    kv = torch.randn(T, D, generator=g, dtype=torch.float64)
    n_comp = [(b - a) // rate for a, b in zip(cu[:-1], cu[1:])]
    comp = torch.randn(sum(n_comp), D, generator=g, dtype=torch.float64)
    sinks = torch.randn(H, generator=g, dtype=torch.float64)
    scale = 0.4
    sel = torch.full((T, 2), -1, dtype=torch.int64)
    for a, b in zip(cu[:-1], cu[1:]):
        for t in range(a, b):
            v = V.compressed_visible(t - a, rate)
            if v:
                sel[t, : min(2, v)] = torch.randperm(v, generator=g)[:2].sort().values
    for comp_sel in (None, sel):
        out, lse = V.core_attention(q, kv, comp, comp_sel, sinks, W, scale, rate, torch.tensor(cu))
        keys = torch.cat([kv, comp])
        m = torch.full((T, T + comp.shape[0]), float("-inf"), dtype=torch.float64)
        off = 0
        for d, (a, b) in enumerate(zip(cu[:-1], cu[1:])):
            for t in range(a, b):
                m[t, max(a, t - W + 1): t + 1] = 0.0
                ws = range(V.compressed_visible(t - a, rate)) if comp_sel is None else [int(x) for x in sel[t] if x >= 0]
                for w in ws:
                    m[t, T + off + w] = 0.0
            off += n_comp[d]
        logits = torch.einsum("thd,sd->ths", q, keys) * scale + m[:, None]
        full = torch.cat([logits, sinks[None, :, None].expand(T, H, 1)], dim=-1)
        p = torch.softmax(full, dim=-1)[..., :-1]
        torch.testing.assert_close(out, torch.einsum("ths,sd->thd", p, keys), rtol=1e-12, atol=1e-12)
        torch.testing.assert_close(lse, torch.logsumexp(full, dim=-1), rtol=1e-12, atol=1e-12)
