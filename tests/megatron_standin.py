"""Stand-ins for the Megatron pieces the absorbed MLA swap touches (Megatron-Core is not installed):
an ``MLASelfAttention`` with the reference's submodule names and shapes (multi_latent_attention.py:
14-187, TP = 1), linear layers returning ``(output, bias)``, a core attention holding the DSA
indexer and the softmax scale, layer specs, and this module's ``apply_rotary_pos_emb`` -- the
reference's patched bshd RoPE (transformer_layer.py:227-278: de-interleave when
``multi_latent_attention``, rotate-half per ``rotary_interleaved``, cos/sin scaled by
``attention_scaling`` and rounded to the input dtype) with THD positions restarting per document.

``reference_forward`` is the reference MLA's un-absorbed forward in float64 for a given top-k:
per-head ``key = [kv_c W_UK^T, k_pe]``, ``value = kv_c W_UV^T``, the un-fused sparse attention
(the oracle's), ``linear_proj``."""
import types

import torch


class Linear(torch.nn.Linear):
    def forward(self, x):
        return super().forward(x), None


def _rotate_half(x, interleaved):
    if not interleaved:
        x1, x2 = torch.chunk(x, 2, dim=-1)
        return torch.cat((-x2, x1), dim=-1)
    x1, x2 = x[..., 0::2], x[..., 1::2]
    return torch.stack((-x2, x1), dim=-1).flatten(start_dim=-2)


def _rope_bshd(t, freqs, config):
    rot = freqs.shape[-1]
    t, t_pass = t[..., :rot], t[..., rot:]
    if config.multi_latent_attention:
        t = torch.cat((t[..., 0::2], t[..., 1::2]), dim=-1)
    cos_ = (torch.cos(freqs) * config.attention_scaling).to(t.dtype)
    sin_ = (torch.sin(freqs) * config.attention_scaling).to(t.dtype)
    t = t * cos_ + _rotate_half(t, config.rotary_interleaved) * sin_
    return torch.cat((t, t_pass), dim=-1)


def apply_rotary_pos_emb(t, freqs, config, cu_seqlens=None, **kw):
    """``t [S, B, h, d]`` with ``freqs [S, 1, 1, d]``; THD ``t [T, h, d]`` with per-document positions."""
    if cu_seqlens is None:
        return _rope_bshd(t, freqs[: t.shape[0]], config)
    out = []
    cu = cu_seqlens.tolist()
    for a, b in zip(cu[:-1], cu[1:]):
        out.append(_rope_bshd(t[a:b].unsqueeze(1), freqs[: b - a], config).squeeze(1))
    return torch.cat(out)


def make_config(H, q_lora_rank, kv_lora_rank=512, qk_head_dim=128, rope=64, v_head_dim=128, coeff=0.0, sparse=True,
                mscale=1.0, rotary_interleaved=False, mla_interleaved=True):
    return types.SimpleNamespace(num_attention_heads=H, q_lora_rank=q_lora_rank, kv_lora_rank=kv_lora_rank,
                                 qk_head_dim=qk_head_dim, qk_pos_emb_head_dim=rope, v_head_dim=v_head_dim,
                                 dsa_indexer_loss_coeff=coeff, dsa_indexer_use_sparse_loss=sparse,
                                 attention_scaling=mscale, rotary_interleaved=rotary_interleaved,
                                 multi_latent_attention=mla_interleaved, layernorm_epsilon=1e-6)


class CoreAttention(torch.nn.Module):
    def __init__(self, indexer, softmax_scale):
        super().__init__()
        self.indexer = indexer
        self.softmax_scale = softmax_scale


class MLASelfAttention(torch.nn.Module):
    """The reference MLA's parameters (TP = 1); its own forward is never called by the tests."""

    def __init__(self, config, hidden, core_attention, device=None, dtype=torch.bfloat16):
        super().__init__()
        kw = dict(device=device, dtype=dtype)
        c = config
        H = c.num_attention_heads
        self.config = c
        self.num_attention_heads_per_partition = H
        self.attn_mask_type = types.SimpleNamespace(name="causal")
        self.linear_q_down_proj = Linear(hidden, c.q_lora_rank, bias=False, **kw)
        self.q_layernorm = torch.nn.RMSNorm(c.q_lora_rank, eps=1e-6, **kw)
        self.linear_q_up_proj = Linear(c.q_lora_rank, H * (c.qk_head_dim + c.qk_pos_emb_head_dim), bias=False, **kw)
        self.linear_kv_down_proj = Linear(hidden, c.kv_lora_rank + c.qk_pos_emb_head_dim, bias=False, **kw)
        self.kv_layernorm = torch.nn.RMSNorm(c.kv_lora_rank, eps=1e-6, **kw)
        self.linear_kv_up_proj = Linear(c.kv_lora_rank, H * (c.qk_head_dim + c.v_head_dim), bias=False, **kw)
        self.linear_proj = Linear(H * c.v_head_dim, hidden, bias=False, **kw)
        self.core_attention = core_attention


def spec_with(module_cls, n_layers=2):
    """A block spec shaped like Megatron's: ``layer_specs[i].submodules.self_attention.module``."""
    mk = lambda: types.SimpleNamespace(submodules=types.SimpleNamespace(
        self_attention=types.SimpleNamespace(module=module_cls)))
    return types.SimpleNamespace(layer_specs=[mk() for _ in range(n_layers)])


def reference_forward(mod, x, rope, topk, oracle):
    """float64 un-absorbed MLA forward of ``mod`` on ``x [S, B, hidden]`` for the selection ``topk
    [B, S, K]`` (multi_latent_attention.py:43-178, 262-290), differentiable in x and every weight
    of ``params`` (returned alongside)."""
    c = mod.config
    H = mod.num_attention_heads_per_partition
    names = ["linear_q_down_proj", "q_layernorm", "linear_q_up_proj", "linear_kv_down_proj", "kv_layernorm",
             "linear_kv_up_proj", "linear_proj"]
    params = {n: getattr(mod, n).weight.detach().double().cpu().requires_grad_() for n in names}
    xd = x.detach().double().cpu().requires_grad_()
    rope, topk = rope.cpu(), topk.cpu()
    rms = lambda v, w: v * torch.rsqrt(v.pow(2).mean(-1, keepdim=True) + 1e-6) * w
    S, B, _ = x.shape
    q_c = rms(xd @ params["linear_q_down_proj"].T, params["q_layernorm"])
    kv = xd @ params["linear_kv_down_proj"].T
    kv_c, k_pe = kv.split([c.kv_lora_rank, c.qk_pos_emb_head_dim], -1)
    kv_c = rms(kv_c, params["kv_layernorm"])
    q = (q_c @ params["linear_q_up_proj"].T).view(S, B, H, -1)
    q_nope, q_pe = q.split([c.qk_head_dim, c.qk_pos_emb_head_dim], -1)
    kvu = (kv_c @ params["linear_kv_up_proj"].T).view(S, B, H, -1)
    k_nope, value = kvu.split([c.qk_head_dim, c.v_head_dim], -1)
    q_pe = apply_rotary_pos_emb(q_pe, rope.double(), c)
    k_pe = apply_rotary_pos_emb(k_pe.unsqueeze(-2), rope.double(), c)
    query = torch.cat([q_nope, q_pe], -1)
    key = torch.cat([k_nope, k_pe.expand(S, B, H, -1)], -1)
    o = oracle.unabsorbed_sparse_attention(query, key, value, topk, mod.core_attention.softmax_scale)
    out = o @ params["linear_proj"].T
    return out, xd, params
