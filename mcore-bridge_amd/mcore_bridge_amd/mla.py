"""Absorbed-layout MLA self-attention for DSA layers, installed through Megatron's layer spec.

mcore-bridge puts its own ``MLASelfAttention`` into every layer spec whose self-attention module
is Megatron's (reference src/mcore_bridge/model/register.py:158-162) and, for DSA models, the DSA
attention spec into each layer (register.py:94-106).  Its forward (multi_latent_attention.py:
14-292) up-projects q and kv per head (``linear_kv_up_proj``), applies RoPE to the rope parts and
calls the core attention -- Megatron's DSAttention: indexer, top-k, un-fused sparse attention
over per-head keys and values -- then ``linear_proj``.

``absorbed_mla_class(base)`` subclasses such an MLA class (the reference's or Megatron's) and
replaces only ``forward``: the same down projections, layernorms, q up-projection and RoPE (the
RoPE function of the base class's own module), then the DSA path of this package in the absorbed
latent layout -- the indexer's kernel path over the core attention's indexer parameters
(``IndexerView``), the causal top-k, and ``absorbed_mla_sparse_attention`` (``W_UK`` folded into
the query, the shared ``[kv_compressed, k_pos_emb]`` latent row, ``W_UV`` after the kernel) --
with the indexer KL loss applied in the attention's backward when training with
``dsa_indexer_loss_coeff > 0`` -- the dense loss by default, the sparse one with
``dsa_indexer_use_sparse_loss`` (model_config.py:204-205).
``install_attention(spec)`` makes the swap in a layer spec, the way register.py:158-162 does.

Recompute flags of the base class (set by Megatron's MLA from the recompute config) are honoured
with non-reentrant activation checkpointing (``torch.utils.checkpoint``):
- ``checkpoint_core_attention`` (in training, multi_latent_attention.py:250-252): the core
  attention -- ``W_UK`` absorption, the sparse attention kernels, ``W_UV`` and, when training the
  indexer, its loss -- is recomputed in the backward instead of keeping its activations.  (The
  reference's checkpointed path does not pass ``x``/``qr`` to DSA; here the indexer runs before
  the checkpointed region, so the flag works with DSA.)
- ``recompute_up_proj`` (multi_latent_attention.py:180-185, 282-285): the reference recomputes the
  per-head q/k/v up-projection and RoPE.  In the absorbed layout the up-projected tensor the
  attention keeps is the absorbed query (``H x 576`` per token, larger than the reference's q), so
  the checkpointed region is the q up-projection, RoPE and the core attention together.

Scope: one tensor-parallel rank holding every head (the kernels' single-GPU share), no
inference cache (the reference's DSA has none either, patcher.py:256), sbhd or THD packing.
"""
from __future__ import annotations

import sys
from typing import Optional

import torch
from torch import Tensor
from torch.utils.checkpoint import checkpoint

from .dsa import (IndexerView, _IndexerComputation, _mask_type_is_causal, _split_packed, _thd_docs,
                  absorbed_mla_sparse_attention)


def _out(r):
    """Megatron's linear layers return ``(output, bias)``."""
    return r[0] if isinstance(r, tuple) else r


def _rope_fn(cls):
    """The ``apply_rotary_pos_emb`` the MLA class's own module uses (multi_latent_attention.py:4),
    so the absorbed forward rotates q_pe and k_pe exactly as the reference caller does."""
    for klass in cls.__mro__:
        fn = getattr(sys.modules.get(klass.__module__), "apply_rotary_pos_emb", None)
        if fn is not None:
            return fn
    raise ImportError(f"{cls.__name__}: no apply_rotary_pos_emb in its module")


class _AbsorbedDSAForward:
    """``forward`` of the absorbed MLA (mixed into a subclass of the caller's MLA class)."""

    indexer_loss_scale: float = 1.0     # scale of the indexer loss gradient (the auto-scaler's role)
    last_indexer_loss: Optional[Tensor] = None

    def _dsa_indexer(self):
        ix = self.core_attention.indexer
        if isinstance(ix, _IndexerComputation):
            return ix
        view = getattr(self, "_dsa_indexer_view", None)
        if view is None or view.linear_wq_b is not ix.linear_wq_b:
            view = IndexerView(ix, self.config)
            self._dsa_indexer_view = view
        return view

    def _dsa_softmax_scale(self) -> float:
        for obj in (self.core_attention, self):
            s = getattr(obj, "softmax_scale", None)
            if s is not None:
                return float(s)
        raise AttributeError("softmax_scale not found on the MLA module or its core attention")

    def forward(self, hidden_states, attention_mask, key_value_states=None, inference_context=None,
                rotary_pos_emb=None, rotary_pos_cos=None, rotary_pos_sin=None, rotary_pos_cos_sin=None,
                attention_bias=None, packed_seq_params=None, position_ids=None, sequence_len_offset=None, *,
                inference_params=None):
        assert attention_bias is None, "Attention bias should not be passed into MLA."
        assert rotary_pos_cos is None and rotary_pos_sin is None, "MLA does not support Flash Decoding"
        assert key_value_states is None, "self-attention only"
        assert inference_context is None and inference_params is None, "the DSA path keeps no inference cache"
        cfg = self.config
        psp, _ = _split_packed(packed_seq_params)
        docs = _thd_docs(psp)
        x = hidden_states
        # down projections and norms (multi_latent_attention.py:43-86)
        if cfg.q_lora_rank is not None:
            q_c = self.q_layernorm(_out(self.linear_q_down_proj(x)))
        else:
            q_c = x
        kv_comb = _out(self.linear_kv_down_proj(x))
        d_rope = cfg.qk_pos_emb_head_dim
        assert kv_comb.shape[-1] == cfg.kv_lora_rank + d_rope, "one tensor-parallel rank holding every head"
        kv_c, k_pe = torch.split(kv_comb, [cfg.kv_lora_rank, d_rope], dim=-1)
        kv_c = self.kv_layernorm(kv_c)
        if docs is not None:                     # THD: [t, 1, ...] -> [t, ...] (:88-96)
            q_c, kv_c, k_pe = q_c.squeeze(1), kv_c.squeeze(1), k_pe.squeeze(1)
        H = self.num_attention_heads_per_partition
        rope = _rope_fn(type(self))
        cu = docs[0] if docs is not None else None
        add_b = (lambda t: t.unsqueeze(1)) if docs is not None else (lambda t: t)   # THD: one [T, 1] "batch"

        def up_proj(q_c, kv_c, k_pe):
            # q up-projection (:104-111); W_UK / W_UV of linear_kv_up_proj are absorbed instead of applied
            q = _out(self.linear_q_up_proj(q_c)) if cfg.q_lora_rank is not None else _out(self.linear_q_proj(q_c))
            q = q.view(*q.shape[:-1], H, cfg.qk_head_dim + d_rope)
            q_nope, q_pe = torch.split(q, [cfg.qk_head_dim, d_rope], dim=-1)
            # RoPE of the rope parts as the caller applies it (:150-162)
            q_pe = rope(q_pe, rotary_pos_emb, config=cfg, cu_seqlens=cu)
            k_pe = rope(k_pe.unsqueeze(-2), rotary_pos_emb, config=cfg, cu_seqlens=cu).squeeze(-2)
            return add_b(q_nope), add_b(q_pe), add_b(kv_c), add_b(k_pe)

        # DSA: indexer over (x, q_compressed) (:255-261), causal top-k, absorbed sparse attention
        assert _mask_type_is_causal(getattr(self, "attn_mask_type", None)), "DSA attention is causal"
        ix = self._dsa_indexer()
        coeff = float(getattr(cfg, "dsa_indexer_loss_coeff", 0.0) or 0.0)
        train_loss = self.training and coeff > 0 and torch.is_grad_enabled()
        if train_loss and ix.fp8:
            raise NotImplementedError("the indexer loss needs the bf16 indexer")
        with torch.set_grad_enabled(train_loss):
            ix_out = ix.forward_before_topk(x, q_c, (psp, rotary_pos_emb))
        _, topk = ix.topk_from_outputs(ix_out, None, docs, causal=True, return_scores=False)
        if docs is not None:
            topk = topk.unsqueeze(0)
            ix_out = tuple(add_b(o) for o in ix_out)
        w_kv = self.linear_kv_up_proj.weight
        scale = self._dsa_softmax_scale()
        sparse = bool(getattr(cfg, "dsa_indexer_use_sparse_loss", False))

        def core_attention(q_nope, q_pe, kv_c, k_pe, *ix_t):
            if not train_loss:
                return absorbed_mla_sparse_attention(q_nope, q_pe, kv_c, k_pe, w_kv, topk, scale, True), None
            return absorbed_mla_sparse_attention(q_nope, q_pe, kv_c, k_pe, w_kv, topk, scale, True,
                                                 indexer_loss=(*ix_t, coeff, self.indexer_loss_scale, sparse, docs))

        # the recompute flags (multi_latent_attention.py:180-185, 250-252): non-reentrant
        # checkpoints of the up-projection + core attention, or of the core attention alone
        grad = torch.is_grad_enabled()
        ix_t = ix_out if train_loss else ()
        if grad and getattr(self, "recompute_up_proj", False):
            out, loss = checkpoint(lambda *a: core_attention(*up_proj(*a[:3]), *a[3:]), q_c, kv_c, k_pe, *ix_t,
                                   use_reentrant=False)
        elif grad and self.training and getattr(self, "checkpoint_core_attention", False):
            out, loss = checkpoint(core_attention, *up_proj(q_c, kv_c, k_pe), *ix_t, use_reentrant=False)
        else:
            out, loss = core_attention(*up_proj(q_c, kv_c, k_pe), *ix_t)
        if train_loss:
            self.last_indexer_loss = loss
        # output projection (:286-290); THD gives (t, 1, h) like the caller's reshape (:281)
        return self.linear_proj(out)


_classes = {}


def absorbed_mla_class(base):
    """Subclass of the MLA class ``base`` whose forward runs the absorbed DSA path (cached per base)."""
    cls = _classes.get(base)
    if cls is None:
        cls = type("Absorbed" + base.__name__, (_AbsorbedDSAForward, base),
                   {"__module__": base.__module__, "_dsa_base": base, "__doc__": (base.__doc__ or "") +
                    "\n\nforward: the absorbed DSA path of mcore_bridge_amd (see mcore_bridge_amd.mla)."})
        _classes[base] = cls
    return cls


def _is_mla(module) -> bool:
    return isinstance(module, type) and any(k.__name__ == "MLASelfAttention" for k in module.__mro__)


def install_attention(transformer_layer_spec) -> int:
    """Swap the absorbed DSA MLA into every layer spec whose self-attention module is an
    ``MLASelfAttention`` (reference register.py:158-162 swaps its own the same way).  Takes a
    block spec with ``layer_specs`` or one layer spec; returns the number of layers swapped."""
    specs = getattr(transformer_layer_spec, "layer_specs", None) or [transformer_layer_spec]
    n = 0
    for layer_spec in specs:
        sa = layer_spec.submodules.self_attention
        if _is_mla(sa.module) and not issubclass(sa.module, _AbsorbedDSAForward):
            sa.module = absorbed_mla_class(sa.module)
            n += 1
    return n


def uninstall_attention(transformer_layer_spec) -> int:
    """Undo ``install_attention`` on a layer spec (restores the base MLA classes)."""
    specs = getattr(transformer_layer_spec, "layer_specs", None) or [transformer_layer_spec]
    n = 0
    for layer_spec in specs:
        sa = layer_spec.submodules.self_attention
        if isinstance(sa.module, type) and issubclass(sa.module, _AbsorbedDSAForward):
            sa.module = sa.module._dsa_base
            n += 1
    return n
