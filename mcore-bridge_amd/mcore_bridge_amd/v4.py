"""DeepSeek-V4 hybrid attention (sliding window + compressed entries, per-head attention sink) on
the DSA kernels of this package.

The reference owns the layer arithmetic of ``DSv4HybridSelfAttention``
(src/mcore_bridge/model/gpts/deepseek_v4.py:61-328): q down / norm / up projection with a
weightless per-head RMS norm, ONE shared 512-wide K = V head, interleaved RoPE on the trailing 64
dims, the inverse RoPE on the output's rope slice, the grouped output projection; its core
attention (sliding window, CSA compressor + lightning indexer, HCA compressor, attention sink:
``core_attention.{attn_sink, compressor, indexer}``, :443-464) is megatron-core's.

Kernel mapping (no new arithmetic kernel):
- the attention is the absorbed sparse MQA of ``sparse_mla_fwd`` / ``_bwd`` (K3 / K4) with the
  512-wide K = V rows stored in the kernels' 576-wide row layout, rope region zero: the kernels'
  ``v = kv[:, :512]`` is then the whole key, and the zero region adds nothing to q . k; the
  512-wide q rows (and dq) are read and written as they are (``d_qk = 512``: no rope part);
- every query's key list -- its sliding window over the raw rows, then the compressed entries it
  may see (CSA: the indexer's top-k; HCA: all of them) -- is one index row over the
  concatenation ``[raw rows; compressed entries]``;
- the sink is a logit with no value, folded into the forward kernel's normaliser (``lse' =
  logaddexp(lse, sink_h)``, ``out' = out * exp(lse - lse')``, ``dsa_sparse_mla_fwd_sink``).  The
  backward of K4 fed ``(out', lse')`` is exactly the sink-augmented attention's (its P and Delta
  are then the sink softmax's), and ``d sink_h = -sum_t exp(sink_h - lse'[t,h]) * Delta[t,h]``
  from B1's Delta rows (``dsa_sparse_mla_bwd_sink``);
- the CSA indexer is K1 + K2 over the compressed index keys: query t's row is its document's
  entries ``w < (t - start + 1) // rate``; the scorer's ``softmax_scale`` is folded into the head
  weights (ReLU is positively homogeneous).
The compressors (softmax-gated window pooling, RMS norm, RoPE) and the projections are torch ops.
"""
from __future__ import annotations

import math
from typing import List, Optional, Sequence, Tuple

import torch
import torch.nn.functional as F
from torch import Tensor

from . import ops

HEAD_DIM = 512
ROPE_DIM = 64


# --------------------------------------------------------------------------------------
# attention core: sparse MQA over one shared K = V head, with a per-head sink
# --------------------------------------------------------------------------------------
class _SinkAttention(torch.autograd.Function):
    @staticmethod
    def forward(ctx, q: Tensor, kv: Tensor, sinks: Tensor, idx: Tensor, scale: float):
        # the kernels take the 512-wide q rows as they are (no rope part) and K = V rows in the
        # 576-wide row layout with a zero rope region (a copy of the N key rows only)
        q = q.contiguous()
        kv_p = F.pad(kv, (0, ops.D_QK - HEAD_DIM)).contiguous()
        out, lse = ops.sparse_mla_fwd_sink(q, kv_p, idx, sinks, scale, False)   # the sink folded in-kernel
        ctx.save_for_backward(q, kv_p, idx, out, lse, sinks)
        ctx.scale = scale
        ctx.kv_dtype = kv.dtype
        ctx.mark_non_differentiable(lse)
        return out, lse

    @staticmethod
    def backward(ctx, dout: Tensor, dlse: Tensor):
        q, kv_p, idx, out, lse, sinks = ctx.saved_tensors
        dq, dkv_p, dsinks = ops.sparse_mla_bwd_sink(q, kv_p, idx, out, dout.contiguous(), lse, sinks, ctx.scale,
                                                    False)
        dq = dq if ctx.needs_input_grad[0] else None
        dkv = dkv_p[:, :HEAD_DIM].to(ctx.kv_dtype) if ctx.needs_input_grad[1] else None
        return dq, dkv, dsinks.to(sinks.dtype) if ctx.needs_input_grad[2] else None, None, None


def sink_attention(q: Tensor, kv: Tensor, sinks: Tensor, idx: Tensor, scale: float) -> Tuple[Tensor, Tensor]:
    """``out[t,h] = sum_j p_j kv[idx[t,j]]`` with ``p = exp(scale q.k_j) / (sum_j exp(scale q.k_j) +
    exp(sinks[h]))`` over the valid entries of ``idx [T, K]`` (``-1`` = none, distinct per row).
    ``q [T, H, 512]``, ``kv [N, 512]`` bf16 (K = V), ``sinks [H]``.  Returns ``(out [T, H, 512] bf16,
    lse [T, H])`` (``lse`` includes the sink); differentiable in ``q``, ``kv`` and ``sinks``.  H a
    multiple of 16, at most 128, for the backward."""
    assert q.shape[-1] == HEAD_DIM and kv.shape[-1] == HEAD_DIM, "512-wide q and K = V rows"
    return _SinkAttention.apply(q, kv, sinks, idx.to(torch.int32).contiguous(), float(scale))


# --------------------------------------------------------------------------------------
# index rows: sliding window + compressed entries, per document
# --------------------------------------------------------------------------------------
def _docs(cu_seqlens: Sequence[int], device):
    cu = [int(x) for x in cu_seqlens]
    lens = torch.tensor([b - a for a, b in zip(cu[:-1], cu[1:])], device=device)
    start = torch.repeat_interleave(torch.tensor(cu[:-1], device=device), lens)
    return cu, lens, start


def compressed_layout(cu_seqlens: Sequence[int], rate: int) -> List[int]:
    """Offsets of each document's compressed entries in the concatenated compressed array
    (``len = n_docs + 1``; document d holds ``(L_d // rate)`` entries)."""
    cu = [int(x) for x in cu_seqlens]
    off = [0]
    for a, b in zip(cu[:-1], cu[1:]):
        off.append(off[-1] + (b - a) // rate)
    return off


def hybrid_indices(cu_seqlens: Sequence[int], window: int, rate: int = 0, comp_sel: Optional[Tensor] = None,
                   device=None) -> Tensor:
    """``[T, window + Kc]`` int32 rows over ``[raw rows (T); compressed entries]``: slots ``j < window``
    hold raw row ``t - window + 1 + j`` when it is in t's document, then either the CSA selection
    ``comp_sel [T, Kc]`` (ids into the compressed array, ``-1`` pad) or, with ``rate`` and no
    selection (HCA), every entry ``w < (t - start + 1) // rate`` of t's document; ``-1`` = none."""
    cu, lens, start = _docs(cu_seqlens, device)
    T = cu[-1]
    t = torch.arange(T, device=device)
    s = t[:, None] - window + 1 + torch.arange(window, device=device)[None]
    win = torch.where(s >= start[:, None], s, torch.full_like(s, -1))
    parts = [win]
    if comp_sel is not None:
        cs = comp_sel.to(torch.int64)
        parts.append(torch.where(cs >= 0, cs + T, torch.full_like(cs, -1)))
    elif rate:
        off = compressed_layout(cu, rate)
        kc = max(max((b - a) // rate for a, b in zip(cu[:-1], cu[1:])), 1)
        offs = torch.repeat_interleave(torch.tensor(off[:-1], device=device), lens)
        vis = (t - start + 1) // rate
        j = torch.arange(kc, device=device)[None]
        parts.append(torch.where(j < vis[:, None], T + offs[:, None] + j, torch.full_like(j.expand(T, -1), -1)))
    return torch.cat(parts, dim=1).to(torch.int32)


def indexer_select(q_idx: Tensor, comp_k: Tensor, w: Tensor, cu_seqlens: Sequence[int], rate: int, topk: int,
                   index_head_dim: int, return_scores: bool = False):
    """The CSA lightning indexer on the kernels: ``I[t, s] = sum_h w[t,h] relu(q_idx[t,h] . k[s]) *
    index_head_dim^-0.5`` over the compressed index keys ``comp_k [Nc, Di]`` of t's document with
    ``s < (t - start + 1) // rate``; returns ``[T, topk]`` int32 ids into the compressed array
    (ascending, ``-1`` pad) and, with ``return_scores``, the fp32 scores ``[T, pitch]`` the top-k
    selected from (column j = entry ``doc offset + j``; ``-inf`` past each row)."""
    cu, lens, start = _docs(cu_seqlens, q_idx.device)
    T = cu[-1]
    if comp_k.shape[0] == 0:   # no document holds a complete window: nothing to select
        idx = torch.full((T, topk), -1, dtype=torch.int32, device=q_idx.device)
        if not return_scores:
            return idx
        return idx, torch.full((T, 4), float("-inf"), dtype=torch.float32, device=q_idx.device)
    off = compressed_layout(cu, rate)
    offs = torch.repeat_interleave(torch.tensor(off[:-1], device=q_idx.device), lens)
    t = torch.arange(T, device=q_idx.device)
    row_len = ((t - start + 1) // rate).to(torch.int32)
    row_base = offs.to(torch.int32)
    max_len = max(max((b - a) // rate for a, b in zip(cu[:-1], cu[1:])), 1)
    pitch = (max_len + 3) // 4 * 4
    wf = w.float() * index_head_dim ** -0.5
    sc = ops.indexer_scores(q_idx.contiguous(), comp_k.contiguous(), wf.contiguous(), row_base, row_len, max_len,
                            pitch, None, None, return_scores)
    idx = ops.topk(sc, row_base, row_len, topk)
    return (idx, sc) if return_scores else idx


# --------------------------------------------------------------------------------------
# host-side pieces of the layer: projections and their norms in torch; per-head norm + RoPE, the
# output's RoPE + grouped layout and the compressors' pooling on HIP kernels
# --------------------------------------------------------------------------------------
class _NormRope(torch.autograd.Function):
    """Per-row weightless RMS norm (``norm``) then interleaved RoPE on the last ``rope_dim`` dims of
    rows ``x [T, H, D]`` (``ops.v4_norm_rope`` / ``_bwd``: one HBM pass each way)."""

    @staticmethod
    def forward(ctx, x, cos, sin, rope_dim, norm, eps, inverse):
        x = x.contiguous()
        ctx.save_for_backward(x if norm else None, cos, sin)
        ctx.cfg = (rope_dim, norm, eps, inverse)
        return ops.v4_norm_rope(x, cos, sin, rope_dim, norm, eps, inverse)

    @staticmethod
    def backward(ctx, g):
        x, cos, sin = ctx.saved_tensors
        rope_dim, norm, eps, inverse = ctx.cfg
        g = g.contiguous()
        dx = ops.v4_norm_rope_bwd(x if norm else g, g, cos, sin, rope_dim, norm, eps, inverse)
        return dx, None, None, None, None, None, None


def norm_rope(x: Tensor, cos: Tensor, sin: Tensor, norm: bool, eps: float = 0.0, inverse: bool = False) -> Tensor:
    """``x [N, ..., D]`` rows: optional weightless RMS norm, then the interleaved RoPE of the last
    ``ROPE_DIM`` dims with row n's token angles (``cos / sin [N, ROPE_DIM / 2]``, mscale applied)."""
    shape = x.shape
    rows = x.reshape(shape[0], math.prod(shape[1:-1]), shape[-1])    # [N, heads, D] (N may be 0)
    return _NormRope.apply(rows, cos, sin, ROPE_DIM, norm, eps, inverse).view(shape)


def rope_tables(angles: Tensor, mscale: float) -> Tuple[Tensor, Tensor]:
    """fp32 ``cos / sin [N, ROPE_DIM / 2]`` of the RoPE angles, times the attention mscale."""
    a = angles.float()
    return (torch.cos(a) * mscale).contiguous(), (torch.sin(a) * mscale).contiguous()


class _OutRopeGroup(torch.autograd.Function):
    """The output's inverse RoPE, written in the grouped projection's layout ``[G, T, H * D / G]``
    (``ops.v4_out_rope_group`` / ``_bwd``)."""

    @staticmethod
    def forward(ctx, o, cos, sin, groups):
        ctx.save_for_backward(cos, sin)
        ctx.n_heads = o.shape[1]
        return ops.v4_out_rope_group(o.contiguous(), cos, sin, ROPE_DIM, groups, True)

    @staticmethod
    def backward(ctx, g):
        cos, sin = ctx.saved_tensors
        return ops.v4_out_rope_group_bwd(g.contiguous(), ctx.n_heads, cos, sin, ROPE_DIM, True), None, None, None


class _GroupedProj(torch.autograd.Function):
    """``out[t, g*N:(g+1)*N] = a[g, t] @ w[g]^T`` for ``a [G, T, K]`` and ``w [G, N, K]`` (the
    grouped output projection ``wo_a``, ``deepseek_v4.py:313-318``), written straight into the
    ``[T, G * N]`` rows the output projection reads; one library GEMM per group each way, on the
    operands as they lie (no transposed copies)."""

    @staticmethod
    def forward(ctx, a, w):
        G, T, _ = a.shape
        N = w.shape[1]
        ctx.save_for_backward(a, w)
        out = torch.empty(T, G * N, dtype=a.dtype, device=a.device)
        for g in range(G):
            torch.mm(a[g], w[g].t(), out=out[:, g * N:(g + 1) * N])
        return out

    @staticmethod
    def backward(ctx, grad):
        a, w = ctx.saved_tensors
        G, N = w.shape[0], w.shape[1]
        da = torch.empty_like(a) if ctx.needs_input_grad[0] else None
        dw = torch.empty_like(w) if ctx.needs_input_grad[1] else None
        for g in range(G):
            gg = grad[:, g * N:(g + 1) * N]
            if da is not None:
                torch.mm(gg, w[g], out=da[g])
            if dw is not None:
                torch.mm(gg.t(), a[g], out=dw[g])
        return da, dw


class _Compress(torch.autograd.Function):
    """The compressor's pooling + norm on the HIP kernels (``ops.v4_compress_fwd`` / ``_bwd``); the
    backward recomputes the pooling from ``kv`` and ``gate``."""

    @staticmethod
    def forward(ctx, kv, gate, ape, norm_w, table, n_entries, n_items, rate, eps, overlap):
        out = ops.v4_compress_fwd(kv, gate, ape, norm_w, table, n_entries, rate, eps, overlap)
        ctx.save_for_backward(kv, gate, ape, norm_w, table)
        ctx.meta = (n_entries, n_items, rate, eps, overlap)
        return out

    @staticmethod
    def backward(ctx, dout):
        kv, gate, ape, norm_w, table = ctx.saved_tensors
        dkv, dgate, dape, dnorm = ops.v4_compress_bwd(kv, gate, ape, norm_w, table, *ctx.meta,
                                                      dout.to(torch.bfloat16).contiguous())
        return dkv, dgate, dape.to(ape.dtype), dnorm.to(norm_w.dtype), None, None, None, None, None, None


def compress(kv: Tensor, gate: Tensor, ape: Tensor, norm_w: Tensor, cu_seqlens: Sequence[int], rate: int, eps: float,
             overlap: bool) -> Tensor:
    """Compressed entries of every document (concatenated in document order): softmax-gated pooling
    of each complete ``rate``-token window (CSA: ``overlap``, ``2 * rate`` slots over the previous
    window's first halves and this window's second halves), RMS norm -- one HIP kernel each way
    (``dsa_v4_compress_fwd`` / ``dsa_v4_compress_bwd``).  ``kv``, ``gate [T, C]`` bf16, ``ape [rate, C]``.
    Returns ``[Nc, D]`` (before RoPE)."""
    cu = [int(x) for x in cu_seqlens]
    ops._require(cu[-1] == kv.shape[0], "cu_seqlens must end at the token count")
    table, n_entries, n_items = ops.compress_doc_table(cu, rate, kv.device)
    return _Compress.apply(kv, gate, ape, norm_w, table, n_entries, n_items, rate, eps, overlap)


def compressed_positions(cu_seqlens: Sequence[int], rate: int, device) -> Tensor:
    """Position (inside its document) of each compressed entry's RoPE: ``w * rate``."""
    cu = [int(x) for x in cu_seqlens]
    return torch.cat([torch.arange((b - a) // rate, device=device) * rate for a, b in zip(cu[:-1], cu[1:])]
                     or [torch.zeros(0, dtype=torch.int64, device=device)])


class _Compressor(torch.nn.Module):
    """Parameters of a V4 compressor, with the reference's names (``ape``, ``linear_wkv``,
    ``linear_wgate``, ``norm``; deepseek_v4.py:447-451)."""

    def __init__(self, hidden: int, dim: int, rate: int, overlap: bool, **kw):
        super().__init__()
        c = 2 * dim if overlap else dim
        self.rate, self.overlap = rate, overlap
        self.linear_wkv = torch.nn.Linear(hidden, c, bias=False, **kw)
        self.linear_wgate = torch.nn.Linear(hidden, c, bias=False, **kw)
        self.ape = torch.nn.Parameter(torch.zeros(rate, c, **kw))
        self.norm = torch.nn.RMSNorm(dim, **kw)

    def forward(self, x: Tensor, cu: Sequence[int], eps: float) -> Tensor:
        return compress(self.linear_wkv(x), self.linear_wgate(x), self.ape, self.norm.weight, cu, self.rate, eps,
                        self.overlap)


class _Indexer(torch.nn.Module):
    """The CSA indexer's parameters (``linear_wq_b``, ``linear_weights_proj``, ``compressor``;
    deepseek_v4.py:453-464)."""

    def __init__(self, hidden: int, q_lora_rank: int, n_heads: int, head_dim: int, topk: int, rate: int, **kw):
        super().__init__()
        self.n_heads, self.head_dim, self.topk = n_heads, head_dim, topk
        self.linear_wq_b = torch.nn.Linear(q_lora_rank, n_heads * head_dim, bias=False, **kw)
        self.linear_weights_proj = torch.nn.Linear(hidden, n_heads, bias=False, **kw)
        self.compressor = _Compressor(hidden, head_dim, rate, True, **kw)


class _CoreAttention(torch.nn.Module):
    def __init__(self, n_heads: int, **kw):
        super().__init__()
        self.attn_sink = torch.nn.Parameter(torch.zeros(n_heads, dtype=torch.float32, device=kw.get("device")))
        self.compressor = None
        self.indexer = None


class DSv4HybridAttention(torch.nn.Module):
    """Host mirror of the reference's ``DSv4HybridSelfAttention`` (deepseek_v4.py:61-328) for one
    layer type (``sliding_attention``, ``compressed_sparse_attention``, ``heavily_compressed_attention``)
    over the DSA kernels.  Parameter names follow the reference's Megatron module, so the keys its
    bridge maps (deepseek_v4.py:432-464: ``linear_proj`` = wo_b, ``linear_o_group_proj`` = wo_a,
    ``linear_q_down_proj`` = wq_a, ``linear_q_up_proj`` = wq_b, ``linear_kv_proj`` = wkv,
    ``q_layernorm`` / ``kv_layernorm``, ``core_attention.attn_sink``, ``core_attention.compressor.*``,
    ``core_attention.indexer.*``) load one to one.

    ``forward(hidden_states [S, B, hidden] or THD [T, 1, hidden], rotary_pos_emb={'main': [S, 1, 1,
    64], 'compress': ...} angles, packed_seq_params=None)`` returns ``(output, None)`` like the
    reference; ``rotary_pos_emb`` holds Megatron's duplicated-half angle rows (the first 32 are the
    interleaved pairs' angles)."""

    def __init__(self, layer_type: str, hidden_size: int, num_heads: int, q_lora_rank: int, o_groups: int,
                 o_lora_rank: int, window: int = 128, compress_rates=(4, 128), index_n_heads: int = 64,
                 index_head_dim: int = 128, index_topk: int = 512, eps: float = 1e-6, mscale: float = 1.0,
                 compress_mscale: float = 1.0, device=None, dtype=torch.bfloat16):
        super().__init__()
        assert layer_type in ("sliding_attention", "compressed_sparse_attention", "heavily_compressed_attention")
        kw = dict(device=device, dtype=dtype)
        self.layer_type, self.H, self.window, self.eps = layer_type, num_heads, window, eps
        self.keep_index_scores = False   # CSA: keep the indexer's fp32 scores in last_index_scores
        self.o_groups, self.o_lora_rank = o_groups, o_lora_rank
        self.rope_layer_type = "main" if layer_type == "sliding_attention" else "compress"
        self.mscale = mscale if self.rope_layer_type == "main" else compress_mscale
        self.linear_q_down_proj = torch.nn.Linear(hidden_size, q_lora_rank, bias=False, **kw)
        self.q_layernorm = torch.nn.RMSNorm(q_lora_rank, eps=eps, **kw)
        self.linear_q_up_proj = torch.nn.Linear(q_lora_rank, num_heads * HEAD_DIM, bias=False, **kw)
        self.linear_kv_proj = torch.nn.Linear(hidden_size, HEAD_DIM, bias=False, **kw)
        self.kv_layernorm = torch.nn.RMSNorm(HEAD_DIM, eps=eps, **kw)
        self.linear_o_group_proj = torch.nn.Parameter(
            torch.empty(o_groups * o_lora_rank, num_heads * HEAD_DIM // o_groups, **kw))
        self.linear_proj = torch.nn.Linear(o_groups * o_lora_rank, hidden_size, bias=False, **kw)
        self.core_attention = _CoreAttention(num_heads, **kw)
        csa_rate, hca_rate = compress_rates
        if layer_type == "compressed_sparse_attention":
            self.rate = csa_rate
            self.core_attention.compressor = _Compressor(hidden_size, HEAD_DIM, csa_rate, True, **kw)
            self.core_attention.indexer = _Indexer(hidden_size, q_lora_rank, index_n_heads, index_head_dim,
                                                   index_topk, csa_rate, **kw)
        elif layer_type == "heavily_compressed_attention":
            self.rate = hca_rate
            self.core_attention.compressor = _Compressor(hidden_size, HEAD_DIM, hca_rate, False, **kw)
        else:
            self.rate = 0
        torch.nn.init.normal_(self.linear_o_group_proj, std=0.02)

    def forward(self, hidden_states: Tensor, attention_mask=None, rotary_pos_emb=None, packed_seq_params=None,
                **kw):
        x3 = hidden_states
        psp = packed_seq_params
        thd = psp is not None and getattr(psp, "qkv_format", "thd") == "thd"
        if thd:
            cu = [int(v) for v in psp.cu_seqlens_q.tolist()]
            x = x3.reshape(x3.shape[0], -1)
            B, S = 1, x.shape[0]
        else:
            S, B, _ = x3.shape
            x = x3.transpose(0, 1).reshape(B * S, -1)        # batch rows as documents
            cu = [b * S for b in range(B + 1)]
        T = x.shape[0]
        dev = x.device
        angles_tab = rotary_pos_emb[self.rope_layer_type].reshape(-1, rotary_pos_emb[self.rope_layer_type].shape[-1])
        angles_tab = angles_tab[:, : ROPE_DIM // 2].float()
        _, _, start = _docs(cu, dev)
        pos = torch.arange(T, device=dev) - start                              # position inside the document
        cs, sn = rope_tables(angles_tab[pos], self.mscale)
        # q path (deepseek_v4.py:114-142): down, norm, up, per-head weightless RMS norm, RoPE
        q_res = self.q_layernorm(self.linear_q_down_proj(x))
        q = self.linear_q_up_proj(q_res).view(T, self.H, HEAD_DIM)
        q = norm_rope(q, cs, sn, True, self.eps)
        # the one K = V head (:144-198)
        kv = norm_rope(self.kv_layernorm(self.linear_kv_proj(x)), cs, sn, False)
        comp_sel = None
        keys = kv
        ca = self.core_attention
        if ca.compressor is not None:
            comp = ca.compressor(x, cu, self.eps)
            ccs, csn = rope_tables(angles_tab[compressed_positions(cu, self.rate, dev)], self.mscale)
            comp = norm_rope(comp, ccs, csn, False)
            keys = torch.cat([kv, comp])
            if ca.indexer is not None:
                ix = ca.indexer
                with torch.no_grad():
                    ck = norm_rope(ix.compressor(x, cu, self.eps), ccs, csn, False)
                    qi = norm_rope(ix.linear_wq_b(q_res).view(T, ix.n_heads, ix.head_dim), cs, sn, False)
                    wi = ix.linear_weights_proj(x).float() * ix.n_heads ** -0.5
                    comp_sel = indexer_select(qi, ck, wi, cu, self.rate, ix.topk, ix.head_dim,
                                              return_scores=self.keep_index_scores)
                    if self.keep_index_scores:
                        comp_sel, self.last_index_scores = comp_sel
                self.last_indexer_selection = comp_sel
        idx = hybrid_indices(cu, self.window, self.rate if comp_sel is None else 0, comp_sel, dev)
        o, _ = sink_attention(q, keys, ca.attn_sink, idx, HEAD_DIM ** -0.5)
        # inverse RoPE on the rope slice of each head's output (:287-311), grouped output (:313-318)
        og = _OutRopeGroup.apply(o, cs, sn, self.o_groups)                     # [G, T, H*D/G]
        wo_a = self.linear_o_group_proj.view(self.o_groups, self.o_lora_rank, -1)
        o = _GroupedProj.apply(og, wo_a)                                       # [T, G * o_lora_rank]
        out = self.linear_proj(o)
        if thd:
            return out.view(T, 1, -1), None
        return out.view(B, S, -1).transpose(0, 1), None
