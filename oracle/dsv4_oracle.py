"""CPU oracle of the DeepSeek-V4 hybrid attention (TEST INFRASTRUCTURE ONLY).

Like ``dsa_oracle``, this module is the checker, never the product: only ``tests/``,
``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may import it.

The reference (mcore-bridge) owns the layer arithmetic of its ``DSv4HybridSelfAttention``
(src/mcore_bridge/model/gpts/deepseek_v4.py:61-328): the q path (``linear_q_down_proj`` ->
``q_layernorm`` -> ``linear_q_up_proj`` -> per-head weightless RMS norm ``_q_rms_norm``, :140-142),
one shared K = V head (``linear_kv_proj`` -> ``kv_layernorm``, :144-145, 193-198), interleaved RoPE
on the trailing ``qk_pos_emb_head_dim`` of q and kv (:165-190), the inverse RoPE on the rope slice of
the attention output (:287-311), and the grouped output projection (``linear_o_group_proj`` as
``wo_a``, then ``linear_proj``, :313-318).  Its core attention -- sliding window + compressed
entries (CSA: an indexer's top-k of 4-token compressed entries; HCA: every 128-token entry), with a
per-head attention sink (``core_attention.attn_sink``, :443) -- and the compressors (``ape``,
``wkv``, ``wgate``, ``norm``, :447-464) live in megatron-core's dev branch, which is absent here;
they are restated from DeepSeek-V4's published algorithm, whose in-container third-party
restatement is ``transformers/models/deepseek_v4/modeling_deepseek_v4.py`` (DeepseekV4Attention,
the CSA / HCA compressors, the indexer).  ``tests/test_oracle_v4.py`` pins every function here
against that module and against brute force.

Layout: one sequence (or packed documents in ``cu_seqlens``), token-major: ``q [T, H, D]``,
``kv [T, D]`` (the shared head), compressed entries ``[Nc, D]``.  float64 throughout.
"""
from __future__ import annotations

import math
from typing import Optional

import torch

NEG_INF = float("-inf")


def rope_interleaved(x: torch.Tensor, positions: torch.Tensor, inv_freq: torch.Tensor, mscale: float = 1.0,
                     inverse: bool = False) -> torch.Tensor:
    """Interleaved RoPE on the trailing ``2 * len(inv_freq)`` dims of ``x [..., N, D]`` (N tokens at
    ``positions``): pair (2i, 2i+1) rotated by ``positions * inv_freq[i]`` (``-`` that angle when
    ``inverse``), cos / sin scaled by ``mscale``.  The reference gets the same pairing by
    de-interleaving, rotating halves and re-interleaving (deepseek_v4.py:165-190,
    ``mla_rotary_interleaved`` + ``mla_output_remove_interleaving``)."""
    rd = 2 * inv_freq.numel()
    x = x.to(torch.float64)
    ang = positions.to(torch.float64)[:, None] * inv_freq.to(torch.float64)[None]     # [N, rd/2]
    cos, sin = torch.cos(ang) * mscale, torch.sin(ang) * mscale
    if inverse:
        sin = -sin
    shape = [1] * (x.dim() - 2) + [positions.numel(), rd // 2]
    cos, sin = cos.view(shape), sin.view(shape)
    nope, rope = x[..., :-rd], x[..., -rd:]
    a, b = rope[..., 0::2], rope[..., 1::2]
    out = torch.stack((a * cos - b * sin, b * cos + a * sin), dim=-1).flatten(-2)
    return torch.cat([nope, out], dim=-1)


def rms_norm(x: torch.Tensor, weight: Optional[torch.Tensor], eps: float) -> torch.Tensor:
    x = x.to(torch.float64)
    y = x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + eps)
    return y if weight is None else y * weight.to(torch.float64)


def compress_windows(kv: torch.Tensor, gate: torch.Tensor, position_bias: torch.Tensor, norm_w: torch.Tensor,
                     rate: int, eps: float, overlap: bool) -> torch.Tensor:
    """Compressed entries of one sequence (no cache): ``kv``, ``gate [T, C]`` are the compressor's
    two projections, ``position_bias [rate, C]`` its learned bias (the reference's ``ape``).

    Without ``overlap`` (HCA, ``C = D``): entry w = RMSNorm(sum over the window's ``rate`` tokens of
    softmax(gate + bias) * kv) -- the softmax per channel over the window.  With ``overlap`` (CSA,
    ``C = 2 D``): entry w pools ``2 * rate`` slots, the previous window's first halves
    (``[..., :D]``) and this window's second halves (``[..., D:]``); window 0 has no previous one.
    Only complete windows produce entries.  Returns ``[T // rate, D]`` (before RoPE)."""
    T = kv.shape[0]
    n = T // rate
    if n == 0:
        return kv.new_zeros((0, norm_w.numel()), dtype=torch.float64)
    kv = kv[: n * rate].to(torch.float64).view(n, rate, -1)
    g = gate[: n * rate].to(torch.float64).view(n, rate, -1) + position_bias.to(torch.float64)
    if overlap:
        D = kv.shape[-1] // 2
        cur_kv, cur_g = kv[..., D:], g[..., D:]
        prev_kv = torch.zeros_like(cur_kv)
        prev_g = torch.full_like(cur_g, NEG_INF)
        prev_kv[1:], prev_g[1:] = kv[:-1, :, :D], g[:-1, :, :D]
        kv = torch.cat([prev_kv, cur_kv], dim=1)
        g = torch.cat([prev_g, cur_g], dim=1)
    pooled = (kv * torch.softmax(g, dim=1)).sum(dim=1)
    return rms_norm(pooled, norm_w, eps)


def compressed_visible(t: int, rate: int) -> int:
    """Number of compressed entries query t may attend to: entry w covers tokens up to (w+1)*rate - 1,
    so it is visible once t >= (w+1)*rate - 1, i.e. w < (t + 1) // rate."""
    return (t + 1) // rate


def indexer_topk(q_idx: torch.Tensor, comp_k: torch.Tensor, w: torch.Tensor, rate: int, topk: int,
                 scale: float) -> torch.Tensor:
    """The CSA lightning indexer's selection: ``I[t, s] = sum_h w[t,h] * relu(q[t,h] . k[s]) * scale``
    over the visible compressed entries (``s < (t+1)//rate``), top ``min(topk, #entries)`` by score
    (ties to the lower index), ``-1`` for slots past the visible ones.  Returns ``[T, K]`` ascending
    (``-1`` last)."""
    T = q_idx.shape[0]
    nc = comp_k.shape[0]
    K = min(topk, nc)
    out = torch.full((T, max(K, 0)), -1, dtype=torch.int64)
    if nc == 0:
        return out
    sc = (torch.relu(q_idx.to(torch.float64) @ comp_k.to(torch.float64).T) * scale
          * w.to(torch.float64)[..., None]).sum(1)                                      # [T, Nc]
    for t in range(T):
        v = compressed_visible(t, rate)
        if v == 0:
            continue
        row = sc[t, :v]
        order = torch.sort(-row, stable=True).indices[:K]
        sel = torch.sort(order).values
        out[t, : sel.numel()] = sel
    return out


def core_attention(q: torch.Tensor, kv: torch.Tensor, comp: Optional[torch.Tensor], comp_sel: Optional[torch.Tensor],
                   sinks: torch.Tensor, window: int, scale: float, rate: int = 1,
                   cu_seqlens: Optional[torch.Tensor] = None):
    """Hybrid attention core over one shared K = V head with a per-head sink:
    query t attends to the raw rows ``s`` of its document with ``t - window < s <= t`` and, when
    ``comp`` is given, to compressed entries -- the listed ones ``comp_sel[t]`` (CSA; ``-1`` pad) or,
    with ``comp_sel=None``, every visible one (HCA, ``w < (t+1)//rate``); compressed entries are
    indexed per document when ``cu_seqlens`` packs several (each document's entries are a
    contiguous run of ``comp``, in document order).  ``p = exp(a) / (sum exp(a) + exp(sink_h))``,
    ``out = sum p * value`` (value = key).  Returns ``(out [T, H, D], lse_with_sink [T, H])``."""
    T, H, D = q.shape
    cu = [0, T] if cu_seqlens is None else [int(x) for x in cu_seqlens]
    q64, kv64 = q.to(torch.float64), kv.to(torch.float64)
    c64 = comp.to(torch.float64) if comp is not None else None
    out = torch.zeros(T, H, D, dtype=torch.float64)
    lse = torch.zeros(T, H, dtype=torch.float64)
    comp_off = 0
    for a, b in zip(cu[:-1], cu[1:]):
        n_doc_comp = (b - a) // rate if comp is not None else 0
        for t in range(a, b):
            rows = [kv64[s] for s in range(max(a, t - window + 1), t + 1)]
            if comp is not None:
                if comp_sel is None:
                    sel = list(range(compressed_visible(t - a, rate)))
                else:
                    sel = [int(x) for x in comp_sel[t] if int(x) >= 0]
                rows += [c64[comp_off + w] for w in sel]
            keys = torch.stack(rows)                                                   # [n, D]
            logits = (q64[t] @ keys.T) * scale                                         # [H, n]
            full = torch.cat([logits, sinks.to(torch.float64)[:, None]], dim=1)
            l = torch.logsumexp(full, dim=1)
            p = torch.exp(logits - l[:, None])
            out[t] = p @ keys
            lse[t] = l
        comp_off += n_doc_comp
    return out, lse


def attention_layer(x: torch.Tensor, p: dict, cfg: dict, layer_type: str, positions: Optional[torch.Tensor] = None,
                    comp_sel: Optional[torch.Tensor] = None):
    """The DeepSeek-V4 attention layer on one sequence ``x [S, hidden]`` (float64), the reference's
    ``DSv4HybridSelfAttention.forward`` (deepseek_v4.py:214-321) around the core attention above.
    ``p``: ``wq_a, q_norm, wq_b, wkv, kv_norm, wo_a [groups * o_lora_rank, H * D / groups], wo_b,
    sinks`` and, for compressed layers, ``comp_{wkv,wgate,ape,norm}`` and (CSA) the indexer's
    ``idx_{wq_b,weights_proj}`` and ``idx_comp_{wkv,wgate,ape,norm}``.  ``cfg``: ``heads, head_dim,
    rope_dim, window, eps, o_groups, index_heads, index_head_dim, index_topk, rates {csa, hca},
    inv_freq {main, compress}, mscale {main, compress}``.  ``comp_sel`` (CSA) replaces the indexer's
    own selection (for comparisons that must not depend on near-tied index scores).  Returns
    ``[S, hidden]``."""
    S = x.shape[0]
    H, D, G = cfg["heads"], cfg["head_dim"], cfg["o_groups"]
    eps = cfg["eps"]
    pos = torch.arange(S) if positions is None else positions
    rtype = "main" if layer_type == "sliding_attention" else "compress"
    inv_freq, ms = cfg["inv_freq"][rtype], cfg["mscale"][rtype]
    x = x.to(torch.float64)
    q_res = rms_norm(x @ p["wq_a"].double().T, p["q_norm"], eps)
    q = (q_res @ p["wq_b"].double().T).view(S, H, D)
    q = rms_norm(q, None, eps)
    q = rope_interleaved(q.transpose(0, 1), pos, inv_freq, ms).transpose(0, 1)
    kv = rms_norm(x @ p["wkv"].double().T, p["kv_norm"], eps)
    kv = rope_interleaved(kv[None], pos, inv_freq, ms)[0]
    comp = None
    given_sel = comp_sel
    rate = 1
    if layer_type != "sliding_attention":
        csa = layer_type == "compressed_sparse_attention"
        rate = cfg["rates"]["csa" if csa else "hca"]
        comp = compress_windows(x @ p["comp_wkv"].double().T, x @ p["comp_wgate"].double().T, p["comp_ape"],
                                p["comp_norm"], rate, eps, overlap=csa)
        cpos = torch.arange(comp.shape[0]) * rate
        comp = rope_interleaved(comp[None], cpos, inv_freq, ms)[0]
        if csa:
            Di = cfg["index_head_dim"]
            ck = compress_windows(x @ p["idx_comp_wkv"].double().T, x @ p["idx_comp_wgate"].double().T,
                                  p["idx_comp_ape"], p["idx_comp_norm"], rate, eps, overlap=True)
            ck = rope_interleaved(ck[None], cpos, inv_freq, ms)[0]
            qi = (q_res @ p["idx_wq_b"].double().T).view(S, cfg["index_heads"], Di)
            qi = rope_interleaved(qi.transpose(0, 1), pos, inv_freq, ms).transpose(0, 1)
            wi = (x @ p["idx_weights_proj"].double().T) * cfg["index_heads"] ** -0.5
            comp_sel = indexer_topk(qi, ck, wi, rate, cfg["index_topk"], Di ** -0.5) if given_sel is None else given_sel
    o, _ = core_attention(q, kv, comp, comp_sel, p["sinks"], cfg["window"], D ** -0.5, rate)
    o = rope_interleaved(o.transpose(0, 1), pos, inv_freq, ms, inverse=True).transpose(0, 1)
    og = o.reshape(S, G, -1)                                                         # [S, G, H*D/G]
    wo_a = p["wo_a"].double().view(G, -1, og.shape[-1])                              # [G, r, H*D/G]
    o = torch.einsum("sgd,grd->sgr", og, wo_a).reshape(S, -1)
    return o @ p["wo_b"].double().T
