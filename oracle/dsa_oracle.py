"""CPU oracle for the DSA sparse-attention hot path (TEST INFRASTRUCTURE ONLY).

This module is the checker, never the product: only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
import it.  The shipped path (``mcore-bridge_amd``) never calls into it and
raises when its HIP library is missing.

It restates, in float64 PyTorch on the CPU, the arithmetic that
mcore-bridge routes through Megatron-Core's DSA module:

* ``DSAIndexer.forward_with_scores`` (reference ``src/mcore_bridge/patcher.py:326-360``)
  calls ``fused_qk_topk_naive(q, k, weights, index_topk, mask)`` (``patcher.py:358``),
  which lives in the third-party dependency ``megatron-core>=0.16,<0.19``
  (``requirements.txt:1``; 0.17.1 recommended at ``README.md:113``), module
  ``megatron.core.transformer.experimental_attention_variant.dsa``.  That package is
  not vendored under the reference and not installed here, so its published algorithm
  is restated: ``I[t,s] = sum_h w[t,h] * relu(q[t,h,:] . k[s,:]) + mask[t,s]`` followed by
  ``topk(I, min(K, S))``.  The same formula is spelled out by the in-container
  third-party analog ``transformers/models/deepseek_v32/modeling_deepseek_v32.py:240-256``.
* ``DSAttention`` (called from ``src/mcore_bridge/model/modules/multi_latent_attention.py:262-270``)
  runs Megatron's un-fused sparse attention: dense ``q.k`` scores, a ``-inf`` mask that
  is ``0`` only at the top-k indices, the causal ``triu`` mask, fp32 softmax and ``P.V``.
  Restated here in gather form (``sparse_mla_fwd``) and in the dense masked form
  (``sparse_mla_fwd_dense``).  Backward is plain autograd in the reference; restated
  here as the closed-form gradient (``sparse_mla_bwd``).

Layouts follow the build's absorbed MQA-latent form (one shared 576-wide KV row per
token, ``v = kv[:, :512]``), packed THD: ``q [T, H, 576]``, ``kv [T, 576]``,
``idx [T, K]`` of global token ids with ``-1`` padding, ``out [T, H, 512]``,
``lse [T, H]``.  Documents are given by ``cu_seqlens`` (``None`` means one
document of length T); "causal" means key ``s`` is visible from query ``t`` iff
``doc_start(t) <= s <= t``.

Pinning (each function is checked by tests/test_oracle.py against something that is
not its own formula): brute-force loops, the Hadamard invariance of the indexer
(``patcher.py:292-293``), positive homogeneity of ReLU (fp8 scale folding), the HF
third-party indexer, the dense masked form, ``scaled_dot_product_attention`` when
``K >= S``, the MLA absorption identity, autograd/gradcheck for the backward, the
per-document split for varlen and the last prefill row for decode.
"""
from __future__ import annotations

import math
from typing import Optional, Tuple

import torch

NEG_INF = float("-inf")


# --------------------------------------------------------------------------------------
# documents / visibility
# --------------------------------------------------------------------------------------
def doc_bounds(T: int, cu_seqlens: Optional[torch.Tensor]) -> Tuple[torch.Tensor, torch.Tensor]:
    """Per-token ``(doc_start, doc_end)`` from ``cu_seqlens`` ([n+1] int, cu[0]=0, cu[-1]=T)."""
    if cu_seqlens is None:
        cu = torch.tensor([0, T], dtype=torch.int64)
    else:
        cu = cu_seqlens.to(torch.int64).cpu()
    assert int(cu[0]) == 0 and int(cu[-1]) == T, "cu_seqlens must start at 0 and end at T"
    start = torch.empty(T, dtype=torch.int64)
    end = torch.empty(T, dtype=torch.int64)
    for i in range(cu.numel() - 1):
        a, b = int(cu[i]), int(cu[i + 1])
        start[a:b] = a
        end[a:b] = b
    return start, end


def visibility_mask(T: int, cu_seqlens: Optional[torch.Tensor] = None, causal: bool = True) -> torch.Tensor:
    """Boolean ``[T, T]``: True where key s is visible from query t."""
    start, end = doc_bounds(T, cu_seqlens)
    s = torch.arange(T)[None, :]
    vis = (s >= start[:, None]) & (s < end[:, None])
    if causal:
        vis &= s <= torch.arange(T)[:, None]
    return vis


# --------------------------------------------------------------------------------------
# lightning indexer  (fused_qk_topk_naive scoring half, called at patcher.py:358)
# --------------------------------------------------------------------------------------
def indexer_scores(q_idx: torch.Tensor, k_idx: torch.Tensor, w: torch.Tensor,
                   cu_seqlens: Optional[torch.Tensor] = None, causal: bool = True,
                   q_scale: Optional[torch.Tensor] = None, k_scale: Optional[torch.Tensor] = None,
                   mask: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Dense ``[T, T]`` float64 index scores, ``-inf`` where the key is not visible.

    ``I[t,s] = sum_h w[t,h] * relu(qd[t,h,:] . kd[s,:])`` with ``qd = q_idx * q_scale[t,h]``
    and ``kd = k_idx * k_scale[s]`` when fp8 scales are given (per-(token, head) block scale
    for q, per-token scale for k).  ``mask`` (optional ``[T, T]`` additive float) is added
    like the reference's ``mask`` argument of ``fused_qk_topk_naive``.
    """
    T, Hi, Di = q_idx.shape
    qd = q_idx.to(torch.float64)
    kd = k_idx.to(torch.float64)
    if q_scale is not None:
        qd = qd * q_scale.to(torch.float64)[:, :, None]
    if k_scale is not None:
        kd = kd * k_scale.to(torch.float64)[:, None]
    logits = torch.einsum("thd,sd->ths", qd, kd)           # [T, Hi, T]
    scores = (torch.relu(logits) * w.to(torch.float64)[:, :, None]).sum(dim=1)  # [T, T]
    vis = visibility_mask(T, cu_seqlens, causal)
    scores = scores.masked_fill(~vis, NEG_INF)
    if mask is not None:
        scores = scores + mask.to(torch.float64)
    return scores


def indexer_scores_rows(q_idx: torch.Tensor, k_idx: torch.Tensor, w: torch.Tensor, rows,
                        cu_seqlens: Optional[torch.Tensor] = None, causal: bool = True,
                        q_scale: Optional[torch.Tensor] = None,
                        k_scale: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Rows ``rows`` of ``indexer_scores`` (``[len(rows), T]`` float64) without forming the
    ``[T, T]`` matrix: the same sum ``sum_h w[t,h] relu(q[t,h] . k[s])`` for each listed query
    over every key, ``-inf`` where the key is not visible.  For full-size checks of sampled
    queries (costs ``len(rows) * Hi * T * Di``)."""
    T = k_idx.shape[0]
    start, end = doc_bounds(T, cu_seqlens)
    kd = k_idx.to(torch.float64)
    if k_scale is not None:
        kd = kd * k_scale.to(torch.float64)[:, None]
    out = torch.full((len(rows), T), NEG_INF, dtype=torch.float64)
    s = torch.arange(T)
    for i, t in enumerate(int(r) for r in rows):
        qd = q_idx[t].to(torch.float64)
        if q_scale is not None:
            qd = qd * q_scale[t].to(torch.float64)[:, None]
        row = (torch.relu(qd @ kd.T) * w[t].to(torch.float64)[:, None]).sum(0)   # [T]
        vis = (s >= start[t]) & (s < end[t])
        if causal:
            vis &= s <= t
        out[i] = row.masked_fill(~vis, NEG_INF)
    return out


def indexer_scores_bruteforce(q_idx, k_idx, w, cu_seqlens=None, causal=True):
    """Triple loop restatement of ``indexer_scores`` for tiny shapes (pins the einsum)."""
    T, Hi, Di = q_idx.shape
    vis = visibility_mask(T, cu_seqlens, causal)
    out = torch.full((T, T), NEG_INF, dtype=torch.float64)
    q = q_idx.to(torch.float64).tolist()
    k = k_idx.to(torch.float64).tolist()
    ww = w.to(torch.float64).tolist()
    for t in range(T):
        for s in range(T):
            if not vis[t, s]:
                continue
            acc = 0.0
            for h in range(Hi):
                dot = 0.0
                for d in range(Di):
                    dot += q[t][h][d] * k[s][d]
                acc += ww[t][h] * max(dot, 0.0)
            out[t, s] = acc
    return out


# --------------------------------------------------------------------------------------
# top-k  (fused_qk_topk_naive selection half)
# --------------------------------------------------------------------------------------
def topk_reference_order(scores: torch.Tensor, k: int) -> torch.Tensor:
    """Top ``min(k, #finite)`` keys per row ordered by (score desc, index asc); ``-1`` pad.

    This is ``torch.topk(scores, min(k, S))`` with the tie rule made explicit (ties go to
    the lower index) and masked (``-inf``) keys never selected.
    """
    T, S = scores.shape
    kk = min(k, S)
    out = torch.full((T, kk), -1, dtype=torch.int64)
    idx = torch.arange(S)
    for t in range(T):
        row = scores[t]
        fin = torch.isfinite(row)
        cand = idx[fin]
        vals = row[fin]
        # stable sort on (-score, index): sort by index first (already), then stable by -score
        order = torch.sort(-vals, stable=True).indices
        sel = cand[order][:kk]
        out[t, : sel.numel()] = sel
    return out


def topk_indices(scores: torch.Tensor, k: int) -> torch.Tensor:
    """Canonical kernel order: the same selected set as ``topk_reference_order``, ascending
    index, ``-1`` padding at the end."""
    ref = topk_reference_order(scores, k)
    big = torch.iinfo(torch.int64).max
    srt = torch.where(ref < 0, torch.full_like(ref, big), ref).sort(dim=1).values
    return torch.where(srt == big, torch.full_like(srt, -1), srt)


def topk_bruteforce(scores: torch.Tensor, k: int) -> torch.Tensor:
    """Python ``sorted`` restatement of ``topk_indices`` (pins the tie rule)."""
    T, S = scores.shape
    kk = min(k, S)
    out = torch.full((T, kk), -1, dtype=torch.int64)
    for t in range(T):
        items = [(-float(scores[t, s]), s) for s in range(S) if math.isfinite(float(scores[t, s]))]
        items.sort()
        sel = sorted(s for _, s in items[:kk])
        out[t, : len(sel)] = torch.tensor(sel, dtype=torch.int64)
    return out


# --------------------------------------------------------------------------------------
# sparse MLA attention (DSAttention's un-fused sparse attention, caller multi_latent_attention.py:262-270)
# --------------------------------------------------------------------------------------
def sparse_mla_fwd(q: torch.Tensor, kv: torch.Tensor, idx: torch.Tensor, sm_scale: float,
                   d_v: int = 512, chunk: int = 256) -> Tuple[torch.Tensor, torch.Tensor]:
    """Gather-form sparse MQA over the latent KV.

    ``out[t,h] = sum_{j: idx[t,j] >= 0} softmax_j(sm_scale * q[t,h] . kv[idx[t,j]]) kv[idx[t,j], :d_v]``
    and ``lse[t,h] = log sum_j exp(sm_scale * q[t,h] . kv[idx[t,j]])`` (natural log).  A row
    with no valid index yields ``out = 0`` and ``lse = -inf``.
    """
    T, H, D = q.shape
    out = torch.zeros(T, H, d_v, dtype=torch.float64)
    lse = torch.full((T, H), NEG_INF, dtype=torch.float64)
    kv64 = kv.to(torch.float64)
    for a in range(0, T, chunk):
        b = min(T, a + chunk)
        ii = idx[a:b].to(torch.int64)
        valid = ii >= 0
        g = kv64[ii.clamp(min=0)]                               # [c, K, D]
        s = torch.einsum("thd,tkd->thk", q[a:b].to(torch.float64), g) * sm_scale
        s = s.masked_fill(~valid[:, None, :], NEG_INF)
        m = s.amax(dim=-1, keepdim=True)
        m = torch.where(torch.isfinite(m), m, torch.zeros_like(m))
        p = torch.exp(s - m)
        l = p.sum(dim=-1, keepdim=True)
        o = torch.einsum("thk,tkd->thd", p, g[..., :d_v])
        nz = l > 0
        out[a:b] = torch.where(nz, o / torch.where(nz, l, torch.ones_like(l)), torch.zeros_like(o))
        lse[a:b] = torch.where(nz[..., 0], (m + torch.log(l))[..., 0], torch.full_like(l[..., 0], NEG_INF))
    return out, lse


def sparse_mla_fwd_dense(q: torch.Tensor, kv: torch.Tensor, idx: torch.Tensor, sm_scale: float,
                         d_v: int = 512, cu_seqlens: Optional[torch.Tensor] = None,
                         causal: bool = True) -> torch.Tensor:
    """Dense masked restatement of Megatron's un-fused sparse attention.

    Scores for all ``[T, T]`` pairs, an index mask that is ``0`` at the selected keys and
    ``-inf`` elsewhere, plus the causal / document mask, float softmax, then ``P V``.
    Differentiable (used with autograd to pin ``sparse_mla_bwd``).
    """
    T, H, D = q.shape
    sel = torch.zeros(T, T, dtype=torch.bool)
    ii = idx.to(torch.int64)
    rows = torch.arange(T)[:, None].expand_as(ii)
    ok = ii >= 0
    sel[rows[ok], ii[ok]] = True
    sel &= visibility_mask(T, cu_seqlens, causal)
    s = torch.einsum("thd,sd->hts", q, kv) * sm_scale          # [H, T, T]
    s = s.masked_fill(~sel[None], NEG_INF)
    p = torch.softmax(s, dim=-1)
    p = torch.nan_to_num(p, nan=0.0)
    return torch.einsum("hts,sd->thd", p, kv[:, :d_v])


def sparse_mla_bwd(q: torch.Tensor, kv: torch.Tensor, idx: torch.Tensor, out: torch.Tensor,
                   dout: torch.Tensor, lse: torch.Tensor, sm_scale: float, d_v: int = 512,
                   chunk: int = 256) -> Tuple[torch.Tensor, torch.Tensor]:
    """Closed-form gradients of ``sparse_mla_fwd``.

    ``P = exp(sm_scale*S - lse)``, ``dP = dO . V^T``, ``Delta = rowsum(dO * O)``,
    ``dS = P * (dP - Delta)``; ``dQ = sm_scale * dS . K``;
    ``dKV[s] += sm_scale * dS^T Q`` (all 576 columns) ``+ P^T dO`` (first ``d_v`` columns),
    summed over every (query, head) that selected key ``s``.
    """
    T, H, D = q.shape
    q64, kv64 = q.to(torch.float64), kv.to(torch.float64)
    do64, o64 = dout.to(torch.float64), out.to(torch.float64)
    dq = torch.zeros(T, H, D, dtype=torch.float64)
    dkv = torch.zeros(kv.shape[0], D, dtype=torch.float64)
    delta = (do64 * o64).sum(-1)                                    # [T, H]
    for a in range(0, T, chunk):
        b = min(T, a + chunk)
        ii = idx[a:b].to(torch.int64)
        valid = ii >= 0
        ic = ii.clamp(min=0)
        g = kv64[ic]                                               # [c, K, D]
        s = torch.einsum("thd,tkd->thk", q64[a:b], g) * sm_scale
        l = lse[a:b].to(torch.float64)[..., None]
        p = torch.where(valid[:, None, :] & torch.isfinite(l), torch.exp(s - l), torch.zeros_like(s))
        dp = torch.einsum("thv,tkv->thk", do64[a:b], g[..., :d_v])
        ds = p * (dp - delta[a:b, :, None])
        dq[a:b] = sm_scale * torch.einsum("thk,tkd->thd", ds, g)
        contrib = sm_scale * torch.einsum("thk,thd->tkd", ds, q64[a:b])
        contrib[..., :d_v] += torch.einsum("thk,thv->tkv", p, do64[a:b])
        contrib = contrib * valid[..., None]
        dkv.index_add_(0, ic.reshape(-1), contrib.reshape(-1, D))
    return dq, dkv


def sparse_mla_bwd_dkv_rows(q: torch.Tensor, kv: torch.Tensor, idx: torch.Tensor, out: torch.Tensor,
                            dout: torch.Tensor, lse: torch.Tensor, sm_scale: float, keys, d_v: int = 512):
    """``dKV`` rows of the listed keys only, by the closed form of ``sparse_mla_bwd`` restricted to
    the (query, head) pairs that selected each key: ``P = exp(sm_scale*q.kv_s - lse)``,
    ``dS = P*(dO.v_s - Delta)``, ``dKV[s] = sum sm_scale*dS*q + P*dO`` (first ``d_v`` columns).
    Costs O(#selecting queries * H * D) per key, so it runs at full problem sizes."""
    rows = []
    kv64 = kv.to(torch.float64)
    for s in keys:
        hit = (idx.to(torch.int64) == int(s)).any(dim=1).nonzero().flatten().cpu()
        acc = torch.zeros(kv.shape[1], dtype=torch.float64)
        if hit.numel():
            qq = q[hit].to(torch.float64)                              # [n, H, D]
            oo, dd = out[hit].to(torch.float64), dout[hit].to(torch.float64)
            l = lse[hit].to(torch.float64)                             # [n, H]
            sc = torch.einsum("nhd,d->nh", qq, kv64[int(s)]) * sm_scale
            p = torch.where(torch.isfinite(l), torch.exp(sc - l), torch.zeros_like(sc))
            dp = torch.einsum("nhv,v->nh", dd, kv64[int(s), :d_v])
            ds = p * (dp - (dd * oo).sum(-1))
            acc = torch.einsum("nh,nhd->d", ds * sm_scale, qq)
            acc[:d_v] += torch.einsum("nh,nhv->v", p, dd)
        rows.append(acc)
    return torch.stack(rows)


# --------------------------------------------------------------------------------------
# decode (no reference counterpart: the reference has no DSA cache, patcher.py:256)
# --------------------------------------------------------------------------------------
def decode_indexer_scores(q_idx: torch.Tensor, k_cache: torch.Tensor, w: torch.Tensor,
                          cache_offsets: torch.Tensor, cache_lens: torch.Tensor,
                          q_scale=None, k_scale=None) -> torch.Tensor:
    """Per-sequence scores of one new query (position L_b - 1) over its whole cache.

    ``q_idx [B, Hi, Di]``, ``k_cache [sum L, Di]`` (rows ``offset_b .. offset_b + L_b``),
    ``w [B, Hi]`` -> ``[B, max L]`` float64 with ``-inf`` beyond ``L_b``.
    """
    B = q_idx.shape[0]
    Lmax = int(cache_lens.max())
    out = torch.full((B, Lmax), NEG_INF, dtype=torch.float64)
    for b in range(B):
        o, L = int(cache_offsets[b]), int(cache_lens[b])
        kd = k_cache[o:o + L].to(torch.float64)
        if k_scale is not None:
            kd = kd * k_scale[o:o + L].to(torch.float64)[:, None]
        qd = q_idx[b].to(torch.float64)
        if q_scale is not None:
            qd = qd * q_scale[b].to(torch.float64)[:, None]
        lg = qd @ kd.T                                            # [Hi, L]
        out[b, :L] = (torch.relu(lg) * w[b].to(torch.float64)[:, None]).sum(0)
    return out


def sparse_mla_decode(q: torch.Tensor, kv_cache: torch.Tensor, idx: torch.Tensor, sm_scale: float,
                      d_v: int = 512) -> Tuple[torch.Tensor, torch.Tensor]:
    """Decode attention: ``q [B, H, 576]`` over rows ``kv_cache[idx[b]]`` (global cache row
    ids, ``-1`` pad).  Same arithmetic as ``sparse_mla_fwd`` with one query per sequence."""
    return sparse_mla_fwd(q, kv_cache, idx, sm_scale, d_v=d_v, chunk=8)


# --------------------------------------------------------------------------------------
# the reference's own naive compositions, fp32 (the CPU baseline that bench.py times)
# --------------------------------------------------------------------------------------
def naive_fused_qk_topk_fp32(q_sbhd: torch.Tensor, k_sbd: torch.Tensor, w_sbh: torch.Tensor,
                             index_topk: int, mask: Optional[torch.Tensor]):
    """Shape-for-shape fp32 restatement of ``fused_qk_topk_naive(q, k, weights, index_topk, mask)``
    as called at ``patcher.py:358``: materialises ``[S, B, Hi, S]`` logits, then a full-row
    ``topk``.  Returns ``(index_scores [B,S,S], topk_indices [B,S,min(K,S)])``."""
    logits = torch.einsum("sbhd,tbd->sbht", q_sbhd.float(), k_sbd.float())
    scores = (torch.relu(logits) * w_sbh.float().unsqueeze(-1)).sum(dim=2).transpose(0, 1)
    if mask is not None:
        scores = scores + mask
    kk = min(index_topk, scores.shape[-1])
    return scores, scores.topk(kk, dim=-1).indices


def naive_unfused_sparse_attn_fp32(q_sbhd: torch.Tensor, kv_sbd: torch.Tensor, topk_idx: torch.Tensor,
                                   sm_scale: float, d_v: int = 512, q_offset: int = 0) -> torch.Tensor:
    """Shape-for-shape fp32 restatement of Megatron's un-fused sparse attention in the absorbed
    layout: dense ``[B*H, S, S]`` scores, index mask scattered to 0 at ``topk_idx``, causal
    ``triu`` mask, float softmax, ``P V``.  ``q [S,B,H,576]``, ``kv [S,B,576]`` -> ``[S,B,H*d_v]``.
    ``q`` may hold a block of ``R`` consecutive query rows at positions ``q_offset ..`` of the
    ``S`` keys (``topk_idx [B,R,K]``): the same dense rows for a row subset of the problem."""
    R, B, H, D = q_sbhd.shape
    S = kv_sbd.shape[0]
    qf = q_sbhd.float().permute(1, 2, 0, 3)                          # [B, H, R, D]
    kf = kv_sbd.float().permute(1, 0, 2)                             # [B, S, D]
    s = torch.matmul(qf, kf.transpose(1, 2).unsqueeze(1)) * sm_scale  # [B, H, R, S]
    imask = torch.full((B, R, S), NEG_INF)
    imask.scatter_(-1, topk_idx, 0.0)
    imask = imask + torch.triu(torch.full((R, S), NEG_INF), diagonal=1 + q_offset)[None]
    p = torch.softmax(s + imask[:, None], dim=-1)
    o = torch.matmul(p, kf[:, None, :, :d_v])                        # [B, H, R, d_v]
    return o.permute(2, 0, 1, 3).reshape(R, B, H * d_v)


def naive_decode_fp32(q: torch.Tensor, kv_cache: torch.Tensor, q_idx: torch.Tensor, k_cache: torch.Tensor,
                      w: torch.Tensor, cache_lens, index_topk: int, sm_scale: float, d_v: int = 512):
    """Per-sequence fp32 composition of the same two stages for decode (one new query per
    sequence over its cache rows, packed by ``cache_lens``): dense index scores over the whole
    cache, ``topk``, then dense attention restricted to the selected rows.  No reference
    counterpart (the reference has no DSA cache); this is the CPU timing of the decode config.
    Returns ``out [B, H, d_v]`` fp32."""
    outs = []
    off = 0
    for b, L in enumerate(int(x) for x in cache_lens):
        kc = k_cache[off:off + L].float()
        sc = (torch.relu(q_idx[b].float() @ kc.T) * w[b].float()[:, None]).sum(0)        # [L]
        sel = sc.topk(min(index_topk, L)).indices
        g = kv_cache[off:off + L].float()[sel]                                          # [k, 576]
        p = torch.softmax((q[b].float() @ g.T) * sm_scale, dim=-1)                      # [H, k]
        outs.append(p @ g[:, :d_v])
        off += L
    return torch.stack(outs)


# --------------------------------------------------------------------------------------
# fp8 (OCP e4m3fn) quantisation used by config 4
# --------------------------------------------------------------------------------------
E4M3_MAX = 448.0


def quantize_e4m3_rows(x: torch.Tensor):
    """Absmax-per-last-dim quantisation to ``torch.float8_e4m3fn``: ``scale = absmax/448``
    (``1`` for an all-zero row); returns ``(x_fp8, scale)`` with ``x ~= x_fp8 * scale``."""
    amax = x.abs().amax(dim=-1).to(torch.float32)
    scale = torch.where(amax > 0, amax / E4M3_MAX, torch.ones_like(amax))
    xq = (x.to(torch.float32) / scale[..., None]).clamp(-E4M3_MAX, E4M3_MAX).to(torch.float8_e4m3fn)
    return xq, scale


# --------------------------------------------------------------------------------------
# indexer prologue: everything between the indexer's projections and the scores
# (reference DSAIndexer.forward_before_topk + _apply_rope, src/mcore_bridge/patcher.py:245-324,
# with the patched RoPE of src/mcore_bridge/model/modules/transformer_layer.py:227-278)
# --------------------------------------------------------------------------------------
def hadamard_rows(x: torch.Tensor) -> torch.Tensor:
    """Normalised Walsh-Hadamard transform over the last dim (natural / Sylvester order),
    computed in float64: ``rotate_activation`` (upstream Megatron, applied at
    ``patcher.py:292-293``) = ``fast_hadamard_transform.hadamard_transform(x, scale=n**-0.5)``
    of the third-party ``fast_hadamard_transform`` package (absent here; its published
    transform is this one).  Returns float64."""
    n = x.shape[-1]
    assert n & (n - 1) == 0, "power-of-two length"
    y = x.to(torch.float64).clone()
    h = 1
    while h < n:
        y = y.reshape(*y.shape[:-1], n // (2 * h), 2, h)
        a, b = y[..., 0, :], y[..., 1, :]
        y = torch.stack((a + b, a - b), dim=-2).reshape(*x.shape[:-1], n)
        h *= 2
    return y * n ** -0.5


def rotate_half(x: torch.Tensor, rotary_interleaved: bool) -> torch.Tensor:
    """Megatron-Core ``rope_utils._rotate_half`` (third-party megatron-core 0.17.1, absent here):
    half-split ``cat(-x2, x1)`` or, interleaved, pairs ``(x[2i], x[2i+1]) -> (-x[2i+1], x[2i])``."""
    if not rotary_interleaved:
        x1, x2 = torch.chunk(x, 2, dim=-1)
        return torch.cat((-x2, x1), dim=-1)
    x1, x2 = x[..., 0::2], x[..., 1::2]
    return torch.stack((-x2, x1), dim=-1).flatten(start_dim=-2)


def indexer_rope(x: torch.Tensor, freqs: torch.Tensor, mscale: float, deinterleave: bool,
                 rotary_interleaved: bool) -> torch.Tensor:
    """Patched ``_apply_rotary_pos_emb_bshd`` (``transformer_layer.py:240-278``) on the RoPE part
    of an indexer row, in the tensor's own dtype (bf16 rounds after every op like the reference;
    float64 gives the exact rotation).  ``x [..., rot]``, ``freqs [..., rot]`` broadcastable fp32
    angles; ``deinterleave`` = ``dsa_indexer_rotary_interleaved`` (``patcher.py:310-321`` swaps it
    into ``multi_latent_attention``), ``rotary_interleaved`` = ``config.rotary_interleaved``."""
    t = x
    if deinterleave:                                                   # :261-264
        t = torch.cat((t[..., 0::2], t[..., 1::2]), dim=-1)
    cos_ = (torch.cos(freqs) * mscale).to(t.dtype)                     # :268-269
    sin_ = (torch.sin(freqs) * mscale).to(t.dtype)
    return (t * cos_) + (rotate_half(t, rotary_interleaved) * sin_)    # :273


def indexer_prologue(q_lin: torch.Tensor, k_lin: torch.Tensor, w_lin: torch.Tensor, ln_weight: torch.Tensor,
                     ln_bias: torch.Tensor, freqs: torch.Tensor, *, eps: float, mscale: float,
                     deinterleave: bool, rotary_interleaved: bool, rope_dim: int = 64,
                     dtype: torch.dtype = torch.bfloat16):
    """``forward_before_topk`` after its three projections (``patcher.py:268-300``).

    ``q_lin [T, Hi, Di]`` = ``linear_wq_b(qr)``, ``k_lin [T, Di]`` = ``linear_wk(x)``, ``w_lin [T, Hi]``
    = ``linear_weights_proj(x)``, all bf16; ``ln_weight/ln_bias [Di]`` the ``k_norm`` LayerNorm
    (it has a bias, ``gpt_bridge.py:1299-1300``); ``freqs [T, rope_dim]`` fp32 rotary angles of each
    token.  The RoPE part is the first ``Di - rope_dim`` dims (``x_pe``, ``patcher.py:307-309``),
    rotated over ``rope_dim`` angles, which is the whole of it only for ``Di = 2 * rope_dim``.
    Returns ``(q [T, Hi, Di], k [T, Di], w [T, Hi])`` in ``dtype`` with
    ``w = weights * Hi**-0.5 * Di**-0.5`` (``:299-300``; ``softmax_scale = Di**-0.5``).  ``dtype`` is
    the rounding type of every step: bf16 like the reference, float64 for exact checks."""
    T, Hi, Di = q_lin.shape
    assert Di == 2 * rope_dim, "the reference's x_pe split matches its rotation only for Di = 2 * rope_dim"
    bf = dtype
    ln_t = torch.float32 if dtype == torch.bfloat16 else dtype          # LayerNorm math type
    k = torch.nn.functional.layer_norm(k_lin.to(ln_t), (Di,), ln_weight.to(ln_t),
                                       ln_bias.to(ln_t), eps).to(bf)                       # :281-282
    f = freqs.to(torch.float32 if dtype == torch.bfloat16 else dtype)

    def rope(x, fr):
        pe, nope = x[..., :Di - rope_dim], x[..., Di - rope_dim:]
        return torch.cat((indexer_rope(pe, fr, mscale, deinterleave, rotary_interleaved), nope), dim=-1)

    q = rope(q_lin.to(bf), f[:, None, :])                                                  # :275
    k = rope(k, f)                                                                         # :287
    q = hadamard_rows(q).to(bf)                                                            # :292
    k = hadamard_rows(k).to(bf)                                                            # :293
    w = (w_lin.to(bf) * (Hi ** -0.5)) * (Di ** -0.5)                                       # :299-300
    return q, k, w



# --------------------------------------------------------------------------------------
# the reference's un-absorbed layout (what DSAttention receives)
# --------------------------------------------------------------------------------------
def unabsorbed_sparse_attention(query: torch.Tensor, key: torch.Tensor, value: torch.Tensor,
                                topk_idx: torch.Tensor, sm_scale: float) -> torch.Tensor:
    """Megatron's un-fused DSA attention on per-head tensors (``query``/``key [S, B, H, dq]``,
    ``value [S, B, H, dv]``, built at ``multi_latent_attention.py:101-178``), float64: dense
    scores, index mask (0 at ``topk_idx [B, S, K]``, negative = none), causal ``triu`` mask,
    softmax, ``P V``.  Returns ``[S, B, H * dv]``."""
    S, B, H, dq = query.shape
    q = query.double().permute(1, 2, 0, 3)                           # [B, H, S, dq]
    k = key.double().permute(1, 2, 0, 3)
    v = value.double().permute(1, 2, 0, 3)
    s = torch.matmul(q, k.transpose(-1, -2)) * sm_scale              # [B, H, S, S]
    ti = topk_idx.to(torch.int64)
    sel = torch.zeros(B, S, S + 1, dtype=torch.bool)                  # column S takes the padding
    sel.scatter_(-1, torch.where(ti >= 0, ti, S), True)
    m = torch.where(sel[..., :S], 0.0, NEG_INF) + torch.triu(torch.full((S, S), NEG_INF, dtype=torch.float64), diagonal=1)
    p = torch.softmax(s + m[:, None], dim=-1).nan_to_num(0.0)
    o = torch.matmul(p, v)                                           # [B, H, S, dv]
    return o.permute(2, 0, 1, 3).reshape(S, B, -1)


# --------------------------------------------------------------------------------------
# indexer KL loss (model_config.py:204-205 dsa_indexer_loss_coeff / dsa_indexer_use_sparse_loss;
# computed by megatron-core's compute_dsa_indexer_loss, third-party and absent here: restated
# from its published algorithm, the DeepSeek-V3.2 report's indexer objective)
# --------------------------------------------------------------------------------------
KL_EPS = 1e-10


def attention_head_probs(q: torch.Tensor, kv: torch.Tensor, idx: torch.Tensor, lse: torch.Tensor,
                         sm_scale: float) -> torch.Tensor:
    """Target of the sparse indexer loss: ``p[t, j] = (1/H) sum_h exp(sm_scale*q[t,h].kv[idx[t,j]] -
    lse[t,h])`` for valid slots (0 elsewhere): the head-summed attention probabilities of the
    selected keys, L1-normalised (each head's probabilities over the selected keys sum to 1)."""
    T, H, D = q.shape
    ii = idx.to(torch.int64)
    valid = ii >= 0
    g = kv.to(torch.float64)[ii.clamp(min=0)]                          # [T, K, D]
    s = torch.einsum("thd,tkd->thk", q.to(torch.float64), g) * sm_scale
    l = lse.to(torch.float64)[..., None]
    p = torch.where(valid[:, None, :] & torch.isfinite(l), torch.exp(s - l), torch.zeros_like(s))
    return p.sum(1) / H


def indexer_kl_sparse(index_sel: torch.Tensor, target: torch.Tensor, valid: torch.Tensor):
    """Per-row KL of the sparse indexer loss over the selected slots:
    ``KL_t = sum_j p_tj (log(p_tj + eps) - log(softmax(I_t)_j + eps))`` with the index-score
    softmax over valid slots only.  Returns ``(kl [T], d kl_t / d I_t [T, K])``; the gradient of
    ``sum_j p log(pI + eps)`` is ``pI * sum_j(p pI/(pI+eps)) - p pI/(pI+eps)`` per slot."""
    I = index_sel.to(torch.float64).masked_fill(~valid, NEG_INF)
    lp = torch.log_softmax(I, dim=-1)
    pI = torch.where(valid, lp.exp(), torch.zeros_like(lp))
    p = target.to(torch.float64)
    kl = (p * (torch.log(p + KL_EPS) - torch.log(pI + KL_EPS))).masked_fill(~valid, 0.0).sum(-1)
    r = torch.where(valid, p * pI / (pI + KL_EPS), torch.zeros_like(pI))
    grad = pI * r.sum(-1, keepdim=True) - r
    return kl, torch.where(valid, grad, torch.zeros_like(grad))


def indexer_scores_bwd(q_idx: torch.Tensor, k_idx: torch.Tensor, w: torch.Tensor, idx: torch.Tensor,
                       d_scores: torch.Tensor, q_scale=None, k_scale=None):
    """Gradients of ``I[t, j] = sum_h w[t,h] relu(q[t,h] . k[idx[t,j]])`` (the indexer scores of the
    selected slots) given ``dI [T, K]``: ``dq[t,h] = w[t,h] sum_j dI[t,j] 1[z>0] k_j``,
    ``dw[t,h] = sum_j dI[t,j] relu(z)``, ``dk[s] += sum_h dI[t,j] w[t,h] 1[z>0] q[t,h]``.  float64."""
    qd = q_idx.to(torch.float64)
    kd = k_idx.to(torch.float64)
    if q_scale is not None:
        qd = qd * q_scale.to(torch.float64)[..., None]
        kd = kd * k_scale.to(torch.float64)[..., None]
    ii = idx.to(torch.int64)
    valid = ii >= 0
    g = kd[ii.clamp(min=0)]                                            # [T, K, Di]
    z = torch.einsum("thd,tkd->thk", qd, g)
    dI = torch.where(valid, d_scores.to(torch.float64), torch.zeros_like(d_scores, dtype=torch.float64))
    gm = dI[:, None, :] * (z > 0) * w.to(torch.float64)[..., None]     # [T, Hi, K]
    dq = torch.einsum("thk,tkd->thd", gm, g)
    dw = torch.einsum("tk,thk->th", dI, z.clamp(min=0))
    dk = torch.zeros_like(kd)
    contrib = torch.einsum("thk,thd->tkd", gm, qd)
    dk.index_add_(0, ii.clamp(min=0).reshape(-1), (contrib * valid[..., None]).reshape(-1, kd.shape[1]))
    return dq, dk, dw


def compute_dsa_indexer_loss_dense(index_scores: torch.Tensor, topk_indices: torch.Tensor, query: torch.Tensor,
                                   key: torch.Tensor, softmax_scale: float, loss_coeff: float,
                                   sparse_loss: bool) -> torch.Tensor:
    """Shape-for-shape restatement of megatron-core's ``compute_dsa_indexer_loss`` (dense form):
    ``index_scores [B, S, S]`` (with the causal mask added, as ``fused_qk_topk_naive`` returns
    them), ``topk_indices [B, S, K]``, per-head ``query``/``key [S, B, H, d]`` (detached in the
    caller).  Target = head-summed fp32 softmax of the causal (+ index, if ``sparse_loss``)
    masked attention scores, L1-normalised; KL(target || softmax(index_scores)) with 1e-10
    inside the logs, summed over keys, averaged over (b, s), times ``loss_coeff``."""
    S, B, H, d = query.shape
    qf = query.double().permute(1, 2, 0, 3)
    kf = key.double().permute(1, 2, 3, 0)
    att = torch.matmul(qf, kf) * softmax_scale                         # [B, H, S, S]
    causal = torch.triu(torch.full((S, S), NEG_INF, dtype=torch.float64), diagonal=1)
    att = att + causal
    isc = index_scores.double()
    if sparse_loss:
        imask = torch.full((B, S, S), NEG_INF, dtype=torch.float64).scatter_(-1, topk_indices.long(), 0.0)
        att = att + imask[:, None]
        isc = isc + imask
    att = torch.softmax(att, dim=-1)
    isc = torch.softmax(isc, dim=-1)
    att = att.sum(1)
    att = att / att.sum(-1, keepdim=True)
    kl = att * (torch.log(att + KL_EPS) - torch.log(isc + KL_EPS))
    return kl.sum(-1).mean() * loss_coeff
