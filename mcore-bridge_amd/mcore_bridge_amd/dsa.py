"""Megatron-compatible entry points of the DSA hot path (sequence-first ``sbhd`` layouts).

``fused_qk_topk_naive`` keeps the name, argument order, layouts and return values of the
function that reference ``DSAIndexer.forward_with_scores`` imports and calls at
src/mcore_bridge/patcher.py:349-358, so reassigning
``megatron.core.transformer.experimental_attention_variant.dsa.fused_qk_topk_naive`` to it
swaps the implementation without model-code changes (see ``patch.py``).

``sparse_mla_attention`` is the absorbed-layout counterpart of the un-fused sparse attention
that DSAttention runs on the indexer output (call site
src/mcore_bridge/model/modules/multi_latent_attention.py:262-270): one shared 576-wide latent KV
head, ``v = kv[..., :512]``, causal ``triu`` mask applied on top of the index mask.

``absorbed_mla_sparse_attention`` is the same attention for the caller's un-absorbed MLA tensors
(multi_latent_attention.py:101-178 builds ``key_h = [kv_compressed W_UK_h^T, k_pos_emb]`` and
``value_h = kv_compressed W_UV_h^T`` from ``linear_kv_up_proj``): the query is absorbed into the
latent space, the kernel runs on ``[kv_compressed, k_pos_emb]``, ``W_UV`` is applied after.

``indexer_forward_before_topk`` is the indexer's producer, reference
``DSAIndexer.forward_before_topk`` (src/mcore_bridge/patcher.py:245-302): the three projections
run as plain GEMMs (hipBLASLt through torch), everything after them in one fused HIP pass.

All of them run in the HIP kernels of libdsa_amd.so; torch ops here only reshape, cast,
reorder indices and (for the projections) multiply matrices.
"""
from __future__ import annotations

from typing import Optional, Tuple

import torch
from torch import Tensor

from . import ops


def _split_packed(packed_seq_params):
    """The caller's ``(psp, rotary_pos_emb)`` tuple (multi_latent_attention.py:260-261)."""
    if isinstance(packed_seq_params, tuple):
        return packed_seq_params
    return packed_seq_params, None


def _thd_docs(psp):
    """``(cu_seqlens_q int32, max_seqlen_q or None)`` of a packed THD ``PackedSeqParams``, else None."""
    if psp is None or getattr(psp, "qkv_format", "thd") != "thd":
        return None
    cu = psp.cu_seqlens_q
    assert cu is not None, "THD packing needs cu_seqlens_q"
    cu = cu.to(torch.int32)
    ms = getattr(psp, "max_seqlen_q", None)
    return cu, (int(ms) if ms is not None else None)


def _mask_type_is_causal(attn_mask_type) -> bool:
    """DSA attention is causal (DSAttention applies the triu mask on top of the index mask); an
    explicit ``attn_mask_type`` (Megatron's AttnMaskType) must be a causal kind."""
    if attn_mask_type is None:
        return True
    return "causal" in getattr(attn_mask_type, "name", str(attn_mask_type)).lower()


def fused_qk_topk_naive(q: Tensor, k: Tensor, weights: Tensor, index_topk: int,
                        mask: Optional[Tensor] = None, *, causal: Optional[bool] = None,
                        return_scores: bool = True, q_scale: Optional[Tensor] = None,
                        k_scale: Optional[Tensor] = None) -> Tuple[Optional[Tensor], Tensor]:
    """Drop-in for Megatron's ``fused_qk_topk_naive`` (called at reference patcher.py:358).

    ``q [S, B, Hi, Di]``, ``k [S, B, Di]``, ``weights [S, B, Hi]``, ``mask [B, S, S]`` float
    (0 / -inf) or None.  Returns ``(index_scores [B, S, S] fp32, topk_indices [B, S, min(K, S)]
    int64)`` with ``index_scores[b,t,s] = sum_h weights[t,b,h] relu(q[t,b,h] . k[s,b]) + mask``
    and the indices ordered like ``torch.topk`` (score descending) with the tie rule made
    explicit: equal scores -- including the ``-inf`` of masked keys -- go to the lower index.

    A ``mask`` is applied as given: the scores of every key are computed and the mask added, which
    is exact for any additive mask, the causal ``triu`` one included, and never inspects the mask
    on the host.  ``causal=True`` declares the mask to be the causal ``triu`` mask (it is then not
    read) and scores only the visible keys, half the work; ``causal=False`` with no mask scores
    every key.

    Keyword extensions: ``causal``; ``return_scores=False`` skips materialising the ``[B, S, S]``
    scores (first output None); ``q_scale [S, B, Hi]`` / ``k_scale [S, B]`` with float8_e4m3fn
    ``q`` / ``k``.  The bf16 index scores are differentiable in ``q``, ``k`` and ``weights`` (head
    dim 128): autograd through them runs the dense score backward, which is what the reference's
    dense indexer loss (compute_dsa_indexer_loss with the default sparse_loss=False) backpropagates
    through; the indices carry none.
    """
    if (return_scores and q_scale is not None and torch.is_grad_enabled()
            and any(t.requires_grad for t in (q, k, weights))):
        raise NotImplementedError("fused_qk_topk_naive: the fp8 index scores carry no gradient")
    S, B, Hi, Di = q.shape
    kk = min(index_topk, S)
    if causal is None:
        causal = False
    general_mask = mask is not None and not causal
    need_scores = return_scores or general_mask
    scores_out = []
    idx_out = torch.empty(B, S, kk, dtype=torch.int64, device=q.device)
    cu = torch.tensor([0, S], dtype=torch.int32, device=q.device)
    for b in range(B):
        qb, kb, wb = q[:, b].contiguous(), k[:, b].contiguous(), weights[:, b].to(torch.float32).contiguous()
        qs = q_scale[:, b].contiguous() if q_scale is not None else None
        ks = k_scale[:, b].contiguous() if k_scale is not None else None
        base, ln = ops.build_rows(cu, S, bool(causal))
        sc = ops.indexer_scores(qb, kb, wb, base, ln, S, S, qs, ks, need_scores)
        if general_mask:
            sc = sc + mask[b].to(torch.float32)
        idx = ops.topk(sc.detach(), base, ln, kk).to(torch.int64)   # ascending key ids, -1 pad
        pad = idx < 0
        if causal:
            # masked (-inf) keys of row t are t+1, t+2, ...: a stable top-k takes them in order,
            # so the padding slot j holds key j.
            slot = torch.arange(kk, device=q.device).expand_as(idx)
            idx = torch.where(pad, slot, idx)
        # reference order: score descending, ties to the lower index (stable sort of an
        # ascending-index list); padded slots score -inf (the masked tail of `sc` is only
        # written when the scores are returned)
        with torch.no_grad():
            vals = torch.gather(sc, 1, idx.clamp(min=0))
            vals = torch.where(pad, torch.full_like(vals, float("-inf")), vals)
            order = torch.sort(vals, dim=1, descending=True, stable=True).indices
            idx_out[b] = torch.gather(idx, 1, order)
        if return_scores:
            scores_out.append(sc)
    return (torch.stack(scores_out) if return_scores else None), idx_out


def sparse_mla_attention(query: Tensor, kv: Tensor, topk_indices: Tensor, softmax_scale: float,
                         d_v: int = 512, causal: bool = True) -> Tensor:
    """Absorbed sparse MLA attention in Megatron's sequence-first layout.

    ``query [S, B, H, 576]`` bf16, ``kv [S, B, 576]`` bf16 (the shared latent head, ``v =
    kv[..., :d_v]``), ``topk_indices [B, S, K]`` (per-batch key positions; negative = none).
    Returns ``[S, B, H * d_v]`` like the un-fused reference attention; differentiable w.r.t.
    ``query`` and ``kv``.  ``causal`` applies the reference's ``triu`` mask on top of the index
    mask.
    """
    S, B, H, D = query.shape
    assert d_v == ops.D_V and D == ops.D_QK, "absorbed MLA layout: 576-wide q/kv, d_v = 512"
    q_thd = query.transpose(0, 1).reshape(B * S, H, D)
    kv_thd = kv.transpose(0, 1).reshape(B * S, D)
    off = (torch.arange(B, device=query.device, dtype=torch.int64) * S).view(B, 1, 1)
    ti = topk_indices.to(torch.int64)
    idx = torch.where(ti >= 0, ti + off, torch.full_like(ti, -1)).reshape(B * S, -1).to(torch.int32)
    out = ops.sparse_mla(q_thd, kv_thd, idx, softmax_scale, causal)     # [B*S, H, 512]
    return out.reshape(B, S, H * d_v).transpose(0, 1)


def indexer_forward_before_topk(x: Tensor, qr: Tensor, wq_b: Tensor, wk: Tensor, k_norm_weight: Tensor,
                                k_norm_bias: Tensor, weights_proj: Tensor, rotary_pos_emb: Tensor, *,
                                index_n_heads: int, eps: float = 1e-6, mscale: float = 1.0,
                                dsa_indexer_rotary_interleaved: bool = False, rotary_interleaved: bool = False,
                                fp8: bool = False, positions: Optional[Tensor] = None):
    """``DSAIndexer.forward_before_topk(x, qr)`` (reference patcher.py:245-302), sequence-first.

    ``positions`` (optional, ``[S * B]`` int64 on the device) gives each token's row of
    ``rotary_pos_emb`` -- for packed THD input (``[T, 1, ...]``), the token's position inside its
    document, where Megatron's THD RoPE restarts the angles; by default token ``(s, b)`` takes row
    ``s``.

    ``x [S, B, hidden]``, ``qr [S, B, q_lora_rank]`` bf16; the weights of ``linear_wq_b``
    (``[Hi * 128, q_lora_rank]``), ``linear_wk`` (``[128, hidden]``), ``k_norm`` (LayerNorm weight
    and bias ``[128]``) and ``linear_weights_proj`` (``[Hi, hidden]``); ``rotary_pos_emb`` the
    ``[S, 1, 1, 64]`` fp32 angles the caller passes in ``packed_seq_params`` (``:255``);
    ``mscale`` = ``config.attention_scaling`` (``transformer_layer.py:249``).  Returns
    ``(q [S, B, Hi, 128], k [S, B, 128], weights [S, B, Hi])`` like the reference (bf16 q/k, fp32
    weights holding bf16 values) or, with ``fp8``, ``(q, q_scale [S, B, Hi], k, k_scale [S, B],
    weights)`` in the fp8 input layout of ``fused_qk_topk_naive``."""
    S, B, _ = x.shape
    T = S * B
    xb = x.reshape(T, -1)
    qrb = qr.reshape(T, -1)
    q_lin = torch.nn.functional.linear(qrb, wq_b)                       # :271
    k_lin = torch.nn.functional.linear(xb, wk)                          # :281
    w_lin = torch.nn.functional.linear(xb, weights_proj)                # :299
    fr = rotary_pos_emb.reshape(-1, rotary_pos_emb.shape[-1]).to(torch.float32)
    if positions is not None:
        fr = fr[positions]                                              # token -> angles of its position
    else:
        fr = fr[:S, None, :].expand(S, B, fr.shape[-1]).reshape(T, -1)  # token (s, b) -> angles of s
    q, qs, k, ks, w = ops.indexer_prologue(q_lin, k_lin, w_lin, k_norm_weight, k_norm_bias, fr, eps, mscale,
                                           dsa_indexer_rotary_interleaved, rotary_interleaved, fp8)
    q = q.view(S, B, index_n_heads, 128)
    k = k.view(S, B, 128)
    w = w.view(S, B, index_n_heads)
    if fp8:
        return q, qs.view(S, B, index_n_heads), k, ks.view(S, B), w
    return q, k, w


class _IndexerKL(torch.autograd.Function):
    """``coeff * mean_t KL_t`` from per-row KLs and their gradients computed in one kernel pass."""

    @staticmethod
    def forward(ctx, index_sel: Tensor, target: Tensor, idx: Tensor, n_kv: int, causal: bool, coeff: float):
        T = idx.shape[0]
        kl, d = ops.indexer_kl_rows(index_sel, target, idx, n_kv, causal, coeff / max(T, 1))
        ctx.save_for_backward(d)
        return kl.sum() * (coeff / max(T, 1))

    @staticmethod
    def backward(ctx, g: Tensor):
        (d,) = ctx.saved_tensors
        return d * g, None, None, None, None, None


def indexer_kl_loss(q: Tensor, kv: Tensor, lse: Tensor, topk_indices: Tensor, q_idx: Tensor, k_idx: Tensor,
                    w: Tensor, softmax_scale: float, loss_coeff: float, causal: bool = True) -> Tensor:
    """Sparse DSA indexer loss in the packed THD layout (``dsa_indexer_loss_coeff`` with
    ``dsa_indexer_use_sparse_loss``, reference src/mcore_bridge/config/model_config.py:204-205;
    megatron-core's ``compute_dsa_indexer_loss`` restricted to the selected keys).

    ``q [T, H, 576]``, ``kv [N, 576]``, ``lse [T, H]`` are the sparse attention's absorbed inputs
    and forward LSE (``ops.sparse_mla_fwd``; detached, as the reference detaches query and key);
    ``topk_indices [T, K]`` the indexer's selection; ``q_idx [T, Hi, 128]``, ``k_idx [N, 128]``
    bf16 and ``w [T, Hi]`` fp32 the indexer's prologue outputs.  The target is the head-summed
    attention probability of each selected key, L1-normalised; the loss is ``loss_coeff *
    mean_t KL(target_t || softmax(I_t))`` over the selected keys with ``I`` the indexer scores at
    those keys, differentiable in ``q_idx``, ``k_idx`` and ``w``."""
    idx = topk_indices.to(torch.int32)
    with torch.no_grad():
        target = ops.indexer_kl_target(q.detach(), kv.detach(), idx, lse.detach(), softmax_scale, causal)
    index_sel = ops.indexer_selected_scores(q_idx, k_idx, w, idx, causal)
    return _IndexerKL.apply(index_sel, target, idx, k_idx.shape[0], causal, float(loss_coeff))


def indexer_kl_loss_dense(q: Tensor, kv: Tensor, q_idx: Tensor, k_idx: Tensor, w: Tensor, softmax_scale: float,
                          loss_coeff: float, cu_seqlens: Optional[Tensor] = None,
                          max_seqlen: Optional[int] = None) -> Tensor:
    """Dense DSA indexer loss in the packed THD layout: the reference's default
    (``dsa_indexer_loss_coeff > 0`` with ``dsa_indexer_use_sparse_loss = False``, reference
    src/mcore_bridge/config/model_config.py:204-205; megatron-core's ``compute_dsa_indexer_loss``
    with ``sparse_loss=False``).

    The target of query t is the head-mean of its dense causal attention probabilities over EVERY
    visible key of its document (``q [T, H, 576]``, ``kv [N, 576]`` absorbed, detached as the
    reference detaches query and key), and the loss is ``loss_coeff * mean_t KL(target_t ||
    softmax(I_t))`` with ``I`` the index scores of all visible keys -- differentiable in ``q_idx [T,
    Hi, 128]``, ``k_idx [N, 128]`` (bf16) and ``w [T, Hi]`` through the dense score backward.
    ``cu_seqlens`` (int32, device) gives the documents (one document of T tokens by default)."""
    T = q.shape[0]
    if cu_seqlens is None:
        cu_seqlens = torch.tensor([0, T], dtype=torch.int32, device=q.device)
        max_seqlen = T
    if max_seqlen is None:
        max_seqlen = int((cu_seqlens[1:] - cu_seqlens[:-1]).max().item())
    base, ln = ops.build_rows(cu_seqlens.to(torch.int32), T, True)
    pitch = max(4, (max_seqlen + 3) // 4 * 4)
    with torch.no_grad():
        qd, kvd = q.detach(), kv.detach()
        lse = ops.dense_attention_lse(qd, kvd, base, ln, max_seqlen, softmax_scale)
        target = ops.dense_attention_target(qd, kvd, lse, base, ln, max_seqlen, pitch, softmax_scale)
        idx = ops.dense_row_indices(base, ln, 0, pitch)
    scores = ops.indexer_scores(q_idx, k_idx, w, base, ln, max_seqlen, pitch, None, None, True)
    return _IndexerKL.apply(scores, target, idx, k_idx.shape[0], False, float(loss_coeff))


class _AttachIndexerLoss(torch.autograd.Function):
    """``out`` unchanged in the forward; the backward also sends ``loss_scale`` into ``loss`` -- the
    way Megatron's DSAIndexerLossAutoScaler attaches the indexer loss to the attention output, so
    the loss needs no separate backward call."""

    @staticmethod
    def forward(ctx, out: Tensor, loss: Tensor, loss_scale: float):
        ctx.loss_scale = loss_scale
        ctx.loss_meta = (loss.shape, loss.dtype, loss.device)
        return out.view_as(out)

    @staticmethod
    def backward(ctx, g: Tensor):
        shape, dtype, dev = ctx.loss_meta
        return g, torch.full(shape, ctx.loss_scale, dtype=dtype, device=dev), None


def attach_indexer_loss(out: Tensor, loss: Tensor, loss_scale: float = 1.0) -> Tensor:
    """``out`` with ``loss_scale * loss`` applied in its backward (see ``_AttachIndexerLoss``)."""
    return _AttachIndexerLoss.apply(out, loss, float(loss_scale))


class _SparseMLAWithIndexerLoss(torch.autograd.Function):
    """Sparse attention whose backward also applies the sparse indexer KL loss (see
    ``sparse_mla_with_indexer_loss``)."""

    @staticmethod
    def forward(ctx, q, kv, q_idx, k_idx, w, idx, sm_scale, coeff, loss_scale, causal, loss_out):
        out, lse = ops.sparse_mla_fwd(q, kv, idx, sm_scale, causal)
        ctx.save_for_backward(q, kv, q_idx, k_idx, w, idx, out, lse)
        ctx.args = (sm_scale, coeff, loss_scale, causal)
        ctx.loss_out = loss_out
        return out

    @staticmethod
    def backward(ctx, dout):
        q, kv, q_idx, k_idx, w, idx, out, lse = ctx.saved_tensors
        sm_scale, coeff, loss_scale, causal = ctx.args
        T, H = q.shape[0], q.shape[1]
        if ops.backward_takes_one_pass(T, kv.shape[0], H, idx.shape[1], q.device):
            dq, dkv, target = ops.sparse_mla_bwd_with_target(q, kv, idx, out, dout, lse, sm_scale, causal)
        else:
            # a workspace cap applies (set, or the device lacks the one-pass memory) or int8 rows
            # are staged: the capped backward cannot keep the P tiles of every query, so the
            # target is recomputed from the forward LSE instead
            dq, dkv = ops.autograd_backward(q, kv, idx, out, dout, lse, sm_scale, causal)
            target = ops.indexer_kl_target(q, kv, idx, lse, sm_scale, causal)
        sel = ops.indexer_selected_scores(q_idx.detach(), k_idx.detach(), w.detach(), idx, causal)
        kl, d = ops.indexer_kl_rows(sel, target, idx, k_idx.shape[0], causal, coeff * loss_scale / max(T, 1))
        ctx.loss_out.copy_(kl.sum() * (coeff / max(T, 1)))
        dqi = dki = dwi = None
        if any(ctx.needs_input_grad[2:5]):
            dqi, dwi, dki = ops.indexer_scores_bwd(q_idx.detach(), k_idx.detach(), w.detach(), idx, d, causal)
            dqi, dki, dwi = dqi.to(q_idx.dtype), dki.to(k_idx.dtype), dwi.to(w.dtype)
        return dq, dkv.to(kv.dtype), dqi, dki, dwi, None, None, None, None, None, None


def sparse_mla_with_indexer_loss(q: Tensor, kv: Tensor, topk_indices: Tensor, q_idx: Tensor, k_idx: Tensor,
                                 w: Tensor, softmax_scale: float, loss_coeff: float, causal: bool = True,
                                 loss_scale: float = 1.0):
    """Sparse MLA attention (``ops.sparse_mla``, packed THD) whose backward also applies the sparse
    indexer KL loss, the way Megatron's ``DSAIndexerLossAutoScaler`` attaches the indexer loss to
    the attention output: the loss needs no separate backward call.  The target comes from the P
    tiles the attention backward recomputes anyway, so no score product is repeated (the
    forward-time ``indexer_kl_loss`` recomputes it).  Under ``ops.set_backward_workspace_limit``
    (when the one-pass workspace exceeds the cap) or ``ops.set_backward_staging("int8")`` the
    backward runs in capped passes / with int8 rows and recomputes the target from the forward LSE.

    Returns ``(out [T, H, 512], loss)``: ``loss`` is a 0-dim fp32 tensor that holds ``loss_coeff *
    mean_t KL_t`` once the backward pass has run (for logging); the gradients reaching ``q_idx``,
    ``k_idx`` and ``w`` are those of ``loss_scale * loss`` (``loss_scale`` plays the role of the
    auto-scaler's loss scale)."""
    loss = torch.zeros((), dtype=torch.float32, device=q.device)
    idx = topk_indices.to(torch.int32)
    out = _SparseMLAWithIndexerLoss.apply(q, kv, q_idx, k_idx, w, idx, float(softmax_scale), float(loss_coeff),
                                          float(loss_scale), bool(causal), loss)
    return out, loss


def _rows_by_head(x: Tensor, H: int, width: int, lo: int = 0) -> Tensor:
    """``[H, N, width]`` view of the columns ``lo .. lo + width`` of each head's row in ``x`` (rows of
    ``H`` heads, token-major, unit column stride): a strided batch for the library GEMMs, no copy."""
    return x.reshape(-1, H, x.shape[-1])[..., lo:lo + width].permute(1, 0, 2)


class _AbsorbQuery(torch.autograd.Function):
    """``query [S, B, H, dc + dr] = [q_no_pe_h W_UK_h, q_pos_emb]``: the per-head products written
    straight into the query rows (one strided batched GEMM, heads as the batch), the rope part
    copied beside them.  ``w_uk [H, dn, dc]``."""

    @staticmethod
    def forward(ctx, q_no_pe: Tensor, q_pos_emb: Tensor, w_uk: Tensor) -> Tensor:
        S, B, H, dn = q_no_pe.shape
        dc, dr = w_uk.shape[-1], q_pos_emb.shape[-1]
        q_no_pe = q_no_pe.contiguous()
        wk = w_uk.contiguous()
        query = torch.empty(S, B, H, dc + dr, dtype=q_no_pe.dtype, device=q_no_pe.device)
        torch.bmm(_rows_by_head(q_no_pe, H, dn), wk, out=_rows_by_head(query, H, dc))
        query[..., dc:] = q_pos_emb
        ctx.save_for_backward(q_no_pe, wk)
        return query

    @staticmethod
    def backward(ctx, dquery: Tensor):
        q_no_pe, wk = ctx.saved_tensors
        H, dn, dc = wk.shape
        dquery = dquery.contiguous()
        dq_lat = _rows_by_head(dquery, H, dc)                                # [H, N, dc] strided
        d_qn = torch.empty_like(q_no_pe)
        torch.bmm(dq_lat, wk.transpose(1, 2).contiguous(), out=_rows_by_head(d_qn, H, dn))
        d_wk = torch.bmm(_rows_by_head(q_no_pe, H, dn).transpose(1, 2).contiguous(), dq_lat)
        return d_qn, dquery[..., dc:].contiguous(), d_wk


class _AbsorbOutput(torch.autograd.Function):
    """``out [S, B, H * dv]``: each head's latent output row times ``W_UV_h^T`` (``w_uv_t [H, dc,
    dv]``), one strided batched GEMM reading the attention's rows and writing the output rows."""

    @staticmethod
    def forward(ctx, o_lat: Tensor, w_uv_t: Tensor) -> Tensor:
        S, B = o_lat.shape[0], o_lat.shape[1]
        H, dc, dv = w_uv_t.shape
        o_lat = o_lat.contiguous()
        wv = w_uv_t.contiguous()
        out = torch.empty(S, B, H * dv, dtype=o_lat.dtype, device=o_lat.device)
        torch.bmm(_rows_by_head(o_lat.view(S, B, H, dc), H, dc), wv, out=_rows_by_head(out.view(S, B, H, dv), H, dv))
        ctx.save_for_backward(o_lat, wv)
        return out

    @staticmethod
    def backward(ctx, g: Tensor):
        o_lat, wv = ctx.saved_tensors
        H, dc, dv = wv.shape
        S, B = o_lat.shape[0], o_lat.shape[1]
        g = g.contiguous()
        gh = _rows_by_head(g.view(S, B, H, dv), H, dv)                        # [H, N, dv] strided
        d_o = torch.empty_like(o_lat)
        torch.bmm(gh, wv.transpose(1, 2).contiguous(), out=_rows_by_head(d_o.view(S, B, H, dc), H, dc))
        # d W_UV_h^T = o_h^T g_h, formed as (g_h^T o_h)^T: the transposed copy is of the dv-wide rows
        d_wv = torch.bmm(gh.transpose(1, 2).contiguous(), _rows_by_head(o_lat.view(S, B, H, dc), H, dc))
        return d_o, d_wv.transpose(1, 2)


def absorbed_mla_sparse_attention(q_no_pe: Tensor, q_pos_emb: Tensor, kv_compressed: Tensor, k_pos_emb: Tensor,
                                  kv_up_proj_weight: Tensor, topk_indices: Tensor, softmax_scale: float,
                                  causal: bool = True, indexer_loss=None):
    """Megatron's DSA core attention (called at reference multi_latent_attention.py:262-270) on
    the MLA's un-absorbed inputs, computed in the absorbed latent space.

    ``q_no_pe [S, B, H, dn]``, ``q_pos_emb [S, B, H, 64]`` (after RoPE), ``kv_compressed [S, B, 512]``
    (after ``kv_layernorm``), ``k_pos_emb [S, B, 64]`` or ``[S, B, 1, 64]`` (after RoPE), bf16;
    ``kv_up_proj_weight [H * (dn + dv), 512]`` the ``linear_kv_up_proj`` weight (per head ``dn`` rows
    of ``W_UK`` then ``dv`` rows of ``W_UV``, ``:121-128``); ``topk_indices [B, S, K]``.  Returns
    ``[S, B, H * dv]`` -- what the un-fused attention returns for ``query = [q_no_pe, q_pos_emb]``,
    ``key_h = [kv_compressed W_UK_h^T, k_pos_emb]``, ``value_h = kv_compressed W_UV_h^T`` -- and is
    differentiable w.r.t. every tensor input (the weight included).

    ``indexer_loss = (q_idx, k_idx, w, loss_coeff, loss_scale[, sparse[, docs]])`` (the indexer's
    bf16 outputs, ``[S, B, Hi, 128]``, ``[S, B, 128]``, ``[S, B, Hi]``) also applies the indexer KL
    loss in the attention's backward -- the sparse loss (``sparse_mla_with_indexer_loss``, default)
    or, with ``sparse=False``, the dense one (``indexer_kl_loss_dense``; its documents are each
    batch row, or ``docs = (cu_seqlens, max_seqlen)`` for packed THD rows in a batch of one); the
    call then returns ``(out, loss)``."""
    S, B, H, dn = q_no_pe.shape
    dc = kv_compressed.shape[-1]
    assert dc + q_pos_emb.shape[-1] == ops.D_QK and dc == ops.D_V, "latent 512 + rope 64"
    W = kv_up_proj_weight.view(H, -1, dc)
    dv = W.shape[1] - dn
    w_uk = W[:, :dn]                                                   # [H, dn, dc]
    w_uv_t = W[:, dn:].transpose(1, 2)                                 # [H, dc, dv]
    query = _AbsorbQuery.apply(q_no_pe, q_pos_emb, w_uk)               # [S, B, H, dc + 64]
    kv = torch.cat([kv_compressed, k_pos_emb.reshape(S, B, -1)], dim=-1)
    loss = None
    if indexer_loss is None:
        o_lat = sparse_mla_attention(query.contiguous(), kv.contiguous(), topk_indices, softmax_scale, ops.D_V,
                                     causal)
    else:
        q_i, k_i, w_i, coeff, loss_scale = indexer_loss[:5]
        sparse = indexer_loss[5] if len(indexer_loss) > 5 else True
        docs = indexer_loss[6] if len(indexer_loss) > 6 else None
        Hi = q_i.shape[-2]
        off = (torch.arange(B, device=query.device, dtype=torch.int64) * S).view(B, 1, 1)
        ti = topk_indices.to(torch.int64)
        idx = torch.where(ti >= 0, ti + off, torch.full_like(ti, -1)).reshape(B * S, -1).to(torch.int32)
        q_thd = query.transpose(0, 1).reshape(B * S, H, ops.D_QK).contiguous()
        kv_thd = kv.transpose(0, 1).reshape(B * S, ops.D_QK).contiguous()
        qi_thd = q_i.transpose(0, 1).reshape(B * S, Hi, -1)
        ki_thd, wi_thd = k_i.transpose(0, 1).reshape(B * S, -1), w_i.transpose(0, 1).reshape(B * S, Hi)
        if sparse:
            o_thd, loss = sparse_mla_with_indexer_loss(q_thd, kv_thd, idx, qi_thd, ki_thd, wi_thd, softmax_scale,
                                                       coeff, causal, loss_scale)
        else:
            o_thd = ops.sparse_mla(q_thd, kv_thd, idx, softmax_scale, causal)
            if docs is None:
                docs = (torch.arange(0, (B + 1) * S, S, device=query.device, dtype=torch.int32), S)
            loss = indexer_kl_loss_dense(q_thd, kv_thd, qi_thd, ki_thd, wi_thd, softmax_scale, coeff, *docs)
            o_thd = attach_indexer_loss(o_thd, loss, loss_scale)
            loss = loss.detach()
        o_lat = o_thd.reshape(B, S, H * ops.D_V).transpose(0, 1)
    out = _AbsorbOutput.apply(o_lat.reshape(S, B, H * dc), w_uv_t)    # [S, B, H * dv]
    return out if indexer_loss is None else (out, loss)


class _IndexerComputation:
    """The indexer's kernel path over parameters named like Megatron's DSAIndexer: ``linear_wq_b``,
    ``linear_wk``, ``k_norm`` (LayerNorm with bias), ``linear_weights_proj`` (modules with a
    ``.weight``), plus ``index_n_heads``, ``index_topk``, ``eps``, ``mscale``, the two RoPE flags and
    ``fp8``.  Shared by the ``DSAIndexer`` mirror and ``IndexerView`` (an installed Megatron indexer)."""

    def forward_before_topk(self, x: Tensor, qr: Tensor, packed_seq_params=None):
        """``(q [S,B,Hi,Di], k [S,B,Di], weights [S,B,Hi])`` (with fp8: ``(q, q_scale, k, k_scale,
        weights)``); ``packed_seq_params`` is the caller's ``(psp, rotary_pos_emb)`` tuple
        (multi_latent_attention.py:260-261).  Packed THD input gives the token-major layout."""
        psp, rotary_pos_emb = _split_packed(packed_seq_params)
        docs = _thd_docs(psp)
        assert psp is None or docs is not None, "only THD packing is supported"
        with torch.set_grad_enabled(torch.is_grad_enabled() and not self.fp8):
            if docs is None:
                return self._before_topk(x, qr, rotary_pos_emb)
            cu, _ = docs
            T = x.shape[0]
            _, row_len = ops.build_rows(cu, T, True)      # causal row length = position in document + 1
            out = self._before_topk(x.reshape(T, 1, -1), qr.reshape(T, 1, -1), rotary_pos_emb,
                                    positions=row_len.to(torch.int64) - 1)
            return tuple(o.reshape(T, *o.shape[2:]) for o in out)

    def _before_topk(self, x: Tensor, qr: Tensor, rotary_pos_emb: Tensor, positions: Optional[Tensor] = None):
        return indexer_forward_before_topk(
            x, qr, self.linear_wq_b.weight, self.linear_wk.weight, self.k_norm.weight, self.k_norm.bias,
            self.linear_weights_proj.weight, rotary_pos_emb, index_n_heads=self.index_n_heads, eps=self.eps,
            mscale=self.mscale, dsa_indexer_rotary_interleaved=self.dsa_indexer_rotary_interleaved,
            rotary_interleaved=self.rotary_interleaved, fp8=self.fp8, positions=positions)

    def topk_from_outputs(self, out, mask: Optional[Tensor] = None, docs=None, causal: Optional[bool] = None,
                          return_scores: bool = True):
        """Scores and top-k from ``forward_before_topk``'s outputs (sbhd, or THD when ``docs`` =
        ``(cu_seqlens, max_seqlen)``)."""
        if self.fp8:
            q, qs, k, ks, w = out
        else:
            (q, k, w), qs, ks = out, None, None
        if docs is None:
            return fused_qk_topk_naive(q.detach(), k.detach(), w.detach(), self.index_topk, mask, causal=causal,
                                       return_scores=return_scores, q_scale=qs, k_scale=ks)
        cu, max_s = docs
        res = ops.indexer_topk(q.detach(), k.detach(), w.detach(), self.index_topk, cu, True, max_s, qs, ks,
                               return_scores=return_scores)
        idx, sc = res if return_scores else (res, None)
        return sc, idx.to(torch.int64)



class IndexerView(_IndexerComputation):
    """The kernel path over the parameters of an existing indexer module (Megatron's DSAIndexer, or
    any module with its parameter names): shares the module's parameters, copies nothing.  The
    hyper-parameters come from the module where it holds them and from the transformer config
    otherwise (``dsa_indexer_topk``, ``layernorm_epsilon``, ``attention_scaling``,
    ``dsa_indexer_rotary_interleaved``, ``rotary_interleaved``; reference model_config.py:199-206)."""

    def __init__(self, module, config=None, fp8: bool = False):
        def pick(name, cfg_name, default):
            v = getattr(module, name, None)
            if v is None and config is not None:
                v = getattr(config, cfg_name, None)
            return default if v is None else v
        self.linear_wq_b, self.linear_wk = module.linear_wq_b, module.linear_wk
        self.k_norm, self.linear_weights_proj = module.k_norm, module.linear_weights_proj
        self.index_n_heads = pick("index_n_heads", "dsa_indexer_n_heads", None)
        self.index_topk = pick("index_topk", "dsa_indexer_topk", None)
        assert self.index_n_heads is not None and self.index_topk is not None, "indexer heads / top-k unknown"
        self.eps = getattr(module.k_norm, "eps", None) or pick("eps", "layernorm_epsilon", 1e-6)
        self.mscale = pick("mscale", "attention_scaling", 1.0)
        self.dsa_indexer_rotary_interleaved = bool(pick("dsa_indexer_rotary_interleaved",
                                                        "dsa_indexer_rotary_interleaved", False))
        self.rotary_interleaved = bool(pick("rotary_interleaved", "rotary_interleaved", False))
        self.fp8 = fp8


class DSAIndexer(_IndexerComputation, torch.nn.Module):
    """Host mirror of the reference's patched ``DSAIndexer`` (src/mcore_bridge/patcher.py:243-380)
    over the HIP kernels: same method names, arguments and returns, and Megatron's parameter names
    (``linear_wq_b``, ``linear_wk``, ``k_norm``, ``linear_weights_proj``), so the indexer keys the
    reference's bridge maps (``wq_b``, ``wk``, ``k_norm.{weight,bias}``, ``weights_proj``,
    gpt_bridge.py:1292-1306) load one to one.

    Packing: the reference asserts that no ``PackedSeqParams`` is given (patcher.py:256).  This
    mirror also accepts packed THD input (``psp.qkv_format == 'thd'`` with ``cu_seqlens_q``, as the
    MLA caller packs it, multi_latent_attention.py:90-96): ``x [T, 1, hidden]``, ``qr [T, q_lora_rank]``
    (or ``[T, 1, ...]``), RoPE angles restarting at each document, indices restricted to the query's
    own document.  THD outputs are token-major: ``q [T, Hi, 128]``, ``k [T, 128]``, ``w [T, Hi]``,
    ``topk_indices [T, K]`` global token ids (ascending, ``-1`` pad) and ``index_scores [T, max_seqlen]``
    (column j = key ``doc_start + j``, ``-inf`` past the causal row).

    ``forward_before_topk`` is differentiable in the bf16 layout (the prologue's backward kernel,
    then the projections' GEMM backward), which is what training the indexer with the sparse KL
    loss needs: pass its outputs to ``indexer_kl_loss`` (sparse) or ``indexer_kl_loss_dense``.
    ``forward_with_scores`` and ``forward`` run under no_grad, as the reference's indices need no
    gradient; the scores of ``fused_qk_topk_naive`` called with grad enabled are differentiable."""

    def __init__(self, hidden_size: int, q_lora_rank: int, index_n_heads: int = 64, index_head_dim: int = 128,
                 index_topk: int = 2048, qk_pos_emb_head_dim: int = 64, layernorm_epsilon: float = 1e-6,
                 attention_scaling: float = 1.0, dsa_indexer_rotary_interleaved: bool = False,
                 rotary_interleaved: bool = False, fp8: bool = False, device=None, dtype=torch.bfloat16):
        super().__init__()
        assert index_head_dim == 128 and qk_pos_emb_head_dim == 64, "index_head_dim 128, rope 64 (DSv3.2)"
        kw = dict(device=device, dtype=dtype)
        self.index_n_heads, self.index_head_dim, self.index_topk = index_n_heads, index_head_dim, index_topk
        self.eps, self.mscale, self.fp8 = layernorm_epsilon, attention_scaling, fp8
        self.dsa_indexer_rotary_interleaved, self.rotary_interleaved = dsa_indexer_rotary_interleaved, rotary_interleaved
        self.linear_wq_b = torch.nn.Linear(q_lora_rank, index_n_heads * index_head_dim, bias=False, **kw)
        self.linear_wk = torch.nn.Linear(hidden_size, index_head_dim, bias=False, **kw)
        self.k_norm = torch.nn.LayerNorm(index_head_dim, eps=layernorm_epsilon, **kw)
        self.linear_weights_proj = torch.nn.Linear(hidden_size, index_n_heads, bias=False, **kw)

    @torch.no_grad()
    def forward_with_scores(self, x: Tensor, qr: Tensor, mask: Optional[Tensor] = None, packed_seq_params=None):
        """``(index_scores [B,S,S] fp32, topk_indices [B,S,index_topk] int64)`` (patcher.py:326-360);
        THD input: ``(index_scores [T, max_seqlen], topk_indices [T, index_topk])`` (the mask is the
        causal one of each document)."""
        psp, _ = _split_packed(packed_seq_params)
        docs = _thd_docs(psp)
        out = self.forward_before_topk(x, qr, packed_seq_params)
        return self.topk_from_outputs(out, mask, docs)

    def forward(self, x: Tensor, qr: Tensor, mask: Optional[Tensor] = None, packed_seq_params=None) -> Tensor:
        """``topk_indices [B, S, index_topk]`` (patcher.py:362-378), ``[T, index_topk]`` for THD."""
        psp, _ = _split_packed(packed_seq_params)
        docs = _thd_docs(psp)
        with torch.no_grad():
            out = self.forward_before_topk(x, qr, packed_seq_params)
            return self.topk_from_outputs(out, mask, docs, return_scores=False)[1]


class DSAttention(torch.nn.Module):
    """Host mirror of Megatron's ``DSAttention``, the core attention that mcore-bridge's MLA calls
    as ``self.core_attention(query, key, value, attention_mask, packed_seq_params=(psp,
    rotary_pos_emb), attn_mask_type=..., x=..., qr=...)`` (reference
    src/mcore_bridge/model/modules/multi_latent_attention.py:262-270), over the HIP kernels.

    Same forward signature, with the tensors in the kernels' absorbed MQA-latent layout:
    ``query [S, B, H, 576]`` (q_nope absorbed through ``W_UK``, then q_pe) and ``key [S, B, 576]``
    = ``[kv_compressed, k_pos_emb]``, the one latent row every head shares; ``value`` is None
    (V = ``key[..., :512]``).  ``absorbed_mla_sparse_attention`` shows the absorption from the
    caller's un-absorbed tensors.  The composition is Megatron's:
    - the indexer's ``forward_before_topk``;
    - the top-k under the causal mask;
    - sparse attention over the selected keys, with the causal mask on top;
    - in training with ``loss_coeff > 0``, the sparse indexer KL loss, applied in the attention's
      backward. Its value is in ``last_indexer_loss`` after the backward pass.
    Returns ``[S, B, H * 512]``.  Packed THD input (``psp.qkv_format == 'thd'``: ``query [T, H, 576]``,
    ``key [T, 576]``, ``x [T, 1, hidden]``, ``qr [T, q_lora_rank]``) attends within each document
    and returns ``[T, H * 512]``, the un-packed caller's THD output (multi_latent_attention.py:272-281).

    The attention is causal by construction, as DSA's is: ``attention_mask`` is not read (so it
    is never inspected on the host), and ``attn_mask_type``, when given, must be a causal kind.
    ``use_sparse_loss=False`` (the default, as the reference's ``dsa_indexer_use_sparse_loss``,
    model_config.py:205) trains the indexer with the dense loss (``indexer_kl_loss_dense``),
    computed in the forward and applied in the output's backward; ``use_sparse_loss=True`` uses
    the sparse loss (``sparse_mla_with_indexer_loss``)."""

    def __init__(self, indexer: DSAIndexer, softmax_scale: float, loss_coeff: float = 0.0,
                 use_sparse_loss: bool = False):
        super().__init__()
        self.indexer = indexer
        self.softmax_scale = float(softmax_scale)
        self.loss_coeff = float(loss_coeff)
        self.use_sparse_loss = use_sparse_loss
        self.last_indexer_loss: Optional[Tensor] = None

    def forward(self, query: Tensor, key: Tensor, value: Optional[Tensor], attention_mask: Optional[Tensor],
                x: Tensor, qr: Tensor, attn_mask_type=None, attention_bias=None, packed_seq_params=None) -> Tensor:
        assert value is None, "absorbed layout: V is key[..., :512]"
        assert attention_bias is None, "DSA takes no attention bias"
        assert _mask_type_is_causal(attn_mask_type), "DSA attention is causal"
        psp, _ = _split_packed(packed_seq_params)
        docs = _thd_docs(psp)
        train_loss = self.training and self.loss_coeff > 0 and torch.is_grad_enabled()
        if train_loss and self.indexer.fp8:
            raise NotImplementedError("the indexer loss needs the bf16 indexer (the fp8 scores carry no gradient)")
        with torch.set_grad_enabled(train_loss):
            out = self.indexer.forward_before_topk(x, qr, packed_seq_params)
        _, topk = self.indexer.topk_from_outputs(out, None, docs, causal=True, return_scores=False)
        if docs is not None:
            # packed THD: global token ids already, one query row per token
            T, H, D = query.shape
            q_thd, kv_thd = query, key.reshape(T, D)
            idx = topk.to(torch.int32)
        else:
            S, B, H, D = query.shape
            if not train_loss:
                return sparse_mla_attention(query, key, topk, self.softmax_scale, causal=True)
            # packed THD with global key ids (batch b's keys are rows b*S ..)
            q_thd = query.transpose(0, 1).reshape(B * S, H, D)
            kv_thd = key.transpose(0, 1).reshape(B * S, D)
            off = (torch.arange(B, device=query.device, dtype=torch.int64) * S).view(B, 1, 1)
            idx = torch.where(topk >= 0, topk + off, torch.full_like(topk, -1)).reshape(B * S, -1).to(torch.int32)
        if not train_loss:
            return ops.sparse_mla(q_thd.contiguous(), kv_thd.contiguous(), idx, self.softmax_scale, True).reshape(T, -1)
        q_i, k_i, w = out
        Hi = q_i.shape[-2]
        if docs is None:
            q_i, k_i, w = (q_i.transpose(0, 1).reshape(B * S, Hi, -1), k_i.transpose(0, 1).reshape(B * S, -1),
                           w.transpose(0, 1).reshape(B * S, Hi))
        if self.use_sparse_loss:
            o, loss = sparse_mla_with_indexer_loss(q_thd.contiguous(), kv_thd.contiguous(), idx, q_i, k_i, w,
                                                   self.softmax_scale, self.loss_coeff, True)
        else:
            # dense loss (the reference default): over every visible key, computed here and applied in
            # the backward of the output
            if docs is not None:
                cu, max_s = docs
            else:
                cu, max_s = torch.arange(0, (B + 1) * S, S, device=query.device, dtype=torch.int32), S
            o = ops.sparse_mla(q_thd.contiguous(), kv_thd.contiguous(), idx, self.softmax_scale, True)
            loss = indexer_kl_loss_dense(q_thd, kv_thd, q_i, k_i, w, self.softmax_scale, self.loss_coeff, cu, max_s)
            o = attach_indexer_loss(o, loss)
            loss = loss.detach()
        self.last_indexer_loss = loss
        if docs is not None:
            return o.reshape(T, H * ops.D_V)
        return o.reshape(B, S, H * ops.D_V).transpose(0, 1)
