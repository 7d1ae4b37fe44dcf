"""PyTorch custom ops over the C ABI (include/dsa_abi.h).

These are the kernel-native ops in the packed THD layout:
  q [T, H, 576] bf16, kv [N, 576] bf16, idx [T, K] int32 (global kv row ids, -1 pad),
  out [T, H, 512] bf16, lse [T, H] fp32.
PyTorch only supplies device memory (caching allocator) and the current stream; every op
launches the HIP kernels of libdsa_amd.so and raises if a tensor is not on the GPU.  The
Megatron-compatible call signatures (sbhd layouts, ``fused_qk_topk_naive``) are in ``dsa.py``.
"""
from __future__ import annotations

import ctypes
from typing import Optional, Tuple

import torch
from torch import Tensor

from . import _lib

D_QK = 576
D_V = 512


def _p(t: Optional[Tensor]):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else ctypes.c_void_p(0)


def _stream(dev: torch.device):
    return ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)


def _require_gpu(*ts: Optional[Tensor]) -> None:
    for t in ts:
        if t is not None and not t.is_cuda:
            raise RuntimeError(f"dsa_amd ops run on the GPU (gfx950) only; got a tensor on {t.device}")


def _require(cond: bool, msg: str) -> None:
    if not cond:
        raise AssertionError(msg)


# --------------------------------------------------------------------------------------
# row descriptors (documents -> per-query visible key ranges)
# --------------------------------------------------------------------------------------
@torch.library.custom_op("dsa_amd::build_rows", mutates_args=())
def build_rows(cu_seqlens: Tensor, total_q: int, causal: bool) -> Tuple[Tensor, Tensor]:
    """Per-token ``(row_base, row_len)`` int32 from ``cu_seqlens`` (int32, on the GPU)."""
    _require_gpu(cu_seqlens)
    cu = cu_seqlens.to(torch.int32).contiguous()
    base = torch.empty(total_q, dtype=torch.int32, device=cu.device)
    ln = torch.empty(total_q, dtype=torch.int32, device=cu.device)
    with torch.cuda.device(cu.device):
        _lib.call("dsa_build_rows", _p(cu), cu.numel() - 1, total_q, int(causal), _p(base), _p(ln), _stream(cu.device))
    return base, ln


@build_rows.register_fake
def _(cu_seqlens, total_q, causal):
    return (cu_seqlens.new_empty(total_q, dtype=torch.int32), cu_seqlens.new_empty(total_q, dtype=torch.int32))


# --------------------------------------------------------------------------------------
# K0 indexer prologue
# --------------------------------------------------------------------------------------
@torch.library.custom_op("dsa_amd::indexer_prologue", mutates_args=())
def indexer_prologue(q_lin: Tensor, k_lin: Tensor, w_lin: Tensor, ln_weight: Tensor, ln_bias: Tensor,
                     freqs: Tensor, eps: float, mscale: float, deinterleave: bool, rotary_interleaved: bool,
                     fp8: bool = False) -> Tuple[Tensor, Tensor, Tensor, Tensor, Tensor]:
    """The indexer's tail after its projections (reference ``forward_before_topk``,
    patcher.py:268-300): ``k_norm`` LayerNorm of ``k``, partial RoPE of the first 64 dims of q
    and k, the normalised 128-point Hadamard rotation, and the head weights
    ``w * Hi**-0.5 * Di**-0.5`` -- one fused HIP pass.

    ``q_lin [T, Hi, 128]`` (or ``[T, Hi * 128]``), ``k_lin [T, 128]``, ``w_lin [T, Hi]`` bf16;
    ``ln_weight``, ``ln_bias [128]``; ``freqs [T, 64]`` fp32 rotary angles (Megatron's
    ``rotary_pos_emb`` rows); ``deinterleave`` = ``dsa_indexer_rotary_interleaved``,
    ``rotary_interleaved`` = ``config.rotary_interleaved``.  Returns ``(q, q_scale, k, k_scale, w)``:
    bf16 ``q [T, Hi, 128]``, ``k [T, 128]`` (empty scales) or, with ``fp8``, float8_e4m3fn rows
    and their absmax scales ``[T, Hi]``, ``[T]``; ``w [T, Hi]`` fp32."""
    _require_gpu(q_lin, k_lin, w_lin, ln_weight, ln_bias, freqs)
    T = q_lin.shape[0]
    q3 = q_lin.reshape(T, -1, 128)
    Hi = q3.shape[1]
    _require(q_lin.dtype == torch.bfloat16 and k_lin.dtype == torch.bfloat16 and w_lin.dtype == torch.bfloat16,
             "q_lin, k_lin, w_lin must be bf16")
    _require(k_lin.shape == (T, 128) and w_lin.shape == (T, Hi), "k_lin [T, 128], w_lin [T, Hi]")
    if not (q3.stride(2) == 1 and q3.stride(1) == 128):
        q3 = q3.contiguous()
    kl = k_lin if k_lin.stride(1) == 1 else k_lin.contiguous()
    wl = w_lin if w_lin.stride(1) == 1 else w_lin.contiguous()
    fr = freqs.reshape(T, -1).to(torch.float32)
    _require(fr.shape[1] == 64, "freqs must hold 64 angles per token")
    fr = fr if fr.stride(1) == 1 else fr.contiguous()
    lw = ln_weight.to(torch.float32).contiguous()
    lb = ln_bias.to(torch.float32).contiguous()
    odt = torch.float8_e4m3fn if fp8 else torch.bfloat16
    q = torch.empty(T, Hi, 128, dtype=odt, device=q_lin.device)
    k = torch.empty(T, 128, dtype=odt, device=q_lin.device)
    w = torch.empty(T, Hi, dtype=torch.float32, device=q_lin.device)
    qs = torch.empty((T, Hi) if fp8 else (0,), dtype=torch.float32, device=q_lin.device)
    ks = torch.empty((T,) if fp8 else (0,), dtype=torch.float32, device=q_lin.device)
    with torch.cuda.device(q_lin.device):
        _lib.call("dsa_indexer_prologue", _p(q3), q3.stride(0), _p(kl), kl.stride(0), _p(wl), wl.stride(0),
                  _p(lw), _p(lb), _p(fr), fr.stride(0), T, Hi, 128, 64, float(eps), float(mscale),
                  float(Hi ** -0.5), float(128 ** -0.5), int(deinterleave), int(rotary_interleaved),
                  _lib.DSA_FP8_E4M3 if fp8 else _lib.DSA_BF16, _p(q), _p(qs if fp8 else None), _p(k),
                  _p(ks if fp8 else None), _p(w), _stream(q_lin.device))
    return q, qs, k, ks, w


@indexer_prologue.register_fake
def _(q_lin, k_lin, w_lin, ln_weight, ln_bias, freqs, eps, mscale, deinterleave, rotary_interleaved, fp8=False):
    T = q_lin.shape[0]
    Hi = q_lin.numel() // (T * 128) if T else 0
    odt = torch.float8_e4m3fn if fp8 else torch.bfloat16
    return (q_lin.new_empty(T, Hi, 128, dtype=odt), q_lin.new_empty((T, Hi) if fp8 else (0,), dtype=torch.float32),
            q_lin.new_empty(T, 128, dtype=odt), q_lin.new_empty((T,) if fp8 else (0,), dtype=torch.float32),
            q_lin.new_empty(T, Hi, dtype=torch.float32))


@torch.library.custom_op("dsa_amd::indexer_prologue_bwd", mutates_args=())
def indexer_prologue_bwd(dq: Tensor, dk: Tensor, dw: Tensor, k_lin: Tensor, ln_weight: Tensor, freqs: Tensor,
                         eps: float, mscale: float, deinterleave: bool,
                         rotary_interleaved: bool) -> Tuple[Tensor, Tensor, Tensor, Tensor, Tensor]:
    """Backward of the bf16 ``indexer_prologue``: ``(dq_lin [T, Hi, 128], dk_lin [T, 128], dw_lin
    [T, Hi]`` bf16, ``dln_weight, dln_bias [128]`` fp32) from the gradients of its outputs."""
    _require_gpu(dq, dk, dw, k_lin, ln_weight, freqs)
    T, Hi = dw.shape
    dq = dq.float().reshape(T, Hi, 128).contiguous()
    dk = dk.float().contiguous()
    dw = dw.float().contiguous()
    kl = k_lin if k_lin.stride(1) == 1 else k_lin.contiguous()
    fr = freqs.reshape(T, -1).to(torch.float32)
    fr = fr if fr.stride(1) == 1 else fr.contiguous()
    lw = ln_weight.to(torch.float32).contiguous()
    dev = dq.device
    dq_lin = torch.empty(T, Hi, 128, dtype=torch.bfloat16, device=dev)
    dk_lin = torch.empty(T, 128, dtype=torch.bfloat16, device=dev)
    dw_lin = torch.empty(T, Hi, dtype=torch.bfloat16, device=dev)
    dlw = torch.empty(128, dtype=torch.float32, device=dev)
    dlb = torch.empty(128, dtype=torch.float32, device=dev)
    ws_bytes = int(_lib.load().dsa_indexer_prologue_bwd_workspace_size(T))
    ws = torch.empty(ws_bytes // 4, dtype=torch.float32, device=dev)
    with torch.cuda.device(dev):
        _lib.call("dsa_indexer_prologue_bwd", _p(dq), _p(dk), _p(dw), _p(kl), kl.stride(0), _p(lw), _p(fr),
                  fr.stride(0), T, Hi, 128, 64, float(eps), float(mscale), float(Hi ** -0.5), float(128 ** -0.5),
                  int(deinterleave), int(rotary_interleaved), _p(dq_lin), Hi * 128, _p(dk_lin), 128, _p(dw_lin), Hi,
                  _p(dlw), _p(dlb), _p(ws), ws_bytes, _stream(dev))
    return dq_lin, dk_lin, dw_lin, dlw, dlb


@indexer_prologue_bwd.register_fake
def _(dq, dk, dw, k_lin, ln_weight, freqs, eps, mscale, deinterleave, rotary_interleaved):
    T, Hi = dw.shape
    return (dq.new_empty(T, Hi, 128, dtype=torch.bfloat16), dq.new_empty(T, 128, dtype=torch.bfloat16),
            dq.new_empty(T, Hi, dtype=torch.bfloat16), dq.new_empty(128, dtype=torch.float32),
            dq.new_empty(128, dtype=torch.float32))


def _pro_setup(ctx, inputs, output):
    q_lin, k_lin, w_lin, ln_weight, ln_bias, freqs, eps, mscale, deinterleave, rotary_interleaved, fp8 = inputs
    ctx.save_for_backward(k_lin, ln_weight, freqs)
    ctx.args = (eps, mscale, deinterleave, rotary_interleaved)
    ctx.fp8 = fp8
    ctx.shapes = (q_lin.shape, q_lin.dtype, w_lin.dtype, ln_weight.dtype, ln_bias.dtype)


def _pro_backward(ctx, dq, dqs, dk, dks, dw):
    if ctx.fp8:
        raise RuntimeError("indexer_prologue: the fp8 outputs are not differentiable; use the bf16 prologue for "
                           "training")
    k_lin, ln_weight, freqs = ctx.saved_tensors
    qshape, qdt, wdt, lwdt, lbdt = ctx.shapes
    T = k_lin.shape[0]
    Hi = qshape[1] if len(qshape) == 3 else qshape[1] // 128
    dq = torch.zeros(T, Hi, 128, dtype=torch.float32, device=k_lin.device) if dq is None else dq
    dk = torch.zeros(T, 128, dtype=torch.float32, device=k_lin.device) if dk is None else dk
    dw = torch.zeros(T, Hi, dtype=torch.float32, device=k_lin.device) if dw is None else dw
    dq_lin, dk_lin, dw_lin, dlw, dlb = indexer_prologue_bwd(dq, dk, dw, k_lin, ln_weight, freqs, *ctx.args)
    return (dq_lin.reshape(qshape).to(qdt), dk_lin, dw_lin.to(wdt), dlw.to(lwdt), dlb.to(lbdt),
            None, None, None, None, None, None)


torch.library.register_autograd("dsa_amd::indexer_prologue", _pro_backward, setup_context=_pro_setup)


# --------------------------------------------------------------------------------------
# K1 indexer scores
# --------------------------------------------------------------------------------------
@torch.library.custom_op("dsa_amd::indexer_scores", mutates_args=())
def indexer_scores(q: Tensor, k: Tensor, w: Tensor, row_base: Tensor, row_len: Tensor, max_row_len: int,
                   pitch: int, q_scale: Optional[Tensor] = None, k_scale: Optional[Tensor] = None,
                   fill_masked: bool = False) -> Tensor:
    """``scores[t, j] = sum_h w[t,h] relu(q[t,h] . k[row_base[t] + j])`` for ``j < row_len[t]``.

    ``q [T, Hi, Di]``, ``k [N, Di]`` bf16 or float8_e4m3fn (then ``q_scale [T, Hi]`` and
    ``k_scale [N]`` fp32), ``w [T, Hi]``.  Returns fp32 ``[T, pitch]``; columns past ``row_len``
    are ``-inf`` when ``fill_masked`` and unspecified otherwise."""
    _require_gpu(q, k, w, row_base, row_len, q_scale, k_scale)
    T, Hi, Di = q.shape
    fp8 = q.dtype == torch.float8_e4m3fn
    _require(k.dtype == q.dtype and k.dim() == 2 and k.shape[1] == Di, "k must be [N, Di] with q's dtype")
    _require(q.dtype in (torch.bfloat16, torch.float8_e4m3fn), "q must be bf16 or float8_e4m3fn")
    _require(not fp8 or (q_scale is not None and k_scale is not None), "fp8 inputs need q_scale and k_scale")
    q = q.contiguous()
    k = k.contiguous()
    w = w.to(torch.float32).contiguous()
    qs = q_scale.to(torch.float32).contiguous() if fp8 else None
    ks = k_scale.to(torch.float32).contiguous() if fp8 else None
    scores = torch.empty(T, pitch, dtype=torch.float32, device=q.device)
    dt = _lib.DSA_FP8_E4M3 if fp8 else _lib.DSA_BF16
    with torch.cuda.device(q.device):
        _lib.call("dsa_indexer_scores", _p(q), dt, _p(qs), _p(k), dt, _p(ks), _p(w), _p(row_base.contiguous()),
                  _p(row_len.contiguous()), T, k.shape[0], Hi, Di, max_row_len, _p(scores), pitch,
                  int(fill_masked), _stream(q.device))
    return scores


@indexer_scores.register_fake
def _(q, k, w, row_base, row_len, max_row_len, pitch, q_scale=None, k_scale=None, fill_masked=False):
    return q.new_empty(q.shape[0], pitch, dtype=torch.float32)


# --------------------------------------------------------------------------------------
# K2 top-k
# --------------------------------------------------------------------------------------
@torch.library.custom_op("dsa_amd::topk", mutates_args=())
def topk(scores: Tensor, row_base: Tensor, row_len: Tensor, k: int) -> Tensor:
    """Per row the ``min(k, row_len)`` largest scores (ties -> lower key) as ascending key ids
    ``row_base + j``, ``-1`` padded.  int32 ``[rows, k]``."""
    _require_gpu(scores, row_base, row_len)
    _require(scores.dtype == torch.float32 and scores.dim() == 2, "scores must be fp32 [rows, pitch]")
    s = scores if scores.stride(1) == 1 else scores.contiguous()
    rows = s.shape[0]
    out = torch.empty(rows, k, dtype=torch.int32, device=s.device)
    # few long rows (decode) split each row over several workgroups through this workspace
    nws = int(_lib.load().dsa_topk_workspace_size(rows, s.stride(0), k))
    ws = torch.empty(max(nws, 1), dtype=torch.uint8, device=s.device)
    with torch.cuda.device(s.device):
        _lib.call("dsa_topk", _p(s), s.stride(0), _p(row_base.contiguous()), _p(row_len.contiguous()), rows, k,
                  _p(out), ctypes.c_void_p(0), _p(ws) if nws else ctypes.c_void_p(0), nws, _stream(s.device))
    return out


@topk.register_fake
def _(scores, row_base, row_len, k):
    return scores.new_empty(scores.shape[0], k, dtype=torch.int32)


def indexer_topk(q: Tensor, k: Tensor, w: Tensor, index_topk: int, cu_seqlens: Optional[Tensor] = None,
                 causal: bool = True, max_seqlen: Optional[int] = None, q_scale: Optional[Tensor] = None,
                 k_scale: Optional[Tensor] = None, return_scores: bool = False):
    """K1 + K2 over packed documents.  Returns ``idx [T, index_topk]`` int32 (global key ids,
    ascending, ``-1`` pad) and, with ``return_scores``, the fp32 scores ``[T, max_seqlen]``
    (column j <-> key ``doc_start(t) + j``)."""
    T = q.shape[0]
    if cu_seqlens is None:
        cu_seqlens = torch.tensor([0, T], dtype=torch.int32, device=q.device)
        max_seqlen = T
    if max_seqlen is None:
        max_seqlen = int((cu_seqlens[1:] - cu_seqlens[:-1]).max().item())
    base, ln = build_rows(cu_seqlens.to(torch.int32), T, causal)
    pitch = max(4, (max_seqlen + 3) // 4 * 4)
    sc = indexer_scores(q, k, w, base, ln, max_seqlen, pitch, q_scale, k_scale, return_scores)
    idx = topk(sc, base, ln, index_topk)
    return (idx, sc) if return_scores else idx


@torch.library.custom_op("dsa_amd::build_decode_rows", mutates_args=())
def build_decode_rows(cu_cache: Tensor) -> Tuple[Tensor, Tensor]:
    """Per-sequence ``(row_base, row_len)`` int32 of one new token per sequence over its whole
    cache: ``row_base[b] = cu_cache[b]``, ``row_len[b] = cu_cache[b+1] - cu_cache[b]``."""
    _require_gpu(cu_cache)
    cu = cu_cache.to(torch.int32).contiguous()
    B = cu.numel() - 1
    base = torch.empty(B, dtype=torch.int32, device=cu.device)
    ln = torch.empty(B, dtype=torch.int32, device=cu.device)
    with torch.cuda.device(cu.device):
        _lib.call("dsa_build_decode_rows", _p(cu), B, _p(base), _p(ln), _stream(cu.device))
    return base, ln


@build_decode_rows.register_fake
def _(cu_cache):
    B = cu_cache.shape[0] - 1
    return cu_cache.new_empty(B, dtype=torch.int32), cu_cache.new_empty(B, dtype=torch.int32)


def decode_indexer_topk(q: Tensor, k_cache: Tensor, w: Tensor, index_topk: int, cu_cache: Tensor,
                        max_cache_len: Optional[int] = None, q_scale: Optional[Tensor] = None,
                        k_scale: Optional[Tensor] = None, return_scores: bool = False):
    """K1 + K2 for decode: ``q [B, Hi, Di]`` (one new token per sequence), ``k_cache [sum L, Di]``
    packed by ``cu_cache [B+1]``.  Returns ``idx [B, index_topk]`` int32 global cache rows
    (ascending, ``-1`` pad) and, with ``return_scores``, the fp32 scores ``[B, max L]``."""
    if max_cache_len is None:
        max_cache_len = int((cu_cache[1:] - cu_cache[:-1]).max().item())
    base, ln = build_decode_rows(cu_cache)
    pitch = max(4, (max_cache_len + 3) // 4 * 4)
    sc = indexer_scores(q, k_cache, w, base, ln, max_cache_len, pitch, q_scale, k_scale, return_scores)
    idx = topk(sc, base, ln, index_topk)
    return (idx, sc) if return_scores else idx


# --------------------------------------------------------------------------------------
# K3 / K4 sparse MLA
# --------------------------------------------------------------------------------------
def _check_attn(q: Tensor, kv: Tensor, idx: Tensor, q512: bool = False) -> None:
    _require_gpu(q, kv, idx)
    if q512:   # the sink entries also take 512-wide q rows (no rope part) over 576-wide kv rows
        _require(q.dim() == 3 and q.shape[-1] in (D_QK, D_V), f"q must be [T, H, {D_QK}] or [T, H, {D_V}]")
    else:
        _require(q.dim() == 3 and q.shape[-1] == D_QK, f"q must be [T, H, {D_QK}]")
    _require(kv.dim() == 2 and kv.shape[-1] == D_QK, f"kv must be [N, {D_QK}]")
    _require(idx.dim() == 2 and idx.shape[0] == q.shape[0], "idx must be [T, K]")
    _require(q.dtype == torch.bfloat16 and kv.dtype == torch.bfloat16, "q and kv must be bf16")


@torch.library.custom_op("dsa_amd::sparse_mla_fwd", mutates_args=())
def sparse_mla_fwd(q: Tensor, kv: Tensor, idx: Tensor, sm_scale: float, causal: bool = False) -> Tuple[Tensor, Tensor]:
    """Absorbed sparse MLA forward: ``(out [T,H,512] bf16, lse [T,H] fp32)``."""
    _check_attn(q, kv, idx)
    q = q.contiguous()
    kv = kv.contiguous()
    idx = idx.to(torch.int32).contiguous()
    T, H, _ = q.shape
    out = torch.empty(T, H, D_V, dtype=torch.bfloat16, device=q.device)
    lse = torch.empty(T, H, dtype=torch.float32, device=q.device)
    with torch.cuda.device(q.device):
        _lib.call("dsa_sparse_mla_fwd", _p(q), _p(kv), _p(idx), T, kv.shape[0], H, D_QK, D_V, idx.shape[1],
                  float(sm_scale), int(causal), _p(out), _p(lse), _stream(q.device))
    return out, lse


@sparse_mla_fwd.register_fake
def _(q, kv, idx, sm_scale, causal=False):
    T, H, _ = q.shape
    return q.new_empty(T, H, D_V), q.new_empty(T, H, dtype=torch.float32)


@torch.library.custom_op("dsa_amd::sparse_mla_fwd_sink", mutates_args=())
def sparse_mla_fwd_sink(q: Tensor, kv: Tensor, idx: Tensor, sinks: Tensor, sm_scale: float,
                        causal: bool = False) -> Tuple[Tensor, Tensor]:
    """``sparse_mla_fwd`` with a per-head attention sink ``sinks [H]`` (a logit with no value row):
    ``(out [T,H,512] bf16, lse [T,H] fp32)``, the sink counted in the softmax and in ``lse``.
    ``q`` may be ``[T,H,512]`` (no rope part; then ``kv``'s columns 512..575 must be zero)."""
    _check_attn(q, kv, idx, q512=True)
    _require_gpu(sinks)
    q = q.contiguous()
    kv = kv.contiguous()
    idx = idx.to(torch.int32).contiguous()
    T, H, _ = q.shape
    sk = sinks.to(torch.float32).contiguous()
    _require(sk.shape == (H,), "sinks must be [H]")
    out = torch.empty(T, H, D_V, dtype=torch.bfloat16, device=q.device)
    lse = torch.empty(T, H, dtype=torch.float32, device=q.device)
    with torch.cuda.device(q.device):
        _lib.call("dsa_sparse_mla_fwd_sink", _p(q), _p(kv), _p(idx), T, kv.shape[0], H, q.shape[-1], D_V,
                  idx.shape[1], float(sm_scale), int(causal), _p(sk), _p(out), _p(lse), _stream(q.device))
    return out, lse


@sparse_mla_fwd_sink.register_fake
def _(q, kv, idx, sinks, sm_scale, causal=False):
    T, H, _ = q.shape
    return q.new_empty(T, H, D_V), q.new_empty(T, H, dtype=torch.float32)


@torch.library.custom_op("dsa_amd::sparse_mla_bwd_sink", mutates_args=())
def sparse_mla_bwd_sink(q: Tensor, kv: Tensor, idx: Tensor, out: Tensor, dout: Tensor, lse: Tensor, sinks: Tensor,
                        sm_scale: float, causal: bool = False) -> Tuple[Tensor, Tensor, Tensor]:
    """Gradients of ``sparse_mla_fwd_sink`` from its ``out`` and ``lse``: ``(dq`` (bf16, the shape of
    ``q``: ``[T,H,576]`` or ``[T,H,512]``), ``dkv [N,576] fp32, dsinks [H] fp32)``.  One pass, or the capped passes of
    ``set_backward_workspace_limit``; dKV partial rows staged as ``set_backward_staging`` says."""
    _check_attn(q, kv, idx, q512=True)
    _require_gpu(out, dout, lse, sinks)
    q, kv, out, lse = q.contiguous(), kv.contiguous(), out.contiguous(), lse.contiguous()
    dout = dout.to(torch.bfloat16).contiguous()
    idx = idx.to(torch.int32).contiguous()
    T, H, _ = q.shape
    N, K = kv.shape[0], idx.shape[1]
    sk = sinks.to(torch.float32).contiguous()
    dq = torch.empty_like(q)
    dkv = torch.empty(N, D_QK, dtype=torch.float32, device=q.device)
    dsk = torch.empty(H, dtype=torch.float32, device=q.device)
    lib = _lib.load()
    g_int8 = _BWD_G_INT8[0]
    flags = DSA_BWD_G_INT8 if g_int8 else 0
    ws_bytes = int(lib.dsa_sparse_mla_bwd_sink_workspace_size(T, N, H, K, flags))
    cap = _workspace_cap(_BWD_WORKSPACE_LIMIT[0], ws_bytes, q.device)
    if 0 < cap < ws_bytes:
        dbytes = (T * H * 4 + 255) // 256 * 256
        ws_bytes = max(cap, bwd_workspace_bytes_chunked(T, N, H, K, 256, g_int8) + dbytes)
    ws = torch.empty(max(ws_bytes, 256), dtype=torch.uint8, device=q.device)
    with torch.cuda.device(q.device):
        _lib.call("dsa_sparse_mla_bwd_sink", _p(q), _p(kv), _p(idx), _p(out), _p(dout), _p(lse), _p(sk), T, N, H,
                  q.shape[-1], D_V, K, float(sm_scale), int(causal), _p(dq), _p(dkv), _p(dsk), flags, _p(ws), ws.numel(),
                  _stream(q.device))
    return dq, dkv, dsk


@sparse_mla_bwd_sink.register_fake
def _(q, kv, idx, out, dout, lse, sinks, sm_scale, causal=False):
    return (torch.empty_like(q), kv.new_empty(kv.shape[0], D_QK, dtype=torch.float32),
            sinks.new_empty(q.shape[1], dtype=torch.float32))


def decode_workspace_bytes(batch: int, n_heads: int, topk_: int) -> int:
    return int(_lib.load().dsa_sparse_mla_decode_workspace_size(batch, n_heads, topk_))


@torch.library.custom_op("dsa_amd::sparse_mla_decode", mutates_args=())
def sparse_mla_decode(q: Tensor, kv_cache: Tensor, idx: Tensor, sm_scale: float) -> Tuple[Tensor, Tensor]:
    """Decode attention of one new token per sequence: ``q [B,H,576]`` over its selected rows
    of ``kv_cache [N,576]`` (``idx [B,K]`` global rows).  ``(out [B,H,512] bf16, lse [B,H])``."""
    _check_attn(q, kv_cache, idx)
    q = q.contiguous()
    kv_cache = kv_cache.contiguous()
    idx = idx.to(torch.int32).contiguous()
    B, H, _ = q.shape
    K = idx.shape[1]
    out = torch.empty(B, H, D_V, dtype=torch.bfloat16, device=q.device)
    lse = torch.empty(B, H, dtype=torch.float32, device=q.device)
    ws_bytes = decode_workspace_bytes(B, H, K)
    ws = torch.empty(max(ws_bytes, 16), dtype=torch.uint8, device=q.device)
    with torch.cuda.device(q.device):
        _lib.call("dsa_sparse_mla_decode", _p(q), _p(kv_cache), _p(idx), B, kv_cache.shape[0], H, D_QK, D_V, K,
                  float(sm_scale), _p(out), _p(lse), _p(ws), ws_bytes, _stream(q.device))
    return out, lse


@sparse_mla_decode.register_fake
def _(q, kv_cache, idx, sm_scale):
    B, H, _ = q.shape
    return q.new_empty(B, H, D_V), q.new_empty(B, H, dtype=torch.float32)


DSA_BWD_G_INT8 = 1   # include/dsa_abi.h


def bwd_workspace_bytes(total_q: int, n_kv: int, n_heads: int, topk_: int, g_int8: bool = False) -> int:
    flags = DSA_BWD_G_INT8 if g_int8 else 0
    return int(_lib.load().dsa_sparse_mla_bwd_workspace_size_ex(total_q, n_kv, n_heads, topk_, 0, flags))


def bwd_workspace_bytes_chunked(total_q: int, n_kv: int, n_heads: int, topk_: int, chunk_q: int,
                                g_int8: bool = False) -> int:
    flags = DSA_BWD_G_INT8 if g_int8 else 0
    return int(_lib.load().dsa_sparse_mla_bwd_workspace_size_ex(total_q, n_kv, n_heads, topk_, max(1, chunk_q),
                                                                 flags))


@torch.library.custom_op("dsa_amd::sparse_mla_bwd", mutates_args=())
def sparse_mla_bwd(q: Tensor, kv: Tensor, idx: Tensor, out: Tensor, dout: Tensor, lse: Tensor, sm_scale: float,
                   causal: bool = False, max_workspace_bytes: int = 0, g_int8: bool = False) -> Tuple[Tensor, Tensor]:
    """Gradients of ``sparse_mla_fwd``: ``(dq [T,H,576] bf16, dkv [N,576] fp32)``.
    ``max_workspace_bytes`` > 0 caps the scratch memory: the backward then runs in passes of as
    many query rows as fit (at least 256), adding each pass's dkv into the previous ones.  With 0
    it runs one pass if that workspace fits 90 % of the memory the device can still allocate, and
    passes under that share otherwise.
    ``g_int8`` stages the per-pair dkv partial rows as int8 with a bf16 scale per 32 dims
    (``DSA_BWD_G_INT8``): less memory traffic and workspace, a larger dkv rounding error."""
    _check_attn(q, kv, idx)
    _require_gpu(out, dout, lse)
    q, kv, out, lse = q.contiguous(), kv.contiguous(), out.contiguous(), lse.contiguous()
    dout = dout.to(torch.bfloat16).contiguous()
    idx = idx.to(torch.int32).contiguous()
    T, H, _ = q.shape
    N, K = kv.shape[0], idx.shape[1]
    dq = torch.empty_like(q)
    dkv = torch.empty(N, D_QK, dtype=torch.float32, device=q.device)
    ws_bytes = bwd_workspace_bytes(T, N, H, K, g_int8)
    cap = _workspace_cap(int(max_workspace_bytes), ws_bytes, q.device)
    if 0 < cap < ws_bytes:
        ws_bytes = max(cap, bwd_workspace_bytes_chunked(T, N, H, K, 256, g_int8))
    ws = torch.empty(max(ws_bytes, 16), dtype=torch.uint8, device=q.device)
    with torch.cuda.device(q.device):
        _lib.call("dsa_sparse_mla_bwd_ex", _p(q), _p(kv), _p(idx), _p(out), _p(dout), _p(lse), T, N, H, D_QK, D_V,
                  K, float(sm_scale), int(causal), _p(dq), _p(dkv), DSA_BWD_G_INT8 if g_int8 else 0, _p(ws),
                  ws_bytes, None, _stream(q.device))
    return dq, dkv


@sparse_mla_bwd.register_fake
def _(q, kv, idx, out, dout, lse, sm_scale, causal=False, max_workspace_bytes=0, g_int8=False):
    return torch.empty_like(q), kv.new_empty(kv.shape[0], D_QK, dtype=torch.float32)


@torch.library.custom_op("dsa_amd::sparse_mla_bwd_with_target", mutates_args=())
def sparse_mla_bwd_with_target(q: Tensor, kv: Tensor, idx: Tensor, out: Tensor, dout: Tensor, lse: Tensor,
                               sm_scale: float, causal: bool = False) -> Tuple[Tensor, Tensor, Tensor]:
    """``sparse_mla_bwd`` plus the sparse indexer loss target ``[T, K]`` fp32, read from the P tiles
    the backward stages (head mean of P; no S recompute)."""
    _check_attn(q, kv, idx)
    _require_gpu(out, dout, lse)
    q, kv, out, lse = q.contiguous(), kv.contiguous(), out.contiguous(), lse.contiguous()
    dout = dout.to(torch.bfloat16).contiguous()
    idx = idx.to(torch.int32).contiguous()
    T, H, _ = q.shape
    N, K = kv.shape[0], idx.shape[1]
    dq = torch.empty_like(q)
    dkv = torch.empty(N, D_QK, dtype=torch.float32, device=q.device)
    tgt = torch.empty(T, K, dtype=torch.float32, device=q.device)
    ws_bytes = bwd_workspace_bytes(T, N, H, K)
    ws = torch.empty(max(ws_bytes, 16), dtype=torch.uint8, device=q.device)
    with torch.cuda.device(q.device):
        _lib.call("dsa_sparse_mla_bwd", _p(q), _p(kv), _p(idx), _p(out), _p(dout), _p(lse), T, N, H, D_QK, D_V, K,
                  float(sm_scale), int(causal), _p(dq), _p(dkv), _p(ws), ws_bytes, _stream(q.device))
        _lib.call("dsa_indexer_kl_target_from_bwd", _p(ws), ws_bytes, _p(idx), T, N, H, K, int(causal), _p(tgt),
                  _stream(q.device))
    return dq, dkv, tgt


@sparse_mla_bwd_with_target.register_fake
def _(q, kv, idx, out, dout, lse, sm_scale, causal=False):
    return (torch.empty_like(q), kv.new_empty(kv.shape[0], D_QK, dtype=torch.float32),
            q.new_empty(q.shape[0], idx.shape[1], dtype=torch.float32))


def _fwd_setup(ctx, inputs, output):
    q, kv, idx, sm_scale, causal = inputs
    out, lse = output
    ctx.save_for_backward(q, kv, idx, out, lse)
    ctx.sm_scale = sm_scale
    ctx.causal = causal


_BWD_WORKSPACE_LIMIT = [0]
_BWD_G_INT8 = [False]


def set_backward_workspace_limit(nbytes: int) -> None:
    """Cap the scratch memory of the autograd backward of ``sparse_mla_fwd`` (0 = one pass over all
    query rows, the fastest, whenever its workspace fits the memory the device can still give;
    otherwise passes of as many rows as fit, at least 256)."""
    _BWD_WORKSPACE_LIMIT[0] = max(0, int(nbytes))


# share of the allocatable device memory an uncapped backward takes for its workspace before it
# switches to passes (the rest stays for the allocator's rounding and the caller's tensors)
_AUTO_CAP_SHARE = 0.9


def available_device_bytes(device: torch.device) -> int:
    """Bytes a new allocation on ``device`` can take: the driver's free memory plus what torch's
    caching allocator holds reserved but unused."""
    free, _ = torch.cuda.mem_get_info(device)
    return int(free + torch.cuda.memory_reserved(device) - torch.cuda.memory_allocated(device))


def _workspace_cap(limit: int, one_pass_bytes: int, device: torch.device) -> int:
    """The cap a backward runs under: ``limit`` when set (> 0); with no limit, 0 (one pass) if the
    one-pass workspace fits ``_AUTO_CAP_SHARE`` of the allocatable memory, else that share."""
    if limit > 0:
        return limit
    budget = int(available_device_bytes(device) * _AUTO_CAP_SHARE)
    return 0 if one_pass_bytes <= budget else max(budget, 1)


def set_backward_staging(g_rows: str) -> None:
    """Format of the per-pair dkv partial rows the autograd backward of ``sparse_mla_fwd`` stages:
    ``"bf16"`` (the default) or ``"int8"`` (a bf16 scale per 32 dims: ~45% less of the backward's
    largest memory traffic and workspace; dkv normalised error ~0.5% instead of ~0.16%, dq
    unchanged).  ``sparse_mla_bwd_with_target`` (the indexer loss's target from the backward's P
    tiles) always stages bf16 rows; the fused attention + indexer loss backward
    (``dsa.sparse_mla_with_indexer_loss``) therefore switches to ``autograd_backward`` plus a
    recomputed target when int8 rows are chosen or the one-pass workspace exceeds the cap."""
    if g_rows not in ("bf16", "int8"):
        raise ValueError(f"g_rows must be 'bf16' or 'int8', got {g_rows!r}")
    _BWD_G_INT8[0] = g_rows == "int8"


def backward_takes_one_pass(total_q: int, n_kv: int, n_heads: int, topk_: int,
                            device: Optional[torch.device] = None) -> bool:
    """True when the settings of ``set_backward_workspace_limit`` and ``set_backward_staging``
    admit the one-pass bf16-row backward (whose workspace ``sparse_mla_bwd_with_target`` needs);
    with no limit set and a ``device`` given, only if that workspace fits its free memory."""
    if _BWD_G_INT8[0]:
        return False
    ws = bwd_workspace_bytes(total_q, n_kv, n_heads, topk_)
    limit = _BWD_WORKSPACE_LIMIT[0]
    if limit == 0 and device is not None:
        limit = _workspace_cap(0, ws, device)
    return limit == 0 or ws <= limit


def autograd_backward(q: Tensor, kv: Tensor, idx: Tensor, out: Tensor, dout: Tensor, lse: Tensor, sm_scale: float,
                      causal: bool) -> Tuple[Tensor, Tensor]:
    """``sparse_mla_bwd`` with the settings of ``set_backward_workspace_limit`` and
    ``set_backward_staging``: what every autograd backward over these kernels calls."""
    return sparse_mla_bwd(q, kv, idx, out, dout, lse, sm_scale, causal, _BWD_WORKSPACE_LIMIT[0], _BWD_G_INT8[0])


def _fwd_backward(ctx, dout, dlse):
    q, kv, idx, out, lse = ctx.saved_tensors
    dq, dkv = autograd_backward(q, kv, idx, out, dout, lse, ctx.sm_scale, ctx.causal)
    return dq, dkv.to(kv.dtype), None, None, None


torch.library.register_autograd("dsa_amd::sparse_mla_fwd", _fwd_backward, setup_context=_fwd_setup)


def sparse_mla(q: Tensor, kv: Tensor, idx: Tensor, sm_scale: float, causal: bool = False) -> Tensor:
    """Differentiable sparse MLA attention output ``[T, H, 512]``."""
    return sparse_mla_fwd(q, kv, idx, sm_scale, causal)[0]


# --------------------------------------------------------------------------------------
# indexer KL loss: target, per-row KL + gradient, selected-slot scores and their backward
# --------------------------------------------------------------------------------------
@torch.library.custom_op("dsa_amd::indexer_kl_target", mutates_args=())
def indexer_kl_target(q: Tensor, kv: Tensor, idx: Tensor, lse: Tensor, sm_scale: float, causal: bool = True) -> Tensor:
    """Head-averaged attention probability of every selected key, ``[T, K]`` fp32 (0 at invalid
    slots), recomputed from the sparse forward's ``lse``: the target of the sparse indexer loss."""
    _check_attn(q, kv, idx)
    _require_gpu(lse)
    q, kv, lse = q.contiguous(), kv.contiguous(), lse.float().contiguous()
    idx = idx.to(torch.int32).contiguous()
    T, H, _ = q.shape
    _require(lse.shape == (T, H), "lse must be [T, H]")
    tgt = torch.empty(T, idx.shape[1], dtype=torch.float32, device=q.device)
    with torch.cuda.device(q.device):
        _lib.call("dsa_indexer_kl_target", _p(q), _p(kv), _p(idx), _p(lse), T, kv.shape[0], H, D_QK, idx.shape[1],
                  float(sm_scale), int(causal), _p(tgt), _stream(q.device))
    return tgt


@indexer_kl_target.register_fake
def _(q, kv, idx, lse, sm_scale, causal=True):
    return q.new_empty(q.shape[0], idx.shape[1], dtype=torch.float32)


@torch.library.custom_op("dsa_amd::indexer_kl_rows", mutates_args=())
def indexer_kl_rows(index_sel: Tensor, target: Tensor, idx: Tensor, n_kv: int, causal: bool,
                    grad_scale: float) -> Tuple[Tensor, Tensor]:
    """Per-query KL of the sparse indexer loss, ``kl [T]``, and ``grad_scale * d kl_t / d index_sel``
    ``[T, K]`` (softmax of the index scores over the valid slots; 1e-10 inside both logs)."""
    _require_gpu(index_sel, target, idx)
    index_sel, target = index_sel.float().contiguous(), target.float().contiguous()
    idx = idx.to(torch.int32).contiguous()
    T, K = idx.shape
    _require(index_sel.shape == (T, K) and target.shape == (T, K), "index_sel and target must be [T, K]")
    kl = torch.empty(T, dtype=torch.float32, device=idx.device)
    d = torch.empty(T, K, dtype=torch.float32, device=idx.device)
    with torch.cuda.device(idx.device):
        _lib.call("dsa_indexer_kl_loss", _p(index_sel), _p(target), _p(idx), T, int(n_kv), K, int(causal),
                  float(grad_scale), _p(kl), _p(d), _stream(idx.device))
    return kl, d


@indexer_kl_rows.register_fake
def _(index_sel, target, idx, n_kv, causal, grad_scale):
    T, K = idx.shape
    return idx.new_empty(T, dtype=torch.float32), idx.new_empty(T, K, dtype=torch.float32)


def _check_idx_sel(q: Tensor, k: Tensor, w: Tensor, idx: Tensor) -> None:
    _require_gpu(q, k, w, idx)
    _require(q.dim() == 3 and q.shape[-1] == 128 and q.dtype == torch.bfloat16, "q must be [T, Hi, 128] bf16")
    _require(k.dim() == 2 and k.shape[-1] == 128 and k.dtype == torch.bfloat16, "k must be [N, 128] bf16")
    _require(w.shape == q.shape[:2], "w must be [T, Hi]")
    _require(idx.dim() == 2 and idx.shape[0] == q.shape[0], "idx must be [T, K]")


@torch.library.custom_op("dsa_amd::indexer_selected_scores", mutates_args=())
def indexer_selected_scores(q: Tensor, k: Tensor, w: Tensor, idx: Tensor, causal: bool = True) -> Tensor:
    """Indexer scores of the selected slots, ``sum_h w[t,h] relu(q[t,h] . k[idx[t,j]])`` ``[T, K]``
    fp32 (-inf at invalid slots); differentiable in q, k and w."""
    _check_idx_sel(q, k, w, idx)
    q, k, w = q.contiguous(), k.contiguous(), w.float().contiguous()
    idx = idx.to(torch.int32).contiguous()
    T, Hi, _ = q.shape
    sc = torch.empty(T, idx.shape[1], dtype=torch.float32, device=q.device)
    with torch.cuda.device(q.device):
        _lib.call("dsa_indexer_selected_scores", _p(q), _p(k), _p(w), _p(idx), T, k.shape[0], Hi, 128,
                  idx.shape[1], int(causal), _p(sc), _stream(q.device))
    return sc


@indexer_selected_scores.register_fake
def _(q, k, w, idx, causal=True):
    return q.new_empty(q.shape[0], idx.shape[1], dtype=torch.float32)


def indexer_scores_bwd_workspace_bytes(total_q: int, n_k: int, topk_: int) -> int:
    return int(_lib.load().dsa_indexer_scores_bwd_workspace_size(total_q, n_k, topk_))


@torch.library.custom_op("dsa_amd::indexer_scores_bwd", mutates_args=())
def indexer_scores_bwd(q: Tensor, k: Tensor, w: Tensor, idx: Tensor, d_scores: Tensor,
                       causal: bool = True) -> Tuple[Tensor, Tensor, Tensor]:
    """Gradients of ``indexer_selected_scores``: ``(dq [T,Hi,128], dw [T,Hi], dk [N,128])`` fp32."""
    _check_idx_sel(q, k, w, idx)
    _require_gpu(d_scores)
    q, k, w = q.contiguous(), k.contiguous(), w.float().contiguous()
    idx = idx.to(torch.int32).contiguous()
    d_scores = d_scores.float().contiguous()
    T, Hi, _ = q.shape
    N, K = k.shape[0], idx.shape[1]
    _require(d_scores.shape == (T, K), "d_scores must be [T, K]")
    dq = torch.empty(T, Hi, 128, dtype=torch.float32, device=q.device)
    dw = torch.empty(T, Hi, dtype=torch.float32, device=q.device)
    dk = torch.empty(N, 128, dtype=torch.float32, device=q.device)
    ws_bytes = indexer_scores_bwd_workspace_bytes(T, N, K)
    ws = torch.empty(max(ws_bytes, 16), dtype=torch.uint8, device=q.device)
    with torch.cuda.device(q.device):
        _lib.call("dsa_indexer_scores_bwd", _p(q), _p(k), _p(w), _p(idx), _p(d_scores), T, N, Hi, 128, K,
                  int(causal), _p(dq), _p(dw), _p(dk), _p(ws), ws_bytes, _stream(q.device))
    return dq, dw, dk


@indexer_scores_bwd.register_fake
def _(q, k, w, idx, d_scores, causal=True):
    T, Hi, _ = q.shape
    return (q.new_empty(T, Hi, 128, dtype=torch.float32), q.new_empty(T, Hi, dtype=torch.float32),
            k.new_empty(k.shape[0], 128, dtype=torch.float32))


def _sel_setup(ctx, inputs, output):
    q, k, w, idx, causal = inputs
    ctx.save_for_backward(q, k, w, idx)
    ctx.causal = causal


def _sel_backward(ctx, d_scores):
    q, k, w, idx = ctx.saved_tensors
    dq, dw, dk = indexer_scores_bwd(q, k, w, idx, d_scores, ctx.causal)
    return dq.to(q.dtype), dk.to(k.dtype), dw.to(w.dtype), None, None


torch.library.register_autograd("dsa_amd::indexer_selected_scores", _sel_backward, setup_context=_sel_setup)


# --------------------------------------------------------------------------------------
# dense rows: every visible key of each query (the reference's [B, S, S] index scores and its
# dense indexer loss): kernels over each row's contiguous key range
# --------------------------------------------------------------------------------------
def dense_row_indices(row_base: Tensor, row_len: Tensor, start: int, width: int) -> Tensor:
    """``[T, width]`` int32: key id ``row_base[t] + start + j`` where ``start + j < row_len[t]``, else -1
    (column block ``[start, start + width)`` of the dense rows)."""
    j = torch.arange(start, start + width, device=row_base.device, dtype=torch.int32)
    ids = row_base.to(torch.int32)[:, None] + j[None]
    return torch.where(j[None] < row_len.to(torch.int32)[:, None], ids, torch.full_like(ids, -1))


def dense_scores_bwd_workspace_bytes(T: int, N: int) -> int:
    return int(_lib.load().dsa_dense_indexer_scores_bwd_workspace_size(T, N))


def indexer_scores_dense_bwd(q: Tensor, k: Tensor, w: Tensor, row_base: Tensor, row_len: Tensor, max_row_len: int,
                             d_scores: Tensor) -> Tuple[Tensor, Tensor, Tensor]:
    """Gradients of ``indexer_scores`` (bf16, head_dim 128) from ``d_scores [T, pitch]``: only columns
    ``j < row_len[t]`` carry gradient (the rest are constants).  ``dsa_dense_indexer_scores_bwd``: a
    query-major kernel for dq / dw and a key-major one for dk over each row's contiguous keys (rows
    monotone in t, as ``build_rows`` / ``build_decode_rows`` give).  ``(dq, dw, dk)`` fp32 (zeros when
    no row has a column, e.g. an empty batch)."""
    T, Hi, D = q.shape
    N = k.shape[0]
    if max_row_len <= 0 or T == 0:
        return (torch.zeros(q.shape, dtype=torch.float32, device=q.device),
                torch.zeros(w.shape, dtype=torch.float32, device=q.device),
                torch.zeros(k.shape, dtype=torch.float32, device=q.device))
    _require_gpu(q, k, w, row_base, row_len, d_scores)
    _require(D == 128 and k.shape[-1] == 128, "indexer head_dim must be 128")
    q, k = q.to(torch.bfloat16).contiguous(), k.to(torch.bfloat16).contiguous()
    w = w.to(torch.float32).contiguous()
    d = d_scores.to(torch.float32).contiguous()
    rb, rl = row_base.to(torch.int32).contiguous(), row_len.to(torch.int32).contiguous()
    dq = torch.empty(T, Hi, 128, dtype=torch.float32, device=q.device)
    dw = torch.empty(T, Hi, dtype=torch.float32, device=q.device)
    dk = torch.empty(N, 128, dtype=torch.float32, device=q.device)
    ws_bytes = dense_scores_bwd_workspace_bytes(T, N)
    ws = torch.empty(max(ws_bytes, 256), dtype=torch.uint8, device=q.device)
    with torch.cuda.device(q.device):
        _lib.call("dsa_dense_indexer_scores_bwd", _p(q), _p(k), _p(w), _p(rb), _p(rl), T, N, Hi, 128, _p(d),
                  d.shape[1], _p(dq), _p(dw), _p(dk), _p(ws), ws.numel(), _stream(q.device))
    return dq, dw, dk


def _isc_setup(ctx, inputs, output):
    q, k, w, row_base, row_len, max_row_len, pitch, q_scale, k_scale, fill_masked = inputs
    ctx.save_for_backward(q, k, w, row_base, row_len)
    ctx.max_row_len = max_row_len
    ctx.fp8 = q_scale is not None


def _isc_backward(ctx, d_scores):
    q, k, w, row_base, row_len = ctx.saved_tensors
    if ctx.fp8 or q.shape[-1] != 128:
        raise NotImplementedError("indexer_scores backward: bf16 inputs with head_dim 128 only")
    dq, dw, dk = indexer_scores_dense_bwd(q, k, w, row_base, row_len, ctx.max_row_len, d_scores)
    return dq.to(q.dtype), dk.to(k.dtype), dw.to(w.dtype), None, None, None, None, None, None, None


torch.library.register_autograd("dsa_amd::indexer_scores", _isc_backward, setup_context=_isc_setup)


def _check_dense(q: Tensor, kv: Tensor, row_base: Tensor, row_len: Tensor) -> None:
    _require_gpu(q, kv, row_base, row_len)
    _require(q.dim() == 3 and q.shape[-1] == D_QK, f"q must be [T, H, {D_QK}]")
    _require(kv.dim() == 2 and kv.shape[-1] == D_QK, f"kv must be [N, {D_QK}]")
    _require(q.dtype == torch.bfloat16 and kv.dtype == torch.bfloat16, "q and kv must be bf16")
    _require(row_base.shape == (q.shape[0],) and row_len.shape == (q.shape[0],), "row_base / row_len must be [T]")


def dense_attention_lse(q: Tensor, kv: Tensor, row_base: Tensor, row_len: Tensor, max_row_len: int,
                        sm_scale: float) -> Tensor:
    """``[T, H]`` natural-log LSE of every query's dense attention over all of its visible keys, the
    kv rows ``row_base[t] .. row_base[t] + row_len[t] - 1`` (``dsa_dense_attention_lse``: the QK
    product alone over each contiguous key range, no index rows; ``-inf`` for an empty row).
    ``max_row_len`` is part of the call contract; the kernel reads the rows themselves."""
    _check_dense(q, kv, row_base, row_len)
    q, kv = q.contiguous(), kv.contiguous()
    T, H, _ = q.shape
    lse = torch.empty(T, H, dtype=torch.float32, device=q.device)
    if T == 0 or max_row_len <= 0:
        return lse.fill_(float("-inf"))
    rb, rl = row_base.to(torch.int32).contiguous(), row_len.to(torch.int32).contiguous()
    with torch.cuda.device(q.device):
        _lib.call("dsa_dense_attention_lse", _p(q), _p(kv), _p(rb), _p(rl), T, kv.shape[0], H, D_QK,
                  float(sm_scale), _p(lse), _stream(q.device))
    return lse


def dense_attention_target(q: Tensor, kv: Tensor, lse: Tensor, row_base: Tensor, row_len: Tensor, max_row_len: int,
                           pitch: int, sm_scale: float) -> Tensor:
    """Target of the dense indexer loss, ``[T, pitch]`` fp32: column j = key ``row_base[t] + j`` holds
    ``(1/H) sum_h exp(sm_scale * q[t,h] . kv[key] - lse[t,h])`` (0 past the row), the head-mean of the
    dense attention probabilities (``lse`` from ``dense_attention_lse``; ``dsa_dense_attention_target``)."""
    _check_dense(q, kv, row_base, row_len)
    q, kv = q.contiguous(), kv.contiguous()
    T, H, _ = q.shape
    _require(lse.shape == (T, H), "lse must be [T, H]")
    tgt = torch.empty(T, pitch, dtype=torch.float32, device=q.device)
    if T == 0 or max_row_len <= 0:
        return tgt.zero_()
    rb, rl = row_base.to(torch.int32).contiguous(), row_len.to(torch.int32).contiguous()
    lse = lse.to(torch.float32).contiguous()
    with torch.cuda.device(q.device):
        _lib.call("dsa_dense_attention_target", _p(q), _p(kv), _p(lse), _p(rb), _p(rl), T, kv.shape[0], H, D_QK,
                  int(pitch), float(sm_scale), _p(tgt), _stream(q.device))
    return tgt


# --------------------------------------------------------------------------------------
# DeepSeek-V4 compressor (softmax-gated window pooling + RMS norm)
# --------------------------------------------------------------------------------------
_DOC_TABLES: dict = {}   # (cu, rate, device) -> table: layers re-use their documents' table


def compress_doc_table(cu_seqlens, rate: int, device) -> Tuple[Tensor, int, int]:
    """Document table of the V4 compressor entry points: int32 ``[3, n_docs + 1]`` on ``device``
    (token offsets, entry offsets = prefix sums of ``len // rate``, backward item offsets = prefix
    sums of ``ceil(len / rate)``), the number of entries and of backward items.  Tables are kept
    per (documents, rate, device), at most 64 of them, so repeated calls copy nothing."""
    cu = [int(x) for x in cu_seqlens]
    key = (tuple(cu), int(rate), str(torch.device(device)))
    hit = _DOC_TABLES.get(key)
    if hit is not None:
        return hit
    _require(len(cu) >= 2 and cu[0] == 0 and all(b >= a for a, b in zip(cu[:-1], cu[1:])),
             "cu_seqlens must start at 0 and be non-decreasing")
    _require(rate >= 1, "rate must be >= 1")
    coff, ioff = [0], [0]
    for a, b in zip(cu[:-1], cu[1:]):
        coff.append(coff[-1] + (b - a) // rate)
        ioff.append(ioff[-1] + (b - a + rate - 1) // rate)
    tab = torch.tensor([cu, coff, ioff], dtype=torch.int32).to(device)
    if len(_DOC_TABLES) >= 64:
        _DOC_TABLES.pop(next(iter(_DOC_TABLES)))
    _DOC_TABLES[key] = (tab, coff[-1], ioff[-1])
    return tab, coff[-1], ioff[-1]


def _check_compress(kv: Tensor, gate: Tensor, ape: Tensor, norm_w: Tensor, table: Tensor, rate: int,
                    overlap: bool) -> Tuple[int, int]:
    _require_gpu(kv, gate, ape, norm_w, table)
    D = norm_w.numel()
    C = 2 * D if overlap else D
    _require(D in (64, 128, 256, 512), "compressor dim must be 64, 128, 256 or 512")
    for name, t in (("kv", kv), ("gate", gate)):
        _require(t.dim() == 2 and t.shape[1] == C and t.dtype == torch.bfloat16,
                 f"{name} must be [T, {C}] bf16")
        _require(t.stride(1) == 1 and t.stride(0) % 8 == 0 and t.data_ptr() % 16 == 0,
                 f"{name} rows must be unit-stride, 16-byte aligned, row stride a multiple of 8")
    _require(kv.shape[0] == gate.shape[0], "kv and gate must have the same rows")
    _require(ape.shape == (rate, C) and ape.dtype == torch.bfloat16, f"ape must be [{rate}, {C}] bf16")
    _require(norm_w.dtype == torch.bfloat16, "norm weight must be bf16")
    _require(table.dtype == torch.int32 and table.dim() == 2 and table.shape[0] == 3, "doc table must be int32 [3, n+1]")
    return C, D


def v4_compress_fwd(kv: Tensor, gate: Tensor, ape: Tensor, norm_w: Tensor, table: Tensor, n_entries: int,
                    rate: int, eps: float, overlap: bool) -> Tensor:
    """Compressed entries ``[n_entries, D]`` bf16 (``dsa_v4_compress_fwd``): every complete window of
    ``rate`` tokens of each document (``table`` from ``compress_doc_table``), softmax(gate + ape)-pooled
    per channel (overlap: the previous window's first halves and this window's second halves), RMS
    norm with ``norm_w``.  ``kv``, ``gate [T, C]`` bf16, ``ape [rate, C]``."""
    C, D = _check_compress(kv, gate, ape, norm_w, table, rate, overlap)
    T = kv.shape[0]
    ape, norm_w = ape.contiguous(), norm_w.contiguous()
    out = torch.empty(n_entries, D, dtype=torch.bfloat16, device=kv.device)
    with torch.cuda.device(kv.device):
        _lib.call("dsa_v4_compress_fwd", _p(kv), _p(gate), kv.stride(0), gate.stride(0), _p(ape), _p(norm_w),
                  _p(table), table.shape[1] - 1, T, int(n_entries), C, D, int(rate), int(bool(overlap)), float(eps),
                  _p(out), _stream(kv.device))
    return out


def v4_compress_bwd(kv: Tensor, gate: Tensor, ape: Tensor, norm_w: Tensor, table: Tensor, n_entries: int,
                    n_items: int, rate: int, eps: float, overlap: bool, dout: Tensor):
    """Backward of ``v4_compress_fwd`` (``dsa_v4_compress_bwd``): ``(dkv, dgate)`` bf16 ``[T, C]`` and
    ``(dape [rate, C], dnorm_w [D])`` fp32, the pooling recomputed from ``kv`` and ``gate``."""
    C, D = _check_compress(kv, gate, ape, norm_w, table, rate, overlap)
    T = kv.shape[0]
    _require(dout.shape == (n_entries, D) and dout.dtype == torch.bfloat16, f"dout must be [{n_entries}, {D}] bf16")
    _require_gpu(dout)
    ape, norm_w, dout = ape.contiguous(), norm_w.contiguous(), dout.contiguous()
    dkv = torch.empty(T, C, dtype=torch.bfloat16, device=kv.device)
    dgate = torch.empty(T, C, dtype=torch.bfloat16, device=kv.device)
    dape = torch.empty(rate, C, dtype=torch.float32, device=kv.device)
    dnorm = torch.empty(D, dtype=torch.float32, device=kv.device)
    ws_bytes = int(_lib.load().dsa_v4_compress_bwd_workspace_size(int(n_entries), int(n_items), C, D, int(rate)))
    ws = torch.empty(max(ws_bytes, 16), dtype=torch.uint8, device=kv.device)
    with torch.cuda.device(kv.device):
        _lib.call("dsa_v4_compress_bwd", _p(kv), _p(gate), kv.stride(0), gate.stride(0), _p(ape), _p(norm_w),
                  _p(table), table.shape[1] - 1, T, int(n_entries), int(n_items), C, D, int(rate),
                  int(bool(overlap)), float(eps), _p(dout), _p(dkv), _p(dgate), C, C, _p(dape), _p(dnorm), _p(ws),
                  ws.numel(), _stream(kv.device))
    return dkv, dgate, dape, dnorm


# --------------------------------------------------------------------------------------
# DeepSeek-V4 row transforms: per-head RMS norm + RoPE of q rows, the output's RoPE in the grouped
# projection's layout
# --------------------------------------------------------------------------------------
def _check_rope(x: Tensor, cos: Tensor, sin: Tensor, rope_dim: int) -> None:
    _require_gpu(x, cos, sin)
    _require(x.dtype == torch.bfloat16 and x.is_contiguous(), "rows must be contiguous bf16")
    _require(cos.dtype == torch.float32 and sin.dtype == torch.float32 and cos.shape == sin.shape,
             "cos / sin must be fp32 tables of one shape")
    _require(cos.dim() == 2 and cos.stride(1) == 1 and sin.stride(0) == cos.stride(0) and cos.shape[1] >= rope_dim // 2,
             "cos / sin must be [tokens, >= rope_dim / 2] with unit column stride")


def v4_norm_rope(x: Tensor, cos: Tensor, sin: Tensor, rope_dim: int, norm: bool, eps: float,
                 inverse: bool = False) -> Tensor:
    """``x [T, H, D]`` bf16 -> per-row weightless RMS norm (``norm``) then interleaved RoPE on the last
    ``rope_dim`` dims with token t's ``cos / sin [T, >= rope_dim/2]`` (``dsa_v4_norm_rope``)."""
    _check_rope(x, cos, sin, rope_dim)
    T, H, D = x.shape
    _require(cos.shape[0] == T, "one cos / sin row per token")
    out = torch.empty_like(x)
    if out.numel() == 0:
        return out
    with torch.cuda.device(x.device):
        _lib.call("dsa_v4_norm_rope", _p(x), T * H, H, D, int(rope_dim), _p(cos), _p(sin), cos.stride(0), int(bool(norm)),
                  float(eps), int(bool(inverse)), _p(out), _stream(x.device))
    return out


def v4_norm_rope_bwd(x: Tensor, dout: Tensor, cos: Tensor, sin: Tensor, rope_dim: int, norm: bool, eps: float,
                     inverse: bool = False) -> Tensor:
    """Gradient of ``v4_norm_rope`` with respect to ``x`` (``dsa_v4_norm_rope_bwd``)."""
    _check_rope(dout, cos, sin, rope_dim)
    _require(x.shape == dout.shape and x.dtype == torch.bfloat16 and x.is_contiguous(), "x must match dout")
    T, H, D = dout.shape
    dx = torch.empty_like(dout)
    if dx.numel() == 0:
        return dx
    with torch.cuda.device(dout.device):
        _lib.call("dsa_v4_norm_rope_bwd", _p(x), _p(dout), T * H, H, D, int(rope_dim), _p(cos), _p(sin), cos.stride(0),
                  int(bool(norm)), float(eps), int(bool(inverse)), _p(dx), _stream(dout.device))
    return dx


def v4_out_rope_group(o: Tensor, cos: Tensor, sin: Tensor, rope_dim: int, groups: int, inverse: bool) -> Tensor:
    """``o [T, H, D]`` -> ``[groups, T, H * D / groups]`` with each row RoPE-rotated (``inverse``: the
    output's inverse rotation; ``dsa_v4_out_rope_group``)."""
    _check_rope(o, cos, sin, rope_dim)
    T, H, D = o.shape
    _require(H % groups == 0 and cos.shape[0] == T, "heads must split into the groups; one cos / sin row per token")
    og = torch.empty(groups, T, H * D // groups, dtype=o.dtype, device=o.device)
    with torch.cuda.device(o.device):
        _lib.call("dsa_v4_out_rope_group", _p(o), T, H, D, int(rope_dim), int(groups), _p(cos), _p(sin), cos.stride(0),
                  int(bool(inverse)), _p(og), _stream(o.device))
    return og


def v4_out_rope_group_bwd(dog: Tensor, n_heads: int, cos: Tensor, sin: Tensor, rope_dim: int, inverse: bool) -> Tensor:
    """Gradient of ``v4_out_rope_group``: ``dog [G, T, H * D / G]`` -> ``do [T, H, D]``."""
    _check_rope(dog, cos, sin, rope_dim)
    G, T, W = dog.shape
    _require((W * G) % n_heads == 0, "the grouped rows must hold whole heads")
    D = W * G // n_heads
    d_o = torch.empty(T, n_heads, D, dtype=dog.dtype, device=dog.device)
    with torch.cuda.device(dog.device):
        _lib.call("dsa_v4_out_rope_group_bwd", _p(dog), T, n_heads, D, int(rope_dim), G, _p(cos), _p(sin),
                  cos.stride(0), int(bool(inverse)), _p(d_o), _stream(dog.device))
    return d_o
