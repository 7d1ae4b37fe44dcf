"""GPU parity of the dense indexer-loss statistics (the reference-default dense loss,
dsa_indexer_use_sparse_loss = False, src/mcore_bridge/config/model_config.py:204-205):
dsa_dense_attention_lse and dsa_dense_attention_target over each query's contiguous key range.

Checks: the float64 oracle (oracle.dsa_oracle.sparse_mla_fwd's lse and attention_head_probs over
the dense index rows, i.e. every visible key) on every row of small packed cases, for each wave
count of the kernels (H = 128, 48, 16); the recompute pass of scores far beyond the first block's
headroom; the zero columns past each row up to the pitch, empty and clipped rows; and, at rows
longer than the sparse kernels' 8192-entry index rows, the same statistics assembled from the
sparse forward's LSE over 8192-column blocks (logaddexp) and the sparse target kernel, both pinned
to the oracle in their own tests.
"""
import pytest
import torch

from oracle import dsa_oracle as O
from mcore_bridge_amd import ops, workloads as W

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _rows(cu):
    T = cu[-1]
    base, ln = ops.build_rows(torch.tensor(cu, dtype=torch.int32, device=DEV), T, True)
    return base, ln, max(b - a for a, b in zip(cu[:-1], cu[1:]))


def _oracle(q, kv, base, ln, pitch, scale, chunk=64):
    """float64 oracle over the dense index rows (every visible key), in row chunks."""
    T, H, _ = q.shape
    idx = ops.dense_row_indices(base, ln, 0, pitch).cpu()
    lse = torch.empty(T, H, dtype=torch.float64)
    tgt = torch.empty(T, pitch, dtype=torch.float64)
    for a in range(0, T, chunk):
        b = min(T, a + chunk)
        _, l = O.sparse_mla_fwd(q[a:b], kv, idx[a:b], scale)
        lse[a:b] = l
        tgt[a:b] = O.attention_head_probs(q[a:b], kv, idx[a:b], l, scale)
    return lse, tgt


def _rel(got, ref):
    return float((got.double().cpu() - ref).norm() / ref.norm().clamp_min(1e-30))


@pytest.mark.parametrize("H", [128, 48, 16])
def test_dense_lse_and_target_match_the_oracle(H):
    cu = [0, 130, 300, 301, 733]   # one row of 1 key, rows up to 432 keys (14 blocks), ragged ends
    print(f"[dense lse/target] H={H} cu={cu}", flush=True)
    g = torch.Generator().manual_seed(H)
    T = cu[-1]
    q = (torch.randn(T, H, 576, generator=g) * 0.1).bfloat16()
    kv = (torch.randn(T, 576, generator=g) * 0.1).bfloat16()
    base, ln, maxlen = _rows(cu)
    pitch = maxlen + 37   # columns past every row stay zero
    lse = ops.dense_attention_lse(q.to(DEV), kv.to(DEV), base, ln, maxlen, W.SM_SCALE)
    tgt = ops.dense_attention_target(q.to(DEV), kv.to(DEV), lse, base, ln, maxlen, pitch, W.SM_SCALE).cpu()
    lse_ref, tgt_ref = _oracle(q, kv, base, ln, pitch, W.SM_SCALE)
    torch.testing.assert_close(lse.cpu().double(), lse_ref, rtol=1e-5, atol=1e-5)
    assert _rel(lse, lse_ref) < 1e-6
    torch.testing.assert_close(tgt.double(), tgt_ref, rtol=1e-4, atol=1e-7)
    assert _rel(tgt, tgt_ref) < 1e-5
    col = torch.arange(pitch)[None]
    assert torch.all(tgt[col >= ln.cpu()[:, None]] == 0)
    # each query's target sums to 1 over its keys (every head's probabilities do)
    torch.testing.assert_close(tgt.double().sum(1), torch.ones(T, dtype=torch.float64), rtol=1e-5, atol=1e-5)


def test_dense_lse_recompute_pass_for_scores_beyond_the_headroom():
    """Keys past the first block score > 2^64 above the first block's maximum (log2 units): the
    query is recomputed with its exact maximum; LSE and target match the oracle."""
    cu = [0, 200]
    T, H = cu[-1], 32
    print("[dense lse/target] large logits", flush=True)
    g = torch.Generator().manual_seed(3)
    q = (torch.randn(T, H, 576, generator=g) * 0.8).bfloat16()
    kv = torch.randn(T, 576, generator=g) * 0.1
    kv[40:] *= 300.0
    kv = kv.bfloat16()
    base, ln, maxlen = _rows(cu)
    lse = ops.dense_attention_lse(q.to(DEV), kv.to(DEV), base, ln, maxlen, W.SM_SCALE)
    tgt = ops.dense_attention_target(q.to(DEV), kv.to(DEV), lse, base, ln, maxlen, maxlen, W.SM_SCALE).cpu()
    lse_ref, tgt_ref = _oracle(q, kv, base, ln, maxlen, W.SM_SCALE)
    # the construction does overshoot: some row's maximum past key 40 is > 64 (log2) above keys 0..31
    s = (q.double()[:, :, None, :] @ kv.double()[None, None, :, :].transpose(-1, -2))[..., 0, :] * W.SM_SCALE
    assert float((s[64:, :, 40:64].amax(-1) - s[64:, :, :32].amax(-1)).max()) * 1.4427 > 64
    torch.testing.assert_close(lse.cpu().double(), lse_ref, rtol=1e-5, atol=1e-4)
    torch.testing.assert_close(tgt.double(), tgt_ref, rtol=1e-3, atol=1e-6)


def test_dense_rows_empty_and_clipped():
    """Rows of length 0 give lse = -inf and zero targets; a row reaching past kv is clipped to it;
    a row with row_base outside kv is empty."""
    print("[dense lse/target] empty and clipped rows", flush=True)
    g = torch.Generator().manual_seed(9)
    T, H, N = 6, 16, 70
    q = (torch.randn(T, H, 576, generator=g) * 0.1).bfloat16()
    kv = (torch.randn(N, 576, generator=g) * 0.1).bfloat16()
    base = torch.tensor([0, 5, 60, 80, -3, 0], dtype=torch.int32)
    ln = torch.tensor([0, 33, 40, 4, 4, 70], dtype=torch.int32)     # row 2 clipped to 10 keys
    eff = torch.tensor([0, 33, 10, 0, 0, 70], dtype=torch.int32)
    pitch = 72
    lse = ops.dense_attention_lse(q.to(DEV), kv.to(DEV), base.to(DEV), ln.to(DEV), 70, W.SM_SCALE)
    tgt = ops.dense_attention_target(q.to(DEV), kv.to(DEV), lse, base.to(DEV), ln.to(DEV), 70, pitch,
                                     W.SM_SCALE).cpu()
    lse_ref, tgt_ref = _oracle(q, kv, base.clamp(min=0).to(DEV), eff.to(DEV), pitch, W.SM_SCALE)
    assert torch.all(torch.isneginf(lse.cpu()[eff == 0]))
    torch.testing.assert_close(lse.cpu().double(), lse_ref, rtol=1e-5, atol=1e-5)
    torch.testing.assert_close(tgt.double(), tgt_ref, rtol=1e-4, atol=1e-7)


def test_dense_statistics_of_rows_longer_than_the_index_rows():
    """One causal document of 9000 tokens (rows up to 9000 keys, past the sparse kernels' 8192-entry
    index rows): LSE against the sparse forward's over 8192-column blocks (logaddexp) and the target
    against the sparse target kernel on the same column blocks."""
    print("[dense lse/target] rows of up to 9000 keys", flush=True)
    g = torch.Generator(device=DEV).manual_seed(5)
    cu = [0, 9000]
    T, H, cols = cu[-1], 16, 8192
    q = (torch.randn(T, H, 576, generator=g, device=DEV) * 0.1).bfloat16()
    kv = (torch.randn(T, 576, generator=g, device=DEV) * 0.1).bfloat16()
    base, ln, maxlen = _rows(cu)
    lse = ops.dense_attention_lse(q, kv, base, ln, maxlen, W.SM_SCALE)
    tgt = ops.dense_attention_target(q, kv, lse, base, ln, maxlen, maxlen, W.SM_SCALE)
    ref = None
    for c0 in range(0, maxlen, cols):
        idx = ops.dense_row_indices(base, ln, c0, min(cols, maxlen - c0))
        _, l = ops.sparse_mla_fwd(q, kv, idx, W.SM_SCALE, False)
        ref = l if ref is None else torch.logaddexp(ref, l)
    torch.testing.assert_close(lse, ref, rtol=1e-5, atol=1e-5)
    for c0 in range(0, maxlen, cols):
        w = min(cols, maxlen - c0)
        idx = ops.dense_row_indices(base, ln, c0, w)
        t_ref = ops.indexer_kl_target(q, kv, idx, lse, W.SM_SCALE, False)
        torch.testing.assert_close(tgt[:, c0:c0 + w], t_ref, rtol=1e-4, atol=1e-9)


def _column_block_scores_bwd(q, k, w, base, ln, max_len, d, cols=4096):
    """The dense score backward as the selected-slot score backward (pinned to the oracle in
    test_gpu_indexer_kl.py) over blocks of dense columns, summed."""
    dq = dw = dk = None
    for c0 in range(0, max_len, cols):
        width = min(cols, max_len - c0)
        idx = ops.dense_row_indices(base, ln, c0, width)
        dd = torch.where(idx >= 0, d[:, c0:c0 + width], torch.zeros_like(d[:, c0:c0 + width])).contiguous()
        a, b, c = ops.indexer_scores_bwd(q, k, w, idx, dd, False)
        dq, dw, dk = (a, b, c) if dq is None else (dq + a, dw + b, dk + c)
    return dq, dw, dk


def _nerr(a, b):
    return float((a.double() - b.double()).norm() / b.double().norm().clamp_min(1e-30))


def test_dense_scores_bwd_matches_the_oracle():
    """dq, dw, dk of the dense index scores over packed causal documents (one row of 1 key, key tiles
    straddling documents) against the float64 oracle's score backward over the dense index rows."""
    print("[dense score bwd] oracle", flush=True)
    g = torch.Generator().manual_seed(12)
    cu = [0, 130, 300, 301, 700]
    T, Hi = cu[-1], 64
    q = (torch.randn(T, Hi, 128, generator=g) * 0.1).bfloat16()
    k = (torch.randn(T, 128, generator=g) * 0.1).bfloat16()
    w = torch.randn(T, Hi, generator=g) / 8
    base, ln, maxlen = _rows(cu)
    pitch = maxlen + 5
    d = torch.randn(T, pitch, generator=g)
    dq, dw, dk = ops.indexer_scores_dense_bwd(q.to(DEV), k.to(DEV), w.to(DEV), base, ln, maxlen, d.to(DEV))
    idx = ops.dense_row_indices(base, ln, 0, pitch).cpu()
    dq_r, dk_r, dw_r = O.indexer_scores_bwd(q, k, w, idx, d)
    for name, a, r in (("dq", dq, dq_r), ("dw", dw, dw_r), ("dk", dk, dk_r)):
        torch.testing.assert_close(a.cpu().double(), r, rtol=2e-2, atol=2e-2, msg=lambda m: f"{name}: {m}")
        assert _nerr(a.cpu(), r) < 5e-3, (name, _nerr(a.cpu(), r))


@pytest.mark.parametrize("case", ["cfg3", "decode"])
def test_dense_scores_bwd_matches_the_column_block_path(case):
    """At the cfg3 size (16384 tokens in 4 causal documents, Hi = 64: every row) and over decode rows
    (one query per sequence over its own cache rows: keys that are not the query tokens), the dense
    score backward equals the selected-slot score backward over 4096-column blocks: dq and dw to
    fp32 summation order, dk to the bf16 rounding of its per-pair gradient (w folded into G here, into
    Q there)."""
    print(f"[dense score bwd] column-block path, {case}", flush=True)
    g = torch.Generator(device=DEV).manual_seed(21)
    Hi = 64
    if case == "cfg3":
        cfg = W.CONFIGS["cfg3"]
        cu = torch.tensor(cfg.cu_seqlens, dtype=torch.int32, device=DEV)
        T = N = cfg.S
        base, ln = ops.build_rows(cu, T, True)
        maxlen = max(b - a for a, b in zip(cfg.cu_seqlens[:-1], cfg.cu_seqlens[1:]))
    else:
        lens = [5000, 1, 777, 12000, 64, 3001]
        cc = [0]
        for x in lens:
            cc.append(cc[-1] + x)
        T, N = len(lens), cc[-1]
        base, ln = ops.build_decode_rows(torch.tensor(cc, dtype=torch.int32, device=DEV))
        maxlen = max(lens)
    q = (torch.randn(T, Hi, 128, generator=g, device=DEV) * 0.1).bfloat16()
    k = (torch.randn(N, 128, generator=g, device=DEV) * 0.1).bfloat16()
    w = torch.randn(T, Hi, generator=g, device=DEV) / 8
    pitch = (maxlen + 3) // 4 * 4
    d = torch.randn(T, pitch, generator=g, device=DEV) * 1e-3
    dq, dw, dk = ops.indexer_scores_dense_bwd(q, k, w, base, ln, maxlen, d)
    dq_r, dw_r, dk_r = _column_block_scores_bwd(q, k, w, base, ln, maxlen, d)
    torch.testing.assert_close(dq, dq_r, rtol=1e-4, atol=1e-7)
    torch.testing.assert_close(dw, dw_r, rtol=1e-4, atol=1e-7)
    assert _nerr(dk, dk_r) < 1e-2, _nerr(dk, dk_r)
    torch.testing.assert_close(dk, dk_r, rtol=5e-2, atol=1e-4)
    # deterministic: a second call gives the same bits
    dq2, dw2, dk2 = ops.indexer_scores_dense_bwd(q, k, w, base, ln, maxlen, d)
    assert torch.equal(dq, dq2) and torch.equal(dw, dw2) and torch.equal(dk, dk2)
