"""Full-size GPU parity of the prefill configurations cfg2 (bf16, S = 4096) and cfg4 (fp8 indexer,
S = 32768): the whole chain indexer -> top-k -> sparse MLA forward at the bench's shapes; and of
cfg5's decode indexer (64 sequences over caches of up to 65,265 keys, bf16 and e4m3 key caches).

Every row is checked where a size-independent check exists:
  - top-k of every row equals a stable descending sort of the kernel's own fp32 scores (ties to
    the lower key), bit for bit;
  - the forward output and LSE of every row match a plain fp32 PyTorch reference on the GPU.
Sampled rows are checked against the float64 CPU oracle, which also pins those GPU-side checks:
top-k bit-exact from the kernel's scores, >= 99.9 % set overlap with the selection from float64
scores of the (dequantised) inputs, scores within tolerance, and out / lse within
rtol = atol = 2e-2 (plus normalised error < 1e-2).
"""
import pytest
import torch

from gpu_reference import close_on_device, sparse_mla_bwd_fp32, sparse_mla_fwd_fp32
from oracle import dsa_oracle as O
from mcore_bridge_amd import ops, workloads as W

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _close(got, ref, rel=1e-2, name="", tol=2e-2):
    got = got.double().cpu()
    ref = ref.double().cpu()
    torch.testing.assert_close(got, ref, rtol=tol, atol=tol, msg=lambda m: f"{name}: {m}")
    err = (got - ref).norm() / ref.norm().clamp_min(1e-30)
    assert err < rel, f"{name}: normalised error {err:.3e} >= {rel}"


def _doc_start(t, cu):
    """First key of query t's document (cu = cumulative document lengths)."""
    d = next(i for i in range(len(cu) - 1) if cu[i] <= t < cu[i + 1])
    return cu[d]


def _topk_every_row_is_a_stable_sort(sc, idx, K, cu=None, chunk=512):
    """idx[t] (ascending global key ids, -1 pad) equals the first min(K, t - start + 1) columns of a
    stable descending sort of row t of the kernel's scores, shifted by the document start (column j
    of a row is key start + j; columns past the row are -inf), for every row of every document."""
    T = sc.shape[0]
    cu = list(cu) if cu is not None else [0, T]
    big = torch.iinfo(torch.int64).max
    for s0, s1 in zip(cu[:-1], cu[1:]):
        for a in range(s0, s1, chunk):
            b = min(s1, a + chunk)
            width = b - s0
            order = torch.sort(sc[a:b, :width], dim=1, descending=True, stable=True).indices[:, :K]
            n = (torch.arange(a, b, device=sc.device) - s0 + 1).clamp(max=K)
            keep = torch.arange(order.shape[1], device=sc.device)[None] < n[:, None]
            want = torch.where(keep, order + s0, torch.full_like(order, big)).sort(dim=1).values
            want = torch.where(want == big, torch.full_like(want, -1), want)
            if want.shape[1] < K:
                want = torch.cat([want, want.new_full((b - a, K - want.shape[1]), -1)], 1)
            bad = (want != idx[a:b].long()).any(dim=1)
            assert not bad.any(), f"top-k rows {(a + bad.nonzero().flatten()).tolist()[:8]} differ from a stable sort"


def _sampled_rows_against_oracle(q_idx, k_idx, w, sc, idx, rows, K, q_scale=None, k_scale=None, score_tol=1e-4,
                                 cu=None):
    cu = list(cu) if cu is not None else [0, sc.shape[0]]
    rows_t = torch.tensor(rows, device=sc.device)
    sc_rows = sc[rows_t].double().cpu()
    idx_rows = idx[rows_t].long().cpu()
    starts = [_doc_start(t, cu) for t in rows]
    # bit-exact against the oracle's selection from the kernel's own fp32 scores
    for i, t in enumerate(rows):
        s0 = starts[i]
        want = O.topk_indices(sc_rows[i:i + 1, :t - s0 + 1], K)[0]
        want = torch.where(want >= 0, want + s0, want)
        want = torch.cat([want, want.new_full((K - want.numel(),), -1)])
        assert torch.equal(idx_rows[i], want), f"row {t}"
    # float64 scores of the same (dequantised) inputs: values and >= 99.9 % overlap
    qc = q_idx[rows_t].float().cpu()
    qsc = q_scale[rows_t].cpu() if q_scale is not None else None
    ref = O.indexer_scores_rows(qc, k_idx.float().cpu(), w[rows_t].cpu(), list(range(len(rows))), None, False,
                                q_scale=qsc, k_scale=k_scale.cpu() if k_scale is not None else None)
    inter = tot = 0
    for i, t in enumerate(rows):
        s0 = starts[i]
        r = ref[i, s0:t + 1]
        torch.testing.assert_close(sc_rows[i, :t - s0 + 1], r, rtol=score_tol, atol=score_tol,
                                   msg=lambda m: f"row {t}: {m}")
        want = set((O.topk_indices(r[None], K)[0] + s0).tolist()) - {s0 - 1}
        got = set(idx_rows[i].tolist()) - {-1}
        inter += len(want & got)
        tot += len(want)
    assert inter / tot >= 0.999, f"overlap {inter / tot:.5f}"
    return inter / tot


def _forward_checks(q, kv, idx, rows):
    out, lse = ops.sparse_mla_fwd(q, kv, idx, W.SM_SCALE, True)
    ref_o, ref_l = sparse_mla_fwd_fp32(q, kv, idx, W.SM_SCALE, True)
    torch.cuda.synchronize()
    # every row against the fp32 reference
    close_on_device(out, ref_o, name="out (all rows, fp32 reference)")
    torch.testing.assert_close(lse, ref_l, rtol=1e-4, atol=1e-4)
    del ref_o, ref_l
    # sampled rows against the float64 oracle (which also pins the fp32 reference there)
    si = torch.tensor(rows, device=q.device)
    ro, rl = O.sparse_mla_fwd(q[si].cpu(), kv.cpu(), idx[si].cpu(), W.SM_SCALE)
    _close(out[si].cpu(), ro, name="out (oracle rows)")
    torch.testing.assert_close(lse[si].cpu().double(), rl, rtol=1e-4, atol=1e-4)
    ref_o, _ = sparse_mla_fwd_fp32(q[si], kv, idx[si], W.SM_SCALE, False)
    _close(ref_o.cpu(), ro, rel=1e-3, name="fp32 reference vs oracle", tol=5e-3)
    return out, lse


def _sample(S, extra, seed):
    g = torch.Generator().manual_seed(seed)
    rnd = torch.randint(0, S, (8,), generator=g).tolist()
    return sorted(set([0, 1, 2046, 2047, 2048, S // 2, S - 2, S - 1] + extra + rnd))


def test_cfg2_full_size_indexer_topk_sparse_fwd():
    """cfg2: one causal document of 4096 tokens, bf16 indexer 64 x 128 (inputs N(0,1)*0.1, w
    N(0,1)/8), top-k 2048, 128-head sparse MLA forward."""
    print("[cfg2 full size] S=4096 bf16 indexer -> top-k 2048 -> sparse fwd", flush=True)
    cfg = W.CONFIGS["cfg2"]
    x = W.make_prefill(cfg, device=DEV, seed=2)
    S, K = cfg.S, cfg.K
    qi, ki, w = x["q_idx"].bfloat16(), x["k_idx"].bfloat16(), x["w"]
    idx, sc = ops.indexer_topk(qi, ki, w, K, return_scores=True)
    _topk_every_row_is_a_stable_sort(sc, idx, K)
    rows = _sample(S, [1000, 3000], 2)
    _sampled_rows_against_oracle(qi, ki, w, sc, idx, rows, K)
    del sc
    _forward_checks(x["q"].bfloat16(), x["kv"].bfloat16(), idx, rows)


def test_cfg4_full_size_fp8_indexer_topk_sparse_fwd():
    """cfg4: one causal document of 32768 tokens; q_idx / k_idx drawn N(0,1) and stored as e4m3fn
    with fp32 absmax scales per (token, head) row of q and per token row of k; fp8 indexer on fp8
    MFMA, top-k 2048 (one workgroup per row: 32768 rows, most longer than the LDS cache), then the
    bf16 sparse MLA forward (128 heads) on those indices."""
    print("[cfg4 full size] S=32768 fp8 indexer -> top-k 2048 -> bf16 sparse fwd", flush=True)
    cfg = W.CONFIGS["cfg4"]
    x = W.make_prefill(cfg, device=DEV, seed=4)
    S, K = cfg.S, cfg.K
    qf = x.pop("q_idx")
    chk = {t: qf[t].cpu() for t in (0, 12345, S - 1)}
    q8, qs = W.quantize_e4m3_rows(qf)
    del qf
    k8, ks = W.quantize_e4m3_rows(x.pop("k_idx"))
    w = x["w"]
    # the workload quantiser (run on the GPU) equals the oracle's on sampled rows: scales within an
    # fp32 ulp (the device division need not round like the host's), codes equal but for values
    # on a rounding boundary of that ulp
    for t, v in chk.items():
        r8, rs = O.quantize_e4m3_rows(v)
        torch.testing.assert_close(qs[t].cpu(), rs, rtol=2.5e-7, atol=0)
        same = (r8.view(torch.uint8) == q8[t].cpu().view(torch.uint8)).float().mean().item()
        assert same >= 0.999, (t, same)
    idx, sc = ops.indexer_topk(q8, k8, w, K, q_scale=qs, k_scale=ks, return_scores=True)
    print("[cfg4 full size] indexer + top-k done", flush=True)
    _topk_every_row_is_a_stable_sort(sc, idx, K)
    rows = _sample(S, [16383, 16384, 16385, 24000, 30001], 4)
    # fp8 products are exact; the fp8 MFMA's accumulation is not bit-for-bit fp32 (~3e-4 relative
    # measured), so scores are held to 2e-3 and the selection to >= 99.9 % overlap
    ov = _sampled_rows_against_oracle(q8, k8, w, sc, idx, rows, K, q_scale=qs, k_scale=ks,
                                      score_tol=2e-3)
    print(f"[cfg4 full size] top-k overlap with float64 selection {ov:.5f}", flush=True)
    del sc
    _forward_checks(x["q"].bfloat16(), x["kv"].bfloat16(), idx, rows)


def test_cfg3_full_size_indexer_topk_sparse_fwd_bwd():
    """cfg3, the bench's headline shape: 16384 packed tokens in 4 causal documents (10363 / 4977 /
    197 / 847), bf16 indexer 64 x 128, top-k 2048, then the 128-head sparse MLA forward and backward
    on those indices.  Every row is checked: the top-k of every query (rows up to 10,363 keys, where
    the top-k kernel sizes its LDS cache per launch) against a stable sort of the kernel's own fp32
    scores inside its document; out / lse of every query and dq of every query and dkv of every key
    against the chunked fp32 GPU references.  The float64 oracle checks sampled rows (top-k from
    the kernel's scores, >= 99.9 % overlap with its own selection, scores, out / lse / dq) and sampled
    keys (dkv), and pins the fp32 references on them."""
    print("[cfg3 full size] T=16384 in 4 documents: indexer -> top-k -> sparse fwd + bwd", flush=True)
    cfg = W.CONFIGS["cfg3"]
    x = W.make_prefill(cfg, device=DEV, seed=3)
    T, K, cu = cfg.S, cfg.K, cfg.docs
    qi, ki, w = x.pop("q_idx").bfloat16(), x.pop("k_idx").bfloat16(), x.pop("w")
    idx, sc = ops.indexer_topk(qi, ki, w, K, x["cu_seqlens"], causal=True, return_scores=True)
    assert sc.shape[1] >= max(b - a for a, b in zip(cu[:-1], cu[1:]))
    _topk_every_row_is_a_stable_sort(sc, idx, K, cu=cu)
    print("[cfg3 full size] top-k of every row = stable sort of the kernel's scores", flush=True)
    rows = sorted({0, 1, 31, 2047, 2048, 5000, 10362, cu[1], cu[1] + 2047, cu[1] + 2100, cu[2] + 100,
                   cu[3] + 5, T - 1} | set(torch.randint(0, T, (8,), generator=torch.Generator().manual_seed(3)).tolist()))
    ov = _sampled_rows_against_oracle(qi, ki, w, sc, idx, rows, K, cu=cu)
    print(f"[cfg3 full size] top-k overlap with float64 selection {ov:.5f}", flush=True)
    del sc, qi, ki, w
    q, kv, dout = x["q"].bfloat16(), x["kv"].bfloat16(), x["dout"].bfloat16()
    del x
    out, lse = _forward_checks(q, kv, idx, rows)
    print("[cfg3 full size] forward checked", flush=True)
    dq, dkv = ops.sparse_mla_bwd(q, kv, idx, out, dout, lse, W.SM_SCALE, True)
    ref_dq, ref_dkv = sparse_mla_bwd_fp32(q, kv, idx, out, dout, lse, W.SM_SCALE, True)
    torch.cuda.synchronize()
    close_on_device(dq, ref_dq, name="dq (every query, fp32 reference)")
    close_on_device(dkv, ref_dkv, name="dkv (every key, fp32 reference)")
    for name, got, ref in (("dq", dq, ref_dq), ("dkv", dkv, ref_dkv)):
        err = ((got.float() - ref).norm() / ref.norm()).item()
        print(f"[cfg3 full size] {name} normalised error vs fp32 reference {err:.2e}", flush=True)
    # the float64 oracle on sampled queries (dq) and keys (dkv) pins both the kernels and the
    # fp32 references there
    si = torch.tensor(rows, device=DEV)
    kvc = kv.cpu()
    rdq, _ = O.sparse_mla_bwd(q[si].cpu(), kvc, idx[si].cpu(), out[si].cpu(), dout[si].cpu(), lse[si].cpu(),
                              W.SM_SCALE)
    _close(dq[si].cpu(), rdq, name="dq (oracle rows)")
    _close(ref_dq[si].cpu(), rdq, rel=1e-3, tol=5e-3, name="fp32 dq reference vs oracle")
    keys = [0, 7, 1000, 2047, 10362, cu[1], cu[2] + 3, cu[3], T - 2048, T - 1]
    rdkv = O.sparse_mla_bwd_dkv_rows(q.cpu(), kvc, idx.cpu(), out.cpu(), dout.cpu(), lse.cpu(), W.SM_SCALE, keys)
    _close(dkv[keys].cpu(), rdkv, name="dkv (oracle keys)")
    _close(ref_dkv[keys].cpu(), rdkv, rel=1e-3, tol=5e-3, name="fp32 dkv reference vs oracle")


@pytest.mark.parametrize("fp8", [False, True])
def test_decode_indexer_cfg5_full_size(fp8):
    """cfg5 at full size (64 sequences, the cache-length fixture up to 65,265 keys, Hi = 64, Di = 128,
    K = 2048) through ops.decode_indexer_topk: every row's selection equals a stable descending sort
    of the kernel's own fp32 scores, bit for bit; every score matches an fp32 GPU reference of the
    same (dequantised) inputs; on sampled sequences the scores match the float64 oracle and the
    selection overlaps the float64 selection by >= 99.9 %.  fp8: e4m3fn q and key cache with one
    fp32 absmax scale per row."""
    cfg = W.CONFIGS["cfg5"]
    print(f"[decode indexer cfg5 full size] fp8={fp8}", flush=True)
    d = W.make_decode(cfg, device=DEV, seed=17)
    lens = [int(x) for x in cfg.decode_lens]
    B, K = len(lens), cfg.K
    cu = torch.tensor([0] + list(torch.tensor(lens).cumsum(0).tolist()), dtype=torch.int32, device=DEV)
    q, k, w = d["q_idx"], d["k_cache"], d["w"]
    del d
    if fp8:
        q8, qs = W.quantize_e4m3_rows(q * 10)
        k8, ks = W.quantize_e4m3_rows(k * 10)
        idx, sc = ops.decode_indexer_topk(q8, k8, w, K, cu, max(lens), qs, ks, return_scores=True)
        qd, kd = q8.float() * qs[..., None], k8.float() * ks[:, None]
    else:
        qb, kb = q.bfloat16(), k.bfloat16()
        idx, sc = ops.decode_indexer_topk(qb, kb, w, K, cu, max(lens), return_scores=True)
        qd, kd = qb.float(), kb.float()
    # every row: bit-exact selection from the kernel's own scores (ascending ids, ties to the lower key)
    off = cu[:-1].long()
    for b, L in enumerate(lens):
        order = torch.sort(sc[b, :L], descending=True, stable=True).indices[:K]
        want = (order.long() + off[b]).sort().values
        got = idx[b].long()
        n = min(K, L)
        assert torch.equal(got[:n], want) and bool((got[n:] == -1).all()), f"row {b}"
    # every score against an fp32 GPU reference
    for b, L in enumerate(lens):
        o = int(off[b])
        ref = (torch.relu(qd[b] @ kd[o:o + L].T) * w[b][:, None]).sum(0)
        torch.testing.assert_close(sc[b, :L], ref, rtol=2e-3 if fp8 else 1e-4, atol=2e-3 if fp8 else 1e-5,
                                   msg=lambda m: f"scores row {b}: {m}")
    # sampled sequences against the float64 oracle (the longest, the shortest and one more)
    rows = sorted({int(torch.tensor(lens).argmax()), int(torch.tensor(lens).argmin()), 7})
    inter = tot = 0
    for b in rows:
        o, L = int(off[b]), lens[b]
        qo = (q8 if fp8 else qb)[b:b + 1].cpu()
        ko = (k8 if fp8 else kb)[o:o + L].cpu()
        kw = dict(q_scale=qs[b:b + 1].cpu(), k_scale=ks[o:o + L].cpu()) if fp8 else {}
        ref64 = O.decode_indexer_scores(qo.float() if fp8 else qo, ko.float() if fp8 else ko, w[b:b + 1].cpu(),
                                        torch.tensor([0]), torch.tensor([L]), **kw)[0]
        torch.testing.assert_close(sc[b, :L].double().cpu(), ref64, rtol=2e-3 if fp8 else 1e-4,
                                   atol=2e-3 if fp8 else 1e-5)
        exact = set((O.topk_indices(ref64[None], K)[0] + o).tolist())
        exact.discard(o - 1)
        got = set(idx[b][idx[b] >= 0].tolist())
        inter += len(got & exact)
        tot += len(exact)
    assert inter / tot >= 0.999, inter / tot
