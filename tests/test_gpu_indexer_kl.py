"""GPU parity of the sparse indexer KL loss path (target, per-row KL + gradient, selected-slot
indexer scores and their backward) against the CPU oracle, through the C ABI.

Bars as for the attention kernels: rtol / atol 2e-2 plus a normalised-error check against the
float64 oracle on the same bf16 inputs; the end-to-end loss and its gradients are checked against
torch autograd through the literal dense restatement of megatron-core's compute_dsa_indexer_loss.
"""
import pytest
import torch

from oracle import dsa_oracle as O
from mcore_bridge_amd import ops, workloads as W
from mcore_bridge_amd.dsa import fused_qk_topk_naive, indexer_kl_loss

pytestmark = pytest.mark.gpu
DEV = "cuda"
RTOL = ATOL = 2e-2


def _close(got, ref, rel=1e-2, name="", atol=ATOL):
    got = got.double().cpu()
    ref = ref.double().cpu()
    torch.testing.assert_close(got, ref, rtol=RTOL, atol=atol, msg=lambda m: f"{name}: {m}")
    err = (got - ref).norm() / ref.norm().clamp_min(1e-30)
    assert err < rel, f"{name}: normalised error {err:.3e} >= {rel}"


def _idx_case(T, K, g, pad=0.1, cu=None):
    vis = O.visibility_mask(T, None if cu is None else torch.tensor(cu, dtype=torch.int32), True)
    idx = torch.full((T, K), -1, dtype=torch.int32)
    for t in range(T):
        cand = torch.nonzero(vis[t]).flatten()
        cand = cand[torch.randperm(cand.numel(), generator=g)][:K]
        m = cand.numel()
        if t % 5 == 0:
            m = max(1, int(m * (1 - pad)))
        idx[t, :m] = torch.sort(cand[:m]).values.to(torch.int32)
    return idx


def _indexer_inputs(T, Hi, g, scale=0.3):
    qi = (torch.randn(T, Hi, 128, generator=g) * scale).bfloat16()
    ki = (torch.randn(T, 128, generator=g) * scale).bfloat16()
    w = (torch.randn(T, Hi, generator=g) * 0.1).bfloat16().float()
    return qi, ki, w


@pytest.mark.parametrize("T,H,K", [(300, 128, 256), (200, 16, 128), (130, 64, 100), (520, 128, 512)])
def test_indexer_kl_target(T, H, K):
    print(f"[kl target] T={T} H={H} K={K}", flush=True)
    g = torch.Generator().manual_seed(T + K)
    q = (torch.randn(T, H, 576, generator=g) * 0.1).bfloat16()
    kv = (torch.randn(T, 576, generator=g) * 0.1).bfloat16()
    idx = _idx_case(T, K, g, cu=[0, T // 3, T])
    _, lse = ops.sparse_mla_fwd(q.to(DEV), kv.to(DEV), idx.to(DEV), W.SM_SCALE, True)
    tgt = ops.indexer_kl_target(q.to(DEV), kv.to(DEV), idx.to(DEV), lse, W.SM_SCALE, True).cpu()
    ref = O.attention_head_probs(q, kv, idx, lse.cpu(), W.SM_SCALE)
    _close(tgt, ref, rel=2e-3, name="target", atol=1e-4)
    valid = idx >= 0
    assert torch.all(tgt[~valid] == 0)
    # every head's probabilities over the selected keys sum to one, so each target row does too
    torch.testing.assert_close(tgt.double().sum(-1), torch.ones(T, dtype=torch.float64), rtol=0, atol=2e-3)


def test_indexer_kl_target_noncausal_and_empty_rows():
    print("[kl target] non-causal, empty rows", flush=True)
    g = torch.Generator().manual_seed(5)
    T, H, K = 96, 32, 64
    q = (torch.randn(T, H, 576, generator=g) * 0.1).bfloat16()
    kv = (torch.randn(T, 576, generator=g) * 0.1).bfloat16()
    idx = torch.stack([torch.randperm(T, generator=g)[:K] for _ in range(T)]).to(torch.int32)
    idx[3] = -1
    idx[7, ::2] = -1
    _, lse = ops.sparse_mla_fwd(q.to(DEV), kv.to(DEV), idx.to(DEV), W.SM_SCALE, False)
    tgt = ops.indexer_kl_target(q.to(DEV), kv.to(DEV), idx.to(DEV), lse, W.SM_SCALE, False).cpu()
    ref = O.attention_head_probs(q, kv, idx, lse.cpu(), W.SM_SCALE)
    _close(tgt, ref, rel=2e-3, name="target", atol=1e-4)
    assert torch.all(tgt[3] == 0)


@pytest.mark.parametrize("T,K", [(200, 128), (64, 2048), (300, 33)])
def test_indexer_kl_rows(T, K):
    print(f"[kl rows] T={T} K={K}", flush=True)
    g = torch.Generator().manual_seed(11 + K)
    idx = torch.stack([torch.randperm(max(T, K), generator=g)[:K] for _ in range(T)]).to(torch.int32)
    idx[torch.rand(T, K, generator=g) < 0.1] = -1
    idx[4] = -1
    n_kv = max(T, K)
    valid = idx >= 0
    index_sel = torch.randn(T, K, generator=g) * 2
    p = torch.rand(T, K, generator=g).double() * valid
    p[2, :] = 0
    p[2, 0] = 1.0 if valid[2, 0] else 0.0
    p = p / p.sum(-1, keepdim=True).clamp_min(1e-30)
    gs = 0.37
    kl, d = ops.indexer_kl_rows(index_sel.to(DEV), p.float().to(DEV), idx.to(DEV), n_kv, False, gs)
    rkl, rd = O.indexer_kl_sparse(index_sel.double(), p.float().double(), valid)
    torch.testing.assert_close(kl.cpu().double(), rkl, rtol=1e-4, atol=1e-5)
    _close(d.cpu(), rd * gs, rel=1e-4, name="d_index", atol=1e-6)
    assert kl[4].item() == 0 and torch.all(d[4] == 0)


def test_indexer_scores_bwd_no_query_rows():
    """No query rows: dq and dw are empty and every key's dk is an empty sum, written as 0."""
    print("[indexer scores bwd no query rows] Nk=300 Hi=64 K=64", flush=True)
    k = torch.randn(300, 128, device=DEV).bfloat16()
    q = torch.empty(0, 64, 128, dtype=torch.bfloat16, device=DEV)
    w = torch.empty(0, 64, device=DEV)
    idx = torch.empty(0, 64, dtype=torch.int32, device=DEV)
    d = torch.empty(0, 64, device=DEV)
    junk = torch.full((300, 128), float("nan"), device=DEV)
    del junk
    dq, dw, dk = ops.indexer_scores_bwd(q, k, w, idx, d, True)
    torch.cuda.synchronize()
    assert dq.shape == (0, 64, 128) and dw.shape == (0, 64) and dk.shape == (300, 128)
    assert torch.equal(dk.cpu(), torch.zeros(300, 128))


@pytest.mark.parametrize("T,Hi,K,cu", [(300, 64, 256, [0, 300]), (200, 4, 128, [0, 90, 200]),
                                       (260, 64, 2048, [0, 260]), (150, 33, 96, [0, 150])])
def test_indexer_selected_scores(T, Hi, K, cu):
    print(f"[selected scores] T={T} Hi={Hi} K={K}", flush=True)
    g = torch.Generator().manual_seed(T + Hi)
    qi, ki, w = _indexer_inputs(T, Hi, g)
    idx = _idx_case(T, K, g, cu=cu)
    got = ops.indexer_selected_scores(qi.to(DEV), ki.to(DEV), w.to(DEV), idx.to(DEV), True).cpu()
    dense = O.indexer_scores(qi, ki, w, torch.tensor(cu, dtype=torch.int32), True)
    valid = idx >= 0
    ref = torch.gather(dense, 1, idx.clamp(min=0).long())
    assert torch.all(torch.isneginf(got[~valid]))
    _close(got[valid], ref[valid], rel=1e-4, name="scores", atol=1e-4)


@pytest.mark.parametrize("T,Hi,K", [(300, 64, 256), (200, 4, 128), (160, 64, 2048), (130, 48, 100)])
def test_indexer_scores_bwd(T, Hi, K):
    print(f"[indexer scores bwd] T={T} Hi={Hi} K={K}", flush=True)
    g = torch.Generator().manual_seed(3 * T + Hi)
    qi, ki, w = _indexer_inputs(T, Hi, g)
    idx = _idx_case(T, K, g, cu=[0, T // 2, T])
    dI = torch.randn(T, K, generator=g) * 0.01
    dq, dw, dk = ops.indexer_scores_bwd(qi.to(DEV), ki.to(DEV), w.to(DEV), idx.to(DEV), dI.to(DEV), True)
    rq, rk, rw = O.indexer_scores_bwd(qi, ki, w, idx, dI)
    _close(dq.cpu(), rq, name="dq")
    _close(dw.cpu(), rw, name="dw")
    _close(dk.cpu(), rk, name="dk")
    never = torch.ones(T, dtype=torch.bool)
    never[idx[idx >= 0].long()] = False
    assert torch.all(dk.cpu()[never] == 0)


def test_indexer_kl_loss_end_to_end_against_dense_megatron_form():
    """Loss and gradients (q_idx, k_idx, w) of the sparse path against torch autograd through the
    float64 dense restatement of compute_dsa_indexer_loss with sparse_loss (MQA form: every head's
    key is the shared latent row)."""
    print("[indexer kl loss e2e]", flush=True)
    g = torch.Generator().manual_seed(17)
    T, H, Hi, K = 256, 32, 64, 64
    q = (torch.randn(T, H, 576, generator=g) * 0.1).bfloat16()
    kv = (torch.randn(T, 576, generator=g) * 0.1).bfloat16()
    qi, ki, w = _indexer_inputs(T, Hi, g)
    idx = _idx_case(T, K, g, pad=0.0)
    sc, coeff = W.SM_SCALE, 0.25
    _, lse = ops.sparse_mla_fwd(q.to(DEV), kv.to(DEV), idx.to(DEV), sc, True)
    qg = qi.to(DEV).requires_grad_()
    kg = ki.to(DEV).requires_grad_()
    wg = w.to(DEV).requires_grad_()
    loss = indexer_kl_loss(q.to(DEV), kv.to(DEV), lse, idx.to(DEV), qg, kg, wg, sc, coeff, True)
    loss.backward()

    qd = qi.double().requires_grad_()
    kd = ki.double().requires_grad_()
    wd = w.double().requires_grad_()
    full = O.indexer_scores(qd, kd, wd)
    topk = torch.where(idx >= 0, idx, idx[:, :1]).long()
    ref = O.compute_dsa_indexer_loss_dense(full[None], topk[None], q.double()[:, None],
                                           kv.double()[:, None, None].expand(T, 1, H, 576), sc, coeff,
                                           sparse_loss=True)
    ref.backward()
    torch.testing.assert_close(loss.detach().cpu().double(), ref.detach(), rtol=2e-3, atol=1e-6)
    for name, got, r in (("dq_idx", qg.grad, qd.grad), ("dk_idx", kg.grad, kd.grad), ("dw", wg.grad, wd.grad)):
        scale = r.abs().max().clamp_min(1e-30)
        _close(got.cpu() / scale, r / scale, rel=2e-2, name=name)


def test_indexer_kl_path_cfg3_full_size():
    """The whole KL path at the bench's full size (T = 16384 in 4 documents, H = 128, Hi = 64,
    K = 2048, indices from the indexer + top-k kernels): target and KL rows of sampled queries
    against the oracle; the selected scores against the dense scores kernel at the same columns;
    dq / dw of sampled queries and dk of sampled keys against the oracle over exactly the pairs
    they depend on."""
    print("[indexer kl cfg3 full size]", flush=True)
    cfg = W.CONFIGS["cfg3"]
    x = W.make_prefill(cfg, device=DEV, seed=3)
    T, cu = cfg.S, x["cu_seqlens"]
    qi, ki, w = x["q_idx"].bfloat16(), x["k_idx"].bfloat16(), x["w"].float()
    idx, dense = ops.indexer_topk(qi, ki, w, cfg.K, cu, causal=True, return_scores=True)
    q, kv = x["q"].bfloat16(), x["kv"].bfloat16()
    del x
    out, lse = ops.sparse_mla_fwd(q, kv, idx, W.SM_SCALE, True)
    tgt = ops.indexer_kl_target(q, kv, idx, lse, W.SM_SCALE, True)
    # the same target from the P tiles of the attention backward (bf16 P, head mean)
    dout = (torch.randn(out.shape, device=DEV, generator=torch.Generator(device=DEV).manual_seed(9)) * 0.01).bfloat16()
    _, _, tgt_b = ops.sparse_mla_bwd_with_target(q, kv, idx, out, dout, lse, W.SM_SCALE, True)
    del out, dout
    assert torch.all(tgt_b[idx < 0] == 0)
    err = ((tgt_b - tgt).norm() / tgt.norm()).item()
    assert err < 2e-3, f"target from the backward's P tiles: normalised error {err:.2e}"
    del tgt_b
    sel = ops.indexer_selected_scores(qi, ki, w, idx, True)
    kl, d = ops.indexer_kl_rows(sel, tgt, idx, T, True, 1.0 / T)
    dq, dw, dk = ops.indexer_scores_bwd(qi, ki, w, idx, d, True)
    torch.cuda.synchronize()
    # selected scores == the dense scores kernel at the selected columns (column j <-> key doc_start + j)
    starts = torch.tensor(cfg.docs[:-1], device=DEV)
    tok = torch.arange(T, device=DEV)
    doc_start = starts[torch.searchsorted(starts, tok, right=True) - 1]
    valid = idx >= 0
    col = (idx.long() - doc_start[:, None]).clamp(min=0)
    ref_sel = torch.gather(dense, 1, col)
    del dense
    torch.testing.assert_close(sel[valid], ref_sel[valid], rtol=1e-4, atol=1e-4)
    assert torch.all(torch.isneginf(sel[~valid]))

    sample = sorted({0, 1, 31, 2047, 2048, 5000, 10362, cfg.docs[1], cfg.docs[1] + 2100, cfg.docs[2] + 100,
                     cfg.docs[3] + 5, T - 1})
    si = torch.tensor(sample)
    sd = si.to(DEV)
    qc, kvc, idc = q[sd].cpu(), kv.cpu(), idx[sd].cpu()
    rt = O.attention_head_probs(qc, kvc, idc, lse[sd].cpu(), W.SM_SCALE)
    _close(tgt[sd].cpu(), rt, rel=2e-3, name="target", atol=1e-4)
    rkl, rd = O.indexer_kl_sparse(sel[sd].cpu().double(), tgt[sd].cpu().double(), idc >= 0)
    torch.testing.assert_close(kl[sd].cpu().double(), rkl, rtol=1e-4, atol=1e-5)
    _close(d[sd].cpu(), rd / T, rel=1e-4, name="d_index", atol=1e-9)

    qic, kic, wc, dc = qi.cpu(), ki.cpu(), w.cpu(), d.cpu()
    rq, _, rw = O.indexer_scores_bwd(qic[si], kic, wc[si], idc, dc[si])
    _close(dq[sd].cpu(), rq, name="dq", atol=1e-6)
    _close(dw[sd].cpu(), rw, name="dw", atol=1e-6)
    idx_c = idx.cpu()
    for s in [0, 7, 1000, 10362, cfg.docs[1], cfg.docs[2] + 3, T - 2048, T - 1]:
        rows = torch.nonzero((idx_c == s).any(1)).flatten()
        if rows.numel() == 0:
            assert torch.all(dk[s] == 0)
            continue
        only = torch.where(idx_c[rows] == s, idx_c[rows], torch.full_like(idx_c[rows], -1))
        _, rk, _ = O.indexer_scores_bwd(qic[rows], kic, wc[rows], only, dc[rows])
        _close(dk[s].cpu(), rk[s], name=f"dk[{s}]", atol=1e-6)


def _pro_case(T, Hi, g):
    q_lin = (torch.randn(T, Hi, 128, generator=g) * 2).bfloat16()
    k_lin = (torch.randn(T, 128, generator=g) * 2 + 0.5).bfloat16()
    w_lin = torch.randn(T, Hi, generator=g).bfloat16()
    lw = 1 + 0.2 * torch.randn(128, generator=g)
    lb = 0.1 * torch.randn(128, generator=g)
    fr = torch.rand(T, 64, generator=g) * 3000
    return q_lin, k_lin, w_lin, lw, lb, fr


@pytest.mark.parametrize("dei,ri,Hi", [(False, False, 64), (True, False, 64), (False, True, 16), (True, True, 33)])
def test_indexer_prologue_backward(dei, ri, Hi):
    """Gradients of the bf16 prologue (HIP backward kernel through the op's autograd) against torch
    autograd through the float64 oracle prologue."""
    print(f"[prologue bwd] dei={dei} ri={ri} Hi={Hi}", flush=True)
    g = torch.Generator().manual_seed(40 + Hi + 2 * dei + ri)
    T, eps, ms = 150, 1e-6, 1.3
    ins = _pro_case(T, Hi, g)
    gq = torch.randn(T, Hi, 128, generator=g)
    gk = torch.randn(T, 128, generator=g)
    gw = torch.randn(T, Hi, generator=g)
    dv = [x.to(DEV).requires_grad_() if i != 5 else x.to(DEV) for i, x in enumerate(ins)]
    q, _, k, _, w = ops.indexer_prologue(*dv, eps, ms, dei, ri)
    ((q.float() * gq.to(DEV)).sum() + (k.float() * gk.to(DEV)).sum() + (w * gw.to(DEV)).sum()).backward()
    rf = [x.double().requires_grad_() if i != 5 else x for i, x in enumerate(ins)]
    rq, rk, rw = O.indexer_prologue(*rf, eps=eps, mscale=ms, deinterleave=dei, rotary_interleaved=ri,
                                    dtype=torch.float64)
    # the kernel receives the upstream gradients of the bf16 outputs q, k rounded to bf16
    gqb, gkb = gq.bfloat16().double(), gk.bfloat16().double()
    ((rq * gqb).sum() + (rk * gkb).sum() + (rw * gw.double()).sum()).backward()
    for name, a, b in zip(("dq_lin", "dk_lin", "dw_lin", "dln_weight", "dln_bias"), dv[:5], rf[:5]):
        assert a.grad.dtype == a.dtype, name
        # tolerances relative to the tensor's scale: dln_* are sums over all tokens
        scale = b.grad.abs().max().clamp_min(1e-30)
        _close(a.grad.cpu() / scale, b.grad / scale, name=name)


def test_indexer_module_trains_with_the_sparse_kl_loss():
    """The whole indexer training path: DSAIndexer.forward_before_topk (GEMMs + prologue), the
    sparse KL loss against the attention's probabilities, and the backward into the indexer's
    parameters.  Reference: float64 autograd of the dense restatement of compute_dsa_indexer_loss
    at the same forward values (the kernels' bf16 q, k, w; the ReLU masks and softmaxes are then
    those of the GPU pass), its gradients carried through the float64 oracle prologue and the
    projections (same top-k indices on both sides)."""
    print("[indexer training e2e]", flush=True)
    from mcore_bridge_amd.dsa import DSAIndexer
    g = torch.Generator().manual_seed(77)
    S, hidden, qlr, Hi, H, K = 192, 256, 192, 64, 16, 48
    mod = DSAIndexer(hidden, qlr, index_n_heads=Hi, index_topk=K, device=DEV)
    with torch.no_grad():
        for p_ in mod.parameters():
            p_.copy_((torch.randn(p_.shape, generator=g) * 0.05).to(p_.dtype))
        mod.k_norm.weight.add_(1.0)
    x = (torch.randn(S, 1, hidden, generator=g)).bfloat16()
    qr = (torch.randn(S, 1, qlr, generator=g)).bfloat16()
    fr = torch.rand(S, 1, 1, 64, generator=g) * 200
    q, k, w = mod.forward_before_topk(x.to(DEV), qr.to(DEV), (None, fr.to(DEV)))
    idx = ops.indexer_topk(q.detach().reshape(S, Hi, 128), k.detach().reshape(S, 128), w.detach().reshape(S, Hi), K)
    qa = (torch.randn(S, H, 576, generator=g) * 0.1).bfloat16()
    kva = (torch.randn(S, 576, generator=g) * 0.1).bfloat16()
    _, lse = ops.sparse_mla_fwd(qa.to(DEV), kva.to(DEV), idx, W.SM_SCALE, True)
    coeff = 0.5
    loss = indexer_kl_loss(qa.to(DEV), kva.to(DEV), lse, idx, q.reshape(S, Hi, 128), k.reshape(S, 128),
                           w.reshape(S, Hi), W.SM_SCALE, coeff, True)
    loss.backward()

    # dense loss at the GPU's forward values
    qv = q.detach().cpu().double().reshape(S, Hi, 128).requires_grad_()
    kvv = k.detach().cpu().double().reshape(S, 128).requires_grad_()
    wv = w.detach().cpu().double().reshape(S, Hi).requires_grad_()
    ic = idx.cpu().long()
    topk = torch.where(ic >= 0, ic, ic[:, :1])
    ref = O.compute_dsa_indexer_loss_dense(O.indexer_scores(qv, kvv, wv)[None], topk[None], qa.double()[:, None],
                                           kva.double()[:, None, None].expand(S, 1, H, 576), W.SM_SCALE, coeff,
                                           sparse_loss=True)
    ref.backward()
    torch.testing.assert_close(loss.detach().cpu().double(), ref.detach(), rtol=1e-3, atol=1e-6)
    # ... carried through the float64 prologue and projections
    P = {n: p_.detach().double().cpu().requires_grad_() for n, p_ in mod.named_parameters()}
    xd, qrd = x.double()[:, 0], qr.double()[:, 0]
    q_lin = (qrd @ P["linear_wq_b.weight"].T).reshape(S, Hi, 128)
    k_lin = xd @ P["linear_wk.weight"].T
    w_lin = xd @ P["linear_weights_proj.weight"].T
    rq, rk, rw = O.indexer_prologue(q_lin, k_lin, w_lin, P["k_norm.weight"], P["k_norm.bias"], fr.reshape(S, 64),
                                    eps=mod.eps, mscale=mod.mscale, deinterleave=False, rotary_interleaved=False,
                                    dtype=torch.float64)
    # the kernels receive the gradients of the bf16 outputs q, k rounded to bf16
    torch.autograd.backward([rq, rk, rw], [qv.grad.bfloat16().double(), kvv.grad.bfloat16().double(), wv.grad])
    for n, p_ in mod.named_parameters():
        r = P[n].grad
        scale = r.abs().max().clamp_min(1e-30)
        _close(p_.grad.cpu() / scale, r / scale, rel=2e-2, name=n)


def test_fused_attention_with_indexer_loss_matches_the_separate_path():
    """sparse_mla_with_indexer_loss (loss applied in the attention's backward, target from its P
    tiles) against sparse_mla + indexer_kl_loss: identical attention gradients, the same loss and
    indexer gradients up to the bf16 rounding of the staged P."""
    print("[fused attention + indexer loss]", flush=True)
    from mcore_bridge_amd.dsa import sparse_mla_with_indexer_loss
    g = torch.Generator().manual_seed(31)
    T, H, Hi, K = 300, 64, 64, 128
    q = (torch.randn(T, H, 576, generator=g) * 0.1).bfloat16().to(DEV)
    kv = (torch.randn(T, 576, generator=g) * 0.1).bfloat16().to(DEV)
    qi, ki, w = (x.to(DEV) for x in _indexer_inputs(T, Hi, g))
    idx = _idx_case(T, K, g, cu=[0, 120, T]).to(DEV)
    dout = (torch.randn(T, H, 512, generator=g) * 0.01).bfloat16().to(DEV)
    sc, coeff = W.SM_SCALE, 0.3
    leaves = lambda: [x.clone().requires_grad_() for x in (q, kv, qi, ki, w)]
    qa, kva, qia, kia, wa = leaves()
    out_a, lse_a = ops.sparse_mla_fwd(qa, kva, idx, sc, True)
    loss_a = indexer_kl_loss(qa, kva, lse_a, idx, qia, kia, wa, sc, coeff, True)
    (out_a.float() * dout.float()).sum().add(loss_a).backward()
    qb, kvb, qib, kib, wb = leaves()
    out_b, loss_b = sparse_mla_with_indexer_loss(qb, kvb, idx, qib, kib, wb, sc, coeff, True)
    assert loss_b.item() == 0.0                      # filled by the backward pass
    (out_b.float() * dout.float()).sum().backward()
    assert torch.equal(out_a, out_b)
    assert torch.equal(qa.grad, qb.grad) and torch.equal(kva.grad, kvb.grad)
    torch.testing.assert_close(loss_b, loss_a.detach(), rtol=2e-3, atol=1e-7)
    for name, a, b in (("q_idx", qia.grad, qib.grad), ("k_idx", kia.grad, kib.grad), ("w", wa.grad, wb.grad)):
        err = ((b.double() - a.double()).norm() / a.double().norm()).item()
        assert err < 1e-2, f"{name}: normalised difference {err:.2e}"


def test_indexer_scores_bwd_more_keys_than_the_lds_pair_order_holds():
    """n_k = 20000 > 16384: the pair order takes its global-atomic path."""
    print("[indexer scores bwd] n_k=20000", flush=True)
    g = torch.Generator().manual_seed(20001)
    T, Hi, K, N = 64, 64, 256, 20000
    qi = (torch.randn(T, Hi, 128, generator=g) * 0.3).bfloat16()
    ki = (torch.randn(N, 128, generator=g) * 0.3).bfloat16()
    w = (torch.randn(T, Hi, generator=g) * 0.1).bfloat16().float()
    idx = torch.stack([torch.randperm(N, generator=g)[:K] for _ in range(T)]).to(torch.int32)
    idx[:, :8] = torch.arange(8, dtype=torch.int32)
    idx[3, 50:] = -1
    dI = torch.randn(T, K, generator=g) * 0.01
    dq, dw, dk = ops.indexer_scores_bwd(qi.to(DEV), ki.to(DEV), w.to(DEV), idx.to(DEV), dI.to(DEV), False)
    rq, rk, rw = O.indexer_scores_bwd(qi, ki, w, idx, dI)
    _close(dq.cpu(), rq, name="dq")
    _close(dw.cpu(), rw, name="dw")
    _close(dk.cpu(), rk, name="dk")


def test_dsattention_module_composes_indexer_attention_and_loss():
    """DSAttention (Megatron's core-attention signature, absorbed layout, batch 2): in eval it
    equals fused_qk_topk_naive on the indexer's outputs + sparse_mla_attention; in training its
    output and attention gradients are the same, the indexer's parameters receive the sparse KL
    loss's gradients and last_indexer_loss holds that loss."""
    print("[DSAttention module]", flush=True)
    from mcore_bridge_amd.dsa import DSAIndexer, DSAttention, fused_qk_topk_naive, sparse_mla_attention
    g = torch.Generator().manual_seed(55)
    S, B, H, hidden, qlr, Hi, K = 160, 2, 16, 256, 192, 64, 48
    indexer = DSAIndexer(hidden, qlr, index_n_heads=Hi, index_topk=K, device=DEV)
    with torch.no_grad():
        for p_ in indexer.parameters():
            p_.copy_((torch.randn(p_.shape, generator=g) * 0.05).to(p_.dtype))
        indexer.k_norm.weight.add_(1.0)
    coeff, sc = 0.5, W.SM_SCALE
    attn = DSAttention(indexer, sc, loss_coeff=coeff, use_sparse_loss=True)
    query = (torch.randn(S, B, H, 576, generator=g) * 0.1).bfloat16().to(DEV)
    key = (torch.randn(S, B, 576, generator=g) * 0.1).bfloat16().to(DEV)
    x = torch.randn(S, B, hidden, generator=g).bfloat16().to(DEV)
    qr = torch.randn(S, B, qlr, generator=g).bfloat16().to(DEV)
    fr = (torch.rand(S, 1, 1, 64, generator=g) * 200).to(DEV)
    mask = torch.triu(torch.full((S, S), float("-inf"), device=DEV), 1).expand(B, S, S)
    psp = (None, fr)

    attn.eval()
    with torch.no_grad():
        out_e = attn(query, key, None, mask, x, qr, packed_seq_params=psp)
        q_i, k_i, w = indexer.forward_before_topk(x, qr, psp)
        _, topk = fused_qk_topk_naive(q_i, k_i, w, K, causal=True, return_scores=False)
        ref = sparse_mla_attention(query, key, topk, sc, causal=True)
    assert torch.equal(out_e, ref)

    attn.train()
    dout = (torch.randn(S, B, H * 512, generator=g) * 0.01).to(DEV)
    qa, ka = query.clone().requires_grad_(), key.clone().requires_grad_()
    out_t = attn(qa, ka, None, mask, x, qr, packed_seq_params=psp)
    assert torch.equal(out_t.detach(), ref)
    (out_t.float() * dout).sum().backward()
    qb, kb = query.clone().requires_grad_(), key.clone().requires_grad_()
    (sparse_mla_attention(qb, kb, topk, sc, causal=True).float() * dout).sum().backward()
    assert torch.equal(qa.grad, qb.grad) and torch.equal(ka.grad, kb.grad)
    for n, p_ in indexer.named_parameters():
        assert p_.grad is not None and bool(torch.isfinite(p_.grad).all()) and p_.grad.abs().sum() > 0, n
    # the loss it applied: indexer_kl_loss on the same packed inputs
    off = (torch.arange(B, device=DEV) * S).view(B, 1, 1)
    idx = torch.where(topk >= 0, topk + off, torch.full_like(topk, -1)).reshape(B * S, -1).to(torch.int32)
    q_thd, kv_thd = query.transpose(0, 1).reshape(B * S, H, 576), key.transpose(0, 1).reshape(B * S, 576)
    _, lse = ops.sparse_mla_fwd(q_thd, kv_thd, idx, sc, True)
    with torch.no_grad():
        ref_loss = indexer_kl_loss(q_thd, kv_thd, lse, idx, q_i.transpose(0, 1).reshape(B * S, Hi, 128),
                                   k_i.transpose(0, 1).reshape(B * S, 128), w.transpose(0, 1).reshape(B * S, Hi),
                                   sc, coeff, True)
    torch.testing.assert_close(attn.last_indexer_loss, ref_loss, rtol=2e-3, atol=1e-7)


@pytest.mark.parametrize("T,K", [(1, 1), (37, 5), (40, 1)])
def test_kl_path_tiny_shapes(T, K):
    """Partial 32-key blocks and single queries through every kernel of the KL path."""
    print(f"[kl path tiny] T={T} K={K}", flush=True)
    g = torch.Generator().manual_seed(100 + T + K)
    H, Hi = 16, 64
    q = (torch.randn(T, H, 576, generator=g) * 0.1).bfloat16()
    kv = (torch.randn(T, 576, generator=g) * 0.1).bfloat16()
    qi, ki, w = _indexer_inputs(T, Hi, g)
    idx = _idx_case(T, K, g, pad=0.5)
    if T > 2:
        idx[2] = -1                                      # a row with no valid key
    _, lse = ops.sparse_mla_fwd(q.to(DEV), kv.to(DEV), idx.to(DEV), W.SM_SCALE, True)
    tgt = ops.indexer_kl_target(q.to(DEV), kv.to(DEV), idx.to(DEV), lse, W.SM_SCALE, True).cpu()
    _close(tgt, O.attention_head_probs(q, kv, idx, lse.cpu(), W.SM_SCALE), rel=2e-3, name="target", atol=1e-4)
    sel = ops.indexer_selected_scores(qi.to(DEV), ki.to(DEV), w.to(DEV), idx.to(DEV), True).cpu()
    valid = idx >= 0
    ref_sel = torch.gather(O.indexer_scores(qi, ki, w), 1, idx.clamp(min=0).long())
    assert torch.all(torch.isneginf(sel[~valid]))
    if valid.any():
        _close(sel[valid], ref_sel[valid], rel=1e-4, name="scores", atol=1e-4)
    kl, d = ops.indexer_kl_rows(sel.to(DEV), tgt.to(DEV), idx.to(DEV), T, True, 1.0 / T)
    rkl, rd = O.indexer_kl_sparse(sel.double(), tgt.double(), valid)
    torch.testing.assert_close(kl.cpu().double(), rkl, rtol=1e-4, atol=1e-6)
    torch.testing.assert_close(d.cpu().double(), rd / T, rtol=1e-3, atol=1e-7)
    dI = torch.randn(T, K, generator=g) * 0.01
    dq, dw, dk = ops.indexer_scores_bwd(qi.to(DEV), ki.to(DEV), w.to(DEV), idx.to(DEV), dI.to(DEV), True)
    rq, rk, rw = O.indexer_scores_bwd(qi, ki, w, idx, dI)
    for name, a, b in (("dq", dq, rq), ("dw", dw, rw), ("dk", dk, rk)):
        torch.testing.assert_close(a.cpu().double(), b, rtol=2e-2, atol=2e-3, msg=lambda m: f"{name}: {m}")


def test_dsattention_thd_packed_equals_per_document():
    """Packed THD through the module mirrors (PackedSeqParams with cu_seqlens_q, as the MLA caller
    packs it, multi_latent_attention.py:90-96): the indexer's outputs, the top-k, the attention
    output and its gradients equal the per-document unpacked calls, and in training the indexer's
    parameter gradients are the token-weighted sum of the per-document ones (the loss is a mean
    over all packed tokens)."""
    import types
    from mcore_bridge_amd.dsa import DSAIndexer, DSAttention
    print("[DSAttention THD packed vs per document]", flush=True)
    g = torch.Generator().manual_seed(77)
    lens = [50, 130, 77]
    cu_l = [0] + [sum(lens[:i + 1]) for i in range(len(lens))]
    T, H, hidden, qlr, Hi, K = cu_l[-1], 16, 256, 192, 64, 40
    indexer = DSAIndexer(hidden, qlr, index_n_heads=Hi, index_topk=K, device=DEV)
    with torch.no_grad():
        for p_ in indexer.parameters():
            p_.copy_((torch.randn(p_.shape, generator=g) * 0.05).to(p_.dtype))
        indexer.k_norm.weight.add_(1.0)
    coeff, sc = 0.5, W.SM_SCALE
    attn = DSAttention(indexer, sc, loss_coeff=coeff, use_sparse_loss=True)
    query = (torch.randn(T, H, 576, generator=g) * 0.1).bfloat16().to(DEV)
    key = (torch.randn(T, 576, generator=g) * 0.1).bfloat16().to(DEV)
    x = torch.randn(T, 1, hidden, generator=g).bfloat16().to(DEV)
    qr = torch.randn(T, qlr, generator=g).bfloat16().to(DEV)
    rope = (torch.rand(max(lens), 1, 1, 64, generator=g) * 200).to(DEV)
    psp = types.SimpleNamespace(qkv_format="thd", cu_seqlens_q=torch.tensor(cu_l, dtype=torch.int32, device=DEV),
                                max_seqlen_q=max(lens))
    dout = (torch.randn(T, H * 512, generator=g) * 0.01).to(DEV)

    def per_doc(train):
        outs, qg, kg, grads = [], [], [], {n: 0 for n, _ in indexer.named_parameters()}
        for d, (a, b) in enumerate(zip(cu_l[:-1], cu_l[1:])):
            S = b - a
            qd = query[a:b].unsqueeze(1).clone().requires_grad_(train)
            kd = key[a:b].unsqueeze(1).clone().requires_grad_(train)
            indexer.zero_grad(set_to_none=True)
            with torch.set_grad_enabled(train):
                o = attn(qd, kd, None, None, x[a:b], qr[a:b].unsqueeze(1), packed_seq_params=(None, rope[:S]))
            outs.append(o.detach()[:, 0])
            if train:
                (o[:, 0].float() * dout[a:b]).sum().backward()
                qg.append(qd.grad[:, 0])
                kg.append(kd.grad[:, 0])
                for n, p_ in indexer.named_parameters():
                    grads[n] = grads[n] + p_.grad.float() * (S / T)
        return torch.cat(outs), (torch.cat(qg) if train else None), (torch.cat(kg) if train else None), grads

    # indexer outputs and top-k (the projections are library GEMMs over T vs per-document rows, so
    # they may round differently: outputs within bf16 rounding, selections >= 99 % equal)
    with torch.no_grad():
        q_p, k_p, w_p = indexer.forward_before_topk(x, qr, (psp, rope))
        idx_p = indexer(x, qr, None, (psp, rope))
        inter = tot = 0
        for a, b in zip(cu_l[:-1], cu_l[1:]):
            q_d, k_d, w_d = indexer.forward_before_topk(x[a:b], qr[a:b].unsqueeze(1), (None, rope[:b - a]))
            _close(q_p[a:b].cpu(), q_d[:, 0].cpu(), rel=1e-2, name="q_idx")
            _close(k_p[a:b].cpu(), k_d[:, 0].cpu(), rel=1e-2, name="k_idx")
            _close(w_p[a:b].cpu(), w_d[:, 0].cpu(), rel=1e-2, name="w")
            i_d = indexer(x[a:b], qr[a:b].unsqueeze(1), None, (None, rope[:b - a]))[0]   # [S, K] local, score order
            for t in range(b - a):
                want = set((i_d[t][i_d[t] <= t] + a).tolist())
                got = set(idx_p[a + t][idx_p[a + t] >= 0].tolist())
                assert all(a <= j <= a + t for j in got), (a, t)        # own document, causal
                inter += len(want & got)
                tot += len(want)
        assert inter / tot >= 0.99, inter / tot
    # eval
    attn.eval()
    with torch.no_grad():
        out_p = attn(query, key, None, None, x, qr, packed_seq_params=(psp, rope))
    out_d, _, _, _ = per_doc(False)
    assert out_p.shape == (T, H * 512)
    _close(out_p.cpu(), out_d.cpu(), rel=1e-2, name="out packed vs per document")
    # training with the sparse indexer loss applied in the backward
    attn.train()
    qa, ka = query.clone().requires_grad_(), key.clone().requires_grad_()
    indexer.zero_grad(set_to_none=True)
    out_t = attn(qa, ka, None, None, x, qr, packed_seq_params=(psp, rope))
    (out_t.float() * dout).sum().backward()
    grads_p = {n: p_.grad.float().clone() for n, p_ in indexer.named_parameters()}
    out_dt, qg, kg, grads_d = per_doc(True)
    _close(out_t.detach().cpu(), out_dt.cpu(), rel=1e-2, name="train out")
    _close(qa.grad.cpu(), qg.cpu(), rel=1e-2, name="dq packed vs per document")
    _close(ka.grad.cpu(), kg.cpu(), rel=1e-2, name="dkv packed vs per document")
    for n in grads_p:
        _close(grads_p[n].cpu(), grads_d[n].cpu(), rel=2e-2, name=f"indexer {n}")


@pytest.mark.parametrize("S,B", [(200, 2), (1100, 1)])
def test_fused_qk_topk_naive_scores_are_differentiable(S, B):
    """The [B, S, S] index scores of the drop-in carry the dense score backward (what the reference's
    dense indexer loss backpropagates through): gradients of q, k, weights against float64 autograd
    of the oracle's scores, with the causal triu mask and without; S = 1100 puts more than one
    512-query chunk on the dk kernel's key tiles."""
    print(f"[index scores autograd] S={S} B={B}", flush=True)
    g = torch.Generator().manual_seed(31)
    Hi = 64
    q = (torch.randn(S, B, Hi, 128, generator=g) * 0.1).bfloat16()
    k = (torch.randn(S, B, 128, generator=g) * 0.1).bfloat16()
    w = torch.randn(S, B, Hi, generator=g) / 8
    R = torch.randn(B, S, S, generator=g)
    mask = torch.triu(torch.full((S, S), float("-inf")), 1)[None].expand(B, S, S)
    for m, causal in ((mask, None), (None, True), (None, False)):
        qd, kd, wd = (x.to(DEV).requires_grad_() for x in (q, k, w))
        sc, _ = fused_qk_topk_naive(qd, kd, wd, 32, m.to(DEV) if m is not None else None, causal=causal)
        (torch.where(torch.isfinite(sc), sc, torch.zeros_like(sc)) * R.to(DEV)).sum().backward()
        qr, kr, wr = (x.double().requires_grad_() for x in (q, k, w))
        ref = torch.stack([O.indexer_scores(qr[:, b], kr[:, b], wr[:, b], causal=causal is not False) for b in range(B)])
        (torch.where(torch.isfinite(ref), ref, torch.zeros_like(ref)) * R.double()).sum().backward()
        for name, a, r in (("dq", qd.grad, qr.grad), ("dk", kd.grad, kr.grad), ("dw", wd.grad, wr.grad)):
            _close(a.cpu(), r, name=f"{name} (mask={m is not None}, causal={causal})")


@pytest.mark.parametrize("cu", [[0, 130, 300, 301, 420], [0, 1100, 1230]])
def test_dense_indexer_loss_matches_float64_autograd(cu):
    """The dense indexer loss (the reference default, dsa_indexer_use_sparse_loss=False) over packed
    documents: loss and gradients of q_idx, k_idx, w against float64 autograd through the oracle's
    dense scores and compute_dsa_indexer_loss(sparse_loss=False), document by document (the
    reference's mean over tokens); the 1100-token document gives key tiles of several query chunks."""
    print(f"[dense indexer loss] cu={cu}", flush=True)
    from mcore_bridge_amd.dsa import indexer_kl_loss_dense
    g = torch.Generator().manual_seed(41)
    T, H, Hi, coeff = cu[-1], 16, 64, 0.4
    q = (torch.randn(T, H, 576, generator=g) * 0.1).bfloat16()
    kv = (torch.randn(T, 576, generator=g) * 0.1).bfloat16()
    qi, ki, w = _indexer_inputs(T, Hi, g)
    qd, kd, wd = (x.to(DEV).requires_grad_() for x in (qi, ki, w))
    loss = indexer_kl_loss_dense(q.to(DEV), kv.to(DEV), qd, kd, wd, W.SM_SCALE, coeff,
                                 torch.tensor(cu, dtype=torch.int32, device=DEV), max(b - a for a, b in zip(cu[:-1], cu[1:])))
    loss.backward()
    qr, kr, wr = (x.double().requires_grad_() for x in (qi, ki, w))
    ref = 0.0
    for a, b in zip(cu[:-1], cu[1:]):
        S = b - a
        I = O.indexer_scores(qr[a:b], kr[a:b], wr[a:b])
        key = kv[a:b].double()[:, None, None, :].expand(S, 1, H, 576)
        topk = torch.zeros(1, S, 1, dtype=torch.long)
        ref = ref + O.compute_dsa_indexer_loss_dense(I[None], topk, q[a:b].double()[:, None], key, W.SM_SCALE,
                                                     coeff, False) * (S / T)
    ref.backward()
    assert abs(loss.item() - ref.item()) <= 2e-3 * abs(ref.item()) + 1e-7, (loss.item(), ref.item())
    for name, a, r in (("dq_idx", qd.grad, qr.grad), ("dk_idx", kd.grad, kr.grad), ("dw", wd.grad, wr.grad)):
        _close(a.cpu(), r, name=name)


def test_dsattention_dense_loss_matches_the_separate_op():
    """DSAttention with use_sparse_loss=False (the reference default): the training output equals the
    eval output, last_indexer_loss equals indexer_kl_loss_dense on the indexer's outputs (batch rows
    as documents), and the indexer parameters receive gradients through the dense score backward."""
    from mcore_bridge_amd.dsa import DSAIndexer, DSAttention, indexer_kl_loss_dense
    print("[DSAttention dense loss]", flush=True)
    g = torch.Generator().manual_seed(57)
    S, B, H, hidden, qlr, Hi, K = 120, 2, 16, 256, 192, 64, 40
    indexer = DSAIndexer(hidden, qlr, index_n_heads=Hi, index_topk=K, device=DEV)
    with torch.no_grad():
        for p_ in indexer.parameters():
            p_.copy_((torch.randn(p_.shape, generator=g) * 0.05).to(p_.dtype))
        indexer.k_norm.weight.add_(1.0)
    attn = DSAttention(indexer, W.SM_SCALE, loss_coeff=0.25, use_sparse_loss=False)
    query = (torch.randn(S, B, H, 576, generator=g) * 0.1).bfloat16().to(DEV)
    key = (torch.randn(S, B, 576, generator=g) * 0.1).bfloat16().to(DEV)
    x = torch.randn(S, B, hidden, generator=g).bfloat16().to(DEV)
    qr = torch.randn(S, B, qlr, generator=g).bfloat16().to(DEV)
    psp = (None, (torch.rand(S, 1, 1, 64, generator=g) * 200).to(DEV))
    attn.eval()
    with torch.no_grad():
        out_e = attn(query, key, None, None, x, qr, packed_seq_params=psp)
    attn.train()
    out_t = attn(query, key, None, None, x, qr, packed_seq_params=psp)
    assert torch.equal(out_t.detach(), out_e)
    (out_t.float() * 0.01).sum().backward()
    for n, p_ in indexer.named_parameters():
        assert p_.grad is not None and bool(torch.isfinite(p_.grad).all()) and p_.grad.abs().sum() > 0, n
    with torch.no_grad():
        q_i, k_i, w = indexer.forward_before_topk(x, qr, psp)
        cu = torch.arange(0, (B + 1) * S, S, device=DEV, dtype=torch.int32)
        ref = indexer_kl_loss_dense(query.transpose(0, 1).reshape(B * S, H, 576), key.transpose(0, 1).reshape(B * S, 576),
                                    q_i.transpose(0, 1).reshape(B * S, Hi, 128), k_i.transpose(0, 1).reshape(B * S, 128),
                                    w.transpose(0, 1).reshape(B * S, Hi), W.SM_SCALE, 0.25, cu, S)
    torch.testing.assert_close(attn.last_indexer_loss, ref, rtol=1e-5, atol=1e-8)


def test_fused_attention_with_indexer_loss_honours_the_workspace_cap():
    """With ops.set_backward_workspace_limit below the one-pass size, the fused attention + indexer
    loss backward runs the capped passes (target recomputed from the forward LSE) and gives the
    uncapped result: the same loss and indexer gradients up to the bf16 rounding of the staged P,
    dq bit-identical, dkv within the rounding of the pass order."""
    print("[fused attention + indexer loss under a workspace cap]", flush=True)
    from mcore_bridge_amd.dsa import sparse_mla_with_indexer_loss
    g = torch.Generator().manual_seed(37)
    T, H, Hi, K = 700, 64, 64, 128
    q = (torch.randn(T, H, 576, generator=g) * 0.1).bfloat16().to(DEV)
    kv = (torch.randn(T, 576, generator=g) * 0.1).bfloat16().to(DEV)
    qi, ki, w = (x.to(DEV) for x in _indexer_inputs(T, Hi, g))
    idx = _idx_case(T, K, g, cu=[0, 400, T]).to(DEV)
    dout = (torch.randn(T, H, 512, generator=g) * 0.01).bfloat16().to(DEV)
    sc, coeff = W.SM_SCALE, 0.3
    cap = ops.bwd_workspace_bytes_chunked(T, T, H, K, 256)
    assert cap < ops.bwd_workspace_bytes(T, T, H, K)
    res = []
    for limit in (0, cap):
        ops.set_backward_workspace_limit(limit)
        try:
            assert ops.backward_takes_one_pass(T, T, H, K) == (limit == 0)
            leaves = [x.clone().requires_grad_() for x in (q, kv, qi, ki, w)]
            out, loss = sparse_mla_with_indexer_loss(*leaves[:2], idx, *leaves[2:], sc, coeff, True)
            (out.float() * dout.float()).sum().backward()
            torch.cuda.synchronize()
            res.append((loss.clone(), [x.grad.clone() for x in leaves]))
        finally:
            ops.set_backward_workspace_limit(0)
    (la, ga), (lb, gb) = res
    torch.testing.assert_close(lb, la, rtol=2e-3, atol=1e-7)
    assert torch.equal(ga[0], gb[0]), "dq differs under the cap"
    err = ((gb[1].double() - ga[1].double()).norm() / ga[1].double().norm()).item()
    assert err < 1e-2, f"dkv: normalised difference {err:.2e}"
    for name, a, b in zip(("q_idx", "k_idx", "w"), ga[2:], gb[2:]):
        err = ((b.double() - a.double()).norm() / a.double().norm()).item()
        assert err < 1e-2, f"{name}: normalised difference {err:.2e}"


def test_uncapped_backward_runs_in_passes_when_the_device_is_short(monkeypatch):
    """With no workspace limit set, a backward whose one-pass workspace exceeds what the device can
    still allocate runs capped passes instead (the availability probe is patched to report a
    budget below the one-pass size): dq bit-identical to one pass, dkv within the rounding of the
    pass order, and the fused indexer-loss backward reports it will not take one pass."""
    print("[uncapped backward under a short device budget]", flush=True)
    from mcore_bridge_amd import _lib
    g = torch.Generator().manual_seed(41)
    T, H, K = 900, 64, 128
    q = (torch.randn(T, H, 576, generator=g) * 0.1).bfloat16().to(DEV)
    kv = (torch.randn(T, 576, generator=g) * 0.1).bfloat16().to(DEV)
    idx = _idx_case(T, K, g, cu=[0, 500, T]).to(DEV)
    dout = (torch.randn(T, H, 512, generator=g) * 0.01).bfloat16().to(DEV)
    out, lse = ops.sparse_mla_fwd(q, kv, idx, W.SM_SCALE, True)
    one = ops.bwd_workspace_bytes(T, T, H, K)
    dq_a, dkv_a = ops.sparse_mla_bwd(q, kv, idx, out, dout, lse, W.SM_SCALE, True)
    assert ops.backward_takes_one_pass(T, T, H, K, q.device)
    budget = ops.bwd_workspace_bytes_chunked(T, T, H, K, 256)
    assert budget < one
    monkeypatch.setattr(ops, "available_device_bytes", lambda device: int(budget / ops._AUTO_CAP_SHARE) + 1)
    sizes = []
    real_call = _lib.call

    def spy(name, *args):
        if name == "dsa_sparse_mla_bwd_ex":
            sizes.append(args[-3])
        return real_call(name, *args)

    monkeypatch.setattr(_lib, "call", spy)
    assert not ops.backward_takes_one_pass(T, T, H, K, q.device)
    dq_b, dkv_b = ops.sparse_mla_bwd(q, kv, idx, out, dout, lse, W.SM_SCALE, True)
    torch.cuda.synchronize()
    assert sizes and sizes[0] < one, f"workspace {sizes} not capped below the one-pass {one}"
    assert torch.equal(dq_a, dq_b), "dq differs in passes"
    err = ((dkv_b.double() - dkv_a.double()).norm() / dkv_a.double().norm()).item()
    assert err < 1e-2, f"dkv: normalised difference {err:.2e}"


def test_dense_indexer_loss_of_an_empty_batch_is_zero():
    """T = 0: the dense indexer loss is 0 and its backward gives empty gradients (no kernel is called
    with zero key columns)."""
    print("[dense indexer loss] empty batch", flush=True)
    from mcore_bridge_amd.dsa import indexer_kl_loss_dense
    q = torch.empty(0, 16, 576, dtype=torch.bfloat16, device=DEV)
    kv = torch.empty(0, 576, dtype=torch.bfloat16, device=DEV)
    qi = torch.empty(0, 64, 128, dtype=torch.bfloat16, device=DEV, requires_grad=True)
    ki = torch.empty(0, 128, dtype=torch.bfloat16, device=DEV, requires_grad=True)
    w = torch.empty(0, 64, dtype=torch.float32, device=DEV, requires_grad=True)
    loss = indexer_kl_loss_dense(q, kv, qi, ki, w, W.SM_SCALE, 0.5)
    assert float(loss.detach()) == 0.0
    loss.backward()
    assert qi.grad.shape == qi.shape and ki.grad.shape == ki.shape and w.grad.shape == w.shape
