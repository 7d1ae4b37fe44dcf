"""GPU parity of the HIP kernels (through the C ABI via mcore_bridge_amd.ops) against the CPU oracle.

Bars: top-k indices bit-exact when computed from identical fp32 scores (ties to
the lower index), >= 99.9 % set overlap from bf16 inputs; outputs and gradients within
rtol 2e-2 / atol 2e-2 of the float64 oracle -- plus a normalised-error check (the absolute
tolerance alone would accept near-zero gradients).
"""
import math

import pytest
import torch

from oracle import dsa_oracle as O
from mcore_bridge_amd import ops, workloads as W
from mcore_bridge_amd.dsa import fused_qk_topk_naive, sparse_mla_attention

pytestmark = pytest.mark.gpu
DEV = "cuda"
RTOL = ATOL = 2e-2


def _close(got, ref, rel=1e-2, name=""):
    got = got.double().cpu()
    ref = ref.double().cpu()
    torch.testing.assert_close(got, ref, rtol=RTOL, atol=ATOL, msg=lambda m: f"{name}: {m}")
    err = (got - ref).norm() / ref.norm().clamp_min(1e-30)
    assert err < rel, f"{name}: normalised error {err:.3e} >= {rel}"


def _rows(cu, T, causal=True):
    start, end = O.doc_bounds(T, torch.tensor(cu))
    t = torch.arange(T)
    ln = (t - start + 1) if causal else (end - start)
    return start.to(torch.int32), ln.to(torch.int32)


# ------------------------------------------------------------------ K2 top-k
# (24 rows longer than 16384 keys take the split selection: n = 16484 leaves a last slice shorter than
#  k, 65268 is cfg5's longest cache with 4 slices, 140000 gives more candidates than LDS caches)
@pytest.mark.parametrize("n,k", [(300, 64), (2048, 2048), (5000, 2048), (20000, 2048), (700, 129), (64, 1),
                                 (16484, 2048), (65268, 2048), (140000, 2048), (40000, 4096)])
def test_topk_bit_exact_from_fp32_scores(n, k):
    print(f"[topk] n={n} k={k}", flush=True)
    g = torch.Generator().manual_seed(n + k)
    rows = 24
    sc = torch.randn(rows, n, generator=g)
    sc[: rows // 2] = torch.round(sc[: rows // 2] * 3) / 3          # many exact ties
    sc[2, :] = 0.0                                                   # all ties
    sc[3, :] = torch.where(torch.rand(n, generator=g) < 0.5, -0.0, 0.0)  # signed zeros tie too
    ln = torch.randint(1, n + 1, (rows,), generator=g).to(torch.int32)
    ln[0] = n
    ln[1] = min(n, k)
    base = torch.randint(0, 1000, (rows,), generator=g).to(torch.int32)
    got = ops.topk(sc.to(DEV), base.to(DEV), ln.to(DEV), k).cpu().long()
    for r in range(rows):
        row = sc[r].double().clone()
        row[int(ln[r]):] = float("-inf")
        ref = O.topk_indices(row[None], k)[0]
        ref = torch.where(ref >= 0, ref + int(base[r]), ref)
        assert torch.equal(got[r], ref[:k] if ref.numel() >= k else torch.cat([ref, ref.new_full((k - ref.numel(),), -1)])), r


@pytest.mark.parametrize("n,k", [(16484, 2048), (32768, 2048), (40000, 4096), (140000, 2048), (20000, 64)])
def test_topk_one_workgroup_long_rows_bit_exact(n, k):
    """Rows longer than the 16384-entry LDS cache in one workgroup per row (no split workspace):
    the three-pass candidate path, and its fallback when the threshold's 12-bit bin holds more
    keys than the candidate list (rows of all-equal or few distinct values)."""
    import ctypes
    from mcore_bridge_amd import _lib
    print(f"[topk one workgroup, long rows] n={n} k={k}", flush=True)
    g = torch.Generator().manual_seed(n + 3 * k)
    rows = 12
    sc = torch.randn(rows, n, generator=g) * torch.rand(rows, 1, generator=g) * 4
    sc[0] = 0.0                                                      # all ties: fallback
    sc[1] = torch.round(sc[1] * 2) / 2                               # few distinct values
    sc[2] = torch.where(torch.rand(n, generator=g) < 0.5, -0.0, 0.0)  # signed zeros tie
    sc[3, : n // 2] = 1.0                                            # a wide tie at the threshold
    sc[4] = torch.relu(sc[4])                                        # many exact zeros below
    ln = torch.randint(k + 1, n + 1, (rows,), generator=g).to(torch.int32)
    ln[:6] = n
    base = torch.randint(0, 1000, (rows,), generator=g).to(torch.int32)
    scd, bd, ld = sc.to(DEV), base.to(DEV), ln.to(DEV)
    out = torch.empty(rows, k, dtype=torch.int32, device=DEV)
    P = lambda t: ctypes.c_void_p(t.data_ptr())
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    assert _lib.load().dsa_topk(P(scd), n, P(bd), P(ld), rows, k, P(out), None, None, 0, st) == 0
    got = out.cpu().long()
    for r in range(rows):
        row = sc[r].double().clone()
        row[int(ln[r]):] = float("-inf")
        ref = O.topk_indices(row[None], k)[0] + int(base[r])
        assert torch.equal(got[r], ref), r


@pytest.mark.parametrize("case", ["random", "quantised", "sample_spikes", "few_values", "rising"])
@pytest.mark.parametrize("n,k", [(12000, 2048), (40000, 4096), (32768, 2048)])
def test_topk_sampled_threshold_rows_bit_exact(case, n, k):
    """Rows the sampled-threshold selection takes (n >= 4096, k small against n): the bound from
    2048 evenly spaced entries is exact on random rows; quantised rows put many keys at the
    threshold (only the lowest-positioned `need` of them are taken); rows whose sampled positions
    hold the largest values make the bound miss low (fewer than k candidates) and rows of few
    distinct values make it miss high (more than the list holds): both fall back to the exact
    paths.  Every row equals the oracle's selection."""
    print(f"[topk sampled threshold] case={case} n={n} k={k}", flush=True)
    g = torch.Generator().manual_seed(n + k + len(case))
    rows = 8
    sc = torch.randn(rows, n, generator=g)
    if case == "quantised":
        sc = torch.round(sc * 200) / 200
    elif case == "sample_spikes":
        starts = (torch.arange(64, dtype=torch.int64) * (n - 32) // 63) // 4 * 4   # the sampled runs
        pos = (starts[:, None] + torch.arange(32)).flatten()
        sc[:, pos] = 10.0 + torch.rand(rows, pos.numel(), generator=g)
    elif case == "few_values":
        sc = torch.round(sc * 2) / 2
    elif case == "rising":
        sc = sc * 0.1 + torch.linspace(0, 4, n)[None]
    ln = torch.full((rows,), n, dtype=torch.int32)
    ln[1::2] = torch.randint(max(k + 1, 4096), n + 1, (rows // 2,), generator=g).to(torch.int32)
    base = torch.randint(0, 1000, (rows,), generator=g).to(torch.int32)
    got = ops.topk(sc.to(DEV), base.to(DEV), ln.to(DEV), k).cpu().long()
    for r in range(rows):
        row = sc[r].double().clone()
        row[int(ln[r]):] = float("-inf")
        ref = O.topk_indices(row[None], k)[0] + int(base[r])
        assert torch.equal(got[r], ref), r


def test_topk_split_equals_one_workgroup_cfg5_full_size():
    """cfg5's 64 cache lengths (up to 65,265 keys): the split selection (slices + merge, through
    the workspace) returns the one-workgroup-per-row selection's indices bit for bit, on scores
    with many exact ties and on the real indexer scores of the decode leg."""
    import ctypes
    from mcore_bridge_amd import _lib
    print("[topk split vs one workgroup, cfg5 full size]", flush=True)
    cfg = W.CONFIGS["cfg5"]
    lens = torch.tensor(cfg.decode_lens, dtype=torch.int32)
    B, L, K = lens.numel(), int(lens.max()), cfg.K
    pitch = (L + 3) // 4 * 4
    g = torch.Generator(device=DEV).manual_seed(5)
    base = (torch.cumsum(lens, 0) - lens).to(torch.int32).to(DEV)
    ln = lens.to(DEV)
    lib = _lib.load()
    nws = int(lib.dsa_topk_workspace_size(B, pitch, K))
    assert nws > 0
    ws = torch.empty(nws, dtype=torch.uint8, device=DEV)
    P = lambda t: ctypes.c_void_p(t.data_ptr())
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    sc_ties = torch.round(torch.randn(B, pitch, generator=g, device=DEV) * 4) / 4
    qi = (torch.randn(B, cfg.Hi, cfg.Di, generator=g, device=DEV) * 0.1).bfloat16()
    ki = (torch.randn(int(lens.sum()), cfg.Di, generator=g, device=DEV) * 0.1).bfloat16()
    w = torch.randn(B, cfg.Hi, generator=g, device=DEV) / 8
    sc_real = ops.indexer_scores(qi, ki, w, base, ln, L, pitch)
    res = {}
    for name, sc in (("ties", sc_ties), ("indexer", sc_real)):
        got = res[name] = torch.empty(B, K, dtype=torch.int32, device=DEV)
        ref = torch.empty(B, K, dtype=torch.int32, device=DEV)
        cnt = torch.empty(B, dtype=torch.int32, device=DEV)
        assert lib.dsa_topk(P(sc), pitch, P(base), P(ln), B, K, P(got), P(cnt), P(ws), nws, st) == 0
        assert lib.dsa_topk(P(sc), pitch, P(base), P(ln), B, K, P(ref), None, None, 0, st) == 0
        torch.cuda.synchronize()
        assert torch.equal(got, ref), name
        assert (cnt == K).all(), name
        assert torch.equal(ops.topk(sc, base, ln, K), ref), name     # the op takes the split path
    # one row against the float64 oracle (the longest)
    r = int(lens.argmax())
    row = sc_ties[r, :L].double().cpu()
    want = O.topk_indices(row[None], K)[0] + int(base[r])
    assert torch.equal(res["ties"][r].cpu().long(), want)


# ------------------------------------------------------------------ K1 indexer
# (at most 512 queries of 128-dim rows take the one-query-per-workgroup form of the scan: the
#  20-head case has heads that do not fill the 32-head MFMA tiles and rows of 1 and 34 keys)
@pytest.mark.parametrize("Hi,Di,cu", [(64, 128, [0, 700]), (4, 64, [0, 300, 512]), (64, 128, [0, 100, 2500, 2600]),
                                      (20, 128, [0, 1, 35, 300]), (64, 128, [0, 512])])
def test_indexer_scores_bf16(Hi, Di, cu):
    print(f"[indexer bf16] Hi={Hi} Di={Di} cu={cu}", flush=True)
    T = cu[-1]
    g = torch.Generator().manual_seed(T)
    q = (torch.randn(T, Hi, Di, generator=g) * 0.1).bfloat16()
    k = (torch.randn(T, Di, generator=g) * 0.1).bfloat16()
    w = torch.randn(T, Hi, generator=g) / 8
    base, ln = _rows(cu, T)
    L = int(ln.max())
    got = ops.indexer_scores(q.to(DEV), k.to(DEV), w.to(DEV), base.to(DEV), ln.to(DEV), L, L, None, None, True).cpu()
    ref = O.indexer_scores(q, k, w, torch.tensor(cu, dtype=torch.int32))
    for t in range(T):
        a, n = int(base[t]), int(ln[t])
        torch.testing.assert_close(got[t, :n].double(), ref[t, a:a + n], rtol=1e-4, atol=1e-5)
        assert torch.isinf(got[t, n:]).all()


def test_indexer_scores_fp8():
    print("[indexer fp8]", flush=True)
    T, Hi, Di = 900, 64, 128
    g = torch.Generator().manual_seed(7)
    q8, qs = O.quantize_e4m3_rows(torch.randn(T, Hi, Di, generator=g))
    k8, ks = O.quantize_e4m3_rows(torch.randn(T, Di, generator=g))
    w = torch.randn(T, Hi, generator=g) / 8
    base, ln = _rows([0, T], T)
    got = ops.indexer_scores(q8.to(DEV), k8.to(DEV), w.to(DEV), base.to(DEV), ln.to(DEV), T, T, qs.to(DEV),
                             ks.to(DEV), False).cpu()
    ref = O.indexer_scores(q8.float(), k8.float(), w, q_scale=qs, k_scale=ks)
    # fp8 products are exact, but the gfx950 fp8 MFMA does not accumulate bit-for-bit like fp32
    # FMAs (measured ~3e-4 relative on single scores); the bar that matters is the selection.
    for t in range(0, T, 7):
        torch.testing.assert_close(got[t, :t + 1].double(), ref[t, :t + 1], rtol=2e-3, atol=2e-3)
    got_idx = O.topk_indices(torch.where(torch.isfinite(ref), got.double(), ref), 256)
    ref_idx = O.topk_indices(ref, 256)
    inter = sum(len(set(a[a >= 0].tolist()) & set(b[b >= 0].tolist())) for a, b in zip(got_idx, ref_idx))
    assert inter / (ref_idx >= 0).sum().item() >= 0.999


@pytest.mark.parametrize("cfgname,S", [("cfg1", 512), ("cfg2", 3000)])
def test_indexer_topk_end_to_end(cfgname, S):
    print(f"[indexer+topk] {cfgname} S={S}", flush=True)
    cfg = W.CONFIGS[cfgname]
    x = W.make_prefill(cfg, S=S)
    q, k, w = x["q_idx"].bfloat16(), x["k_idx"].bfloat16(), x["w"]
    idx, sc = ops.indexer_topk(q.to(DEV), k.to(DEV), w.to(DEV), cfg.K, return_scores=True)
    idx = idx.cpu().long()
    # bit-exact against the oracle's selection applied to the kernel's own fp32 scores
    assert torch.equal(idx, O.topk_indices(sc.cpu().double(), cfg.K))
    # >= 99.9 % set overlap against float64 scores of the same bf16 inputs
    ref = O.topk_indices(O.indexer_scores(q, k, w), cfg.K)
    inter = tot = 0
    for t in range(S):
        a = set(idx[t][idx[t] >= 0].tolist())
        b = set(ref[t][ref[t] >= 0].tolist())
        inter += len(a & b)
        tot += len(b)
    assert inter / tot >= 0.999, inter / tot



# ------------------------------------------------------------------ K0 indexer prologue
def _prologue_case(T, Hi, seed, scale=2.0):
    g = torch.Generator().manual_seed(seed)
    q_lin = (torch.randn(T, Hi, 128, generator=g) * scale).bfloat16()
    k_lin = (torch.randn(T, 128, generator=g) * scale + 0.5).bfloat16()
    w_lin = torch.randn(T, Hi, generator=g).bfloat16()
    lw = 1 + 0.2 * torch.randn(128, generator=g)
    lb = 0.1 * torch.randn(128, generator=g)
    fr = torch.rand(T, 64, generator=g) * 3000            # angles of positions up to ~16k
    return q_lin, k_lin, w_lin, lw, lb, fr


def _bf16_rows_close(got, ref, name):
    # every step rounds to bf16 like the reference; the kernel's fp32 sums (LayerNorm, Hadamard)
    # and cos/sin may sit on the other side of a rounding boundary, so: >= 99.9 % bit-equal,
    # the rest within 2 bf16 ulp (relative) or 1e-3 of the row's magnitude
    got, ref = got.float().cpu(), ref.float().cpu()
    same = (got == ref).float().mean().item()
    assert same >= 0.999, f"{name}: only {same:.5f} bit-equal"
    d = (got - ref).abs()
    lim = torch.maximum(ref.abs() * 2 ** -6, ref.abs().amax(-1, keepdim=True) * 1e-3)
    assert (d <= lim).all(), f"{name}: max excess {(d - lim).max().item():.3e}"


@pytest.mark.parametrize("dei,ri", [(False, False), (True, False), (False, True), (True, True)])
def test_indexer_prologue_bf16(dei, ri):
    print(f"[indexer prologue bf16] deinterleave={dei} rotary_interleaved={ri}", flush=True)
    T, Hi = 333, 64
    q_lin, k_lin, w_lin, lw, lb, fr = _prologue_case(T, Hi, 11 + 2 * dei + ri)
    rq, rk, rw = O.indexer_prologue(q_lin, k_lin, w_lin, lw, lb, fr, eps=1e-6, mscale=1.07, deinterleave=dei,
                                    rotary_interleaved=ri)
    q, qs, k, ks, w = ops.indexer_prologue(q_lin.to(DEV), k_lin.to(DEV), w_lin.to(DEV), lw.to(DEV), lb.to(DEV),
                                           fr.to(DEV), 1e-6, 1.07, dei, ri)
    assert q.dtype == torch.bfloat16 and qs.numel() == 0 and ks.numel() == 0
    assert torch.equal(w.cpu(), rw.float())                 # two bf16 roundings, bit for bit
    _bf16_rows_close(q, rq, "q")
    _bf16_rows_close(k, rk, "k")


def test_indexer_prologue_fp8_and_strided_inputs():
    print("[indexer prologue fp8]", flush=True)
    T, Hi = 257, 16
    q_lin, k_lin, w_lin, lw, lb, fr = _prologue_case(T, Hi, 21, scale=5.0)
    q_lin[3] = 0                                            # all-zero rows -> scale 1
    rq, rk, rw = O.indexer_prologue(q_lin, k_lin, w_lin, lw, lb, fr, eps=1e-6, mscale=1.0, deinterleave=True,
                                    rotary_interleaved=False)
    # q_lin as a column slice of a wider GEMM output, k_lin with a padded token stride
    wide = torch.zeros(T, Hi * 128 + 64, dtype=torch.bfloat16)
    wide[:, :Hi * 128] = q_lin.reshape(T, -1)
    kpad = torch.zeros(T, 192, dtype=torch.bfloat16)
    kpad[:, :128] = k_lin
    args = (wide.to(DEV)[:, :Hi * 128], kpad.to(DEV)[:, :128], w_lin.to(DEV), lw.to(DEV), lb.to(DEV), fr.to(DEV),
            1e-6, 1.0, True, False)
    q8, qs, k8, ks, w = ops.indexer_prologue(*args, True)
    qb, _, kb, _, wb = ops.indexer_prologue(*args, False)
    assert q8.dtype == torch.float8_e4m3fn and qs.shape == (T, Hi) and ks.shape == (T,)
    assert torch.equal(w.cpu(), rw.float()) and torch.equal(wb.cpu(), rw.float())
    # the bf16 rows meet the bf16 bar; the fp8 rows are exactly the oracle's absmax e4m3fn
    # quantisation (RNE, scale = absmax / 448) of those bf16 rows, codes and scales bit for bit
    _bf16_rows_close(qb, rq, "q")
    _bf16_rows_close(kb, rk, "k")
    for got8, gs, own in ((q8, qs, qb), (k8, ks, kb)):
        r8, rs = O.quantize_e4m3_rows(own.cpu())
        assert torch.equal(gs.cpu(), rs)
        assert torch.equal(got8.cpu().view(torch.uint8), r8.view(torch.uint8))
    assert float(qs[3].max()) == 1.0 and (q8[3].cpu().float() == 0).all()


def test_indexer_prologue_then_topk_end_to_end():
    # Megatron layout, projections included: x, qr -> GEMMs -> fused prologue -> K1 + K2,
    # against the oracle prologue and selection on the same projected rows
    print("[indexer prologue + topk] S=1500", flush=True)
    S, B, hidden, lora, Hi, K = 1500, 1, 256, 192, 64, 256
    g = torch.Generator().manual_seed(31)
    x = (torch.randn(S, B, hidden, generator=g)).bfloat16()
    qr = (torch.randn(S, B, lora, generator=g)).bfloat16()
    wq_b = (torch.randn(Hi * 128, lora, generator=g) / lora ** 0.5).bfloat16()
    wk = (torch.randn(128, hidden, generator=g) / hidden ** 0.5).bfloat16()
    wproj = (torch.randn(Hi, hidden, generator=g) / hidden ** 0.5).bfloat16()
    lw, lb = 1 + 0.1 * torch.randn(128, generator=g), 0.1 * torch.randn(128, generator=g)
    inv = 1.0 / (10000 ** (torch.arange(0, 64, 2, dtype=torch.float32) / 64))
    ang = torch.arange(S, dtype=torch.float32)[:, None] * inv
    rope = torch.cat([ang, ang], -1).view(S, 1, 1, 64)
    from mcore_bridge_amd.dsa import indexer_forward_before_topk
    q, k, w = indexer_forward_before_topk(x.to(DEV), qr.to(DEV), wq_b.to(DEV), wk.to(DEV), lw.to(DEV), lb.to(DEV),
                                          wproj.to(DEV), rope.to(DEV), index_n_heads=Hi, eps=1e-6, mscale=1.0)
    assert q.shape == (S, B, Hi, 128) and k.shape == (S, B, 128) and w.shape == (S, B, Hi)
    # oracle from the same projected rows (the GEMMs are the library's; their rounding is not
    # the prologue's)
    q_lin = torch.nn.functional.linear(qr.to(DEV).reshape(S, -1), wq_b.to(DEV)).cpu().view(S, Hi, 128)
    k_lin = torch.nn.functional.linear(x.to(DEV).reshape(S, -1), wk.to(DEV)).cpu()
    w_lin = torch.nn.functional.linear(x.to(DEV).reshape(S, -1), wproj.to(DEV)).cpu()
    rq, rk, rw = O.indexer_prologue(q_lin, k_lin, w_lin, lw, lb, rope.view(S, 64), eps=1e-6, mscale=1.0,
                                    deinterleave=False, rotary_interleaved=False)
    _bf16_rows_close(q[:, 0], rq, "q")
    _bf16_rows_close(k[:, 0], rk, "k")
    idx = ops.indexer_topk(q[:, 0].contiguous(), k[:, 0].contiguous(), w[:, 0].contiguous(), K).cpu()
    ref = O.topk_indices(O.indexer_scores(rq, rk, rw.float()), K)
    inter = tot = 0
    for t in range(S):
        a = set(idx[t][idx[t] >= 0].tolist())
        b = set(ref[t][ref[t] >= 0].tolist())
        inter += len(a & b)
        tot += len(b)
    assert inter / tot >= 0.999, inter / tot




def test_dsa_indexer_module_forward_with_scores():
    # the DSAIndexer mirror end to end (its own parameters, (psp, rotary_pos_emb) tuple, causal
    # mask): indices in torch.topk order over the oracle's prologue + scores of the same
    # projected rows, >= 99.9 % overlap; the scores returned are the kernel's for those rows
    print("[DSAIndexer module] S=700 B=2", flush=True)
    from mcore_bridge_amd.dsa import DSAIndexer
    S, B, hidden, lora, K = 700, 2, 256, 128, 128
    torch.manual_seed(41)
    ix = DSAIndexer(hidden, lora, index_n_heads=64, index_topk=K, attention_scaling=1.1,
                    dsa_indexer_rotary_interleaved=True, device=DEV)
    with torch.no_grad():
        for p_ in ix.parameters():
            p_.copy_(torch.randn_like(p_.float()).mul_(p_.shape[-1] ** -0.5 if p_.dim() == 2 else 0.1).add_(
                1.0 if p_ is ix.k_norm.weight else 0.0))
    x = torch.randn(S, B, hidden, device=DEV).bfloat16()
    qr = torch.randn(S, B, lora, device=DEV).bfloat16()
    inv = 1.0 / (10000 ** (torch.arange(0, 64, 2, dtype=torch.float32) / 64))
    ang = torch.arange(S, dtype=torch.float32)[:, None] * inv
    rope = torch.stack([ang, ang], -1).reshape(S, 1, 1, 64).to(DEV)          # interleaved duplication
    mask = torch.triu(torch.full((S, S), float("-inf"), device=DEV), diagonal=1).expand(B, S, S)
    sc, idx = ix.forward_with_scores(x, qr, mask, (None, rope))
    assert sc.shape == (B, S, S) and idx.shape == (B, S, K) and idx.dtype == torch.int64
    for b in range(B):
        q_lin = torch.nn.functional.linear(qr[:, b], ix.linear_wq_b.weight).cpu().view(S, 64, 128)
        k_lin = torch.nn.functional.linear(x[:, b], ix.linear_wk.weight).cpu()
        w_lin = torch.nn.functional.linear(x[:, b], ix.linear_weights_proj.weight).cpu()
        rq, rk, rw = O.indexer_prologue(q_lin, k_lin, w_lin, ix.k_norm.weight.detach().cpu(),
                                        ix.k_norm.bias.detach().cpu(), rope.view(S, 64).cpu(), eps=1e-6,
                                        mscale=1.1, deinterleave=True, rotary_interleaved=False)
        ref = O.topk_reference_order(O.indexer_scores(rq, rk, rw.float()), K)
        got = idx[b].cpu()
        inter = tot = 0
        for t in range(S):
            a = set(got[t][: min(K, t + 1)].tolist())
            r = set(ref[t][ref[t] >= 0].tolist())
            inter += len(a & r)
            tot += len(r)
        assert inter / tot >= 0.999, inter / tot
        # the returned order is the score order of the returned scores (ties to the lower key)
        vals = torch.gather(sc[b].cpu(), 1, got.clamp(min=0))
        assert (vals[:, 1:] <= vals[:, :-1]).all()


# ------------------------------------------------------------------ MLA absorption adapter
@pytest.mark.parametrize("S,B,H,K", [(160, 2, 16, 48), (300, 1, 128, 128)])
def test_absorbed_mla_adapter_matches_unabsorbed_reference(S, B, H, K):
    # the caller's un-absorbed tensors (multi_latent_attention.py:101-178) -> absorbed kernels;
    # reference: the un-fused attention on key_h = [c W_UK_h^T, k_pe], value_h = c W_UV_h^T in
    # float64, output and the gradients of every input, weight included
    print(f"[absorbed MLA adapter] S={S} B={B} H={H} K={K}", flush=True)
    from mcore_bridge_amd.dsa import absorbed_mla_sparse_attention
    g = torch.Generator().manual_seed(S + H)
    dn, dr, dc, dv = 128, 64, 512, 128
    qn = (torch.randn(S, B, H, dn, generator=g)).bfloat16()
    qp = (torch.randn(S, B, H, dr, generator=g)).bfloat16()
    c = (torch.randn(S, B, dc, generator=g)).bfloat16()
    kp = (torch.randn(S, B, dr, generator=g)).bfloat16()
    W = (torch.randn(H * (dn + dv), dc, generator=g) / dc ** 0.5).bfloat16()
    idx = torch.stack([_attn_case(S, 1, K, S + b)[2] for b in range(B)]).long()   # [B, S, K] per batch
    scale = (dn + dr) ** -0.5
    dout = (torch.randn(S, B, H * dv, generator=g) * 0.1).bfloat16()
    # reference, float64 on the CPU
    ins = [x.double().requires_grad_() for x in (qn, qp, c, kp, W)]
    rqn, rqp, rc, rkp, rW = ins
    Wh = rW.view(H, dn + dv, dc)
    key = torch.cat([torch.einsum("sbc,hnc->sbhn", rc, Wh[:, :dn]), rkp[:, :, None].expand(S, B, H, dr)], -1)
    val = torch.einsum("sbc,hvc->sbhv", rc, Wh[:, dn:])
    ref = O.unabsorbed_sparse_attention(torch.cat([rqn, rqp], -1), key, val, idx, scale)
    ref.backward(dout.double())
    # absorbed, on the GPU
    gins = [x.to(DEV).requires_grad_() for x in (qn, qp, c, kp, W)]
    out = absorbed_mla_sparse_attention(*gins, idx.to(DEV), scale)
    out.backward(dout.to(DEV))
    _close(out.detach(), ref.detach(), name="out")
    for name, a, r in zip(("dq_no_pe", "dq_pos_emb", "dkv_compressed", "dk_pos_emb", "dW_kv_up"), gins, ins):
        _close(a.grad, r.grad, name=name)


# ------------------------------------------------------------------ K3 forward
def _attn_case(T, H, K, seed, cu=None, pad=0.1):
    g = torch.Generator().manual_seed(seed)
    q = (torch.randn(T, H, 576, generator=g) * 0.1).bfloat16()
    kv = (torch.randn(T, 576, generator=g) * 0.1).bfloat16()
    vis = O.visibility_mask(T, None if cu is None else torch.tensor(cu, dtype=torch.int32), True)
    idx = torch.full((T, K), -1, dtype=torch.int32)
    for t in range(T):
        cand = torch.nonzero(vis[t]).flatten()
        cand = cand[torch.randperm(cand.numel(), generator=g)][:K]
        m = cand.numel()
        if t % 5 == 0:
            m = max(1, int(m * (1 - pad)))
        idx[t, :m] = torch.sort(cand[:m]).values.to(torch.int32)
    return q, kv, idx


@pytest.mark.parametrize("T,H,K", [(300, 128, 256), (200, 16, 128), (130, 64, 100), (2100, 128, 2048)])
def test_sparse_fwd(T, H, K):
    print(f"[sparse fwd] T={T} H={H} K={K}", flush=True)
    q, kv, idx = _attn_case(T, H, K, T + H)
    out, lse = ops.sparse_mla_fwd(q.to(DEV), kv.to(DEV), idx.to(DEV), W.SM_SCALE, True)
    rows = torch.arange(T) if T <= 300 else torch.cat([torch.arange(0, 40), torch.arange(T - 60, T)])
    o_ref, l_ref = O.sparse_mla_fwd(q[rows], kv, idx[rows], W.SM_SCALE, chunk=16)
    _close(out.cpu()[rows], o_ref, name="out")
    _close(lse.cpu()[rows], l_ref, rel=1e-4, name="lse")


def test_sparse_fwd_edge_cases():
    print("[sparse fwd edges]", flush=True)
    T, H, K = 96, 32, 64
    q, kv, idx = _attn_case(T, H, K, 3)
    idx[5] = -1                                       # empty row -> out 0, lse -inf
    idx[7, 3] = T + 50                                # out of range -> ignored
    idx[9, 0] = 95                                    # future key under causal -> ignored
    idx[11] = idx[11].flip(0)                         # padding first, unsorted
    out, lse = ops.sparse_mla_fwd(q.to(DEV), kv.to(DEV), idx.to(DEV), W.SM_SCALE, True)
    ref_idx = idx.clone().long()
    ref_idx[(ref_idx >= T) | (ref_idx > torch.arange(T)[:, None])] = -1
    o_ref, l_ref = O.sparse_mla_fwd(q, kv, ref_idx, W.SM_SCALE)
    assert (out[5] == 0).all() and torch.isinf(lse[5]).all()
    _close(out.cpu(), o_ref, name="out")
    ok = torch.isfinite(l_ref)
    _close(lse.cpu()[ok], l_ref[ok], rel=1e-4, name="lse")


def test_sparse_fwd_large_logits_redo_pass():
    # scores spread far beyond the 2^64 headroom of the first block -> the recompute path
    print("[sparse fwd large logits]", flush=True)
    T, H, K = 64, 32, 64
    q, kv, idx = _attn_case(T, H, K, 4, pad=0.0)
    kv = kv.float()
    kv[40:] *= 60.0
    q = (q.float() * 8).bfloat16()
    kv = kv.bfloat16()
    out, lse = ops.sparse_mla_fwd(q.to(DEV), kv.to(DEV), idx.to(DEV), W.SM_SCALE, True)
    o_ref, l_ref = O.sparse_mla_fwd(q, kv, idx, W.SM_SCALE)
    # V rows were scaled by 60: compare at the unscaled magnitude (bf16 P rounding scales with V)
    _close(out.cpu() / 60, o_ref / 60, name="out")
    _close(lse.cpu(), l_ref, rel=1e-4, name="lse")


# ------------------------------------------------------------------ K4 backward
@pytest.mark.parametrize("T,H,K", [(160, 128, 128), (120, 16, 64), (300, 64, 256)])
def test_sparse_bwd(T, H, K):
    print(f"[sparse bwd] T={T} H={H} K={K}", flush=True)
    q, kv, idx = _attn_case(T, H, K, 100 + T)
    g = torch.Generator().manual_seed(5)
    dout = (torch.randn(T, H, 512, generator=g) * 0.01).bfloat16()
    out, lse = ops.sparse_mla_fwd(q.to(DEV), kv.to(DEV), idx.to(DEV), W.SM_SCALE, True)
    dq, dkv = ops.sparse_mla_bwd(q.to(DEV), kv.to(DEV), idx.to(DEV), out, dout.to(DEV), lse, W.SM_SCALE, True)
    o_ref, l_ref = O.sparse_mla_fwd(q, kv, idx, W.SM_SCALE)
    dq_ref, dkv_ref = O.sparse_mla_bwd(q, kv, idx, out.cpu(), dout, lse.cpu(), W.SM_SCALE)
    _close(dq.cpu(), dq_ref, name="dq")
    _close(dkv.cpu(), dkv_ref, name="dkv")


def test_autograd_through_custom_op():
    print("[autograd]", flush=True)
    T, H, K = 64, 32, 48
    q, kv, idx = _attn_case(T, H, K, 77)
    qd = q.to(DEV).requires_grad_()
    kvd = kv.to(DEV).requires_grad_()
    out = ops.sparse_mla(qd, kvd, idx.to(DEV), W.SM_SCALE, True)
    g = torch.Generator().manual_seed(1)
    dout = (torch.randn(T, H, 512, generator=g) * 0.01).bfloat16()
    out.backward(dout.to(DEV))
    q64 = q.double().requires_grad_()
    kv64 = kv.double().requires_grad_()
    ref = O.sparse_mla_fwd_dense(q64, kv64, idx, W.SM_SCALE)
    ref.backward(dout.double())
    _close(out.detach().cpu(), ref.detach(), name="out")
    _close(qd.grad.cpu(), q64.grad, name="dq")
    _close(kvd.grad.cpu(), kv64.grad, name="dkv")


# ------------------------------------------------------------------ Megatron-compatible drop-ins
def test_fused_qk_topk_naive_dropin():
    print("[fused_qk_topk_naive]", flush=True)
    cfg = W.CONFIGS["cfg1"]
    S = 256
    x = W.make_prefill(cfg, S=S)
    q = x["q_idx"].bfloat16()[:, None]
    k = x["k_idx"].bfloat16()[:, None]
    w = x["w"][:, None]
    mask = torch.triu(torch.full((S, S), float("-inf")), 1)[None]
    sc, ti = fused_qk_topk_naive(q.to(DEV), k.to(DEV), w.to(DEV), cfg.K, mask.to(DEV))
    ref_sc = O.indexer_scores(q[:, 0], k[:, 0], w[:, 0])
    fin = torch.isfinite(ref_sc)
    torch.testing.assert_close(sc[0].cpu().double()[fin], ref_sc[fin], rtol=1e-4, atol=1e-5)
    assert torch.isinf(sc[0].cpu()[~fin]).all()
    # exactly a stable torch.topk of the returned scores (score desc, ties -> lower index)
    ref_ti = O.topk_reference_order(sc[0].cpu().double().nan_to_num(neginf=-1e300), cfg.K)
    assert torch.equal(ti[0].cpu(), ref_ti)
    # without the scores (the masked tail of the score rows is then never written): the same
    # indices in the same order, padded rows included (rows t < K - 1 hold masked keys)
    for causal in (None, True):
        none, ti2 = fused_qk_topk_naive(q.to(DEV), k.to(DEV), w.to(DEV), cfg.K, mask.to(DEV), causal=causal,
                                        return_scores=False)
        assert none is None and torch.equal(ti2, ti)


def test_sparse_mla_attention_sbhd_batch2():
    print("[sparse_mla_attention sbhd]", flush=True)
    S, B, H, K = 80, 2, 32, 40
    g = torch.Generator().manual_seed(2)
    q = (torch.randn(S, B, H, 576, generator=g) * 0.1).bfloat16()
    kv = (torch.randn(S, B, 576, generator=g) * 0.1).bfloat16()
    def row(t):  # distinct keys (as any top-k yields), always including the row's own visible key
        perm = torch.randperm(S, generator=g)
        return torch.cat([torch.tensor([t]), perm[perm != t]])[:K]
    ti = torch.stack([torch.stack([row(t) for t in range(S)]) for _ in range(B)])
    out = sparse_mla_attention(q.to(DEV), kv.to(DEV), ti.to(DEV), W.SM_SCALE).cpu()
    for b in range(B):
        ref = O.naive_unfused_sparse_attn_fp32(q[:, b:b + 1].float(), kv[:, b:b + 1].float(), ti[b:b + 1], W.SM_SCALE)
        _close(out[:, b], ref[:, 0], name=f"batch {b}")


# ------------------------------------------------------------------ K5/K6 decode
def _cu(lens):
    cu = [0]
    for L in lens:
        cu.append(cu[-1] + L)
    return torch.tensor(cu, dtype=torch.int32)


def _decode_idx(lens, K, seed, device="cpu"):
    """Per sequence a sorted random distinct subset of min(K, L) of its cache rows (global ids)."""
    g = torch.Generator(device=device).manual_seed(seed)
    cu = _cu(lens).tolist()
    idx = torch.full((len(lens), K), -1, dtype=torch.int32, device=device)
    for b, L in enumerate(lens):
        m = min(K, L)
        sel = torch.randperm(L, generator=g, device=device)[:m].sort().values
        idx[b, :m] = (sel + cu[b]).to(torch.int32)
    return idx


@pytest.mark.parametrize("fp8", [False, True])
def test_decode_indexer_topk(fp8):
    lens = [3000, 5000, 20000, 1500, 700, 2048]
    print(f"[decode indexer+topk] fp8={fp8} lens={lens}", flush=True)
    cfg = W.CONFIGS["cfg5"]
    d = W.make_decode(cfg, lens=lens, H=16, seed=11)
    cu = _cu(lens)
    q, k, w = d["q_idx"], d["k_cache"], d["w"]
    if fp8:
        q8, qs = O.quantize_e4m3_rows(q * 10)
        k8, ks = O.quantize_e4m3_rows(k * 10)
        args = (q8.to(DEV), k8.to(DEV), w.to(DEV), cfg.K, cu.to(DEV), max(lens), qs.to(DEV), ks.to(DEV))
        ref = O.decode_indexer_scores(q8.float(), k8.float(), w, cu[:-1], torch.tensor(lens), q_scale=qs, k_scale=ks)
    else:
        q, k = q.bfloat16(), k.bfloat16()
        args = (q.to(DEV), k.to(DEV), w.to(DEV), cfg.K, cu.to(DEV), max(lens))
        ref = O.decode_indexer_scores(q, k, w, cu[:-1], torch.tensor(lens))
    idx, sc = ops.decode_indexer_topk(*args, return_scores=True)
    idx, sc = idx.cpu().long(), sc.cpu().double()
    tol = dict(rtol=2e-3, atol=2e-3) if fp8 else dict(rtol=1e-4, atol=1e-5)
    for b, L in enumerate(lens):
        torch.testing.assert_close(sc[b, :L], ref[b, :L], **tol)
    # bit-exact selection from the kernel's own fp32 scores; >= 99.9 % overlap vs float64 scores
    masked = sc.clone()
    for b, L in enumerate(lens):
        masked[b, L:] = float("-inf")
    off = cu[:-1].long()[:, None]
    want = O.topk_indices(masked, cfg.K)
    assert torch.equal(idx, torch.where(want >= 0, want + off, want))
    exact = O.topk_indices(ref, cfg.K)
    inter = tot = 0
    for b in range(len(lens)):
        a = set(idx[b][idx[b] >= 0].tolist())
        r = set((exact[b][exact[b] >= 0] + off[b]).tolist())
        inter += len(a & r)
        tot += len(r)
    assert inter / tot >= 0.999, inter / tot
    assert (idx[4, 700:] == -1).all() and (idx[4, :700] == torch.arange(700) + int(cu[4])).all()


def test_decode_fp8_rows_kernel_partial_heads_and_chunks():
    """fp8 decode rows kernel with 20 indexer heads (zero-padded A rows), rows shorter than one
    32-key block and a row spanning several wave chunks, against the float64 oracle."""
    lens = [5, 777, 4100, 31, 9000]
    print(f"[decode fp8 rows] Hi=20 lens={lens}", flush=True)
    g = torch.Generator().manual_seed(77)
    Hi, N = 20, sum(lens)
    q8, qs = O.quantize_e4m3_rows(torch.randn(len(lens), Hi, 128, generator=g))
    k8, ks = O.quantize_e4m3_rows(torch.randn(N, 128, generator=g))
    w = torch.randn(len(lens), Hi, generator=g)
    cu = _cu(lens)
    idx, sc = ops.decode_indexer_topk(q8.to(DEV), k8.to(DEV), w.to(DEV), 64, cu.to(DEV), max(lens), qs.to(DEV),
                                      ks.to(DEV), return_scores=True)
    ref = O.decode_indexer_scores(q8.float(), k8.float(), w, cu[:-1], torch.tensor(lens), q_scale=qs, k_scale=ks)
    sc = sc.cpu().double()
    for b, L in enumerate(lens):
        torch.testing.assert_close(sc[b, :L], ref[b, :L], rtol=2e-3, atol=2e-3)
    masked = sc.clone()
    for b, L in enumerate(lens):
        masked[b, L:] = float("-inf")
    off = cu[:-1].long()[:, None]
    want = O.topk_indices(masked, 64)
    assert torch.equal(idx.cpu().long(), torch.where(want >= 0, want + off, want))


@pytest.mark.parametrize("lens,H,K", [([3000, 700, 5000, 1200, 64], 128, 2048), ([4096], 128, 2048),
                                      ([900, 333, 2100], 16, 512), ([500, 600], 64, 100)])
def test_sparse_decode(lens, H, K):
    print(f"[decode attention] lens={lens} H={H} K={K}", flush=True)
    d = W.make_decode(W.CONFIGS["cfg5"], lens=lens, H=H, seed=len(lens) + H)
    q, kv = d["q"].bfloat16(), d["kv_cache"].bfloat16()
    idx = _decode_idx(lens, K, seed=K)
    out, lse = ops.sparse_mla_decode(q.to(DEV), kv.to(DEV), idx.to(DEV), W.SM_SCALE)
    o_ref, l_ref = O.sparse_mla_decode(q, kv, idx, W.SM_SCALE)
    _close(out.cpu(), o_ref, name="out")
    _close(lse.cpu(), l_ref, rel=1e-4, name="lse")


def test_sparse_decode_empty_rows():
    print("[decode attention empty rows]", flush=True)
    lens = [300, 300, 300]
    d = W.make_decode(W.CONFIGS["cfg5"], lens=lens, H=32, seed=5)
    q, kv = d["q"].bfloat16(), d["kv_cache"].bfloat16()
    idx = _decode_idx(lens, 2048, seed=1)
    idx[1] = -1                                   # nothing selected -> out 0, lse -inf
    idx[2, 5] = 10 ** 6                           # out of range -> ignored
    out, lse = ops.sparse_mla_decode(q.to(DEV), kv.to(DEV), idx.to(DEV), W.SM_SCALE)
    ref_idx = idx.clone()
    ref_idx[2, 5] = -1
    o_ref, l_ref = O.sparse_mla_decode(q, kv, ref_idx, W.SM_SCALE)
    assert (out[1] == 0).all() and torch.isinf(lse[1]).all() and (lse[1] < 0).all()
    _close(out.cpu(), o_ref, name="out")
    ok = torch.isfinite(l_ref)
    _close(lse.cpu()[ok], l_ref[ok], rel=1e-4, name="lse")


def test_sparse_fwd_bwd_no_query_rows():
    """No query rows (an empty batch): the forward returns empty out / lse, the backward an empty
    dq and dkv = 0 for every key -- written, not left as the allocator's contents (the output
    buffer is first filled with NaN through a same-size allocation freed just before)."""
    print("[sparse fwd/bwd no query rows] N=300 H=32 K=64", flush=True)
    g = torch.Generator().manual_seed(3)
    kv = (torch.randn(300, 576, generator=g) * 0.1).bfloat16().to(DEV)
    q = torch.empty(0, 32, 576, dtype=torch.bfloat16, device=DEV)
    idx = torch.empty(0, 64, dtype=torch.int32, device=DEV)
    out, lse = ops.sparse_mla_fwd(q, kv, idx, W.SM_SCALE, True)
    assert out.shape == (0, 32, 512) and lse.shape == (0, 32)
    junk = torch.full((300, 576), float("nan"), device=DEV)
    del junk
    dq, dkv = ops.sparse_mla_bwd(q, kv, idx, out, torch.empty(0, 32, 512, dtype=torch.bfloat16, device=DEV), lse,
                                 W.SM_SCALE, True)
    torch.cuda.synchronize()
    assert dq.shape == (0, 32, 576) and dkv.shape == (300, 576)
    assert torch.equal(dkv.cpu(), torch.zeros(300, 576))



def test_sparse_decode_cfg5_full_size():
    """cfg5 at full size: the split decode equals the unsplit non-causal forward kernel on the same
    inputs (a size-independent property), and the oracle on two whole sequences."""
    print("[decode attention cfg5 full size]", flush=True)
    cfg = W.CONFIGS["cfg5"]
    lens = cfg.decode_lens
    g = torch.Generator(device=DEV).manual_seed(0)
    q = (torch.randn(len(lens), cfg.H, 576, generator=g, device=DEV) * 0.1).bfloat16()
    kv = (torch.randn(sum(lens), 576, generator=g, device=DEV) * 0.1).bfloat16()
    idx = _decode_idx(lens, cfg.K, seed=3, device=DEV)
    out, lse = ops.sparse_mla_decode(q, kv, idx, W.SM_SCALE)
    ref_o, ref_l = ops.sparse_mla_fwd(q, kv, idx, W.SM_SCALE, False)
    _close(out, ref_o, rel=5e-3, name="decode vs fwd out")
    _close(lse, ref_l, rel=1e-5, name="decode vs fwd lse")
    for b in (0, 31):
        rows = idx[b][idx[b] >= 0].long()
        o_ref, l_ref = O.sparse_mla_decode(q[b:b + 1].cpu(), kv[rows].cpu(),
                                           torch.arange(rows.numel(), dtype=torch.int32)[None], W.SM_SCALE)
        _close(out[b:b + 1].cpu(), o_ref, name=f"seq {b}")
        _close(lse[b:b + 1].cpu(), l_ref, rel=1e-4, name=f"lse {b}")


def test_sparse_bwd_more_keys_than_the_lds_pair_order_holds():
    """n_kv = 20000 > 16384: the pair order runs over two LDS key tiles."""
    print("[sparse bwd] n_kv=20000", flush=True)
    g = torch.Generator().manual_seed(20000)
    T, H, K, N = 64, 16, 256, 20000
    q = (torch.randn(T, H, 576, generator=g) * 0.1).bfloat16()
    kv = (torch.randn(N, 576, generator=g) * 0.1).bfloat16()
    idx = torch.stack([torch.randperm(N, generator=g)[:K] for _ in range(T)]).to(torch.int32)
    idx[:, :8] = torch.arange(8, dtype=torch.int32)          # shared keys: several pairs per key
    idx[5, 100:] = -1
    dout = (torch.randn(T, H, 512, generator=g) * 0.01).bfloat16()
    out, lse = ops.sparse_mla_fwd(q.to(DEV), kv.to(DEV), idx.to(DEV), W.SM_SCALE, False)
    dq, dkv = ops.sparse_mla_bwd(q.to(DEV), kv.to(DEV), idx.to(DEV), out, dout.to(DEV), lse, W.SM_SCALE, False)
    rdq, rdkv = O.sparse_mla_bwd(q, kv, idx.long(), out.cpu(), dout, lse.cpu(), W.SM_SCALE)
    _close(dq.cpu(), rdq, name="dq")
    _close(dkv.cpu(), rdkv, name="dkv")


def test_decode_step_replays_in_a_hip_graph():
    """The whole decode step (decode rows, indexer scores, top-k, split attention, merge) captured
    in a HIP graph: every replay, with eager work in between and after the inputs change in
    place, equals the eager step bit for bit (no memset or host sync is recorded)."""
    print("[decode step in a HIP graph]", flush=True)
    g = torch.Generator().manual_seed(7)
    lens = [3000, 700, 5000, 1200]
    B, H, K, Hi, Di = len(lens), 128, 2048, 64, 128
    N, Lmax = sum(lens), max(lens)
    cu = torch.tensor([0] + [sum(lens[:i + 1]) for i in range(B)], dtype=torch.int32, device=DEV)
    qi = (torch.randn(B, Hi, Di, generator=g) * 0.1).bfloat16().to(DEV)
    kc = (torch.randn(N, Di, generator=g) * 0.1).bfloat16().to(DEV)
    w = (torch.randn(B, Hi, generator=g) / 8).to(DEV)
    q = (torch.randn(B, H, 576, generator=g) * 0.1).bfloat16().to(DEV)
    kv = (torch.randn(N, 576, generator=g) * 0.1).bfloat16().to(DEV)

    def step():
        idx = ops.decode_indexer_topk(qi, kc, w, K, cu, Lmax)
        out, lse = ops.sparse_mla_decode(q, kv, idx, W.SM_SCALE)
        return idx, out, lse

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        step()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        static = step()
    for rep in range(2):
        for r in range(3):
            junk = torch.randn(1 << 20, device=DEV).sum()   # eager work between replays
            graph.replay()
            torch.cuda.synchronize()
            eager = step()
            torch.cuda.synchronize()
            for a, b in zip(static, eager):
                assert torch.equal(a, b), f"replay {r} after input set {rep}"
            del junk
        q.copy_((torch.randn(B, H, 576, generator=g) * 0.1).bfloat16())
        qi.copy_((torch.randn(B, Hi, Di, generator=g) * 0.1).bfloat16())
