"""Run-to-run determinism of the backward reductions that sum per-pair partial rows per key:
the sparse attention backward's dKV (B4 pair order + B5 per-key sums) and the indexer score
backward's dk (the same pair order + K11).  Every selected (query, slot) pair gets its key-major
slot from integer counts in ascending query order, so repeated calls must agree bit for bit --
the bound on the run-to-run difference is zero.  Cases: keys shared by most queries (long key
segments cut over many query runs), and more keys than one LDS tile of the pair ordering holds.
dq/dw are per-query and carry no cross-query sum; they are compared too."""
import pytest
import torch

from mcore_bridge_amd import ops, workloads as W

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _shared_causal_idx(T, K, n_shared, seed):
    """causal top-K rows of random scores with the first n_shared keys boosted: every query
    past n_shared selects them, so their key segments hold ~T pairs each."""
    g = torch.Generator(device=DEV).manual_seed(seed)
    s = torch.rand(T, T, generator=g, device=DEV)
    s[:, :n_shared] += 2.0
    s = s.masked_fill(torch.ones(T, T, dtype=torch.bool, device=DEV).triu(1), float("-inf"))
    v, i = torch.topk(s, K, dim=1)
    return torch.where(torch.isfinite(v), i, torch.full_like(i, -1)).to(torch.int32).contiguous()


@pytest.mark.parametrize("T,N,H,K,causal", [(3000, 3000, 64, 512, True), (384, 20000, 16, 1024, False)])
def test_sparse_bwd_is_bitwise_repeatable(T, N, H, K, causal):
    print(f"[determinism sparse bwd] T={T} N={N} H={H} K={K}", flush=True)
    g = torch.Generator(device=DEV).manual_seed(T + N)
    q = (torch.randn(T, H, 576, generator=g, device=DEV) * 0.1).bfloat16()
    kv = (torch.randn(N, 576, generator=g, device=DEV) * 0.1).bfloat16()
    if causal:
        idx = _shared_causal_idx(T, K, 64, seed=1)
    else:
        idx = torch.argsort(torch.rand(T, N, generator=g, device=DEV), dim=1)[:, :K].to(torch.int32)
        idx[:, :64] = torch.arange(64, dtype=torch.int32, device=DEV) * 311   # shared keys in both tiles
        idx = idx.contiguous()
    dout = (torch.randn(T, H, 512, generator=g, device=DEV) * 0.01).bfloat16()
    out, lse = ops.sparse_mla_fwd(q, kv, idx, W.SM_SCALE, causal)
    runs = [ops.sparse_mla_bwd(q, kv, idx, out, dout, lse, W.SM_SCALE, causal) for _ in range(3)]
    for dq, dkv in runs[1:]:
        assert torch.equal(dq, runs[0][0]), "dq differs between runs"
        assert torch.equal(dkv, runs[0][1]), "dkv differs between runs"
    # the fused-target variant shares the pair order: same dkv
    _, dkv_t, _ = ops.sparse_mla_bwd_with_target(q, kv, idx, out, dout, lse, W.SM_SCALE, causal)
    assert torch.equal(dkv_t, runs[0][1])


def test_indexer_score_bwd_is_bitwise_repeatable():
    print("[determinism indexer score bwd] T=3000 Hi=64 K=512", flush=True)
    T, Hi, K = 3000, 64, 512
    g = torch.Generator(device=DEV).manual_seed(5)
    q = torch.randn(T, Hi, 128, generator=g, device=DEV).bfloat16()
    k = torch.randn(T, 128, generator=g, device=DEV).bfloat16()
    w = torch.randn(T, Hi, generator=g, device=DEV)
    idx = _shared_causal_idx(T, K, 64, seed=2)
    d = torch.randn(T, K, generator=g, device=DEV)
    runs = [ops.indexer_scores_bwd(q, k, w, idx, d, True) for _ in range(3)]
    for r in runs[1:]:
        for a, b, name in zip(r, runs[0], ("dq", "dw", "dk")):
            assert torch.equal(a, b), f"{name} differs between runs"


@pytest.mark.parametrize("T,N,H,K", [(3000, 3000, 64, 512), (1100, 20000, 16, 256)])
def test_chunked_sparse_bwd_matches_one_pass(T, N, H, K):
    """A workspace below the one-pass size runs the backward in passes of whole 256-row units
    (the causal test then takes each pass's query offset, and later passes add into dkv).  The
    index rows also hold future keys (causal: to be dropped) and keys past n_kv.  dq equals the
    one-pass dq bit for bit (no cross-query sum); dkv agrees to fp32 reordering and repeats bit
    for bit."""
    print(f"[chunked sparse bwd] T={T} N={N} H={H} K={K}", flush=True)
    g = torch.Generator(device=DEV).manual_seed(T * 7 + K)
    q = (torch.randn(T, H, 576, generator=g, device=DEV) * 0.1).bfloat16()
    kv = (torch.randn(N, 576, generator=g, device=DEV) * 0.1).bfloat16()
    idx = torch.argsort(torch.rand(T, N, generator=g, device=DEV), dim=1)[:, :K].to(torch.int32)
    idx[:, :32] = torch.arange(32, dtype=torch.int32, device=DEV)     # shared keys, all passes
    idx[::7, -1] = N + 5                                               # out of range: ignored
    idx = idx.contiguous()
    dout = (torch.randn(T, H, 512, generator=g, device=DEV) * 0.01).bfloat16()
    out, lse = ops.sparse_mla_fwd(q, kv, idx, W.SM_SCALE, True)
    dq1, dkv1 = ops.sparse_mla_bwd(q, kv, idx, out, dout, lse, W.SM_SCALE, True)
    cap = ops.bwd_workspace_bytes_chunked(T, N, H, K, 512)               # passes of 512 rows
    assert cap < ops.bwd_workspace_bytes(T, N, H, K)
    dq2, dkv2 = ops.sparse_mla_bwd(q, kv, idx, out, dout, lse, W.SM_SCALE, True, cap)
    dq3, dkv3 = ops.sparse_mla_bwd(q, kv, idx, out, dout, lse, W.SM_SCALE, True, cap)
    assert torch.equal(dq2, dq1)
    assert torch.equal(dq3, dq2) and torch.equal(dkv3, dkv2)
    torch.testing.assert_close(dkv2, dkv1, rtol=1e-5, atol=1e-7)
    err = (dkv2 - dkv1).norm() / dkv1.norm()
    assert err < 1e-6, float(err)
