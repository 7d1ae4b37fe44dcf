"""The sparse backward with int8 G-row staging (DSA_BWD_G_INT8): per-pair dKV partial rows held as
int8 with a bf16 scale per 32 dims instead of bf16.  dq never reads those rows, so it must equal
the bf16-staged dq bit for bit; dkv must meet the same bars as every gradient (rtol 2e-2 / atol
2e-2 of the float64 oracle and normalised error < 1e-2), repeat bit for bit, and agree between one
pass and passes of query rows."""
import pytest
import torch

from oracle import dsa_oracle as O
from mcore_bridge_amd import ops, workloads as W

pytestmark = pytest.mark.gpu
DEV = "cuda"
RTOL = ATOL = 2e-2


def _close(got, ref, rel=1e-2, name=""):
    got = got.double().cpu()
    ref = ref.double().cpu()
    torch.testing.assert_close(got, ref, rtol=RTOL, atol=ATOL, msg=lambda m: f"{name}: {m}")
    err = (got - ref).norm() / ref.norm().clamp_min(1e-30)
    assert err < rel, f"{name}: normalised error {err:.3e} >= {rel}"
    return float(err)


def _case(T, H, K, seed):
    """causal rows of K random visible keys (ascending; every 5th row shorter, -1 padded)."""
    g = torch.Generator().manual_seed(seed)
    q = (torch.randn(T, H, 576, generator=g) * 0.1).bfloat16()
    kv = (torch.randn(T, 576, generator=g) * 0.1).bfloat16()
    idx = torch.full((T, K), -1, dtype=torch.int32)
    for t in range(T):
        cand = torch.randperm(t + 1, generator=g)[:K]
        m = cand.numel() if t % 5 else max(1, cand.numel() - cand.numel() // 10)
        idx[t, :m] = torch.sort(cand[:m]).values.to(torch.int32)
    dout = (torch.randn(T, H, 512, generator=g) * 0.01).bfloat16()
    return q, kv, idx, dout


@pytest.mark.parametrize("T,H,K", [(300, 64, 256), (160, 128, 128), (120, 16, 64), (77, 48, 96), (90, 128, 16)])
def test_int8_staging_against_fp64_oracle(T, H, K):
    """H = 48 runs B3's 4-step head loop with a zero last step; T = 77 ends in a partial block;
    K = 16 gives every query a single key block, stored only after B3's block loop."""
    print(f"[int8 staging vs oracle] T={T} H={H} K={K}", flush=True)
    q, kv, idx, dout = _case(T, H, K, 900 + T)
    qd, kvd, idxd, doutd = q.to(DEV), kv.to(DEV), idx.to(DEV), dout.to(DEV)
    out, lse = ops.sparse_mla_fwd(qd, kvd, idxd, W.SM_SCALE, True)
    dq16, dkv16 = ops.sparse_mla_bwd(qd, kvd, idxd, out, doutd, lse, W.SM_SCALE, True)
    dq8, dkv8 = ops.sparse_mla_bwd(qd, kvd, idxd, out, doutd, lse, W.SM_SCALE, True, 0, True)
    assert torch.equal(dq8, dq16), "dq depends on the G-row format"
    assert not torch.equal(dkv8, dkv16), "int8 staging did not run"
    dq_ref, dkv_ref = O.sparse_mla_bwd(q, kv, idx, out.cpu(), dout, lse.cpu(), W.SM_SCALE)
    _close(dq8.cpu(), dq_ref, name="dq")
    e16 = _close(dkv16.cpu(), dkv_ref, name="dkv (bf16 rows)")
    e8 = _close(dkv8.cpu(), dkv_ref, name="dkv (int8 rows)")
    print(f"  dkv normalised error: bf16 rows {e16:.2e}, int8 rows {e8:.2e}", flush=True)


def test_int8_staging_cfg3_full_size():
    """cfg3 at the bench's size: dkv against the oracle's per-key closed form on sampled keys
    (every query that selected them), the whole dkv against the bf16-staged one, dq unchanged, and
    bit-for-bit repeats."""
    print("[int8 staging cfg3 full size]", flush=True)
    cfg = W.CONFIGS["cfg3"]
    x = W.make_prefill(cfg, device=DEV, seed=3)
    T = cfg.S
    idx = ops.indexer_topk(x["q_idx"].bfloat16(), x["k_idx"].bfloat16(), x["w"], cfg.K, x["cu_seqlens"],
                           causal=True)
    q, kv, dout = x["q"].bfloat16(), x["kv"].bfloat16(), x["dout"].bfloat16()
    del x
    out, lse = ops.sparse_mla_fwd(q, kv, idx, W.SM_SCALE, True)
    dq16, dkv16 = ops.sparse_mla_bwd(q, kv, idx, out, dout, lse, W.SM_SCALE, True)
    dq8, dkv8 = ops.sparse_mla_bwd(q, kv, idx, out, dout, lse, W.SM_SCALE, True, 0, True)
    dq8b, dkv8b = ops.sparse_mla_bwd(q, kv, idx, out, dout, lse, W.SM_SCALE, True, 0, True)
    torch.cuda.synchronize()
    assert torch.equal(dq8, dq16)
    assert torch.equal(dq8b, dq8) and torch.equal(dkv8b, dkv8), "int8-staged backward not repeatable"
    err = float((dkv8 - dkv16).norm() / dkv16.norm())
    print(f"  dkv int8 vs bf16 rows: normalised difference {err:.2e}", flush=True)
    torch.testing.assert_close(dkv8, dkv16, rtol=RTOL, atol=ATOL)
    assert err < 1e-2
    starts = cfg.docs[:-1]
    keys = [0, 1000, starts[1], T - 1]
    rdkv = O.sparse_mla_bwd_dkv_rows(q.cpu(), kv.cpu(), idx.cpu(), out.cpu(), dout.cpu(), lse.cpu(), W.SM_SCALE,
                                     keys)
    _close(dkv8[keys].cpu(), rdkv, name="dkv sampled keys (int8 rows)")


def test_int8_staging_chunked_matches_one_pass():
    """Passes of 512 query rows with int8 rows: dq bit for bit, dkv to fp32 reordering."""
    T, N, H, K = 3000, 3000, 64, 512
    print(f"[int8 staging chunked] T={T} N={N} H={H} K={K}", flush=True)
    g = torch.Generator(device=DEV).manual_seed(41)
    q = (torch.randn(T, H, 576, generator=g, device=DEV) * 0.1).bfloat16()
    kv = (torch.randn(N, 576, generator=g, device=DEV) * 0.1).bfloat16()
    idx = torch.argsort(torch.rand(T, N, generator=g, device=DEV), dim=1)[:, :K].to(torch.int32)
    idx[:, :32] = torch.arange(32, dtype=torch.int32, device=DEV)     # shared keys, all passes
    idx = idx.contiguous()
    dout = (torch.randn(T, H, 512, generator=g, device=DEV) * 0.01).bfloat16()
    out, lse = ops.sparse_mla_fwd(q, kv, idx, W.SM_SCALE, True)
    dq1, dkv1 = ops.sparse_mla_bwd(q, kv, idx, out, dout, lse, W.SM_SCALE, True, 0, True)
    cap = ops.bwd_workspace_bytes_chunked(T, N, H, K, 512, True)
    assert cap < ops.bwd_workspace_bytes(T, N, H, K, True) < ops.bwd_workspace_bytes(T, N, H, K)
    dq2, dkv2 = ops.sparse_mla_bwd(q, kv, idx, out, dout, lse, W.SM_SCALE, True, cap, True)
    assert torch.equal(dq2, dq1)
    torch.testing.assert_close(dkv2, dkv1, rtol=1e-5, atol=1e-7)
    assert float((dkv2 - dkv1).norm() / dkv1.norm()) < 1e-6


def test_int8_staging_through_autograd():
    """ops.set_backward_staging('int8') routes the autograd backward through the int8 rows."""
    T, H, K = 200, 32, 96
    print(f"[int8 staging autograd] T={T} H={H} K={K}", flush=True)
    q, kv, idx, dout = _case(T, H, K, 17)
    qd, kvd, idxd, doutd = q.to(DEV), kv.to(DEV), idx.to(DEV), dout.to(DEV)
    out, lse = ops.sparse_mla_fwd(qd, kvd, idxd, W.SM_SCALE, True)
    dq8, dkv8 = ops.sparse_mla_bwd(qd, kvd, idxd, out, doutd, lse, W.SM_SCALE, True, 0, True)
    ops.set_backward_staging("int8")
    try:
        qg, kvg = qd.clone().requires_grad_(), kvd.float().requires_grad_()
        ops.sparse_mla(qg, kvg.bfloat16(), idxd, W.SM_SCALE, True).backward(doutd)
    finally:
        ops.set_backward_staging("bf16")
    assert torch.equal(qg.grad, dq8)
    assert torch.equal(kvg.grad, dkv8.to(torch.bfloat16).float())
    with pytest.raises(ValueError):
        ops.set_backward_staging("fp8")


def test_int8_staging_in_the_v4_sink_attention_backward():
    """The DeepSeek-V4 sink attention's backward runs the same kernels through
    ops.autograd_backward, so the staging setting reaches it: dq identical to bf16 staging, dkv
    within the gradient bars of it."""
    from mcore_bridge_amd import v4
    T, H, K = 256, 32, 64
    print(f"[int8 staging v4 sink attention] T={T} H={H} K={K}", flush=True)
    g = torch.Generator().manual_seed(23)
    q = (torch.randn(T, H, 512, generator=g) * 0.1).bfloat16().to(DEV)
    kv = (torch.randn(T, 512, generator=g) * 0.1).bfloat16().to(DEV)
    sinks = (torch.randn(H, generator=g) * 0.5).to(DEV)
    idx = torch.full((T, K), -1, dtype=torch.int32)
    for t in range(T):
        sel = torch.randperm(t + 1, generator=g)[:K]
        idx[t, :sel.numel()] = torch.sort(sel).values.to(torch.int32)
    idx = idx.to(DEV)
    dout = (torch.randn(T, H, 512, generator=g) * 0.01).bfloat16().to(DEV)
    grads = {}
    for fmt in ("bf16", "int8"):
        ops.set_backward_staging(fmt)
        try:
            qg, kg = q.clone().requires_grad_(), kv.clone().requires_grad_()
            out, _ = v4.sink_attention(qg, kg, sinks, idx, 512 ** -0.5)
            out.backward(dout)
        finally:
            ops.set_backward_staging("bf16")
        grads[fmt] = (qg.grad, kg.grad)
    assert torch.equal(grads["int8"][0], grads["bf16"][0])
    assert not torch.equal(grads["int8"][1], grads["bf16"][1]), "int8 staging did not reach the V4 backward"
    _close(grads["int8"][1], grads["bf16"][1], name="dkv (int8 vs bf16 rows)")
