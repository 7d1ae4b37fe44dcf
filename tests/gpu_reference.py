"""Plain PyTorch fp32 references of the floating-point kernels, run on the GPU (test helper).

They check the kernels over EVERY row of a full-size problem, where the float64 CPU oracle can
only afford sampled rows; the oracle in turn pins them on those sampled rows inside the tests.
Every batched product gets contiguous fp32 operands (no transposed bf16 views reach bmm).
"""
import torch


def sparse_mla_fwd_fp32(q: torch.Tensor, kv: torch.Tensor, idx: torch.Tensor, sm_scale: float, causal: bool,
                        chunk: int = 128, d_v: int = 512):
    """``(out [T, H, d_v], lse [T, H])`` fp32 of sparse MQA over the latent rows ``kv[idx[t, j]]``
    (``-1`` = none; with ``causal`` keys after the query's own position ``t`` are ignored, as the
    kernels' ``causal`` flag does for global ids).  Rows without a key give out 0, lse -inf."""
    T, H, D = q.shape
    out = torch.empty(T, H, d_v, dtype=torch.float32, device=q.device)
    lse = torch.empty(T, H, dtype=torch.float32, device=q.device)
    for a in range(0, T, chunk):
        b = min(T, a + chunk)
        ii = idx[a:b].long()
        valid = ii >= 0
        if causal:
            valid &= ii <= torch.arange(a, b, device=q.device)[:, None]
        g = kv[ii.clamp(min=0)].float()                                   # [c, K, D]
        qq = q[a:b].float().contiguous()                                  # [c, H, D]
        s = torch.bmm(qq, g.transpose(1, 2).contiguous()) * sm_scale       # [c, H, K]
        s = s.masked_fill(~valid[:, None, :], float("-inf"))
        m = s.amax(-1, keepdim=True)
        m = torch.where(torch.isfinite(m), m, torch.zeros_like(m))
        p = torch.exp(s - m)
        l = p.sum(-1, keepdim=True)
        o = torch.bmm(p, g[..., :d_v].contiguous())
        nz = l > 0
        out[a:b] = torch.where(nz, o / torch.where(nz, l, torch.ones_like(l)), torch.zeros_like(o))
        lse[a:b] = torch.where(nz[..., 0], (m + torch.log(l))[..., 0], torch.full_like(l[..., 0], float("-inf")))
    return out, lse


def close_on_device(got: torch.Tensor, ref: torch.Tensor, name: str = "", tol: float = 2e-2, rel: float = 1e-2):
    """The parity bar (rtol = atol = ``tol`` elementwise, normalised error < ``rel``) evaluated on the
    tensors' own device in fp32 (full-size outputs are too large to copy to the host as float64)."""
    g, r = got.float(), ref.float()
    torch.testing.assert_close(g, r, rtol=tol, atol=tol, msg=lambda m: f"{name}: {m}")
    err = ((g - r).norm() / r.norm().clamp_min(1e-30)).item()
    assert err < rel, f"{name}: normalised error {err:.3e} >= {rel}"


def sparse_mla_bwd_fp32(q: torch.Tensor, kv: torch.Tensor, idx: torch.Tensor, out: torch.Tensor,
                        dout: torch.Tensor, lse: torch.Tensor, sm_scale: float, causal: bool,
                        chunk: int = 64, d_v: int = 512):
    """``(dq [T, H, D], dkv [N, D])`` fp32 of ``sparse_mla_fwd_fp32`` by its closed form, over
    every query and key: ``P = exp(sm_scale*S - lse)``, ``Delta = rowsum(dO*O)``,
    ``dS = P*(dO.V^T - Delta)``, ``dq = sm_scale*dS.K``, and per selected slot the dKV row
    ``sm_scale*dS^T.q + P^T.dO`` (first ``d_v`` columns), summed into its key with ``index_add_``.
    ``out`` and ``lse`` are the forward's (the kernels' backward takes them as inputs too)."""
    T, H, D = q.shape
    N = kv.shape[0]
    dq = torch.empty(T, H, D, dtype=torch.float32, device=q.device)
    dkv = torch.zeros(N, D, dtype=torch.float32, device=q.device)
    for a in range(0, T, chunk):
        b = min(T, a + chunk)
        ii = idx[a:b].long()
        valid = (ii >= 0) & (ii < N)
        if causal:
            valid &= ii <= torch.arange(a, b, device=q.device)[:, None]
        ic = torch.where(valid, ii, torch.zeros_like(ii))
        g = kv[ic].float()                                                 # [c, K, D]
        qq = q[a:b].float().contiguous()                                   # [c, H, D]
        do = dout[a:b].float().contiguous()                                # [c, H, d_v]
        l = lse[a:b].float()[..., None]                                    # [c, H, 1]
        s = torch.bmm(qq, g.transpose(1, 2).contiguous()) * sm_scale        # [c, H, K]
        live = valid[:, None, :] & torch.isfinite(l)
        p = torch.where(live, torch.exp(s - torch.where(torch.isfinite(l), l, torch.zeros_like(l))),
                        torch.zeros_like(s))
        dp = torch.bmm(do, g[..., :d_v].transpose(1, 2).contiguous())       # [c, H, K]
        delta = (do * out[a:b].float()).sum(-1, keepdim=True)              # [c, H, 1]
        ds = p * (dp - delta)
        dq[a:b] = torch.bmm(ds, g) * sm_scale
        contrib = torch.bmm(ds.transpose(1, 2).contiguous(), qq) * sm_scale  # [c, K, D]
        contrib[..., :d_v] += torch.bmm(p.transpose(1, 2).contiguous(), do)
        contrib *= valid[..., None]
        dkv.index_add_(0, ic.reshape(-1), contrib.reshape(-1, D))
    return dq, dkv
