"""GPU parity of the DeepSeek-V4 hybrid attention (mcore_bridge_amd.v4) against the float64 oracle
(oracle/dsv4_oracle.py, itself pinned against transformers' DeepseekV4Attention):
- the sink attention core over sliding-window + compressed index rows (HCA: every visible entry,
  CSA: a selection), two packed documents: out, lse and the gradients of q, K = V rows and sinks;
- the layer mirror DSv4HybridAttention for the three layer types against the oracle's layer with
  the same weights (CSA with the kernels' own indexer selection, which is checked against the
  oracle's selection separately), and THD packing against per-document calls.
Bar: rtol = atol = 2e-2 plus normalised error < 1e-2 (sinks and selections: see each check)."""
import types

import pytest
import torch

from oracle import dsv4_oracle as V
from mcore_bridge_amd import v4

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _close(got, ref, rel=1e-2, name="", tol=2e-2):
    got, ref = got.double().cpu(), ref.double().cpu()
    torch.testing.assert_close(got, ref, rtol=tol, atol=tol, msg=lambda m: f"{name}: {m}")
    err = (got - ref).norm() / ref.norm().clamp_min(1e-30)
    assert err < rel, f"{name}: normalised error {err:.3e} >= {rel}"


@pytest.mark.parametrize("mode", ["hca", "csa", "window"])
def test_sink_attention_core_matches_oracle_fwd_bwd(mode):
    print(f"[v4 sink attention] {mode}", flush=True)
    g = torch.Generator().manual_seed({"hca": 1, "csa": 2, "window": 3}[mode])
    cu = [0, 70, 150]
    T, H, D, W, rate = cu[-1], 16, 512, 16, 4
    q = (torch.randn(T, H, D, generator=g) * 0.05).bfloat16()
    kv = (torch.randn(T, D, generator=g)).bfloat16()
    n_comp = [(b - a) // rate for a, b in zip(cu[:-1], cu[1:])]
    comp = (torch.randn(sum(n_comp), D, generator=g)).bfloat16()
    sinks = torch.randn(H, generator=g)
    scale = D ** -0.5
    sel_local = None
    if mode == "csa":
        K = 6
        sel_local = torch.full((T, K), -1, dtype=torch.int64)
        sel_glob = sel_local.clone()
        off = 0
        for d, (a, b) in enumerate(zip(cu[:-1], cu[1:])):
            for t in range(a, b):
                v = V.compressed_visible(t - a, rate)
                if v:
                    s = torch.randperm(v, generator=g)[:K].sort().values
                    sel_local[t, : s.numel()] = s
                    sel_glob[t, : s.numel()] = s + off
            off += n_comp[d]
        idx = v4.hybrid_indices(cu, W, 0, sel_glob.to(DEV), DEV)
    elif mode == "hca":
        idx = v4.hybrid_indices(cu, W, rate, None, DEV)
    else:
        idx = v4.hybrid_indices(cu, W, 0, None, DEV)
    keys = torch.cat([kv, comp]) if mode != "window" else kv
    qd, kd, sd = q.to(DEV).requires_grad_(), keys.to(DEV).requires_grad_(), sinks.to(DEV).requires_grad_()
    out, lse = v4.sink_attention(qd, kd, sd, idx, scale)
    dout = torch.randn(T, H, D, generator=g) * 0.1
    out.backward(dout.bfloat16().to(DEV))
    # float64 oracle with autograd
    qr, kr, sr = q.double().requires_grad_(), keys.double().requires_grad_(), sinks.double().requires_grad_()
    comp_r = kr[T:] if mode != "window" else None
    ro, rl = V.core_attention(qr, kr[:T], comp_r, sel_local, sr, W, scale, rate if mode != "window" else 1,
                              torch.tensor(cu))
    ro.backward(dout.double())
    _close(out.detach(), ro.detach(), name="out")
    torch.testing.assert_close(lse.cpu().double(), rl.detach(), rtol=1e-4, atol=1e-4)
    _close(qd.grad, qr.grad, name="dq")
    _close(kd.grad, kr.grad, name="dkv")
    _close(sd.grad, sr.grad, rel=2e-2, name="dsinks")


def _layer(layer_type, seed):
    g = torch.Generator().manual_seed(seed)
    hidden, H, qlr = 256, 16, 128
    m = v4.DSv4HybridAttention(layer_type, hidden, H, qlr, o_groups=4, o_lora_rank=64, window=32,
                               compress_rates=(4, 16), index_n_heads=16, index_head_dim=128, index_topk=12,
                               device=DEV)
    with torch.no_grad():
        for n, p in m.named_parameters():
            if n.endswith("ape"):
                p.copy_(torch.randn(p.shape, generator=g) * 0.5)
            elif n.endswith("attn_sink"):
                p.copy_(torch.randn(p.shape, generator=g))
            elif p.dim() == 1:
                p.copy_((1 + 0.1 * torch.randn(p.shape, generator=g)).to(p.dtype))
            else:
                p.copy_((torch.randn(p.shape, generator=g) / p.shape[1] ** 0.5).to(p.dtype))
    return m, g


def _oracle_params(m):
    ca = m.core_attention
    p = {"wq_a": m.linear_q_down_proj.weight, "q_norm": m.q_layernorm.weight, "wq_b": m.linear_q_up_proj.weight,
         "wkv": m.linear_kv_proj.weight, "kv_norm": m.kv_layernorm.weight, "wo_a": m.linear_o_group_proj,
         "wo_b": m.linear_proj.weight, "sinks": ca.attn_sink}
    if ca.compressor is not None:
        c = ca.compressor
        p.update(comp_wkv=c.linear_wkv.weight, comp_wgate=c.linear_wgate.weight, comp_ape=c.ape, comp_norm=c.norm.weight)
    if ca.indexer is not None:
        ix = ca.indexer
        p.update(idx_wq_b=ix.linear_wq_b.weight, idx_weights_proj=ix.linear_weights_proj.weight,
                 idx_comp_wkv=ix.compressor.linear_wkv.weight, idx_comp_wgate=ix.compressor.linear_wgate.weight,
                 idx_comp_ape=ix.compressor.ape, idx_comp_norm=ix.compressor.norm.weight)
    return {k: v.detach().double().cpu() for k, v in p.items()}


def _rope_tables(S, dev):
    inv_main = 1.0 / (10000 ** (torch.arange(0, 64, 2, dtype=torch.float32) / 64))
    inv_comp = 1.0 / (160000 ** (torch.arange(0, 64, 2, dtype=torch.float32) / 64))
    pos = torch.arange(S, dtype=torch.float32)[:, None]
    tab = lambda inv: torch.cat([pos * inv, pos * inv], -1)[:, None, None, :].to(dev)   # Megatron [S, 1, 1, 64]
    return {"main": tab(inv_main), "compress": tab(inv_comp)}, {"main": inv_main, "compress": inv_comp}


@pytest.mark.parametrize("layer_type", ["sliding_attention", "compressed_sparse_attention",
                                        "heavily_compressed_attention"])
def test_v4_layer_mirror_matches_oracle(layer_type):
    print(f"[v4 layer] {layer_type}", flush=True)
    m, g = _layer(layer_type, {"sliding_attention": 5, "compressed_sparse_attention": 6,
                               "heavily_compressed_attention": 7}[layer_type])
    S, hidden = 160, 256
    x = torch.randn(S, 1, hidden, generator=g).bfloat16().to(DEV)
    rope, inv = _rope_tables(S, DEV)
    with torch.no_grad():
        out, _ = m(x, None, rotary_pos_emb=rope)
    cfg = {"heads": 16, "head_dim": 512, "window": 32, "eps": 1e-6, "o_groups": 4, "index_heads": 16,
           "index_head_dim": 128, "index_topk": 12, "rates": {"csa": 4, "hca": 16},
           "inv_freq": {k: v.double() for k, v in inv.items()}, "mscale": {"main": 1.0, "compress": 1.0}}
    sel = None
    if layer_type == "compressed_sparse_attention":
        sel = m.last_indexer_selection.long().cpu()
        # the kernels' selection against the oracle's float64 selection (same weights, same inputs):
        # near-tied index scores may swap, so >= 97 % overlap; the layer check below uses the
        # kernels' own selection
        pr = _oracle_params(m)
        xd = x[:, 0].double().cpu()
        q_res = V.rms_norm(xd @ pr["wq_a"].T, pr["q_norm"], 1e-6)
        ck = V.compress_windows(xd @ pr["idx_comp_wkv"].T, xd @ pr["idx_comp_wgate"].T, pr["idx_comp_ape"],
                                pr["idx_comp_norm"], 4, 1e-6, True)
        ck = V.rope_interleaved(ck[None], torch.arange(ck.shape[0]) * 4, cfg["inv_freq"]["compress"])[0]
        qi = (q_res @ pr["idx_wq_b"].T).view(S, 16, 128)
        qi = V.rope_interleaved(qi.transpose(0, 1), torch.arange(S), cfg["inv_freq"]["compress"]).transpose(0, 1)
        wi = (xd @ pr["idx_weights_proj"].T) * 16 ** -0.5
        ref_sel = V.indexer_topk(qi, ck, wi, 4, 12, 128 ** -0.5)
        inter = sum(len(set(a[a >= 0].tolist()) & set(b[b >= 0].tolist())) for a, b in zip(sel, ref_sel))
        tot = int((ref_sel >= 0).sum())
        assert inter / tot >= 0.97, inter / tot
        assert torch.equal((sel >= 0).sum(1), (ref_sel >= 0).sum(1))          # same visible counts
    ref = V.attention_layer(x[:, 0].cpu(), _oracle_params(m), cfg, layer_type, comp_sel=sel)
    _close(out[:, 0], ref, name=f"{layer_type} output")


def test_v4_layer_mirror_thd_equals_per_document():
    print("[v4 layer] THD packed vs per document", flush=True)
    m, g = _layer("compressed_sparse_attention", 8)
    lens = [70, 96, 41]
    cu = [0] + [sum(lens[:i + 1]) for i in range(len(lens))]
    T, hidden = cu[-1], 256
    x = torch.randn(T, 1, hidden, generator=g).bfloat16().to(DEV)
    rope, _ = _rope_tables(max(lens), DEV)
    psp = types.SimpleNamespace(qkv_format="thd", cu_seqlens_q=torch.tensor(cu, dtype=torch.int32, device=DEV))
    with torch.no_grad():
        out_p, _ = m(x, None, rotary_pos_emb=rope, packed_seq_params=psp)
        assert out_p.shape == (T, 1, hidden)
        for a, b in zip(cu[:-1], cu[1:]):
            out_d, _ = m(x[a:b], None, rotary_pos_emb=rope)
            _close(out_p[a:b], out_d, name=f"document {a}:{b}")
