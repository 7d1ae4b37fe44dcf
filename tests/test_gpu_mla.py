"""The absorbed DSA MLA swapped into a layer spec (mcore_bridge_amd.mla), on the GPU, against the
reference MLA's un-absorbed forward (multi_latent_attention.py:43-178, 262-290) in float64 built
from the same module's weights: output and the gradients of the input and of every weight, sbhd
with batch 2, THD packing against per-document calls, and the training path with the sparse and
the dense indexer loss.  The Megatron modules are stand-ins (tests/megatron_standin.py) with the reference's names."""
import types

import pytest
import torch

import megatron_standin as M
from oracle import dsa_oracle as O
from mcore_bridge_amd import dsa, mla

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _close(got, ref, rel=1e-2, name="", tol=2e-2):
    got, ref = got.double().cpu(), ref.double().cpu()
    torch.testing.assert_close(got, ref, rtol=tol, atol=tol, msg=lambda m: f"{name}: {m}")
    err = (got - ref).norm() / ref.norm().clamp_min(1e-30)
    assert err < rel, f"{name}: normalised error {err:.3e} >= {rel}"


def _build(H=16, hidden=256, qlr=192, Hi=64, K=48, coeff=0.0, seed=0):
    g = torch.Generator().manual_seed(seed)
    cfg = M.make_config(H, qlr, coeff=coeff, mscale=1.05)
    indexer = dsa.DSAIndexer(hidden, qlr, index_n_heads=Hi, index_topk=K, attention_scaling=1.05, device=DEV)
    core = M.CoreAttention(indexer, softmax_scale=(cfg.qk_head_dim + cfg.qk_pos_emb_head_dim) ** -0.5)
    spec = M.spec_with(M.MLASelfAttention)
    assert mla.install_attention(spec) == 2
    mod = spec.layer_specs[0].submodules.self_attention.module(cfg, hidden, core, device=DEV)
    assert isinstance(mod, M.MLASelfAttention)
    with torch.no_grad():
        for n, p in mod.named_parameters():
            if p.dim() == 2:
                p.copy_((torch.randn(p.shape, generator=g) / p.shape[1] ** 0.5).to(p.dtype))
            else:
                p.copy_((1 + 0.1 * torch.randn(p.shape, generator=g)).to(p.dtype))
        indexer.k_norm.bias.copy_((0.1 * torch.randn(128, generator=g)).to(indexer.k_norm.bias.dtype))
    return mod, indexer, g


def _topk_used(mod, indexer, x, rope, psp=None):
    with torch.no_grad():
        q_c = mod.q_layernorm(mod.linear_q_down_proj(x)[0])
        docs = dsa._thd_docs(psp)
        if docs is not None:
            q_c = q_c.squeeze(1)
        out = indexer.forward_before_topk(x, q_c, (psp, rope))
        return indexer.topk_from_outputs(out, None, docs, causal=True, return_scores=False)[1]


def test_absorbed_mla_swap_matches_unabsorbed_reference():
    print("[absorbed MLA swap] sbhd S=96 B=2 H=16", flush=True)
    mod, indexer, g = _build()
    S, B, hidden = 96, 2, 256
    x = torch.randn(S, B, hidden, generator=g).bfloat16().to(DEV).requires_grad_()
    rope = (torch.rand(S, 1, 1, 64, generator=g) * 100).to(DEV)
    out, bias = mod(x, None, rotary_pos_emb=rope)
    assert bias is None and out.shape == (S, B, hidden)
    topk = _topk_used(mod, indexer, x.detach(), rope)
    ref, xd, params = M.reference_forward(mod, x.detach().cpu(), rope.cpu(), topk.cpu(), O)
    _close(out.detach(), ref.detach(), name="out")
    dout = torch.randn(S, B, hidden, generator=g) * 0.1
    out.backward(dout.bfloat16().to(DEV))
    ref.backward(dout.double())
    _close(x.grad, xd.grad, name="d hidden_states")
    for n, p in params.items():
        _close(getattr(mod, n).weight.grad, p.grad, name=f"d {n}")


def test_absorbed_mla_swap_thd_equals_per_document():
    print("[absorbed MLA swap] THD packed vs per document", flush=True)
    mod, indexer, g = _build(seed=1)
    lens = [40, 90, 33]
    cu = [0] + [sum(lens[:i + 1]) for i in range(len(lens))]
    T, hidden = cu[-1], 256
    x = torch.randn(T, 1, hidden, generator=g).bfloat16().to(DEV)
    rope = (torch.rand(max(lens), 1, 1, 64, generator=g) * 100).to(DEV)
    psp = types.SimpleNamespace(qkv_format="thd", cu_seqlens_q=torch.tensor(cu, dtype=torch.int32, device=DEV),
                                cu_seqlens_kv=torch.tensor(cu, dtype=torch.int32, device=DEV), max_seqlen_q=max(lens))
    with torch.no_grad():
        out_p, _ = mod(x, None, rotary_pos_emb=rope, packed_seq_params=psp)
        assert out_p.shape == (T, 1, hidden)
        for a, b in zip(cu[:-1], cu[1:]):
            out_d, _ = mod(x[a:b], None, rotary_pos_emb=rope[:b - a])
            _close(out_p[a:b], out_d, name=f"document {a}:{b}")


def test_absorbed_mla_swap_trains_the_indexer_with_the_sparse_loss():
    print("[absorbed MLA swap] training with the sparse indexer loss", flush=True)
    mod, indexer, g = _build(coeff=0.3, seed=2)
    S, B, hidden = 80, 2, 256
    x = torch.randn(S, B, hidden, generator=g).bfloat16().to(DEV)
    rope = (torch.rand(S, 1, 1, 64, generator=g) * 100).to(DEV)
    mod.eval()
    with torch.no_grad():
        out_e, _ = mod(x, None, rotary_pos_emb=rope)
    mod.train()
    out_t, _ = mod(x, None, rotary_pos_emb=rope)
    _close(out_t.detach(), out_e, rel=1e-3, name="training forward = eval forward")
    (out_t.float() * 0.01).sum().backward()
    loss = mod.last_indexer_loss
    assert loss is not None and bool(torch.isfinite(loss)) and float(loss) > 0
    for n, p in indexer.named_parameters():
        assert p.grad is not None and bool(torch.isfinite(p.grad).all()) and float(p.grad.abs().sum()) > 0, n
    # the dense loss (the reference default): same forward, the loss over every visible key
    mod.config.dsa_indexer_use_sparse_loss = False
    indexer.zero_grad(set_to_none=True)
    out_d, _ = mod(x, None, rotary_pos_emb=rope)
    _close(out_d.detach(), out_e, rel=1e-3, name="dense-loss training forward = eval forward")
    (out_d.float() * 0.01).sum().backward()
    loss_d = mod.last_indexer_loss
    assert bool(torch.isfinite(loss_d)) and float(loss_d) > 0
    for n, p in indexer.named_parameters():
        assert p.grad is not None and bool(torch.isfinite(p.grad).all()) and float(p.grad.abs().sum()) > 0, n


@pytest.mark.parametrize("flag", ["checkpoint_core_attention", "recompute_up_proj"])
@pytest.mark.parametrize("sparse", [True, False])
def test_absorbed_mla_recompute_flags_give_the_same_training_step(flag, sparse):
    """The reference's recompute flags (multi_latent_attention.py:180-185, 250-252) checkpoint the
    absorbed attention (and the q up-projection): the kernels run again in the backward and give the
    same output, indexer loss and gradients as without the flag, bit for bit (the kernels are
    deterministic)."""
    print(f"[absorbed MLA swap] {flag}, sparse loss {sparse}", flush=True)
    res = []
    for on in (False, True):
        mod, indexer, g = _build(coeff=0.3, seed=4)
        mod.config.dsa_indexer_use_sparse_loss = sparse
        if on:
            setattr(mod, flag, True)
        S, B, hidden = 64, 2, 256
        x = torch.randn(S, B, hidden, generator=g).bfloat16().to(DEV).requires_grad_()
        rope = (torch.rand(S, 1, 1, 64, generator=g) * 100).to(DEV)
        mod.train()
        out, _ = mod(x, None, rotary_pos_emb=rope)
        (out.float() * 0.01).sum().backward()
        torch.cuda.synchronize()
        grads = {n: p.grad.clone() for n, p in list(mod.named_parameters()) + list(indexer.named_parameters(prefix="ix"))
                 if p.grad is not None}
        res.append((out.detach(), x.grad.clone(), grads, mod.last_indexer_loss.clone()))
    (o0, dx0, g0, l0), (o1, dx1, g1, l1) = res
    assert torch.equal(o0, o1) and torch.equal(dx0, dx1) and torch.equal(l0, l1)
    assert float(l1) > 0
    assert g0.keys() == g1.keys()
    for n in g0:
        assert torch.equal(g0[n], g1[n]), n
