"""CPU checks of the absorbed MLA's handling of the reference's recompute flags
(``checkpoint_core_attention``, multi_latent_attention.py:250-252; ``recompute_up_proj``, :180-185 and
:282-285) with the Megatron stand-ins of tests/megatron_standin.py.  The kernels need a GPU, so the
absorbed attention and the indexer are replaced by small differentiable torch stand-ins here: what
is checked is the plumbing -- the checkpointed region runs again in the backward, and the outputs,
the indexer loss and every gradient equal those of the run without the flag."""
import copy

import pytest
import torch

import megatron_standin as M
from mcore_bridge_amd import dsa, mla


class _FakeIndexer(dsa._IndexerComputation, torch.nn.Module):
    """Indexer stand-in: a differentiable (q, k, w) from (x, qr), a fixed causal selection."""

    fp8 = False

    def __init__(self, hidden, qlr, K):
        torch.nn.Module.__init__(self)
        self.lq = torch.nn.Linear(qlr, 2 * 8, bias=False)
        self.lk = torch.nn.Linear(hidden, 8, bias=False)
        self.lw = torch.nn.Linear(hidden, 2, bias=False)
        self.K = K

    def forward_before_topk(self, x, qr, packed_seq_params=None):
        S, B = x.shape[:2]
        return self.lq(qr).view(S, B, 2, 8), self.lk(x), self.lw(x)

    def topk_from_outputs(self, out, mask=None, docs=None, causal=None, return_scores=True):
        q = out[0]
        S, B = q.shape[:2]
        t = torch.arange(S)[:, None] - torch.arange(self.K)[None]
        return None, torch.where(t >= 0, t, torch.full_like(t, -1)).expand(B, S, self.K)


def _fake_attention(calls):
    def attn(q_nope, q_pe, kv_c, k_pe, w_kv, topk, scale, causal, indexer_loss=None):
        calls.append(1)
        S, B, H, dn = q_nope.shape
        W = w_kv.view(H, -1, kv_c.shape[-1])
        q_lat = torch.einsum("sbhd,hdc->sbhc", q_nope, W[:, :dn])
        v = torch.einsum("sbc,hvc->sbhv", kv_c, W[:, dn:])
        gate = torch.tanh(scale * (q_lat * kv_c[:, :, None]).sum(-1, keepdim=True) + q_pe.sum(-1, keepdim=True)
                          + k_pe.sum(-1)[:, :, None, None])
        out = (gate * v).reshape(S, B, -1)
        if indexer_loss is None:
            return out
        q_i, k_i, w_i, coeff, loss_scale = indexer_loss[:5]
        loss = coeff * ((q_i.sum(-1) * w_i).pow(2).mean() + k_i.pow(2).mean())
        return dsa.attach_indexer_loss(out, loss, loss_scale), loss.detach()
    return attn


def _module(flag, coeff, seed=0):
    torch.manual_seed(seed)
    H, hidden, qlr = 4, 48, 32
    cfg = M.make_config(H, qlr, coeff=coeff, sparse=False)
    core = M.CoreAttention(_FakeIndexer(hidden, qlr, K=5), softmax_scale=0.1)
    cls = mla.absorbed_mla_class(M.MLASelfAttention)
    mod = cls(cfg, hidden, core, dtype=torch.float32)
    if flag:
        setattr(mod, flag, True)
    return mod


@pytest.mark.parametrize("coeff", [0.0, 0.5])
@pytest.mark.parametrize("flag", ["checkpoint_core_attention", "recompute_up_proj"])
def test_recompute_flags_checkpoint_the_absorbed_attention(flag, coeff, monkeypatch):
    calls = []
    monkeypatch.setattr(mla, "absorbed_mla_sparse_attention", _fake_attention(calls))
    base = _module(None, coeff)
    flagged = _module(flag, coeff)
    flagged.load_state_dict(copy.deepcopy(base.state_dict()))
    g = torch.Generator().manual_seed(1)
    S, B = 12, 2
    x = torch.randn(S, B, 48, generator=g)
    rope = torch.rand(S, 1, 1, 64, generator=g) * 10
    dout = torch.randn(S, B, 48, generator=g)
    res = []
    for mod in (base, flagged):
        mod.train()
        ups = []
        h = mod.linear_q_up_proj.register_forward_hook(lambda *a: ups.append(1))
        calls.clear()
        xi = x.clone().requires_grad_()
        out, _ = mod(xi, None, rotary_pos_emb=rope)
        n_fwd = len(calls)
        (out * dout).sum().backward()
        h.remove()
        grads = {n: p.grad.clone() for n, p in mod.named_parameters() if p.grad is not None}
        res.append((out.detach(), xi.grad, grads, mod.last_indexer_loss, n_fwd, len(calls), len(ups)))
    (o0, dx0, g0, l0, f0, c0, u0), (o1, dx1, g1, l1, f1, c1, u1) = res
    assert f0 == f1 == 1
    assert c0 == 1 and c1 == 2, "the flagged run recomputes the core attention in the backward"
    assert u0 == 1 and u1 == (2 if flag == "recompute_up_proj" else 1)
    assert torch.equal(o0, o1) and torch.equal(dx0, dx1)
    assert g0.keys() == g1.keys() and all(torch.equal(g0[n], g1[n]) for n in g0)
    if coeff:
        assert l0 is not None and torch.equal(l0, l1)
        assert any(n.startswith("core_attention.indexer") for n in g1)
    # no recomputation without gradients (and checkpoint_core_attention only in training)
    calls.clear()
    with torch.no_grad():
        flagged(x, None, rotary_pos_emb=rope)
    flagged.eval()
    flagged(x.clone().requires_grad_(), None, rotary_pos_emb=rope)[0].sum().backward()
    assert len(calls) == (2 if flag == "checkpoint_core_attention" else 3)
