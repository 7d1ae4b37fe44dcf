"""DeepSeek-V4 compressor kernels (``dsa_v4_compress_fwd`` / ``dsa_v4_compress_bwd`` through
``v4.compress``) against

- the float64 oracle ``oracle/dsv4_oracle.py::compress_windows`` (pinned through the whole layer
  against transformers' DeepseekV4Attention in ``tests/test_oracle_v4.py``), forward and float64
  autograd backward,
  document by document: CSA main (rate 4, overlap, D 512) and index (D 128) compressors, HCA
  (rates 16 and 128, D 512), odd rates and multi-chunk windows (rate 3 / 12 with overlap), ragged
  documents with partial tails, documents shorter than a window and empty ones, strided rows;
- a torch fp32 restatement with the module's bf16 steps (pooled sums and the normalised row
  rounded to bf16), for a tighter forward bar, and at the V4 bench size (T = 16384);
- the structure of the gradient: exact zeros where a token feeds no entry, bit-identical reruns.

Bars: forward within rtol = atol = 2e-2 of float64 (normalised error < 1e-2), within 1.6e-2 /
1e-2 of the bf16-step restatement (normalised < 3e-3); every gradient normalised error < 1e-2
against float64 autograd."""
import pytest
import torch

from oracle import dsv4_oracle as V
from mcore_bridge_amd import v4

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
EPS = 1e-6


def _inputs(T, D, rate, overlap, seed, row_pad=0):
    g = torch.Generator().manual_seed(seed)
    C = 2 * D if overlap else D
    kv = torch.randn(T, C + row_pad, generator=g).bfloat16()
    gate = (torch.randn(T, C + row_pad, generator=g) * 2).bfloat16()
    ape = (torch.randn(rate, C, generator=g) * 0.5).bfloat16()
    norm_w = (1 + 0.2 * torch.randn(D, generator=g)).bfloat16()
    return kv, gate, ape, norm_w


def _oracle(kv, gate, ape, norm_w, cu, rate, overlap):
    outs = [V.compress_windows(kv[a:b], gate[a:b], ape, norm_w, rate, EPS, overlap) for a, b in zip(cu[:-1], cu[1:])]
    return torch.cat(outs)


def _bf16_steps(kv, gate, ape, norm_w, cu, rate, overlap):
    """torch fp32 restatement with the module's dtype steps (pooled sum and normalised row in bf16)."""
    outs = []
    for a, b in zip(cu[:-1], cu[1:]):
        n = (b - a) // rate
        if n == 0:
            continue
        k = kv[a:a + n * rate].float().view(n, rate, -1)
        g = gate[a:a + n * rate].float().view(n, rate, -1) + ape.float()
        if overlap:
            D = k.shape[-1] // 2
            pk = torch.zeros_like(k[..., D:])
            pg = torch.full_like(g[..., D:], float("-inf"))
            pk[1:], pg[1:] = k[:-1, :, :D], g[:-1, :, :D]
            k = torch.cat([pk, k[..., D:]], dim=1)
            g = torch.cat([pg, g[..., D:]], dim=1)
        outs.append((k * torch.softmax(g, dim=1)).sum(1))
    x = torch.cat(outs).to(torch.bfloat16).float()
    y = (x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + EPS)).to(torch.bfloat16)
    return y * norm_w


def _err(got, ref):
    got, ref = got.double().cpu(), ref.double().cpu()
    return ((got - ref).norm() / ref.norm().clamp_min(1e-30)).item()


CASES = [  # (doc lengths, D, rate, overlap, row_pad)
    ([37, 64, 3, 0, 21], 512, 4, True, 0),     # CSA main compressor, ragged documents
    ([50, 29], 128, 4, True, 0),               # CSA index compressor
    ([70, 96, 41], 512, 16, False, 0),         # HCA (the layer tests' rate)
    ([300, 129, 5], 512, 128, False, 0),       # HCA at its model rate: 16 chunks per window
    ([10, 7, 2], 64, 3, True, 8),              # odd rate, strided rows
    ([61, 24], 256, 12, True, 0),              # 24 slots: three chunks, the first window clamped
]


@pytest.mark.parametrize("lens,D,rate,overlap,row_pad", CASES)
def test_v4_compress_forward_backward_match_oracle(lens, D, rate, overlap, row_pad):
    print(f"[v4 compress] lens={lens} D={D} rate={rate} overlap={overlap}", flush=True)
    cu = [0]
    for n in lens:
        cu.append(cu[-1] + n)
    T = cu[-1]
    C = 2 * D if overlap else D
    kv_w, gate_w, ape, norm_w = _inputs(T, D, rate, overlap, seed=len(lens) * 100 + rate, row_pad=row_pad)
    kv_c, gate_c = kv_w[:, :C], gate_w[:, :C]

    # GPU: leaves on strided views (row stride C + row_pad)
    kvd = kv_w.to(DEV)[:, :C].detach().requires_grad_()
    gd = gate_w.to(DEV)[:, :C].detach().requires_grad_()
    ad = ape.to(DEV).requires_grad_()
    nd = norm_w.to(DEV).requires_grad_()
    out = v4.compress(kvd, gd, ad, nd, cu, rate, EPS, overlap)
    n_ent = sum(n // rate for n in lens)
    assert out.shape == (n_ent, D) and out.dtype == torch.bfloat16
    dout = (torch.randn(n_ent, D, generator=torch.Generator().manual_seed(7)) * 0.1).bfloat16()
    out.backward(dout.to(DEV))
    torch.cuda.synchronize()

    # forward against float64 and against the bf16-step restatement
    ref = _oracle(kv_c, gate_c, ape, norm_w, cu, rate, overlap)
    got = out.detach().double().cpu()
    e = _err(got, ref)
    assert e < 1e-2 and torch.allclose(got, ref, rtol=2e-2, atol=2e-2), f"forward vs float64: {e:.3e}"
    ref16 = _bf16_steps(kv_c, gate_c, ape, norm_w, cu, rate, overlap).double()
    e16 = _err(got, ref16)
    assert e16 < 3e-3 and torch.allclose(got, ref16, rtol=1.6e-2, atol=1e-2), f"forward vs bf16 steps: {e16:.3e}"

    # backward against float64 autograd through the oracle
    leaves = [t.double().requires_grad_() for t in (kv_c, gate_c, ape, norm_w)]
    ref_o = _oracle(*leaves, cu, rate, overlap)
    ref_o.backward(dout.double())
    for name, g_got, leaf in (("dkv", kvd.grad, leaves[0]), ("dgate", gd.grad, leaves[1]),
                              ("dape", ad.grad, leaves[2]), ("dnorm_w", nd.grad, leaves[3])):
        eg = _err(g_got, leaf.grad)
        print(f"  {name}: normalised error {eg:.2e}", flush=True)
        assert eg < 1e-2, f"{name}: normalised error {eg:.3e}"

    # gradients are exactly zero where a token feeds no entry
    covered = torch.zeros(T, C, dtype=torch.bool)
    for a, b in zip(cu[:-1], cu[1:]):
        n = (b - a) // rate
        if overlap:
            covered[a:a + n * rate, C // 2:] = True
            covered[a:a + max(n - 1, 0) * rate, :C // 2] = True
        else:
            covered[a:a + n * rate] = True
    for g_got in (kvd.grad, gd.grad):
        assert torch.count_nonzero(g_got.cpu()[~covered]) == 0

    # a second backward gives the same bits
    kv2, g2 = kvd.detach().requires_grad_(), gd.detach().requires_grad_()
    a2, n2 = ad.detach().requires_grad_(), nd.detach().requires_grad_()
    v4.compress(kv2, g2, a2, n2, cu, rate, EPS, overlap).backward(dout.to(DEV))
    for x, y in ((kv2.grad, kvd.grad), (g2.grad, gd.grad), (a2.grad, ad.grad), (n2.grad, nd.grad)):
        assert torch.equal(x, y)


def test_v4_compress_bench_size_matches_torch_restatement():
    """The CSA main compressor at the V4 bench size (one document of T = 16384 tokens, rate 4,
    D 512): forward against the bf16-step restatement, gradients against float64 autograd through
    the oracle (both on the GPU)."""
    print("[v4 compress] T=16384 rate 4 overlap D 512", flush=True)
    T, D, rate = 16384, 512, 4
    kv, gate, ape, norm_w = (t.to(DEV) for t in _inputs(T, D, rate, True, seed=11))
    leaves = [t.detach().requires_grad_() for t in (kv, gate, ape, norm_w)]
    out = v4.compress(*leaves, [0, T], rate, EPS, True)
    dout = (torch.randn(T // rate, D, device=DEV, generator=torch.Generator(device=DEV).manual_seed(3)) * 0.1).bfloat16()
    out.backward(dout)
    rl = [t.detach().float().requires_grad_() for t in (kv, gate, ape, norm_w)]
    ref = _bf16_steps(rl[0], rl[1], rl[2], rl[3], [0, T], rate, True)
    e = _err(out.detach(), ref.detach())
    assert e < 3e-3 and torch.allclose(out.detach().float(), ref.detach().float(), rtol=1.6e-2, atol=1e-2), e
    # float64 autograd through the oracle (no bf16 steps)
    ref32 = V.compress_windows(rl[0], rl[1], rl[2], rl[3], rate, EPS, True)
    ref32.backward(dout.double())
    for name, g_got, leaf in zip(("dkv", "dgate", "dape", "dnorm_w"), (t.grad for t in leaves), rl):
        eg = _err(g_got, leaf.grad)
        print(f"  {name}: normalised error {eg:.2e}", flush=True)
        assert eg < 1e-2, f"{name}: normalised error {eg:.3e}"


@pytest.mark.parametrize("T,D,rate", [(140_000, 64, 4), (530_000, 64, 64)])
def test_v4_compress_many_entries_grid_stride(T, D, rate):
    """More backward items than the backward grid holds (1024 workgroups of 32 items at D = 64;
    of 8 items when rate-64 overlapped windows are split over the waves), three documents: forward
    and gradients against the bf16-step restatement and its fp32 autograd on the GPU."""
    print(f"[v4 compress] grid stride T={T} D={D} rate={rate}", flush=True)
    cu = [0, T // 3 + 1, 2 * (T // 3) - 5, T]
    kv, gate, ape, norm_w = (t.to(DEV) for t in _inputs(T, D, rate, True, seed=T % 97))
    leaves = [t.detach().requires_grad_() for t in (kv, gate, ape, norm_w)]
    out = v4.compress(*leaves, cu, rate, EPS, True)
    n_ent = sum((b - a) // rate for a, b in zip(cu[:-1], cu[1:]))
    dout = (torch.randn(n_ent, D, device=DEV, generator=torch.Generator(device=DEV).manual_seed(5)) * 0.1).bfloat16()
    out.backward(dout)
    rl = [t.detach().float().requires_grad_() for t in (kv, gate, ape, norm_w)]
    ref = _bf16_steps(rl[0], rl[1], rl[2], rl[3], cu, rate, True)
    e = _err(out.detach(), ref.detach())
    assert e < 3e-3, f"forward: {e:.3e}"
    ref.float().backward(dout.float())
    for name, g_got, leaf in zip(("dkv", "dgate", "dape", "dnorm_w"), (t.grad for t in leaves), rl):
        eg = _err(g_got, leaf.grad)
        print(f"  {name}: normalised error {eg:.2e}", flush=True)
        assert eg < 1e-2, f"{name}: normalised error {eg:.3e}"


@pytest.mark.parametrize("draw", range(12))
def test_v4_compress_seeded_sweep(draw):
    """Seeded draws (inputs from the seed alone): dim 64..512, rate 1..20, with and without
    overlap, 1..4 documents of 0..70 tokens (empty ones, ones shorter than a window, partial
    tails); forward and gradients against float64, gradients zero where a token feeds no entry."""
    r = torch.Generator().manual_seed(1000 + draw)
    D = [64, 128, 256, 512][int(torch.randint(0, 4, (1,), generator=r))]
    rate = int(torch.randint(1, 21, (1,), generator=r))
    overlap = bool(torch.randint(0, 2, (1,), generator=r))
    lens = [int(x) for x in torch.randint(0, 71, (int(torch.randint(1, 5, (1,), generator=r)),), generator=r)]
    if sum(n // rate for n in lens) == 0:
        lens.append(rate * 2 + 1)
    print(f"[v4 compress sweep] draw {draw}: D={D} rate={rate} overlap={overlap} lens={lens}", flush=True)
    cu = [0]
    for n in lens:
        cu.append(cu[-1] + n)
    T, C = cu[-1], (2 * D if overlap else D)
    kv, gate, ape, norm_w = _inputs(T, D, rate, overlap, seed=2000 + draw)
    leaves = [t.to(DEV).requires_grad_() for t in (kv, gate, ape, norm_w)]
    out = v4.compress(*leaves, cu, rate, EPS, overlap)
    n_ent = sum(n // rate for n in lens)
    dout = (torch.randn(n_ent, D, generator=r) * 0.1).bfloat16()
    out.backward(dout.to(DEV))
    ref_l = [t.double().requires_grad_() for t in (kv, gate, ape, norm_w)]
    ref = _oracle(*ref_l, cu, rate, overlap)
    ref.backward(dout.double())
    e = _err(out.detach(), ref.detach())
    assert e < 1e-2, f"forward {e:.3e}"
    for name, got, leaf in zip(("dkv", "dgate", "dape", "dnorm_w"), (t.grad for t in leaves), ref_l):
        eg = _err(got, leaf.grad)
        assert eg < 1e-2, f"{name}: {eg:.3e}"
    covered = torch.zeros(T, C, dtype=torch.bool)
    for a, b in zip(cu[:-1], cu[1:]):
        n = (b - a) // rate
        if overlap:
            covered[a:a + n * rate, C // 2:] = True
            covered[a:a + max(n - 1, 0) * rate, :C // 2] = True
        else:
            covered[a:a + n * rate] = True
    for got in (leaves[0].grad, leaves[1].grad):
        assert torch.count_nonzero(got.cpu()[~covered]) == 0


def test_v4_compress_no_complete_window():
    """Documents all shorter than a window: no entry, and every gradient zero (dkv, dgate, dape,
    dnorm_w) -- the backward still runs its partial-tail items and column sums."""
    print("[v4 compress] no complete window", flush=True)
    cu, rate, D = [0, 3, 3, 6], 4, 128
    kv, gate, ape, norm_w = _inputs(6, D, rate, True, seed=9)
    leaves = [t.to(DEV).requires_grad_() for t in (kv, gate, ape, norm_w)]
    out = v4.compress(*leaves, cu, rate, EPS, True)
    assert out.shape == (0, D)
    out.backward(torch.zeros(0, D, dtype=torch.bfloat16, device=DEV))
    for t in leaves:
        assert t.grad is not None and torch.count_nonzero(t.grad) == 0
