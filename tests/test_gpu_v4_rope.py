"""DeepSeek-V4 row transforms on the HIP kernels (``dsa_v4_norm_rope`` / ``dsa_v4_out_rope_group``
and their backwards, through ``v4.norm_rope`` and the layer's ``_OutRopeGroup`` / ``_GroupedProj``)
against the torch composition they replace (deepseek_v4.py:114-142 and :287-318: weightless per-head
RMS norm, interleaved RoPE on the last 64 dims, the inverse RoPE of the output, the grouped output
projection) and against float64 autograd.

Bars: the rotations (no norm) and the grouped layout are bit-exact against the fp32 torch
composition, forward and backward (same rounding steps: each product rounded, then the sum, then
bf16); with the RMS norm, within one bf16 step of each rotation input of the composition (the
mean's summation order differs), on under 1 % of the elements, and normalised error < 1e-2 of
float64 autograd for the gradient; the grouped projection
within rtol = atol = 2e-2 of float64."""
import pytest
import torch

from mcore_bridge_amd import v4

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
RD = 64


def _torch_rope(x, cos, sin, inverse=False):
    """The interleaved RoPE as the layer composed it in torch (fp32 rotation of the last RD dims)."""
    shape = [cos.shape[0]] + [1] * (x.dim() - 2) + [cos.shape[-1]]
    c, s = cos.view(shape), sin.view(shape)
    if inverse:
        s = -s
    nope, rope = x[..., :-RD], x[..., -RD:].float()
    a, b = rope[..., 0::2], rope[..., 1::2]
    out = torch.stack((a * c - b * s, b * c + a * s), dim=-1).flatten(-2)
    return torch.cat([nope, out.to(x.dtype)], dim=-1)


def _torch_rms(x, eps):
    y = x.float() * torch.rsqrt(x.float().pow(2).mean(-1, keepdim=True) + eps)
    return y.to(x.dtype)


def _tables(T, seed, mscale=1.0):
    g = torch.Generator(device=DEV).manual_seed(seed)
    inv = 1.0 / (10000 ** (torch.arange(0, RD, 2, device=DEV).float() / RD))
    pos = torch.randint(0, 40000, (T,), device=DEV, generator=g).float()
    return v4.rope_tables(torch.outer(pos, inv), mscale)


def _err(got, ref):
    got, ref = got.double(), ref.double()
    return ((got - ref).norm() / ref.norm().clamp_min(1e-30)).item()


@pytest.mark.parametrize("T,H,D", [(333, 16, 512), (1000, 64, 128), (17, 1, 512)])
def test_rope_only_bit_exact_fwd_bwd(T, H, D):
    print(f"[v4 rope] rope only T={T} H={H} D={D}", flush=True)
    cos, sin = _tables(T, T + H, mscale=1.3)
    g = torch.Generator(device=DEV).manual_seed(1)
    x = torch.randn(T, H, D, device=DEV, generator=g).bfloat16()
    dy = torch.randn(T, H, D, device=DEV, generator=g).bfloat16()
    for inverse in (False, True):
        xa = x.clone().requires_grad_()
        ya = v4._NormRope.apply(xa, cos, sin, RD, False, 0.0, inverse)
        ya.backward(dy)
        xb = x.clone().requires_grad_()
        yb = _torch_rope(xb, cos, sin, inverse)
        yb.backward(dy)
        assert torch.equal(ya, yb), f"forward inverse={inverse}"
        assert torch.equal(xa.grad, xb.grad), f"backward inverse={inverse}"


@pytest.mark.parametrize("T,H,D", [(257, 128, 512), (300, 16, 128)])
def test_norm_rope_matches_composition_and_float64(T, H, D):
    print(f"[v4 rope] norm + rope T={T} H={H} D={D}", flush=True)
    cos, sin = _tables(T, 7)
    g = torch.Generator(device=DEV).manual_seed(2)
    x = (torch.randn(T, H, D, device=DEV, generator=g) * 3).bfloat16()
    dy = torch.randn(T, H, D, device=DEV, generator=g).bfloat16()
    eps = 1e-6
    xa = x.clone().requires_grad_()
    ya = v4.norm_rope(xa, cos, sin, True, eps)
    ya.backward(dy)
    yn = _torch_rms(x, eps)
    yb = _torch_rope(yn, cos, sin)
    # the normed row may differ by one bf16 step (the mean's summation order), rarely; through the
    # rotation such a step moves an output by at most a step of |a| + |b| of its pair, plus the
    # output's own rounding
    diff = (ya.float() - yb.float()).abs()
    mag = yn.float().abs()
    pair = mag[..., -RD:].view(T, H, RD // 2, 2).sum(-1, keepdim=True).expand(T, H, RD // 2, 2).reshape(T, H, RD)
    mag = torch.cat([mag[..., :-RD], pair], -1)
    bound = (mag + yb.float().abs()) * 2 ** -7
    assert bool((diff <= bound).all()), f"max diff {diff.max().item()}"
    assert (diff > 0).float().mean().item() < 0.01
    # gradient against float64 autograd of the same composition
    xd = x.double().requires_grad_()
    yd = xd * torch.rsqrt(xd.pow(2).mean(-1, keepdim=True) + eps)
    c, s = cos.double().view(T, 1, -1), sin.double().view(T, 1, -1)
    a, b = yd[..., -RD:][..., 0::2], yd[..., -RD:][..., 1::2]
    yd = torch.cat([yd[..., :-RD], torch.stack((a * c - b * s, b * c + a * s), -1).flatten(-2)], -1)
    yd.backward(dy.double())
    e = _err(xa.grad, xd.grad)
    assert e < 1e-2, f"dx normalised error {e:.3e}"
    e_f = _err(ya, yd.detach())
    assert e_f < 1e-2, f"forward vs float64 {e_f:.3e}"


@pytest.mark.parametrize("T,H,G", [(200, 128, 8), (77, 16, 4), (5, 8, 1)])
def test_out_rope_group_bit_exact_fwd_bwd(T, H, G):
    print(f"[v4 rope] output rope + groups T={T} H={H} G={G}", flush=True)
    D = 512
    cos, sin = _tables(T, 11, mscale=0.8)
    g = torch.Generator(device=DEV).manual_seed(3)
    o = torch.randn(T, H, D, device=DEV, generator=g).bfloat16()
    dog = torch.randn(G, T, H * D // G, device=DEV, generator=g).bfloat16()
    oa = o.clone().requires_grad_()
    og = v4._OutRopeGroup.apply(oa, cos, sin, G)
    og.backward(dog)
    ob = o.clone().requires_grad_()
    ref = _torch_rope(ob, cos, sin, inverse=True).reshape(T, G, -1).transpose(0, 1)
    ref.backward(dog)
    assert og.shape == (G, T, H * D // G) and og.is_contiguous()
    assert torch.equal(og, ref)
    assert torch.equal(oa.grad, ob.grad)


def test_grouped_projection_matches_float64():
    print("[v4 rope] grouped projection", flush=True)
    G, T, K, N = 4, 300, 1024, 256
    g = torch.Generator(device=DEV).manual_seed(4)
    a = (torch.randn(G, T, K, device=DEV, generator=g) * 0.1).bfloat16().requires_grad_()
    w = (torch.randn(G, N, K, device=DEV, generator=g) * 0.05).bfloat16().requires_grad_()
    out = v4._GroupedProj.apply(a, w)
    gout = torch.randn(T, G * N, device=DEV, generator=g).bfloat16()
    out.backward(gout)
    ad, wd = a.detach().double().requires_grad_(), w.detach().double().requires_grad_()
    ref = torch.bmm(ad, wd.transpose(1, 2).contiguous()).transpose(0, 1).reshape(T, -1)
    ref.backward(gout.double())
    for name, got, r in (("out", out, ref), ("da", a.grad, ad.grad), ("dw", w.grad, wd.grad)):
        e = _err(got, r.detach())
        assert e < 1e-2 and torch.allclose(got.double(), r.detach(), rtol=2e-2, atol=2e-2 * r.abs().max().item()), \
            f"{name}: {e:.3e}"


@pytest.mark.parametrize("draw", range(12))
def test_norm_rope_seeded_sweep(draw):
    """Seeded draws: dim 64..512, rope_dim 0..dim in steps of 8, 1..130 heads, norm on / off,
    inverse or not, mscale 0.5..1.5: forward and backward of the HIP rows against the torch
    composition (bit-exact without the norm) and float64 autograd (with it)."""
    r = torch.Generator().manual_seed(3000 + draw)
    D = [64, 128, 256, 512][int(torch.randint(0, 4, (1,), generator=r))]
    rd = 8 * int(torch.randint(0, D // 8 + 1, (1,), generator=r))
    H = int(torch.randint(1, 131, (1,), generator=r))
    T = int(torch.randint(1, 90, (1,), generator=r))
    norm = bool(torch.randint(0, 2, (1,), generator=r))
    inverse = bool(torch.randint(0, 2, (1,), generator=r))
    mscale = 0.5 + float(torch.rand(1, generator=r))
    print(f"[v4 rope sweep] draw {draw}: T={T} H={H} D={D} rope={rd} norm={norm} inverse={inverse}", flush=True)
    inv = 1.0 / (10000 ** (torch.arange(0, max(rd, 2), 2).double() / max(rd, 2)))
    ang = torch.outer(torch.randint(0, 20000, (T,), generator=r).double(), inv).float().to(DEV)
    cos, sin = v4.rope_tables(ang, mscale)
    x = (torch.randn(T, H, D, generator=r) * 2).bfloat16().to(DEV)
    dy = torch.randn(T, H, D, generator=r).bfloat16().to(DEV)
    xa = x.clone().requires_grad_()
    ya = v4._NormRope.apply(xa, cos, sin, rd, norm, 1e-6, inverse)
    ya.backward(dy)
    # float64 composition
    xd = x.double().requires_grad_()
    yd = xd * torch.rsqrt(xd.pow(2).mean(-1, keepdim=True) + 1e-6) if norm else xd
    if rd:
        c, s = cos.double()[:, : rd // 2].view(T, 1, -1), sin.double()[:, : rd // 2].view(T, 1, -1)
        if inverse:
            s = -s
        a, b = yd[..., D - rd:][..., 0::2], yd[..., D - rd:][..., 1::2]
        yd = torch.cat([yd[..., :D - rd], torch.stack((a * c - b * s, b * c + a * s), -1).flatten(-2)], -1)
    yd.backward(dy.double())
    assert _err(ya, yd.detach()) < 1e-2
    assert _err(xa.grad, xd.grad) < 1e-2
    if not norm and rd == RD:   # the rotation alone: the fp32 torch composition bit for bit
        xb = x.clone().requires_grad_()
        yb = _torch_rope(xb, cos[:, : rd // 2].contiguous(), sin[:, : rd // 2].contiguous(), inverse)
        yb.backward(dy)
        assert torch.equal(ya, yb) and torch.equal(xa.grad, xb.grad)
