"""Inputs of the golden cases.  Each case is regenerated from a seed (CPU generator, fixed draw
order) or a fixed rule; the fixture files hold checksums of these inputs, so RNG drift shows up
as a checksum mismatch instead of a silent change of the expected outputs.

All values are those the kernels take: q, kv, q_idx, k_idx and dO rounded to bf16 (held here as
float32 tensors with bf16-exact values), w in float32.

Cases (DSA prefill chain: indexer scores -> top-k -> sparse MLA forward -> backward):
  cfg1            config 1 (S = 512 causal, H = 16, Hi = 4, Di = 64, K = 128, w ~ U(0, 1), seed 0)
  ties            3 distinct key rows repeated: every query row holds long runs of equal scores,
                  the lower index must win (exact dyadic values, exact in fp32)
  s_lt_k          two documents shorter than K = 128: every visible key selected, -1 padding
  one_token_docs  documents of one token among longer ones: K = 4
  zero_relu       q_idx <= 0 <= k_idx: every ReLU is zero, all scores are 0 (some -0 through
                  negative head weights), so the lowest indices win
"""
import numpy as np
import torch

from mcore_bridge_amd import workloads as W

SM_SCALE = W.SM_SCALE
H = 16                     # attention heads of every case
NAMES = ("cfg1", "ties", "s_lt_k", "one_token_docs", "zero_relu")


def _bf16(x: torch.Tensor) -> torch.Tensor:
    return x.to(torch.bfloat16).to(torch.float32)


def _attention_inputs(T: int, g: torch.Generator):
    q = _bf16(torch.randn(T, H, 576, generator=g) * 0.1)
    kv = _bf16(torch.randn(T, 576, generator=g) * 0.1)
    dout = _bf16(torch.randn(T, H, 512, generator=g) * 0.01)
    return q, kv, dout


def inputs(name: str) -> dict:
    """``{q, kv, q_idx, k_idx, w, dout, cu_seqlens (list), K, causal}`` of case ``name``."""
    if name == "cfg1":
        d = W.make_prefill(W.CONFIGS["cfg1"], seed=0)
        return dict(q=_bf16(d["q"]), kv=_bf16(d["kv"]), q_idx=_bf16(d["q_idx"]), k_idx=_bf16(d["k_idx"]),
                    w=d["w"].float(), dout=_bf16(d["dout"]), cu_seqlens=[0, 512], K=128, causal=True)
    if name == "ties":
        T, Hi, Di = 96, 4, 64
        g = torch.Generator().manual_seed(101)
        q, kv, dout = _attention_inputs(T, g)
        base = torch.zeros(3, Di)
        base[0, :8] = 0.25            # the three key classes score 2, 1 and 0.5 against q_idx
        base[1, :4] = 0.25
        base[2, :2] = 0.25
        k_idx = base[torch.arange(T) % 3]
        q_idx = torch.zeros(T, Hi, Di)
        q_idx[:, :, :8] = 1.0
        w = torch.full((T, Hi), 0.5)
        return dict(q=q, kv=kv, q_idx=q_idx, k_idx=k_idx, w=w, dout=dout, cu_seqlens=[0, 50, T], K=16,
                    causal=True)
    if name == "s_lt_k":
        T, Hi, Di = 100, 4, 64
        g = torch.Generator().manual_seed(102)
        q, kv, dout = _attention_inputs(T, g)
        q_idx = _bf16(torch.randn(T, Hi, Di, generator=g) * 0.1)
        k_idx = _bf16(torch.randn(T, Di, generator=g) * 0.1)
        w = torch.randn(T, Hi, generator=g) / 8
        return dict(q=q, kv=kv, q_idx=q_idx, k_idx=k_idx, w=w, dout=dout, cu_seqlens=[0, 37, T], K=128,
                    causal=True)
    if name == "one_token_docs":
        T, Hi, Di = 24, 4, 64
        g = torch.Generator().manual_seed(103)
        q, kv, dout = _attention_inputs(T, g)
        q_idx = _bf16(torch.randn(T, Hi, Di, generator=g) * 0.1)
        k_idx = _bf16(torch.randn(T, Di, generator=g) * 0.1)
        w = torch.rand(T, Hi, generator=g)
        return dict(q=q, kv=kv, q_idx=q_idx, k_idx=k_idx, w=w, dout=dout, cu_seqlens=[0, 1, 2, 3, 9, 10, 23, T],
                    K=4, causal=True)
    if name == "zero_relu":
        T, Hi, Di = 200, 4, 64
        g = torch.Generator().manual_seed(104)
        q, kv, dout = _attention_inputs(T, g)
        q_idx = -_bf16(torch.randn(T, Hi, Di, generator=g).abs() * 0.1)
        k_idx = _bf16(torch.randn(T, Di, generator=g).abs() * 0.1)
        w = torch.randn(T, Hi, generator=g)
        return dict(q=q, kv=kv, q_idx=q_idx, k_idx=k_idx, w=w, dout=dout, cu_seqlens=[0, T], K=64, causal=True)
    raise KeyError(name)


def rows_from_bits(a) -> torch.Tensor:
    """float32 tensor of a fixture's bf16 bit-pattern array (uint16)."""
    return torch.from_numpy(np.asarray(a).view(np.int16).copy()).view(torch.bfloat16).to(torch.float32)


def load(name: str, directory: str) -> dict:
    """The fixture arrays of case ``name`` (numpy, no pickles)."""
    with np.load(f"{directory}/{name}.npz", allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def checksums(d: dict) -> torch.Tensor:
    """float64 [sum, sum of |x|] of every tensor input, in a fixed order."""
    out = []
    for k in ("q", "kv", "q_idx", "k_idx", "w", "dout"):
        x = d[k].to(torch.float64)
        out += [x.sum(), x.abs().sum()]
    return torch.stack(out)
