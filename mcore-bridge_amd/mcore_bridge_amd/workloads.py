"""Synthetic workloads of the five benchmark configurations (shapes and input statistics).

Inputs are drawn in the fixed order q, kv, q_idx, k_idx, w, dO from one seeded generator,
in fp32, then cast; ``device="cpu"`` reproduces bit-identical values for the CPU oracle, a
CUDA device draws on the GPU (fast, used by bench.py for the large configurations).
Integer fixtures (document lengths, cache lengths) are constants, not RNG output.
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field
from typing import Dict, List, Optional

import torch

SM_SCALE = 1.0 / math.sqrt(192.0)

# config 3: lengths 10363/4977/197/847 (sort(randperm(16383, seed 0)[:3] + 1) as constants)
CFG3_CU_SEQLENS = [0, 10363, 15340, 15537, 16384]
# config 5: per-sequence cache lengths (seed 0, randint(16384, 65537, (64,))) as constants
CFG5_CACHE_LENS = [20313, 40917, 62041, 44181, 25990, 60965, 48328, 39991, 54127, 51709, 62624, 21439, 25032,
                   38089, 52196, 43645, 37228, 45180, 63066, 24503, 44970, 62705, 46033, 25818, 40053, 34112,
                   27319, 25785, 21262, 42271, 32076, 64088, 49549, 54816, 63170, 55314, 65124, 55144, 29882,
                   57541, 27979, 48828, 22290, 27474, 58736, 20854, 30761, 25819, 54064, 43951, 17076, 47385,
                   23579, 37710, 53263, 40753, 59393, 24228, 64364, 65265, 53335, 47717, 25991, 45035]


@dataclass
class Config:
    name: str
    S: int                      # total query tokens (prefill) / batch (decode)
    H: int = 128
    Hi: int = 64
    Di: int = 128
    K: int = 2048
    cu_seqlens: Optional[List[int]] = None
    w_uniform: bool = False     # w ~ U(0,1) (config 1) instead of N(0,1)/8
    fp8_indexer: bool = False
    backward: bool = False
    decode_lens: Optional[List[int]] = None
    dtype: torch.dtype = torch.bfloat16
    notes: str = ""

    @property
    def docs(self) -> List[int]:
        return self.cu_seqlens if self.cu_seqlens is not None else [0, self.S]


CONFIGS: Dict[str, Config] = {
    "cfg1": Config("cfg1", S=512, H=16, Hi=4, Di=64, K=128, w_uniform=True, backward=True, dtype=torch.float32,
                   notes="CPU-runnable tiny DSA, fp32 reference"),
    "cfg2": Config("cfg2", S=4096, notes="bf16 DSA forward, causal"),
    "cfg3": Config("cfg3", S=16384, cu_seqlens=CFG3_CU_SEQLENS, backward=True,
                   notes="bf16 DSA forward+backward, packed varlen, causal per document"),
    "cfg4": Config("cfg4", S=32768, fp8_indexer=True, notes="fp8 indexer + bf16 sparse forward"),
    "cfg5": Config("cfg5", S=64, decode_lens=CFG5_CACHE_LENS, notes="decode over long latent caches"),
}


def n_sel(cu_seqlens: List[int], K: int) -> int:
    """Attended (query, key) pairs per head: sum_q min(K, #causally visible keys)."""
    tot = 0
    for a, b in zip(cu_seqlens[:-1], cu_seqlens[1:]):
        n = b - a
        m = min(K, n)
        tot += m * (m + 1) // 2 + (n - m) * K
    return tot


def n_pairs(cu_seqlens: List[int]) -> int:
    """Causally visible (query, key) pairs (indexer work)."""
    return sum((b - a) * (b - a + 1) // 2 for a, b in zip(cu_seqlens[:-1], cu_seqlens[1:]))


def make_prefill(cfg: Config, device="cpu", seed: int = 0, S: Optional[int] = None,
                 cu_seqlens: Optional[List[int]] = None, H: Optional[int] = None) -> Dict[str, torch.Tensor]:
    """Draw the prefill inputs of ``cfg`` (optionally with a smaller S / H / document split)."""
    S = S or cfg.S
    H = H or cfg.H
    cu = cu_seqlens or (cfg.cu_seqlens if (cfg.cu_seqlens and S == cfg.S) else [0, S])
    g = torch.Generator(device=device).manual_seed(seed)
    f32 = dict(dtype=torch.float32, device=device, generator=g)
    out = {}
    out["q"] = torch.randn(S, H, 576, **f32) * 0.1
    out["kv"] = torch.randn(S, 576, **f32) * 0.1
    if cfg.fp8_indexer:
        out["q_idx"] = torch.randn(S, cfg.Hi, cfg.Di, **f32)
        out["k_idx"] = torch.randn(S, cfg.Di, **f32)
    else:
        out["q_idx"] = torch.randn(S, cfg.Hi, cfg.Di, **f32) * 0.1
        out["k_idx"] = torch.randn(S, cfg.Di, **f32) * 0.1
    if cfg.w_uniform:
        out["w"] = torch.rand(S, cfg.Hi, **f32)
    else:
        out["w"] = torch.randn(S, cfg.Hi, **f32) / 8
    if cfg.backward:
        out["dout"] = torch.randn(S, H, 512, **f32) * 0.01
    out["cu_seqlens"] = torch.tensor(cu, dtype=torch.int32, device=device)
    return out


E4M3_MAX = 448.0


def quantize_e4m3_rows(x: torch.Tensor, rows_per_chunk: int = 4096):
    """cfg4's storage format of the indexer inputs: OCP e4m3fn with one fp32 absmax scale per row
    of the last dim (``scale = absmax / 448``, 1 for an all-zero row), ``x ~= x8 * scale``.
    Runs on ``x``'s device in chunks of rows (bounded temporaries).  Returns ``(x8, scale)``."""
    lead = x.shape[:-1]
    flat = x.reshape(-1, x.shape[-1])
    x8 = torch.empty(flat.shape, dtype=torch.float8_e4m3fn, device=x.device)
    sc = torch.empty(flat.shape[0], dtype=torch.float32, device=x.device)
    for a in range(0, flat.shape[0], rows_per_chunk):
        c = flat[a:a + rows_per_chunk].to(torch.float32)
        amax = c.abs().amax(dim=-1)
        s = torch.where(amax > 0, amax / E4M3_MAX, torch.ones_like(amax))
        x8[a:a + rows_per_chunk] = (c / s[:, None]).clamp(-E4M3_MAX, E4M3_MAX).to(torch.float8_e4m3fn)
        sc[a:a + rows_per_chunk] = s
    return x8.view(*lead, x.shape[-1]), sc.view(lead)


def make_decode(cfg: Config, device="cpu", seed: int = 0, lens: Optional[List[int]] = None,
                H: Optional[int] = None) -> Dict[str, torch.Tensor]:
    """Decode inputs: one query per sequence at position L_b - 1 over a packed latent cache."""
    lens = lens or cfg.decode_lens
    H = H or cfg.H
    B = len(lens)
    total = sum(lens)
    g = torch.Generator(device=device).manual_seed(seed)
    f32 = dict(dtype=torch.float32, device=device, generator=g)
    out = {}
    out["q"] = torch.randn(B, H, 576, **f32) * 0.1
    out["kv_cache"] = torch.randn(total, 576, **f32) * 0.1
    out["q_idx"] = torch.randn(B, cfg.Hi, cfg.Di, **f32) * 0.1
    out["k_cache"] = torch.randn(total, cfg.Di, **f32) * 0.1
    out["w"] = torch.randn(B, cfg.Hi, **f32) / 8
    offs = [0]
    for L in lens[:-1]:
        offs.append(offs[-1] + L)
    out["cache_offsets"] = torch.tensor(offs, dtype=torch.int32, device=device)
    out["cache_lens"] = torch.tensor(lens, dtype=torch.int32, device=device)
    return out
