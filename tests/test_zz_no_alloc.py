"""The allocation-free decode entry point (dsa_sparse_mla_decode_noalloc, static device scratch)
against the workspace entry point (dsa_sparse_mla_decode) through the C ABI: the same kernels and
split, so out and lse must be equal bit for bit -- on two calls in a row, the second with a
smaller input (the scratch keeps the first call's partials; the second must not read them)."""
import ctypes

import pytest
import torch

from mcore_bridge_amd import _lib, workloads as W

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _case(lens, H, K, seed):
    g = torch.Generator(device=DEV).manual_seed(seed)
    B, N = len(lens), sum(lens)
    q = (torch.randn(B, H, 576, generator=g, device=DEV) * 0.1).bfloat16()
    kv = (torch.randn(N, 576, generator=g, device=DEV) * 0.1).bfloat16()
    idx = torch.full((B, K), -1, dtype=torch.int32, device=DEV)
    off = 0
    for b, L in enumerate(lens):
        n = min(K, L)
        idx[b, :n] = (torch.randperm(L, generator=g, device=DEV)[:n] + off).sort().values.to(torch.int32)
        off += L
    return q, kv, idx


def _p(t):
    return ctypes.c_void_p(t.data_ptr())


def _both(lib, q, kv, idx):
    B, H, _ = q.shape
    N, K = kv.shape[0], idx.shape[1]
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    ws_bytes = int(lib.dsa_sparse_mla_decode_workspace_size(B, H, K))
    assert 0 < ws_bytes <= int(lib.dsa_sparse_mla_decode_scratch_bytes())
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=DEV)
    o_ref = torch.empty(B, H, 512, dtype=torch.bfloat16, device=DEV)
    l_ref = torch.empty(B, H, dtype=torch.float32, device=DEV)
    o_na = torch.full_like(o_ref, float("nan"))
    l_na = torch.full_like(l_ref, float("nan"))
    rc = lib.dsa_sparse_mla_decode(_p(q), _p(kv), _p(idx), B, N, H, 576, 512, K, W.SM_SCALE, _p(o_ref), _p(l_ref),
                                   _p(ws), ws_bytes, st)
    assert rc == 0, _lib.strerror(rc)
    rc = lib.dsa_sparse_mla_decode_noalloc(_p(q), _p(kv), _p(idx), B, N, H, 576, 512, K, W.SM_SCALE, _p(o_na),
                                           _p(l_na), st)
    assert rc == 0, _lib.strerror(rc)
    torch.cuda.synchronize()
    return o_ref, l_ref, o_na, l_na


def test_decode_noalloc_equals_workspace_entry_point():
    lib = _lib.load()
    assert int(lib.dsa_sparse_mla_decode_scratch_bytes()) == 64 << 20
    # first call: cfg5's 64 sequences (32768 partial rows, 33.7 MB of scratch); second call: a
    # smaller batch with fewer heads and a shorter top-k (more splits per sequence, 2.6 MB)
    cases = [(W.CONFIGS["cfg5"].decode_lens, 128, 2048, 1), ([3000, 700, 5000, 1200, 64], 64, 1024, 2)]
    for lens, H, K, seed in cases:
        print(f"[decode noalloc] batch={len(lens)} H={H} K={K}", flush=True)
        q, kv, idx = _case(lens, H, K, seed)
        o_ref, l_ref, o_na, l_na = _both(lib, q, kv, idx)
        assert torch.equal(o_na, o_ref), f"out differs (batch {len(lens)})"
        assert torch.equal(l_na, l_ref), f"lse differs (batch {len(lens)})"
        assert torch.isfinite(l_na).all()
