"""Benchmark of the DSA hot path on one MI355X (the driver's contract).

Workload (the one its metric is quoted on): bf16 DSA forward+backward
over T = 16384 packed tokens in 4 causal documents (cu_seqlens 0/10363/15340/15537/16384),
128 query heads over one shared 576-wide latent KV head (d_v 512, scale 1/sqrt(192)), indexer
64 heads x 128, top-k 2048.  One step = lightning-indexer scores + top-k + sparse MLA forward
+ sparse MLA backward, all in the HIP kernels of libdsa_amd.so, inputs resident in HBM.

value = algorithmic FLOPs of the step / step time:
  sparse fwd 2176*H*N_sel + sparse bwd 5504*H*N_sel + indexer 2*Di*Hi*N_pairs
(N_sel = sum_q min(K, visible keys) = 27,602,695; N_pairs = causally visible pairs).
The line also carries:
  "roofline"          the dominant kernel by time against the roofline of its algorithmic work
                      (MFMA flops, or HBM bytes for B5), with its counter traffic from the
                      committed rocprofv3 summary; "backward_traffic" the whole backward's;
  "cfg2" / "cfg4"     the prefill chain (indexer -> top-k -> forward) at configs[1] (S = 4096,
                      bf16) and configs[3] (S = 32768, fp8 indexer against the fp8 peak);
  "decode"            configs[4] (cfg5), HBM-bound: gathered bytes of the selected cache rows /
                      decode attention time, plus the decode indexer over a bf16 and over an
                      e4m3 key cache, and the graph-replayed step;
  "indexer_prologue"  the fused producer of the indexer's inputs at the cfg3 token count (HBM);
  "indexer_kl"        the sparse indexer KL loss and the indexer-score backward at cfg3;
  "indexer_kl_dense"  the dense indexer KL loss (the reference default) at cfg3: its LSE and target
                      kernels and the whole loss forward + backward;
  "mla"               the absorbed MLA path of the layer-spec swap (W_UK into q, the sparse kernels,
                      W_UV after) forward + backward at T = 16384, H = 128, top-k 2048;
  "v4"                the DeepSeek-V4 CSA layer core (sink attention fwd + bwd, 512-wide K = V) at
                      T = 16384, H = 128, window 128 + top-512 compressed entries, and the layer's
                      main compressor (pooling + norm kernels, forward and forward + backward);
  "cpu_baseline"      the oracle's reference-shaped fp32 compositions timed on the host per config
                      (cfg1 whole; cfg2/cfg3/cfg4 a few query rows, extrapolated by visible keys;
                      cfg5 every sequence) -- a reported baseline, not the target.
"""
from __future__ import annotations

import argparse
import ctypes
import json
import math
import os
import platform
import statistics
import subprocess
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for p in (ROOT, os.path.join(ROOT, "mcore-bridge_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)

METRIC = "DSA sparse-attn fwd+bwd ms & TFLOP/s at S=16k, topk=2048; % of roofline"
PEAK_BF16_TFLOPS = 2500.0
PEAK_HBM_GBS = 8000.0


def _cpu_model() -> str:
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        for line in out.splitlines():
            if line.startswith("Model name"):
                return line.split(":", 1)[1].strip()
    except Exception:
        pass
    return platform.processor() or "unknown"


TRAFFIC_PROFILE = os.path.join(ROOT, "profiles", "dsa_cfg3_hbm_traffic.md")


def measured_traffic(kernel: str):
    """HBM bytes per launch of `kernel` from the committed rocprofv3 PMC summary (FETCH_SIZE and
    WRITE_SIZE, calibrated on a copy of known size; see that file), or None if absent."""
    try:
        for line in open(TRAFFIC_PROFILE):
            cells = [c.strip() for c in line.strip().strip("|").split("|")]
            if len(cells) >= 5 and cells[0] == kernel:
                return int(cells[4].replace(",", ""))
    except OSError:
        pass
    return None


def _median_time(fn, runs: int = 3):
    """1 warm-up call, then the median wall time of `runs` calls (seconds)."""
    fn()
    ts = []
    for _ in range(runs):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    return statistics.median(ts)


def _cpu_rows_case(torch, O, W, name, cfg, L, rows, backward, fp8=False, runs=3):
    """Time the reference's dense naive path (fused_qk_topk_naive + un-fused masked attention, fp32,
    autograd backward when `backward`) for the `rows` last query rows of one causal document of L
    tokens, all heads.  The naive path computes every key of a row (masked, not skipped), so its
    work is linear in (rows x document length); returns seconds and the extrapolation unit."""
    H, Hi, Di, K = cfg.H, cfg.Hi, cfg.Di, cfg.K
    g = torch.Generator().manual_seed(0)
    a = L - rows
    q = torch.randn(rows, 1, H, 576, generator=g) * 0.1
    kv = torch.randn(L, 1, 576, generator=g) * 0.1
    sd = 1.0 if fp8 else 0.1
    qi = torch.randn(rows, 1, Hi, Di, generator=g) * sd
    ki = torch.randn(L, 1, Di, generator=g) * sd
    if fp8:   # cfg4 stores the indexer inputs as e4m3fn + scales; the naive path dequantises them
        q8, qs = W.quantize_e4m3_rows(qi)
        k8, ks = W.quantize_e4m3_rows(ki)
        qi, ki = (q8, qs), (k8, ks)
    w = torch.randn(rows, 1, Hi, generator=g) / 8
    dout = torch.randn(rows, 1, H * 512, generator=g) * 0.01
    mask = torch.triu(torch.full((rows, L), float("-inf")), diagonal=1 + a)[None]

    def run():
        qq, kk = qi, ki
        if fp8:
            qq = qi[0].float() * qi[1][..., None]
            kk = ki[0].float() * ki[1][..., None]
        _, ti = O.naive_fused_qk_topk_fp32(qq, kk, w, K, mask)
        qg = q.clone().requires_grad_(backward)
        kg = kv.clone().requires_grad_(backward)
        with torch.set_grad_enabled(backward):
            o = O.naive_unfused_sparse_attn_fp32(qg, kg, ti, W.SM_SCALE, q_offset=a)
            if backward:
                o.backward(dout)
        return o

    return _median_time(run, runs), rows * L


def cpu_baseline(torch, dev):
    """The reference's algorithm class on the host cores, per configuration (the oracle's fp32
    restatements of fused_qk_topk_naive and the un-fused masked attention; autograd backward):
      cfg1: the whole fwd+bwd (S=512);
      cfg2 / cfg3 / cfg4: a block of the last query rows of the longest document, all heads,
        timed and extrapolated linearly in (query rows x document length) -- the naive path
        computes every key of every row, masked or not -- to the config's documents;
      cfg5: every sequence's dense index scan + top-k + attention over the selected rows.
    1 warm-up, median of 3.  value = the config's algorithmic FLOPs (the same counts as the GPU
    numbers) / measured or extrapolated time.  The headline object is cfg3's."""
    from oracle import dsa_oracle as O
    from mcore_bridge_amd import workloads as W
    threads = torch.get_num_threads()
    per = {}

    def flops(cu, K, H, Hi, Di, backward):
        return ((7680 if backward else 2176) * H * W.n_sel(cu, K) + 2 * Di * Hi * W.n_pairs(cu))

    # cfg1: whole problem
    c1 = W.CONFIGS["cfg1"]
    t, _ = _cpu_rows_case(torch, O, W, "cfg1", c1, c1.S, c1.S, True)
    f = flops([0, c1.S], c1.K, c1.H, c1.Hi, c1.Di, True)
    per["cfg1"] = {"value": round(f / t / 1e12, 6), "unit": "TFLOP/s", "ms": round(t * 1e3, 2),
                   "sample": "whole fwd+bwd, S=512, H=16, Hi=4, Di=64, top-k 128"}
    for name, rows, backward, fp8 in (("cfg2", 64, False, False), ("cfg3", 32, True, False), ("cfg4", 16, False, True)):
        c = W.CONFIGS[name]
        cu = c.docs
        lens = [b - a for a, b in zip(cu[:-1], cu[1:])]
        L = max(lens)
        t, unit = _cpu_rows_case(torch, O, W, name, c, L, rows, backward, fp8)
        full_units = sum(x * x for x in lens)
        t_full = t * full_units / unit
        f = flops(cu, c.K, c.H, c.Hi, c.Di, backward)
        per[name] = {"value": round(f / t_full / 1e12, 6), "unit": "TFLOP/s",
                     "ms_extrapolated": round(t_full * 1e3, 1), "ms_sample": round(t * 1e3, 1),
                     "sample": (f"last {rows} query rows of a causal document of {L} tokens, H={c.H}, Hi={c.Hi}, "
                                f"top-k {c.K}, {'fwd+bwd' if backward else 'fwd'}"
                                f"{', indexer inputs e4m3fn dequantised' if fp8 else ''}; extrapolated x"
                                f"{full_units / unit:.1f} (sum of document length^2 / (rows x {L}))")}
    # cfg5: all 64 sequences (bf16 inputs drawn on the device, copied to the host, converted to
    # fp32 per sequence inside the timed region)
    c5 = W.CONFIGS["cfg5"]
    lens = c5.decode_lens
    g = torch.Generator(device=dev).manual_seed(0)
    N = sum(lens)
    kv = torch.empty(N, 576, dtype=torch.bfloat16)
    for a0 in range(0, N, 1 << 20):
        n = min(N - a0, 1 << 20)
        kv[a0:a0 + n] = (torch.randn(n, 576, generator=g, device=dev) * 0.1).bfloat16().cpu()
    kc = (torch.randn(N, c5.Di, generator=g, device=dev) * 0.1).bfloat16().cpu()
    q = (torch.randn(len(lens), c5.H, 576, generator=g, device=dev) * 0.1).bfloat16().cpu()
    qi = (torch.randn(len(lens), c5.Hi, c5.Di, generator=g, device=dev) * 0.1).bfloat16().cpu()
    w = (torch.randn(len(lens), c5.Hi, generator=g, device=dev) / 8).cpu()
    t = _median_time(lambda: O.naive_decode_fp32(q, kv, qi, kc, w, lens, c5.K, W.SM_SCALE))
    sel = sum(min(c5.K, L) for L in lens)
    f = 2176 * c5.H * sel + 2 * c5.Di * c5.Hi * N
    gather = sel * 576 * 2 + q.numel() * 2 + len(lens) * c5.H * 512 * 2 + len(lens) * c5.K * 4
    per["cfg5"] = {"value": round(f / t / 1e12, 6), "unit": "TFLOP/s", "ms": round(t * 1e3, 2),
                   "gather_GBs": round(gather / t / 1e9, 2),
                   "sample": "all 64 sequences: dense index scan of the whole cache, top-k 2048, attention over "
                             "the selected rows (128 heads)"}
    del kv, kc
    c3 = per["cfg3"]
    return {
        "value": c3["value"], "unit": "TFLOP/s", "cores": threads, "kind": "port",
        "sample": (f"cfg3 ({c3['sample']}); fp32 oracle restatements of the reference's naive path; "
                   f"cpu {_cpu_model()}, os.cpu_count()={os.cpu_count()}, torch threads {threads}"),
        "per_config": per,
    }


def decode_leg(torch, dev, reps: int = 50):
    """cfg5 decode through the C ABI with preallocated buffers:
    64 sequences, one new token each at position L_b - 1, cache lengths of the committed
    fixture (sum 2,724,446 rows of 576 bf16), indexer 64 x 128 bf16, top-k 2048, 128 heads.
    The attention is HBM-bound: gather bytes = sum_b min(K, L_b)*576*2 + q + O + idx."""
    from mcore_bridge_amd import _lib, ops, workloads as W
    cfg = W.CONFIGS["cfg5"]
    lens = cfg.decode_lens
    B, H, K = len(lens), cfg.H, cfg.K
    N = sum(lens)
    g = torch.Generator(device=dev).manual_seed(0)
    q = (torch.randn(B, H, 576, generator=g, device=dev) * 0.1).bfloat16()
    kv = torch.empty(N, 576, dtype=torch.bfloat16, device=dev)
    for a in range(0, N, 1 << 20):   # fill in slices (bounded fp32 temporaries)
        n = min(N - a, 1 << 20)
        kv[a:a + n] = (torch.randn(n, 576, generator=g, device=dev) * 0.1).bfloat16()
    qi = (torch.randn(B, cfg.Hi, cfg.Di, generator=g, device=dev) * 0.1).bfloat16()
    ki = (torch.randn(N, cfg.Di, generator=g, device=dev) * 0.1).bfloat16()
    w = torch.randn(B, cfg.Hi, generator=g, device=dev) / 8
    cu = torch.tensor([0] + [sum(lens[:i + 1]) for i in range(B)], dtype=torch.int32, device=dev)
    Lmax = max(lens)

    def timed(fn):
        for _ in range(3):
            fn()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            fn()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / reps * 1e3   # us per call

    idx = ops.decode_indexer_topk(qi, ki, w, K, cu, Lmax)
    t_sel = timed(lambda: ops.decode_indexer_topk(qi, ki, w, K, cu, Lmax))
    # the same scan over an e4m3fn key cache with one fp32 scale per row (and e4m3 q rows with
    # per-(token, head) scales): 132 instead of 256 bytes per cached key
    qi8, qis = W.quantize_e4m3_rows(qi.float())
    ki8, kis = W.quantize_e4m3_rows(ki)
    t_sel8 = timed(lambda: ops.decode_indexer_topk(qi8, ki8, w, K, cu, Lmax, qis, kis))
    del qi8, ki8
    out = torch.empty(B, H, 512, dtype=torch.bfloat16, device=dev)
    lse = torch.empty(B, H, dtype=torch.float32, device=dev)
    ws_bytes = ops.decode_workspace_bytes(B, H, K)
    ws = torch.empty(max(ws_bytes, 16), dtype=torch.uint8, device=dev)
    stream = torch.cuda.current_stream(dev).cuda_stream
    lib = _lib.load()
    args = (q.data_ptr(), kv.data_ptr(), idx.data_ptr(), B, N, H, 576, 512, K, W.SM_SCALE, out.data_ptr(),
            lse.data_ptr(), ws.data_ptr(), ws_bytes, stream)
    _lib.check("dsa_sparse_mla_decode", lib.dsa_sparse_mla_decode(*args))
    t_attn = timed(lambda: lib.dsa_sparse_mla_decode(*args))
    # the whole decode step (rows, indexer scores, top-k, split attention, merge) replayed from a
    # HIP graph: the serving path, launch gaps removed
    def decode_step():
        ix = ops.decode_indexer_topk(qi, ki, w, K, cu, Lmax)
        return ops.sparse_mla_decode(q, kv, ix, W.SM_SCALE)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        decode_step()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        decode_step()
    t_step_graph = timed(graph.replay)
    del graph
    gather = sum(min(K, L) for L in lens) * 576 * 2 + q.numel() * 2 + out.numel() * 2 + idx.numel() * 4
    scan = N * cfg.Di * 2
    gbs = gather / (t_attn * 1e-6) / 1e9
    return {
        "workload": "cfg5: decode, 64 sequences x 1 token, cache lengths fixture (sum 2,724,446 rows), H=128, "
                    "d_qk=576, d_v=512, indexer 64x128 bf16, top-k 2048",
        "attention_us": round(t_attn, 2), "gather_bytes": gather, "gather_GBs": round(gbs, 1),
        "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                     "frac": round(gbs / PEAK_HBM_GBS, 4)},
        "attention_tflops": round(2176 * H * sum(min(K, L) for L in lens) / (t_attn * 1e-6) / 1e12, 1),
        "indexer_topk_us": round(t_sel, 2), "indexer_scan_bytes": scan,
        "indexer_scan_GBs": round(scan / (t_sel * 1e-6) / 1e9, 1),
        "indexer_topk_fp8_us": round(t_sel8, 2), "indexer_scan_fp8_bytes": N * (cfg.Di + 4),
        "indexer_scan_fp8_GBs": round(N * (cfg.Di + 4) / (t_sel8 * 1e-6) / 1e9, 1),
        "n_split": ws_bytes // (B * H * (512 * 2 + 4)) if ws_bytes else 1,
        "decode_step_us_hip_graph": round(t_step_graph, 2),
    }


def prologue_leg(torch, dev, reps: int = 50):
    """Indexer prologue (the producer of the indexer's q, k, w; reference forward_before_topk,
    patcher.py:268-300) at the cfg3 token count: T = 16384, Hi = 64, Di = 128, through the C ABI
    with preallocated buffers, bf16 and fp8 outputs.  One pass over the projected rows, HBM-bound:
    algorithmic bytes = q_lin + k_lin + w_lin + freqs read once + q, k (+ scales) + w written."""
    from mcore_bridge_amd import _lib
    T, Hi = 16384, 64
    g = torch.Generator(device=dev).manual_seed(5)
    q_lin = (torch.randn(T, Hi * 128, generator=g, device=dev) * 2).bfloat16()
    k_lin = (torch.randn(T, 128, generator=g, device=dev) * 2).bfloat16()
    w_lin = torch.randn(T, Hi, generator=g, device=dev).bfloat16()
    lw = torch.ones(128, device=dev)
    lb = torch.zeros(128, device=dev)
    inv = 1.0 / (10000 ** (torch.arange(0, 64, 2, dtype=torch.float32, device=dev) / 64))
    ang = torch.arange(T, dtype=torch.float32, device=dev)[:, None] * inv
    fr = torch.cat([ang, ang], -1).contiguous()
    lib = _lib.load()
    stream = torch.cuda.current_stream(dev).cuda_stream
    res = {"workload": "indexer prologue at cfg3 size: T=16384 tokens, Hi=64, Di=128, rope 64 (LayerNorm + "
                       "partial RoPE + 128-point Hadamard + head weights, one fused pass; projections excluded)"}
    for fp8 in (False, True):
        odt = torch.float8_e4m3fn if fp8 else torch.bfloat16
        q = torch.empty(T, Hi, 128, dtype=odt, device=dev)
        k = torch.empty(T, 128, dtype=odt, device=dev)
        w = torch.empty(T, Hi, dtype=torch.float32, device=dev)
        qs = torch.empty(T, Hi, dtype=torch.float32, device=dev)
        ks = torch.empty(T, dtype=torch.float32, device=dev)
        args = (q_lin.data_ptr(), Hi * 128, k_lin.data_ptr(), 128, w_lin.data_ptr(), Hi, lw.data_ptr(), lb.data_ptr(),
                fr.data_ptr(), 64, T, Hi, 128, 64, 1e-6, 1.0, Hi ** -0.5, 128 ** -0.5, 0, 0,
                _lib.DSA_FP8_E4M3 if fp8 else _lib.DSA_BF16, q.data_ptr(), qs.data_ptr(), k.data_ptr(),
                ks.data_ptr(), w.data_ptr(), stream)
        for _ in range(3):
            _lib.check("dsa_indexer_prologue", lib.dsa_indexer_prologue(*args))
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            lib.dsa_indexer_prologue(*args)
        e1.record()
        torch.cuda.synchronize()
        us = e0.elapsed_time(e1) / reps * 1e3
        ob = 1 if fp8 else 2
        nbytes = (T * Hi * 128 * 2 + T * 128 * 2 + T * Hi * 2 + T * 64 * 4
                  + T * Hi * 128 * ob + T * 128 * ob + T * Hi * 4 + (T * Hi * 4 + T * 4 if fp8 else 0))
        gbs = nbytes / (us * 1e-6) / 1e9
        res["fp8" if fp8 else "bf16"] = {"us": round(us, 2), "bytes": nbytes, "GBs": round(gbs, 1),
                                         "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": PEAK_HBM_GBS,
                                                      "unit": "GB/s", "frac": round(gbs / PEAK_HBM_GBS, 4)}}
    return res


def indexer_kl_leg(torch, dev, q, kv, idx, lse, qi, ki, w, scale: float, nsel: int, bwd_ws, reps: int = 10):
    """Sparse indexer KL loss at the cfg3 size (dsa_indexer_loss_coeff with the sparse loss,
    model_config.py:204-205): the attention target from the forward LSE, the selected-slot indexer
    scores, the per-row KL + gradient, and the indexer-score backward (pair order, per-query
    dq / dw / dk rows, key reduction), each through the C ABI with preallocated buffers.
    Algorithmic work per selected pair: target 2*576*H flops (S recompute); scores 2*128*Hi;
    backward 4 x 2*128*Hi (Z, Z^T, dq, dk rows) + its 256-byte dk row written and read back."""
    from mcore_bridge_amd import _lib
    lib = _lib.load()
    stream = torch.cuda.current_stream(dev).cuda_stream
    T, H, _ = q.shape
    N, K = kv.shape[0], idx.shape[1]
    Hi = qi.shape[1]
    tgt = torch.empty(T, K, dtype=torch.float32, device=dev)
    sel = torch.empty(T, K, dtype=torch.float32, device=dev)
    kl = torch.empty(T, dtype=torch.float32, device=dev)
    d = torch.empty(T, K, dtype=torch.float32, device=dev)
    dq = torch.empty(T, Hi, 128, dtype=torch.float32, device=dev)
    dw = torch.empty(T, Hi, dtype=torch.float32, device=dev)
    dk = torch.empty(N, 128, dtype=torch.float32, device=dev)
    ws_bytes = int(lib.dsa_indexer_scores_bwd_workspace_size(T, N, K))
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
    calls = {
        "target": lambda: lib.dsa_indexer_kl_target(q.data_ptr(), kv.data_ptr(), idx.data_ptr(), lse.data_ptr(), T, N,
                                                    H, 576, K, scale, 1, tgt.data_ptr(), stream),
        "selected_scores": lambda: lib.dsa_indexer_selected_scores(qi.data_ptr(), ki.data_ptr(), w.data_ptr(),
                                                                   idx.data_ptr(), T, N, Hi, 128, K, 1,
                                                                   sel.data_ptr(), stream),
        "kl_rows": lambda: lib.dsa_indexer_kl_loss(sel.data_ptr(), tgt.data_ptr(), idx.data_ptr(), T, N, K, 1,
                                                   1.0 / T, kl.data_ptr(), d.data_ptr(), stream),
        "scores_bwd": lambda: lib.dsa_indexer_scores_bwd(qi.data_ptr(), ki.data_ptr(), w.data_ptr(), idx.data_ptr(),
                                                         d.data_ptr(), T, N, Hi, 128, K, 1, dq.data_ptr(),
                                                         dw.data_ptr(), dk.data_ptr(), ws.data_ptr(), ws_bytes,
                                                         stream),
        # the target from the P tiles the attention backward already staged (its workspace, filled by
        # the last timed step on the same indices): the variant that applies the loss in the backward
        "target_from_bwd": lambda: lib.dsa_indexer_kl_target_from_bwd(bwd_ws.data_ptr(), bwd_ws.numel(),
                                                                      idx.data_ptr(), T, N, H, K, 1, tgt.data_ptr(),
                                                                      stream),
    }
    res = {"workload": f"sparse indexer KL loss at cfg3 size: T={T}, H={H}, Hi={Hi}, top-k {K}, "
                       f"{nsel} selected pairs"}
    for name, fn in calls.items():
        for _ in range(2):
            _lib.check("dsa_" + name, fn())
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            fn()
        e1.record()
        torch.cuda.synchronize()
        res[name + "_ms"] = round(e0.elapsed_time(e1) / reps, 4)
    fl_t = 2 * 576 * H * nsel
    fl_b = 4 * 2 * 128 * Hi * nsel
    res["target_tflops"] = round(fl_t / (res["target_ms"] * 1e-3) / 1e12, 1)
    res["scores_bwd_tflops"] = round(fl_b / (res["scores_bwd_ms"] * 1e-3) / 1e12, 1)
    rest = ("selected_scores", "kl_rows", "scores_bwd")
    res["total_ms"] = round(res["target_ms"] + sum(res[n + "_ms"] for n in rest), 3)
    res["total_in_attention_bwd_ms"] = round(res["target_from_bwd_ms"] + sum(res[n + "_ms"] for n in rest), 3)
    res["loss"] = round(float(kl.sum().item()) / T, 6)
    return res


def _time_ms(torch, fn, reps: int, warm: int = 2, windows: int = 3):
    """ms per fn() call: the median over `windows` timed windows of the average of `reps` calls,
    HIP events on torch's current stream (every op here launches on it).  One slow window (seen
    once: a 5-call window at 1.5x the others) then does not set the figure."""
    for _ in range(warm):
        fn()
    per = []
    for _ in range(windows):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            fn()
        e1.record()
        torch.cuda.synchronize()
        per.append(e0.elapsed_time(e1) / reps)
    return sorted(per)[len(per) // 2]


PEAK_FP8_TFLOPS = 5000.0


def indexer_kl_dense_leg(torch, dev, q, kv, qi, ki, w, cu_t, max_seqlen: int, scale: float, npairs: int,
                         reps: int = 5):
    """Dense indexer KL loss at the cfg3 size (the reference default: dsa_indexer_loss_coeff with
    dsa_indexer_use_sparse_loss = False, model_config.py:204-205; the target is the head-summed
    dense attention of each query over EVERY visible key): the dense LSE and target kernels alone,
    then the whole loss forward + backward through autograd (LSE, target, dense index scores, KL
    rows, score backward).  LSE and target each cost 2*576*H flops per visible pair (QK only)."""
    from mcore_bridge_amd import ops, dsa
    T, H, _ = q.shape
    base, ln = ops.build_rows(cu_t, T, True)
    pitch = max(4, (max_seqlen + 3) // 4 * 4)
    lse = ops.dense_attention_lse(q, kv, base, ln, max_seqlen, scale)
    t_lse = _time_ms(torch, lambda: ops.dense_attention_lse(q, kv, base, ln, max_seqlen, scale), reps)
    t_tgt = _time_ms(torch, lambda: ops.dense_attention_target(q, kv, lse, base, ln, max_seqlen, pitch, scale), reps)
    qd, kd, wd = (x.detach().requires_grad_() for x in (qi, ki, w))
    loss_val = [0.0]

    def loss_step():
        loss = dsa.indexer_kl_loss_dense(q, kv, qd, kd, wd, scale, 1.0, cu_t, max_seqlen)
        loss.backward()
        loss_val[0] = loss

    t_all = _time_ms(torch, loss_step, reps)
    fl = 2 * 576 * H * npairs
    tf_lse = fl / (t_lse * 1e-3) / 1e12
    return {"workload": f"dense indexer KL loss at cfg3 size: T={T} in 4 causal documents, H={H}, Hi={qi.shape[1]}, "
                        f"{npairs} visible (query, key) pairs",
            "lse_ms": round(t_lse, 3), "target_ms": round(t_tgt, 3), "loss_fwd_bwd_ms": round(t_all, 3),
            "lse_tflops": round(tf_lse, 1), "target_tflops": round(fl / (t_tgt * 1e-3) / 1e12, 1),
            "loss": round(float(loss_val[0].detach().item()), 6),
            "roofline": {"bound": "mfma", "kernel": "dense_lse_kernel", "achieved": round(tf_lse, 1),
                         "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s", "frac": round(tf_lse / PEAK_BF16_TFLOPS, 4)}}


def v4_leg(torch, dev, reps: int = 5):
    """DeepSeek-V4 compressed sparse attention layer core (reference deepseek_v4.py:61-328; the core
    attention of its CSA layers) on the DSA kernels: one document of T = 16384 tokens, H = 128 heads
    over ONE shared 512-wide K = V head, a 128-token sliding window plus the CSA indexer's top-512
    of the rate-4 compressed entries (index row width 640), per-head attention sink; forward +
    backward of v4.sink_attention.  Algorithmic work with the 512-wide keys: forward 2 (512 + 512)
    H per attended (query, key) pair, backward 2 (3 x 512 + 2 x 512) H.  The kernels read the
    512-wide q rows as they are (their instantiations without the rope part: 512-deep scores,
    1024-byte G rows), take the K = V rows in the 576-wide row layout (rope region zero)
    and fold the sink in (the forward's epilogue, Delta from B1, one d sink kernel), so
    `kernels_ms` (the sink entry points on pre-padded key rows) is what the kernels take and
    `host_composition_ms` the rest: the key rows' pad copy, the dkv slice, autograd.
    `csa_compressor_*_ms`: the CSA main compressor (rate 4, overlapping windows, 2 x 512-channel
    kv / gate rows of the T tokens) through v4.compress, host calls and autograd included.
    `csa_layer_fwd_bwd_ms`: the whole DSv4HybridAttention CSA layer (hidden 4096, q_lora_rank
    1024, 8 output groups of rank 1024, random weights) forward + backward, library GEMMs included."""
    from mcore_bridge_amd import ops, v4
    T, H, D, Wn, rate, Kc, Hi, Di = 16384, 128, 512, 128, 4, 512, 64, 128
    cu = [0, T]
    g = torch.Generator(device=dev).manual_seed(44)
    q = (torch.randn(T, H, D, generator=g, device=dev) * 0.05).bfloat16()
    Nc = T // rate
    keys = (torch.randn(T + Nc, D, generator=g, device=dev)).bfloat16()
    sinks = torch.randn(H, generator=g, device=dev)
    qi = (torch.randn(T, Hi, Di, generator=g, device=dev) * 0.1).bfloat16()
    ck = (torch.randn(Nc, Di, generator=g, device=dev) * 0.1).bfloat16()
    wi = torch.randn(T, Hi, generator=g, device=dev) / 8
    sel = v4.indexer_select(qi, ck, wi, cu, rate, Kc, Di)
    idx = v4.hybrid_indices(cu, Wn, 0, sel, dev)
    nsel = int((idx >= 0).sum().item())
    dout = (torch.randn(T, H, D, generator=g, device=dev) * 0.01).bfloat16()
    scale = D ** -0.5
    t_sel = _time_ms(torch, lambda: v4.indexer_select(qi, ck, wi, cu, rate, Kc, Di), reps)

    def layer_core():
        qd, kd, sd = q.detach().requires_grad_(), keys.detach().requires_grad_(), sinks.detach().requires_grad_()
        out, _ = v4.sink_attention(qd, kd, sd, idx, scale)
        out.backward(dout)

    kp = torch.nn.functional.pad(keys, (0, ops.D_QK - D)).contiguous()

    def kernels_only():
        out, lse = ops.sparse_mla_fwd_sink(q, kp, idx, sinks, scale, False)
        ops.sparse_mla_bwd_sink(q, kp, idx, out, dout, lse, sinks, scale, False)

    t_all = _time_ms(torch, layer_core, reps)
    t_k = _time_ms(torch, kernels_only, reps)
    # the CSA layer's main compressor (kv / gate projections of the T tokens, rate 4, overlapping
    # windows of 2 x 512 channels) through v4.compress on the HIP kernels, host calls included
    C = 2 * D
    ckv = torch.randn(T, C, generator=g, device=dev).bfloat16()
    cgt = (torch.randn(T, C, generator=g, device=dev) * 2).bfloat16()
    cape = (torch.randn(rate, C, generator=g, device=dev) * 0.5).bfloat16()
    cnw = torch.ones(D, device=dev, dtype=torch.bfloat16)
    cdo = (torch.randn(T // rate, D, generator=g, device=dev) * 0.1).bfloat16()

    def comp_fwd_bwd():
        leaves = [t.detach().requires_grad_() for t in (ckv, cgt, cape, cnw)]
        v4.compress(*leaves, cu, rate, 1e-6, True).backward(cdo)

    with torch.no_grad():
        t_cf = _time_ms(torch, lambda: v4.compress(ckv, cgt, cape, cnw, cu, rate, 1e-6, True), reps)
    t_cfb = _time_ms(torch, comp_fwd_bwd, reps)
    # the whole CSA layer mirror (hidden 4096, q_lora_rank 1024, 8 output groups of rank 1024,
    # random weights): projections, norms and RoPE, both compressors, the indexer's top-k, the
    # sink attention and the grouped output projection, forward + backward
    layer = v4.DSv4HybridAttention("compressed_sparse_attention", 4096, H, 1024, o_groups=8, o_lora_rank=1024,
                                   window=Wn, compress_rates=(rate, 128), index_n_heads=Hi, index_head_dim=Di,
                                   index_topk=Kc, device=dev)
    with torch.no_grad():
        for prm in layer.parameters():
            if prm.dim() >= 2:
                prm.normal_(0, 0.02, generator=g)
    lx = torch.randn(T, 1, 4096, generator=g, device=dev).bfloat16()
    ldo = (torch.randn(T, 1, 4096, generator=g, device=dev) * 0.01).bfloat16()
    inv_f = 1.0 / (10000 ** (torch.arange(0, 64, 2, device=dev).float() / 64))
    tab = torch.outer(torch.arange(T, device=dev).float(), inv_f).repeat(1, 2).view(T, 1, 1, 64)

    def layer_fwd_bwd():
        xx = lx.detach().requires_grad_()
        out, _ = layer(xx, None, rotary_pos_emb={"main": tab, "compress": tab})
        out.backward(ldo)

    t_layer = _time_ms(torch, layer_fwd_bwd, 3)
    del layer
    fl = (2 * (D + D) + 2 * (3 * D + 2 * D)) * H * nsel
    tf = fl / (t_all * 1e-3) / 1e12
    tfk = fl / (t_k * 1e-3) / 1e12
    return {"workload": "DeepSeek-V4 CSA layer core: T=16384 (one document), H=128, one shared 512-wide K=V head, "
                        "window 128 + top-512 of rate-4 compressed entries (indexer 64x128), attention sink; "
                        "sink_attention fwd+bwd",
            "n_sel": nsel, "flops": fl, "ms": round(t_all, 3), "tflops": round(tf, 1),
            "kernels_ms": round(t_k, 3), "kernels_tflops": round(tfk, 1),
            "host_composition_ms": round(t_all - t_k, 3), "csa_indexer_ms": round(t_sel, 3),
            "csa_compressor_fwd_ms": round(t_cf, 3), "csa_compressor_fwd_bwd_ms": round(t_cfb, 3),
            "csa_layer_fwd_bwd_ms": round(t_layer, 3),
            "roofline": {"bound": "mfma", "achieved": round(tf, 1), "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                         "frac": round(tf / PEAK_BF16_TFLOPS, 4)}}


def mla_leg(torch, dev, qi, ki, w, reps: int = 3):
    """The absorbed MLA path of the layer-spec swap (absorbed_mla_sparse_attention, the core of
    reference multi_latent_attention.py:262-270 on MLASelfAttention's un-absorbed tensors) at one
    causal document of T = 16384 tokens: H = 128, qk_nope = v_head = 128, kv_lora_rank 512, rope
    64, top-k 2048 from the bench's indexer inputs over that document.  `ms` is the autograd path
    forward + backward (W_UK folded into q, the sparse kernels, W_UV after, every gradient incl. the
    up-projection weight's); `attention_ms` the same sparse forward + backward on the prepared
    query / kv alone, so `ms - attention_ms` is what the absorption costs.  Algorithmic work: the
    sparse attention's 7680*H per selected pair plus the absorption products, 2*T*H*(dn*512 +
    512*dv) forward and twice that backward."""
    from mcore_bridge_amd import dsa, ops
    T, H, dn, dv, K = qi.shape[0], 128, 128, 128, 2048
    g = torch.Generator(device=dev).manual_seed(55)
    q_no_pe = (torch.randn(T, 1, H, dn, generator=g, device=dev) * 0.1).bfloat16()
    q_pe = (torch.randn(T, 1, H, 64, generator=g, device=dev) * 0.1).bfloat16()
    kvc = (torch.randn(T, 1, 512, generator=g, device=dev) * 0.1).bfloat16()
    kpe = (torch.randn(T, 1, 64, generator=g, device=dev) * 0.1).bfloat16()
    wkv = (torch.randn(H * (dn + dv), 512, generator=g, device=dev) * 0.02).bfloat16()
    dout = (torch.randn(T, 1, H * dv, generator=g, device=dev) * 0.01).bfloat16()
    cu1 = torch.tensor([0, T], dtype=torch.int32, device=dev)
    idx = ops.indexer_topk(qi, ki, w, K, cu1, True, T).view(1, T, K)
    nsel = int((idx >= 0).sum().item())
    scale = 192 ** -0.5

    def absorbed():
        ls = [x.detach().requires_grad_() for x in (q_no_pe, q_pe, kvc, kpe, wkv)]
        dsa.absorbed_mla_sparse_attention(*ls, idx, scale).backward(dout)

    with torch.no_grad():
        q_lat = torch.bmm(q_no_pe[:, 0].permute(1, 0, 2).float().contiguous(),
                          wkv.view(H, dn + dv, 512)[:, :dn].float().contiguous())        # [H, T, 512]
        qq = torch.cat([q_lat.permute(1, 0, 2).unsqueeze(1).bfloat16(), q_pe], -1).contiguous()
        kk = torch.cat([kvc, kpe], -1).contiguous()
    do_lat = (torch.randn(T, 1, H * 512, generator=g, device=dev) * 0.01).bfloat16()

    def attention_only():
        a, b = qq.detach().requires_grad_(), kk.detach().requires_grad_()
        dsa.sparse_mla_attention(a, b, idx, scale).backward(do_lat)

    t_all = _time_ms(torch, absorbed, reps)
    t_att = _time_ms(torch, attention_only, reps)
    fl = 7680 * H * nsel + 3 * 2 * T * H * (dn * 512 + 512 * dv)
    return {"workload": "absorbed MLA (layer-spec swap) core: T=16384 one causal document, H=128, qk_nope=v=128, "
                        "kv_lora 512 + rope 64, top-k 2048; forward + backward incl. W_UK / W_UV and their gradients",
            "n_sel": nsel, "ms": round(t_all, 3), "attention_ms": round(t_att, 3),
            "absorption_ms": round(t_all - t_att, 3), "tflops": round(fl / (t_all * 1e-3) / 1e12, 1),
            "roofline": {"bound": "mfma", "achieved": round(fl / (t_all * 1e-3) / 1e12, 1), "peak": PEAK_BF16_TFLOPS,
                         "unit": "TFLOP/s", "frac": round(fl / (t_all * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 4)}}


def prefill_fwd_leg(torch, dev, name: str, reps: int = 10):
    """cfg2 (bf16 indexer) or cfg4 (fp8 e4m3fn indexer with absmax row scales, S = 32768): one
    causal document, indexer scores, top-k 2048 and the bf16 sparse MLA forward (H = 128), each
    timed on its own with preallocated inputs.  Indexer: 2*Di*Hi flops per visible pair on bf16 /
    fp8 MFMA; top-k: the fp32 score rows it reads (N_pairs * 4 bytes); forward: 2176*H flops per
    selected pair on bf16 MFMA."""
    from mcore_bridge_amd import ops, workloads as W
    cfg = W.CONFIGS[name]
    S, H, K = cfg.S, cfg.H, cfg.K
    x = W.make_prefill(cfg, device=dev, seed=0)
    q, kv, w = x["q"].bfloat16(), x["kv"].bfloat16(), x["w"]
    if cfg.fp8_indexer:
        qi, qs = W.quantize_e4m3_rows(x.pop("q_idx"))
        ki, ks = W.quantize_e4m3_rows(x.pop("k_idx"))
    else:
        qi, ki = x.pop("q_idx").bfloat16(), x.pop("k_idx").bfloat16()
        qs = ks = None
    del x
    cu = torch.tensor([0, S], dtype=torch.int32, device=dev)
    base, ln = ops.build_rows(cu, S, True)
    sc = ops.indexer_scores(qi, ki, w, base, ln, S, S, qs, ks, False)
    idx = ops.topk(sc, base, ln, K)
    t_sc = _time_ms(torch, lambda: ops.indexer_scores(qi, ki, w, base, ln, S, S, qs, ks, False), reps)
    t_tk = _time_ms(torch, lambda: ops.topk(sc, base, ln, K), reps)
    t_fw = _time_ms(torch, lambda: ops.sparse_mla_fwd(q, kv, idx, W.SM_SCALE, True), reps)
    npairs, nsel = W.n_pairs([0, S]), W.n_sel([0, S], K)
    fl_i = 2 * cfg.Di * cfg.Hi * npairs
    fl_f = 2176 * H * nsel
    peak_i = PEAK_FP8_TFLOPS if cfg.fp8_indexer else PEAK_BF16_TFLOPS
    ti = fl_i / (t_sc * 1e-3) / 1e12
    tf = fl_f / (t_fw * 1e-3) / 1e12
    res = {
        "workload": (f"{name}: one causal document S={S}, H={H}, d_qk=576, d_v=512, indexer {cfg.Hi}x{cfg.Di} "
                     f"{'fp8 e4m3fn (absmax row scales)' if cfg.fp8_indexer else 'bf16'}, top-k {K}"),
        "indexer_ms": round(t_sc, 4), "indexer_tflops": round(ti, 1),
        "indexer_roofline": {"bound": "mfma", "dtype": "fp8" if cfg.fp8_indexer else "bf16", "achieved": round(ti, 1),
                             "peak": peak_i, "unit": "TFLOP/s", "frac": round(ti / peak_i, 4),
                             "algorithmic": fl_i},
        "topk_ms": round(t_tk, 4), "topk_score_bytes": npairs * 4,
        "topk_GBs": round(npairs * 4 / (t_tk * 1e-3) / 1e9, 1),
        "sparse_fwd_ms": round(t_fw, 4), "sparse_fwd_tflops": round(tf, 1),
        "sparse_fwd_roofline": {"bound": "mfma", "dtype": "bf16", "achieved": round(tf, 1), "peak": PEAK_BF16_TFLOPS,
                                "unit": "TFLOP/s", "frac": round(tf / PEAK_BF16_TFLOPS, 4), "algorithmic": fl_f},
        "chain_ms": round(t_sc + t_tk + t_fw, 4),
    }
    del q, kv, qi, ki, sc, idx
    torch.cuda.empty_cache()
    return res


def int8_staging_leg(torch, lib, _lib, q, kv, qi, ki, w, dout, cu_t, max_seqlen, scale, dkv_bf16, ws, stream,
                     fl_fwd, fl_bwd, t_fwd, t_bwd, reps: int = 5):
    """The same cfg3 backward with the per-pair dKV rows staged as int8 with a bf16 scale per 32 dims
    (DSA_BWD_G_INT8, opt-in): per-stage times and the dkv difference from the default bf16 rows
    (dkv_bf16 of the timed steps; dq does not depend on the format).  Not the headline: the
    headline backward is the default bf16 staging."""
    from mcore_bridge_amd import ops
    T, H, _ = q.shape
    N, K = kv.shape[0], 2048
    idx = ops.indexer_topk(qi, ki, w, K, cu_t, True, max_seqlen)
    out, lse = ops.sparse_mla_fwd(q, kv, idx, scale, True)
    need = ops.bwd_workspace_bytes(T, N, H, K, g_int8=True)
    assert need <= ws.numel()
    dq = torch.empty_like(q)
    dkv = torch.empty_like(dkv_bf16)
    stages = ("bwd_pairs", "bwd_sp", "bwd_dq", "bwd_g", "bwd_dkv_reduce")
    times = {k: [] for k in stages}
    for r in range(reps + 1):
        se = [torch.cuda.Event(enable_timing=True) for _ in range(6)]
        for e in se:
            e.record()
        arr = (ctypes.c_void_p * 6)(*[e.cuda_event for e in se])
        _lib.check("dsa_sparse_mla_bwd_ex", lib.dsa_sparse_mla_bwd_ex(
            q.data_ptr(), kv.data_ptr(), idx.data_ptr(), out.data_ptr(), dout.data_ptr(), lse.data_ptr(), T, N, H,
            576, 512, K, scale, 1, dq.data_ptr(), dkv.data_ptr(), ops.DSA_BWD_G_INT8,
            ws.data_ptr(), need, arr, stream))
        torch.cuda.synchronize()
        if r:
            for i, k in enumerate(stages):
                times[k].append(se[i].elapsed_time(se[i + 1]))
    t = {k: statistics.mean(v) for k, v in times.items()}
    t_b = sum(t.values())
    diff = float((dkv - dkv_bf16).norm() / dkv_bf16.norm())
    return {
        "note": "opt-in DSA_BWD_G_INT8 (per-pair dKV rows as int8 + bf16 scale per 32 dims, 640 B/row "
                "instead of 1152); the headline uses the default bf16 rows",
        "ms": round(t_b, 3),
        "breakdown_ms": {k: round(v, 3) for k, v in t.items()},
        "sparse_bwd_tflops": round(fl_bwd / t_b / 1e9, 2),
        "sparse_fwd_bwd_frac_bf16_peak": round((fl_fwd + fl_bwd) / (t_fwd + t_b) / 1e9 / PEAK_BF16_TFLOPS, 4),
        "vs_bf16_rows_ms": round(t_bwd, 3),
        "dkv_normalised_difference_vs_bf16_rows": round(diff, 5),
        "workspace_bytes": need,
        "workspace_bytes_bf16_rows": ops.bwd_workspace_bytes(T, N, H, K),
    }


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=30)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-decode", action="store_true", help="skip every leg after the cfg3 step")
    ap.add_argument("--legs", default="all",
                    help="comma list of the legs after the cfg3 step to run: int8, decode, prologue, indexer_kl, "
                         "indexer_kl_dense, mla, v4, cfg2, cfg4 (default all)")
    ap.add_argument("--pmc-calibration", action="store_true",
                    help="only copy a 1 GiB tensor (known HBM bytes) to calibrate FETCH_SIZE / WRITE_SIZE")
    args = ap.parse_args()
    if args.pmc_calibration:
        import torch
        x = torch.empty(1 << 28, dtype=torch.float32, device="cuda").fill_(1.0)
        y = torch.empty_like(x)
        for _ in range(3):
            y.copy_(x)              # 1 GiB read + 1 GiB written per copy
        torch.cuda.synchronize()
        print("pmc calibration copies done", flush=True)
        return
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (this build runs the DSA path on a single MI355X); "
              f"--gpus {args.gpus} is not supported", file=sys.stderr)
        sys.exit(2)

    import torch
    from mcore_bridge_amd import ops, workloads as W

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    cfg = W.CONFIGS["cfg3"]
    T, H, K = cfg.S, cfg.H, cfg.K
    cu = cfg.cu_seqlens
    max_seqlen = max(b - a for a, b in zip(cu[:-1], cu[1:]))
    x = W.make_prefill(cfg, device=dev)
    q, kv = x["q"].bfloat16(), x["kv"].bfloat16()
    qi, ki, w = x["q_idx"].bfloat16(), x["k_idx"].bfloat16(), x["w"]
    dout = x["dout"].bfloat16()
    cu_t = x["cu_seqlens"]
    del x
    scale = W.SM_SCALE

    # backward through the C ABI with preallocated outputs/workspace and per-stage events
    from mcore_bridge_amd import _lib
    lib = _lib.load()
    N = kv.shape[0]
    dq = torch.empty_like(q)
    dkv = torch.empty(N, 576, dtype=torch.float32, device=dev)
    ws_bytes = ops.bwd_workspace_bytes(T, N, H, K)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
    stream = torch.cuda.current_stream(dev).cuda_stream
    STAGES = ("bwd_pairs", "bwd_sp", "bwd_dq", "bwd_g", "bwd_dkv_reduce")
    ev = {k: [] for k in ("indexer_topk", "sparse_fwd") + STAGES}

    def new_event():
        e = torch.cuda.Event(enable_timing=True)
        e.record()          # materialise the handle; re-recorded by the library
        return e

    def step(record: bool):
        e0 = new_event() if record else None
        idx = ops.indexer_topk(qi, ki, w, K, cu_t, True, max_seqlen)
        e1 = new_event() if record else None
        out, lse = ops.sparse_mla_fwd(q, kv, idx, scale, True)
        se = [new_event() for _ in range(6)] if record else None
        arr = (ctypes.c_void_p * 6)(*[e.cuda_event for e in se]) if record else None
        _lib.check("dsa_sparse_mla_bwd_timed", lib.dsa_sparse_mla_bwd_timed(
            q.data_ptr(), kv.data_ptr(), idx.data_ptr(), out.data_ptr(), dout.data_ptr(), lse.data_ptr(), T, N, H,
            576, 512, K, scale, 1, dq.data_ptr(), dkv.data_ptr(), ws.data_ptr(), ws_bytes, arr, stream))
        if record:
            ev["indexer_topk"].append((e0, e1))
            ev["sparse_fwd"].append((e1, se[0]))
            for i, name in enumerate(STAGES):
                ev[name].append((se[i], se[i + 1]))
        return dq, dkv

    for i in range(args.warmup):
        step(False)
        print(f"[bench] warmup step {i + 1}/{args.warmup} done", file=sys.stderr, flush=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        step(True)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_step = wall / args.steps * 1e3
    print(f"[bench] {args.steps} timed steps: {ms_step:.3f} ms/step", file=sys.stderr, flush=True)

    def avg_ms(name):
        return statistics.mean(a.elapsed_time(b) for a, b in ev[name])

    nsel = W.n_sel(cu, K)
    npairs = W.n_pairs(cu)
    fl_fwd = 2176 * H * nsel
    fl_bwd = 5504 * H * nsel
    fl_idx = 2 * cfg.Di * cfg.Hi * npairs
    total = fl_fwd + fl_bwd + fl_idx
    value = total / (ms_step * 1e-3) / 1e12
    t = {k: avg_ms(k) for k in ev}
    t_fwd, t_idx = t["sparse_fwd"], t["indexer_topk"]
    t_bwd = sum(t[k] for k in STAGES)
    # Algorithmic work of each hot kernel (one launch per step) and the roofline that bounds it:
    # the attention products are bf16 MFMA flops (fwd 2176*H, B1 S+dP 2176*H, B2 dQ 1152*H, B3 dKV
    # rows 2176*H per selected pair); B5 streams the per-pair dKV rows, so HBM bytes.  The
    # algorithmic bytes of each kernel are the operands it must read and the results it must write
    # (q, O, dO, dq: T*H*(576|512)*2; kv rows N*1152; idx T*K*4; lse T*H*4; dKV N*576*4) -- the
    # staged P / dS tiles and dKV rows are this design's intermediates and are not counted.
    qb, ob, kvb, ib, lb = T * H * 576 * 2, T * H * 512 * 2, N * 1152, T * K * 4, T * H * 4
    work = {
        "sparse_fwd": ("mfma", 2176 * H * nsel, "sparse_mla_fwd_kernel", qb + kvb + ib + ob + lb),
        "bwd_sp": ("mfma", 2176 * H * nsel, "bwd_sp_kernel", qb + kvb + ib + 2 * ob + lb),
        "bwd_dq": ("mfma", 1152 * H * nsel, "bwd_dq8_kernel" if H == 128 else "bwd_dq_kernel", kvb + ib + qb),
        "bwd_g": ("mfma", 2176 * H * nsel, "bwd_g_kernel", qb + ob + kvb + ib),
        "bwd_dkv_reduce": ("hbm", nsel * 1152 + N * 576 * 4 + N * 8, "bwd_dkv_reduce_kernel", N * 576 * 4),
    }
    dom = max(work, key=lambda k: t[k])
    bound, amount, kname, alg_bytes = work[dom]
    if bound == "mfma":
        achieved, peak, unit = amount / (t[dom] * 1e-3) / 1e12, PEAK_BF16_TFLOPS, "TFLOP/s"
    else:
        achieved, peak, unit = amount / (t[dom] * 1e-3) / 1e9, PEAK_HBM_GBS, "GB/s"
    traffic = measured_traffic(kname)
    bwd_kernels = [work[k][2] for k in STAGES if k in work] + ["csr_hist_kernel", "csr_colscan_kernel", "csr_fill_kernel"]
    bwd_counter = [measured_traffic(k) for k in bwd_kernels]
    bwd_alg = qb + kvb + ib + 2 * ob + lb + qb + N * 576 * 4
    bwd_traffic = {
        "algorithmic_bytes": bwd_alg,
        "counter_bytes": sum(bwd_counter) if all(b is not None for b in bwd_counter) else None,
        "per_kernel_counter_bytes": dict(zip(bwd_kernels, bwd_counter)),
        "source": "profiles/dsa_cfg3_hbm_traffic.md (rocprofv3 --pmc FETCH_SIZE, WRITE_SIZE; calibrated)",
    }
    if bwd_traffic["counter_bytes"]:
        bwd_traffic["ratio"] = round(bwd_traffic["counter_bytes"] / bwd_alg, 2)
    res = {
        "metric": METRIC,
        "value": round(value, 3),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {
            "workload": "cfg3: bf16 DSA fwd+bwd, T=16384 packed varlen (cu_seqlens 0/10363/15340/15537/16384, "
                        "causal per document), H=128, d_qk=576, d_v=512, indexer 64x128, top-k 2048",
            "global_batch": 1, "seq_len": T, "parallelism": "single GPU",
        },
        "breakdown_ms": {k: round(v, 3) for k, v in t.items()} | {"sparse_bwd": round(t_bwd, 3)},
        "breakdown_tflops": {"indexer": round(fl_idx / t_idx / 1e9, 2), "sparse_fwd": round(fl_fwd / t_fwd / 1e9, 2),
                             "sparse_bwd": round(fl_bwd / t_bwd / 1e9, 2),
                             "sparse_fwd_bwd": round((fl_fwd + fl_bwd) / (t_fwd + t_bwd) / 1e9, 2),
                             "sparse_fwd_bwd_frac_bf16_peak": round((fl_fwd + fl_bwd) / (t_fwd + t_bwd) / 1e9
                                                                    / PEAK_BF16_TFLOPS, 4)},
        "roofline": {"bound": bound, "kernel": kname, "achieved": round(achieved, 2), "peak": peak, "unit": unit,
                     "frac": round(achieved / peak, 4), "traffic": traffic,
                     "traffic_source": "profiles/dsa_cfg3_hbm_traffic.md (committed rocprofv3 PMC summary)",
                     "algorithmic": amount, "algorithmic_bytes": alg_bytes,
                     "traffic_over_algorithmic_bytes": round(traffic / alg_bytes, 2) if traffic else None,
                     "ms": round(t[dom], 3)},
        "backward_traffic": bwd_traffic,
    }
    legs = set(args.legs.split(",")) if args.legs != "all" else None

    def want(name):
        return not args.no_decode and (legs is None or name in legs)

    if legs is None or "int8" in legs:
        res["sparse_bwd_int8_staging"] = int8_staging_leg(torch, lib, _lib, q, kv, qi, ki, w, dout, cu_t, max_seqlen,
                                                          scale, dkv, ws, stream, fl_fwd, fl_bwd, t_fwd, t_bwd)
        print(f"[bench] int8-staging backward leg done: {res['sparse_bwd_int8_staging']['ms']} ms", file=sys.stderr,
              flush=True)
    if want("decode"):
        res["decode"] = decode_leg(torch, dev)
        print(f"[bench] decode leg done: {res['decode']['attention_us']} us", file=sys.stderr, flush=True)
    if want("prologue"):
        res["indexer_prologue"] = prologue_leg(torch, dev)
        print(f"[bench] prologue leg done: {res['indexer_prologue']['bf16']['us']} us", file=sys.stderr, flush=True)
    if want("indexer_kl"):
        idx = ops.indexer_topk(qi, ki, w, K, cu_t, True, max_seqlen)
        _, lse = ops.sparse_mla_fwd(q, kv, idx, scale, True)
        res["indexer_kl"] = indexer_kl_leg(torch, dev, q, kv, idx, lse, qi, ki, w, scale, nsel, ws)
        del idx, lse
        print(f"[bench] indexer KL leg done: {res['indexer_kl']['total_ms']} ms", file=sys.stderr, flush=True)
    if want("indexer_kl_dense"):
        res["indexer_kl_dense"] = indexer_kl_dense_leg(torch, dev, q, kv, qi, ki, w, cu_t, max_seqlen, scale, npairs)
        print(f"[bench] dense indexer KL leg done: {res['indexer_kl_dense']['loss_fwd_bwd_ms']} ms", file=sys.stderr,
              flush=True)
    if want("mla"):
        res["mla"] = mla_leg(torch, dev, qi, ki, w)
        print(f"[bench] mla leg done: {res['mla']['ms']} ms", file=sys.stderr, flush=True)
    if want("v4"):
        res["v4"] = v4_leg(torch, dev)
        print(f"[bench] v4 leg done: {res['v4']['ms']} ms", file=sys.stderr, flush=True)
    for name in ("cfg2", "cfg4"):
        if want(name):
            res[name] = prefill_fwd_leg(torch, dev, name)
            print(f"[bench] {name} leg done: chain {res[name]['chain_ms']} ms", file=sys.stderr, flush=True)
    if not args.no_cpu_baseline:
        res["cpu_baseline"] = cpu_baseline(torch, dev)
        print("[bench] cpu baseline done", file=sys.stderr, flush=True)
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
