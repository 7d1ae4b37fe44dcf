"""Write the golden fixtures tests/golden/<case>.npz from the float64 CPU oracle
(oracle/dsa_oracle.py), on the inputs of tests/golden/cases.py.

    python tests/golden/make_golden.py

Per case: checksums of the inputs, the top-k indices (canonical order: ascending key id, -1
padding to K), lse, and of out / dq / dkv their per-row sums and sums of squares plus a few full
rows (as bf16 bit patterns in uint16: the float32 sums pin the values to float32 precision, the
rows pin the layout).  The reference ships no golden vectors for this path; these pin the
oracle's outputs (itself pinned by tests/test_oracle.py) so that a change in either the oracle
or the kernels shows up against fixed numbers.
"""
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
for p in (ROOT, os.path.join(ROOT, "mcore-bridge_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)

sys.path.insert(0, HERE)
from oracle import dsa_oracle as O  # noqa: E402
import cases  # noqa: E402


def sample_rows(T: int):
    return sorted({0, T // 2, T - 1})


def compute(name: str) -> dict:
    d = cases.inputs(name)
    T, K = d["q"].shape[0], d["K"]
    cu = torch.tensor(d["cu_seqlens"])
    scores = O.indexer_scores(d["q_idx"], d["k_idx"], d["w"], cu, causal=d["causal"])
    sel = O.topk_indices(scores, K)
    idx = torch.full((T, K), -1, dtype=torch.int64)
    idx[:, : sel.shape[1]] = sel
    out, lse = O.sparse_mla_fwd(d["q"], d["kv"], idx, cases.SM_SCALE)
    dq, dkv = O.sparse_mla_bwd(d["q"], d["kv"], idx, out, d["dout"], lse, cases.SM_SCALE)
    rows = sample_rows(T)
    f32 = lambda x: x.to(torch.float32).numpy()
    bf16_bits = lambda x: x.to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    return {
        "checksums": cases.checksums(d).numpy(),
        "idx": idx.to(torch.int16).numpy(),
        "lse": f32(lse),
        "out_sum": f32(out.sum(-1)), "out_sq": f32((out * out).sum(-1)), "out_rows": bf16_bits(out[rows]),
        "dq_sum": f32(dq.sum(-1)), "dq_sq": f32((dq * dq).sum(-1)), "dq_rows": bf16_bits(dq[rows]),
        "dkv_sum": f32(dkv.sum(-1)), "dkv_sq": f32((dkv * dkv).sum(-1)), "dkv_rows": bf16_bits(dkv[rows]),
        "rows": np.asarray(rows, dtype=np.int64),
    }


def main():
    for name in cases.NAMES:
        arrays = compute(name)
        path = os.path.join(HERE, f"{name}.npz")
        np.savez_compressed(path, **arrays)
        print(f"{path}: {os.path.getsize(path)} bytes")


if __name__ == "__main__":
    main()
