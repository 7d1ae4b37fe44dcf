"""Golden fixtures (tests/golden/*.npz, written by tests/golden/make_golden.py from the float64
oracle): their inputs regenerate bit for bit, the oracle still reproduces them, and the index
sets of the edge cases equal what the selection rule fixes by hand -- ties to the lower key,
every visible key when a document is shorter than K, the token itself in a 1-token document,
the lowest keys when every score is zero."""
import os
import sys

import numpy as np
import pytest
import torch

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
sys.path.insert(0, HERE)
import cases  # noqa: E402
import make_golden  # noqa: E402

EDGE = ("ties", "s_lt_k", "one_token_docs", "zero_relu")


@pytest.mark.parametrize("name", cases.NAMES)
def test_golden_inputs_regenerate(name):
    fx = cases.load(name, HERE)
    got = cases.checksums(cases.inputs(name)).numpy()
    np.testing.assert_allclose(got, fx["checksums"], rtol=1e-12, atol=0,
                               err_msg=f"{name}: inputs drifted (RNG change?) -- regenerate the fixtures")


@pytest.mark.parametrize("name", cases.NAMES)
def test_oracle_reproduces_golden(name):
    fx = cases.load(name, HERE)
    new = make_golden.compute(name)
    assert np.array_equal(new["idx"], fx["idx"]), f"{name}: top-k indices changed"
    for k in ("lse", "out_sum", "out_sq", "dq_sum", "dq_sq", "dkv_sum", "dkv_sq"):
        scale = max(float(np.abs(fx[k][np.isfinite(fx[k])]).max(initial=0.0)), 1e-30)
        np.testing.assert_allclose(new[k], fx[k], rtol=1e-5, atol=1e-6 * scale, err_msg=f"{name}: {k}")
    for k in ("out_rows", "dq_rows", "dkv_rows"):
        a, b = cases.rows_from_bits(new[k]), cases.rows_from_bits(fx[k])
        torch.testing.assert_close(a, b, rtol=2 ** -7, atol=1e-3 * float(b.abs().max()), msg=f"{name}: {k}")


def _visible(cu, t):
    for a, b in zip(cu[:-1], cu[1:]):
        if a <= t < b:
            return list(range(a, t + 1))
    raise ValueError(t)


def _expected_edge_idx(name):
    """Index rows the selection rule fixes without computing a score."""
    d = cases.inputs(name)
    T, K, cu = d["q"].shape[0], d["K"], d["cu_seqlens"]
    out = np.full((T, K), -1, dtype=np.int64)
    for t in range(T):
        vis = _visible(cu, t)
        if name == "ties":        # class s % 3 scores 4, 2, 1: best class first, lower key within it
            sel = sorted(vis, key=lambda s: (s % 3, s))[:K]
        else:                     # s_lt_k / one_token_docs: all visible when <= K; zero_relu: lowest
            sel = vis[:K]
        sel = sorted(sel)
        out[t, : len(sel)] = sel
    return out


@pytest.mark.parametrize("name", EDGE)
def test_golden_edge_indices_follow_the_selection_rule(name):
    fx = cases.load(name, HERE)
    exp = _expected_edge_idx(name)
    if name in ("s_lt_k", "one_token_docs"):
        # the rule only fixes rows with at most K visible keys
        d = cases.inputs(name)
        rows = [t for t in range(exp.shape[0]) if len(_visible(d["cu_seqlens"], t)) <= d["K"]]
        assert rows, name
        assert np.array_equal(fx["idx"][rows], exp[rows])
    else:
        assert np.array_equal(fx["idx"], exp)


def test_golden_zero_relu_scores_are_zero():
    d = cases.inputs("zero_relu")
    logits = torch.einsum("thd,sd->ths", d["q_idx"].double(), d["k_idx"].double())
    assert (logits <= 0).all()
