"""CPU checks of the C ABI: the library loads, exports every symbol include/dsa_abi.h declares,
and rejects invalid arguments before touching a device (so these run without a GPU)."""
import ctypes
import os
import re

import pytest

from mcore_bridge_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "dsa_abi.h")


def _declared():
    src = open(HEADER).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b(dsa_[a-z0-9_]+)\s*\(", src)))


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    names = _declared()
    assert len(names) >= 8
    for n in names:
        assert hasattr(lib, n), n
        assert n in _lib.SIGNATURES, f"{n} has no ctypes signature"


def test_version_and_strerror():
    lib = _lib.load()
    assert lib.dsa_abi_version() >= 100
    for code in (0, -1, -2, -3, -4, -5):
        assert len(_lib.strerror(code)) >= 2
    assert "unknown" in _lib.strerror(-99)


N = ctypes.c_void_p(0)
P = ctypes.c_void_p(4096)  # never dereferenced: validation fails first


def test_invalid_arguments_rejected_before_launch():
    lib = _lib.load()
    # d_qk must be 576 (512-wide q rows only through the sink entry points)
    assert lib.dsa_sparse_mla_fwd(P, P, P, 4, 4, 16, 512, 512, 8, 0.1, 1, P, P, N) == _lib.DSA_ERR_UNSUPPORTED
    # null pointer
    assert lib.dsa_sparse_mla_fwd(N, P, P, 4, 4, 16, 576, 512, 8, 0.1, 1, P, P, N) == _lib.DSA_ERR_INVALID_ARG
    # misaligned
    assert lib.dsa_sparse_mla_fwd(ctypes.c_void_p(4098), P, P, 4, 4, 16, 576, 512, 8, 0.1, 1, P, P, N) == _lib.DSA_ERR_INVALID_ARG
    # non-finite scale
    assert lib.dsa_sparse_mla_fwd(P, P, P, 4, 4, 16, 576, 512, 8, float("nan"), 1, P, P, N) == _lib.DSA_ERR_INVALID_ARG
    # zero-size work is a no-op
    assert lib.dsa_sparse_mla_fwd(N, N, N, 0, 4, 16, 576, 512, 8, 0.1, 1, N, N, N) == _lib.DSA_OK
    # indexer: too many heads / bad head_dim / dtype mismatch / fp8 without scales
    args = lambda hi, di, qd, kd, qs: (P, qd, qs, P, kd, qs, P, P, P, 4, 4, hi, di, 4, P, 4, 0, N)
    assert lib.dsa_indexer_scores(*args(65, 128, 0, 0, P)) == _lib.DSA_ERR_UNSUPPORTED
    assert lib.dsa_indexer_scores(*args(64, 96, 0, 0, P)) == _lib.DSA_ERR_UNSUPPORTED
    assert lib.dsa_indexer_scores(*args(64, 128, 0, 1, P)) == _lib.DSA_ERR_UNSUPPORTED
    assert lib.dsa_indexer_scores(*args(64, 128, 1, 1, N)) == _lib.DSA_ERR_INVALID_ARG
    # pitch smaller than the longest row
    assert lib.dsa_indexer_scores(P, 0, N, P, 0, N, P, P, P, 4, 4, 4, 64, 9, P, 8, 0, N) == _lib.DSA_ERR_INVALID_ARG
    # top-k: k < 1, null output
    assert lib.dsa_topk(P, 8, P, P, 4, 0, P, N, N, 0, N) == _lib.DSA_ERR_INVALID_ARG
    assert lib.dsa_topk(P, 8, P, P, 4, 2, N, N, N, 0, N) == _lib.DSA_ERR_INVALID_ARG
    # top-k split workspace: few rows longer than a slice only; too small a workspace is refused
    ws = lib.dsa_topk_workspace_size(64, 65268, 2048)
    assert ws == 64 * 4 * 2048 * 8                               # 4 slices of 16384 keys
    assert lib.dsa_topk_workspace_size(256, 65268, 2048) == 0    # the rows alone fill the device
    assert lib.dsa_topk_workspace_size(64, 16384, 2048) == 0     # one slice per row
    assert lib.dsa_topk_workspace_size(0, 65268, 2048) == 0
    assert lib.dsa_topk(P, 65268, P, P, 64, 2048, P, N, P, ws - 1, N) == _lib.DSA_ERR_WORKSPACE
    # backward: 512-wide q only through the sink entry points; heads not a multiple of 16,
    # workspace too small
    assert lib.dsa_sparse_mla_bwd(P, P, P, P, P, P, 4, 4, 32, 512, 512, 8, 0.1, 1, P, P, P, 1 << 30, N) == _lib.DSA_ERR_UNSUPPORTED
    assert lib.dsa_sparse_mla_bwd_sink(P, P, P, P, P, P, P, 4, 4, 32, 448, 512, 8, 0.1, 1, P, P, P, 0, P, 1 << 30,
                                       N) == _lib.DSA_ERR_UNSUPPORTED
    assert lib.dsa_sparse_mla_fwd_sink(P, P, P, 4, 4, 16, 448, 512, 8, 0.1, 1, P, P, P, N) == _lib.DSA_ERR_UNSUPPORTED
    assert lib.dsa_sparse_mla_bwd(P, P, P, P, P, P, 4, 4, 24, 576, 512, 8, 0.1, 1, P, P, P, 1 << 30, N) == _lib.DSA_ERR_UNSUPPORTED
    assert lib.dsa_sparse_mla_bwd(P, P, P, P, P, P, 4, 4, 32, 576, 512, 8, 0.1, 1, P, P, P, 16, N) == _lib.DSA_ERR_WORKSPACE
    # no query rows: dkv is still written (must be given), nothing else is needed; no stages to time
    assert lib.dsa_sparse_mla_bwd(N, N, N, N, N, N, 0, 4, 32, 576, 512, 8, 0.1, 1, N, N, N, 0, N) == _lib.DSA_ERR_INVALID_ARG
    ev = (ctypes.c_void_p * 6)(*([P] * 6))
    assert lib.dsa_sparse_mla_bwd_timed(N, N, N, N, N, N, 0, 4, 32, 576, 512, 8, 0.1, 1, N, P, N, 0, ev, N) == \
        _lib.DSA_ERR_INVALID_ARG
    # rows: bad n_seq
    assert lib.dsa_build_rows(P, 0, 4, 1, P, P, N) == _lib.DSA_ERR_INVALID_ARG


def test_bwd_workspace_size_formula():
    lib = _lib.load()
    T, N, H, K = 16384, 16384, 128, 2048
    ws = lib.dsa_sparse_mla_bwd_workspace_size(T, N, H, K)
    stage = T * H * K * 2
    # P and dS tiles, G rows, pair rows, key offsets, and the pair ordering's integer counters:
    # 257 rows (256 query runs + totals) of N
    fixed = 2 * stage + T * K * 576 * 2 + T * K * 8 + (N + 1) * 8 + 257 * N * 4
    assert fixed <= ws < fixed + 4096
    assert lib.dsa_sparse_mla_bwd_workspace_size(-1, N, H, K) == 0
    # the flags form: one pass (chunk_q = 0) with bf16 rows is the same layout; int8 rows are
    # 640 bytes (5 lines) instead of 1152; passes round up to 256 rows; unknown flags size 0
    assert lib.dsa_sparse_mla_bwd_workspace_size_ex(T, N, H, K, 0, 0) == ws
    ws8 = lib.dsa_sparse_mla_bwd_workspace_size_ex(T, N, H, K, 0, 1)
    assert ws - ws8 == (T * K + 1) * (1152 - 640)
    assert lib.dsa_sparse_mla_bwd_workspace_size_ex(T, N, H, K, 300, 0) == \
        lib.dsa_sparse_mla_bwd_workspace_size_chunked(T, N, H, K, 512)
    assert lib.dsa_sparse_mla_bwd_workspace_size_ex(T, N, H, K, 300, 1) < \
        lib.dsa_sparse_mla_bwd_workspace_size_ex(T, N, H, K, 300, 0)
    assert lib.dsa_sparse_mla_bwd_workspace_size_ex(T, N, H, K, 0, 2) == 0
    assert lib.dsa_sparse_mla_bwd_workspace_size_ex(T, N, H, K, -1, 0) == 0


def test_bwd_flags_validated_before_launch():
    lib = _lib.load()
    big = 1 << 40
    # unknown flag bits, also with no query rows
    assert lib.dsa_sparse_mla_bwd_ex(P, P, P, P, P, P, 4, 4, 32, 576, 512, 8, 0.1, 1, P, P, 2, P, big, N, N) == \
        _lib.DSA_ERR_INVALID_ARG
    assert lib.dsa_sparse_mla_bwd_ex(N, N, N, N, N, N, 0, 4, 32, 576, 512, 8, 0.1, 1, N, P, 4, N, 0, N, N) == \
        _lib.DSA_ERR_INVALID_ARG
    # an int8-row workspace one byte short of the smallest pass is refused
    need = lib.dsa_sparse_mla_bwd_workspace_size_ex(4, 4, 32, 8, 256, 1)
    assert lib.dsa_sparse_mla_bwd_ex(P, P, P, P, P, P, 4, 4, 32, 576, 512, 8, 0.1, 1, P, P, 1, P, need - 1, N, N) == \
        _lib.DSA_ERR_WORKSPACE


def test_decode_entry_points_validate_and_size():
    lib = _lib.load()
    # batch 64 x 128 heads fills 64 of 256 CUs -> 4 key splits of 512 slots: bf16 partial rows + fp32 LSEs
    rows = 64 * 4 * 128
    assert lib.dsa_sparse_mla_decode_workspace_size(64, 128, 2048) == rows * 512 * 2 + rows * 4
    assert lib.dsa_sparse_mla_decode_workspace_size(256, 128, 2048) == 0     # the batch alone fills the device
    assert lib.dsa_sparse_mla_decode_workspace_size(64, 128, 64) == 0        # too few keys to split
    assert lib.dsa_sparse_mla_decode_workspace_size(0, 0, 2048) == 0
    dec = lambda q, dqk, ws, nbytes, batch=64: lib.dsa_sparse_mla_decode(q, P, P, batch, 100, 128, dqk, 512, 2048, 0.1,
                                                                         P, P, ws, nbytes, N)
    assert dec(P, 512, P, 1 << 30) == _lib.DSA_ERR_UNSUPPORTED
    assert dec(N, 576, P, 1 << 30) == _lib.DSA_ERR_INVALID_ARG
    assert dec(P, 576, N, 0) == _lib.DSA_ERR_WORKSPACE
    assert dec(P, 576, P, 1024) == _lib.DSA_ERR_WORKSPACE
    assert dec(N, 576, N, 0, batch=0) == _lib.DSA_OK
    assert lib.dsa_build_decode_rows(N, 4, P, P, N) == _lib.DSA_ERR_INVALID_ARG
    assert lib.dsa_build_decode_rows(N, 0, N, N, N) == _lib.DSA_OK


def test_ops_refuse_cpu_tensors():
    import torch
    from mcore_bridge_amd import ops
    q = torch.zeros(4, 16, 576, dtype=torch.bfloat16)
    kv = torch.zeros(4, 576, dtype=torch.bfloat16)
    idx = torch.zeros(4, 2, dtype=torch.int32)
    with pytest.raises(RuntimeError, match="GPU"):
        ops.sparse_mla_fwd(q, kv, idx, 0.1, True)


def test_indexer_loss_entry_points_validate_and_size():
    lib = _lib.load()
    # KL target: d_qk must be 576, at most 128 heads, finite positive scale; empty work is a no-op
    tgt = lambda q, dqk, H, sc, T=4: lib.dsa_indexer_kl_target(q, P, P, P, T, 8, H, dqk, 16, sc, 1, P, N)
    assert tgt(P, 512, 16, 0.1) == _lib.DSA_ERR_UNSUPPORTED
    assert tgt(P, 576, 129, 0.1) == _lib.DSA_ERR_UNSUPPORTED
    assert tgt(N, 576, 16, 0.1) == _lib.DSA_ERR_INVALID_ARG
    assert tgt(P, 576, 16, float("nan")) == _lib.DSA_ERR_INVALID_ARG
    assert tgt(ctypes.c_void_p(4100), 576, 16, 0.1) == _lib.DSA_ERR_INVALID_ARG
    assert tgt(N, 576, 16, 0.1, T=0) == _lib.DSA_OK
    # target from the attention backward's workspace: its head limits, and a workspace of its size
    fb = lambda H, nbytes: lib.dsa_indexer_kl_target_from_bwd(P, nbytes, P, 4, 8, H, 16, 1, P, N)
    assert fb(24, 1 << 30) == _lib.DSA_ERR_UNSUPPORTED
    assert fb(32, lib.dsa_sparse_mla_bwd_workspace_size(4, 8, 32, 16) - 1) == _lib.DSA_ERR_WORKSPACE
    # KL rows: finite gradient scale, non-null buffers
    assert lib.dsa_indexer_kl_loss(P, P, P, 4, 8, 16, 1, float("inf"), P, P, N) == _lib.DSA_ERR_INVALID_ARG
    assert lib.dsa_indexer_kl_loss(P, P, P, 4, 8, 16, 1, 1.0, P, N, N) == _lib.DSA_ERR_INVALID_ARG
    assert lib.dsa_indexer_kl_loss(N, N, N, 0, 8, 16, 1, 1.0, N, N, N) == _lib.DSA_OK
    # selected scores: head_dim 128, <= 64 heads, top-k <= 4096, aligned rows
    sel = lambda q, H, D, K, T=4: lib.dsa_indexer_selected_scores(q, P, P, P, T, 8, H, D, K, 1, P, N)
    assert sel(P, 64, 64, 16) == _lib.DSA_ERR_UNSUPPORTED
    assert sel(P, 65, 128, 16) == _lib.DSA_ERR_UNSUPPORTED
    assert sel(P, 64, 128, 4097) == _lib.DSA_ERR_UNSUPPORTED
    assert sel(ctypes.c_void_p(4104), 64, 128, 16) == _lib.DSA_ERR_INVALID_ARG
    assert sel(N, 64, 128, 16, T=0) == _lib.DSA_OK
    # scores backward: workspace = dk rows (T*K + 1) x 256 B + pair rows T*K x 8 B + key offsets
    # + the pair ordering's counters (256 query runs + totals) x Nk
    T, Nk, K = 16384, 16384, 2048
    ws = lib.dsa_indexer_scores_bwd_workspace_size(T, Nk, K)
    fixed = (T * K + 1) * 256 + T * K * 8 + (Nk + 1) * 8 + 257 * Nk * 4
    assert fixed <= ws < fixed + 1024
    assert lib.dsa_indexer_scores_bwd_workspace_size(-1, Nk, K) == 0
    bwd = lambda dq, ws_, nbytes: lib.dsa_indexer_scores_bwd(P, P, P, P, P, 4, 8, 64, 128, 16, 1, dq, P, P, ws_, nbytes, N)
    assert bwd(P, P, 16) == _lib.DSA_ERR_WORKSPACE
    assert bwd(P, N, 1 << 30) == _lib.DSA_ERR_WORKSPACE
    assert bwd(N, P, 1 << 30) == _lib.DSA_ERR_INVALID_ARG
    # no query rows: only dk is needed (written as zeros); without it the call is refused
    assert lib.dsa_indexer_scores_bwd(N, N, N, N, N, 0, 8, 64, 128, 16, 1, N, N, N, N, 0, N) == _lib.DSA_ERR_INVALID_ARG
    # prologue backward: (T + 64) rows of 256 floats of workspace; limits as the forward
    assert lib.dsa_indexer_prologue_bwd_workspace_size(1000) == (1000 + 64) * 256 * 4
    pb = lambda dq, H, ws_, nbytes, stride=64 * 128: lib.dsa_indexer_prologue_bwd(
        dq, P, P, P, 128, P, P, 64, 4, H, 128, 64, 1e-6, 1.0, 0.125, 0.088, 0, 0, P, stride, P, 128, P, 64, P, P,
        ws_, nbytes, N)
    assert pb(P, 65, P, 1 << 20) == _lib.DSA_ERR_UNSUPPORTED
    assert pb(P, 64, P, 16) == _lib.DSA_ERR_WORKSPACE
    assert pb(ctypes.c_void_p(4100), 64, P, 1 << 20) == _lib.DSA_ERR_INVALID_ARG
    assert pb(P, 64, P, 1 << 20, stride=127) == _lib.DSA_ERR_INVALID_ARG


def test_indexer_loss_ops_refuse_cpu_tensors():
    import torch
    from mcore_bridge_amd import ops
    q = torch.zeros(4, 16, 576, dtype=torch.bfloat16)
    kv = torch.zeros(4, 576, dtype=torch.bfloat16)
    idx = torch.zeros(4, 2, dtype=torch.int32)
    with pytest.raises(RuntimeError, match="GPU"):
        ops.indexer_kl_target(q, kv, idx, torch.zeros(4, 16), 0.1, True)
    qi = torch.zeros(4, 8, 128, dtype=torch.bfloat16)
    ki = torch.zeros(4, 128, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="GPU"):
        ops.indexer_selected_scores(qi, ki, torch.zeros(4, 8), idx, True)
    with pytest.raises(RuntimeError, match="GPU"):
        ops.indexer_kl_rows(torch.zeros(4, 2), torch.zeros(4, 2), idx, 4, True, 1.0)


def test_decode_split_follows_the_device_cu_count():
    """The decode key splits fill the device's compute units: sized for a whole MI355X (256 CUs, also
    the assumption without a current device) and for partitions with fewer."""
    lib = _lib.load()
    f = lib.dsa_sparse_mla_decode_workspace_size_for
    assert f(64, 128, 2048, 256) == 64 * 4 * 128 * (512 * 2 + 4)
    if not _has_device():
        assert lib.dsa_sparse_mla_decode_workspace_size(64, 128, 2048) == f(64, 128, 2048, 256)
    assert f(64, 128, 2048, 128) == 64 * 2 * 128 * (512 * 2 + 4)   # 128 CUs: 2 splits
    assert f(64, 128, 2048, 32) == 0                               # 32 CUs: the batch alone fills them
    assert f(8, 128, 2048, 32) == 8 * 4 * 128 * (512 * 2 + 4)      # 8 sequences on 32 CUs: 4 splits
    assert f(1, 128, 2048, 32) == 1 * 16 * 128 * (512 * 2 + 4)     # at most one split per 4 key blocks
    assert f(64, 128, 2048, 0) == 0 and f(-1, 128, 2048, 256) == 0


def _has_device():
    import torch
    return torch.cuda.device_count() > 0


def test_launching_entry_points_report_a_missing_device():
    """Valid arguments without a usable gfx950 device: every launching entry point returns
    DSA_ERR_DEVICE (checked once per device, after the argument checks) instead of a launch error."""
    if _has_device():
        pytest.skip("a device is present")
    lib = _lib.load()
    dev = _lib.DSA_ERR_DEVICE
    assert lib.dsa_build_rows(P, 1, 4, 1, P, P, N) == dev
    assert lib.dsa_build_decode_rows(P, 4, P, P, N) == dev
    assert lib.dsa_sparse_mla_fwd(P, P, P, 4, 4, 16, 576, 512, 8, 0.1, 1, P, P, N) == dev
    assert lib.dsa_indexer_scores(P, 0, N, P, 0, N, P, P, P, 4, 4, 4, 64, 4, P, 4, 0, N) == dev
    assert lib.dsa_topk(P, 8, P, P, 4, 2, P, N, N, 0, N) == dev
    ws = lib.dsa_sparse_mla_bwd_workspace_size(4, 4, 32, 8)
    assert lib.dsa_sparse_mla_bwd(P, P, P, P, P, P, 4, 4, 32, 576, 512, 8, 0.1, 1, P, P, P, ws, N) == dev
    assert lib.dsa_sparse_mla_bwd(N, N, N, N, N, N, 0, 4, 32, 576, 512, 8, 0.1, 1, N, P, N, 0, N) == dev
    need = lib.dsa_sparse_mla_decode_workspace_size(64, 128, 2048)
    assert lib.dsa_sparse_mla_decode(P, P, P, 64, 100, 128, 576, 512, 2048, 0.1, P, P, P, need, N) == dev
    assert lib.dsa_sparse_mla_decode_noalloc(P, P, P, 64, 100, 128, 576, 512, 2048, 0.1, P, P, N) == dev
    # argument errors are still reported as such, ahead of the device check
    assert lib.dsa_sparse_mla_fwd(N, P, P, 4, 4, 16, 576, 512, 8, 0.1, 1, P, P, N) == _lib.DSA_ERR_INVALID_ARG
    assert lib.dsa_sparse_mla_decode(P, P, P, 64, 100, 128, 576, 512, 2048, 0.1, P, P, P, need - 1, N) == \
        _lib.DSA_ERR_WORKSPACE


def test_dense_loss_entry_points_validate_and_size():
    """The dense indexer-loss entry points: d_qk 576 and at most 128 heads for the attention
    statistics, head_dim 128 and at most 64 heads for the score backward, a pitch of at least one
    column, aligned rows, a workspace of the documented size; empty work is a no-op."""
    lib = _lib.load()
    lse = lambda q, dqk, H, sc, T=4: lib.dsa_dense_attention_lse(q, P, P, P, T, 8, H, dqk, sc, P, N)
    assert lse(P, 512, 16, 0.1) == _lib.DSA_ERR_UNSUPPORTED
    assert lse(P, 576, 129, 0.1) == _lib.DSA_ERR_UNSUPPORTED
    assert lse(N, 576, 16, 0.1) == _lib.DSA_ERR_INVALID_ARG
    assert lse(ctypes.c_void_p(4100), 576, 16, 0.1) == _lib.DSA_ERR_INVALID_ARG
    assert lse(P, 576, 16, float("nan")) == _lib.DSA_ERR_INVALID_ARG
    assert lse(P, 576, 16, -1.0) == _lib.DSA_ERR_INVALID_ARG
    assert lse(N, 576, 16, 0.1, T=0) == _lib.DSA_OK
    assert lib.dsa_dense_attention_lse(P, P, P, P, 4, 8, 16, 576, 0.1, N, N) == _lib.DSA_ERR_INVALID_ARG
    tgt = lambda pitch, lse_, T=4: lib.dsa_dense_attention_target(P, P, lse_, P, P, T, 8, 16, 576, pitch, 0.1, P, N)
    assert tgt(0, P) == _lib.DSA_ERR_INVALID_ARG
    assert tgt(8, N) == _lib.DSA_ERR_INVALID_ARG
    assert tgt(8, N, T=0) == _lib.DSA_OK
    # score backward: one 64 KB partial dk tile per (128-key tile, 256-query chunk)
    T, Nk = 16384, 16384
    ws = lib.dsa_dense_indexer_scores_bwd_workspace_size(T, Nk)
    assert ws == (Nk // 128) * (T // 256) * 128 * 128 * 4
    assert lib.dsa_dense_indexer_scores_bwd_workspace_size(0, Nk) == 0
    assert lib.dsa_dense_indexer_scores_bwd_workspace_size(T, 0) == 0
    bwd = lambda H, D, pitch, ws_, nbytes, dq=P: lib.dsa_dense_indexer_scores_bwd(
        P, P, P, P, P, 4, 8, H, D, P, pitch, dq, P, P, ws_, nbytes, N)
    need = lib.dsa_dense_indexer_scores_bwd_workspace_size(4, 8)
    assert bwd(65, 128, 8, P, need) == _lib.DSA_ERR_UNSUPPORTED
    assert bwd(64, 64, 8, P, need) == _lib.DSA_ERR_UNSUPPORTED
    assert bwd(64, 128, 0, P, need) == _lib.DSA_ERR_INVALID_ARG
    assert bwd(64, 128, 8, P, need, dq=N) == _lib.DSA_ERR_INVALID_ARG
    assert bwd(64, 128, 8, P, need - 1) == _lib.DSA_ERR_WORKSPACE
    assert bwd(64, 128, 8, N, need) == _lib.DSA_ERR_WORKSPACE
    # no query rows: only dk is needed (written as zeros); without it the call is refused
    assert lib.dsa_dense_indexer_scores_bwd(N, N, N, N, N, 0, 8, 64, 128, N, 8, N, N, N, N, 0, N) == \
        _lib.DSA_ERR_INVALID_ARG
    if not _has_device():
        assert lib.dsa_dense_attention_lse(P, P, P, P, 4, 8, 16, 576, 0.1, P, N) == _lib.DSA_ERR_DEVICE
        assert lib.dsa_dense_indexer_scores_bwd(P, P, P, P, P, 4, 8, 64, 128, P, 8, P, P, P, P, need, N) == \
            _lib.DSA_ERR_DEVICE


def test_dense_loss_ops_refuse_cpu_tensors():
    import torch
    from mcore_bridge_amd import ops
    q = torch.zeros(4, 16, 576, dtype=torch.bfloat16)
    kv = torch.zeros(4, 576, dtype=torch.bfloat16)
    rows = torch.zeros(4, dtype=torch.int32)
    with pytest.raises(RuntimeError, match="GPU"):
        ops.dense_attention_lse(q, kv, rows, rows + 1, 1, 0.1)
    with pytest.raises(RuntimeError, match="GPU"):
        ops.indexer_scores_dense_bwd(torch.zeros(4, 8, 128, dtype=torch.bfloat16), torch.zeros(4, 128, dtype=torch.bfloat16),
                                     torch.zeros(4, 8), rows, rows + 1, 1, torch.zeros(4, 4))


def test_v4_compressor_entry_points_validate_and_size():
    """The V4 compressor entry points: dim 64 / 128 / 256 / 512, channels = 2 * dim with overlap
    (dim without), row strides of at least the channels in multiples of 8, entry and item counts
    that the token count can hold, a workspace of the documented size; no entries is a no-op
    forward."""
    lib = _lib.load()
    fwd = lambda C, D, ov, T=16, ne=4, stride=None, eps=1e-6, kv=P, out=P: lib.dsa_v4_compress_fwd(
        kv, P, stride or C, stride or C, P, P, P, 1, T, ne, C, D, 4, ov, eps, out, N)
    assert fwd(200, 100, 1) == _lib.DSA_ERR_UNSUPPORTED
    assert fwd(512, 512, 1) == _lib.DSA_ERR_INVALID_ARG          # overlap needs 2 * dim channels
    assert fwd(1024, 512, 0) == _lib.DSA_ERR_INVALID_ARG
    assert fwd(1024, 512, 1, stride=1028) == _lib.DSA_ERR_INVALID_ARG
    assert fwd(1024, 512, 1, ne=5) == _lib.DSA_ERR_INVALID_ARG   # 5 windows of 4 in 16 tokens
    assert fwd(1024, 512, 1, eps=float("nan")) == _lib.DSA_ERR_INVALID_ARG
    assert fwd(1024, 512, 1, kv=N) == _lib.DSA_ERR_INVALID_ARG
    assert fwd(1024, 512, 1, kv=ctypes.c_void_p(4100)) == _lib.DSA_ERR_INVALID_ARG
    assert fwd(1024, 512, 1, ne=0, out=N) == _lib.DSA_OK
    assert fwd(1024, 512, 1, out=N) == _lib.DSA_ERR_INVALID_ARG
    # workspace: dnorm partials (one row per backward workgroup, at most 1024) + dape partials
    # (entry chunks x rate x channels, at most 256 chunks) + each entry's first token; CSA main
    # compressor at T = 16384, rate 4
    ws = lib.dsa_v4_compress_bwd_workspace_size(4096, 4096, 1024, 512, 4)
    assert ws == 1024 * 512 * 4 + 256 * 4 * 1024 * 4 + 4096 * 4
    assert lib.dsa_v4_compress_bwd_workspace_size(-1, 0, 1024, 512, 4) == 0
    bwd = lambda ws_, nbytes, dkv=P, dout=P, ni=4: lib.dsa_v4_compress_bwd(
        P, P, 1024, 1024, P, P, P, 1, 16, 4, ni, 1024, 512, 4, 1, 1e-6, dout, dkv, P, 1024, 1024, P, P, ws_, nbytes, N)
    need = lib.dsa_v4_compress_bwd_workspace_size(4, 4, 1024, 512, 4)
    assert need > 0
    assert bwd(P, need, ni=3) == _lib.DSA_ERR_INVALID_ARG        # fewer items than entries
    assert bwd(P, need, dkv=N) == _lib.DSA_ERR_INVALID_ARG
    assert bwd(P, need, dout=N) == _lib.DSA_ERR_INVALID_ARG
    assert bwd(P, need - 1) == _lib.DSA_ERR_WORKSPACE
    assert bwd(N, need) == _lib.DSA_ERR_WORKSPACE
    if not _has_device():
        assert fwd(1024, 512, 1) == _lib.DSA_ERR_DEVICE
        assert bwd(P, need) == _lib.DSA_ERR_DEVICE


def test_v4_compressor_doc_table():
    """compress_doc_table: token offsets, entry offsets (complete windows) and item offsets
    (complete windows plus each partial tail) per document; bad offsets are refused."""
    import torch
    from mcore_bridge_amd import ops
    tab, ne, ni = ops.compress_doc_table([0, 10, 10, 13, 21], 4, "cpu")
    assert tab.dtype == torch.int32 and tab.tolist() == [[0, 10, 10, 13, 21], [0, 2, 2, 2, 4], [0, 3, 3, 4, 6]]
    assert (ne, ni) == (4, 6)
    with pytest.raises(AssertionError):
        ops.compress_doc_table([0, 5, 3], 4, "cpu")
    with pytest.raises(AssertionError):
        ops.compress_doc_table([1, 5], 4, "cpu")
    with pytest.raises(RuntimeError, match="GPU"):
        ops.v4_compress_fwd(torch.zeros(8, 256, dtype=torch.bfloat16), torch.zeros(8, 256, dtype=torch.bfloat16),
                            torch.zeros(4, 256, dtype=torch.bfloat16), torch.ones(128, dtype=torch.bfloat16), tab, 2, 4,
                            1e-6, True)


def test_v4_row_transform_entry_points_validate():
    """The V4 row transforms: dim 64 / 128 / 256 / 512, rope_dim a multiple of 8 up to dim, rows a
    whole number of tokens, angle tables wide enough, heads that split into the groups."""
    lib = _lib.load()
    nr = lambda rows=64, H=4, D=512, rd=64, stride=32, cos=P, x=P, norm=1, eps=1e-6: lib.dsa_v4_norm_rope(
        x, rows, H, D, rd, cos, P, stride, norm, eps, 0, P, N)
    assert nr(D=96) == _lib.DSA_ERR_UNSUPPORTED
    assert nr(rows=66) == _lib.DSA_ERR_INVALID_ARG       # not a whole number of tokens
    assert nr(rd=60) == _lib.DSA_ERR_INVALID_ARG
    assert nr(rd=520) == _lib.DSA_ERR_INVALID_ARG
    assert nr(stride=31) == _lib.DSA_ERR_INVALID_ARG
    assert nr(cos=N) == _lib.DSA_ERR_INVALID_ARG
    assert nr(x=ctypes.c_void_p(4100)) == _lib.DSA_ERR_INVALID_ARG
    assert nr(eps=float("nan")) == _lib.DSA_ERR_INVALID_ARG
    assert nr(rows=0, x=N) == _lib.DSA_OK
    bwd = lambda x=P, norm=1: lib.dsa_v4_norm_rope_bwd(x, P, 64, 4, 512, 64, P, P, 32, norm, 1e-6, 0, P, N)
    assert bwd(x=N) == _lib.DSA_ERR_INVALID_ARG          # the norm's backward needs the forward input
    og = lambda H=8, G=3, T=4: lib.dsa_v4_out_rope_group(P, T, H, 512, 64, G, P, P, 32, 1, P, N)
    assert og() == _lib.DSA_ERR_INVALID_ARG              # 8 heads do not split into 3 groups
    assert og(T=-1, G=4) == _lib.DSA_ERR_INVALID_ARG
    assert og(T=0, G=4) == _lib.DSA_OK
    assert lib.dsa_v4_out_rope_group_bwd(P, 4, 8, 512, 64, 0, P, P, 32, 1, P, N) == _lib.DSA_ERR_INVALID_ARG
    if not _has_device():
        assert nr(rd=0, cos=N) == _lib.DSA_ERR_DEVICE     # no rope part: no angle tables needed
        assert og(G=4) == _lib.DSA_ERR_DEVICE
        assert bwd() == _lib.DSA_ERR_DEVICE
