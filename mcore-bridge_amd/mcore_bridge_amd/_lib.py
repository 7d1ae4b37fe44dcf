"""ctypes binding of libdsa_amd.so (the C ABI declared in include/dsa_abi.h).

The shared library is built in-tree by ``__graft_entry__.build()`` (``make -C
mcore-bridge_amd/csrc``) and lives next to this file.  Loading it needs no GPU (argument
checks and error strings work on any host); every entry point that launches work needs a
gfx950 device.  There is no fallback: a missing library raises ``ImportError`` with build
guidance, mirroring the reference's own ImportError for a missing fused_qk_topk_naive
(reference src/mcore_bridge/patcher.py:349-351).
"""
from __future__ import annotations

import ctypes
import os
from ctypes import c_float, c_int, c_int64, c_size_t, c_void_p, c_char_p

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libdsa_amd.so")

DSA_OK = 0
DSA_ERR_INVALID_ARG = -1
DSA_ERR_UNSUPPORTED = -2
DSA_ERR_WORKSPACE = -3
DSA_ERR_LAUNCH = -4
DSA_ERR_DEVICE = -5
DSA_ERR_SCRATCH = -6

DSA_BF16 = 0
DSA_FP8_E4M3 = 1

# name -> (restype, argtypes); must match include/dsa_abi.h
SIGNATURES = {
    "dsa_abi_version": (c_int, []),
    "dsa_strerror": (c_char_p, [c_int]),
    "dsa_build_rows": (c_int, [c_void_p, c_int, c_int, c_int, c_void_p, c_void_p, c_void_p]),
    "dsa_indexer_scores": (c_int, [c_void_p, c_int, c_void_p, c_void_p, c_int, c_void_p, c_void_p, c_void_p,
                                   c_void_p, c_int, c_int, c_int, c_int, c_int, c_void_p, c_int64, c_int,
                                   c_void_p]),
    "dsa_topk_workspace_size": (c_size_t, [c_int, c_int64, c_int]),
    "dsa_topk": (c_int, [c_void_p, c_int64, c_void_p, c_void_p, c_int, c_int, c_void_p, c_void_p, c_void_p,
                         c_size_t, c_void_p]),
    "dsa_indexer_prologue": (c_int, [c_void_p, c_int64, c_void_p, c_int64, c_void_p, c_int64, c_void_p, c_void_p,
                                     c_void_p, c_int64, c_int, c_int, c_int, c_int, c_float, c_float, c_float,
                                     c_float, c_int, c_int, c_int, c_void_p, c_void_p, c_void_p, c_void_p,
                                     c_void_p, c_void_p]),
    "dsa_indexer_prologue_bwd_workspace_size": (c_size_t, [c_int]),
    "dsa_indexer_prologue_bwd": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_int64, c_void_p, c_void_p,
                                         c_int64, c_int, c_int, c_int, c_int, c_float, c_float, c_float, c_float,
                                         c_int, c_int, c_void_p, c_int64, c_void_p, c_int64, c_void_p, c_int64,
                                         c_void_p, c_void_p, c_void_p, c_size_t, c_void_p]),
    "dsa_sparse_mla_fwd": (c_int, [c_void_p, c_void_p, c_void_p, c_int, c_int, c_int, c_int, c_int, c_int,
                                   c_float, c_int, c_void_p, c_void_p, c_void_p]),
    "dsa_sparse_mla_fwd_sink": (c_int, [c_void_p, c_void_p, c_void_p, c_int, c_int, c_int, c_int, c_int, c_int,
                                        c_float, c_int, c_void_p, c_void_p, c_void_p, c_void_p]),
    "dsa_sparse_mla_bwd_sink_workspace_size": (c_size_t, [c_int, c_int, c_int, c_int, c_int]),
    "dsa_sparse_mla_bwd_sink": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_int,
                                        c_int, c_int, c_int, c_int, c_int, c_float, c_int, c_void_p, c_void_p,
                                        c_void_p, c_int, c_void_p, c_size_t, c_void_p]),
    "dsa_build_decode_rows": (c_int, [c_void_p, c_int, c_void_p, c_void_p, c_void_p]),
    "dsa_sparse_mla_decode_workspace_size": (c_size_t, [c_int, c_int, c_int]),
    "dsa_sparse_mla_decode_workspace_size_for": (c_size_t, [c_int, c_int, c_int, c_int]),
    "dsa_sparse_mla_decode": (c_int, [c_void_p, c_void_p, c_void_p, c_int, c_int, c_int, c_int, c_int, c_int,
                                      c_float, c_void_p, c_void_p, c_void_p, c_size_t, c_void_p]),
    "dsa_sparse_mla_decode_scratch_bytes": (c_size_t, []),
    "dsa_sparse_mla_decode_noalloc": (c_int, [c_void_p, c_void_p, c_void_p, c_int, c_int, c_int, c_int, c_int,
                                              c_int, c_float, c_void_p, c_void_p, c_void_p]),
    "dsa_sparse_mla_bwd_workspace_size": (c_size_t, [c_int, c_int, c_int, c_int]),
    "dsa_sparse_mla_bwd_workspace_size_chunked": (c_size_t, [c_int, c_int, c_int, c_int, c_int]),
    "dsa_sparse_mla_bwd": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_int,
                                   c_int, c_int, c_int, c_int, c_float, c_int, c_void_p, c_void_p, c_void_p,
                                   c_size_t, c_void_p]),
    "dsa_sparse_mla_bwd_workspace_size_ex": (c_size_t, [c_int, c_int, c_int, c_int, c_int, c_int]),
    "dsa_sparse_mla_bwd_ex": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_int,
                                      c_int, c_int, c_int, c_int, c_float, c_int, c_void_p, c_void_p, c_int,
                                      c_void_p, c_size_t, c_void_p, c_void_p]),
    "dsa_sparse_mla_bwd_timed": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_int,
                                         c_int, c_int, c_int, c_int, c_float, c_int, c_void_p, c_void_p,
                                         c_void_p, c_size_t, c_void_p, c_void_p]),
    "dsa_indexer_kl_target": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_int, c_int, c_int, c_int,
                                      c_float, c_int, c_void_p, c_void_p]),
    "dsa_indexer_kl_target_from_bwd": (c_int, [c_void_p, c_size_t, c_void_p, c_int, c_int, c_int, c_int, c_int,
                                               c_void_p, c_void_p]),
    "dsa_dense_attention_lse": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_int, c_int, c_int, c_float,
                                        c_void_p, c_void_p]),
    "dsa_dense_attention_target": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_int, c_int,
                                           c_int, c_int, c_float, c_void_p, c_void_p]),
    "dsa_dense_indexer_scores_bwd_workspace_size": (c_size_t, [c_int, c_int]),
    "dsa_dense_indexer_scores_bwd": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_int, c_int,
                                             c_int, c_void_p, c_int, c_void_p, c_void_p, c_void_p, c_void_p, c_size_t,
                                             c_void_p]),
    "dsa_v4_compress_fwd": (c_int, [c_void_p, c_void_p, c_int64, c_int64, c_void_p, c_void_p, c_void_p, c_int, c_int,
                                    c_int, c_int, c_int, c_int, c_int, c_float, c_void_p, c_void_p]),
    "dsa_v4_compress_bwd_workspace_size": (c_size_t, [c_int, c_int, c_int, c_int, c_int]),
    "dsa_v4_compress_bwd": (c_int, [c_void_p, c_void_p, c_int64, c_int64, c_void_p, c_void_p, c_void_p, c_int, c_int,
                                    c_int, c_int, c_int, c_int, c_int, c_int, c_float, c_void_p, c_void_p, c_void_p,
                                    c_int64, c_int64, c_void_p, c_void_p, c_void_p, c_size_t, c_void_p]),
    "dsa_v4_norm_rope": (c_int, [c_void_p, c_int64, c_int, c_int, c_int, c_void_p, c_void_p, c_int64, c_int, c_float,
                                 c_int, c_void_p, c_void_p]),
    "dsa_v4_norm_rope_bwd": (c_int, [c_void_p, c_void_p, c_int64, c_int, c_int, c_int, c_void_p, c_void_p, c_int64,
                                     c_int, c_float, c_int, c_void_p, c_void_p]),
    "dsa_v4_out_rope_group": (c_int, [c_void_p, c_int, c_int, c_int, c_int, c_int, c_void_p, c_void_p, c_int64, c_int,
                                      c_void_p, c_void_p]),
    "dsa_v4_out_rope_group_bwd": (c_int, [c_void_p, c_int, c_int, c_int, c_int, c_int, c_void_p, c_void_p, c_int64,
                                          c_int, c_void_p, c_void_p]),
    "dsa_indexer_kl_loss": (c_int, [c_void_p, c_void_p, c_void_p, c_int, c_int, c_int, c_int, c_float, c_void_p,
                                    c_void_p, c_void_p]),
    "dsa_indexer_selected_scores": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_int, c_int, c_int,
                                            c_int, c_int, c_void_p, c_void_p]),
    "dsa_indexer_scores_bwd_workspace_size": (c_size_t, [c_int, c_int, c_int]),
    "dsa_indexer_scores_bwd": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_int, c_int, c_int,
                                       c_int, c_int, c_void_p, c_void_p, c_void_p, c_void_p, c_size_t, c_void_p]),
}


class DSAError(RuntimeError):
    """A non-zero dsa_status returned by the C ABI."""

    def __init__(self, fn: str, status: int, msg: str):
        super().__init__(f"{fn} failed with status {status}: {msg}")
        self.status = status


_lib = None


def load() -> ctypes.CDLL:
    """Load (once) and return the library with typed entry points."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise ImportError(
            f"libdsa_amd.so not found at {LIB_PATH}. Build it with `python -c \"import __graft_entry__ as g; "
            f"g.build()\"` or `make -C mcore-bridge_amd/csrc` (needs hipcc, targets gfx950).")
    lib = ctypes.CDLL(LIB_PATH)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def strerror(status: int) -> str:
    return load().dsa_strerror(status).decode()


def check(fn: str, status: int) -> None:
    if status != DSA_OK:
        raise DSAError(fn, status, strerror(status))


def call(fn: str, *args) -> None:
    """Call an int-returning ABI entry point and raise DSAError on failure."""
    check(fn, getattr(load(), fn)(*args))
