"""ctypes binding of ``libdsa_amd.so`` (the C ABI declared in include/dsa_amd.h).

The product path has no fallback: if the library is missing or fails to load,
importing an op raises. Build it with ``python -m nanoengine_amd.build``.
"""
from __future__ import annotations

import ctypes
import os
from ctypes import c_float, c_int, c_int64, c_size_t, c_void_p
from pathlib import Path

# DSA_AMD_LIB may name another build of the same library (a variant under test)
LIB_PATH = Path(os.environ.get("DSA_AMD_LIB", Path(__file__).resolve().parent / "libdsa_amd.so"))

# name -> (restype, argtypes); mirrors include/dsa_amd.h one to one.
_P = c_void_p
SIGNATURES = {
    "dsa_version": (c_int, []),
    "dsa_last_error": (ctypes.c_char_p, []),
    "dsa_num_cus": (c_int, [c_int]),
    "dsa_topk_max_len": (c_int, []),
    "dsa_indexer_schedule": (c_int, [_P, c_int, c_int, c_int, _P, _P]),
    "dsa_indexer_logits": (c_int, [_P, _P, _P, _P, _P, c_int64, c_int, c_int, c_int, c_int, c_int,
                                   c_int64, _P, c_int64, _P]),
    "dsa_indexer_topk_workspace_bytes": (c_size_t, [c_int, c_int, c_int64]),
    "dsa_indexer_topk": (c_int, [_P, _P, _P, _P, _P, c_int64, c_int, c_int, c_int, c_int, c_int, c_int64, c_int,
                                 _P, _P, _P, c_size_t, _P, _P]),
    "dsa_topk_workspace_bytes": (c_size_t, [c_int]),
    "dsa_topk_transform": (c_int, [_P, c_int64, _P, _P, c_int64, _P, _P, c_int, c_int64, c_int, c_int, _P,
                                   c_size_t, _P]),
    "dsa_topk_transform_noalloc": (c_int, [_P, c_int64, _P, _P, c_int64, _P, _P, c_int, c_int64, c_int, c_int,
                                           _P]),
    "dsa_indexer_select": (c_int, [_P, c_int64, _P, _P, c_int, c_int64, c_int, _P, c_size_t, _P]),
    "dsa_topk_transform_ragged": (c_int, [_P, c_int64, _P, _P, _P, _P, c_int, c_int64, c_int, _P, c_size_t,
                                          _P]),
    "dsa_topk_to_physical": (c_int, [_P, c_int64, _P, c_int64, c_int, c_int, c_int, c_int, c_int, _P, _P]),
    "dsa_sparse_mla_num_splits": (c_int, [c_int, c_int, c_int, c_int]),
    "dsa_sparse_mla_workspace_bytes": (c_size_t, [c_int, c_int, c_int]),
    "dsa_sparse_mla_decode": (c_int, [_P, c_int64, c_int64, _P, c_int64, c_int, c_int64, _P, c_int64, c_int,
                                      c_int, c_int, c_float, _P, _P, c_int, _P, c_size_t, _P]),
    "dsa_mla_kv_store": (c_int, [_P, c_int64, _P, c_int, c_int, _P, c_int64, c_int, _P]),
    "dsa_indexer_k_store": (c_int, [_P, c_int64, _P, c_int, c_int, _P, c_int, _P]),
    "dsa_indexer_q_prologue": (c_int, [_P, _P, c_int64, c_float, _P, c_int64, _P, c_int, c_int, c_int, c_int, _P,
                                       _P, _P]),
    "dsa_mqa_logits": (c_int, [_P, _P, _P, _P, c_int64, _P, _P, c_int, c_int64, c_int, _P, c_int64, c_int64, c_int,
                               _P]),
    "dsa_mqa_topk_workspace_bytes": (c_size_t, [c_int, c_int64, c_int]),
    "dsa_mqa_topk": (c_int, [_P, _P, _P, _P, c_int64, _P, _P, c_int, c_int64, c_int, c_int64, c_int, _P, _P, c_size_t,
                             _P]),
    "dsa_sparse_mla_prefill": (c_int, [_P, c_int64, c_int64, _P, c_int64, c_int64, _P, c_int64, c_int, c_int, c_int,
                                       c_float, _P, _P, _P, _P]),
    "dsa_gather_indexer_cache": (c_int, [_P, c_int64, c_int, c_int, _P, c_int64, _P, c_int, c_int, c_int64, _P, _P,
                                         _P]),
    "dsa_sparse_mla_prefill_paged_workspace_bytes": (c_size_t, [c_int, c_int]),
    "dsa_sparse_mla_prefill_paged": (c_int, [_P, c_int64, c_int64, _P, c_int64, c_int, c_int64, _P, c_int64, c_int,
                                             _P, _P, c_int, c_int, c_int64, _P, c_int64, c_int64, _P, c_int64, c_int, c_int,
                                             c_int, c_float, _P, _P, _P, _P, c_size_t, _P]),
    "dsa_mla_prefill_kv": (c_int, [_P, c_int64, c_int, c_int64, _P, c_int64, c_int, _P, _P, c_int, c_int, c_int64,
                                   _P, c_int64, _P, c_int64, _P]),
    "dsa_prefill_windows": (c_int, [_P, _P, c_int, c_int, c_int, c_int, _P, _P, _P, _P]),
    "dsa_indexer_k_transform_store": (c_int, [_P, c_int64, _P, _P, c_float, _P, c_int64, _P, c_int, _P, c_int,
                                              c_int, _P, c_int, _P]),
}

_lib = None


class DsaError(RuntimeError):
    """A non-zero status from the C ABI."""


def load() -> ctypes.CDLL:
    """Load (once) and return the library; raise ImportError if absent."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise ImportError(
                f"{LIB_PATH} is missing: build it with `python -m nanoengine_amd.build` "
                "(the DSA path has no CPU fallback)")
        lib = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
    return _lib


def check(status: int, what: str) -> None:
    if status != 0:
        msg = load().dsa_last_error().decode(errors="replace")
        if status == 1:
            raise ValueError(f"{what}: {msg}")
        raise DsaError(f"{what} failed (status {status}): {msg}")


def call(name: str, *args) -> None:
    check(getattr(load(), name)(*args), name)
