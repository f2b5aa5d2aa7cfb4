"""ctypes loader of libmi355_dsa.so (the HIP kernels behind a C ABI).

The library is loaded after `import torch` so that its NEEDED
libamdhip64.so.7 resolves to the HIP runtime torch already mapped: one
runtime per process, and torch's stream handles are valid in the library.
There is no fallback: a missing library raises.
"""
from __future__ import annotations

import ctypes
import os

import torch  # noqa: F401  (must precede the CDLL load, see module doc)

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(PKG_DIR, "libmi355_dsa.so")

_c_int = ctypes.c_int
_c_i64 = ctypes.c_int64
_c_f32 = ctypes.c_float
_c_size = ctypes.c_size_t
_p = ctypes.c_void_p

# name -> (restype, argtypes); mirrors include/mi355_dsa.h
SIGNATURES = {
    "mi355_dsa_last_error": (ctypes.c_char_p, []),
    "mi355_dsa_abi_version": (_c_int, []),
    "mi355_dsa_selfcheck": (_c_int, [_p]),
    "mi355_dsa_indexer_k_store": (_c_int, [_p, _c_int, _c_i64, _p, _c_i64, _c_int, _p, _p]),
    "mi355_dsa_mla_decode_workspace_size": (_c_size, [_c_int, _c_int, _c_int]),
    "mi355_dsa_mla_decode": (_c_int, [_p, _p, _p, _c_int, _c_int, _p, _c_i64, _c_int, _p, _c_int,
                                      _p, _c_f32, _p, _c_size, _p]),
    "mi355_dsa_varlen_attention": (_c_int, [_p, _p, _p, _p, _p, _c_int, _c_int, _c_int, _c_int,
                                            _c_int, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64,
                                            _c_i64, _c_i64, _c_i64, _p, _p, _c_int, _c_int,
                                            _c_f32, _c_int, _p]),
    "mi355_dsa_indexer_shard_merge": (_c_int, [_p, _c_i64, _c_i64, _p, _c_int, _c_int, _c_int,
                                               _p, _c_int, _p]),
    "mi355_dsa_head_proj": (_c_int, [_p, _c_i64, _c_i64, _p, _c_i64, _c_i64, _p, _c_int, _c_int,
                                     _c_int, _c_int, _c_int, _p]),
    "mi355_dsa_concat_and_cache_mla": (_c_int, [_p, _c_int, _c_i64, _p, _c_i64, _p, _c_i64,
                                                _c_int, _c_i64, _p, _c_int, _p]),
    "mi355_dsa_decode_layer_attention": (_c_int, [_p, _c_i64, _p, _p, _p, _c_int, _c_int, _p,
                                                  _c_int, _c_i64, _c_int, _p, _c_int, _p, _c_int,
                                                  _p, _c_f32, _p, _c_int, _p, _c_size, _p]),
    "mi355_dsa_decode_layer_prologue": (_c_int, [_p, _c_i64, _c_i64, _p, _c_i64, _c_i64, _p,
                                                 _c_int, _c_int, _c_int, _c_int, _c_int,
                                                 _p, _c_int, _c_i64, _p, _c_i64, _p, _c_i64,
                                                 _c_int, _p, _c_int, _p, _c_int, _c_i64, _p, _p,
                                                 _p, _c_i64, _p]),
    "mi355_dsa_decode_layer_indexer": (_c_int, [_c_int, _p, _c_int, _c_i64, _p, _c_i64, _p,
                                                _c_i64, _c_int, _p, _c_int, _p, _c_int, _c_i64,
                                                _p, _p, _p, _c_int, _c_int, _p, _p, _c_int, _p,
                                                _c_int, _p, _p, _p]),
    "mi355_dsa_indexer_logits": (_c_int, [_p, _c_int, _c_int, _p, _c_int, _c_int, _p, _c_int,
                                          _c_i64, _c_int, _p, _p, _c_int, _p, _p, _p]),
    "mi355_dsa_indexer_logits_packed": (_c_int, [_p, _c_int, _c_int, _p, _p, _c_int, _c_i64,
                                                 _c_int, _p, _p, _c_int, _p, _p]),
    "mi355_dsa_decode_topk_workspace_size": (_c_size, [_c_int, _c_int, _c_int]),
    "mi355_dsa_decode_topk": (_c_int, [_p, _p, _p, _p, _c_int, _c_int, _c_int, _p, _c_size, _p]),
    "mi355_dsa_decode_layer_topk": (_c_int, [_p, _p, _p, _p, _c_int, _c_int, _c_int, _p,
                                             _c_size, _p, _c_i64, _c_i64, _p, _c_i64, _c_i64,
                                             _p, _c_int, _c_int, _c_int, _c_int, _c_int, _p]),
    "mi355_dsa_persistent_topk_workspace_size": (_c_size, [_c_int, _c_int, _c_int]),
    "mi355_dsa_persistent_topk": (_c_int, [_p, _c_int, _c_int, _p, _p, _c_int, _c_int, _p,
                                           _c_size, _p]),
    "mi355_dsa_sparse_mla_workspace_size": (_c_size, [_c_int, _c_int, _c_int]),
    "mi355_dsa_sparse_mla_decode": (_c_int, [_p, _p, _p, _c_int, _c_int, _p, _c_int, _c_i64,
                                             _c_int, _p, _c_int, _p, _c_int, _p, _c_f32, _p,
                                             _c_size, _p]),
    "mi355_dsa_sparse_mla_noalloc_max_bytes": (_c_size, []),
    "mi355_dsa_sparse_mla_decode_noalloc": (_c_int, [_p, _p, _p, _c_int, _c_int, _p, _c_int,
                                                     _c_i64, _c_int, _p, _c_int, _p, _c_int, _p,
                                                     _c_f32, _p]),
    "mi355_dsa_attn_fp8_gemv": (_c_int, [_p, _p, _p, _p, _c_int, _c_int, _c_int, _p]),
    "mi355_dsa_attn_fp8_dequant": (_c_int, [_p, _p, _p, _c_int, _c_int, _p]),
    "mi355_dsa_attn_fp8_quantize": (_c_int, [_p, _p, _p, _c_int, _c_int, _p]),
}

_lib = None


def lib() -> ctypes.CDLL:
    """Loads (once) and returns the library; raises if it is not built."""
    global _lib
    if _lib is None:
        path = os.environ.get("MI355_DSA_LIB", LIB_PATH)
        if not os.path.exists(path):
            raise RuntimeError(
                f"{path} is missing: build the HIP library first "
                "(python glm5-on-v100_amd/build.py or __graft_entry__.build())")
        L = ctypes.CDLL(path)
        missing = [n for n in SIGNATURES if not hasattr(L, n)]
        if missing:
            raise RuntimeError(f"{path} lacks entry points {missing}: rebuild it")
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def last_error() -> str:
    msg = lib().mi355_dsa_last_error()
    return msg.decode() if msg else ""


def call(name: str, *args) -> None:
    """Calls an int-returning entry point; raises RuntimeError on failure."""
    rc = getattr(lib(), name)(*args)
    if rc != 0:
        raise RuntimeError(f"{last_error()} [{name}, rc={rc}]")
