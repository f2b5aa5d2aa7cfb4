"""ctypes binding of the C restatement (dsa_ref.c) -- TEST INFRASTRUCTURE ONLY."""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np
import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "_build", "liboracle_dsa.so")
_lib = None


def build() -> str:
    """Compile dsa_ref.c with the committed Makefile (always rebuilds)."""
    subprocess.check_call(["make", "-s", "-B", "-C", _HERE])
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        L.oracle_e4m3_encode.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64]
        L.oracle_e4m3_decode.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64]
        L.oracle_topk_rows.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_int64,
                                       ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p]
        L.oracle_topk_rows.restype = ctypes.c_int
        _lib = L
    return _lib


def e4m3_encode(x: torch.Tensor) -> torch.Tensor:
    a = np.ascontiguousarray(x.detach().cpu().to(torch.float32).numpy())
    out = np.empty(a.shape, dtype=np.uint8)
    lib().oracle_e4m3_encode(a.ctypes.data, out.ctypes.data, a.size)
    return torch.from_numpy(out)


def e4m3_decode(b: torch.Tensor) -> torch.Tensor:
    a = np.ascontiguousarray(b.detach().cpu().numpy().astype(np.uint8))
    out = np.empty(a.shape, dtype=np.float32)
    lib().oracle_e4m3_decode(a.ctypes.data, out.ctypes.data, a.size)
    return torch.from_numpy(out)


def topk_rows(score: torch.Tensor, seq_lens: torch.Tensor, k: int) -> torch.Tensor:
    s = np.ascontiguousarray(score.detach().cpu().to(torch.float32).numpy())
    sl = np.ascontiguousarray(seq_lens.detach().cpu().to(torch.int32).numpy().reshape(-1))
    R, W = s.shape
    out = np.empty((R, k), dtype=np.int32)
    rc = lib().oracle_topk_rows(s.ctypes.data, R, W, sl.ctypes.data, k, out.ctypes.data)
    if rc != 0:
        raise RuntimeError("oracle_topk_rows failed")
    return torch.from_numpy(out)
