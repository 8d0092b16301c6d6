"""ctypes binding of the C restatement c/kv_attn_ref.c.

TEST INFRASTRUCTURE ONLY (checker and CPU baseline; see oracle/__init__.py).
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle_kv.so")

_lib = None


def build() -> str:
    subprocess.run(["make", "-B", "-C", HERE, "liboracle_kv.so"], check=True,
                   capture_output=True, text=True)
    return LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = ctypes.CDLL(LIB_PATH)
        L.oracle_threads.restype = ctypes.c_int
        L.oracle_decode_attn.restype = None
        P = ctypes.c_void_p
        I = ctypes.c_int
        L.oracle_decode_attn.argtypes = [P, P, P, P, P, I, I, I, I, I, I, P]
        _lib = L
    return _lib


def threads() -> int:
    return lib().oracle_threads()


def decode_attn(q: np.ndarray, k_cache: np.ndarray, v_cache: np.ndarray, lens: np.ndarray,
                cache_bf16: bool) -> np.ndarray:
    """q [B,Hq,D] fp32; caches [B,T_cap,Hkv,D] fp32 or uint16 bf16 bits."""
    q = np.ascontiguousarray(q, dtype=np.float32)
    k = np.ascontiguousarray(k_cache)
    v = np.ascontiguousarray(v_cache)
    lens = np.ascontiguousarray(lens, dtype=np.int32)
    B, Hq, D = q.shape
    T_cap, Hkv = k.shape[1], k.shape[2]
    out = np.empty_like(q)
    scratch = np.empty(threads() * T_cap, dtype=np.float32)
    lib().oracle_decode_attn(out.ctypes.data, q.ctypes.data, k.ctypes.data, v.ctypes.data,
                             lens.ctypes.data, B, Hq, Hkv, D, T_cap, int(cache_bf16),
                             scratch.ctypes.data)
    return out
