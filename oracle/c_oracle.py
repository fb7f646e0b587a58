"""ctypes loader for the scalar C oracle (oracle/kda_recurrent_ref.c).

TEST INFRASTRUCTURE ONLY.  Builds the library with `make -C oracle` on first
use if it is missing."""

from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent
LIB = HERE / "build" / "libkda_oracle.so"
_lib = None


def build() -> Path:
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return LIB


def _load():
    global _lib
    if _lib is None:
        if not LIB.exists():
            build()
        lib = ctypes.CDLL(str(LIB))
        dp = ctypes.POINTER(ctypes.c_double)
        lp = ctypes.POINTER(ctypes.c_long)
        lib.kda_recurrent_ref.restype = None
        lib.kda_recurrent_ref.argtypes = [dp, dp, dp, dp, dp, dp, lp, dp, dp] + [ctypes.c_long] * 5
        _lib = lib
    return _lib


def recurrent_ref(q, k, v, g, beta, initial_state=None, valid=None):
    """float64 recurrence; returns (out [B,T,H,V], final state [B,H,K,V]) as torch tensors."""
    lib = _load()
    B, T, H, K = q.shape
    V = v.shape[-1]
    arrs = [np.ascontiguousarray(t.detach().double().cpu().numpy()) for t in (q, k, v, g, beta)]
    s0 = None if initial_state is None else np.ascontiguousarray(initial_state.detach().double().cpu().numpy())
    vl = None if valid is None else np.ascontiguousarray(np.asarray(valid, dtype=np.int64))
    out = np.zeros((B, T, H, V))
    sf = np.zeros((B, H, K, V))
    dp = ctypes.POINTER(ctypes.c_double)
    as_d = lambda a: None if a is None else a.ctypes.data_as(dp)  # noqa: E731
    lib.kda_recurrent_ref(*(as_d(a) for a in arrs), as_d(s0),
                          None if vl is None else vl.ctypes.data_as(ctypes.POINTER(ctypes.c_long)),
                          as_d(out), as_d(sf), B, T, H, K, V)
    return torch.from_numpy(out), torch.from_numpy(sf)
