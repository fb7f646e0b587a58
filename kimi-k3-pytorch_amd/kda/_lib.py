"""ctypes binding of ``libkda_mi355x.so`` (C ABI in include/kda_mi355x.h).

The library is built in-tree by ``kimi-k3-pytorch_amd/build_lib.py``.  When it
is missing or fails to load, every operator raises ``RuntimeError``: there is no
CPU or eager-PyTorch fallback.
"""

from __future__ import annotations

import ctypes
import threading
from pathlib import Path

import torch

LIB_PATH = Path(__file__).resolve().with_name("libkda_mi355x.so")
ABI_VERSION = 10

KDA_OK = 0
KDA_ERR_INVALID_ARGUMENT = 1
KDA_ERR_UNSUPPORTED = 2
KDA_ERR_WORKSPACE = 3
KDA_ERR_LAUNCH = 4

# KDA_NOALLOC_SCRATCH_BYTES: the static device scratch of kda_chunk_fwd_noalloc
NOALLOC_SCRATCH_BYTES = 128 << 20

DTYPE_CODES = {
    torch.float32: 0,
    torch.float16: 1,
    torch.bfloat16: 2,
    torch.float64: 3,
}

# Every exported symbol with (restype, argtypes); include/kda_mi355x.h is the source of truth.
_P = ctypes.c_void_p
_I = ctypes.c_int
_L = ctypes.c_int64
_S = ctypes.c_size_t
SIGNATURES = {
    "kda_abi_version": (_I, []),
    "kda_status_string": (ctypes.c_char_p, [_I]),
    "kda_recurrent_fwd": (
        _I,
        [_P, _P, _P, _P, _P, _I, _P, _P, _I, _P, _P, _P, _L, _P, _L, _L, _L, _L, _L, _P],
    ),
    "kda_decode_step": (_I, [_P, _P, _P, _P, _P, _I, _P, _P, _I, _P, _L, _L, _L, _L, _P]),
    "kda_chunk_fwd_workspace_bytes": (_S, [_L, _L, _L, _L, _L, _L, _I]),
    "kda_chunk_fwd_plan": (_I, [_L, _L, _L, _L, _L, _L, _I, _P, _P]),
    "kda_set_segment_chunks": (_I, [_L]),
    "kda_chunk_fwd": (
        _I,
        [_P, _P, _P, _P, _P, _I, _P, _P, _I, _P, _P, _L, _P, _L, _L, _L, _L, _L, _P, _S, _P],
    ),
    "kda_chunk_fwd_decay": (
        _I,
        [_P, _P, _P, _P, _P, _P, ctypes.c_double, _P, _I, _P, _P, _I, _P, _P, _L, _P, _L, _L, _L, _L, _L, _P, _S,
         _P],
    ),
    "kda_chunk_fwd_noalloc": (
        _I,
        [_P, _P, _P, _P, _P, _I, _P, _P, _I, _P, _P, _L, _P, _L, _L, _L, _L, _L, _P],
    ),
    "kda_chunk_fwd_profiled": (
        _I,
        [_P, _P, _P, _P, _P, _I, _P, _P, _I, _P, _P, _L, _P, _L, _L, _L, _L, _L, _P, _S, _P, _P, _P],
    ),
    "kda_ut_transform": (_I, [_P, _P, _P, _P, _I, _P, _P, _P, _P, _P, _I, _L, _L, _L, _L, _L, _P]),
    "kda_conv_silu_fwd": (
        _I,
        [_P, _P, _P, _P, _P, _P, _P, _L, _L, _L, _L, _L, _I, ctypes.c_double, _I, _P],
    ),
    "kda_gates_fwd": (
        _I,
        [_P, _P, _P, ctypes.c_double, _P, _P, _P, _P, _L, _L, _L, _I, _P],
    ),
    "kda_rmsnorm_gate_fwd": (_I, [_P, _P, _I, _P, _P, _L, _L, _L, ctypes.c_double, _I, _P]),
    "kda_conv_silu_bwd": (_I, [_P] * 11 + [_L] * 5 + [_I, ctypes.c_double, _I, _P]),
    "kda_gates_bwd": (_I, [_P, _P, _P, ctypes.c_double] + [_P] * 8 + [_L, _L, _L, _I, _P]),
    "kda_rmsnorm_gate_bwd": (_I, [_P, _P, _I, _P, _P, _P, _P, _P, _L, _L, _L, ctypes.c_double, _I, _P]),
    "kda_ut_transform_bwd_workspace_bytes": (_S, [_L, _L, _L, _L, _I]),
    "kda_ut_transform_bwd": (_I, [_P, _P, _P, _P, _I] + [_P] * 9 + [_I, _L, _L, _L, _L, _L, _P, _S, _P]),
    "kda_chunk_bwd_workspace_bytes": (_S, [_L, _L, _L, _L, _L, _I]),
    "kda_chunk_bwd": (
        _I,
        [_P, _P, _P, _P, _P, _P, _I, _P, _P, _P, _P, _P, _P, _P, _P, _L, _L, _L, _L, _L, _P, _S, _P],
    ),
    "kda_chunk_grad_tangent_workspace_bytes": (_S, [_L, _L, _L, _L, _L]),
    "kda_chunk_grad_tangent": (_I, [_P] * 22 + [_L] * 5 + [_P, _S, _P]),
    "kda_cache_gather": (_I, [_P, _P, _P, _I, _P, _L, _L, _P, _P]),
    "kda_recurrent_bwd_workspace_bytes": (_S, [_L, _L, _L, _L, _I]),
    "kda_recurrent_bwd": (_I, [_P] * 16 + [_L] * 5 + [_I, _P, _S, _P]),
}

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None


def load() -> ctypes.CDLL:
    """Load and type the shared library once (raises RuntimeError if absent)."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"{LIB_PATH.name} is not built; run `python kimi-k3-pytorch_amd/build_lib.py` "
                "(the MI355X KDA backend has no fallback path)"
            )
        lib = ctypes.CDLL(str(LIB_PATH))
        for name, (restype, argtypes) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = restype
            fn.argtypes = argtypes
        version = lib.kda_abi_version()
        if version != ABI_VERSION:
            raise RuntimeError(f"{LIB_PATH.name} ABI version {version} != expected {ABI_VERSION}")
        _lib = lib
    return _lib


def check(status: int) -> None:
    if status != KDA_OK:
        text = load().kda_status_string(status).decode(errors="replace")
        raise RuntimeError(f"kda_mi355x: {text}")


def set_segment_chunks(chunks_per_segment: int) -> None:
    """Force the MFMA prefill's segment length (process-wide): L >= 1 chunks
    per segment, 0 one segment per sequence, -1 the library's own plan."""
    check(load().kda_set_segment_chunks(int(chunks_per_segment)))


def dtype_code(dtype: torch.dtype) -> int:
    try:
        return DTYPE_CODES[dtype]
    except KeyError:
        raise TypeError(f"unsupported dtype {dtype} for the MI355X KDA backend") from None


def ptr(tensor: torch.Tensor | None) -> int | None:
    return None if tensor is None else tensor.data_ptr()


def stream_of(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def require_gpu(tensor: torch.Tensor) -> None:
    if tensor.device.type != "cuda":
        raise RuntimeError(
            "the MI355X KDA backend runs on ROCm GPU tensors only "
            f"(got a tensor on {tensor.device})"
        )
