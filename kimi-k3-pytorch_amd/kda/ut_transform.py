"""UT transform of independent chunks on the gfx950 backend.

Drop-in for ``ut_transform`` / ``UTTransformOutput``
(src/kda/ut_transform.py:12-20, 61-92).  ``M`` is returned as ``[B,H,C,C]``;
U/W/log_gamma/k_gamma keep the canonical ``[B,C,H,*]`` layout.  The kernel
computes in f32 (f64 for f64 inputs) and the results are returned in the
input dtype, as the reference (which does not upcast here) returns them.
The result does not depend on ``secondary_tile_size`` (the reference pins
that bit-exactly, tests/kda/test_kda_ut_transform.py:94-103).
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from . import _lib, _prep


@dataclass
class UTTransformOutput:
    """Upper-triangular transformed tensors used by chunkwise KDA."""

    M: torch.Tensor
    U: torch.Tensor
    W: torch.Tensor
    log_gamma: torch.Tensor
    k_gamma: torch.Tensor


def ut_transform(
    k: torch.Tensor,
    v: torch.Tensor,
    g: torch.Tensor,
    beta: torch.Tensor,
    secondary_tile_size: int = 16,
) -> UTTransformOutput:
    """Public UT transform for canonical ``[B,C,H,*]`` inputs."""
    if k.ndim != 4 or g.shape != k.shape:
        raise ValueError("k and g must have shape [B,C,H,K]")
    if v.ndim != 4 or v.shape[:3] != k.shape[:3]:
        raise ValueError("v must have shape [B,C,H,V]")
    if beta.shape != k.shape[:3]:
        raise ValueError("beta must have shape [B,C,H]")
    if secondary_tile_size <= 0:
        raise ValueError("tile_size must be > 0")
    _lib.require_gpu(k)
    _prep.reject_autograd(k, v, g, beta)
    lib = _lib.load()
    batch, count, heads, key_dim = k.shape
    value_dim = v.shape[-1]
    dtypes = {t.dtype for t in (k, v, g, beta)}
    arith = torch.float64 if torch.float64 in dtypes else torch.float32
    if len(dtypes) == 1 and next(iter(dtypes)) in (torch.bfloat16, torch.float16, torch.float32, torch.float64):
        kernel_dtype = next(iter(dtypes))
    else:
        kernel_dtype = arith
    kc, vc, gc, bc = (t.to(kernel_dtype).contiguous() for t in (k, v, g, beta))
    device = k.device
    M = torch.empty(batch, heads, count, count, dtype=arith, device=device)
    U = torch.empty(batch, count, heads, value_dim, dtype=arith, device=device)
    W = torch.empty(batch, count, heads, key_dim, dtype=arith, device=device)
    lg = torch.empty(batch, count, heads, key_dim, dtype=arith, device=device)
    kg = torch.empty(batch, count, heads, key_dim, dtype=arith, device=device)
    status = lib.kda_ut_transform(
        kc.data_ptr(), vc.data_ptr(), gc.data_ptr(), bc.data_ptr(), _lib.dtype_code(kernel_dtype),
        M.data_ptr(), U.data_ptr(), W.data_ptr(), lg.data_ptr(), kg.data_ptr(), _lib.dtype_code(arith),
        batch, count, heads, key_dim, value_dim, _prep.stream(device),
    )
    _lib.check(status)
    result_dtype = k.dtype
    cast = (lambda x: x) if result_dtype == arith else (lambda x: x.to(result_dtype))
    return UTTransformOutput(M=cast(M), U=cast(U), W=cast(W), log_gamma=cast(lg), k_gamma=cast(kg))
