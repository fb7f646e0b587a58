"""UT transform of independent chunks on the gfx950 backend.

Drop-in for ``ut_transform`` / ``UTTransformOutput``
(src/kda/ut_transform.py:12-20, 61-92).  ``M`` is returned as ``[B,H,C,C]``;
U/W/log_gamma/k_gamma keep the canonical ``[B,C,H,*]`` layout.  The kernel
computes in f32 (f64 for f64 inputs) and the results are returned in the
input dtype, as the reference (which does not upcast here) returns them.
The result does not depend on ``secondary_tile_size`` (the reference pins
that bit-exactly, tests/kda/test_kda_ut_transform.py:94-103).  Under autograd
the backward is ``kda_ut_transform_bwd`` (the reference's transform is plain
torch and differentiable).
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
    result_dtype = k.dtype
    cast = (lambda x: x) if result_dtype == _arith(k, v, g, beta) else (lambda x: x.to(result_dtype))
    if torch.is_grad_enabled() and any(t.requires_grad for t in (k, v, g, beta)):
        M, U, W, lg, kg = _UTTransformFunction.apply(k, v, g, beta)
    else:
        M, U, W, lg, kg = _forward(k, v, g, beta)
    return UTTransformOutput(M=cast(M), U=cast(U), W=cast(W), log_gamma=cast(lg), k_gamma=cast(kg))


def _arith(*tensors) -> torch.dtype:
    return torch.float64 if any(t.dtype == torch.float64 for t in tensors) else torch.float32


def _kernel_inputs(k, v, g, beta):
    dtypes = {t.dtype for t in (k, v, g, beta)}
    arith = _arith(k, v, g, beta)
    if len(dtypes) == 1 and next(iter(dtypes)) in (torch.bfloat16, torch.float16, torch.float32, torch.float64):
        kernel_dtype = next(iter(dtypes))
    else:
        kernel_dtype = arith
    return tuple(t.to(kernel_dtype).contiguous() for t in (k, v, g, beta)), kernel_dtype, arith


def _forward(k, v, g, beta):
    """M, U, W, log_gamma, k_gamma in the arithmetic type (f32, f64 for f64)."""
    lib = _lib.load()
    batch, count, heads, key_dim = k.shape
    value_dim = v.shape[-1]
    (kc, vc, gc, bc), kernel_dtype, arith = _kernel_inputs(k, v, g, beta)
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
    return M, U, W, lg, kg


class _UTTransformFunction(torch.autograd.Function):
    """ut_transform under autograd: the native forward and ``kda_ut_transform_bwd``
    (the gradients autograd takes through src/kda/ut_transform.py:23-92)."""

    @staticmethod
    def forward(ctx, k, v, g, beta):
        ctx.save_for_backward(k, v, g, beta)
        return _forward(k, v, g, beta)

    @staticmethod
    @torch.autograd.function.once_differentiable
    def backward(ctx, dM, dU, dW, dlg, dkg):
        k, v, g, beta = ctx.saved_tensors
        lib = _lib.load()
        (kc, vc, gc, bc), kernel_dtype, arith = _kernel_inputs(k, v, g, beta)
        batch, count, heads, key_dim = k.shape
        value_dim = v.shape[-1]
        up = lambda t: None if t is None else t.to(arith).contiguous()  # noqa: E731
        dM, dU, dW, dlg, dkg = (up(t) for t in (dM, dU, dW, dlg, dkg))
        dk, dg = torch.empty_like(kc, dtype=arith), torch.empty_like(gc, dtype=arith)
        dv, db = torch.empty_like(vc, dtype=arith), torch.empty_like(bc, dtype=arith)
        ws_bytes = lib.kda_ut_transform_bwd_workspace_bytes(batch, count, heads, key_dim, _lib.dtype_code(arith))
        ws = _prep.workspace(ws_bytes, k.device, "the ut_transform backward")
        _lib.check(lib.kda_ut_transform_bwd(
            kc.data_ptr(), vc.data_ptr(), gc.data_ptr(), bc.data_ptr(), _lib.dtype_code(kernel_dtype),
            _lib.ptr(dM), _lib.ptr(dU), _lib.ptr(dW), _lib.ptr(dlg), _lib.ptr(dkg), dk.data_ptr(), dv.data_ptr(),
            dg.data_ptr(), db.data_ptr(), _lib.dtype_code(arith), batch, count, heads, key_dim, value_dim,
            _lib.ptr(ws), ws_bytes, _prep.stream(k.device),
        ))
        return dk.to(k.dtype), dv.to(v.dtype), dg.to(g.dtype), db.to(beta.dtype)
