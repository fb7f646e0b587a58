"""Chunkwise-parallel KDA prefill on the gfx950 backend.

Drop-in for ``chunkwise_kda`` (src/kda/chunkwise.py:17-107): same signature,
defaults, validation errors and dtype rules.  The kernels use a fixed
64-token chunk with 16-row sub-tiles internally; the exact chunkwise
algorithm's result does not depend on ``chunk_size`` or
``secondary_tile_size`` (the reference pins that invariance in
tests/kda/test_kda_chunkwise_equivalence.py:42-57 and
tests/kda/test_kda_ut_transform.py:94-103), so both are validated exactly as
the reference does and otherwise only select nothing.

Additive keyword-only extension: ``cu_seqlens`` (packed documents
``[1, sum T, H, *]``, state reset at every document start, per-document
``initial_state``/``final_state`` of shape ``[N,H,K,V]``).
"""

from __future__ import annotations

import torch

from . import _lib, _prep
from .recurrent import KDAOperatorOutput
from .utils import accumulation_dtype, validate_core_inputs, validate_cu_seqlens


def chunkwise_kda(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    g: torch.Tensor,
    beta: torch.Tensor,
    initial_state: torch.Tensor | None = None,
    output_final_state: bool = False,
    attention_mask: torch.Tensor | None = None,
    *,
    chunk_size: int = 64,
    secondary_tile_size: int = 16,
    accumulate_state_in_fp32: bool = True,
    cu_seqlens: torch.Tensor | list[int] | None = None,
) -> KDAOperatorOutput:
    """Exact chunkwise KDA using UT/WY parallel computation within each chunk."""
    if chunk_size <= 0 or secondary_tile_size <= 0:
        raise ValueError("chunk_size and secondary_tile_size must be > 0")
    if secondary_tile_size > chunk_size:
        raise ValueError("secondary_tile_size must be <= chunk_size")
    offsets = None
    if cu_seqlens is not None:
        offsets = validate_cu_seqlens(cu_seqlens, q.shape[0] if q.ndim == 4 else -1,
                                      q.shape[1] if q.ndim == 4 else -1, attention_mask)
    num_states = None if offsets is None else len(offsets) - 1
    batch, tokens, heads, key_dim, value_dim = validate_core_inputs(
        q, k, v, g, beta, initial_state, attention_mask, num_states=num_states
    )
    _lib.require_gpu(q)
    _prep.reject_autograd(q, k, v, g, beta, initial_state)
    lib = _lib.load()

    work_dtype = accumulation_dtype(v.dtype, accumulate_state_in_fp32)
    (qc, kc, vc, gc, bc), kernel_dtype, arith = _prep.kernel_inputs(q, k, v, g, beta, work_dtype)
    device = q.device
    n_seq = batch if offsets is None else len(offsets) - 1
    total = batch * tokens
    s_in = _prep.state_arg(initial_state, arith)
    s_out = (
        torch.empty(n_seq, heads, key_dim, value_dim, dtype=arith, device=device)
        if output_final_state
        else None
    )
    out = torch.empty(batch, tokens, heads, value_dim, dtype=kernel_dtype, device=device)
    cu = None if offsets is None else _prep.cu_tensor(offsets, device)
    valid = _prep.valid_lengths(attention_mask, device)
    code = _lib.dtype_code(kernel_dtype)
    ws_bytes = lib.kda_chunk_fwd_workspace_bytes(n_seq, total, heads, key_dim, value_dim, code)
    workspace = torch.empty(ws_bytes, dtype=torch.uint8, device=device) if ws_bytes else None
    status = lib.kda_chunk_fwd(
        qc.data_ptr(), kc.data_ptr(), vc.data_ptr(), gc.data_ptr(), bc.data_ptr(), code,
        _lib.ptr(s_in), _lib.ptr(s_out), _lib.dtype_code(arith), out.data_ptr(),
        _lib.ptr(cu), tokens, _lib.ptr(valid), n_seq, total, heads, key_dim, value_dim,
        _lib.ptr(workspace), ws_bytes, _prep.stream(device),
    )
    _lib.check(status)
    hidden = out if out.dtype == v.dtype else out.to(v.dtype)
    final = None
    if s_out is not None:
        final = s_out if s_out.dtype == work_dtype else s_out.to(work_dtype)
    return KDAOperatorOutput(hidden_states=hidden, final_state=final)
