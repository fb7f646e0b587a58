"""Cache plumbing for serving: reorder and clone whole decode caches on the GPU.

A serving loop keeps one ``KDAState`` per KDA layer (recurrent state
``[B,H,K,V]``, three ShortConv histories ``[B,K_conv-1,width]`` and int64
``sequence_offset [B]``, src/kda/state.py:12-39).  Beam search reorders the
batch of every layer with the same indices (``HybridBackboneCache.reorder``,
src/hybrid_backbone/cache.py:118-126, one ``index_select`` per tensor per
layer in ``KDAState.reorder``, src/kda/state.py:50-67), and speculative or
branching decoders clone it (src/kda/state.py:41-48).  Here every tensor of
every layer is gathered by ``kda_cache_gather`` (csrc/kda_cache.hip): one
launch per 64 tensors, each selected row read once and written once.

``reorder_states(states, indices)`` and ``clone_states(states)`` take a
sequence of ``KDAState``; ``gather_rows`` is the tensor-level form.  GPU
tensors only: without the HIP library these raise ``RuntimeError``.
"""

from __future__ import annotations

import ctypes
from collections.abc import Sequence

import torch

from . import _lib, _prep
from .state import KDAState, ShortConvState


def _rows(t: torch.Tensor) -> torch.Tensor:
    return t if t.is_contiguous() else t.contiguous()


def gather_rows(tensors: Sequence[torch.Tensor], indices: torch.Tensor | None) -> list[torch.Tensor]:
    """``[t.index_select(0, indices) for t in tensors]`` in one native pass.

    ``indices=None`` copies every tensor (a clone).  All tensors share the
    batch size of dimension 0 and live on one GPU; ``indices`` is a rank-1
    ``torch.long`` tensor on that GPU.  An index outside ``[0, batch)`` raises
    ``IndexError``, as ``index_select`` does.  Like ``index_select`` and
    ``clone`` (src/kda/state.py:41-67) the result is differentiable: the
    gradient of a source row is the sum of the gradients of the rows gathered
    from it.
    """
    tensors = [_rows(t) for t in tensors]
    if not tensors:
        return []
    if torch.is_grad_enabled() and any(t.requires_grad for t in tensors):
        return list(_GatherRows.apply(indices, *tensors))
    return _gather(tensors, indices)


def _gather(tensors: list[torch.Tensor], indices: torch.Tensor | None) -> list[torch.Tensor]:
    device = tensors[0].device
    for t in tensors:
        _lib.require_gpu(t)
        if t.device != device:
            raise ValueError("all cache tensors must be on one device")
        if t.ndim == 0:
            raise ValueError("cache tensors must have a batch dimension")
    n_src = tensors[0].shape[0]
    if any(t.shape[0] != n_src for t in tensors):
        raise ValueError("all cache tensors must share the batch size")
    if indices is not None:
        if indices.ndim != 1 or indices.dtype != torch.long:
            raise ValueError("indices must be a rank-1 torch.long tensor")
        if indices.device != device:
            raise ValueError("indices and state must be on the same device")
        indices = _rows(indices)
    n_out = n_src if indices is None else indices.shape[0]
    if n_src == 0 and n_out > 0:
        raise IndexError("index out of range for an empty cache batch")
    outs = [torch.empty((n_out, *t.shape[1:]), dtype=t.dtype, device=device) for t in tensors]
    if n_out == 0:
        return outs
    lib = _lib.load()
    n = len(tensors)
    src = (ctypes.c_void_p * n)(*[t.data_ptr() for t in tensors])
    dst = (ctypes.c_void_p * n)(*[o.data_ptr() for o in outs])
    row_bytes = (ctypes.c_int64 * n)(*[t[0].numel() * t.element_size() if n_src else 0 for t in tensors])
    status = None if indices is None else torch.zeros(1, dtype=torch.int32, device=device)
    _lib.check(
        lib.kda_cache_gather(
            src, dst, row_bytes, n, _lib.ptr(indices), n_src, n_out, _lib.ptr(status), _prep.stream(device)
        )
    )
    if status is not None and int(status.item()) != 0:
        raise IndexError(f"index out of range for a cache batch of {n_src}")
    return outs


class _GatherRows(torch.autograd.Function):
    """The native gather under autograd.  Backward: a clone passes gradients
    through; a reorder adds each output row's gradient into the source row it
    was read from (rows picked several times accumulate)."""

    @staticmethod
    def forward(ctx, indices, *tensors):
        ctx.indices = indices
        ctx.shapes = [t.shape for t in tensors]
        return tuple(_gather(list(tensors), indices))

    @staticmethod
    def backward(ctx, *grads):
        idx = ctx.indices
        out = []
        for shape, gr in zip(ctx.shapes, grads):
            if gr is None or idx is None:
                out.append(gr)
            else:
                out.append(torch.zeros(shape, dtype=gr.dtype, device=gr.device).index_add_(0, idx, gr))
        return (None, *out)


def _flatten(state: KDAState) -> list[torch.Tensor]:
    return [
        state.recurrent_state,
        state.q_conv_state.buffer,
        state.k_conv_state.buffer,
        state.v_conv_state.buffer,
        state.sequence_offset,
    ]


def _rebuild(parts: list[torch.Tensor]) -> KDAState:
    return KDAState(
        recurrent_state=parts[0],
        q_conv_state=ShortConvState(parts[1]),
        k_conv_state=ShortConvState(parts[2]),
        v_conv_state=ShortConvState(parts[3]),
        sequence_offset=parts[4],
    )


def reorder_states(states: Sequence[KDAState], indices: torch.Tensor) -> list[KDAState]:
    """Every layer's ``KDAState.reorder(indices)`` (src/kda/state.py:50-67) in one pass."""
    if indices.ndim != 1 or indices.dtype != torch.long:
        raise ValueError("indices must be a rank-1 torch.long tensor")
    flat = [t for s in states for t in _flatten(s)]
    if flat and indices.device != flat[0].device:
        raise ValueError("indices and state must be on the same device")
    out = gather_rows(flat, indices)
    return [_rebuild(out[5 * i : 5 * i + 5]) for i in range(len(states))]


def clone_states(states: Sequence[KDAState]) -> list[KDAState]:
    """Every layer's ``KDAState.clone()`` (src/kda/state.py:41-48) in one pass."""
    flat = [t for s in states for t in _flatten(s)]
    out = gather_rows(flat, None)
    return [_rebuild(out[5 * i : 5 * i + 5]) for i in range(len(states))]
