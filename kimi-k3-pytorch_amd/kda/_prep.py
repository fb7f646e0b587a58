"""Shared argument preparation for the operator wrappers (host side only)."""

from __future__ import annotations

import torch

from . import _lib


def workspace(nbytes: int, device: torch.device, what: str) -> torch.Tensor | None:
    """A caller-owned kernel workspace from the torch allocator (None for 0
    bytes).  A request the allocator cannot serve raises a RuntimeError that
    names the call, the size and the device's free memory in place of the
    allocator's own out-of-memory error.  (No memory statistics are read on
    the way: they cost tens of microseconds per call.)"""
    if nbytes == 0:
        return None
    try:
        return torch.empty(nbytes, dtype=torch.uint8, device=device)
    except torch.cuda.OutOfMemoryError:
        free, _ = torch.cuda.mem_get_info(device)
        raise RuntimeError(
            f"{what} needs a workspace of {nbytes / 2**30:.2f} GiB and the device has "
            f"{free / 2**30:.2f} GiB free; split the batch or the documents into smaller calls"
        ) from None


def kernel_inputs(q, k, v, g, beta, work_dtype: torch.dtype):
    """Pick the element type the kernels read and make the inputs contiguous.

    The reference casts every input to the work dtype before any arithmetic
    (src/kda/chunkwise.py:41-45, src/kda/recurrent.py:42-46).  The kernels do
    that upcast on load, so inputs that already share one dtype are passed
    as they are (bf16 stays bf16 in HBM).  Mixed dtypes are cast to the
    arithmetic type first, which loses nothing.  A bf16/f16 work dtype
    (``accumulate_state_in_fp32=False``) rounds every input to it first, as
    the reference's cast does; the kernels then compute in f32 on those
    rounded values, with results in the work dtype.
    """
    if work_dtype in (torch.bfloat16, torch.float16):
        q, k, v, g, beta = (t.to(work_dtype) for t in (q, k, v, g, beta))
    tensors = (q, k, v, g, beta)
    dtypes = {t.dtype for t in tensors}
    arith = torch.float64 if work_dtype == torch.float64 else torch.float32
    if len(dtypes) == 1:
        (common,) = dtypes
        if arith == torch.float64:
            kernel_dtype = torch.float64
        elif common in (torch.bfloat16, torch.float16, torch.float32):
            kernel_dtype = common
        else:
            kernel_dtype = arith
    else:
        kernel_dtype = arith
    out = tuple(t.to(kernel_dtype).contiguous() for t in tensors)
    return out, kernel_dtype, arith


def valid_lengths(attention_mask: torch.Tensor | None, device: torch.device) -> torch.Tensor | None:
    """Monotone right-padding mask -> int32 valid length per row."""
    if attention_mask is None:
        return None
    return attention_mask.to(device=device).sum(dim=1, dtype=torch.int32).contiguous()


def state_arg(initial_state: torch.Tensor | None, arith: torch.dtype,
              work_dtype: torch.dtype | None = None) -> torch.Tensor | None:
    """The initial state in the kernels' arithmetic type.  The reference starts
    from ``initial_state.to(work_dtype)`` (src/kda/chunkwise.py:49-58,
    src/kda/recurrent.py:50-59), so a bf16/f16 work dtype rounds it first."""
    if initial_state is None:
        return None
    if work_dtype in (torch.bfloat16, torch.float16):
        initial_state = initial_state.to(work_dtype)
    return initial_state.to(arith).contiguous()


def cu_tensor(offsets: list[int], device: torch.device) -> torch.Tensor:
    return torch.tensor(offsets, dtype=torch.int32, device=device)


def longest_document(offsets: list[int] | None) -> int:
    """Tokens of the longest packed document (0 for dense sequences): the
    chunk prefill's scheduling hint, passed in the C ABI's `dense_span` and
    `longest_tokens` for packed documents."""
    if offsets is None:
        return 0
    return max(b - a for a, b in zip(offsets[:-1], offsets[1:]))


def stream(device: torch.device) -> int:
    return _lib.stream_of(device)
