"""Input contract of the KDA operators.

Same checks, messages and exception types as the reference's validators so
that callers see identical errors before any compute:
``validate_attention_mask`` (src/kda/utils.py:8-29), ``validate_core_inputs``
(src/kda/utils.py:32-71) and ``accumulation_dtype`` (src/kda/utils.py:74-79).
``validate_cu_seqlens`` covers the packed-document extension, which the
reference does not have.
"""

from __future__ import annotations

import torch


def validate_attention_mask(
    attention_mask: torch.Tensor | None,
    batch: int,
    tokens: int,
    *,
    require_nonempty: bool = True,
) -> torch.Tensor | None:
    if attention_mask is None:
        return None
    if attention_mask.shape != (batch, tokens):
        raise ValueError(
            f"attention_mask must have shape {(batch, tokens)}, got {tuple(attention_mask.shape)}"
        )
    if attention_mask.dtype != torch.bool:
        raise TypeError("attention_mask must be boolean (True means valid)")
    if tokens > 1 and bool(((~attention_mask[:, :-1]) & attention_mask[:, 1:]).any()):
        raise ValueError("attention_mask must be monotonic right-padding")
    if require_nonempty and bool((attention_mask.sum(dim=1) == 0).any()):
        raise ValueError("all-padding sequences are not supported")
    return attention_mask


def validate_core_inputs(q, k, v, g, beta, initial_state, attention_mask, *, num_states: int | None = None):
    """Shape/device/dtype checks; returns (B, T, H, K, V).

    ``num_states`` overrides the expected leading size of ``initial_state``
    (the number of packed documents when ``cu_seqlens`` is used)."""
    if q.ndim != 4:
        raise ValueError(f"q must have shape [B,T,H,K], got {tuple(q.shape)}")
    batch, tokens, heads, key_dim = q.shape
    if tokens == 0:
        raise ValueError("KDA does not support empty sequences")
    if k.shape != q.shape or g.shape != q.shape:
        raise ValueError("k and g must have the same shape as q")
    if v.ndim != 4 or v.shape[:3] != (batch, tokens, heads):
        raise ValueError("v must have shape [B,T,H,V] matching q")
    value_dim = v.shape[-1]
    if beta.shape != (batch, tokens, heads):
        raise ValueError(f"beta must have shape {(batch, tokens, heads)}, got {tuple(beta.shape)}")
    tensors = (q, k, v, g, beta)
    if any(t.device != q.device for t in tensors):
        raise ValueError("all KDA inputs must be on the same device")
    if any(not t.dtype.is_floating_point for t in tensors):
        raise TypeError("all KDA inputs must use floating-point dtypes")
    if initial_state is not None:
        lead = batch if num_states is None else num_states
        expected = (lead, heads, key_dim, value_dim)
        if initial_state.shape != expected:
            raise ValueError(
                f"initial_state must have shape {expected}, got {tuple(initial_state.shape)}"
            )
        if initial_state.device != q.device:
            raise ValueError("initial_state and inputs must be on the same device")
    validate_attention_mask(attention_mask, batch, tokens)
    return batch, tokens, heads, key_dim, value_dim


def accumulation_dtype(dtype: torch.dtype, accumulate_state_in_fp32: bool) -> torch.dtype:
    if accumulate_state_in_fp32 and dtype in (torch.float16, torch.bfloat16):
        return torch.float32
    return dtype


def validate_cu_seqlens(cu_seqlens, batch: int, tokens: int, attention_mask) -> list[int]:
    """Packed documents: B == 1, offsets 0 = c_0 < c_1 < ... < c_N = T.

    Returns the offsets as Python ints.  Empty documents are rejected, like
    all-padding rows (src/kda/utils.py:27-28)."""
    if batch != 1:
        raise ValueError(f"cu_seqlens requires packed inputs with B == 1, got B={batch}")
    if attention_mask is not None:
        raise ValueError("attention_mask and cu_seqlens cannot be combined")
    if isinstance(cu_seqlens, torch.Tensor):
        if cu_seqlens.ndim != 1:
            raise ValueError("cu_seqlens must be a 1-D tensor of N+1 offsets")
        if cu_seqlens.dtype not in (torch.int32, torch.int64):
            raise TypeError("cu_seqlens must be int32 or int64")
        offsets = [int(x) for x in cu_seqlens.detach().cpu().tolist()]
    else:
        offsets = [int(x) for x in cu_seqlens]
    if len(offsets) < 2:
        raise ValueError("cu_seqlens must hold at least two offsets")
    if offsets[0] != 0 or offsets[-1] != tokens:
        raise ValueError(f"cu_seqlens must start at 0 and end at T={tokens}, got {offsets[0]}..{offsets[-1]}")
    if any(b <= a for a, b in zip(offsets[:-1], offsets[1:])):
        raise ValueError("cu_seqlens must be strictly increasing (empty documents are not supported)")
    return offsets
