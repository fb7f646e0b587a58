"""Incremental KDA state carried by the inference cache.

Same layout contract as the reference's ``KDAState`` (src/kda/state.py:12-67)
and ``ShortConvState`` (src/kimi_primitives/states.py:10-27): the recurrent
state is one plain ``[B,H,K,V]`` tensor (f32 for bf16 models), next to three
ShortConv buffers ``[B, K_conv-1, width]`` and an int64 ``sequence_offset``.
The decode kernel reads and writes ``recurrent_state`` in exactly this
layout, so the byte accounting of inference/cache.py:32-38 is unchanged.
``clone`` and ``reorder`` of a state held on the GPU run the native batch-row
gather of ``kda.cache`` (one launch for all five tensors); a state held in
host memory keeps torch's copies.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch


@dataclass
class ShortConvState:
    """Rolling causal-convolution history ``[B, K_conv-1, width]``."""

    buffer: torch.Tensor

    def __post_init__(self) -> None:
        if self.buffer.ndim != 3:
            raise ValueError("ShortConv state buffer must have shape [B,K-1,C]")

    def clone(self) -> "ShortConvState":
        if self.buffer.is_cuda:
            from .cache import gather_rows

            return ShortConvState(gather_rows([self.buffer], None)[0])
        return ShortConvState(self.buffer.clone())


@dataclass
class KDAState:
    """Incremental KDA state containing recurrence and short-convolution buffers."""

    recurrent_state: torch.Tensor
    q_conv_state: ShortConvState
    k_conv_state: ShortConvState
    v_conv_state: ShortConvState
    sequence_offset: torch.Tensor

    def __post_init__(self) -> None:
        if self.recurrent_state.ndim != 4:
            raise ValueError("recurrent_state must have shape [B,H,K,V]")
        batch = self.recurrent_state.shape[0]
        if self.sequence_offset.shape != (batch,):
            raise ValueError(
                f"sequence_offset must have shape {(batch,)}, got {tuple(self.sequence_offset.shape)}"
            )
        if self.sequence_offset.dtype != torch.long:
            raise TypeError("sequence_offset must use torch.long")
        conv_batches = (
            self.q_conv_state.buffer.shape[0],
            self.k_conv_state.buffer.shape[0],
            self.v_conv_state.buffer.shape[0],
        )
        if conv_batches != (batch, batch, batch):
            raise ValueError("all ShortConv states must match recurrent batch size")

    def clone(self) -> "KDAState":
        if self.recurrent_state.is_cuda:
            from .cache import clone_states

            return clone_states([self])[0]
        return KDAState(
            recurrent_state=self.recurrent_state.clone(),
            q_conv_state=self.q_conv_state.clone(),
            k_conv_state=self.k_conv_state.clone(),
            v_conv_state=self.v_conv_state.clone(),
            sequence_offset=self.sequence_offset.clone(),
        )

    def reorder(self, indices: torch.Tensor) -> "KDAState":
        if indices.ndim != 1 or indices.dtype != torch.long:
            raise ValueError("indices must be a rank-1 torch.long tensor")
        if indices.device != self.recurrent_state.device:
            raise ValueError("indices and state must be on the same device")
        if self.recurrent_state.is_cuda:
            from .cache import reorder_states

            return reorder_states([self], indices)[0]
        pick = lambda t: t.index_select(0, indices)  # noqa: E731
        return KDAState(
            recurrent_state=pick(self.recurrent_state),
            q_conv_state=ShortConvState(pick(self.q_conv_state.buffer)),
            k_conv_state=ShortConvState(pick(self.k_conv_state.buffer)),
            v_conv_state=ShortConvState(pick(self.v_conv_state.buffer)),
            sequence_offset=pick(self.sequence_offset),
        )
