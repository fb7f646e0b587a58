"""A KDA layer composed from this backend's kernels.

The caller path of the operators in the reference is
``KimiDeltaAttention.forward`` (src/kda/kda.py:98-206): the projections
(src/kda/projections.py:144-225), the lower-bounded decay (src/kda/decay.py:28-43),
the operator (``recurrent_kda`` for ``mode="recurrent"``/``"decode"``,
``chunkwise_kda`` otherwise, kda.py:133-151), the head-wise RMSNorm and the
output gate (kda.py:153-161) and the ``KDAState`` handed to the next call
(kda.py:163-183).  ``kda_attention_forward`` runs that path on the GPU:

* q, k, v: the projection GEMM (``torch.nn.functional.linear``, as the
  reference's ``nn.Linear``), then ``fused.conv_silu`` (ShortConv + SiLU, L2
  norm per head for q and k, right padding and the decode history);
* beta: the projection, then ``fused.beta_gate``;
* decay: the low-rank projection, then ``fused.lower_bounded_decay``, which
  feeds the operator (the chunk kernel can also form g from the logits
  itself, ``fused.chunkwise_kda_with_decay``, bit-identical but measured
  slower, so the layer keeps the two launches);
* output: ``fused.rmsnorm_gate`` (RMSNorm times the sigmoid gate of the gate
  projection), the output projection, and the mask.

The projection GEMMs are torch's; everything between them runs in this
library's HIP kernels.  Weights are plain tensors (``KDALayerWeights``), so a
reference module's parameters can be handed over with ``from_module``.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Literal

import torch
import torch.nn.functional as F

from . import fused
from .chunkwise import chunkwise_kda
from .recurrent import recurrent_kda
from .state import KDAState
from .utils import validate_attention_mask


@dataclass
class KDALayerWeights:
    """The parameters of one KDA layer, in the reference's layouts
    (src/kda/projections.py:35-73, src/kda/decay.py:24-26, src/kda/kda.py:50-62):
    linear weights ``[out, in]``, ShortConv weights ``[C, K_conv]`` in lag order."""

    num_heads: int
    key_head_dim: int
    value_head_dim: int
    q_proj: torch.Tensor
    k_proj: torch.Tensor
    v_proj: torch.Tensor
    q_conv: torch.Tensor
    k_conv: torch.Tensor
    v_conv: torch.Tensor
    beta_proj: torch.Tensor
    alpha_down: torch.Tensor
    alpha_up: torch.Tensor
    b_alpha: torch.Tensor
    a_log: torch.Tensor
    norm_weight: torch.Tensor | None
    gate_proj: torch.Tensor
    output_proj: torch.Tensor
    g_min: float = -5.0
    eps: float = 1e-6
    accumulate_state_in_fp32: bool = True
    q_proj_bias: torch.Tensor | None = None
    k_proj_bias: torch.Tensor | None = None
    v_proj_bias: torch.Tensor | None = None
    q_conv_bias: torch.Tensor | None = None
    k_conv_bias: torch.Tensor | None = None
    v_conv_bias: torch.Tensor | None = None
    beta_bias: torch.Tensor | None = None
    gate_bias: torch.Tensor | None = None
    output_bias: torch.Tensor | None = None

    @property
    def d_model(self) -> int:
        return self.gate_proj.shape[0]

    @property
    def key_width(self) -> int:
        return self.num_heads * self.key_head_dim

    @property
    def value_width(self) -> int:
        return self.num_heads * self.value_head_dim

    @property
    def conv_kernel_size(self) -> int:
        return self.q_conv.shape[1]

    @classmethod
    def from_module(cls, module, *, detach: bool = True) -> "KDALayerWeights":
        """The parameters of a module with the reference's attribute names
        (``KimiDeltaAttention``, src/kda/kda.py:45-62).  ``detach=False``
        keeps the module's parameters themselves, so that a backward through
        ``kda_attention_forward`` fills their ``.grad`` (training);
        the default hands over detached views (inference)."""
        cfg, p = module.config, module.projections
        d = (lambda t: t.detach()) if detach else (lambda t: t)  # noqa: E731
        bias = lambda lin: None if lin.bias is None else d(lin.bias)  # noqa: E731
        conv_bias = lambda c: None if c.bias is None else d(c.bias)  # noqa: E731
        norm = module.output_norm.weight
        return cls(
            num_heads=cfg.num_heads, key_head_dim=cfg.key_head_dim, value_head_dim=cfg.value_head_dim,
            q_proj=d(p.q_proj.weight), k_proj=d(p.k_proj.weight), v_proj=d(p.v_proj.weight),
            q_conv=d(p.q_conv.weight), k_conv=d(p.k_conv.weight), v_conv=d(p.v_conv.weight),
            beta_proj=d(p.beta_proj.weight), alpha_down=d(p.alpha_down.weight),
            alpha_up=d(p.alpha_up.weight), b_alpha=d(p.b_alpha), a_log=d(module.decay.A_log),
            norm_weight=None if norm is None else d(norm),
            gate_proj=d(module.output_gate.gate_proj.weight),
            output_proj=d(module.output_gate.output_proj.weight),
            g_min=cfg.g_min, eps=cfg.eps, accumulate_state_in_fp32=cfg.accumulate_state_in_fp32,
            q_proj_bias=bias(p.q_proj), k_proj_bias=bias(p.k_proj), v_proj_bias=bias(p.v_proj),
            q_conv_bias=conv_bias(p.q_conv), k_conv_bias=conv_bias(p.k_conv), v_conv_bias=conv_bias(p.v_conv),
            beta_bias=bias(p.beta_proj), gate_bias=bias(module.output_gate.gate_proj),
            output_bias=bias(module.output_gate.output_proj),
        )


@dataclass
class KDALayerOutput:
    """Output and next cache state of one layer call (src/kda/kda.py:29-35)."""

    hidden_states: torch.Tensor
    state: KDAState | None = None


def _validate_state(w: KDALayerWeights, hidden_states: torch.Tensor, state: KDAState | None) -> None:
    """The cache-shape checks of KimiDeltaAttention._validate_state (src/kda/kda.py:64-96)."""
    if state is None:
        return
    batch = hidden_states.shape[0]
    expected_recurrent = (batch, w.num_heads, w.key_head_dim, w.value_head_dim)
    if state.recurrent_state.shape != expected_recurrent:
        raise ValueError(f"state recurrent tensor must have shape {expected_recurrent}")
    history = w.conv_kernel_size - 1
    expected_buffers = ((batch, history, w.key_width), (batch, history, w.key_width), (batch, history, w.value_width))
    actual_buffers = (state.q_conv_state.buffer.shape, state.k_conv_state.buffer.shape,
                      state.v_conv_state.buffer.shape)
    if actual_buffers != expected_buffers:
        raise ValueError(f"state ShortConv buffers must have shapes {expected_buffers}")
    if state.recurrent_state.device != hidden_states.device:
        raise ValueError("state and hidden_states must be on the same device")


def kda_attention_forward(
    w: KDALayerWeights,
    hidden_states: torch.Tensor,
    attention_mask: torch.Tensor | None = None,
    state: KDAState | None = None,
    mode: Literal["recurrent", "chunkwise", "decode"] = "chunkwise",
    output_final_state: bool = False,
    *,
    update_state_in_place: bool = False,
) -> KDALayerOutput:
    """One KDA layer call, as ``KimiDeltaAttention.forward`` (src/kda/kda.py:98-183)
    without the diagnostics.  ``update_state_in_place`` (decode only) writes the
    new recurrent state over ``state.recurrent_state`` instead of a new tensor."""
    if hidden_states.ndim != 3 or hidden_states.shape[-1] != w.d_model:
        raise ValueError(f"hidden_states must have shape [B,T,{w.d_model}], got {tuple(hidden_states.shape)}")
    batch, tokens, _ = hidden_states.shape
    if tokens == 0:
        raise ValueError("KDA does not support empty sequences")
    if mode not in ("recurrent", "chunkwise", "decode"):
        raise ValueError(f"unsupported KDA mode {mode!r}")
    if mode == "decode" and tokens != 1:
        raise ValueError("decode mode requires exactly one token")
    validate_attention_mask(attention_mask, batch, tokens)
    _validate_state(w, hidden_states, state)
    x = hidden_states
    H, K, V = w.num_heads, w.key_head_dim, w.value_head_dim
    return_state = output_final_state or mode == "decode"

    # projections (src/kda/projections.py:164-218)
    qs, ks, vs = (None, None, None) if state is None else (state.q_conv_state, state.k_conv_state,
                                                             state.v_conv_state)
    q, q_next = fused.conv_silu(F.linear(x, w.q_proj, w.q_proj_bias), w.q_conv, w.q_conv_bias, qs, attention_mask,
                                num_heads=H, normalize=True, eps=w.eps, output_final_state=return_state)
    k, k_next = fused.conv_silu(F.linear(x, w.k_proj, w.k_proj_bias), w.k_conv, w.k_conv_bias, ks, attention_mask,
                                num_heads=H, normalize=True, eps=w.eps, output_final_state=return_state)
    v, v_next = fused.conv_silu(F.linear(x, w.v_proj, w.v_proj_bias), w.v_conv, w.v_conv_bias, vs, attention_mask,
                                num_heads=H, output_final_state=return_state)
    beta = fused.beta_gate(F.linear(x, w.beta_proj, w.beta_bias))
    decay_logits = F.linear(F.linear(x, w.alpha_down), w.alpha_up).reshape(batch, tokens, H, K)

    # the operator (src/kda/kda.py:131-151)
    initial = None if state is None else state.recurrent_state
    keep_state = return_state
    # the decay kernel, then the operator: measured faster than forming g
    # inside the chunk kernel (fused.chunkwise_kda_with_decay, bit-identical),
    # whose extra VALU work lands on the chunk kernel's latency-bound loaders
    g, _ = fused.lower_bounded_decay(decay_logits, w.a_log, w.g_min, bias=w.b_alpha)
    if mode == "chunkwise":
        core = chunkwise_kda(q, k, v, g, beta, initial, keep_state, attention_mask,
                             accumulate_state_in_fp32=w.accumulate_state_in_fp32)
    else:
        core = recurrent_kda(q, k, v, g, beta, initial, keep_state, attention_mask,
                             accumulate_state_in_fp32=w.accumulate_state_in_fp32,
                             update_state_in_place=update_state_in_place and mode == "decode" and initial is not None)

    # RMSNorm x output gate, output projection, mask (src/kda/kda.py:153-161)
    gated = fused.rmsnorm_gate(core.hidden_states, w.norm_weight, w.eps,
                               gate_logits=F.linear(x, w.gate_proj, w.gate_bias))
    out = F.linear(gated.reshape(batch, tokens, H * V), w.output_proj, w.output_bias)
    if attention_mask is not None:
        out = out * attention_mask[..., None].to(out.dtype)

    next_state = None
    if return_state:
        # src/kda/kda.py:163-183
        if attention_mask is None:
            lengths = torch.full((batch,), tokens, dtype=torch.long, device=x.device)
        else:
            lengths = attention_mask.sum(dim=1).to(torch.long)
        offset = lengths if state is None else state.sequence_offset.to(x.device) + lengths
        next_state = KDAState(recurrent_state=core.final_state, q_conv_state=q_next, k_conv_state=k_next,
                              v_conv_state=v_next, sequence_offset=offset)
    return KDALayerOutput(hidden_states=out, state=next_state)


__all__ = ["KDALayerOutput", "KDALayerWeights", "kda_attention_forward"]
