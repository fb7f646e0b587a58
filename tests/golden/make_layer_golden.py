"""Writes the KDA layer fixtures in this folder from the reference module itself.

The layer composition (projections, ShortConv + SiLU + L2 norm, the
lower-bounded decay, the operator, head-wise RMSNorm, the output gate, the
mask and the ``KDAState`` handed to the next call) is pinned by no stored
vector of the reference and by no closed form, so this script imports the
reference's ``KimiDeltaAttention`` (src/kda/kda.py:39-206 of
pablo-reyes8/kimi-k3-pytorch, read from /root/reference) in this container
only, and freezes what it computes on seeded weights and inputs.  Only the
resulting arrays are committed; nothing of the reference travels with them.

Scenario (per dtype, f32 and bf16): a right-padded chunkwise prefill with
``output_final_state=True``, then two ``mode="decode"`` steps carrying the
``KDAState``; a ``mode="recurrent"`` call on the same prefill.  Every bias of
the module is enabled and every parameter is perturbed away from its
initial value, so that a dropped bias, gate or norm weight changes the
outputs.  bf16 values are stored as their exact float32 images.

Usage:  python tests/golden/make_layer_golden.py   (needs /root/reference)
"""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent
REFERENCE = Path("/root/reference")

# d_model = H * V (the reference requires it); K = 32 and V = 32 sit on the
# MFMA grid (multiples of 16) of the bf16 chunk kernels
CONFIG = dict(d_model=64, num_heads=2, key_head_dim=32, value_head_dim=32, short_conv_kernel_size=4,
              decay_rank=16, g_min=-5.0, chunk_size=16, secondary_tile_size=8, eps=1e-6, projection_bias=True,
              short_conv_bias=True, beta_bias=True, output_gate_bias=True, output_bias=True,
              accumulate_state_in_fp32=True)
BATCH, TOKENS, VALID = 2, 21, (21, 15)  # the second row is right-padded after 15 tokens


def _module(dtype):
    sys.path.insert(0, str(REFERENCE))
    from src.kda import KDAConfig, KimiDeltaAttention  # noqa: E402  (the reference, this container only)

    torch.manual_seed(1234)
    module = KimiDeltaAttention(KDAConfig(**CONFIG))
    gen = torch.Generator().manual_seed(99)
    with torch.no_grad():
        for name, p in sorted(module.named_parameters()):
            # off the initial values (zeros / ones) so every term is visible
            p.add_(0.05 * torch.randn(p.shape, generator=gen, dtype=p.dtype))
    return module.to(dtype).eval()


def _weights(module) -> dict[str, np.ndarray]:
    """The module's parameters under the field names of kda.layer.KDALayerWeights."""
    p, gate = module.projections, module.output_gate
    named = dict(
        q_proj=p.q_proj.weight, k_proj=p.k_proj.weight, v_proj=p.v_proj.weight,
        q_conv=p.q_conv.weight, k_conv=p.k_conv.weight, v_conv=p.v_conv.weight,
        beta_proj=p.beta_proj.weight, alpha_down=p.alpha_down.weight, alpha_up=p.alpha_up.weight,
        b_alpha=p.b_alpha, a_log=module.decay.A_log, norm_weight=module.output_norm.weight,
        gate_proj=gate.gate_proj.weight, output_proj=gate.output_proj.weight,
        q_proj_bias=p.q_proj.bias, k_proj_bias=p.k_proj.bias, v_proj_bias=p.v_proj.bias,
        q_conv_bias=p.q_conv.bias, k_conv_bias=p.k_conv.bias, v_conv_bias=p.v_conv.bias,
        beta_bias=p.beta_proj.bias, gate_bias=gate.gate_proj.bias, output_bias=gate.output_proj.bias,
    )
    return {f"w_{k}": v.detach().float().numpy() for k, v in named.items() if v is not None}


def _state(prefix, st) -> dict[str, np.ndarray]:
    return {
        f"{prefix}_recurrent": st.recurrent_state.detach().float().numpy(),
        f"{prefix}_q_hist": st.q_conv_state.buffer.detach().float().numpy(),
        f"{prefix}_k_hist": st.k_conv_state.buffer.detach().float().numpy(),
        f"{prefix}_v_hist": st.v_conv_state.buffer.detach().float().numpy(),
        f"{prefix}_offset": st.sequence_offset.detach().numpy(),
    }


def make(dtype, name):
    module = _module(dtype)
    gen = torch.Generator().manual_seed(7)
    x = torch.randn(BATCH, TOKENS, CONFIG["d_model"], generator=gen).to(dtype)
    steps = [torch.randn(BATCH, 1, CONFIG["d_model"], generator=gen).to(dtype) for _ in range(2)]
    mask = torch.zeros(BATCH, TOKENS, dtype=torch.bool)
    for b, n in enumerate(VALID):
        mask[b, :n] = True
    arrays = dict(_weights(module))
    with torch.no_grad():
        pre = module(x, attention_mask=mask, mode="chunkwise", output_final_state=True)
        rec = module(x, attention_mask=mask, mode="recurrent", output_final_state=True)
        arrays.update(x=x.float().numpy(), mask=mask.numpy(), prefill_out=pre.hidden_states.float().numpy(),
                      recurrent_out=rec.hidden_states.float().numpy(), **_state("prefill", pre.state),
                      **_state("recurrent", rec.state))
        state = pre.state
        for i, xs in enumerate(steps):
            step = module(xs, state=state, mode="decode")
            state = step.state
            arrays.update({f"x_step{i}": xs.float().numpy(), f"step{i}_out": step.hidden_states.float().numpy(),
                           **_state(f"step{i}", state)})
    arrays["config"] = np.array(repr(CONFIG))
    arrays["dtype"] = np.array(str(dtype).replace("torch.", ""))
    np.savez_compressed(HERE / name, **arrays)
    print(f"wrote {name}: {len(arrays)} arrays")


if __name__ == "__main__":
    make(torch.float32, "layer_ref_f32_B2_T21_H2_K32_V32.npz")
    make(torch.bfloat16, "layer_ref_bf16_B2_T21_H2_K32_V32.npz")
