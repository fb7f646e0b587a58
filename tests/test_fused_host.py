"""Argument checks of kda.fused (CPU: every error is raised before any launch;
CPU tensors are refused, there is no CPU fallback)."""

from __future__ import annotations

import pytest
import torch

import kda
from kda import fused


def test_conv_silu_argument_checks():
    x = torch.zeros(2, 5, 128)
    w = torch.zeros(128, 4)
    with pytest.raises(ValueError):
        fused.conv_silu(torch.zeros(2, 5), w)
    with pytest.raises(ValueError):
        fused.conv_silu(torch.zeros(2, 0, 128), w)
    with pytest.raises(ValueError):
        fused.conv_silu(x, torch.zeros(64, 4))
    with pytest.raises(TypeError):
        fused.conv_silu(x, w.double())
    with pytest.raises(ValueError):
        fused.conv_silu(x, w, state=kda.ShortConvState(torch.zeros(2, 2, 128)))
    with pytest.raises(ValueError):
        fused.conv_silu(x, w, num_heads=3)
    with pytest.raises(ValueError):
        fused.conv_silu(x, w, normalize=True)
    with pytest.raises(ValueError):
        fused.conv_silu(x, w, attention_mask=torch.ones(2, 4, dtype=torch.bool))
    with pytest.raises(RuntimeError, match="GPU|cuda|device"):
        fused.conv_silu(x, w, num_heads=1)


def test_gate_and_norm_argument_checks():
    with pytest.raises(ValueError):
        fused.lower_bounded_decay(torch.zeros(2, 3, 4), torch.zeros(3))
    with pytest.raises(RuntimeError, match="GPU|cuda|device"):
        fused.lower_bounded_decay(torch.zeros(1, 2, 3, 8), torch.zeros(3))
    with pytest.raises(RuntimeError, match="GPU|cuda|device"):
        fused.beta_gate(torch.zeros(1, 2, 3))
    with pytest.raises(ValueError):
        fused.rmsnorm_gate(torch.zeros(2, 3, 64))
    with pytest.raises(ValueError):
        fused.rmsnorm_gate(torch.zeros(1, 2, 3, 64), torch.zeros(5))
    with pytest.raises(ValueError):
        fused.rmsnorm_gate(torch.zeros(1, 2, 3, 64), gate_logits=torch.zeros(1, 2, 64))
    with pytest.raises(RuntimeError, match="GPU|cuda|device"):
        fused.rmsnorm_gate(torch.zeros(1, 2, 3, 64))
