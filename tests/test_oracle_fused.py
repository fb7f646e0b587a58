"""Pins for the oracle's fused stages around the operator (CPU).

* short_conv: torch.nn.functional.conv1d on the history-padded input (a
  library routine), and streaming (two calls chained through the returned
  history equal one call);
* conv_silu: masked rows equal the truncated run with zero padding, unit
  head norms after normalisation, SiLU against its closed form x*sigmoid(x);
* lower_bounded_decay / beta_gate: the sigmoid midpoint (g_min/2, 1/2), the
  clamp bounds, monotonicity in the logits, alpha = exp(g);
* rmsnorm_gate: unit mean square, scale invariance, the gate midpoint (1/2).
"""

from __future__ import annotations

import pytest
import torch
import torch.nn.functional as F

from oracle import kda_oracle as ora


def _conv1d_ref(x, w, b, hist):
    taps = w.shape[1]
    combined = torch.cat((hist, x), dim=1)
    return F.conv1d(combined.transpose(1, 2), w.flip(-1).unsqueeze(1), b, groups=x.shape[2]).transpose(1, 2)


@pytest.mark.parametrize("taps", [1, 2, 4, 7])
def test_short_conv_equals_conv1d(taps):
    gen = torch.Generator().manual_seed(taps)
    x = torch.randn(2, 11, 6, generator=gen, dtype=torch.float64)
    w = torch.randn(6, taps, generator=gen, dtype=torch.float64)
    b = torch.randn(6, generator=gen, dtype=torch.float64)
    hist = torch.randn(2, taps - 1, 6, generator=gen, dtype=torch.float64)
    y, nxt = ora.short_conv(x, w, b, hist)
    assert torch.allclose(y, _conv1d_ref(x, w, b, hist), atol=1e-12)
    assert torch.equal(nxt, torch.cat((hist, x), dim=1)[:, 11 + taps - 1 - (taps - 1):])


def test_short_conv_streams_through_its_history():
    gen = torch.Generator().manual_seed(3)
    x = torch.randn(1, 20, 4, generator=gen, dtype=torch.float64)
    w = torch.randn(4, 4, generator=gen, dtype=torch.float64)
    full, hist_full = ora.short_conv(x, w)
    y1, h1 = ora.short_conv(x[:, :7], w)
    y2, h2 = ora.short_conv(x[:, 7:], w, None, h1)
    assert torch.allclose(torch.cat((y1, y2), dim=1), full, atol=1e-12)
    assert torch.equal(h2, hist_full)


def test_conv_silu_mask_normalisation_and_silu():
    gen = torch.Generator().manual_seed(5)
    x = torch.randn(2, 9, 8, generator=gen, dtype=torch.float64)
    w = torch.randn(8, 3, generator=gen, dtype=torch.float64)
    mask = torch.arange(9)[None, :] < torch.tensor([9, 5])[:, None]
    y, hist = ora.conv_silu(x, w, None, None, mask, num_heads=2, normalize=True)
    # padded rows are zero, valid rows equal the truncated run
    assert torch.count_nonzero(y[1, 5:]) == 0
    y_trunc, h_trunc = ora.conv_silu(x[1:, :5], w, None, None, None, num_heads=2, normalize=True)
    assert torch.allclose(y[1:, :5], y_trunc, atol=1e-12)
    assert torch.equal(hist[1:], h_trunc)
    # unit norms per head
    norms = y[0].reshape(9, 2, 4).square().sum(-1).sqrt()
    assert torch.allclose(norms, torch.ones_like(norms), atol=1e-12)
    # SiLU without normalisation: x * sigmoid(x) of the convolution
    raw, _ = ora.short_conv(x, w)
    y_plain, _ = ora.conv_silu(x, w)
    assert torch.allclose(y_plain, raw / (1 + torch.exp(-raw)), atol=1e-12)


def test_lower_bounded_decay_and_beta_gate():
    z = torch.tensor([[[[0.0, 1e4, -1e4, 0.5, -0.5, 2.0]]]], dtype=torch.float64)
    a_log = torch.zeros(1, dtype=torch.float64)
    g, alpha = ora.lower_bounded_decay(z, a_log, -5.0)
    eps = torch.finfo(torch.float64).eps
    assert g[..., 0].item() == pytest.approx(-2.5, abs=1e-15)
    assert g[..., 1].item() == pytest.approx(-5.0 * (1 - eps), abs=1e-15)  # clamp from above
    assert g[..., 2].item() == pytest.approx(-5.0 * eps, abs=1e-20)        # clamp from below
    assert g[..., 3] < g[..., 4]                                            # decreasing in z
    assert torch.allclose(alpha, g.exp())
    # A_log scales the logits; a bias shifts them
    g2, _ = ora.lower_bounded_decay(z, torch.tensor([0.6931471805599453], dtype=torch.float64), -5.0)
    g3, _ = ora.lower_bounded_decay(2 * z, a_log, -5.0)
    assert torch.allclose(g2, g3, atol=1e-12)
    g4, _ = ora.lower_bounded_decay(z, a_log, -5.0, bias=torch.full((1, 6), 0.5, dtype=torch.float64))
    g5, _ = ora.lower_bounded_decay(z + 0.5, a_log, -5.0)
    assert torch.allclose(g4, g5, atol=1e-12)
    beta = ora.beta_gate(torch.tensor([0.0, 50.0, -50.0], dtype=torch.bfloat16))
    eps16 = torch.finfo(torch.bfloat16).eps
    assert beta.tolist() == pytest.approx([0.5, 1 - eps16, eps16])


def test_rmsnorm_gate_invariants():
    gen = torch.Generator().manual_seed(9)
    x = torch.randn(2, 3, 4, 16, generator=gen, dtype=torch.float64)
    y = ora.rmsnorm_gate(x, eps=1e-12)
    assert torch.allclose(y.square().mean(-1), torch.ones(2, 3, 4, dtype=torch.float64), atol=1e-9)
    assert torch.allclose(ora.rmsnorm_gate(7.0 * x, eps=1e-12), y, atol=1e-9)
    w = torch.randn(4, 16, generator=gen, dtype=torch.float64)
    assert torch.allclose(ora.rmsnorm_gate(x, w, eps=1e-12), y * w, atol=1e-12)
    gated = ora.rmsnorm_gate(x, w, 1e-12, torch.zeros(2, 3, 64, dtype=torch.float64))
    assert torch.allclose(gated, 0.5 * y * w, atol=1e-12)
