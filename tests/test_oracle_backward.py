"""Pins of the oracle's chunkwise backward (oracle.kda_oracle.chunkwise_backward):
the explicit per-chunk gradient formulas against torch.autograd through the
oracle's forward (chunkwise and recurrent, f64), the reference's own gradient
tests (tests/kda/test_kda_chunkwise_equivalence.py:92-134: recurrent and
chunkwise gradients agree; gradcheck), chunk-size invariance and extreme decays."""

from __future__ import annotations

import pytest
import torch

from oracle import kda_oracle as ora

F64 = torch.float64


def _core(B, T, H, K, V, seed, decay=2.0, beta_zero_tail=0):
    gen = torch.Generator().manual_seed(seed)
    r = lambda *s: torch.randn(*s, generator=gen, dtype=F64)  # noqa: E731
    q, k, v = r(B, T, H, K), r(B, T, H, K), r(B, T, H, V)
    k = k / k.norm(dim=-1, keepdim=True)
    g = -torch.rand(B, T, H, K, generator=gen, dtype=F64) * decay
    beta = torch.rand(B, T, H, generator=gen, dtype=F64)
    if beta_zero_tail:
        beta[:, -beta_zero_tail:] = 0.0
        q[:, -beta_zero_tail:] = 0.0
        g[:, -beta_zero_tail:] = 0.0
    s0 = r(B, H, K, V)
    d_out, d_final = r(B, T, H, V), r(B, H, K, V)
    return (q, k, v, g, beta, s0), d_out, d_final


def _autograd(fn, inputs, d_out, d_final):
    leaves = [t.clone().requires_grad_() for t in inputs]
    out, final = fn(*leaves)
    loss = (out * d_out).sum() + (final * d_final).sum() if d_final is not None else (out * d_out).sum()
    return torch.autograd.grad(loss, leaves)


def _max_rel(a, b):
    return float((a - b).abs().max() / b.abs().max().clamp_min(1e-300))


@pytest.mark.parametrize("B,T,H,K,V,C,decay,tail", [
    (2, 37, 2, 8, 6, 16, 2.0, 0),     # ragged last chunk
    (1, 64, 1, 16, 16, 64, 0.5, 0),   # one full chunk
    (1, 70, 2, 4, 3, 64, 40.0, 0),    # extreme per-token decay (exp underflows inside a chunk)
    (2, 20, 1, 5, 7, 8, 1.0, 6),      # masked tail: q, g, beta zero
])
def test_backward_equals_autograd_through_chunkwise(B, T, H, K, V, C, decay, tail):
    inputs, d_out, d_final = _core(B, T, H, K, V, seed=B * T + K, decay=decay, beta_zero_tail=tail)
    ref = _autograd(lambda *x: ora.chunkwise(*x, chunk_size=C, secondary_tile_size=min(C, 4)), inputs, d_out,
                    d_final)
    got = ora.chunkwise_backward(*inputs, d_out, d_final, chunk_size=C)
    for name, a, b in zip(("dq", "dk", "dv", "dg", "dbeta", "ds0"), got, ref):
        assert torch.isfinite(a).all(), name
        assert _max_rel(a, b) < 1e-11, name


def test_backward_equals_autograd_through_recurrent():
    # the reference's recurrent-vs-chunkwise gradient test, shape of test_kda_chunkwise_equivalence.py:92-113
    inputs, d_out, d_final = _core(1, 5, 2, 2, 3, seed=3)
    ref = _autograd(lambda *x: ora.recurrent(*x)[:2], inputs, d_out, d_final)
    got = ora.chunkwise_backward(*inputs, d_out, d_final, chunk_size=3)
    for a, b in zip(got, ref):
        torch.testing.assert_close(a, b, rtol=2e-10, atol=2e-11)


def test_backward_without_final_state_gradient_or_initial_state():
    (q, k, v, g, beta, _), d_out, _ = _core(1, 19, 1, 4, 4, seed=4)
    leaves = [t.clone().requires_grad_() for t in (q, k, v, g, beta)]
    out, _ = ora.chunkwise(*leaves, None, chunk_size=8, secondary_tile_size=4)
    ref = torch.autograd.grad((out * d_out).sum(), leaves)
    got = ora.chunkwise_backward(q, k, v, g, beta, None, d_out, None, chunk_size=8)
    for a, b in zip(got[:5], ref):
        assert _max_rel(a, b) < 1e-11


def test_backward_is_chunk_size_invariant():
    inputs, d_out, d_final = _core(1, 48, 2, 6, 5, seed=5)
    a = ora.chunkwise_backward(*inputs, d_out, d_final, chunk_size=4)
    b = ora.chunkwise_backward(*inputs, d_out, d_final, chunk_size=16)
    for x, y in zip(a, b):
        assert _max_rel(x, y) < 1e-11


def test_chunkwise_gradcheck():
    # the reference's gradcheck, test_kda_chunkwise_equivalence.py:116-134
    inputs, _, _ = _core(1, 3, 1, 2, 2, seed=6)
    leaves = tuple(t.clone().requires_grad_() for t in inputs)
    assert torch.autograd.gradcheck(lambda *x: ora.chunkwise(*x, chunk_size=2, secondary_tile_size=1), leaves,
                                    fast_mode=True)


def test_planted_mistake_is_caught():
    # a transposed Aqk in dVt (a plausible slip) breaks agreement with autograd
    inputs, d_out, d_final = _core(1, 16, 1, 4, 4, seed=7)
    ref = _autograd(lambda *x: ora.chunkwise(*x, chunk_size=8, secondary_tile_size=4), inputs, d_out, d_final)
    original = torch.Tensor.transpose

    def wrong_transpose(self, d0, d1):  # turns Aqk^T into Aqk for square 8x8 chunk matrices
        if self.dim() == 4 and self.shape[-1] == self.shape[-2] == 8 and (d0, d1) == (-2, -1):
            return self
        return original(self, d0, d1)

    torch.Tensor.transpose = wrong_transpose
    try:
        got = ora.chunkwise_backward(*inputs, d_out, d_final, chunk_size=8)
    finally:
        torch.Tensor.transpose = original
    assert max(_max_rel(a, b) for a, b in zip(got, ref)) > 1e-3
