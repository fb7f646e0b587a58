"""Seeded synthetic KDA inputs shared by the tests.

``random_core`` draws the same distributions as the reference's test fixture
(tests/kda/conftest.py:27-55: q,k,v ~ N(0,1), g = -5 U(0,1), beta = U(0,1),
a random initial state).  ``workload`` draws the benchmark workloads: q, k
L2-normalised N(0,1), v ~ N(0,1), beta = sigmoid(N(0,1)), per-channel
g = -softplus(N(0,1) + shift), state ~ N(0, state_std).
"""

from __future__ import annotations

import torch


def random_core(batch=2, tokens=7, heads=3, key_dim=2, value_dim=4, dtype=torch.float64, seed=11):
    gen = torch.Generator().manual_seed(seed)
    q = torch.randn(batch, tokens, heads, key_dim, generator=gen, dtype=dtype)
    k = torch.randn(batch, tokens, heads, key_dim, generator=gen, dtype=dtype)
    v = torch.randn(batch, tokens, heads, value_dim, generator=gen, dtype=dtype)
    g = -5 * torch.rand(batch, tokens, heads, key_dim, generator=gen, dtype=dtype)
    beta = torch.rand(batch, tokens, heads, generator=gen, dtype=dtype)
    state = torch.randn(batch, heads, key_dim, value_dim, generator=gen, dtype=dtype)
    return q, k, v, g, beta, state


def workload(batch, tokens, heads, key_dim, value_dim, *, g_shift=2.0, state_std=None, seed=0,
             dtype=torch.bfloat16):
    """Returns (q, k, v, g, beta, state) on the CPU; inputs in `dtype`, state f32."""
    gen = torch.Generator().manual_seed(seed)
    shape_k = (batch, tokens, heads, key_dim)
    q = torch.nn.functional.normalize(torch.randn(shape_k, generator=gen), dim=-1)
    k = torch.nn.functional.normalize(torch.randn(shape_k, generator=gen), dim=-1)
    v = torch.randn(batch, tokens, heads, value_dim, generator=gen)
    g = -torch.nn.functional.softplus(torch.randn(shape_k, generator=gen) + g_shift)
    beta = torch.sigmoid(torch.randn(batch, tokens, heads, generator=gen))
    state = None
    if state_std is not None:
        state = torch.randn(batch, heads, key_dim, value_dim, generator=gen) * state_std
    cast = lambda t: t.to(dtype)  # noqa: E731
    return cast(q), cast(k), cast(v), cast(g), cast(beta), state


def rel_err(actual: torch.Tensor, expected: torch.Tensor) -> float:
    """max |actual - expected| / max |expected| (per-tensor relative error)."""
    a = actual.detach().double().cpu()
    e = expected.detach().double().cpu()
    scale = e.abs().max().item()
    diff = (a - e).abs().max().item()
    return diff / scale if scale > 0 else diff
