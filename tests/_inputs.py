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


# Measured parity margins of the full-size tests: (test, tensor, error,
# tolerance) rows, written at the end of the session to the JSON file that
# KDA_PARITY_RECORD names (tests/conftest.py), when it is set.
MARGINS: list[dict] = []


def record_margin(case: str, tol: float, **errors: float) -> None:
    """Keep the measured errors of one parity check for the session record."""
    for tensor, err in errors.items():
        MARGINS.append({"case": case, "tensor": tensor, "rel_err": float(err), "tol": float(tol)})


def rel_err(actual: torch.Tensor, expected: torch.Tensor) -> float:
    """max |actual - expected| / max |expected| (per-tensor relative error)."""
    a = actual.detach().double().cpu()
    e = expected.detach().double().cpu()
    scale = e.abs().max().item()
    diff = (a - e).abs().max().item()
    return diff / scale if scale > 0 else diff


def layer_weights(d_model, heads, key_dim, value_dim, *, conv=4, rank=None, dtype=torch.float64, seed=17, std=0.1,
                  biases=False):
    """Seeded parameters of one KDA layer as a dict with the fields of
    ``kda.layer.KDALayerWeights`` (the reference's layouts,
    src/kda/projections.py:35-103, src/kda/decay.py:24-26, src/kda/kda.py:50-62).
    Linear weights N(0, std); ShortConv weights N(0, 0.3); b_alpha by the
    reference's FLA recipe (log-uniform dt in [1e-3, 1e-1], inverse softplus,
    projections.py:90-101); A_log = 0.1 N(0,1); RMSNorm weight 1 + 0.1 N(0,1)."""
    import math

    gen = torch.Generator().manual_seed(seed)
    rank = value_dim if rank is None else rank
    kw, vw = heads * key_dim, heads * value_dim
    rnd = lambda *shape, s=std: (torch.randn(*shape, generator=gen, dtype=torch.float64) * s).to(dtype)  # noqa: E731
    dt = torch.exp(torch.rand(heads, key_dim, generator=gen, dtype=torch.float64)
                   * (math.log(0.1) - math.log(0.001)) + math.log(0.001)).clamp_min(1e-4)
    w = dict(
        num_heads=heads, key_head_dim=key_dim, value_head_dim=value_dim,
        q_proj=rnd(kw, d_model), k_proj=rnd(kw, d_model), v_proj=rnd(vw, d_model),
        q_conv=rnd(kw, conv, s=0.3), k_conv=rnd(kw, conv, s=0.3), v_conv=rnd(vw, conv, s=0.3),
        beta_proj=rnd(heads, d_model), alpha_down=rnd(rank, d_model), alpha_up=rnd(kw, rank),
        b_alpha=(dt + torch.log(-torch.expm1(-dt))).to(dtype),
        a_log=(0.1 * torch.randn(heads, generator=gen, dtype=torch.float64)).float(),
        norm_weight=(1 + 0.1 * torch.randn(heads, value_dim, generator=gen, dtype=torch.float64)).to(dtype),
        gate_proj=rnd(d_model, d_model), output_proj=rnd(d_model, d_model),
        g_min=-5.0, eps=1e-6,
    )
    if biases:
        w.update(q_proj_bias=rnd(kw), k_proj_bias=rnd(kw), v_proj_bias=rnd(vw), q_conv_bias=rnd(kw),
                 k_conv_bias=rnd(kw), v_conv_bias=rnd(vw), beta_bias=rnd(heads), gate_bias=rnd(d_model),
                 output_bias=rnd(d_model))
    return w
