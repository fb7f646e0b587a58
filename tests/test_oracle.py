"""Pins the CPU oracle (oracle/kda_oracle.py) before the GPU results are compared with it.

Each oracle function is checked against something other than its own formula:
the reference's literal known-answer tests, closed forms, an explicit matrix
inverse, brute-force pairwise sums, an independent scalar C implementation
(oracle/kda_recurrent_ref.c) and the chunkwise == recurrent identity.  The
mutation tests at the end plant plausible mistakes in copies of the oracle and
show that these pins catch them.
"""

from __future__ import annotations

import math

import pytest
import torch

from oracle import c_oracle
from oracle import kda_oracle as ora
from tests._inputs import random_core

F64 = torch.float64


def _kat_failures(recurrent_fn) -> list[str]:
    """Literal known-answer tests from the reference (tests/kda/test_kda_recurrent.py:70-139)."""
    failures = []
    one = torch.tensor([[[[1.0]]]], dtype=F64)
    # read after write: q=k=1, v=3, g=0, beta=1 -> o = 3   (:70-76)
    o, _, _ = recurrent_fn(one, one, 3 * one, 0 * one, torch.ones(1, 1, 1, dtype=F64))
    if not torch.equal(o, 3 * one):
        failures.append("read-after-write")
    # decay before error and update: S0=2, alpha=.5, beta=.5, v=0 -> S = 0.5   (:79-89)
    _, s, _ = recurrent_fn(one, one, 0 * one, math.log(0.5) * one, torch.full((1, 1, 1), 0.5, dtype=F64),
                           2 * one)
    if not torch.allclose(s, 0.5 * one, rtol=0, atol=1e-15):
        failures.append("decay-before-update")
    # beta = 0 only decays the state   (:92-97)
    q, k, v, g, beta, state = random_core(tokens=4)
    _, s, _ = recurrent_fn(q, k, v, g, torch.zeros_like(beta), state)
    if not torch.allclose(s, state * g.sum(dim=1).exp()[..., None], rtol=1e-12, atol=1e-12):
        failures.append("beta-zero")
    # zero state: first write is beta k v^T   (:108-114)
    q, k, v, g, beta, _ = random_core(batch=1, tokens=1, heads=2, key_dim=3, value_dim=4)
    _, s, _ = recurrent_fn(q, k, v, g, beta)
    expect = (beta[:, 0, :, None] * k[:, 0]).unsqueeze(-1) * v[:, 0].unsqueeze(-2)
    if not torch.allclose(s, expect, rtol=1e-12, atol=1e-12):
        failures.append("first-write")
    # zero reconstruction error means no update   (:117-127)
    kk = torch.tensor([[[[1.0, 0.0]]]], dtype=F64)
    gg = torch.log(torch.tensor([[[[0.5, 0.8]]]], dtype=F64))
    s0 = torch.tensor([[[[0.3, -1.2, 2.0], [0.7, 0.1, -0.4]]]], dtype=F64)
    decayed = s0 * gg[:, 0].exp()[..., None]
    vv = (decayed * kk[:, 0].unsqueeze(-1)).sum(-2)[:, None]
    _, s, _ = recurrent_fn(kk.clone(), kk, vv, gg, torch.ones(1, 1, 1, dtype=F64), s0)
    if not torch.allclose(s, decayed, rtol=1e-12, atol=1e-12):
        failures.append("zero-error")
    # unit key, beta=1, g=0: the new state recalls v in the key direction   (:130-139)
    q, k, v, g, beta, state = random_core(batch=1, tokens=1, heads=1, key_dim=3, value_dim=2)
    k = torch.nn.functional.normalize(k, dim=-1)
    _, s, _ = recurrent_fn(q, k, v, torch.zeros_like(g), torch.ones_like(beta), state)
    recalled = (s * k[:, 0].unsqueeze(-1)).sum(-2)
    if not torch.allclose(recalled, v[:, 0], rtol=1e-12, atol=1e-12):
        failures.append("unit-key-recall")
    # matrix form S' = (I - beta k k^T) diag(alpha) S + beta k v^T   (:48-67)
    q, k, v, g, beta, state = random_core(batch=1, tokens=1, heads=1, key_dim=2, value_dim=3)
    alpha = g[:, 0].exp()
    ident = torch.eye(2, dtype=F64).reshape(1, 1, 2, 2)
    trans = ident - beta[:, 0, :, None, None] * k[:, 0].unsqueeze(-1) * k[:, 0].unsqueeze(-2)
    expect = trans @ (alpha[..., None] * state) + (beta[:, 0, :, None] * k[:, 0]).unsqueeze(-1) * v[:, 0].unsqueeze(-2)
    _, s, _ = recurrent_fn(q, k, v, g, beta, state)
    if not torch.allclose(s, expect, rtol=1e-12, atol=1e-12):
        failures.append("matrix-form")
    return failures


def _oracle_recurrent(q, k, v, g, beta, state=None):
    return ora.recurrent(q, k, v, g, beta, state)


def test_recurrent_known_answers():
    assert _kat_failures(_oracle_recurrent) == []


@pytest.mark.parametrize("shape", [(1, 5, 2, 2, 3), (2, 9, 3, 4, 5), (1, 33, 1, 16, 16)])
def test_recurrent_matches_independent_scalar_c(shape):
    q, k, v, g, beta, state = random_core(*shape)
    o, s, _ = ora.recurrent(q, k, v, g, beta, state)
    co, cs = c_oracle.recurrent_ref(q, k, v, g, beta, state)
    torch.testing.assert_close(o, co, rtol=1e-12, atol=1e-12)
    torch.testing.assert_close(s, cs, rtol=1e-12, atol=1e-12)


def test_recurrent_mask_matches_c_and_freezes_state():
    q, k, v, g, beta, state = random_core(batch=2, tokens=6, heads=2, key_dim=3, value_dim=4)
    mask = torch.tensor([[True] * 6, [True] * 4 + [False] * 2])
    o, s, hist = ora.recurrent(q, k, v, g, beta, state, mask, return_states=True)
    co, cs = c_oracle.recurrent_ref(q, k, v, g, beta, state, valid=[6, 4])
    torch.testing.assert_close(o, co, rtol=1e-12, atol=1e-12)
    torch.testing.assert_close(s, cs, rtol=1e-12, atol=1e-12)
    assert torch.count_nonzero(o[1, 4:]) == 0
    torch.testing.assert_close(hist[3][1], hist[5][1], rtol=0, atol=0)


def test_recurrent_batch_and_head_independence():
    q, k, v, g, beta, state = random_core(batch=2, heads=3)
    base, _, _ = ora.recurrent(q, k, v, g, beta, state)
    v2 = v.clone()
    v2[1, :, 2] += 100
    changed, _, _ = ora.recurrent(q, k, v2, g, beta, state)
    torch.testing.assert_close(base[0], changed[0], rtol=0, atol=0)
    torch.testing.assert_close(base[1, :, :2], changed[1, :, :2], rtol=0, atol=0)


def test_tiled_decay_dot_matches_brute_force():
    gen = torch.Generator().manual_seed(3)
    left = torch.randn(1, 2, 7, 3, generator=gen, dtype=F64)
    right = torch.randn(1, 2, 7, 3, generator=gen, dtype=F64)
    lg = -torch.rand(1, 2, 7, 3, generator=gen, dtype=F64).cumsum(2)
    for diag in (True, False):
        got = ora.tiled_causal_decay_dot(left, right, lg, lg, 3, include_diagonal=diag)
        want = torch.zeros(1, 2, 7, 7, dtype=F64)
        for h in range(2):
            for i in range(7):
                for j in range(7):
                    if j < i or (diag and j == i):
                        want[0, h, i, j] = sum(
                            left[0, h, i, c] * math.exp(lg[0, h, i, c] - lg[0, h, j, c]) * right[0, h, j, c]
                            for c in range(3)
                        )
        torch.testing.assert_close(got, want, rtol=1e-13, atol=1e-13)


@pytest.mark.parametrize("tile", [1, 2, 3, 8])
def test_ut_transform_tile_invariance(tile):
    _, k, v, g, beta, _ = random_core(batch=1, tokens=7, heads=2, key_dim=3, value_dim=4)
    ki, vi, gi, bi = k.transpose(1, 2), v.transpose(1, 2), g.transpose(1, 2), beta.transpose(1, 2)
    base = ora.ut_transform_internal(ki, vi, gi, bi, 1)
    got = ora.ut_transform_internal(ki, vi, gi, bi, tile)
    for key in ("M", "W", "U"):
        torch.testing.assert_close(got[key], base[key], rtol=0, atol=0)


def test_ut_transform_matches_explicit_inverse_and_forward_substitution():
    _, k, v, g, beta, _ = random_core(batch=2, tokens=6, heads=2, key_dim=3, value_dim=4)
    ki, vi, gi, bi = k.transpose(1, 2), v.transpose(1, 2), g.transpose(1, 2), beta.transpose(1, 2)
    got = ora.ut_transform_internal(ki, vi, gi, bi, 2)
    C = ki.shape[2]
    lg = gi.cumsum(2)
    lower = torch.eye(C, dtype=F64).expand(2, 2, C, C).clone()
    for i in range(C):
        for j in range(i):
            lower[:, :, i, j] = bi[:, :, i] * (ki[:, :, i] * (lg[:, :, i] - lg[:, :, j]).exp() * ki[:, :, j]).sum(-1)
    m_inv = torch.linalg.inv(lower) @ torch.diag_embed(bi)
    kgam = lg.exp() * ki
    torch.testing.assert_close(got["M"], m_inv, rtol=1e-11, atol=1e-12)
    torch.testing.assert_close(got["W"], m_inv @ kgam, rtol=1e-11, atol=1e-12)
    torch.testing.assert_close(got["U"], m_inv @ vi, rtol=1e-11, atol=1e-12)
    # row-by-row forward substitution (tests/kda/test_kda_ut_transform.py:54-74)
    w_rows, u_rows = [], []
    for i in range(C):
        w_i = bi[:, :, i, None] * kgam[:, :, i]
        u_i = bi[:, :, i, None] * vi[:, :, i]
        for j in range(i):
            w_i = w_i - lower[:, :, i, j, None] * w_rows[j]
            u_i = u_i - lower[:, :, i, j, None] * u_rows[j]
        w_rows.append(w_i)
        u_rows.append(u_i)
    torch.testing.assert_close(got["W"], torch.stack(w_rows, 2), rtol=1e-11, atol=1e-12)
    torch.testing.assert_close(got["U"], torch.stack(u_rows, 2), rtol=1e-11, atol=1e-12)


SHAPES = [(1, 1, 1, 1, 1), (1, 2, 1, 2, 3), (2, 7, 3, 2, 5), (1, 16, 2, 4, 3), (1, 17, 1, 3, 5),
          (2, 31, 2, 1, 3), (1, 65, 1, 2, 1)]


@pytest.mark.parametrize("shape", SHAPES)
@pytest.mark.parametrize("chunk", [1, 2, 4, 8, 16])
def test_chunkwise_equals_recurrent_float64(shape, chunk):
    inputs = random_core(*shape)
    ro, rs, _ = ora.recurrent(*inputs)
    co, cs = ora.chunkwise(*inputs, chunk_size=chunk, secondary_tile_size=min(chunk, 4))
    torch.testing.assert_close(co, ro, rtol=2e-11, atol=2e-12)
    torch.testing.assert_close(cs, rs, rtol=2e-11, atol=2e-12)


def test_chunkwise_partial_chunks_and_chunk64():
    inputs = random_core(tokens=19, key_dim=3, value_dim=5)
    ro, rs, _ = ora.recurrent(*inputs)
    for chunk in (1, 2, 4, 8, 16, 64):
        co, cs = ora.chunkwise(*inputs, chunk_size=chunk, secondary_tile_size=min(chunk, 4))
        torch.testing.assert_close(co, ro, rtol=2e-11, atol=2e-12)
        torch.testing.assert_close(cs, rs, rtol=2e-11, atol=2e-12)


@pytest.mark.parametrize("prefix", range(1, 9))
def test_chunkwise_prefix_causality(prefix):
    q, k, v, g, beta, state = random_core(tokens=9)
    base, _ = ora.chunkwise(q, k, v, g, beta, state, chunk_size=4, secondary_tile_size=2)
    changed = [t.clone() for t in (q, k, v, g, beta)]
    for t in changed:
        t[:, prefix:] = torch.randn_like(t[:, prefix:]) * 50
    got, _ = ora.chunkwise(*changed, state, chunk_size=4, secondary_tile_size=2)
    torch.testing.assert_close(base[:, :prefix], got[:, :prefix], rtol=0, atol=0)


def test_chunkwise_mask_equals_truncated_run():
    q, k, v, g, beta, state = random_core(batch=1, tokens=9, heads=2, key_dim=3, value_dim=4)
    mask = torch.tensor([[True] * 6 + [False] * 3])
    co, cs = ora.chunkwise(q, k, v, g, beta, state, mask, chunk_size=4, secondary_tile_size=2)
    vo, vs, _ = ora.recurrent(q[:, :6], k[:, :6], v[:, :6], g[:, :6], beta[:, :6], state)
    torch.testing.assert_close(co[:, :6], vo)
    assert torch.count_nonzero(co[:, 6:]) == 0
    torch.testing.assert_close(cs, vs)


def test_chunkwise_finite_for_long_negative_decay():
    q, k, v, _, beta, state = random_core(batch=1, tokens=96, heads=1, key_dim=4, value_dim=3, dtype=torch.float32)
    g = torch.full_like(q, -4.999)
    o, s = ora.chunkwise(q, k, v, g, beta, state, chunk_size=64, secondary_tile_size=16)
    assert torch.isfinite(o).all() and torch.isfinite(s).all()


def test_bf16_inputs_upcast_exactly():
    # bf16 inputs: the work dtype is f32 and the inputs are upcast exactly, so
    # the oracle on bf16 inputs equals the oracle on the same values in f32.
    q, k, v, g, beta, state = random_core(batch=1, tokens=9, heads=2, key_dim=4, value_dim=4, dtype=torch.float32)
    b16 = [t.to(torch.bfloat16) for t in (q, k, v, g, beta)]
    o_b, s_b = ora.chunkwise(*b16, state, chunk_size=4, secondary_tile_size=2)
    o_f, s_f = ora.chunkwise(*(t.float() for t in b16), state, chunk_size=4, secondary_tile_size=2)
    assert o_b.dtype == torch.bfloat16 and s_b.dtype == torch.float32
    torch.testing.assert_close(o_b, o_f.to(torch.bfloat16), rtol=0, atol=0)
    torch.testing.assert_close(s_b, s_f, rtol=0, atol=0)


def test_varlen_documents_are_independent():
    q, k, v, g, beta, _ = random_core(batch=1, tokens=23, heads=2, key_dim=3, value_dim=4)
    cu = [0, 5, 17, 23]
    init = torch.randn(3, 2, 3, 4, dtype=F64, generator=torch.Generator().manual_seed(5))
    o, s = ora.varlen_chunkwise(q, k, v, g, beta, cu, init, chunk_size=4, secondary_tile_size=2)
    ro, rs = ora.varlen_recurrent(q, k, v, g, beta, cu, init)
    torch.testing.assert_close(o, ro, rtol=2e-11, atol=2e-12)
    torch.testing.assert_close(s, rs, rtol=2e-11, atol=2e-12)
    # the middle document equals a stand-alone run from its own initial state
    mo, ms, _ = ora.recurrent(q[:, 5:17], k[:, 5:17], v[:, 5:17], g[:, 5:17], beta[:, 5:17], init[1:2])
    torch.testing.assert_close(o[:, 5:17], mo, rtol=2e-11, atol=2e-12)
    torch.testing.assert_close(s[1:2], ms, rtol=2e-11, atol=2e-12)
    # changing the first document does not leak into the second (state reset)
    q2 = q.clone()
    q2[:, :5] += 3.0
    k2 = k.clone()
    k2[:, :5] -= 1.0
    o2, s2 = ora.varlen_chunkwise(q2, k2, v, g, beta, cu, init, chunk_size=4, secondary_tile_size=2)
    torch.testing.assert_close(o2[:, 5:], o[:, 5:], rtol=0, atol=0)
    torch.testing.assert_close(s2[1:], s[1:], rtol=0, atol=0)


# ---------------------------------------------------------------------------
# Mutation tests: plausible mistakes planted in copies of the oracle are caught.

def _mutant(kind):
    def run(q, k, v, g, beta, state=None):
        B, T, H, K = q.shape
        V = v.shape[-1]
        S = torch.zeros(B, H, K, V, dtype=F64) if state is None else state.clone().to(F64)
        outs = []
        for t in range(T):
            a = g[:, t].exp().unsqueeze(-1)
            if kind == "update-before-decay":
                err = v[:, t] - (S * k[:, t].unsqueeze(-1)).sum(-2)
                S = S + (beta[:, t].unsqueeze(-1) * k[:, t]).unsqueeze(-1) * err.unsqueeze(-2)
                S = S * a
            else:
                S = S * a
                err = v[:, t] - (S * k[:, t].unsqueeze(-1)).sum(-2)
                bk = k[:, t] if kind == "dropped-beta" else beta[:, t].unsqueeze(-1) * k[:, t]
                upd = bk.unsqueeze(-1) * err.unsqueeze(-2)
                S = S + upd
            if kind == "read-before-write":
                outs.append(((S - (beta[:, t].unsqueeze(-1) * k[:, t]).unsqueeze(-1) * err.unsqueeze(-2))
                             * q[:, t].unsqueeze(-1)).sum(-2))
            elif kind == "transposed-read" and K == V:
                outs.append((S * q[:, t].unsqueeze(-2)).sum(-1))
            else:
                outs.append((S * q[:, t].unsqueeze(-1)).sum(-2))
        return torch.stack(outs, 1), S, None

    return run


def _pin_failures(recurrent_fn) -> list[str]:
    """Known answers plus the comparison with the scalar C implementation."""
    failures = _kat_failures(recurrent_fn)
    q, k, v, g, beta, state = random_core(batch=1, tokens=5, heads=2, key_dim=3, value_dim=3)
    o, s, _ = recurrent_fn(q, k, v, g, beta, state)
    co, cs = c_oracle.recurrent_ref(q, k, v, g, beta, state)
    if not (torch.allclose(o, co, rtol=1e-12, atol=1e-12) and torch.allclose(s, cs, rtol=1e-12, atol=1e-12)):
        failures.append("scalar-c")
    return failures


def test_pin_suite_accepts_the_oracle():
    assert _pin_failures(_oracle_recurrent) == []


@pytest.mark.parametrize("kind", ["update-before-decay", "dropped-beta", "read-before-write", "transposed-read"])
def test_pins_catch_planted_mistakes(kind):
    assert _pin_failures(_mutant(kind)), f"mutation {kind!r} was not caught"


def test_chunk_identity_catches_sign_error_in_pseudo_values():
    inputs = random_core(batch=1, tokens=9, heads=1, key_dim=3, value_dim=2)
    ro, _, _ = ora.recurrent(*inputs)
    original = ora.ut_transform_internal

    def flipped(*args):
        out = original(*args)
        out["W"] = -out["W"]
        return out

    ora.ut_transform_internal = flipped
    try:
        co, _ = ora.chunkwise(*inputs, chunk_size=4, secondary_tile_size=2)
    finally:
        ora.ut_transform_internal = original
    assert not torch.allclose(co, ro, rtol=1e-6, atol=1e-6)
