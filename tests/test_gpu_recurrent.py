"""GPU parity of the recurrence / decode kernels against the CPU oracle.

Tolerances (per tensor, max|x - ref| / max|ref|):
* f64 inputs: 1e-10 against the f64 oracle;
* f32 inputs: 1e-4 against the f64 oracle;
* bf16 inputs: 2e-2 against the f32 oracle on the same bf16 inputs
  (the reference upcasts bf16 exactly, src/kda/recurrent.py:42-46).
"""

from __future__ import annotations

import math

import pytest
import torch

import kda
from oracle import kda_oracle as ora
from tests._inputs import random_core, rel_err, workload

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _to(dev, *ts):
    return [None if t is None else t.to(dev) for t in ts]


@pytest.mark.parametrize("shape", [(1, 1, 1, 1, 1), (2, 7, 3, 2, 5), (1, 17, 1, 3, 5), (2, 31, 2, 16, 16),
                                   (1, 9, 2, 128, 128), (1, 5, 1, 200, 33)])
def test_recurrent_f64_matches_oracle(shape):
    q, k, v, g, beta, state = random_core(*shape)
    ro, rs, _ = ora.recurrent(q, k, v, g, beta, state)
    got = kda.recurrent_kda(*_to(DEV, q, k, v, g, beta, state), output_final_state=True)
    assert got.hidden_states.dtype == torch.float64 and got.final_state.dtype == torch.float64
    assert rel_err(got.hidden_states, ro) < 1e-10
    assert rel_err(got.final_state, rs) < 1e-10


@pytest.mark.parametrize("shape", [(2, 32, 2, 16, 16), (1, 40, 3, 128, 128), (2, 9, 2, 64, 48)])
def test_recurrent_f32_within_1e4(shape):
    q, k, v, g, beta, state = random_core(*shape, dtype=torch.float32)
    ro, rs, _ = ora.recurrent(*(t.double() for t in (q, k, v, g, beta, state)))
    got = kda.recurrent_kda(*_to(DEV, q, k, v, g, beta, state), output_final_state=True)
    assert got.hidden_states.dtype == torch.float32
    assert rel_err(got.hidden_states, ro) < 1e-4
    assert rel_err(got.final_state, rs) < 1e-4


@pytest.mark.parametrize("shape", [(2, 24, 4, 128, 128), (1, 12, 2, 32, 64)])
def test_recurrent_bf16_within_2e2(shape):
    q, k, v, g, beta, state = workload(*shape, state_std=0.02, seed=1)
    ro, rs, _ = ora.recurrent(q, k, v, g, beta, state)
    got = kda.recurrent_kda(*_to(DEV, q, k, v, g, beta, state), output_final_state=True)
    assert got.hidden_states.dtype == torch.bfloat16 and got.final_state.dtype == torch.float32
    assert rel_err(got.hidden_states, ro.float()) < 2e-2
    assert rel_err(got.final_state, rs) < 2e-2


def test_known_answers_on_gpu():
    one = torch.tensor([[[[1.0]]]], dtype=torch.float64, device=DEV)
    out = kda.recurrent_kda(one, one, 3 * one, 0 * one, torch.ones(1, 1, 1, dtype=torch.float64, device=DEV))
    assert out.hidden_states.item() == 3.0
    res = kda.recurrent_kda(one, one, 0 * one, math.log(0.5) * one,
                            torch.full((1, 1, 1), 0.5, dtype=torch.float64, device=DEV), 2 * one, True)
    assert abs(res.final_state.item() - 0.5) < 1e-15


def test_mask_and_states_per_token():
    q, k, v, g, beta, state = random_core(batch=2, tokens=6, heads=2, key_dim=3, value_dim=4)
    mask = torch.tensor([[True] * 6, [True] * 4 + [False] * 2])
    ro, rs, rh = ora.recurrent(q, k, v, g, beta, state, mask, return_states=True)
    got = kda.recurrent_kda(*_to(DEV, q, k, v, g, beta, state), True, mask.to(DEV), return_states_per_token=True)
    assert rel_err(got.hidden_states, ro) < 1e-10
    assert rel_err(got.final_state, rs) < 1e-10
    assert torch.count_nonzero(got.hidden_states[1, 4:]) == 0
    assert len(got.states_per_token) == 6
    for a, b in zip(got.states_per_token, rh):
        assert rel_err(a, b) < 1e-10


def test_varlen_recurrent_matches_per_document():
    q, k, v, g, beta, _ = random_core(batch=1, tokens=40, heads=2, key_dim=16, value_dim=8)
    cu = [0, 7, 8, 33, 40]
    init = torch.randn(4, 2, 16, 8, dtype=torch.float64)
    ro, rs = ora.varlen_recurrent(q, k, v, g, beta, cu, init)
    got = kda.recurrent_kda(*_to(DEV, q, k, v, g, beta, init), True,
                            cu_seqlens=torch.tensor(cu, dtype=torch.int32, device=DEV))
    assert rel_err(got.hidden_states, ro) < 1e-10
    assert rel_err(got.final_state, rs) < 1e-10


def test_decode_in_place_matches_token_loop():
    B, H, K, V = 4, 3, 128, 128
    q, k, v, g, beta, state = workload(B, 6, H, K, V, state_std=0.02, seed=2)
    ro, rs, _ = ora.recurrent(q, k, v, g, beta, state)
    s = state.to(DEV).contiguous()
    outs = []
    for t in range(6):
        step = kda.recurrent_kda(*_to(DEV, q[:, t:t + 1], k[:, t:t + 1], v[:, t:t + 1], g[:, t:t + 1],
                                      beta[:, t:t + 1]), s, True, update_state_in_place=True)
        assert step.final_state.data_ptr() == s.data_ptr()
        outs.append(step.hidden_states)
    assert rel_err(torch.cat(outs, 1), ro.float()) < 2e-2
    assert rel_err(s, rs) < 2e-2


def test_functional_decode_leaves_input_state_untouched():
    q, k, v, g, beta, state = workload(2, 1, 2, 128, 128, state_std=0.02, seed=3)
    s = state.to(DEV)
    before = s.clone()
    res = kda.recurrent_kda(*_to(DEV, q, k, v, g, beta), s, True)
    assert torch.equal(s, before)
    assert res.final_state.data_ptr() != s.data_ptr()


def test_decode_full_size_subset_parity():
    # B=256, H=32, K=V=128 f32 state (512 MiB), updated in place for several
    # steps; sequences and heads are independent, so a sampled subset of
    # (b, h) pairs is checked against the oracle run on that subset only.
    B, H, K, V, steps = 256, 32, 128, 128, 3
    gen = torch.Generator(device="cpu").manual_seed(7)
    s = (torch.randn(B, H, K, V, generator=gen) * 0.02).to(DEV)
    s0_rows = {}
    picks = [(0, 0), (17, 5), (128, 31), (255, 16)]
    for b, h in picks:
        s0_rows[(b, h)] = s[b, h].cpu().clone()
    q, k, v, g, beta, _ = workload(B, steps, H, K, V, seed=8)
    outs = []
    for t in range(steps):
        res = kda.recurrent_kda(*_to(DEV, q[:, t:t + 1], k[:, t:t + 1], v[:, t:t + 1], g[:, t:t + 1],
                                     beta[:, t:t + 1]), s, True, update_state_in_place=True)
        outs.append(res.hidden_states.cpu())
    out = torch.cat(outs, 1)
    final = s.cpu()
    for b, h in picks:
        sl = lambda x: x[b:b + 1, :, h:h + 1]  # noqa: E731
        ro, rs, _ = ora.recurrent(sl(q), sl(k), sl(v), sl(g), beta[b:b + 1, :, h:h + 1],
                                  s0_rows[(b, h)][None, None])
        assert rel_err(out[b:b + 1, :, h:h + 1], ro.float()) < 2e-2
        assert rel_err(final[b, h][None, None], rs) < 2e-2


def test_ut_transform_matches_oracle():
    _, k, v, g, beta, _ = random_core(batch=2, tokens=9, heads=2, key_dim=5, value_dim=3)
    ki, vi, gi, bi = k.transpose(1, 2), v.transpose(1, 2), g.transpose(1, 2), beta.transpose(1, 2)
    ref = ora.ut_transform_internal(ki, vi, gi, bi, 4)
    got = kda.ut_transform(*_to(DEV, k, v, g, beta), secondary_tile_size=4)
    assert rel_err(got.M, ref["M"]) < 1e-10
    assert rel_err(got.W.transpose(1, 2), ref["W"]) < 1e-10
    assert rel_err(got.U.transpose(1, 2), ref["U"]) < 1e-10
    assert rel_err(got.log_gamma.transpose(1, 2), ref["log_gamma"]) < 1e-12
    assert rel_err(got.k_gamma.transpose(1, 2), ref["k_gamma"]) < 1e-10


@pytest.mark.parametrize("dtype,tol", [(torch.float64, 1e-10), (torch.float32, 1e-4)])
@pytest.mark.parametrize("shape", [(2, 9, 2, 5, 3), (1, 64, 2, 128, 64), (1, 37, 3, 16, 128), (2, 1, 1, 8, 4)])
def test_ut_transform_gradients_match_oracle_autograd(dtype, tol, shape):
    # ut_transform under autograd (the reference's transform is plain torch,
    # src/kda/ut_transform.py:23-92): every output carries a gradient
    B, C, H, K, V = shape
    _, k, v, g, beta, _ = random_core(batch=B, tokens=C, heads=H, key_dim=K, value_dim=V, dtype=torch.float64,
                                      seed=C + K)
    k = torch.nn.functional.normalize(k, dim=-1)
    leaves = [t.to(dtype) for t in (k, v, g, beta)]
    gpu = [t.to(DEV).requires_grad_() for t in leaves]
    cpu = [t.double().requires_grad_() for t in leaves]
    gen = torch.Generator().manual_seed(3)
    w_m = torch.randn(B, H, C, C, generator=gen, dtype=torch.float64)
    w_u = torch.randn(B, C, H, V, generator=gen, dtype=torch.float64)
    w_w, w_l, w_k = (torch.randn(B, C, H, K, generator=gen, dtype=torch.float64) for _ in range(3))
    out = kda.ut_transform(*gpu, secondary_tile_size=4)
    ((out.M.double() * w_m.to(DEV)).sum() + (out.U.double() * w_u.to(DEV)).sum()
     + (out.W.double() * w_w.to(DEV)).sum() + (out.log_gamma.double() * w_l.to(DEV)).sum()
     + (out.k_gamma.double() * w_k.to(DEV)).sum()).backward()
    ki, vi, gi, bi = (t.transpose(1, 2) for t in cpu)
    ref = ora.ut_transform_internal(ki, vi, gi, bi, 4)
    ((ref["M"] * w_m).sum() + (ref["U"].transpose(1, 2) * w_u).sum() + (ref["W"].transpose(1, 2) * w_w).sum()
     + (ref["log_gamma"].transpose(1, 2) * w_l).sum() + (ref["k_gamma"].transpose(1, 2) * w_k).sum()).backward()
    for name, a, b in zip("kvgb", gpu, cpu):
        e = rel_err(a.grad, b.grad)
        print(f"ut_transform {dtype} {shape} d{name}: {e:.2e}")
        assert e < tol, (name, e)


@pytest.mark.parametrize("dtype,tol", [(torch.float64, 1e-10), (torch.float32, 1e-4)])
def test_states_per_token_gradients_match_oracle_autograd(dtype, tol):
    # recurrent_kda(return_states_per_token=True) under autograd: every returned
    # state carries a gradient (kda_recurrent_bwd); the oracle's token loop,
    # differentiated by torch autograd in f64 on the CPU, is the reference
    q, k, v, g, beta, state = random_core(batch=2, tokens=6, heads=2, key_dim=3, value_dim=4)
    mask = torch.tensor([[True] * 6, [True] * 4 + [False] * 2])
    gen = torch.Generator().manual_seed(5)
    d_out = torch.randn(2, 6, 2, 4, generator=gen, dtype=torch.float64)
    d_states = [torch.randn(2, 2, 3, 4, generator=gen, dtype=torch.float64) for _ in range(6)]
    d_final = torch.randn(2, 2, 3, 4, generator=gen, dtype=torch.float64)

    def loss(out, final, states):
        total = (out.double() * d_out.to(out.device)).sum() + (final.double() * d_final.to(out.device)).sum()
        return total + sum((s.double() * d.to(out.device)).sum() for s, d in zip(states, d_states))

    ref_leaves = [t.clone().requires_grad_() for t in (q, k, v, g, beta, state)]
    ro, rs, rh = ora.recurrent(*ref_leaves, mask, return_states=True)
    loss(ro, rs, rh).backward()
    leaves = [t.to(dtype).to(DEV).requires_grad_() for t in (q, k, v, g, beta, state)]
    got = kda.recurrent_kda(*leaves, True, mask.to(DEV), return_states_per_token=True)
    loss(got.hidden_states, got.final_state, got.states_per_token).backward()
    for name, a, b in zip(("dq", "dk", "dv", "dg", "dbeta", "ds0"), leaves, ref_leaves):
        assert a.grad.dtype == dtype, name
        assert rel_err(a.grad, b.grad) < tol, (name, rel_err(a.grad, b.grad))


def test_states_per_token_gradcheck():
    q, k, v, g, beta, state = random_core(batch=1, tokens=3, heads=1, key_dim=2, value_dim=2)
    leaves = tuple(t.to(DEV).requires_grad_() for t in (q, k, v, g, beta, state))

    def function(*xs):
        res = kda.recurrent_kda(*xs, True, return_states_per_token=True)
        return (res.hidden_states, res.final_state, *res.states_per_token)

    assert torch.autograd.gradcheck(function, leaves, fast_mode=True)
