"""GPU parity of the operator flags and the public UT transform at full chunk size.

``accumulate_state_in_fp32=False`` with bf16 inputs makes the reference's
work dtype bf16 (src/kda/utils.py:74-79): every input and the initial state
are rounded to bf16 (src/kda/chunkwise.py:41-58, src/kda/recurrent.py:42-59),
the arithmetic runs in bf16 and the final state comes back in bf16.  This
backend rounds the same inputs and state, computes in f32 on them and returns
the output and the final state in bf16.  Checked:
* dtypes: output bf16, final state bf16;
* against the oracle with the same flag (its bf16-arithmetic recurrence; the
  reference's chunkwise form cannot run in bf16 on the CPU, whose triangular
  solve has no bf16 kernel, and equals the recurrence in exact arithmetic):
  2e-2 (the bf16 recurrence itself sits 6e-3 off the f32 result here);
* against the f32 oracle on the rounded inputs and state: 2e-2;
* against this backend's own f32-work call on the rounded state: the same
  output bit for bit, and the final state equal to its bf16 rounding.

The public ``ut_transform`` (src/kda/ut_transform.py:61-92) at C = 64 and
K = V = 128: bf16 inputs against the f64 oracle on the same values (2e-2,
the results are bf16), f32 inputs at 1e-4.
"""

from __future__ import annotations

import pytest
import torch

import kda
from oracle import kda_oracle as ora
from tests._inputs import rel_err, workload

pytestmark = pytest.mark.gpu
DEV = "cuda"
TOL16 = 2e-2


def _dev(*ts):
    return [None if t is None else t.to(DEV) for t in ts]


@pytest.mark.parametrize("mode", ["chunkwise", "recurrent", "decode"])
def test_bf16_work_dtype_matches_oracle_with_the_same_flag(mode):
    T = {"chunkwise": 200, "recurrent": 70, "decode": 1}[mode]
    q, k, v, g, beta, s0 = workload(2, T, 2, 128, 128, state_std=0.02, seed=61)
    mask = None
    if mode != "decode":
        mask = torch.ones(2, T, dtype=torch.bool)
        mask[1, T - 9:] = False
    op = kda.chunkwise_kda if mode == "chunkwise" else kda.recurrent_kda
    got = op(*_dev(q, k, v, g, beta, s0), True, None if mask is None else mask.to(DEV),
             accumulate_state_in_fp32=False)
    assert got.hidden_states.dtype == torch.bfloat16 and got.final_state.dtype == torch.bfloat16
    # the oracle with the same flag: bf16 arithmetic on the bf16-rounded state
    bo, bs, _ = ora.recurrent(q, k, v, g, beta, s0, mask, accumulate_state_in_fp32=False)
    assert bs.dtype == torch.bfloat16
    # the f32 oracle on the same rounded inputs and state
    ro, rs, _ = ora.recurrent(*(t.float() for t in (q, k, v, g, beta)), s0.to(torch.bfloat16).float(), mask)
    e_same, s_same = rel_err(got.hidden_states, bo), rel_err(got.final_state, bs)
    e32, s32 = rel_err(got.hidden_states, ro), rel_err(got.final_state, rs)
    print(f"{mode} bf16 work: vs bf16 oracle {e_same:.2e}/{s_same:.2e}, vs f32 oracle {e32:.2e}/{s32:.2e}")
    assert e_same < TOL16 and s_same < TOL16 and e32 < TOL16 and s32 < TOL16
    # the same kernels as the f32-work call on the rounded state
    ref = op(*_dev(q, k, v, g, beta, s0.to(torch.bfloat16).float()), True,
             None if mask is None else mask.to(DEV))
    assert torch.equal(got.hidden_states, ref.hidden_states)
    assert torch.equal(got.final_state, ref.final_state.to(torch.bfloat16))


def test_bf16_work_dtype_rounds_mixed_inputs():
    # v in bf16 sets the work dtype; q, k, g, beta given in f32 are rounded to
    # bf16 first, as the reference's casts do
    q, k, v, g, beta, s0 = workload(1, 90, 2, 64, 64, state_std=0.02, seed=62, dtype=torch.float32)
    got = kda.chunkwise_kda(*_dev(q, k, v.to(torch.bfloat16), g, beta, s0), True, accumulate_state_in_fp32=False)
    rounded = [t.to(torch.bfloat16) for t in (q, k, v, g, beta)]
    ref = kda.chunkwise_kda(*_dev(*rounded, s0.to(torch.bfloat16).float()), True)
    assert torch.equal(got.hidden_states, ref.hidden_states)
    assert torch.equal(got.final_state, ref.final_state.to(torch.bfloat16))


@pytest.mark.parametrize("dtype,tol", [(torch.bfloat16, 2e-2), (torch.float32, 1e-4)])
def test_ut_transform_full_chunk_matches_oracle(dtype, tol):
    # B=1, C=64, H=2, K=V=128 with the workload's distributions (q, k
    # L2-normalised, g = -softplus(N(0,1) + 2), beta = sigmoid(N(0,1)))
    _, k, v, g, beta, _ = workload(1, 64, 2, 128, 128, seed=63, dtype=dtype)
    got = kda.ut_transform(*_dev(k, v, g, beta), secondary_tile_size=16)
    for t in (got.M, got.U, got.W, got.log_gamma, got.k_gamma):
        assert t.dtype == dtype
    ki, vi, gi, bi = (t.double().transpose(1, 2) for t in (k, v, g, beta))
    ref = ora.ut_transform_internal(ki, vi, gi, bi, 16)
    errs = {
        "M": rel_err(got.M, ref["M"]),
        "U": rel_err(got.U.transpose(1, 2), ref["U"]),
        "W": rel_err(got.W.transpose(1, 2), ref["W"]),
        "log_gamma": rel_err(got.log_gamma.transpose(1, 2), ref["log_gamma"]),
        "k_gamma": rel_err(got.k_gamma.transpose(1, 2), ref["k_gamma"]),
    }
    print(f"ut_transform {dtype} C=64 K=V=128: " + " ".join(f"{n} {e:.2e}" for n, e in errs.items()))
    assert all(e < tol for e in errs.values()), errs
