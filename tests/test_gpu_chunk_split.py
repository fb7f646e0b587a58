"""GPU parity of the split-bf16 chunk path: the chunkwise prefill for dense
calls that the bf16 MFMA path does not take (f32 inputs, bf16/f16 with key or
value dims off its grid), K and V up to 128, against the CPU oracle.

Tolerance (max|x - ref| / max|ref|, per tensor): f32 inputs <= 1e-4 against
the f64 oracle (the scalar C recurrence, oracle/kda_recurrent_ref.c, or the
chunkwise restatement); bf16 inputs <= 2e-2 against the f32 oracle on the same
values.  Every case checks the output and the final state.
"""

from __future__ import annotations

import ctypes

import pytest
import torch

import kda
from kda import _lib
from oracle import c_oracle
from oracle import kda_oracle as ora
from tests._inputs import random_core, record_margin, rel_err, workload

pytestmark = pytest.mark.gpu
DEV = "cuda"
TOL32 = 1e-4
TOL16 = 2e-2


def _dev(*ts):
    return [None if t is None else t.to(DEV) for t in ts]


def _plan(B, T, H, K, V, dtype):
    L, segs = ctypes.c_int64(0), ctypes.c_int64(0)
    _lib.check(_lib.load().kda_chunk_fwd_plan(B, B * T, 0, H, K, V, _lib.dtype_code(dtype), ctypes.byref(L),
                                              ctypes.byref(segs)))
    return L.value


def _check(got, ro, rs, tol, label, record=False):
    eo, es = rel_err(got.hidden_states, ro), rel_err(got.final_state, rs)
    print(f"{label}: output rel err {eo:.2e}  state rel err {es:.2e}")
    if record:
        record_margin(label, tol, output=eo, final_state=es)
    assert eo < tol and es < tol, (label, eo, es)


def test_f32_long_context_full_length():
    # B=1, T=8192, H=16, K=V=128 in f32 with an N(0, 0.02) initial state: the
    # split-bf16 chunk path; two heads checked at full length against the
    # f64 scalar recurrence
    assert _plan(1, 8192, 16, 128, 128, torch.float32) == -2
    q, k, v, g, beta, state = workload(1, 8192, 16, 128, 128, state_std=0.02, seed=41, dtype=torch.float32)
    got = kda.chunkwise_kda(*_dev(q, k, v, g, beta, state), True)
    assert got.hidden_states.dtype == torch.float32 and got.final_state.dtype == torch.float32
    for h in (2, 13):
        sl = slice(h, h + 1)
        ro, rs = c_oracle.recurrent_ref(q[:, :, sl], k[:, :, sl], v[:, :, sl], g[:, :, sl], beta[:, :, sl],
                                        state[:, sl])
        _check(kda.KDAOperatorOutput(got.hidden_states[:, :, sl], got.final_state[:, sl]), ro, rs, TOL32,
               f"prefill B=1 T=8192 H=16 K=V=128 f32, N(0,0.02) state, head {h}", record=True)


@pytest.mark.parametrize(
    "shape",
    [
        (1, 1, 1, 128, 128),    # a single token
        (1, 64, 1, 128, 128),   # exactly one chunk
        (2, 200, 2, 128, 128),  # partial last chunk
        (2, 130, 3, 128, 64),
        (1, 150, 2, 64, 64),    # the gpu_48gb head (K = V = 64)
        (1, 100, 2, 40, 32),    # K off the MFMA grid
        (2, 70, 2, 16, 16),
        (1, 97, 2, 3, 5),       # tiny, odd dims
        (1, 80, 2, 128, 100),   # V not a multiple of 32
        (1, 66, 1, 65, 128),    # K just above 64 (padded to 128)
    ],
)
def test_f32_shapes_match_f64_oracle(shape):
    q, k, v, g, beta, state = workload(*shape, state_std=0.02, seed=42, dtype=torch.float32)
    assert _plan(*shape, torch.float32) == -2
    ro, rs = c_oracle.recurrent_ref(q, k, v, g, beta, state)
    got = kda.chunkwise_kda(*_dev(q, k, v, g, beta, state), True)
    _check(got, ro, rs, TOL32, f"f32 {shape}")


def test_f32_reference_fixture_decays_without_state():
    # the reference fixture's distributions (g = -5 U(0,1), beta = U(0,1),
    # tests/kda/conftest.py:27-55) with normalised q, k and no initial state:
    # the final state starts from zero
    q, k, v, g, beta, _ = random_core(2, 150, 2, 64, 48, dtype=torch.float32, seed=43)
    q, k = (torch.nn.functional.normalize(t, dim=-1) for t in (q, k))
    ro, rs = c_oracle.recurrent_ref(q, k, v, g, beta)
    got = kda.chunkwise_kda(*_dev(q, k, v, g, beta), None, True)
    _check(got, ro, rs, TOL32, "f32 fixture decays")


def test_f32_right_padding_mask():
    # attention mask as right padding: padded positions give zero output and
    # leave the state untouched (src/kda/utils.py:82-94)
    B, T, H, K, V = 3, 140, 2, 128, 64
    q, k, v, g, beta, state = workload(B, T, H, K, V, state_std=0.02, seed=44, dtype=torch.float32)
    lens = [140, 77, 1]
    mask = torch.zeros(B, T, dtype=torch.bool)
    for b, n in enumerate(lens):
        mask[b, :n] = True
    ro, rs = c_oracle.recurrent_ref(q, k, v, g, beta, state, valid=lens)
    got = kda.chunkwise_kda(*_dev(q, k, v, g, beta, state), True, mask.to(DEV))
    _check(got, ro, rs, TOL32, "f32 right padding")
    assert torch.count_nonzero(got.hidden_states[1, 77:]) == 0 and torch.count_nonzero(got.hidden_states[2, 1:]) == 0


def test_f32_rising_and_near_zero_decays():
    # g = 0.02 N(0, 1) (both signs) and one chunk of moderately positive g: such
    # chunks take the exact pairwise-exponent products
    B, T, H, K, V = 1, 200, 2, 64, 64
    q, k, v, _, beta, state = workload(B, T, H, K, V, state_std=0.02, seed=45, dtype=torch.float32)
    gen = torch.Generator().manual_seed(46)
    g = 0.02 * torch.randn(B, T, H, K, generator=gen)
    g[:, 64:128] = 0.05 * torch.rand(B, 64, H, K, generator=gen)
    ro, rs = c_oracle.recurrent_ref(q, k, v, g, beta, state)
    got = kda.chunkwise_kda(*_dev(q, k, v, g, beta, state), True)
    _check(got, ro, rs, TOL32, "f32 rising decays")


def test_bf16_off_grid_key_dim():
    # bf16 with K = 40 (not a multiple of 16): the split path, checked against
    # the f32 oracle on the same values
    assert _plan(1, 100, 2, 40, 32, torch.bfloat16) == -2
    q, k, v, g, beta, state = workload(1, 100, 2, 40, 32, state_std=0.02, seed=47)
    ro, rs = ora.chunkwise(*(t.float() for t in (q, k, v, g, beta)), state, None, chunk_size=64,
                           secondary_tile_size=16)
    got = kda.chunkwise_kda(*_dev(q, k, v, g, beta, state), True)
    assert got.hidden_states.dtype == torch.bfloat16
    _check(got, ro, rs, TOL16, "bf16 K=40")


def test_split_path_equals_the_recurrence_kernel():
    # the same sequences dense, as packed documents with their longest length
    # (gathered into a padded batch on the split path) and as packed documents
    # without it (the exact recurrence kernel): the three agree, and the split
    # path refuses a missing workspace
    B, T, H, K, V = 2, 150, 2, 64, 32
    q, k, v, g, beta, state = _dev(*workload(B, T, H, K, V, state_std=0.02, seed=48, dtype=torch.float32))
    lib = _lib.load()
    code = _lib.dtype_code(torch.float32)
    stream = _lib.stream_of(q.device)
    cu = torch.tensor([0, T, 2 * T], dtype=torch.int32, device=DEV)
    outs = []
    for packed, span in ((False, T), (True, T), (True, 0)):
        out = torch.empty(B, T, H, V, device=DEV)
        s_out = torch.empty(B, H, K, V, device=DEV)
        # (packed documents without their longest length need no workspace)
        n = 0 if packed and span == 0 else lib.kda_chunk_fwd_workspace_bytes(B, B * T, span if packed else 0, H, K,
                                                                             V, code)
        ws = torch.empty(n, dtype=torch.uint8, device=DEV) if n else None
        _lib.check(lib.kda_chunk_fwd(q.data_ptr(), k.data_ptr(), v.data_ptr(), g.data_ptr(), beta.data_ptr(), code,
                                     state.data_ptr(), s_out.data_ptr(), code, out.data_ptr(),
                                     cu.data_ptr() if packed else None, span, None, B, B * T, H, K, V, _lib.ptr(ws),
                                     n, stream))
        outs.append((out, s_out))
    torch.cuda.synchronize()
    # each path is within about 1e-5 of the f64 oracle (the split products keep ~2^-17)
    for o, s in outs[1:]:
        assert rel_err(outs[0][0], o) < TOL32 and rel_err(outs[0][1], s) < TOL32
    # the padded batch runs the same kernels on the same values as the dense call
    assert torch.equal(outs[0][0], outs[1][0]) and torch.equal(outs[0][1], outs[1][1])
    status = lib.kda_chunk_fwd(q.data_ptr(), k.data_ptr(), v.data_ptr(), g.data_ptr(), beta.data_ptr(), code,
                               None, None, code, outs[0][0].data_ptr(), None, T, None, B, B * T, H, K, V, None, 0,
                               stream)
    assert status == _lib.KDA_ERR_WORKSPACE


def _packed(lens, H, K, V, dtype, seed):
    cu = [0]
    for n in lens:
        cu.append(cu[-1] + n)
    q, k, v, g, beta, _ = workload(1, cu[-1], H, K, V, seed=seed, dtype=dtype)
    s0 = torch.randn(len(lens), H, K, V, generator=torch.Generator().manual_seed(seed)) * 0.02
    return cu, (q, k, v, g, beta), s0


@pytest.mark.parametrize("dtype,K,V", [(torch.float32, 128, 128), (torch.float32, 64, 200), (torch.bfloat16, 40, 72),
                                       (torch.float16, 128, 40), (torch.bfloat16, 128, 320)])
def test_packed_documents_off_the_mfma_path(dtype, K, V):
    # packed documents that the bf16 MFMA path does not take (f32 inputs, key
    # or value dims off its grid, V past 256) run the split-bf16 chunk path on
    # a zero-padded batch: every document against the f64 scalar recurrence
    lens = [130, 1, 64, 257]
    H = 2
    cu, ins, s0 = _packed(lens, H, K, V, dtype, seed=50 + K + V)
    assert _plan(len(lens), cu[-1], H, K, V, dtype) == -2
    got = kda.chunkwise_kda(*_dev(*ins, s0), True, cu_seqlens=cu)
    assert got.hidden_states.dtype == dtype and got.final_state.shape == (len(lens), H, K, V)
    tol = TOL32 if dtype == torch.float32 else TOL16
    for d in range(len(lens)):
        a, b = cu[d], cu[d + 1]
        ro, rs = c_oracle.recurrent_ref(*(t[:, a:b] for t in ins), s0[d:d + 1])
        _check(kda.KDAOperatorOutput(got.hidden_states[:, a:b], got.final_state[d:d + 1]), ro, rs, tol,
               f"packed {dtype} K={K} V={V} document {d} ({b - a} tokens)")


@pytest.mark.parametrize("dtype,V", [(torch.float32, 200), (torch.bfloat16, 272)])
def test_value_dims_past_the_slices(dtype, V):
    # dense calls with V past 128 (f32) or past 256 (bf16) run in column slices
    # of at most 128: right padding, an initial state, against the f64 recurrence
    B, T, H, K = 2, 150, 2, 64
    q, k, v, g, beta, state = workload(B, T, H, K, V, state_std=0.02, seed=52, dtype=dtype)
    assert _plan(B, T, H, K, V, dtype) == -2
    mask = torch.ones(B, T, dtype=torch.bool)
    mask[0, 120:] = False
    got = kda.chunkwise_kda(*_dev(q, k, v, g, beta, state), True, mask.to(DEV))
    ro, rs = c_oracle.recurrent_ref(q, k, v, g, beta, state, valid=[120, T])
    _check(got, ro, rs, TOL32 if dtype == torch.float32 else TOL16, f"{dtype} V={V} slices")


def test_packed_f32_long_document():
    # one 8192-token f32 document at H=16 (the long-context shape) through the
    # packed path equals the dense call bit for bit (the padded batch is the
    # dense batch), two heads checked against the f64 recurrence
    q, k, v, g, beta, state = workload(1, 8192, 16, 128, 128, state_std=0.02, seed=53, dtype=torch.float32)
    args = _dev(q, k, v, g, beta, state)
    dense = kda.chunkwise_kda(*args, True)
    packed = kda.chunkwise_kda(*args, True, cu_seqlens=[0, 8192])
    assert torch.equal(dense.hidden_states, packed.hidden_states)
    assert torch.equal(dense.final_state, packed.final_state)
    for h in (4, 9):
        sl = slice(h, h + 1)
        ro, rs = c_oracle.recurrent_ref(q[:, :, sl], k[:, :, sl], v[:, :, sl], g[:, :, sl], beta[:, :, sl],
                                        state[:, sl])
        _check(kda.KDAOperatorOutput(packed.hidden_states[:, :, sl], packed.final_state[:, sl]), ro, rs, TOL32,
               f"packed f32 T=8192 head {h}")


@pytest.mark.parametrize("dtype,K", [(torch.float32, 128), (torch.bfloat16, 100)])
def test_prefill_in_head_groups(monkeypatch, dtype, K):
    # a dense prefill on the split-bf16 chunk path (f32 inputs, or bf16 off the
    # MFMA grid) whose workspace passes WORKSPACE_LIMIT runs its heads in
    # groups (5 heads in groups of 2, 2 and 1, with right padding): output and
    # final state equal the single call's (to rounding: the groups' plans
    # differ) and the recurrence's
    from kda import chunkwise

    B, T, H, V = 2, 150, 5, 64
    q, k, v, g, beta, state = workload(B, T, H, K, V, state_std=0.02, seed=45, dtype=dtype)
    mask = torch.ones(B, T, dtype=torch.bool)
    mask[1, 90:] = False
    args = (*_dev(q, k, v, g, beta, state), True, mask.to(DEV))
    whole = kda.chunkwise_kda(*args)
    lib = _lib.load()
    code = _lib.dtype_code(dtype)
    limit = lib.kda_chunk_fwd_workspace_bytes(B, B * T, 0, 2, K, V, code)
    assert lib.kda_chunk_fwd_workspace_bytes(B, B * T, 0, 3, K, V, code) > limit
    monkeypatch.setattr(chunkwise, "WORKSPACE_LIMIT", limit)
    grouped = kda.chunkwise_kda(*args)
    ro, rs = c_oracle.recurrent_ref(q, k, v, g, beta, state, valid=[T, 90])
    same = 1e-5 if dtype == torch.float32 else 1e-2
    assert rel_err(grouped.hidden_states, whole.hidden_states) < same
    assert rel_err(grouped.final_state, whole.final_state) < same
    _check(grouped, ro, rs, TOL32 if dtype == torch.float32 else TOL16, f"{dtype} head groups")
