"""GPU parity of the chunkwise prefill (MFMA path for bf16/f16 with K <= 128 a
multiple of 16, the split-bf16 chunk path or the exact recurrence otherwise)
against the CPU oracle.

Tolerance (max|x - ref| / max|ref|, per tensor): bf16/f16 inputs <= 2e-2
against the f32 oracle run on the same (exactly upcast) inputs; f32 inputs
<= 1e-4 and f64 inputs <= 1e-10 against the f64 oracle.  Every case checks
both the output and the final state.
"""

from __future__ import annotations

import pytest
import torch

import kda
from oracle import kda_oracle as ora
from tests._inputs import random_core, record_margin, rel_err, workload

pytestmark = pytest.mark.gpu
DEV = "cuda"
TOL16 = 2e-2


def _dev(*ts):
    return [None if t is None else t.to(DEV) for t in ts]


def _oracle_f32(q, k, v, g, beta, state=None, mask=None):
    """The oracle on the same values in f32 (the reference upcasts bf16 exactly)."""
    o, s = ora.chunkwise(*(t.float() for t in (q, k, v, g, beta)), state, mask,
                         chunk_size=64, secondary_tile_size=16)
    return o, s


def _check(got, ref_o, ref_s, tol=TOL16, label=""):
    eo = rel_err(got.hidden_states, ref_o)
    es = rel_err(got.final_state, ref_s)
    print(f"{label} output rel err {eo:.2e}  state rel err {es:.2e}")
    assert eo < tol and es < tol, (eo, es)


@pytest.mark.parametrize(
    "shape,state_std,g_shift",
    [
        ((1, 64, 1, 128, 128), None, 2.0),     # exactly one chunk
        ((2, 200, 2, 128, 128), 0.02, 2.0),    # partial last chunk, initial state
        ((1, 1, 1, 128, 128), 0.02, 2.0),      # a single token
        ((2, 130, 3, 128, 64), 0.02, 2.0),     # V = 64
        ((1, 257, 2, 128, 256), 0.02, 2.0),    # V = 256
        ((1, 320, 2, 128, 128), 0.02, -2.0),   # slow decay: -softplus(N(0,1) - 2)
        ((1, 192, 2, 128, 128), 0.5, 0.0),     # larger state, moderate decay
    ],
)
def test_chunkwise_bf16_matches_oracle(shape, state_std, g_shift):
    q, k, v, g, beta, state = workload(*shape, g_shift=g_shift, state_std=state_std, seed=11)
    ro, rs = _oracle_f32(q, k, v, g, beta, state)
    got = kda.chunkwise_kda(*_dev(q, k, v, g, beta, state), True)
    assert got.hidden_states.dtype == torch.bfloat16 and got.final_state.dtype == torch.float32
    _check(got, ro, rs, label=str(shape))


def test_chunkwise_f16_matches_oracle():
    q, k, v, g, beta, state = workload(2, 150, 2, 128, 128, state_std=0.02, seed=12, dtype=torch.float16)
    ro, rs = _oracle_f32(q, k, v, g, beta, state)
    got = kda.chunkwise_kda(*_dev(q, k, v, g, beta, state), True)
    assert got.hidden_states.dtype == torch.float16
    _check(got, ro, rs, label="f16")


def test_chunkwise_reference_fixture_decays():
    # the reference test fixture's decay and beta distributions, g = -5 U(0,1)
    # (including near-zero decay) and beta = U(0,1) (tests/kda/conftest.py:27-55),
    # with q and k L2-normalised as the KDA module always feeds the operator
    # (src/kda/projections.py:188-203)
    q, k, v, g, beta, state = random_core(2, 100, 2, 128, 128, dtype=torch.float32, seed=13)
    q, k = (torch.nn.functional.normalize(t, dim=-1) for t in (q, k))
    q, k, v, g, beta = (t.to(torch.bfloat16) for t in (q, k, v, g, beta))
    ro, rs = _oracle_f32(q, k, v, g, beta, state)
    got = kda.chunkwise_kda(*_dev(q, k, v, g, beta, state), True)
    _check(got, ro, rs, label="uniform g, beta")


def test_chunkwise_mask_equals_truncated_runs():
    q, k, v, g, beta, state = workload(2, 150, 2, 128, 128, state_std=0.02, seed=14)
    lengths = [150, 77]
    mask = torch.arange(150)[None, :] < torch.tensor(lengths)[:, None]
    ro, rs = _oracle_f32(q, k, v, g, beta, state, mask)
    got = kda.chunkwise_kda(*_dev(q, k, v, g, beta, state), True, mask.to(DEV))
    _check(got, ro, rs, label="mask")
    assert torch.count_nonzero(got.hidden_states[1, 77:]) == 0
    # the padded row's final state equals the state of a run on the valid prefix only
    solo = kda.chunkwise_kda(*_dev(q[1:, :77], k[1:, :77], v[1:, :77], g[1:, :77], beta[1:, :77],
                                   state[1:]), True)
    assert rel_err(got.final_state[1:], solo.final_state) < 1e-6


def test_chunkwise_varlen_matches_per_document():
    q, k, v, g, beta, _ = workload(1, 300, 2, 128, 128, seed=15)
    cu = [0, 100, 164, 165, 300]
    init = torch.randn(4, 2, 128, 128, generator=torch.Generator().manual_seed(16)) * 0.02
    ro, rs = ora.varlen_chunkwise(*(t.float() for t in (q, k, v, g, beta)), cu, init,
                                  chunk_size=64, secondary_tile_size=16)
    got = kda.chunkwise_kda(*_dev(q, k, v, g, beta, init), True,
                            cu_seqlens=torch.tensor(cu, dtype=torch.int32, device=DEV))
    _check(got, ro, rs, label="varlen")
    # each document equals an independent call
    for d, (a, b) in enumerate(zip(cu[:-1], cu[1:])):
        solo = kda.chunkwise_kda(*_dev(q[:, a:b], k[:, a:b], v[:, a:b], g[:, a:b], beta[:, a:b], init[d:d + 1]),
                                 True)
        assert rel_err(got.hidden_states[:, a:b], solo.hidden_states) < 1e-6
        assert rel_err(got.final_state[d:d + 1], solo.final_state) < 1e-6


def test_chunkwise_dominant_document_is_cut_into_segments():
    # three documents at H=64 fill the GPU with one chain per (document, head),
    # and the first is eight times longer than the others: with the longest
    # document as the schedule's hint every document is cut into segments
    # (the plan asserted below); results equal independent per-document calls
    import ctypes

    from kda import _lib

    cu = [0, 2048, 2304, 2560]
    H = 64
    q, k, v, g, beta, _ = workload(1, cu[-1], H, 128, 128, seed=61)
    init = torch.randn(3, H, 128, 128, generator=torch.Generator().manual_seed(62)) * 0.02
    cps, segs = ctypes.c_int64(0), ctypes.c_int64(0)
    _lib.check(_lib.load().kda_chunk_fwd_plan(3, cu[-1], 2048, H, 128, 128, _lib.dtype_code(torch.bfloat16),
                                              ctypes.byref(cps), ctypes.byref(segs)))
    assert cps.value > 0  # segmented; without the hint the plan keeps one segment per document
    got = kda.chunkwise_kda(*_dev(q, k, v, g, beta, init), True, cu_seqlens=cu)
    for d, (a, b) in enumerate(zip(cu[:-1], cu[1:])):
        solo = kda.chunkwise_kda(*_dev(q[:, a:b], k[:, a:b], v[:, a:b], g[:, a:b], beta[:, a:b], init[d:d + 1]),
                                 True)
        assert rel_err(got.hidden_states[:, a:b], solo.hidden_states) < 1e-2, d
        assert rel_err(got.final_state[d:d + 1], solo.final_state) < 1e-2, d
    # two heads of the long document against the oracle
    hs = [0, 37]
    ro, rs = _oracle_f32(*(t[:, :2048, hs] for t in (q, k, v, g, beta)), init[0:1, hs])
    _check(type(got)(hidden_states=got.hidden_states[:, :2048, hs], final_state=got.final_state[0:1, hs]), ro, rs,
           label="dominant document")


def test_chunkwise_extreme_decay_takes_exact_path():
    # g = -4.999 everywhere: a 16-row block decays by e^-75 < 2^-100, so the
    # diagonal blocks use the exact pairwise-exponent path
    # (mirrors tests/kda/test_kda_chunkwise_equivalence.py:137-148 at K=128)
    q, k, v, _, beta, state = workload(1, 96, 2, 128, 128, state_std=0.02, seed=17)
    g = torch.full_like(q, -4.999)
    ro, rs = _oracle_f32(q, k, v, g, beta, state)
    got = kda.chunkwise_kda(*_dev(q, k, v, g, beta, state), True)
    assert torch.isfinite(got.hidden_states.float()).all() and torch.isfinite(got.final_state).all()
    _check(got, ro, rs, label="extreme decay")


@pytest.mark.parametrize("segment_chunks", [None, "1"])
@pytest.mark.parametrize("regime", ["mixed_small", "rising_chunk", "rising_block_past_2e100"])
def test_chunkwise_rising_decays(segments, regime, segment_chunks):
    # The reference operator accepts a decay of either sign (src/kda/utils.py:32-71).
    # mixed_small: g = 0.02 N(0,1) everywhere; rising_chunk: one whole chunk at
    # g = +0.3 (the chunk grows by e^19.2); rising_block_past_2e100: one 16-row
    # block at g = +5 (e^80 > 2^100, the exact diagonal path) followed by a
    # block at g = -5.  Both schedules: one segment per sequence and one chunk
    # per segment.
    if segment_chunks is not None:
        segments(int(segment_chunks))
    q, k, v, g, beta, state = workload(1, 200, 2, 128, 128, state_std=0.02, seed=19)
    gen = torch.Generator().manual_seed(23)
    if regime == "mixed_small":
        g = (0.02 * torch.randn(q.shape, generator=gen)).to(torch.bfloat16)
    elif regime == "rising_chunk":
        g = g.clone()
        g[:, 64:128] = 0.3
    else:
        g = g.clone()
        g[:, 80:96] = 5.0
        g[:, 96:112] = -5.0
    ro, rs = _oracle_f32(q, k, v, g, beta, state)
    assert torch.isfinite(ro).all() and torch.isfinite(rs).all()
    got = kda.chunkwise_kda(*_dev(q, k, v, g, beta, state), True)
    assert torch.isfinite(got.hidden_states.float()).all() and torch.isfinite(got.final_state).all()
    _check(got, ro, rs, label=f"{regime} L={segment_chunks}")


def test_chunkwise_zero_decay_delta_rule():
    # g = 0 (classic delta rule, no forgetting) over several chunks
    q, k, v, _, beta, state = workload(1, 256, 2, 128, 128, state_std=0.02, seed=18)
    g = torch.zeros_like(q)
    ro, rs = _oracle_f32(q, k, v, g, beta, state)
    got = kda.chunkwise_kda(*_dev(q, k, v, g, beta, state), True)
    _check(got, ro, rs, label="g=0")


def test_chunkwise_matches_gpu_recurrent_and_decode():
    q, k, v, g, beta, state = workload(2, 130, 2, 128, 128, state_std=0.02, seed=19)
    d = _dev(q, k, v, g, beta, state)
    chunked = kda.chunkwise_kda(*d, True)
    rec = kda.recurrent_kda(*d, True)
    assert rel_err(chunked.hidden_states, rec.hidden_states.float()) < TOL16
    assert rel_err(chunked.final_state, rec.final_state) < TOL16
    # prefill the first 70 tokens, then decode the rest token by token
    pre = kda.chunkwise_kda(*[t[:, :70] for t in d[:5]], d[5], True)
    s = pre.final_state.clone()
    outs = [pre.hidden_states]
    for t in range(70, 130):
        step = kda.recurrent_kda(*[x[:, t:t + 1] for x in d[:5]], s, True, update_state_in_place=True)
        outs.append(step.hidden_states)
    assert rel_err(torch.cat(outs, 1), rec.hidden_states.float()) < TOL16
    assert rel_err(s, rec.final_state) < TOL16


@pytest.mark.parametrize("shape", [(2, 7, 3, 2, 5), (1, 65, 1, 2, 1), (2, 31, 2, 16, 16)])
def test_chunkwise_f64_equals_oracle_recurrent(shape):
    # non-MFMA shapes/dtypes: exact recurrence kernel; chunkwise == recurrent at f64 precision
    inputs = random_core(*shape)
    ro, rs, _ = ora.recurrent(*inputs)
    got = kda.chunkwise_kda(*_dev(*inputs), True, chunk_size=4, secondary_tile_size=2)
    assert rel_err(got.hidden_states, ro) < 1e-10 and rel_err(got.final_state, rs) < 1e-10


@pytest.mark.parametrize("dtype,tol", [(torch.bfloat16, TOL16), (torch.float32, 1e-4)])
def test_chunkwise_key_dim_past_128_runs_the_recurrence_with_a_warning(dtype, tol):
    # K > 128: the chunk kernels hold at most 128 key channels, so the exact
    # token recurrence runs (kda_chunk_fwd_plan -1), with a RuntimeWarning
    assert _plan(1, 100, 2, 160, 32, dtype=dtype) == -1
    q, k, v, g, beta, state = workload(1, 100, 2, 160, 32, state_std=0.02, seed=29, dtype=dtype)
    ro, rs = _oracle_f32(q, k, v, g, beta, state)
    with pytest.warns(RuntimeWarning, match="key_dim 160 > 128"):
        got = kda.chunkwise_kda(*_dev(q, k, v, g, beta, state), True)
    assert rel_err(got.hidden_states, ro) < tol and rel_err(got.final_state, rs) < tol


def test_chunkwise_f32_cpu_smoke_config_within_1e4():
    # B=2, T=32, H=2, K=V=16, f32, chunk 16, g = -softplus(N(0,1)), zero state
    q, k, v, g, beta, _ = workload(2, 32, 2, 16, 16, g_shift=0.0, seed=0, dtype=torch.float32)
    ro, rs, _ = ora.recurrent(*(t.double() for t in (q, k, v, g, beta)))
    got = kda.chunkwise_kda(*_dev(q, k, v, g, beta), None, True, chunk_size=16, secondary_tile_size=16)
    assert rel_err(got.hidden_states, ro) < 1e-4 and rel_err(got.final_state, rs) < 1e-4


def _plan(B, T, H, K, V, dtype=torch.bfloat16):
    import ctypes

    from kda import _lib

    L, segs = ctypes.c_int64(0), ctypes.c_int64(0)
    _lib.check(_lib.load().kda_chunk_fwd_plan(B, B * T, 0, H, K, V, _lib.dtype_code(dtype), ctypes.byref(L),
                                              ctypes.byref(segs)))
    return L.value


def test_chunkwise_bf16_small_head_dim():
    # K = 16 runs the MFMA path with channels 16..127 zero-padded in the kernel
    assert _plan(2, 40, 3, 16, 32) >= 0
    q, k, v, g, beta, state = workload(2, 40, 3, 16, 32, state_std=0.02, seed=20)
    ro, rs = _oracle_f32(q, k, v, g, beta, state)
    got = kda.chunkwise_kda(*_dev(q, k, v, g, beta, state), True)
    _check(got, ro, rs, label="K=16")


@pytest.mark.parametrize("segment_chunks", [None, "1"])
@pytest.mark.parametrize(
    "shape",
    [
        (1, 300, 2, 64, 64),    # the gpu_48gb profile's head (K = V = 64)
        (2, 130, 2, 64, 128),   # K = 64, V = 128
        (1, 200, 3, 32, 48),
        (1, 150, 2, 96, 128),
        (2, 70, 2, 16, 16),     # the smallest key dim of the MFMA path
        (1, 150, 2, 64, 256),   # K = 64 with two full column groups
        (2, 100, 3, 32, 176),   # K = 32, the second column group 48 columns wide
    ],
)
def test_chunkwise_key_dims_below_128(segments, shape, segment_chunks):
    # the reference's chunk algorithm runs at any K (src/kda/chunkwise.py:61-102);
    # K <= 128, a multiple of 16, takes the MFMA path, padded to 128 channels in the kernel
    if segment_chunks is not None:
        segments(int(segment_chunks))
    assert _plan(*shape) >= 0 and _plan(*shape, dtype=torch.float32) == -2
    q, k, v, g, beta, state = workload(*shape, state_std=0.02, seed=24)
    ro, rs = _oracle_f32(q, k, v, g, beta, state)
    got = kda.chunkwise_kda(*_dev(q, k, v, g, beta, state), True)
    _check(got, ro, rs, label=f"{shape} L={segment_chunks}")


def test_chunkwise_key_dim_off_the_mfma_grid():
    # K = 40 (not a multiple of 16) runs the split-bf16 chunk path
    assert _plan(1, 100, 2, 40, 32) == -2
    q, k, v, g, beta, state = workload(1, 100, 2, 40, 32, state_std=0.02, seed=26)
    ro, rs = _oracle_f32(q, k, v, g, beta, state)
    _check(kda.chunkwise_kda(*_dev(q, k, v, g, beta, state), True), ro, rs, label="K=40")


def test_gpu_48gb_shape_full_length():
    # B=1, T=8192, H=16, K=V=64 bf16 (config/kimi_full_pipeline/gpu_48gb/model.yaml:19,
    # V = d_model / H): the segmented MFMA schedule; two heads checked at full
    # length against the oracle
    assert _plan(1, 8192, 16, 64, 64) > 0
    q, k, v, g, beta, state = workload(1, 8192, 16, 64, 64, state_std=0.02, seed=25)
    got = kda.chunkwise_kda(*_dev(q, k, v, g, beta, state), True)
    for h in (3, 14):
        sl = slice(h, h + 1)
        ro, rs = _oracle_f32(q[:, :, sl], k[:, :, sl], v[:, :, sl], g[:, :, sl], beta[:, :, sl], state[:, sl])
        eo = rel_err(got.hidden_states[:, :, sl], ro)
        es = rel_err(got.final_state[:, sl], rs)
        print(f"K=V=64 T=8192 head {h}: output rel err {eo:.2e} state rel err {es:.2e}")
        record_margin(f"prefill B=1 T=8192 H=16 K=V=64 bf16, head {h}", TOL16, output=eo, final_state=es)
        assert eo < TOL16 and es < TOL16


def test_long_context_full_length_single_head():
    # B=1, T=8192, H=16, K=V=128 bf16 with an N(0,0.02) initial state.  Heads are
    # independent, so two heads are checked at full length against the oracle
    # run on those heads only.
    q, k, v, g, beta, state = workload(1, 8192, 16, 128, 128, state_std=0.02, seed=21)
    got = kda.chunkwise_kda(*_dev(q, k, v, g, beta, state), True)
    for h in (0, 11):
        sl = slice(h, h + 1)
        ro, rs = _oracle_f32(q[:, :, sl], k[:, :, sl], v[:, :, sl], g[:, :, sl], beta[:, :, sl], state[:, sl])
        eo = rel_err(got.hidden_states[:, :, sl], ro)
        es = rel_err(got.final_state[:, sl], rs)
        print(f"T=8192 head {h}: output rel err {eo:.2e} state rel err {es:.2e}")
        record_margin(f"prefill B=1 T=8192 H=16 K=V=128 bf16, N(0,0.02) state, head {h}", TOL16, output=eo,
                      final_state=es)
        assert eo < TOL16 and es < TOL16


# ---------------------------------------------------------------------------
# Segmented schedule: the chunk chain is cut into segments whose affine state
# maps are composed (kda_set_segment_chunks forces the segment length; the
# default plan only segments when batch * heads is small).  The result must
# match the oracle whatever the segment length.

@pytest.mark.parametrize("chunks_per_segment", ["1", "2", "3"])
def test_chunkwise_segmented_matches_oracle(segments, chunks_per_segment):
    segments(int(chunks_per_segment))
    q, k, v, g, beta, state = workload(2, 64 * 10 + 17, 2, 128, 128, state_std=0.02, seed=31)
    ro, rs = _oracle_f32(q, k, v, g, beta, state)
    got = kda.chunkwise_kda(*_dev(q, k, v, g, beta, state), True)
    _check(got, ro, rs, label=f"segments of {chunks_per_segment} chunks")


@pytest.mark.parametrize("value_dim", [64, 256])
def test_chunkwise_segmented_value_widths(segments, value_dim):
    segments(2)
    q, k, v, g, beta, state = workload(1, 64 * 7 + 5, 2, 128, value_dim, state_std=0.02, seed=32)
    ro, rs = _oracle_f32(q, k, v, g, beta, state)
    got = kda.chunkwise_kda(*_dev(q, k, v, g, beta, state), True)
    _check(got, ro, rs, label=f"segmented V={value_dim}")


def test_chunkwise_segmented_varlen_and_slow_decay(segments):
    segments(2)
    q, k, v, g, beta, _ = workload(1, 600, 2, 128, 128, g_shift=-2.0, seed=33)
    cu = [0, 100, 164, 165, 600]
    init = torch.randn(4, 2, 128, 128, generator=torch.Generator().manual_seed(34)) * 0.02
    ro, rs = ora.varlen_chunkwise(*(t.float() for t in (q, k, v, g, beta)), cu, init,
                                  chunk_size=64, secondary_tile_size=16)
    got = kda.chunkwise_kda(*_dev(q, k, v, g, beta, init), True,
                            cu_seqlens=torch.tensor(cu, dtype=torch.int32, device=DEV))
    _check(got, ro, rs, label="segmented varlen, slow decay")


def test_chunkwise_segmented_mask_and_zero_decay(segments):
    segments(1)
    q, k, v, _, beta, state = workload(2, 300, 2, 128, 128, state_std=0.02, seed=35)
    g = torch.zeros_like(q)
    mask = torch.arange(300)[None, :] < torch.tensor([300, 130])[:, None]
    ro, rs = _oracle_f32(q, k, v, g, beta, state, mask)
    got = kda.chunkwise_kda(*_dev(q, k, v, g, beta, state), True, mask.to(DEV))
    _check(got, ro, rs, label="segmented mask, g=0")
    assert torch.count_nonzero(got.hidden_states[1, 130:]) == 0


def test_chunkwise_segmented_equals_single_segment(segments):
    q, k, v, g, beta, state = workload(1, 64 * 12, 3, 128, 128, state_std=0.02, seed=36)
    d = _dev(q, k, v, g, beta, state)
    segments(0)
    one = kda.chunkwise_kda(*d, True)
    segments(4)
    seg = kda.chunkwise_kda(*d, True)
    assert rel_err(seg.hidden_states, one.hidden_states.float()) < 1e-2
    assert rel_err(seg.final_state, one.final_state) < 1e-2
    # the first segment of a sequence runs the unsegmented kernel's arithmetic
    # except for the rounding of its Q~, Kgamma and K~ operands (the segmented
    # output pass rounds them once from f32, the unsegmented kernel twice,
    # through its decayed natural tiles): within two bf16 steps of the
    # largest output
    assert rel_err(seg.hidden_states[:, :256], one.hidden_states[:, :256].float()) < 8e-3
