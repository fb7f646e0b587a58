"""GPU parity at the full sizes of the benchmark configurations.

* B=8, T=1024, H=8, K=V=128, bf16, zero initial state, g = -softplus(N(0,1)+2):
  every head against the f32 oracle.
* Packed documents, cu_seqlens = [0, 32768, 49152, 61440, 65536], H=64,
  K=V=128, bf16: three heads of every document against the f32 oracle (heads
  are independent, so the oracle runs on those heads only), and the full
  packed call against separate calls on each document under the same
  one-segment-per-sequence schedule (each document's output and final state
  equal an independent call; size-independent).
* Decode B=256, H=32, K=V=128, f32 state updated in place for 64 steps: the
  sampled (sequence, head) pairs against the oracle recurrence.

Tolerance (max|x - ref| / max|ref| per tensor): 2e-2 for bf16 inputs against
the f32 oracle on the same (exactly upcast) values; 1e-6 between the packed
call and separate calls (the same kernels on the same values).
"""

from __future__ import annotations

import ctypes

import pytest
import torch

import kda
from kda import _lib
from oracle import kda_oracle as ora
from tests._inputs import record_margin, rel_err, workload

pytestmark = pytest.mark.gpu
DEV = "cuda"
TOL16 = 2e-2


def _gpu_workload(tokens, heads, key_dim, value_dim, seed):
    """[1, tokens, heads, *] bf16 inputs drawn on the GPU (q, k L2-normalised,
    g = -softplus(N(0,1) + 2), beta = sigmoid(N(0,1)))."""
    gen = torch.Generator(device=DEV).manual_seed(seed)
    shape_k = (1, tokens, heads, key_dim)
    q = torch.nn.functional.normalize(torch.randn(shape_k, generator=gen, device=DEV), dim=-1).bfloat16()
    k = torch.nn.functional.normalize(torch.randn(shape_k, generator=gen, device=DEV), dim=-1).bfloat16()
    v = torch.randn(1, tokens, heads, value_dim, generator=gen, device=DEV).bfloat16()
    g = (-torch.nn.functional.softplus(torch.randn(shape_k, generator=gen, device=DEV) + 2.0)).bfloat16()
    beta = torch.sigmoid(torch.randn(1, tokens, heads, generator=gen, device=DEV)).bfloat16()
    return q, k, v, g, beta


def test_prefill_b8_t1024_h8_full_size():
    q, k, v, g, beta, _ = workload(8, 1024, 8, 128, 128, seed=31)
    got = kda.chunkwise_kda(*(t.to(DEV) for t in (q, k, v, g, beta)), None, True)
    ro, rs = ora.chunkwise(*(t.float() for t in (q, k, v, g, beta)), None, None,
                           chunk_size=64, secondary_tile_size=16)
    eo = rel_err(got.hidden_states, ro)
    es = rel_err(got.final_state, rs)
    print(f"B=8 T=1024 H=8: output rel err {eo:.2e} state rel err {es:.2e}")
    record_margin("prefill B=8 T=1024 H=8 K=V=128 bf16 (all heads)", TOL16, output=eo, final_state=es)
    assert eo < TOL16 and es < TOL16


def test_prefill_packed_documents_h64_full_size(segments):
    cu = [0, 32768, 49152, 61440, 65536]
    H, K, V = 64, 128, 128
    q, k, v, g, beta = _gpu_workload(cu[-1], H, K, V, seed=32)
    cu_t = torch.tensor(cu, dtype=torch.int32, device=DEV)
    got = kda.chunkwise_kda(q, k, v, g, beta, None, True, cu_seqlens=cu_t)
    assert got.final_state.shape == (len(cu) - 1, H, K, V)
    cps, segs = ctypes.c_int64(0), ctypes.c_int64(0)
    _lib.check(_lib.load().kda_chunk_fwd_plan(len(cu) - 1, cu[-1], 32768, H, K, V, _lib.dtype_code(torch.bfloat16),
                                              ctypes.byref(cps), ctypes.byref(segs)))
    per_segment = cps.value
    assert per_segment > 0
    heads = [0, 31, 63]
    for d in range(len(cu) - 1):
        s0, s1 = cu[d], cu[d + 1]
        # the oracle on three heads of the document
        sl = lambda t: t[:, s0:s1, heads].float().cpu()  # noqa: E731
        ro, rs = ora.chunkwise(sl(q), sl(k), sl(v), sl(g), sl(beta), None, None,
                               chunk_size=64, secondary_tile_size=16)
        eo = rel_err(got.hidden_states[:, s0:s1, heads], ro)
        es = rel_err(got.final_state[d:d + 1, heads], rs)
        print(f"document {d} ({s1 - s0} tokens): output rel err {eo:.2e} state rel err {es:.2e}")
        record_margin(f"packed H=64 bf16, document {d} ({s1 - s0} tokens), heads {heads}", TOL16, output=eo,
                      final_state=es)
        assert eo < TOL16 and es < TOL16
        # the packed call equals a separate call on the document (all heads)
        # held to the packed call's schedule: 4 documents x 64 heads fill the
        # GPU, and the first document, twice the chunk-steps per CU of a
        # balanced pass, has every document cut into segments of that many
        # chunks (the library's plan for the longest document's hint)
        segments(per_segment)
        alone = kda.chunkwise_kda(q[:, s0:s1], k[:, s0:s1], v[:, s0:s1], g[:, s0:s1], beta[:, s0:s1], None, True)
        segments(-1)
        assert rel_err(got.hidden_states[:, s0:s1], alone.hidden_states) < 1e-6
        assert rel_err(got.final_state[d:d + 1], alone.final_state) < 1e-6


def test_decode_b256_h32_64_steps_in_place():
    B, H, K, V, steps = 256, 32, 128, 128, 64
    gen = torch.Generator(device="cpu").manual_seed(33)
    s = (torch.randn(B, H, K, V, generator=gen) * 0.02).to(DEV)
    picks = [(0, 0), (17, 5), (128, 31), (255, 16)]
    s0 = {p: s[p[0], p[1]].cpu().clone() for p in picks}
    q, k, v, g, beta, _ = workload(B, steps, H, K, V, seed=34)
    qd, kd, vd, gd, bd = (t.to(DEV) for t in (q, k, v, g, beta))
    outs = []
    for t in range(steps):
        res = kda.recurrent_kda(qd[:, t:t + 1], kd[:, t:t + 1], vd[:, t:t + 1], gd[:, t:t + 1], bd[:, t:t + 1], s,
                                True, update_state_in_place=True)
        outs.append(res.hidden_states[:, :, [p[1] for p in picks]].cpu())
    out = torch.cat(outs, 1)
    final = s.cpu()
    for i, (b, h) in enumerate(picks):
        sl = lambda x: x[b:b + 1, :, h:h + 1].float()  # noqa: E731
        ro, rs, _ = ora.recurrent(sl(q), sl(k), sl(v), sl(g), beta[b:b + 1, :, h:h + 1].float(), s0[(b, h)][None, None])
        eo = rel_err(out[b:b + 1, :, i:i + 1], ro)
        es = rel_err(final[b, h][None, None], rs)
        print(f"decode b={b} h={h}: output rel err {eo:.2e} state rel err {es:.2e}")
        record_margin(f"decode B=256 H=32 bf16, 64 in-place steps, b={b} h={h}", TOL16, output=eo, final_state=es)
        assert eo < TOL16 and es < TOL16
