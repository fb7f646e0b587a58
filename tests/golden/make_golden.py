"""Writes the golden KDA fixtures in this folder from the float64 oracle.

The reference stores no golden vectors: its tests draw seeded inputs at run
time (tests/kda/conftest.py:27-55 of pablo-reyes8/kimi-k3-pytorch).  These
fixtures freeze seeded inputs and the oracle's float64 results so that the
GPU parity tests and the oracle itself are checked against fixed data.
Inputs that are bf16 in the workload are stored as the exact float32 values
of the bf16 numbers (bf16 -> f32 is exact), expected values as float64.

Usage:  python tests/golden/make_golden.py
"""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent
REPO = HERE.parents[1]
if str(REPO) not in sys.path:
    sys.path.insert(0, str(REPO))

from oracle import kda_oracle as ora  # noqa: E402
from tests._inputs import workload  # noqa: E402


def _np(t):
    return None if t is None else t.detach().cpu().numpy()


def _save(name, **arrays):
    arrays = {k: v for k, v in arrays.items() if v is not None}
    np.savez_compressed(HERE / name, **arrays)
    print(f"wrote {name}: " + ", ".join(f"{k}{tuple(v.shape)}" for k, v in arrays.items()))


def cpu_smoke():
    # B=2, T=32, H=2, K=V=16, f32, g = -softplus(N(0,1)), zero state, chunk 16
    q, k, v, g, beta, _ = workload(2, 32, 2, 16, 16, g_shift=0.0, seed=100, dtype=torch.float32)
    o, s, _ = ora.recurrent(*(t.double() for t in (q, k, v, g, beta)))
    _save("cpu_smoke_f32_B2_T32_H2_d16.npz", q=_np(q), k=_np(k), v=_np(v), g=_np(g), beta=_np(beta),
          out=_np(o), final_state=_np(s), chunk_size=np.array(16))


def prefill_bf16():
    # bf16 inputs, K=V=128, a partial chunk, N(0, 0.02) initial state
    q, k, v, g, beta, s0 = workload(1, 70, 1, 128, 128, state_std=0.02, seed=101)
    o, s = ora.chunkwise(*(t.double() for t in (q, k, v, g, beta)), s0.double(), chunk_size=64,
                         secondary_tile_size=16)
    _save("prefill_bf16_B1_T70_H1_d128.npz", q=_np(q.float()), k=_np(k.float()), v=_np(v.float()),
          g=_np(g.float()), beta=_np(beta.float()), initial_state=_np(s0), out=_np(o), final_state=_np(s))


def varlen_bf16():
    # packed documents with a state reset at each start, per-document states
    q, k, v, g, beta, _ = workload(1, 100, 1, 128, 32, seed=102)
    cu = [0, 40, 41, 100]
    init = torch.randn(3, 1, 128, 32, generator=torch.Generator().manual_seed(103)) * 0.02
    o, s = ora.varlen_chunkwise(*(t.double() for t in (q, k, v, g, beta)), cu, init.double(), chunk_size=64,
                                secondary_tile_size=16)
    _save("varlen_bf16_T100_H1_K128_V32.npz", q=_np(q.float()), k=_np(k.float()), v=_np(v.float()),
          g=_np(g.float()), beta=_np(beta.float()), initial_state=_np(init), cu_seqlens=np.array(cu, np.int32),
          out=_np(o), final_state=_np(s))


def decode_bf16():
    # one decode step for 3 sequences, 1 head, from a non-zero cached state
    q, k, v, g, beta, s0 = workload(3, 1, 1, 128, 128, state_std=0.02, seed=104)
    o, s, _ = ora.recurrent(*(t.double() for t in (q, k, v, g, beta)), s0.double())
    _save("decode_bf16_B3_H1_d128.npz", q=_np(q.float()), k=_np(k.float()), v=_np(v.float()),
          g=_np(g.float()), beta=_np(beta.float()), initial_state=_np(s0), out=_np(o), final_state=_np(s))


def masked_f64():
    # reference-fixture distributions (g = -5 U(0,1), beta = U(0,1)) with right padding
    gen = torch.Generator().manual_seed(105)
    B, T, H, K, V = 2, 9, 2, 3, 4
    q = torch.randn(B, T, H, K, generator=gen, dtype=torch.float64)
    k = torch.randn(B, T, H, K, generator=gen, dtype=torch.float64)
    v = torch.randn(B, T, H, V, generator=gen, dtype=torch.float64)
    g = -5 * torch.rand(B, T, H, K, generator=gen, dtype=torch.float64)
    beta = torch.rand(B, T, H, generator=gen, dtype=torch.float64)
    s0 = torch.randn(B, H, K, V, generator=gen, dtype=torch.float64)
    mask = torch.tensor([[True] * 9, [True] * 5 + [False] * 4])
    o, s, _ = ora.recurrent(q, k, v, g, beta, s0, mask)
    _save("masked_f64_B2_T9_H2_K3_V4.npz", q=_np(q), k=_np(k), v=_np(v), g=_np(g), beta=_np(beta),
          initial_state=_np(s0), attention_mask=_np(mask), out=_np(o), final_state=_np(s))


if __name__ == "__main__":
    cpu_smoke()
    prefill_bf16()
    varlen_bf16()
    decode_bf16()
    masked_f64()
