"""Golden fixtures (tests/golden/*.npz, written by tests/golden/make_golden.py).

CPU: the oracle reproduces every fixture (a frozen record of its float64
results on seeded inputs).  GPU: the HIP path matches the fixtures within the
stated tolerances (max|x - ref| / max|ref| per tensor): f64 inputs 1e-10,
f32 inputs 1e-4, bf16 inputs 2e-2.
"""

from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import kda_oracle as ora
from tests._inputs import rel_err

GOLDEN = Path(__file__).resolve().parent / "golden"


def load(name):
    with np.load(GOLDEN / name) as z:
        return {key: torch.from_numpy(z[key]) for key in z.files}


def _inputs(f, dtype=None):
    ts = [f[n] for n in ("q", "k", "v", "g", "beta")]
    return [t.to(dtype) for t in ts] if dtype is not None else ts


def test_fixture_inventory():
    # the layer fixtures of the reference module are covered by test_layer_reference_fixture.py
    names = sorted(p.name for p in GOLDEN.glob("*.npz") if not p.name.startswith("layer_ref_"))
    assert names == [
        "cpu_smoke_f32_B2_T32_H2_d16.npz",
        "decode_bf16_B3_H1_d128.npz",
        "masked_f64_B2_T9_H2_K3_V4.npz",
        "prefill_bf16_B1_T70_H1_d128.npz",
        "varlen_bf16_T100_H1_K128_V32.npz",
    ]


def test_oracle_reproduces_cpu_smoke_fixture():
    f = load("cpu_smoke_f32_B2_T32_H2_d16.npz")
    o, s = ora.chunkwise(*_inputs(f, torch.float64), chunk_size=16, secondary_tile_size=16)
    assert rel_err(o, f["out"]) < 1e-12 and rel_err(s, f["final_state"]) < 1e-12
    # the f32 operator (chunk 16, as the configuration states) is within 1e-4 of it
    o32, s32 = ora.chunkwise(*_inputs(f), chunk_size=16, secondary_tile_size=16)
    assert rel_err(o32, f["out"]) < 1e-4 and rel_err(s32, f["final_state"]) < 1e-4


def test_oracle_reproduces_prefill_fixture():
    f = load("prefill_bf16_B1_T70_H1_d128.npz")
    o, s, _ = ora.recurrent(*_inputs(f, torch.float64), f["initial_state"].double())
    assert rel_err(o, f["out"]) < 1e-11 and rel_err(s, f["final_state"]) < 1e-11


def test_oracle_reproduces_varlen_fixture():
    f = load("varlen_bf16_T100_H1_K128_V32.npz")
    o, s = ora.varlen_recurrent(*_inputs(f, torch.float64), f["cu_seqlens"], f["initial_state"].double())
    assert rel_err(o, f["out"]) < 1e-11 and rel_err(s, f["final_state"]) < 1e-11


def test_oracle_reproduces_decode_fixture():
    f = load("decode_bf16_B3_H1_d128.npz")
    o, s, _ = ora.recurrent(*_inputs(f, torch.float64), f["initial_state"].double())
    assert rel_err(o, f["out"]) < 1e-12 and rel_err(s, f["final_state"]) < 1e-12


def test_oracle_reproduces_masked_fixture():
    f = load("masked_f64_B2_T9_H2_K3_V4.npz")
    o, s = ora.chunkwise(*_inputs(f), f["initial_state"], f["attention_mask"], chunk_size=4, secondary_tile_size=2)
    assert rel_err(o, f["out"]) < 1e-11 and rel_err(s, f["final_state"]) < 1e-11
    assert torch.count_nonzero(f["out"][1, 5:]) == 0


# ---------------------------------------------------------------------------
# GPU parity against the fixtures

DEV = "cuda"


def _dev(ts):
    return [t.to(DEV) for t in ts]


@pytest.mark.gpu
def test_gpu_cpu_smoke_fixture_f32():
    import kda

    f = load("cpu_smoke_f32_B2_T32_H2_d16.npz")
    got = kda.chunkwise_kda(*_dev(_inputs(f)), None, True, chunk_size=16, secondary_tile_size=16)
    assert rel_err(got.hidden_states, f["out"]) < 1e-4 and rel_err(got.final_state, f["final_state"]) < 1e-4


@pytest.mark.gpu
def test_gpu_prefill_fixture_bf16():
    import kda

    f = load("prefill_bf16_B1_T70_H1_d128.npz")
    got = kda.chunkwise_kda(*_dev(_inputs(f, torch.bfloat16)), f["initial_state"].to(DEV), True)
    assert got.hidden_states.dtype == torch.bfloat16
    assert rel_err(got.hidden_states, f["out"]) < 2e-2 and rel_err(got.final_state, f["final_state"]) < 2e-2


@pytest.mark.gpu
def test_gpu_varlen_fixture_bf16():
    import kda

    f = load("varlen_bf16_T100_H1_K128_V32.npz")
    got = kda.chunkwise_kda(*_dev(_inputs(f, torch.bfloat16)), f["initial_state"].to(DEV), True,
                            cu_seqlens=f["cu_seqlens"].to(DEV))
    assert rel_err(got.hidden_states, f["out"]) < 2e-2 and rel_err(got.final_state, f["final_state"]) < 2e-2


@pytest.mark.gpu
def test_gpu_decode_fixture_bf16():
    import kda

    f = load("decode_bf16_B3_H1_d128.npz")
    got = kda.recurrent_kda(*_dev(_inputs(f, torch.bfloat16)), f["initial_state"].to(DEV), True)
    assert rel_err(got.hidden_states, f["out"]) < 2e-2 and rel_err(got.final_state, f["final_state"]) < 2e-2


@pytest.mark.gpu
def test_gpu_masked_fixture_f64():
    import kda

    f = load("masked_f64_B2_T9_H2_K3_V4.npz")
    got = kda.chunkwise_kda(*_dev(_inputs(f)), f["initial_state"].to(DEV), True, f["attention_mask"].to(DEV),
                            chunk_size=4, secondary_tile_size=2)
    assert rel_err(got.hidden_states, f["out"]) < 1e-10 and rel_err(got.final_state, f["final_state"]) < 1e-10
    rec = kda.recurrent_kda(*_dev(_inputs(f)), f["initial_state"].to(DEV), True, f["attention_mask"].to(DEV))
    assert rel_err(rec.hidden_states, f["out"]) < 1e-10 and rel_err(rec.final_state, f["final_state"]) < 1e-10
