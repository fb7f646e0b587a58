"""The layer composition pinned to the reference module itself.

The fixtures ``tests/golden/layer_ref_{f32,bf16}_B2_T21_H2_K32_V32.npz`` hold
what the reference's ``KimiDeltaAttention`` (src/kda/kda.py:98-183, with
src/kda/projections.py:144-225, src/kda/decay.py:28-43 and the head-wise
RMSNorm / output gate, kda.py:153-161) computed on seeded weights (every bias
on, every parameter off its initial value) for a right-padded chunkwise
prefill, a recurrent-mode prefill and two decode steps carrying the
``KDAState`` (written by tests/golden/make_layer_golden.py).

CPU: the oracle's layer (``oracle.kda_layer``) reproduces them, and three
planted composition mistakes (the decay bias dropped, an L2 norm applied to
v, the output bias dropped) each miss them by far more than the tolerance.
GPU: ``kda.layer.kda_attention_forward`` (this backend's kernels) matches
them.  Tolerances, max|x - ref| / max|ref| per tensor: f32 1e-4; bf16 2e-2
(the reference runs each bf16 stage in bf16 arithmetic, the oracle and the
backend in f32 with bf16 results, which measures 1.4e-2 on the prefill
output); the ShortConv histories are copies of the projections (1e-2 in bf16,
1e-5 in f32) and the sequence offsets are integers (exact).
"""

from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import kda_oracle as ora
from tests._inputs import rel_err

GOLDEN = Path(__file__).resolve().parent / "golden"
FIXTURES = ["layer_ref_f32_B2_T21_H2_K32_V32.npz", "layer_ref_bf16_B2_T21_H2_K32_V32.npz"]
STATE_FIELDS = ("recurrent", "q_hist", "k_hist", "v_hist", "offset")


def load(name):
    with np.load(GOLDEN / name) as z:
        f = {key: z[key] for key in z.files}
    dt = torch.float32 if str(f["dtype"]) == "float32" else torch.bfloat16
    cfg = {}
    for item in str(f["config"]).strip("{}").split(","):
        key, val = (s.strip().strip("'") for s in item.split(":"))
        cfg[key] = val
    w = {k[2:]: torch.from_numpy(v).to(dt) for k, v in f.items() if k.startswith("w_")}
    w["a_log"] = torch.from_numpy(f["w_a_log"]).float()
    w.update(num_heads=int(cfg["num_heads"]), key_head_dim=int(cfg["key_head_dim"]),
             value_head_dim=int(cfg["value_head_dim"]), g_min=float(cfg["g_min"]), eps=float(cfg["eps"]))
    t = {k: torch.from_numpy(v) for k, v in f.items() if not k.startswith("w_") and k not in ("dtype", "config")}
    return dt, w, t


def tolerances(dt):
    return (1e-4, 1e-5) if dt == torch.float32 else (2e-2, 1e-2)


def expected_state(t, prefix):
    return tuple(t[f"{prefix}_{n}"] for n in STATE_FIELDS)


def check(out, state, t, prefix, dt, label):
    tol, hist_tol = tolerances(dt)
    eo = rel_err(out, t[f"{prefix}_out"])
    exp = expected_state(t, prefix)
    es = rel_err(state[0], exp[0])
    eh = max(rel_err(state[i], exp[i]) for i in (1, 2, 3))
    msg = f"{label} {prefix}: output {eo:.2e} state {es:.2e} histories {eh:.2e}"
    assert eo < tol and es < tol and eh < hist_tol, msg
    assert state[4].cpu().tolist() == exp[4].tolist(), msg
    print(msg)


def oracle_run(w, dt, t):
    x = t["x"].to(dt)
    mask = t["mask"]
    pre = ora.kda_layer(w, x, mask, mode="chunkwise", output_final_state=True)
    rec = ora.kda_layer(w, x, mask, mode="recurrent", output_final_state=True)
    steps, st = [], pre[1]
    for i in range(2):
        out, st = ora.kda_layer(w, t[f"x_step{i}"].to(dt), None, st, mode="decode")
        steps.append((out, st))
    return pre, rec, steps


def test_fixture_inventory():
    assert sorted(p.name for p in GOLDEN.glob("layer_ref_*.npz")) == sorted(FIXTURES)


@pytest.mark.parametrize("name", FIXTURES)
def test_oracle_layer_reproduces_reference_module(name):
    dt, w, t = load(name)
    pre, rec, steps = oracle_run(w, dt, t)
    check(pre[0], pre[1], t, "prefill", dt, name)
    check(rec[0], rec[1], t, "recurrent", dt, name)
    for i, (out, st) in enumerate(steps):
        check(out, st, t, f"step{i}", dt, name)


@pytest.mark.parametrize("mistake", ["no_decay_bias", "v_l2_norm", "no_output_bias"])
def test_planted_composition_mistakes_miss_the_fixture(mistake, monkeypatch):
    # each mistake is planted in the oracle's layer (on the CPU); the fixture
    # must reject it by far more than the f32 tolerance
    dt, w, t = load(FIXTURES[0])
    w = dict(w)
    if mistake == "no_decay_bias":
        w["b_alpha"] = torch.zeros_like(w["b_alpha"])
    elif mistake == "no_output_bias":
        w["output_bias"] = None
    else:
        conv = ora.conv_silu

        def conv_normalizing_v(*args, normalize=False, **kwargs):
            return conv(*args, normalize=True, **kwargs)

        monkeypatch.setattr(ora, "conv_silu", conv_normalizing_v)
    out, _ = ora.kda_layer(w, t["x"].to(dt), t["mask"], mode="chunkwise", output_final_state=True)
    assert rel_err(out, t["prefill_out"]) > 100 * tolerances(dt)[0]


# ---------------------------------------------------------------------------
# GPU: the backend's layer against the reference module's record

@pytest.mark.gpu
@pytest.mark.parametrize("name", FIXTURES)
def test_backend_layer_matches_reference_module(name):
    from kda import KDAState, ShortConvState
    from kda.layer import KDALayerWeights, kda_attention_forward

    dt, w, t = load(name)
    dev = "cuda"
    gw = KDALayerWeights(**{k: (v.to(dev) if isinstance(v, torch.Tensor) else v) for k, v in w.items()})
    x = t["x"].to(dt).to(dev)
    mask = t["mask"].to(dev)

    def as_tuple(st):
        return (st.recurrent_state, st.q_conv_state.buffer, st.k_conv_state.buffer, st.v_conv_state.buffer,
                st.sequence_offset)

    with torch.no_grad():
        pre = kda_attention_forward(gw, x, mask, mode="chunkwise", output_final_state=True)
        rec = kda_attention_forward(gw, x, mask, mode="recurrent", output_final_state=True)
        assert pre.hidden_states.dtype == dt and pre.state.recurrent_state.dtype == torch.float32
        check(pre.hidden_states, as_tuple(pre.state), t, "prefill", dt, name)
        check(rec.hidden_states, as_tuple(rec.state), t, "recurrent", dt, name)
        state = pre.state
        for i in range(2):
            step = kda_attention_forward(gw, t[f"x_step{i}"].to(dt).to(dev), state=state, mode="decode")
            state = step.state
            check(step.hidden_states, as_tuple(state), t, f"step{i}", dt, name)
        assert isinstance(state, KDAState) and isinstance(state.q_conv_state, ShortConvState)
