"""The operators inside their caller: a KDA layer (src/kda/kda.py:98-183) run
through this backend (kda.layer.kda_attention_forward: projection GEMMs, the
fused ShortConv/SiLU/L2 and gate kernels, the chunk kernel forming g from
the decay logits, the decode step, RMSNorm x output gate) against the same
composition of the oracle's stages on the CPU (oracle.kda_layer), with the
reference module tests' scenarios (tests/kda/test_kda_decode.py:33-157,
tests/kda/test_kda_full_module.py:10-53) and the cache accounting of
inference/cache.py:32-38.

Tolerances (max|x - ref| / max|ref| per tensor): bf16 activations 2e-2 for
outputs and recurrent states against the oracle in f32 on the same bf16
weights and inputs (the ShortConv histories are copies of the projections:
1e-2); f64 1e-10 against the oracle in f64.
"""

from __future__ import annotations

import pytest
import torch

import kda
from kda import _lib, fused
from kda.layer import KDALayerWeights, kda_attention_forward
from oracle import kda_oracle as ora
from tests._inputs import layer_weights, rel_err, workload

pytestmark = pytest.mark.gpu
DEV = "cuda"

# one layer on the MFMA shapes: d_model = H * V = 256, K = V = 128
BIG = dict(d_model=256, heads=2, key_dim=128, value_dim=128, conv=4, rank=32)


def _weights(cfg, dtype, seed=17, biases=False):
    w = layer_weights(cfg["d_model"], cfg["heads"], cfg["key_dim"], cfg["value_dim"], conv=cfg["conv"],
                      rank=cfg["rank"], dtype=dtype, seed=seed, biases=biases)
    gw = KDALayerWeights(**{k: (v.to(DEV) if isinstance(v, torch.Tensor) else v) for k, v in w.items()})
    return w, gw


def _x(cfg, b, t, dtype, seed=0):
    return torch.randn(b, t, cfg["d_model"], generator=torch.Generator().manual_seed(seed)).to(dtype)


def _state_tuple(st):
    return (st.recurrent_state, st.q_conv_state.buffer, st.k_conv_state.buffer, st.v_conv_state.buffer,
            st.sequence_offset)


def _check(out, st, ref_out, ref_st, tol=2e-2, hist_tol=1e-2, label=""):
    eo = rel_err(out, ref_out)
    msg = f"{label} output {eo:.2e}"
    assert eo < tol, msg
    if ref_st is not None:
        got = _state_tuple(st)
        es = rel_err(got[0], ref_st[0])
        eh = max(rel_err(got[i], ref_st[i]) for i in (1, 2, 3))
        msg += f" state {es:.2e} histories {eh:.2e}"
        assert es < tol and eh < hist_tol, msg
        assert got[4].cpu().tolist() == ref_st[4].tolist()
    print(msg)


def _gpu_state(ref_st):
    rec, qh, kh, vh, off = ref_st
    return kda.KDAState(rec.to(DEV), kda.ShortConvState(qh.to(DEV)), kda.ShortConvState(kh.to(DEV)),
                        kda.ShortConvState(vh.to(DEV)), off.to(DEV))


@pytest.mark.parametrize("mode", ["chunkwise", "recurrent"])
@pytest.mark.parametrize("biases", [False, True])
def test_layer_matches_oracle_bf16(mode, biases):
    w, gw = _weights(BIG, torch.bfloat16, biases=biases)
    x = _x(BIG, 2, 150, torch.bfloat16)
    ref_out, ref_st = ora.kda_layer(w, x, mode=mode, output_final_state=True)
    with torch.no_grad():
        got = kda_attention_forward(gw, x.to(DEV), mode=mode, output_final_state=True)
    assert got.hidden_states.dtype == torch.bfloat16 and got.state.recurrent_state.dtype == torch.float32
    _check(got.hidden_states, got.state, ref_out, ref_st, label=f"{mode} biases={biases}")


def test_layer_key_dim_64_matches_oracle_bf16():
    # the head shape of the reference's gpu_48gb profile (K = V = 64) on the
    # MFMA path, chunkwise prefill then decode steps
    cfg = dict(d_model=128, heads=2, key_dim=64, value_dim=64, conv=4, rank=16)
    w, gw = _weights(cfg, torch.bfloat16, seed=19)
    x = _x(cfg, 2, 140, torch.bfloat16, seed=20)
    ref_out, ref_st = ora.kda_layer(w, x, mode="recurrent", output_final_state=True)
    xd = x.to(DEV)
    with torch.no_grad():
        pre = kda_attention_forward(gw, xd[:, :136], mode="chunkwise", output_final_state=True)
        state, outs = pre.state, [pre.hidden_states]
        for t in range(136, 140):
            step = kda_attention_forward(gw, xd[:, t:t + 1], state=state, mode="decode")
            state, outs = step.state, outs + [step.hidden_states]
    _check(torch.cat(outs, 1), state, ref_out, ref_st, label="K=V=64 layer")


@pytest.mark.parametrize("in_place", [False, True])
def test_split_prefill_then_decode_matches_one_shot_bf16(in_place):
    # prefill 100 tokens (chunkwise, fused decay), then 8 decode steps carrying
    # the KDAState (recurrent state and the three ShortConv histories), against
    # the oracle's one-shot recurrence over all 108 tokens
    w, gw = _weights(BIG, torch.bfloat16, seed=3)
    x = _x(BIG, 2, 108, torch.bfloat16, seed=4)
    ref_out, ref_st = ora.kda_layer(w, x, mode="recurrent", output_final_state=True)
    xd = x.to(DEV)
    with torch.no_grad():
        pre = kda_attention_forward(gw, xd[:, :100], mode="chunkwise", output_final_state=True)
        state, outs = pre.state, [pre.hidden_states]
        for t in range(100, 108):
            step = kda_attention_forward(gw, xd[:, t:t + 1], state=state, mode="decode",
                                         update_state_in_place=in_place)
            if in_place:
                assert step.state.recurrent_state.data_ptr() == state.recurrent_state.data_ptr()
            state = step.state
            outs.append(step.hidden_states)
    _check(torch.cat(outs, 1), state, ref_out, ref_st, label=f"split in_place={in_place}")


def test_irregular_streaming_matches_full_bf16():
    # chunkwise calls of several sizes (one chunk, several chunks, a partial
    # chunk) interleaved with decode steps, as tests/kda/test_kda_decode.py:64-83
    w, gw = _weights(BIG, torch.bfloat16, seed=5)
    sizes = [3, 5, 1, 70, 1, 64, 7, 1]
    x = _x(BIG, 2, sum(sizes), torch.bfloat16, seed=6)
    ref_out, ref_st = ora.kda_layer(w, x, mode="recurrent", output_final_state=True)
    xd = x.to(DEV)
    state, off, outs = None, 0, []
    with torch.no_grad():
        for size in sizes:
            res = kda_attention_forward(gw, xd[:, off:off + size], state=state,
                                        mode="decode" if size == 1 else "chunkwise", output_final_state=True)
            outs.append(res.hidden_states)
            state = res.state
            off += size
    _check(torch.cat(outs, 1), state, ref_out, ref_st, label="irregular streaming")


def test_right_padded_batch_matches_oracle_bf16():
    w, gw = _weights(BIG, torch.bfloat16, seed=7, biases=True)
    x = _x(BIG, 3, 130, torch.bfloat16, seed=8)
    mask = torch.ones(3, 130, dtype=torch.bool)
    mask[1, 90:] = False
    mask[2, 1:] = False
    ref_out, ref_st = ora.kda_layer(w, x, mask, mode="chunkwise", output_final_state=True)
    with torch.no_grad():
        got = kda_attention_forward(gw, x.to(DEV), mask.to(DEV), mode="chunkwise", output_final_state=True)
    assert torch.count_nonzero(got.hidden_states[1, 90:]) == 0
    _check(got.hidden_states, got.state, ref_out, ref_st, label="right padding")
    # a continuation from the padded prefix state
    x2 = _x(BIG, 3, 20, torch.bfloat16, seed=9)
    ref2, ref2_st = ora.kda_layer(w, x2, state=ref_st, mode="chunkwise", output_final_state=True)
    with torch.no_grad():
        got2 = kda_attention_forward(gw, x2.to(DEV), state=got.state, mode="chunkwise", output_final_state=True)
    _check(got2.hidden_states, got2.state, ref2, ref2_st, label="after padding")


def test_f64_modes_agree_and_match_oracle():
    # f64 end to end on a small layer (K = V = 16: the exact recurrence kernel
    # for both operator modes), recurrent == chunkwise == token decode
    cfg = dict(d_model=32, heads=2, key_dim=16, value_dim=16, conv=3, rank=5)
    w, gw = _weights(cfg, torch.float64, seed=11, biases=True)
    x = _x(cfg, 2, 11, torch.float64, seed=12)
    ref_out, ref_st = ora.kda_layer(w, x, mode="recurrent", output_final_state=True)
    xd = x.to(DEV)
    res = {}
    with torch.no_grad():
        for mode in ("recurrent", "chunkwise"):
            r = kda_attention_forward(gw, xd, mode=mode, output_final_state=True)
            res[mode] = r
            _check(r.hidden_states, r.state, ref_out, ref_st, tol=1e-10, hist_tol=1e-14, label=f"f64 {mode}")
        state, outs = None, []
        for t in range(11):
            r = kda_attention_forward(gw, xd[:, t:t + 1], state=state, mode="decode")
            outs.append(r.hidden_states)
            state = r.state
    _check(torch.cat(outs, 1), state, ref_out, ref_st, tol=1e-10, hist_tol=1e-14, label="f64 decode")
    torch.testing.assert_close(res["recurrent"].hidden_states, res["chunkwise"].hidden_states, rtol=1e-10,
                               atol=1e-12)


def test_cache_bytes_constant_and_equal_to_the_reference_layout():
    # inference/cache.py:32-38 sums numel * element_size over the cache's
    # tensors: the state a layer hands on keeps the reference's layout (f32
    # [B,H,K,V], three [B, K_conv-1, width] histories in the activation dtype,
    # int64 offsets) and does not grow with the context
    w, gw = _weights(BIG, torch.bfloat16, seed=13)
    nbytes = lambda ts: sum(t.numel() * t.element_size() for t in ts)  # noqa: E731
    sizes = []
    with torch.no_grad():
        for t in (2, 50, 200):
            st = kda_attention_forward(gw, _x(BIG, 2, t, torch.bfloat16).to(DEV), output_final_state=True).state
            sizes.append(nbytes(_state_tuple(st)))
    ref_st = ora.kda_layer(w, _x(BIG, 2, 2, torch.bfloat16), output_final_state=True)[1]
    assert sizes[0] == sizes[1] == sizes[2] == nbytes(ref_st)
    B, H, K, V, C = 2, BIG["heads"], BIG["key_dim"], BIG["value_dim"], BIG["conv"]
    assert sizes[0] == 4 * B * H * K * V + 2 * B * (C - 1) * (2 * H * K + H * V) + 8 * B


# ---- the decay fused into the chunk kernel ------------------------------------

def _decay_inputs(B, T, H, K, V, dtype, seed, z_shift=0.0):
    q, k, v, _, beta, state = workload(B, T, H, K, V, state_std=0.02, seed=seed, dtype=dtype)
    gen = torch.Generator().manual_seed(seed + 100)
    z = (torch.randn(B, T, H, K, generator=gen) + z_shift).to(dtype)
    bias = (0.5 * torch.randn(H, K, generator=gen)).to(dtype)
    a_log = 0.3 * torch.randn(H, generator=gen)
    return q, k, v, z, beta, state, bias, a_log


@pytest.mark.parametrize(
    "case",
    ["dense", "masked", "packed", "segmented", "extreme_decay", "f16", "value_64", "key_64"],
)
def test_fused_decay_prefill_equals_two_step_and_oracle(segments, case):
    dtype = torch.float16 if case == "f16" else torch.bfloat16
    B, T, H, V = (1, 260, 2, 128) if case in ("packed", "segmented") else (2, 200, 2, 64 if case == "value_64" else 128)
    K = 64 if case == "key_64" else 128
    q, k, v, z, beta, state, bias, a_log = _decay_inputs(B, T, H, K, V, dtype, seed=21,
                                                         z_shift=25.0 if case == "extreme_decay" else 0.0)
    mask = cu = None
    if case == "masked":
        mask = torch.ones(B, T, dtype=torch.bool)
        mask[1, 133:] = False
    if case == "packed":
        cu = [0, 70, 71, 200, 260]
        state = torch.randn(4, H, K, V, generator=torch.Generator().manual_seed(5)) * 0.02
    if case == "segmented":
        segments(1)
    dv = lambda t: None if t is None else t.to(DEV)  # noqa: E731
    kw = dict(initial_state=dv(state), output_final_state=True, attention_mask=dv(mask), cu_seqlens=cu)
    with torch.no_grad():
        fused_res = fused.chunkwise_kda_with_decay(dv(q), dv(k), dv(v), dv(z), dv(a_log), dv(beta), decay_bias=dv(bias),
                                                   g_min=-5.0, **kw)
        g, _ = fused.lower_bounded_decay(dv(z), dv(a_log), -5.0, bias=dv(bias))
        two = kda.chunkwise_kda(dv(q), dv(k), dv(v), g, dv(beta), dv(state), True, dv(mask), cu_seqlens=cu)
    # the same g bits feed the same chunk arithmetic
    assert torch.equal(fused_res.hidden_states, two.hidden_states), case
    assert torch.equal(fused_res.final_state, two.final_state), case
    rg, _ = ora.lower_bounded_decay(z, a_log, -5.0, bias=bias)
    rg = rg.to(dtype)
    if cu is None:
        ro, rs = ora.chunkwise(*(t.float() for t in (q, k, v, rg, beta)), state, mask, chunk_size=64,
                               secondary_tile_size=16)
    else:
        ro, rs = ora.varlen_chunkwise(*(t.float() for t in (q, k, v, rg, beta)), cu, state, chunk_size=64,
                                      secondary_tile_size=16)
    eo, es = rel_err(fused_res.hidden_states, ro), rel_err(fused_res.final_state, rs)
    print(f"{case}: output {eo:.2e} state {es:.2e}")
    assert eo < 2e-2 and es < 2e-2


def test_fused_decay_entry_refuses_shapes_off_the_mfma_path():
    lib = _lib.load()
    # V = 20, not a multiple of 16 (nothing is launched: the shape check comes first)
    status = lib.kda_chunk_fwd_decay(1, 1, 1, 1, None, 1, -5.0, 1, _lib.dtype_code(torch.bfloat16), None, None, 0,
                                     1, None, 64, None, 1, 64, 1, 128, 20, None, 0, None)
    assert status == _lib.KDA_ERR_UNSUPPORTED
    assert "MFMA path" in lib.kda_status_string(status).decode()
    # the Python entry runs the two steps there, still on the GPU
    q, k, v, _, beta, state = workload(1, 70, 2, 128, 20, state_std=0.02, seed=2)
    z = torch.randn(1, 70, 2, 128, generator=torch.Generator().manual_seed(3)).to(torch.bfloat16)
    a_log = torch.zeros(2)
    with torch.no_grad():
        got = fused.chunkwise_kda_with_decay(*(t.to(DEV) for t in (q, k, v, z, a_log, beta)),
                                             initial_state=state.to(DEV), output_final_state=True)
    rg = ora.lower_bounded_decay(z, a_log, -5.0)[0].to(torch.bfloat16)
    ro, rs = ora.chunkwise(*(t.float() for t in (q, k, v, rg, beta)), state, chunk_size=64, secondary_tile_size=16)
    assert rel_err(got.hidden_states, ro) < 2e-2 and rel_err(got.final_state, rs) < 2e-2
