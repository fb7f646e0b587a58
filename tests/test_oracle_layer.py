"""Pins of the oracle's layer composition (oracle.kda_layer, following
src/kda/kda.py:98-183) by the reference's own module-level invariants, in
f64 on the CPU (tests/kda/test_kda_decode.py:33-157,
tests/kda/test_kda_full_module.py:37-75): every stage inside it is pinned on
its own in test_oracle.py and test_oracle_fused.py."""

from __future__ import annotations

import pytest
import torch

from oracle import kda_oracle as ora
from tests._inputs import layer_weights

# the reference's tiny module (tests/kda/conftest.py:6-24): d_model 12, 3 heads,
# K=2, V=4, ShortConv 3, decay rank 5, chunk 4 with tile 2
TINY = dict(d_model=12, heads=3, key_dim=2, value_dim=4, conv=3, rank=5)


def _w(**over):
    w = layer_weights(TINY["d_model"], TINY["heads"], TINY["key_dim"], TINY["value_dim"], conv=TINY["conv"],
                      rank=TINY["rank"], **over)
    w.update(chunk_size=4, secondary_tile_size=2)
    return w


def _x(b, t, seed=0):
    return torch.randn(b, t, TINY["d_model"], generator=torch.Generator().manual_seed(seed), dtype=torch.float64)


def _decode_tokens(w, x, state=None, layer=ora.kda_layer):
    outs = []
    for t in range(x.shape[1]):
        o, state = layer(w, x[:, t:t + 1], state=state, mode="decode")
        outs.append(o)
    return torch.cat(outs, dim=1), state


def _assert_states(a, b, tol=2e-11):
    torch.testing.assert_close(a[0], b[0], rtol=tol, atol=tol * 0.1)
    for i in (1, 2, 3):
        torch.testing.assert_close(a[i], b[i], rtol=2e-14, atol=2e-15)
    assert torch.equal(a[4], b[4])


def test_recurrent_chunkwise_and_token_decode_agree():
    w = _w()
    x = _x(2, 11)
    rec = ora.kda_layer(w, x, mode="recurrent", output_final_state=True)
    chk = ora.kda_layer(w, x, mode="chunkwise", output_final_state=True)
    dec = _decode_tokens(w, x)
    for o, s in (rec, chk):
        torch.testing.assert_close(o, dec[0], rtol=2e-11, atol=2e-12)
        _assert_states(s, dec[1])


@pytest.mark.parametrize("split", [1, 2, 5, 8, 10])
@pytest.mark.parametrize("prefill_mode", ["recurrent", "chunkwise"])
def test_split_prefill_then_decode_matches_one_shot(split, prefill_mode):
    w = _w()
    x = _x(2, 11, seed=1)
    full = ora.kda_layer(w, x, mode="recurrent", output_final_state=True)
    pre = ora.kda_layer(w, x[:, :split], mode=prefill_mode, output_final_state=True)
    suf, fin = _decode_tokens(w, x[:, split:], pre[1])
    torch.testing.assert_close(torch.cat((pre[0], suf), 1), full[0], rtol=2e-11, atol=2e-12)
    _assert_states(fin, full[1])


def test_irregular_streaming_chunks_match_full():
    w = _w()
    x = _x(2, 19, seed=2)
    full = ora.kda_layer(w, x, mode="recurrent", output_final_state=True)
    state, off, outs = None, 0, []
    for size in (3, 5, 1, 7, 3):
        o, state = ora.kda_layer(w, x[:, off:off + size], state=state, mode="decode" if size == 1 else "chunkwise",
                                 output_final_state=True)
        outs.append(o)
        off += size
    torch.testing.assert_close(torch.cat(outs, 1), full[0], rtol=2e-11, atol=2e-12)
    _assert_states(state, full[1])


def test_cache_size_is_constant_with_context_length():
    w = _w()
    short = ora.kda_layer(w, _x(2, 2), output_final_state=True)[1]
    long = ora.kda_layer(w, _x(2, 50), output_final_state=True)[1]
    size = lambda st: sum(t.numel() * t.element_size() for t in st)  # noqa: E731
    assert size(short) == size(long)


def test_new_state_reset_removes_previous_sequence_dependency():
    w = _w()
    prefix = ora.kda_layer(w, _x(1, 5, seed=3), mode="recurrent", output_final_state=True)
    suffix = _x(1, 3, seed=4)
    continued = ora.kda_layer(w, suffix, state=prefix[1], mode="recurrent")[0]
    reset = ora.kda_layer(w, suffix, state=None, mode="recurrent")[0]
    assert not torch.allclose(continued, reset)
    torch.testing.assert_close(reset, ora.kda_layer(w, suffix, mode="recurrent")[0], rtol=0, atol=0)


def test_zero_parameters_give_zero_output():
    # no residual connection is hidden inside the layer (tests/kda/test_kda_full_module.py:68-75)
    w = _w()
    for key, val in list(w.items()):
        if isinstance(val, torch.Tensor):
            w[key] = torch.zeros_like(val)
    assert torch.count_nonzero(ora.kda_layer(w, _x(2, 3), mode="recurrent")[0]) == 0


def test_right_padding_equals_truncated_rows():
    w = _w(biases=True)
    x = _x(2, 9, seed=5)
    mask = torch.ones(2, 9, dtype=torch.bool)
    mask[1, 6:] = False
    out, st = ora.kda_layer(w, x, mask, mode="chunkwise", output_final_state=True)
    assert torch.count_nonzero(out[1, 6:]) == 0
    solo, sst = ora.kda_layer(w, x[1:2, :6], mode="recurrent", output_final_state=True)
    torch.testing.assert_close(out[1:2, :6], solo, rtol=2e-11, atol=2e-12)
    for i in range(4):
        torch.testing.assert_close(st[i][1:2], sst[i], rtol=2e-11, atol=2e-12)
    assert st[4].tolist() == [9, 6]


def test_planted_mistakes_are_caught(monkeypatch):
    # a history that is not carried between calls, and an offset that is not
    # accumulated, each fail the split-prefill pin
    w = _w()
    x = _x(2, 11, seed=1)
    full = ora.kda_layer(w, x, mode="recurrent", output_final_state=True)
    real_conv = ora.conv_silu

    def forgetful(x, weight, bias=None, history=None, *a, **k):
        return real_conv(x, weight, bias, None, *a, **k)

    monkeypatch.setattr(ora, "conv_silu", forgetful)
    pre = ora.kda_layer(w, x[:, :5], mode="chunkwise", output_final_state=True)
    suf, _ = _decode_tokens(w, x[:, 5:], pre[1])
    assert not torch.allclose(torch.cat((pre[0], suf), 1), full[0], rtol=1e-6, atol=1e-8)
    monkeypatch.setattr(ora, "conv_silu", real_conv)
    pre = ora.kda_layer(w, x[:, :5], mode="chunkwise", output_final_state=True)
    bad = (pre[1][0], pre[1][1], pre[1][2], pre[1][3], torch.zeros_like(pre[1][4]))
    _, fin = _decode_tokens(w, x[:, 5:], bad)
    assert not torch.equal(fin[4], full[1][4])
