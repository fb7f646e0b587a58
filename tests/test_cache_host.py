"""Host-side checks of the cache gather entry point (no GPU, nothing launched).

``kda_cache_gather`` validates its descriptors before any launch; these calls
use fake device addresses and are all rejected (or are empty) on the host.
"""

from __future__ import annotations

import ctypes

import pytest
import torch

from kda import _lib, cache
from kda.state import KDAState, ShortConvState


def _call(src, dst, rows, index=None, n_src=4, n_out=4):
    lib = _lib.load()
    n = len(rows)
    return lib.kda_cache_gather(
        (ctypes.c_void_p * n)(*src), (ctypes.c_void_p * n)(*dst), (ctypes.c_int64 * n)(*rows), n,
        index, n_src, n_out, None, None,
    )


def test_rejections_before_any_launch():
    base = 1 << 20
    ok_src, ok_dst = [base], [base + 4096]
    assert _call(ok_src, ok_dst, [64], n_out=0, index=base * 4) == _lib.KDA_OK  # nothing to do
    assert _call(ok_src, ok_dst, [16], n_out=3) == _lib.KDA_ERR_INVALID_ARGUMENT  # no index: n_out == n_src
    assert _call(ok_src, ok_dst, [-16]) == _lib.KDA_ERR_INVALID_ARGUMENT  # negative row bytes
    assert _call(ok_src, [0], [16]) == _lib.KDA_ERR_INVALID_ARGUMENT  # null output
    assert _call([base], [base + 32], [16]) == _lib.KDA_ERR_INVALID_ARGUMENT  # output overlaps the source
    assert _call([base, base + 8192], [base + 4096, base + 4096 + 32], [16, 16]) == _lib.KDA_ERR_INVALID_ARGUMENT
    assert _call(ok_src, ok_dst, [16], index=base * 4, n_src=0, n_out=2) == _lib.KDA_ERR_INVALID_ARGUMENT
    assert _call(ok_src, ok_dst, [1 << 62], index=base * 4) == _lib.KDA_ERR_INVALID_ARGUMENT  # size overflow


def test_gather_refuses_host_tensors():
    with pytest.raises(RuntimeError, match="GPU"):
        cache.gather_rows([torch.zeros(2, 3)], None)


def _state(batch):
    gen = torch.Generator().manual_seed(batch)
    conv = lambda: ShortConvState(torch.randn(batch, 3, 8, generator=gen))  # noqa: E731
    return KDAState(torch.randn(batch, 2, 4, 4, generator=gen), conv(), conv(), conv(),
                    torch.arange(batch, dtype=torch.long) + 10)


def test_host_state_reorder_and_clone_keep_reference_semantics():
    s = _state(3)
    idx = torch.tensor([2, 0, 2], dtype=torch.long)
    r = s.reorder(idx)
    torch.testing.assert_close(r.recurrent_state, s.recurrent_state[idx])
    torch.testing.assert_close(r.v_conv_state.buffer, s.v_conv_state.buffer[idx])
    assert r.sequence_offset.tolist() == [12, 10, 12]
    c = s.clone()
    assert c.recurrent_state.data_ptr() != s.recurrent_state.data_ptr()
    with pytest.raises(ValueError):
        s.reorder(idx.int())
    with pytest.raises(ValueError):
        cache.reorder_states([s], idx[None])
