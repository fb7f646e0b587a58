"""GPU parity of the whole-cache reorder and clone (``kda.cache``,
``kda_cache_gather``) against the oracle's byte gather.

The bar is bit equality: every tensor is compared as raw bytes.  Cases: every
unit width the kernel picks (16, 8, 4, 2 and 1 bytes, from row sizes and
addresses), rows shorter and longer than one tile, duplicated and expanding
indices, more tensors than one launch takes, empty batches, out-of-range
indices, and a permutation round trip at the decode cache size of a
B=64, H=32, K=V=128 layer (2 MiB state rows).
"""

from __future__ import annotations

import pytest
import torch

from kda import cache
from kda.state import KDAState, ShortConvState
from oracle import kda_oracle as ora

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _bytes(t: torch.Tensor):
    """[rows, bytes per row] of a tensor's host copy."""
    t = t.detach().cpu().contiguous()
    return t.reshape(t.shape[0], -1).view(torch.uint8).numpy()


def _check(outs, srcs, index):
    ref = ora.gather_rows([_bytes(s) for s in srcs], None if index is None else index.cpu().tolist())
    for o, r in zip(outs, ref):
        assert o.is_cuda
        assert (_bytes(o) == r).all()


def _odd(shape, dtype, shift_bytes, seed):
    """A contiguous GPU tensor whose address is shifted by shift_bytes from a 256-byte boundary."""
    gen = torch.Generator().manual_seed(seed)
    n = 1
    for s in shape:
        n *= s
    esize = torch.empty((), dtype=dtype).element_size()
    raw = torch.empty(n * esize + 256, dtype=torch.uint8, device=DEV)
    t = raw[shift_bytes : shift_bytes + n * esize].view(dtype).view(shape)
    t.copy_(torch.randint(-100, 100, shape, generator=gen).to(dtype))
    return t


def test_every_unit_width_and_duplicate_indices():
    B = 5
    srcs = [
        _odd((B, 2, 8, 8), torch.float32, 0, 1),    # 512-byte rows: 16-byte units
        _odd((B, 3, 37), torch.bfloat16, 0, 2),     # 222-byte rows: 2-byte units
        _odd((B,), torch.int64, 0, 3),              # 8-byte rows
        _odd((B, 3), torch.float32, 4, 4),          # 4-byte aligned address
        _odd((B, 13), torch.uint8, 1, 5),           # 1-byte units
        _odd((B, 3, 24), torch.bfloat16, 0, 6),     # 144-byte rows: 16-byte units
    ]
    idx = torch.tensor([4, 0, 0, 3, 1, 4, 2], dtype=torch.long, device=DEV)
    outs = cache.gather_rows(srcs, idx)
    assert [o.shape[0] for o in outs] == [7] * len(srcs)
    _check(outs, srcs, idx)
    clones = cache.gather_rows(srcs, None)
    _check(clones, srcs, None)
    assert all(c.data_ptr() != s.data_ptr() for c, s in zip(clones, srcs))


@pytest.mark.parametrize("rows", [1, 3, 64])
def test_rows_longer_than_a_tile(rows):
    # 2 MiB rows (H=32, K=V=128 f32) split over 128 tiles each; a ragged 16-byte-unit tail row too
    srcs = [_odd((rows, 32, 128, 128), torch.float32, 0, 7), _odd((rows, 1031, 4), torch.float32, 0, 8)]
    gen = torch.Generator().manual_seed(rows)
    idx = torch.randint(0, rows, (rows + 1,), generator=gen).to(DEV)
    _check(cache.gather_rows(srcs, idx), srcs, idx)


def _state(B, H, K, V, width, seed):
    return KDAState(
        recurrent_state=_odd((B, H, K, V), torch.float32, 0, seed),
        q_conv_state=ShortConvState(_odd((B, 3, width), torch.bfloat16, 0, seed + 1)),
        k_conv_state=ShortConvState(_odd((B, 3, width), torch.bfloat16, 0, seed + 2)),
        v_conv_state=ShortConvState(_odd((B, 3, width), torch.bfloat16, 0, seed + 3)),
        sequence_offset=torch.arange(B, dtype=torch.long, device=DEV) * 7,
    )


def test_many_layers_span_several_launches():
    # 30 layers x 5 tensors = 150 descriptors: three launches of at most 64
    states = [_state(4, 2, 16, 16, 48, 10 * i) for i in range(30)]
    idx = torch.tensor([3, 3, 1, 0, 2, 1], dtype=torch.long, device=DEV)
    got = cache.reorder_states(states, idx)
    for s, r in zip(states, got):
        srcs = [s.recurrent_state, s.q_conv_state.buffer, s.k_conv_state.buffer, s.v_conv_state.buffer,
                s.sequence_offset]
        outs = [r.recurrent_state, r.q_conv_state.buffer, r.k_conv_state.buffer, r.v_conv_state.buffer,
                r.sequence_offset]
        _check(outs, srcs, idx)
    clones = cache.clone_states(states)
    for s, c in zip(states, clones):
        assert torch.equal(c.recurrent_state, s.recurrent_state)
        assert c.recurrent_state.data_ptr() != s.recurrent_state.data_ptr()


def test_state_methods_match_the_host_state():
    s = _state(3, 4, 32, 32, 64, 3)
    idx = torch.tensor([2, 0, 2], dtype=torch.long)
    host = KDAState(
        s.recurrent_state.cpu(), ShortConvState(s.q_conv_state.buffer.cpu()),
        ShortConvState(s.k_conv_state.buffer.cpu()), ShortConvState(s.v_conv_state.buffer.cpu()),
        s.sequence_offset.cpu(),
    ).reorder(idx)
    dev = s.reorder(idx.to(DEV))
    assert torch.equal(dev.recurrent_state.cpu(), host.recurrent_state)
    assert torch.equal(dev.k_conv_state.buffer.cpu(), host.k_conv_state.buffer)
    assert dev.sequence_offset.cpu().tolist() == host.sequence_offset.tolist()
    c = s.clone()
    assert torch.equal(c.v_conv_state.buffer, s.v_conv_state.buffer)
    assert c.v_conv_state.buffer.data_ptr() != s.v_conv_state.buffer.data_ptr()
    sc = s.q_conv_state.clone()
    assert torch.equal(sc.buffer, s.q_conv_state.buffer) and sc.buffer.data_ptr() != s.q_conv_state.buffer.data_ptr()


def test_empty_and_out_of_range():
    s = _state(2, 1, 16, 16, 16, 5)
    empty = s.reorder(torch.empty(0, dtype=torch.long, device=DEV))
    assert empty.recurrent_state.shape == (0, 1, 16, 16)
    for bad in ([2], [-1], [0, 5]):
        with pytest.raises(IndexError):
            s.reorder(torch.tensor(bad, dtype=torch.long, device=DEV))
    # the state is untouched and a later reorder still works
    ok = s.reorder(torch.tensor([1, 0], dtype=torch.long, device=DEV))
    assert torch.equal(ok.recurrent_state[0], s.recurrent_state[1])


def test_permutation_round_trip_at_decode_cache_size():
    B = 64
    s = _state(B, 32, 128, 128, 4096, 11)
    perm = torch.randperm(B, generator=torch.Generator().manual_seed(0)).to(DEV)
    once = s.reorder(perm)
    back = once.reorder(torch.argsort(perm))
    assert torch.equal(back.recurrent_state, s.recurrent_state)
    assert torch.equal(back.q_conv_state.buffer, s.q_conv_state.buffer)
    assert torch.equal(back.sequence_offset, s.sequence_offset)
    assert torch.equal(once.recurrent_state[5], s.recurrent_state[perm[5]])


def test_reorder_and_clone_are_differentiable_like_index_select():
    # KDAState.reorder / clone in the reference are index_select / clone, both
    # differentiable (src/kda/state.py:41-67): the native gather gives the same
    # gradients, duplicated indices accumulating
    gen = torch.Generator().manual_seed(4)
    src = torch.randn(4, 2, 16, 16, generator=gen).to(DEV).requires_grad_()
    buf = torch.randn(4, 3, 64, generator=gen).to(DEV).requires_grad_()
    idx = torch.tensor([3, 0, 3, 1, 3], dtype=torch.long, device=DEV)
    w1 = torch.randn(5, 2, 16, 16, generator=gen).to(DEV)
    w2 = torch.randn(5, 3, 64, generator=gen).to(DEV)
    out = cache.gather_rows([src, buf], idx)
    ((out[0] * w1).sum() + (out[1] * w2).sum()).backward()
    ref_src, ref_buf = src.detach().clone().requires_grad_(), buf.detach().clone().requires_grad_()
    ((ref_src.index_select(0, idx) * w1).sum() + (ref_buf.index_select(0, idx) * w2).sum()).backward()
    torch.testing.assert_close(src.grad, ref_src.grad, rtol=1e-6, atol=1e-6)
    torch.testing.assert_close(buf.grad, ref_buf.grad, rtol=1e-6, atol=1e-6)
    src.grad = None
    (cache.gather_rows([src], None)[0] * w1[:4]).sum().backward()
    torch.testing.assert_close(src.grad, w1[:4])
