"""Host-side behaviour of the operator wrappers that needs no GPU: the same
validation errors as the reference (src/kda/utils.py:8-71,
src/kda/chunkwise.py:34-37) raised before any compute, and a loud error —
never a CPU fallback — for tensors that are not on a ROCm GPU."""

from __future__ import annotations

import pytest
import torch

import kda
from kda.utils import accumulation_dtype, validate_cu_seqlens
from tests._inputs import random_core


def _core(**kw):
    return random_core(**kw)


@pytest.mark.parametrize("fn", [kda.chunkwise_kda, kda.recurrent_kda])
def test_shape_errors_match_reference(fn):
    q, k, v, g, beta, state = _core()
    with pytest.raises(ValueError, match=r"q must have shape"):
        fn(q[0], k, v, g, beta)
    with pytest.raises(ValueError, match="empty sequences"):
        fn(q[:, :0], k[:, :0], v[:, :0], g[:, :0], beta[:, :0])
    with pytest.raises(ValueError, match="same shape as q"):
        fn(q, k[..., :1], v, g, beta)
    with pytest.raises(ValueError, match=r"v must have shape"):
        fn(q, k, v[:, :, :1], g, beta)
    with pytest.raises(ValueError, match="beta must have shape"):
        fn(q, k, v, g, beta[..., :1])
    with pytest.raises(ValueError, match="initial_state must have shape"):
        fn(q, k, v, g, beta, state[:, :, :1])
    with pytest.raises(TypeError, match="floating-point"):
        fn(q, k, v, g, (beta * 10).long())


@pytest.mark.parametrize("fn", [kda.chunkwise_kda, kda.recurrent_kda])
@pytest.mark.parametrize(
    "mask",
    [
        torch.ones(2, 7),
        torch.ones(2, 6, dtype=torch.bool),
        torch.tensor([[True, False, True] + [True] * 4, [True] * 7]),
        torch.zeros(2, 7, dtype=torch.bool),
    ],
)
def test_invalid_masks_rejected(fn, mask):
    q, k, v, g, beta, _ = _core()
    with pytest.raises((TypeError, ValueError)):
        fn(q, k, v, g, beta, attention_mask=mask)


def test_chunk_argument_checks():
    q, k, v, g, beta, _ = _core()
    with pytest.raises(ValueError, match="must be > 0"):
        kda.chunkwise_kda(q, k, v, g, beta, chunk_size=0)
    with pytest.raises(ValueError, match="secondary_tile_size must be <= chunk_size"):
        kda.chunkwise_kda(q, k, v, g, beta, chunk_size=4, secondary_tile_size=8)


def test_cu_seqlens_validation():
    assert validate_cu_seqlens(torch.tensor([0, 3, 7]), 1, 7, None) == [0, 3, 7]
    with pytest.raises(ValueError, match="B == 1"):
        validate_cu_seqlens([0, 7], 2, 7, None)
    with pytest.raises(ValueError, match="start at 0 and end"):
        validate_cu_seqlens([0, 3, 6], 1, 7, None)
    with pytest.raises(ValueError, match="strictly increasing"):
        validate_cu_seqlens([0, 3, 3, 7], 1, 7, None)
    with pytest.raises(TypeError):
        validate_cu_seqlens(torch.tensor([0.0, 7.0]), 1, 7, None)
    with pytest.raises(ValueError, match="cannot be combined"):
        validate_cu_seqlens([0, 7], 1, 7, torch.ones(1, 7, dtype=torch.bool))


def test_accumulation_dtype_rule():
    assert accumulation_dtype(torch.bfloat16, True) == torch.float32
    assert accumulation_dtype(torch.float16, True) == torch.float32
    assert accumulation_dtype(torch.bfloat16, False) == torch.bfloat16
    assert accumulation_dtype(torch.float64, True) == torch.float64


@pytest.mark.parametrize("fn", [kda.chunkwise_kda, kda.recurrent_kda])
def test_cpu_tensors_fail_loudly(fn):
    q, k, v, g, beta, state = _core()
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        fn(q, k, v, g, beta, state, True)


def test_ut_transform_validation_and_cpu_error():
    _, k, v, g, beta, _ = _core()
    with pytest.raises(ValueError):
        kda.ut_transform(k[..., :1], v, g, beta)
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        kda.ut_transform(k, v, g, beta)


def test_state_dataclass_contract():
    state = kda.KDAState(
        recurrent_state=torch.zeros(2, 3, 4, 5),
        q_conv_state=kda.ShortConvState(torch.zeros(2, 3, 12)),
        k_conv_state=kda.ShortConvState(torch.zeros(2, 3, 12)),
        v_conv_state=kda.ShortConvState(torch.zeros(2, 3, 15)),
        sequence_offset=torch.tensor([4, 6]),
    )
    clone = state.clone()
    assert clone.recurrent_state.data_ptr() != state.recurrent_state.data_ptr()
    picked = state.reorder(torch.tensor([1, 1, 0]))
    assert picked.recurrent_state.shape == (3, 3, 4, 5)
    assert picked.sequence_offset.tolist() == [6, 6, 4]
    with pytest.raises(TypeError):
        kda.KDAState(state.recurrent_state, state.q_conv_state, state.k_conv_state, state.v_conv_state,
                     torch.tensor([4.0, 6.0]))
    with pytest.raises(ValueError):
        state.reorder(torch.tensor([0.0]))


def test_packed_backward_buckets_group_documents_of_similar_length():
    from kda.chunkwise import _document_buckets

    lens = [70, 1, 130, 64, 128, 100]
    buckets = _document_buckets(lens, lambda n, tokens: True)
    # every document exactly once, and within a bucket no document is shorter
    # than 0.8 of the bucket's first (longest)
    assert sorted(i for b in buckets for i in b) == list(range(len(lens)))
    for b in buckets:
        assert all(5 * lens[i] >= 4 * lens[b[0]] and lens[i] <= lens[b[0]] for i in b)
    assert [[lens[i] for i in b] for b in buckets] == [[130, 128], [100], [70, 64], [1]]
    # the workspace bound caps a bucket's size
    capped = _document_buckets([100] * 5, lambda n, tokens: n <= 2)
    assert [len(b) for b in capped] == [2, 2, 1]


def test_head_groups_fit_the_workspace_limit(monkeypatch):
    # a call whose workspace passes WORKSPACE_LIMIT runs the largest head
    # groups that fit (at least one head a group)
    from kda import chunkwise

    def need(B, T):
        return lambda H: 1000 + B * T * H * 10

    monkeypatch.setattr(chunkwise, "WORKSPACE_LIMIT", 1000 + 10 * 64 * 10)
    assert chunkwise._head_group(need(1, 10), 64) == 64
    assert chunkwise._head_group(need(2, 10), 64) == 32
    assert chunkwise._head_group(need(1, 30), 64) == 21
    assert chunkwise._head_group(need(1, 10 ** 6), 64) == 1
    assert chunkwise._head_group(lambda H: 0, 8) == 8
