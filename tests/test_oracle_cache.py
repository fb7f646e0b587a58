"""Pins of the oracle's cache gather (``gather_rows``) on the CPU.

The reference's reorder test (tests/hybrid_backbone/test_hybrid_cache.py:82-101)
picks batch rows [2, 0, 2] of every layer's state; the checks below use
literal expected rows, the permutation/inverse round trip and the clone's
byte equality, so an off-by-one row, a transposed copy or a shared buffer
fails one of them.
"""

from __future__ import annotations

import numpy as np
import pytest

from oracle import kda_oracle as ora


def test_reference_reorder_picks_literal_rows():
    state = np.arange(3 * 2 * 2, dtype=np.float32).reshape(3, 2, 2)
    offsets = np.array([5, 6, 7], dtype=np.int64)
    got_state, got_offsets = ora.gather_rows([state, offsets], [2, 0, 2])
    np.testing.assert_array_equal(got_state, [[[8, 9], [10, 11]], [[0, 1], [2, 3]], [[8, 9], [10, 11]]])
    np.testing.assert_array_equal(got_offsets, [7, 5, 7])


def test_permutation_then_inverse_is_identity_for_any_dtype():
    rng = np.random.default_rng(0)
    arrays = [
        rng.standard_normal((7, 3, 5)).astype(np.float32),
        rng.integers(-(2**15), 2**15, size=(7, 3, 37), dtype=np.int16),  # bf16 bits
        rng.integers(0, 255, size=(7, 13), dtype=np.uint8),
        rng.integers(0, 10**9, size=7, dtype=np.int64),
    ]
    perm = rng.permutation(7)
    inv = np.argsort(perm)
    once = ora.gather_rows(arrays, perm)
    back = ora.gather_rows(once, inv)
    for a, p, b in zip(arrays, once, back):
        np.testing.assert_array_equal(p, a[perm])
        np.testing.assert_array_equal(b, a)


def test_clone_is_an_independent_byte_copy():
    a = np.arange(24, dtype=np.float64).reshape(4, 6)
    (c,) = ora.gather_rows([a])
    np.testing.assert_array_equal(c, a)
    assert not np.shares_memory(c, a)


def test_expanding_and_empty_index():
    a = np.arange(6, dtype=np.int32).reshape(2, 3)
    (wide,) = ora.gather_rows([a], [1, 1, 0, 1])
    np.testing.assert_array_equal(wide, [[3, 4, 5], [3, 4, 5], [0, 1, 2], [3, 4, 5]])
    (empty,) = ora.gather_rows([a], [])
    assert empty.shape == (0, 3)


@pytest.mark.parametrize("bad", [[2], [-1], [0, 3]])
def test_out_of_range_index_raises(bad):
    with pytest.raises(IndexError):
        ora.gather_rows([np.zeros((2, 4), dtype=np.float32)], bad)
