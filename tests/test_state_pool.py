"""Slot bookkeeping of the pooled states (host logic; CPU tensors, no kernels)."""

from __future__ import annotations

import pytest
import torch

from multiplex_amd import PooledBatch, StatePool


def make(n=6):
    return StatePool(n, 2, 4, 8, device="cpu")


def test_alloc_release_and_exhaustion():
    p = make()
    a = p.alloc(2)
    assert a == [0, 1] and p.n_free == 4
    assert torch.count_nonzero(p.states[a]) == 0
    b = p.alloc(4)
    assert sorted(a + b) == list(range(6))
    with pytest.raises(RuntimeError):
        p.alloc(1)
    p.release([1])
    with pytest.raises(ValueError):
        p.release([1])                   # double release
    assert p.alloc(1) == [1]


def test_alloc_zeroes_reused_slots():
    p = make()
    s = p.alloc(1)
    p.states[s[0]] = 3.0
    p.release(s)
    assert p.alloc(1) == s and torch.count_nonzero(p.states[s[0]]) == 0


def test_filter_extract_merge_move_indices_only():
    p = make(8)
    batch = PooledBatch.new(p, 4)
    for i, s in enumerate(batch.slots):
        p.states[s] = float(i + 1)
    before = p.states.clone()
    batch.filter([3, 1])
    assert batch.slots == [3, 1] and p.n_free == 6
    assert batch.index.tolist() == [3, 1] and batch.index.dtype == torch.int32
    one = batch.extract(0)
    assert one.slots == [3]
    new = PooledBatch.new(p, 1)
    merged = PooledBatch.merge([batch, new])
    assert merged.slots == [3, 1, new.slots[0]]
    # no state moved
    assert torch.equal(p.states[[3, 1]], before[[3, 1]])


def test_snapshot_restore_and_dense_round_trip():
    p = make(8)
    batch = PooledBatch.new(p, 2)
    p.states[batch.slots[0]] = 1.0
    p.states[batch.slots[1]] = 2.0
    snap = batch.snapshot()
    assert set(snap.slots).isdisjoint(batch.slots)
    p.states[batch.slots] = 7.0
    assert torch.all(p.states[snap.slots[0]] == 1.0)
    batch.restore(snap)
    assert torch.all(p.states[batch.slots[1]] == 2.0)
    dense = p.gather(batch.slots)
    assert dense.shape == (2, 2, 4, 8)
    other = PooledBatch.new(p, 2)
    p.scatter(other.slots, dense)
    assert torch.equal(p.gather(other.slots), dense)
    with pytest.raises(ValueError):
        p.scatter(other.slots, dense[:1])
    with pytest.raises(ValueError):
        PooledBatch.merge([batch, PooledBatch(make(), [0])])
