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


def test_filter_and_merge_move_indices_only():
    p = make(8)
    batch = PooledBatch.new(p, 4)
    for i, s in enumerate(batch.slots):
        p.states[s] = float(i + 1)
    before = p.states.clone()
    batch.filter([3, 1])
    assert batch.slots == [3, 1] and p.n_free == 6
    assert batch.index.tolist() == [3, 1] and batch.index.dtype == torch.int32
    with pytest.raises(ValueError):
        batch.filter([0, 0])            # two rows on one state
    new = PooledBatch.new(p, 1)
    n0 = new.slots[0]
    merged = PooledBatch.merge([batch, new])
    assert merged.slots == [3, 1, n0] and batch.slots == [] and new.slots == []
    assert p.n_free == 5
    # no state moved
    assert torch.equal(p.states[[3, 1]], before[[3, 1]])


def test_extract_copies_and_batches_own_their_slots():
    p = make(6)
    batch = PooledBatch.new(p, 2)
    p.states[batch.slots[1]] = 5.0
    row = batch.extract(1)
    assert row.slots[0] not in batch.slots
    assert torch.all(p.states[row.slots[0]] == 5.0)
    p.states[batch.slots[1]] = 6.0                 # the extracted copy is independent
    assert torch.all(p.states[row.slots[0]] == 5.0)
    free = p.n_free
    del row                                        # garbage collection returns the slot
    assert p.n_free == free + 1
    batch.release()
    assert p.n_free == 6 and batch.slots == []


def test_arrays_cache_verbs_on_a_pooled_state():
    from multiplex_amd import ArraysCache, merge_layer, restore_ssm, snapshot_ssm

    p = make(10)
    c = ArraysCache()
    c[0] = torch.arange(3 * 2 * 5, dtype=torch.float32).reshape(3, 2, 5)
    c[1] = PooledBatch.new(p, 3)
    for i, s in enumerate(c[1].slots):
        p.states[s] = float(i)
    assert c.batch_size == 3 and c.nbytes == c[0].numel() * 4 + 3 * 2 * 4 * 8 * 4
    snap = snapshot_ssm([c, None])
    assert isinstance(snap[0][1], PooledBatch) and set(snap[0][1].slots).isdisjoint(c[1].slots)
    c.filter([2, 0])
    assert torch.equal(c[0][:, 0, 0], torch.tensor([20.0, 0.0]))
    assert [float(p.states[s][0, 0, 0]) for s in c[1].slots] == [2.0, 0.0]
    row = c.extract(1)
    assert float(p.states[row[1].slots[0]][0, 0, 0]) == 0.0 and row[1].slots[0] not in c[1].slots
    m = merge_layer([c, row])
    assert m.batch_size == 3 and m[1].slots[:2] != [] and c[1].slots == []
    restore_ssm([c], [snap[0]])
    assert [float(p.states[s][0, 0, 0]) for s in c[1].slots] == [0.0, 1.0, 2.0]


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
