"""State-container verbs (host logic; CPU tensors suffice)."""

from __future__ import annotations

import torch

from multiplex_amd.cache import (ArraysCache, clone_ssm, merge_layer, restore_ssm, restore_ssm_snapshot,
                                 snapshot_ssm)


def make(B, seed=0):
    g = torch.Generator().manual_seed(seed)
    c = ArraysCache()
    c[0] = torch.randn(B, 3, 16, generator=g).to(torch.bfloat16)
    c[1] = torch.randn(B, 2, 4, 8, generator=g)
    return c


class _Attn:  # a non-GDN layer cache stands in for attention KV
    pass


def test_not_trimmable_and_shapes():
    c = make(3)
    assert not c.is_trimmable()
    assert c.batch_size == 3 and len(c) == 2
    assert c.nbytes == 3 * 3 * 16 * 2 + 3 * 2 * 4 * 8 * 4
    assert ArraysCache().batch_size == 0


def test_filter_extract_merge_round_trip():
    c = make(4)
    rows = [c.extract(i) for i in range(4)]
    assert all(r.batch_size == 1 for r in rows)
    m = merge_layer([rows[2], rows[0], rows[3]])
    ref = make(4)
    ref.filter([2, 0, 3])
    for a, b in zip(m.cache, ref.cache):
        assert torch.equal(a, b)
    # extract copies: writing into the extracted row leaves the batch intact
    rows[1][1].zero_()
    assert torch.count_nonzero(c[1][1]) > 0
    assert torch.equal(ArraysCache.merge(rows[:2])[0], c[0][:2])


def test_snapshot_restore_are_copies():
    caches = [make(2, 1), _Attn(), make(2, 2)]
    snap = snapshot_ssm(caches)
    assert snap[1] is None
    before = [v.clone() for v in caches[0].cache]
    caches[0][1].add_(1.0)
    assert not torch.equal(caches[0][1], before[1])
    restore_ssm(caches, snap)
    assert torch.equal(caches[0][1], before[1]) and torch.equal(caches[0][0], before[0])
    # the restored arrays are copies: mutating them leaves the snapshot intact
    caches[0][1].add_(1.0)
    assert torch.equal(snap[0][1], before[1])


def test_prefix_cache_clone_and_restore():
    src = [make(1, 3), _Attn()]
    blob = clone_ssm(src)
    fresh = [ArraysCache(), _Attn()]
    restore_ssm_snapshot(fresh, blob)
    assert torch.equal(fresh[0][1], src[0][1]) and fresh[0][1].data_ptr() != src[0][1].data_ptr()


def test_none_entries_survive_verbs():
    c = ArraysCache()
    c[1] = torch.zeros(2, 1, 2, 2)
    c.filter([1])
    assert c[0] is None and c[1].shape[0] == 1
    m = merge_layer([c, c])
    assert m[0] is None and m[1].shape[0] == 2
