"""GPU checks of pooled states (``state_index``): every kernel path gives
bit-identical results whether a row's state sits in a dense batch tensor or
in a pool slot, slots of other rows are untouched, rows whose slot lies
outside the pool are skipped, and a batch lifecycle (steps, filter, merge)
through the pool equals the dense ArraysCache lifecycle."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import multiplex_amd as mx
from gdn_cases import STATE_TOL, Y_TOL, draw, head_errs_state, row_errs_y, to_torch
from oracle import gdn

pytestmark = pytest.mark.gpu
DEV = "cuda"
Hk, Hv, D = 2, 4, 128


def pool_with(seed, n_slots):
    g = torch.Generator().manual_seed(seed)
    pool = mx.StatePool(n_slots, Hv, D, D, device=DEV)
    pool.states.copy_(torch.randn(pool.states.shape, generator=g) * 0.02)
    return pool


def inputs(seed, B, T):
    t, _ = to_torch(draw(seed, B, T, Hk, Hv, D, D, state=False), DEV)
    return t


def gdn_args(t):
    return t["q"], t["k"], t["v"], t["a"], t["b"], t["A_log"], t["dt_bias"]


def others_unchanged(pool, before, slots):
    rest = [s for s in range(pool.n_slots) if s not in set(slots)]
    assert torch.equal(pool.states[rest], before[rest])


def test_decode_pooled_equals_dense():
    pool = pool_with(1, 11)
    slots = [7, 2, 9, 0, 5, 3]
    t = inputs(2, len(slots), 1)
    before = pool.states.clone()
    dense = before[slots].clone()
    y_d, S_d = mx.gated_delta_update(*gdn_args(t), dense)
    idx = pool.index(slots)
    y_p, out = mx.gated_delta_update(*gdn_args(t), pool.states, state_index=idx)
    torch.cuda.synchronize()
    assert out.data_ptr() == pool.states.data_ptr()      # in place on the pool
    assert torch.equal(y_p, y_d)
    assert torch.equal(pool.states[slots], S_d)
    others_unchanged(pool, before, slots)


def test_verify_and_commit_pooled_equal_dense():
    pool = pool_with(3, 9)
    slots = [8, 1, 4, 6]
    T = 4
    t = inputs(4, len(slots), T)
    n = torch.tensor([1, 4, 0, 3], dtype=torch.int32)
    before = pool.states.clone()
    dense = before[slots].clone()
    y_d, _ = mx.gated_delta_verify(*gdn_args(t), dense)
    S_d = mx.gated_delta_commit(*gdn_args(t)[1:], dense, n)
    idx = pool.index(slots)
    y_p, _ = mx.gated_delta_verify(*gdn_args(t), pool.states, state_index=idx)
    torch.cuda.synchronize()
    assert torch.equal(pool.states, before)               # verify writes nothing
    mx.gated_delta_commit(*gdn_args(t)[1:], pool.states, n, state_index=idx)
    torch.cuda.synchronize()
    assert torch.equal(y_p, y_d)
    assert torch.equal(pool.states[slots], S_d)
    others_unchanged(pool, before, slots)


@pytest.mark.parametrize("fresh", [False, True])
def test_chunked_prefill_pooled_equals_dense(fresh):
    pool = pool_with(5, 7)
    slots = [5, 0, 3]
    lens = [100, 64, 200]
    cu = [0, 100, 164, 364]
    t = inputs(6, 1, sum(lens))
    before = pool.states.clone()
    dense = None if fresh else before[slots].clone()
    y_d, S_d = mx.gated_delta_update(*gdn_args(t), dense, cu_seqlens=cu, chunked=True)
    idx = pool.index(slots)
    if fresh:
        y_p, _ = mx.gated_delta_update(*gdn_args(t), None, cu_seqlens=cu, chunked=True, state_index=idx,
                                       state_out=pool.states)
    else:
        y_p, _ = mx.gated_delta_update(*gdn_args(t), pool.states, cu_seqlens=cu, chunked=True, state_index=idx)
    torch.cuda.synchronize()
    assert torch.equal(y_p, y_d)
    assert torch.equal(pool.states[slots], S_d)
    others_unchanged(pool, before, slots)


def test_rows_with_out_of_range_slots_are_skipped():
    pool = pool_with(7, 6)
    slots = [1, -1, 6, 4]                                  # rows 1 and 2 have no valid slot
    t = inputs(8, len(slots), 3)
    before = pool.states.clone()
    dense = torch.zeros(len(slots), Hv, D, D, device=DEV)
    dense[0], dense[3] = before[1], before[4]
    y_d, S_d = mx.gated_delta_update(*gdn_args(t), dense)
    y_p, _ = mx.gated_delta_update(*gdn_args(t), pool.states, state_index=torch.tensor(slots, dtype=torch.int32,
                                                                                        device=DEV))
    torch.cuda.synchronize()
    for b, s in ((0, 1), (3, 4)):
        assert torch.equal(y_p[b], y_d[b])
        assert torch.equal(pool.states[s], S_d[b])
    others_unchanged(pool, before, [1, 4])


def test_batch_lifecycle_through_the_pool_equals_dense():
    """Three decode steps on 4 rows, drop rows 1 and 3, add a fresh row,
    two more steps: pooled (indices only) vs dense (index_select + cat),
    and both against the float64 oracle."""
    pool = pool_with(9, 8)
    batch = mx.PooledBatch(pool, pool.alloc(4, zero=False))
    dense = pool.gather(batch.slots)
    ref_state = dense.double().cpu().numpy()

    def step(seed, dense, ref_state):
        t, r = to_torch(draw(seed, len(batch), 1, Hk, Hv, D, D, state=False), DEV)
        y_d, dense = mx.gated_delta_update(*gdn_args(t), dense)
        y_p, _ = mx.gated_delta_update(*gdn_args(t), pool.states, state_index=batch.index)
        torch.cuda.synchronize()
        assert torch.equal(y_p, y_d)
        assert torch.equal(pool.gather(batch.slots), dense)
        y_r, ref_state = gdn.gated_delta_update(r["q"], r["k"], r["v"], r["a"], r["b"], r["A_log"], r["dt_bias"],
                                                ref_state)
        assert row_errs_y(y_p.float().cpu().numpy(), y_r).max() <= Y_TOL
        assert head_errs_state(dense.cpu().numpy(), ref_state).max() <= STATE_TOL
        return dense, ref_state

    for s in range(3):
        dense, ref_state = step(20 + s, dense, ref_state)
    batch.filter([0, 2])
    dense = dense.index_select(0, torch.tensor([0, 2], device=DEV))
    ref_state = ref_state[[0, 2]]
    new = mx.PooledBatch.new(pool, 1)
    batch = mx.PooledBatch.merge([batch, new])
    dense = torch.cat([dense, torch.zeros(1, Hv, D, D, device=DEV)])
    ref_state = np.concatenate([ref_state, np.zeros((1, Hv, D, D))])
    for s in range(2):
        dense, ref_state = step(30 + s, dense, ref_state)


def test_prepared_pooled_decode_equals_call():
    pool = pool_with(11, 5)
    slots = [4, 1]
    t = inputs(12, 2, 1)
    ref_pool = pool.states.clone()
    idx = pool.index(slots)
    y_c, _ = mx.gated_delta_update(*gdn_args(t), ref_pool, state_index=idx)
    plan = mx.prepare_recurrent(*gdn_args(t), pool.states, state_index=idx, state_out=pool.states)
    plan.launch()
    torch.cuda.synchronize()
    assert torch.equal(plan.outputs[0], y_c)
    assert torch.equal(pool.states, ref_pool)


@torch.no_grad()
def test_mixer_on_pooled_states_equals_dense():
    """The GatedDeltaNet mixer with ``cache[1]`` a PooledBatch: prefill,
    decode, verify + commit, filter and merge give bit-identical outputs and
    states to the dense ArraysCache path."""
    hid = 256
    m = mx.GatedDeltaNet(hid, Hk, Hv, D, D, device=DEV)
    m.reset_parameters(torch.Generator().manual_seed(31))
    pool = mx.StatePool(12, Hv, D, D, device=DEV)
    g = torch.Generator().manual_seed(32)

    def x(B, S):
        return torch.randn(B, S, hid, generator=g).to(torch.bfloat16).to(DEV)

    def same(dense, pooled):
        assert torch.equal(dense[0], pooled[0])
        assert torch.equal(dense[1], pool.gather(pooled[1].slots))

    dense, pooled = mx.ArraysCache(), mx.ArraysCache()
    pooled[1] = mx.PooledBatch.new(pool, 3)
    x0 = x(3, 7)
    assert torch.equal(m(x0, None, dense), m(x0, None, pooled))
    same(dense, pooled)
    x1 = x(3, 1)
    assert torch.equal(m(x1, None, dense), m(x1, None, pooled))
    same(dense, pooled)
    xv, n = x(3, 4), torch.tensor([1, 4, 2], dtype=torch.int32)
    o_d = m(xv, None, dense, verify=True)
    m.commit(dense, n)
    o_p = m(xv, None, pooled, verify=True)
    m.commit(pooled, n)
    assert torch.equal(o_d, o_p)
    same(dense, pooled)
    dense.filter([2, 0])
    pooled.filter([2, 0])
    fresh_d, fresh_p = mx.ArraysCache(), mx.ArraysCache()
    fresh_p[1] = mx.PooledBatch.new(pool, 1)
    xf = x(1, 5)
    assert torch.equal(m(xf, None, fresh_d), m(xf, None, fresh_p))
    dense = mx.merge_layer([dense, fresh_d])
    pooled = mx.merge_layer([pooled, fresh_p])
    x2 = x(3, 1)
    assert torch.equal(m(x2, None, dense), m(x2, None, pooled))
    same(dense, pooled)
    assert pool.n_free == 12 - 3


def test_verify_paths_skip_out_of_range_slots():
    """A plain verify (the MFMA verify kernel) and a verify that commits the
    previous round (the stepping kernel) skip rows whose slot lies outside
    the pool: their y and slots are untouched, the other rows equal the
    dense launch."""
    pool = pool_with(11, 6)
    slots = [1, -1, 6, 4]
    idx = torch.tensor(slots, dtype=torch.int32, device=DEV)
    t = inputs(12, len(slots), 4)
    before = pool.states.clone()
    dense = torch.zeros(len(slots), Hv, D, D, device=DEV)
    dense[0], dense[3] = before[1], before[4]
    y_d, _ = mx.gated_delta_verify(*gdn_args(t), dense)
    y_p, _ = mx.gated_delta_verify(*gdn_args(t), pool.states, state_index=idx)
    torch.cuda.synchronize()
    for b in (0, 3):
        assert torch.equal(y_p[b], y_d[b])
    assert torch.equal(pool.states, before)
    prev = inputs(13, len(slots), 4)
    pv = tuple(prev[n] for n in ("q", "k", "v", "a", "b"))
    n_prev = [2, 1, 3, 4]
    y_d2, S_d2 = mx.gated_delta_commit_verify(pv, n_prev, *gdn_args(t), dense)
    y_p2, _ = mx.gated_delta_commit_verify(pv, n_prev, *gdn_args(t), pool.states, state_index=idx)
    torch.cuda.synchronize()
    for b, s in ((0, 1), (3, 4)):
        assert torch.equal(y_p2[b], y_d2[b])
        assert torch.equal(pool.states[s], S_d2[b])
    others_unchanged(pool, before, [1, 4])
