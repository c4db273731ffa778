"""GPU path of the prefix-cache state records: an asynchronous device ->
pinned-host snapshot taken right after a kernel, written by the background
writer, read back and uploaded; a mixer restored from the record continues
exactly like the one it was taken from."""

from __future__ import annotations

import torch

import multiplex_amd as mx
from multiplex_amd import prefix_state as ps

import pytest

pytestmark = pytest.mark.gpu
DEV = "cuda"
HID, HK, HV, D = 256, 2, 4, 128


def test_staged_copy_sees_the_preceding_kernel():
    g = torch.Generator().manual_seed(1)
    B = 3
    q = (torch.randn(B, 1, HK, D, generator=g) / 16).to(torch.bfloat16).to(DEV)
    k = torch.nn.functional.normalize(torch.randn(B, 1, HK, D, generator=g), dim=-1).to(torch.bfloat16).to(DEV)
    v = torch.randn(B, 1, HV, D, generator=g).to(torch.bfloat16).to(DEV)
    a = torch.randn(B, 1, HV, generator=g).to(torch.bfloat16).to(DEV)
    b = torch.randn(B, 1, HV, generator=g).to(torch.bfloat16).to(DEV)
    A_log, dt_bias = torch.rand(HV).to(DEV), torch.rand(HV).to(DEV)
    state = (torch.randn(B, HV, D, D, generator=g) * 0.02).to(DEV)
    _, new_state = mx.gated_delta_update(q, k, v, a, b, A_log, dt_bias, state, state_out=state)
    staged = ps.stage_to_host([[None, new_state]])      # queued behind the kernel, no sync here
    host = staged.wait()
    assert host[0][1].is_pinned()
    assert torch.equal(host[0][1], new_state.cpu())


def test_staged_clone_survives_a_later_in_place_update_and_reuse():
    """Stage a clone, drop it, then queue an in-place decode of the live
    state and an allocation of the same size: the snapshot still holds the
    pre-update state (the source is marked used on the copy stream, so its
    memory is not handed out while the copy is pending)."""
    g = torch.Generator().manual_seed(4)
    B = 64
    q = (torch.randn(B, 1, HK, D, generator=g) / 16).to(torch.bfloat16).to(DEV)
    k = torch.nn.functional.normalize(torch.randn(B, 1, HK, D, generator=g), dim=-1).to(torch.bfloat16).to(DEV)
    v = torch.randn(B, 1, HV, D, generator=g).to(torch.bfloat16).to(DEV)
    a = torch.randn(B, 1, HV, generator=g).to(torch.bfloat16).to(DEV)
    b = torch.randn(B, 1, HV, generator=g).to(torch.bfloat16).to(DEV)
    A_log, dt_bias = torch.rand(HV).to(DEV), torch.rand(HV).to(DEV)
    state = (torch.randn(B, HV, D, D, generator=g) * 0.02).to(DEV)
    expect = state.cpu()
    snap = state.clone()
    staged = ps.stage_to_host([snap])
    del snap
    for _ in range(4):
        mx.gated_delta_update(q, k, v, a, b, A_log, dt_bias, state, state_out=state)
    junk = torch.full_like(state, 7.0)
    host = staged.wait()
    assert torch.equal(host[0], expect)
    assert not torch.equal(state.cpu(), expect) and bool((junk == 7.0).all())


@torch.no_grad()
def test_record_round_trip_restores_a_mixer(tmp_path):
    m = mx.GatedDeltaNet(HID, HK, HV, D, D, device=DEV)
    m.reset_parameters(torch.Generator().manual_seed(2))
    g = torch.Generator().manual_seed(3)
    x = torch.randn(2, 9, HID, generator=g).to(torch.bfloat16).to(DEV)
    caches = [mx.ArraysCache(), None, mx.ArraysCache()]
    m(x, None, caches[0])
    m(x.flip(1).contiguous(), None, caches[2])
    snap = mx.clone_ssm(caches)
    writer = ps.AsyncStateWriter(tmp_path)
    try:
        writer.submit("c0" * 32, ps.stage_to_host(snap), tokens=list(range(9)), pos=9)
        writer.flush()
        restored = writer.load_ssm("c0" * 32, device=DEV)
    finally:
        writer.close()
    fresh = [mx.ArraysCache(), None, mx.ArraysCache()]
    mx.restore_ssm_snapshot(fresh, restored)
    for c0, c1 in ((caches[0], fresh[0]), (caches[2], fresh[2])):
        assert torch.equal(c0[0], c1[0]) and torch.equal(c0[1], c1[1])
    x2 = torch.randn(2, 1, HID, generator=g).to(torch.bfloat16).to(DEV)
    for i in (0, 2):
        assert torch.equal(m(x2, None, caches[i]), m(x2, None, fresh[i]))
        assert torch.equal(caches[i][1], fresh[i][1])
