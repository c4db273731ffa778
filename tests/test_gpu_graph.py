"""HIP-graph capture of a decode step of the GDN path (fused prologue, the
recurrent kernel updating the state in place, fused gated RMSNorm).

The library only enqueues kernels on the caller's stream (no allocation, no
memset, no synchronisation), so a serving loop can capture a step once and
replay it.  The graph is replayed several times with eager work (input
refills, the conv-state hand-over) and synchronisations between replays,
and every replay is checked bit for bit against the same step run eagerly.
"""

from __future__ import annotations

import pytest
import torch

import multiplex_amd as mx

pytestmark = pytest.mark.gpu
DEV = "cuda"
B, Hk, Hv, D = 8, 2, 4, 128
C = 2 * Hk * D + Hv * D


def step(qkv, w, cs, a, b, A_log, dt_bias, state, z, nw):
    q, k, v, cs_new = mx.gdn_conv_prologue(qkv, w, Hk, Hv, D, D, cs)
    y, _ = mx.gated_delta_update(q, k, v, a, b, A_log, dt_bias, state, state_out=state)
    return mx.gated_rms_norm(y, z, nw), cs_new


@torch.no_grad()
def test_decode_step_graph_replays_match_eager():
    g = torch.Generator().manual_seed(41)
    w = (torch.randn(C, 4, generator=g) * 0.1).to(torch.bfloat16).to(DEV)
    A_log = (torch.rand(Hv, generator=g) * 2.7).to(DEV)
    dt_bias = (torch.rand(Hv, generator=g) * 2 - 1).to(DEV)
    nw = (1 + 0.1 * torch.randn(D, generator=g)).to(torch.bfloat16).to(DEV)
    qkv = torch.empty(B, 1, C, dtype=torch.bfloat16, device=DEV)
    a = torch.empty(B, 1, Hv, dtype=torch.bfloat16, device=DEV)
    b = torch.empty_like(a)
    z = torch.empty(B, 1, Hv, D, dtype=torch.bfloat16, device=DEV)
    cs = (torch.randn(B, 3, C, generator=g)).to(torch.bfloat16).to(DEV)
    state = (torch.randn(B, Hv, D, D, generator=g) * 0.02).to(DEV)

    def fill(i):
        gi = torch.Generator().manual_seed(100 + i)
        qkv.copy_(torch.randn(B, 1, C, generator=gi).to(torch.bfloat16))
        a.copy_(torch.randn(B, 1, Hv, generator=gi).to(torch.bfloat16))
        b.copy_(torch.randn(B, 1, Hv, generator=gi).to(torch.bfloat16))
        z.copy_(torch.randn(B, 1, Hv, D, generator=gi).to(torch.bfloat16))

    ref_state, ref_cs = state.clone(), cs.clone()
    fill(0)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out_g, cs_new_g = step(qkv, w, cs, a, b, A_log, dt_bias, state, z, nw)
    # capture records the launches without running them
    assert torch.equal(state, ref_state)

    for i in range(4):
        fill(i)
        out_e, cs_e = step(qkv, w, ref_cs, a, b, A_log, dt_bias, ref_state, z, nw)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out_g, out_e), f"replay {i}: output"
        assert torch.equal(state, ref_state), f"replay {i}: state"
        assert torch.equal(cs_new_g, cs_e), f"replay {i}: conv state"
        # eager work between replays: the conv state moves to the input buffer
        cs.copy_(cs_new_g)
        ref_cs = cs_e
        torch.cuda.synchronize()


@torch.no_grad()
def test_prepared_launches_replay_in_a_graph():
    """Prepared launches (validated once) captured with ``launch(stream)``:
    50 decode steps in one graph equal 50 eager launches."""
    g = torch.Generator().manual_seed(43)
    q = torch.nn.functional.normalize(torch.randn(B, 1, Hk, D, generator=g), dim=-1).to(torch.bfloat16).to(DEV)
    k = torch.nn.functional.normalize(torch.randn(B, 1, Hk, D, generator=g), dim=-1).to(torch.bfloat16).to(DEV)
    v = torch.randn(B, 1, Hv, D, generator=g).to(torch.bfloat16).to(DEV)
    a = torch.randn(B, 1, Hv, generator=g).to(torch.bfloat16).to(DEV)
    b = torch.randn(B, 1, Hv, generator=g).to(torch.bfloat16).to(DEV)
    A_log = (torch.rand(Hv, generator=g) * 2.7).to(DEV)
    dt_bias = (torch.rand(Hv, generator=g) * 2 - 1).to(DEV)
    state = (torch.randn(B, Hv, D, D, generator=g) * 0.02).to(DEV)
    ref = state.clone()
    plan = mx.prepare_recurrent(q, k, v, a, b, A_log, dt_bias, state, state_out=state)
    eager = mx.prepare_recurrent(q, k, v, a, b, A_log, dt_bias, ref, state_out=ref)
    graph, n = torch.cuda.CUDAGraph(), 50
    with torch.cuda.graph(graph):
        cap = torch.cuda.current_stream()
        for _ in range(n):
            plan.launch(cap)
    assert torch.equal(state, ref)
    for r in range(3):
        for _ in range(n):
            eager.launch()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(state, ref), f"replay {r}"
        assert torch.equal(plan.outputs[0], eager.outputs[0]), f"replay {r}: y"


@torch.no_grad()
def test_packed_calls_with_device_offsets_capture_in_a_graph():
    """Packed calls whose ``cu_seqlens`` (and commit lengths) are device
    tensors read nothing back to the host, so they can be captured: the
    chunked and the recurrent packed updates and a packed commit, replayed
    with the offsets and inputs changed between replays."""
    g = torch.Generator().manual_seed(47)
    n_tok, n_seqs = 300, 3
    q = torch.nn.functional.normalize(torch.randn(1, n_tok, Hk, D, generator=g), dim=-1).to(torch.bfloat16).to(DEV)
    k = torch.nn.functional.normalize(torch.randn(1, n_tok, Hk, D, generator=g), dim=-1).to(torch.bfloat16).to(DEV)
    v = torch.randn(1, n_tok, Hv, D, generator=g).to(torch.bfloat16).to(DEV)
    a = torch.randn(1, n_tok, Hv, generator=g).to(torch.bfloat16).to(DEV)
    b = torch.randn(1, n_tok, Hv, generator=g).to(torch.bfloat16).to(DEV)
    A_log = (torch.rand(Hv, generator=g) * 2.7).to(DEV)
    dt_bias = (torch.rand(Hv, generator=g) * 2 - 1).to(DEV)
    state = (torch.randn(n_seqs, Hv, D, D, generator=g) * 0.02).to(DEV)
    cu = torch.tensor([0, 100, 130, 300], dtype=torch.int32, device=DEV)
    n_commit = torch.tensor([5, 0, 64], dtype=torch.int32, device=DEV)

    def calls():
        yc, Sc = mx.gated_delta_update(q, k, v, a, b, A_log, dt_bias, state, cu_seqlens=cu, chunked=True)
        yr, Sr = mx.gated_delta_update(q, k, v, a, b, A_log, dt_bias, state, cu_seqlens=cu, chunked=False)
        Sm = mx.gated_delta_commit(k, v, a, b, A_log, dt_bias, state, n_commit, cu_seqlens=cu)
        return yc, Sc, yr, Sr, Sm

    calls()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        outs = calls()
    for r, offsets in enumerate(([0, 100, 130, 300], [0, 64, 64, 300], [0, 1, 299, 300])):
        cu.copy_(torch.tensor(offsets, dtype=torch.int32))
        v.mul_(-1.0)
        eager = calls()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for i, (x, y) in enumerate(zip(outs, eager)):
            assert torch.equal(x, y), f"replay {r}: output {i}"
