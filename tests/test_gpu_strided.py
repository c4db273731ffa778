"""Column slices of one fused in_proj output, read in place: qkv (prologue and
conv-state commit), z (gated RMSNorm) and a / b (recurrent, verify, commit
and chunked kernels) give bit-identical results to contiguous copies."""

from __future__ import annotations

import pytest
import torch

import multiplex_amd as mx

pytestmark = pytest.mark.gpu
DEV = "cuda"
Hk, Hv, D = 2, 4, 128
C = 2 * Hk * D + Hv * D


def fused(B, T, seed, extra=24):
    """One [B, T, C + Hv*D + 2 Hv + extra] buffer and its qkv / z / b / a slices."""
    g = torch.Generator().manual_seed(seed)
    width = C + Hv * D + 2 * Hv + extra
    buf = torch.randn(B, T, width, generator=g).to(torch.bfloat16).to(DEV)
    qkv = buf[..., :C]
    z = buf[..., C:C + Hv * D].unflatten(-1, (Hv, D))
    b = buf[..., C + Hv * D:C + Hv * D + Hv]
    a = buf[..., C + Hv * D + Hv:C + Hv * D + 2 * Hv]
    return qkv, z, a, b


def params(seed):
    g = torch.Generator().manual_seed(seed)
    w = (torch.randn(C, 4, generator=g) * 0.1).to(torch.bfloat16).to(DEV)
    A_log = (torch.rand(Hv, generator=g) * 2.7).to(DEV)
    dt_bias = (torch.rand(Hv, generator=g) * 2 - 1).to(DEV)
    state = (torch.randn(3, Hv, D, D, generator=g) * 0.02).to(DEV)
    return w, A_log, dt_bias, state


@pytest.mark.parametrize("T", [1, 4, 9])
def test_prologue_and_conv_commit_read_a_qkv_slice(T):
    qkv, _, _, _ = fused(3, T, 1 + T)
    assert not qkv.is_contiguous()
    w, _, _, _ = params(2)
    cs = torch.randn(3, 3, C, generator=torch.Generator().manual_seed(3)).to(torch.bfloat16).to(DEV)
    got = mx.gdn_conv_prologue(qkv, w, Hk, Hv, D, D, cs)
    ref = mx.gdn_conv_prologue(qkv.contiguous(), w, Hk, Hv, D, D, cs)
    for x, y in zip(got, ref):
        assert torch.equal(x, y)
    n = torch.tensor([0, T, min(2, T)], dtype=torch.int32)
    assert torch.equal(mx.conv_state_commit(cs, qkv, n), mx.conv_state_commit(cs, qkv.contiguous(), n))


def test_norm_reads_z_lines():
    _, z, _, _ = fused(3, 5, 4)
    assert not z.is_contiguous()
    y = torch.randn(3, 5, Hv, D, generator=torch.Generator().manual_seed(5)).to(torch.bfloat16).to(DEV)
    nw = torch.linspace(0.5, 1.5, D).to(torch.bfloat16).to(DEV)
    assert torch.equal(mx.gated_rms_norm(y, z, nw), mx.gated_rms_norm(y, z.contiguous(), nw))
    plan = mx.prepare_gated_rms_norm(y, z, nw)
    plan.launch()
    torch.cuda.synchronize()
    assert torch.equal(plan.outputs[0], mx.gated_rms_norm(y, z.contiguous(), nw))


def qkv_heads(qkv):
    B, T = qkv.shape[:2]
    q = torch.nn.functional.normalize(qkv[..., :Hk * D].float().reshape(B, T, Hk, D), dim=-1) / 11.3
    k = torch.nn.functional.normalize(qkv[..., Hk * D:2 * Hk * D].float().reshape(B, T, Hk, D), dim=-1)
    v = qkv[..., 2 * Hk * D:].reshape(B, T, Hv, D)
    return q.to(torch.bfloat16).contiguous(), k.to(torch.bfloat16).contiguous(), v.contiguous()


@pytest.mark.parametrize("T", [1, 4, 12])
def test_recurrent_kernels_read_gate_slices(T):
    qkv, _, a, b = fused(3, T, 10 + T)
    assert not a.is_contiguous() and not b.is_contiguous()
    q, k, v = qkv_heads(qkv)
    _, A_log, dt_bias, state = params(11)
    ac, bc = a.contiguous(), b.contiguous()
    y1, s1 = mx.gated_delta_update(q, k, v, a, b, A_log, dt_bias, state)
    y2, s2 = mx.gated_delta_update(q, k, v, ac, bc, A_log, dt_bias, state)
    assert torch.equal(y1, y2) and torch.equal(s1, s2)
    y1, _ = mx.gated_delta_verify(q, k, v, a, b, A_log, dt_bias, state)
    y2, _ = mx.gated_delta_verify(q, k, v, ac, bc, A_log, dt_bias, state)
    assert torch.equal(y1, y2)
    n = torch.tensor([0, T, (T + 1) // 2], dtype=torch.int32)
    assert torch.equal(mx.gated_delta_commit(k, v, a, b, A_log, dt_bias, state, n),
                       mx.gated_delta_commit(k, v, ac, bc, A_log, dt_bias, state, n))
    plan = mx.prepare_recurrent(q, k, v, a, b, A_log, dt_bias, state, write_state=False)
    plan.launch()
    torch.cuda.synchronize()
    assert torch.equal(plan.outputs[0], y2)


def test_decode_odd_gate_offsets_take_the_general_body():
    """One-token gates at odd element offsets and an odd row stride (2-byte
    aligned, so the lean decode body's dword reads of them are not taken):
    the general body gives the results of the lean one, bit for bit."""
    B = 3
    g = torch.Generator().manual_seed(21)
    buf = torch.randn(B, 1, 2 * Hv + 3, generator=g).to(torch.bfloat16).to(DEV)  # odd width
    a, b = buf[..., 1:1 + Hv], buf[..., 1 + Hv:1 + 2 * Hv]  # odd offsets
    assert a.data_ptr() % 4 == 2 and b.stride(1) % 2 == 1
    qkv, _, _, _ = fused(B, 1, 22)
    q, k, v = qkv_heads(qkv)
    _, A_log, dt_bias, state = params(23)
    y1, s1 = mx.gated_delta_update(q, k, v, a, b, A_log, dt_bias, state)
    y2, s2 = mx.gated_delta_update(q, k, v, a.contiguous(), b.contiguous(), A_log, dt_bias, state)
    assert torch.equal(y1, y2) and torch.equal(s1, s2)


def test_chunked_kernel_reads_gate_slices():
    T = 200
    qkv, _, a, b = fused(1, T, 20)
    q, k, v = qkv_heads(qkv)
    _, A_log, dt_bias, state = params(21)
    y1, s1 = mx.gated_delta_update(q, k, v, a, b, A_log, dt_bias, state[:1], chunked=True)
    y2, s2 = mx.gated_delta_update(q, k, v, a.contiguous(), b.contiguous(), A_log, dt_bias, state[:1], chunked=True)
    assert torch.equal(y1, y2) and torch.equal(s1, s2)


def test_mismatched_gate_strides_fall_back_to_copies():
    qkv, _, a, _ = fused(2, 3, 30)
    q, k, v = qkv_heads(qkv)
    _, A_log, dt_bias, state = params(31)
    b = torch.randn(2, 3, Hv, generator=torch.Generator().manual_seed(32)).to(torch.bfloat16).to(DEV)
    y1, s1 = mx.gated_delta_update(q, k, v, a, b, A_log, dt_bias, state[:2])
    y2, s2 = mx.gated_delta_update(q, k, v, a.contiguous(), b, A_log, dt_bias, state[:2])
    assert torch.equal(y1, y2) and torch.equal(s1, s2)
