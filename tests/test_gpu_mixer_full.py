"""The GatedDeltaNet mixer at the width the benchmark runs it: hidden 2048,
16 k-heads and 32 v-heads of 128 dims, as ``bench_mixer_layer`` calls it --
a pooled B=64 decode step (states updated in their pool slots) and a
T=4096 prefill on the chunked kernel.

The per-kernel tests check every kernel at full size; what these add is the
full-width wiring: the fused in_proj output read in place as column slices
(q|k|v at 8192 channels, z at 4096, b and a at 32), the strides the
prologue, the GDN kernel and the norm take from it, and the pool slots.
The decode step runs at B=64 (the separate norm kernel and the library
out_proj) and at B=8 (the norm fused into out_proj's operand load).
Each call is decomposed at the library GEMMs:

* the prologue's q, k, v from the mixer's own projection against the
  oracle on all 8192 channels (2e-3) and the conv state bit for bit;
* the GDN update: the kernel's y and state against the float64 oracle on a
  subset of heads (2e-3 and 1e-4), from the same q, k, v and gates;
* the epilogue: the mixer's output against a float64 gated RMSNorm and
  out_proj of the kernel's y (2e-3), which fixes the norm's head layout
  and the out_proj input order.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import multiplex_amd as mx
from gdn_cases import STATE_TOL, Y_TOL, head_errs_state, rel_err
from oracle import gdn

pytestmark = pytest.mark.gpu
DEV = "cuda"
HID, HK, HV, D = 2048, 16, 32, 128
HEADS = [0, 1, 17, 30, 31]  # v-heads checked against the oracle (k-heads 0, 8, 15)


def _np(t):
    return t.detach().double().cpu().numpy()


def _mixer(seed):
    m = mx.GatedDeltaNet(HID, HK, HV, D, D, device=DEV)
    m.reset_parameters(torch.Generator().manual_seed(seed))
    with torch.no_grad():
        m.norm_weight.copy_((torch.randn(D, generator=torch.Generator().manual_seed(seed + 1)) * 0.2 + 1.0))
    return m


def _check(m, x, cs_before, s_before, out, s_after, cs_after):
    """The decomposition described in the module docstring."""
    B, S = x.shape[:2]
    qkv, z, a, b = m._project(x)
    q, k, v, _ = mx.gdn_conv_prologue(qkv, m.conv1d_weight, HK, HV, D, D, cs_before)
    qr, kr, vr, csr, _ = gdn.conv_prologue(_np(qkv), _np(m.conv1d_weight), HK, HV, D, D,
                                           None if cs_before is None else _np(cs_before))
    for got, ref in ((q, qr), (k, kr), (v, vr)):
        assert rel_err(got.float().cpu().numpy(), ref) <= Y_TOL
    np.testing.assert_array_equal(cs_after.float().cpu().numpy(), csr)
    # the GDN kernel on the same inputs (the mixer ran the same kernel)
    y_dev, _ = mx.gated_delta_update(q, k, v, a, b, m.A_log, m.dt_bias, s_before)
    grp = HV // HK
    hk = [h // grp for h in HEADS]
    g = gdn.compute_g(_np(m.A_log)[HEADS], _np(a)[:, :, HEADS], _np(m.dt_bias)[HEADS])
    beta = gdn.compute_beta(_np(b)[:, :, HEADS])
    y_ref, s_ref = gdn.recurrent(_np(q)[:, :, hk], _np(k)[:, :, hk], _np(v)[:, :, HEADS], g, beta,
                                 None if s_before is None else _np(s_before)[:, HEADS])
    assert rel_err(y_dev[:, :, HEADS].float().cpu().numpy(), y_ref) <= Y_TOL
    assert head_errs_state(s_after[:, HEADS].cpu().numpy(), s_ref).max() <= STATE_TOL
    # epilogue wiring: gated RMSNorm per v-head, then out_proj over [Hv*Dv]
    yn = gdn.gated_rms_norm(_np(y_dev), _np(z), _np(m.norm_weight), m.rms_norm_eps, round_fn=gdn.bf16_round)
    o_ref = gdn.bf16_round(yn.reshape(B, S, HV * D) @ _np(m.out_proj.weight).T)
    assert rel_err(out.float().cpu().numpy(), o_ref) <= Y_TOL


@pytest.mark.parametrize("B", [64, 8])
@torch.no_grad()
def test_full_width_pooled_decode(B):
    m = _mixer(81)
    gen = torch.Generator().manual_seed(82 + B)
    pool = mx.StatePool(80, HV, D, D, device=DEV)
    cache = mx.ArraysCache()
    batch = mx.PooledBatch.new(pool, B)  # zeroes its slots: nonzero states are set after
    pool.states.copy_(torch.randn(pool.states.shape, generator=gen) * 0.02)
    cache[1] = batch
    cache[0] = (torch.randn(B, 3, m.conv_dim, generator=gen) * 0.5).to(torch.bfloat16).to(DEV)
    x = torch.randn(B, 1, HID, generator=gen).to(torch.bfloat16).to(DEV)
    cs_before = cache[0].clone()
    slots = batch.index.long()
    s_before = pool.states.index_select(0, slots).clone()
    out = m(x, None, cache)
    s_after = pool.states.index_select(0, slots)
    _check(m, x, cs_before, s_before, out, s_after, cache[0])


@torch.no_grad()
def test_full_width_prefill_t4096_chunked():
    m = _mixer(83)
    gen = torch.Generator().manual_seed(84)
    x = torch.randn(1, 4096, HID, generator=gen).to(torch.bfloat16).to(DEV)
    cache = mx.ArraysCache()
    out = m(x, None, cache)
    _check(m, x, None, None, out, cache[1], cache[0])
