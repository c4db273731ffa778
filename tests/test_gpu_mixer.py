"""GPU checks of the GatedDeltaNet mixer stand-in.

* forward (prefill then decode through the cache), decomposed at the
  library GEMMs: the mixer's own projections (the fused in_proj GEMM) feed
  the oracle's prologue, the kernels' q/k/v and gates feed the oracle's GDN
  update, and the oracle's y goes through the oracle's gated norm and a
  float64 out_proj.  The state is held to the contract's 1e-4, the prologue
  and the output to 2e-3.  (``mixer_forward``'s wiring itself is pinned to
  transformers' module in ``tests/test_oracle.py``.)
* verify + commit equals running only each row's accepted prefix.
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
HID, HK, HV, D = 256, 2, 4, 128


def make_mixer(seed):
    m = mx.GatedDeltaNet(HID, HK, HV, D, D, device=DEV)
    m.reset_parameters(torch.Generator().manual_seed(seed))
    p = {
        "in_proj_qkv": m.in_proj_qkv.weight, "in_proj_z": m.in_proj_z.weight, "in_proj_b": m.in_proj_b.weight,
        "in_proj_a": m.in_proj_a.weight, "conv1d": m.conv1d_weight, "A_log": m.A_log, "dt_bias": m.dt_bias,
        "norm": m.norm_weight, "out_proj": m.out_proj.weight,
    }
    return m, {k: v.detach().double().cpu().numpy() for k, v in p.items()}


def inputs(seed, B, S):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(B, S, HID, generator=g).to(torch.bfloat16)
    return x.to(DEV), x.double().numpy()


def _np(t):
    return t.double().cpu().numpy()


def _check_step(m, p, x, cs_before, state_before, out, cache):
    """One mixer call against the oracle, decomposed at the library GEMMs."""
    B, S = x.shape[:2]
    qkv, z, a, b = m._project(x)
    q, k, v, cs = mx.gdn_conv_prologue(qkv, m.conv1d_weight, HK, HV, D, D, cs_before)
    qr, kr, vr, csr, _ = gdn.conv_prologue(_np(qkv), p["conv1d"], HK, HV, D, D,
                                           None if cs_before is None else _np(cs_before))
    for got, ref in ((q, qr), (k, kr), (v, vr)):
        assert rel_err(got.float().cpu().numpy(), ref) <= Y_TOL
    np.testing.assert_array_equal(cache[0].float().cpu().numpy(), csr)
    y_ref, s_ref = gdn.gated_delta_update(_np(q), _np(k), _np(v), _np(a), _np(b), p["A_log"], p["dt_bias"],
                                          None if state_before is None else _np(state_before))
    assert head_errs_state(cache[1].cpu().numpy(), s_ref).max() <= STATE_TOL
    yn = gdn.gated_rms_norm(gdn.bf16_round(y_ref), _np(z), p["norm"], 1e-6, round_fn=gdn.bf16_round)
    o_ref = gdn.bf16_round(yn.reshape(B, S, -1) @ p["out_proj"].T)
    assert rel_err(out.float().cpu().numpy(), o_ref) <= Y_TOL


@torch.no_grad()
def test_forward_prefill_then_decode_matches_oracle():
    m, p = make_mixer(1)
    cache = mx.ArraysCache()
    x, _ = inputs(2, 2, 7)
    out = m(x, None, cache)
    _check_step(m, p, x, None, None, out, cache)
    for step, seed in enumerate((3, 4)):
        cs0, s0 = cache[0].clone(), cache[1].clone()
        x2, _ = inputs(seed, 2, 1 if step == 0 else 70)
        out2 = m(x2, None, cache)
        _check_step(m, p, x2, cs0, s0, out2, cache)


@torch.no_grad()
def test_verify_then_commit_equals_accepted_prefix():
    m, _ = make_mixer(4)
    B, T = 4, 4
    base = mx.ArraysCache()
    x0, _ = inputs(5, B, 6)
    m(x0, None, base)
    xv, _ = inputs(6, B, T)
    n = [0, 1, 3, 4]
    # verify: outputs for all T tokens, cache untouched
    cache = base.clone()
    before = [v.clone() for v in cache.cache]
    out_v = m(xv, None, cache, verify=True)
    assert all(torch.equal(a, b) for a, b in zip(cache.cache, before))
    ref_all = base.clone()
    out_f = m(xv, None, ref_all)
    # verify runs the unrolled verify kernel, the forward steps the state:
    # the same outputs up to fp32 rounding order, then bf16 and the GEMM
    assert rel_err(out_v.float().cpu().numpy(), out_f.float().cpu().numpy()) <= 2e-3
    # commit the ragged accepted prefixes in one pass
    m.commit(cache, torch.tensor(n, dtype=torch.int32))
    for b in range(B):
        row = base.extract(b)
        if n[b] > 0:
            m(xv[b:b + 1, : n[b]], None, row)
        # the row-alone projections may round differently from the batched
        # GEMM, so compare within bf16 / fp32-state tolerances (an off-by-one
        # commit would differ by O(1))
        assert rel_err(cache[0][b].float().cpu().numpy(), row[0][0].float().cpu().numpy()) <= 1e-2, f"conv row {b}"
        assert rel_err(cache[1][b].cpu().numpy(), row[1][0].cpu().numpy()) <= STATE_TOL, f"state row {b}"


@torch.no_grad()
def test_merged_batch_equals_rows():
    m, _ = make_mixer(7)
    rows = []
    for r in range(3):
        c = mx.ArraysCache()
        x, _ = inputs(10 + r, 1, 3 + r)
        m(x, None, c)
        rows.append(c)
    merged = mx.merge_layer(rows)
    x, _ = inputs(20, 3, 1)
    out = m(x, None, merged)
    for r in range(3):
        o = m(x[r:r + 1], None, rows[r])
        assert rel_err(out[r].float().cpu().numpy(), o[0].float().cpu().numpy()) < 1e-2
        assert rel_err(merged[1][r].cpu().numpy(), rows[r][1][0].cpu().numpy()) <= STATE_TOL
