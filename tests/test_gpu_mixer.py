"""GPU checks of the GatedDeltaNet mixer stand-in.

* forward (prefill then decode through the cache) against the float64 mixer
  restatement with bf16 rounding at the same materialisation points;
* verify + commit equals running only each row's accepted prefix.

Tolerances: the GDN contract's 1e-4 (state) applies to the recurrent state;
the mixer output also passes through library bf16 GEMMs whose accumulation
order differs from numpy's, so it is held to 1e-2 norm-wise.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import multiplex_amd as mx
from gdn_cases import STATE_TOL, head_errs_state, rel_err
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


@torch.no_grad()
def test_forward_prefill_then_decode_matches_oracle():
    m, p = make_mixer(1)
    cache = mx.ArraysCache()
    x, xr = inputs(2, 2, 7)
    out = m(x, None, cache)
    o_ref, cs_ref, s_ref = gdn.mixer_forward(p, xr, HK, HV, D, D)
    assert rel_err(out.float().cpu().numpy(), o_ref) < 1e-2
    np.testing.assert_allclose(cache[0].float().cpu().numpy(), cs_ref, rtol=1e-2, atol=1e-2)
    assert head_errs_state(cache[1].cpu().numpy(), s_ref).max() <= 5 * STATE_TOL
    x2, xr2 = inputs(3, 2, 1)
    out2 = m(x2, None, cache)
    o_ref2, _, s_ref2 = gdn.mixer_forward(p, xr2, HK, HV, D, D, conv_state=cs_ref, state=s_ref)
    assert rel_err(out2.float().cpu().numpy(), o_ref2) < 1e-2
    assert head_errs_state(cache[1].cpu().numpy(), s_ref2).max() <= 5 * STATE_TOL


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
