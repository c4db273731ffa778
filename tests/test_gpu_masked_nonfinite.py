"""GPU checks that NaN and inf at masked positions stay out of every result.

The reference masks a step with where(mask, new, old): the state is kept and
nothing computed from the masked token's q, k, v, a or b survives (the
oracle's ``recurrent`` applies the same rule, and its y at a masked token is
0).  Padding in a batched prefill or a verify can hold anything, so each
path is run with NaN and +-inf written into q, k, v, a and b at every masked
position, against the oracle on the unmasked ones.

The decode, tile and commit kernels skip a masked step outright.  The
chunked pass and the verify kernels give a masked token g = 1 and beta = 0
and also store its k, q (and, in the scan, its R) as zeros, since beta = 0
alone would let 0 * inf through.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import multiplex_amd as mx
from gdn_cases import STATE_TOL, Y_TOL, draw, head_errs_state, row_errs_y, to_torch
from oracle import gdn

pytestmark = pytest.mark.gpu
DEV = "cuda"
BAD = (float("nan"), float("inf"), -float("inf"))


def _poisoned(seed, B, T, Hk, Hv, dtype="bf16", mask_p=0.3):
    d = draw(seed, B, T, Hk, Hv, 128, 128, mask_p=mask_p)
    d["mask"][0, 0] = False
    d["mask"][-1, -1] = False
    t, r = to_torch(d, DEV, dtype=dtype)
    m = torch.tensor(d["mask"], device=DEV)
    n_bad = int((~m).sum())
    for i, key in enumerate(("q", "k", "v", "a", "b")):
        bad = torch.tensor(BAD, device=DEV)[(torch.arange(n_bad, device=DEV) + i) % 3]
        shape = (n_bad,) + (1,) * (t[key].dim() - 2)
        t[key][~m] = bad.reshape(shape).to(t[key].dtype)
    t["mask"] = m
    return d, t, r


def _oracle(d, r, Hk, Hv, cu=None):
    g = gdn.compute_g(r["A_log"], r["a"], r["dt_bias"])
    rep = [h // (Hv // Hk) for h in range(Hv)]
    beta = gdn.compute_beta(r["b"])
    if cu is None:
        return gdn.recurrent(r["q"][:, :, rep], r["k"][:, :, rep], r["v"], g, beta, r["state"], d["mask"])
    return gdn.recurrent_varlen(r["q"][:, :, rep], r["k"][:, :, rep], r["v"], g, beta, cu, r["state"], d["mask"])


def _check(d, y, S, y_ref, S_ref):
    m = d["mask"]
    yn = y.float().cpu().numpy()
    assert np.isfinite(yn).all(), "a non-finite value at a masked position reached y"
    assert not yn[~m].any(), "a masked token's y is not 0"
    assert row_errs_y(yn[m][None], y_ref[m][None]).max() <= Y_TOL
    if S is not None:
        Sn = S.float().cpu().numpy()
        assert np.isfinite(Sn).all(), "a non-finite value at a masked position reached the state"
        assert head_errs_state(Sn, S_ref).max() <= STATE_TOL


@pytest.mark.parametrize("T,chunked", [(1, False), (8, False), (200, True)])
def test_update_paths(T, chunked):
    """Decode (T = 1), the tile kernel (T = 8) and the chunked pass."""
    d, t, r = _poisoned(600 + T, 2, T, 2, 4)
    y, S = mx.gated_delta_update(t["q"], t["k"], t["v"], t["a"], t["b"], t["A_log"], t["dt_bias"], t["state"],
                                 t["mask"], chunked=chunked)
    torch.cuda.synchronize()
    _check(d, y, S, *_oracle(d, r, 2, 4))


@pytest.mark.parametrize("B,packed", [(1, False), (2, False), (2, True)])
def test_chunked_scan_forms_at_full_width(B, packed):
    """Hv = 32: one row (the record's K^T), two equal rows (K^T from LDS, two
    tiles a workgroup) and two packed sequences (K^T from LDS, one tile)."""
    Hk, Hv, T = 16, 32, 160
    d, t, r = _poisoned(640 + B + packed, B, T, Hk, Hv)
    if packed:
        cu = np.array([0, 70, 2 * T], dtype=np.int32)
        flat = {k: (v.reshape(1, B * T, *v.shape[2:]) if k in ("q", "k", "v", "a", "b") else v) for k, v in t.items()}
        dr = dict(d, mask=d["mask"].reshape(1, B * T))
        rr = {k: (v.reshape(1, B * T, *v.shape[2:]) if k in ("q", "k", "v", "a", "b") else v) for k, v in r.items()}
        st = t["state"]  # one state per packed sequence (B of them)
        y, S = mx.gated_delta_update(flat["q"], flat["k"], flat["v"], flat["a"], flat["b"], t["A_log"], t["dt_bias"],
                                     st, t["mask"].reshape(1, B * T), cu_seqlens=cu.tolist(), chunked=True)
        torch.cuda.synchronize()
        _check(dr, y, S, *_oracle(dr, rr, Hk, Hv, cu=cu))
    else:
        y, S = mx.gated_delta_update(t["q"], t["k"], t["v"], t["a"], t["b"], t["A_log"], t["dt_bias"], t["state"],
                                     t["mask"], chunked=True)
        torch.cuda.synchronize()
        _check(d, y, S, *_oracle(d, r, Hk, Hv))


@pytest.mark.parametrize("dtype", ["bf16", "f32"])
def test_verify_and_commit(dtype):
    """Verify (bf16 at Dk = 128: the MFMA kernel; fp32: the WY kernel), then
    the commit of every token."""
    d, t, r = _poisoned(660 + (dtype == "f32"), 4, 4, 2, 4, dtype=dtype)
    y_ref, S_ref = _oracle(d, r, 2, 4)
    y, _ = mx.gated_delta_verify(t["q"], t["k"], t["v"], t["a"], t["b"], t["A_log"], t["dt_bias"], t["state"],
                                 t["mask"])
    S = mx.gated_delta_commit(t["k"], t["v"], t["a"], t["b"], t["A_log"], t["dt_bias"], t["state"], [4, 4, 4, 4],
                              t["mask"])
    torch.cuda.synchronize()
    _check(d, y, S, y_ref, S_ref)
