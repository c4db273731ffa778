"""The no-allocation chunked entry point (``gdn_chunk_fwd_noalloc``, records
in the library's static 64 MiB scratch array) against ``gdn_chunk_fwd``
with a caller's workspace, through the C ABI: two calls in a row, the second
smaller than the first (the array keeps the first call's records), both
bit-identical to the workspace call and within tolerance of the oracle."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from gdn_cases import STATE_TOL, Y_TOL, draw, head_errs_state, rel_err, to_torch
from multiplex_amd import _lib
from multiplex_amd.gated_delta import _chunk_args
from oracle import gdn

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _both(t, cu=None):
    lib = _lib.load()
    raw = _lib.GATES_RAW
    common = (t["q"], t["k"], t["v"], t["a"], t["b"], raw, t["A_log"], t["dt_bias"], t["state"])
    args, keep, y_ws, s_ws, _ = _chunk_args(*common, cu_seqlens=cu)
    assert lib.gdn_chunk_fwd(*args) == _lib.OK
    args2, keep2, y_na, s_na, _ = _chunk_args(*common, cu_seqlens=cu)
    # same arguments without (workspace, workspace_bytes)
    rc = lib.gdn_chunk_fwd_noalloc(*args2[:-3], args2[-1])
    assert rc == _lib.OK, lib.gdn_last_error()
    torch.cuda.synchronize()
    return y_ws, s_ws, y_na, s_na


def _oracle(r, heads, cu=None):
    hks = [h // 2 for h in heads]
    g = gdn.compute_g(r["A_log"][heads], r["a"][:, :, heads], r["dt_bias"][heads])
    beta = gdn.compute_beta(r["b"][:, :, heads])
    args = (r["q"][:, :, hks], r["k"][:, :, hks], r["v"][:, :, heads], g, beta)
    st = r["state"][:, heads]
    return gdn.recurrent(*args, st) if cu is None else gdn.recurrent_varlen(*args, cu, st)


def test_noalloc_matches_workspace_call_twice():
    heads = [0, 5, 31]
    # first call: one sequence of 1000 tokens (16 chunks), 43 MB of records
    d = draw(7001, 1, 1000, 16, 32, 128, 128)
    t, r = to_torch(d, DEV)
    y_ws, s_ws, y_na, s_na = _both(t)
    assert torch.equal(y_ws, y_na) and torch.equal(s_ws, s_na)
    y_ref, s_ref = _oracle(r, heads)
    assert rel_err(y_na[:, :, heads].float().cpu().numpy(), y_ref) <= Y_TOL
    assert head_errs_state(s_na[:, heads].cpu().numpy(), s_ref).max() <= STATE_TOL
    # second call, smaller: four packed sequences (one empty) with prefix states
    lens = [100, 37, 0, 200]
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    d = draw(7002, 1, int(cu[-1]), 16, 32, 128, 128, state=False)
    d["state"] = np.random.default_rng(7003).normal(0.0, 0.02, (4, 32, 128, 128))
    t, r = to_torch(d, DEV)
    y_ws, s_ws, y_na, s_na = _both(t, cu=torch.tensor(cu))
    assert torch.equal(y_ws, y_na) and torch.equal(s_ws, s_na)
    y_ref, s_ref = _oracle(r, heads, cu)
    assert rel_err(y_na[:, :, heads].float().cpu().numpy(), y_ref) <= Y_TOL
    assert head_errs_state(s_na[:, heads].cpu().numpy(), s_ref).max() <= STATE_TOL
