"""GPU parity of the benchmark workloads exactly as ``bench.py`` launches them.

* Prefill T=4096: the fused conv prologue over the full 8192-channel mixed
  projection feeds the chunked pass through its output buffers (prepared
  launches, as timed).  The prologue is checked against the oracle on the
  channels of a head subset (the conv is depthwise and the norm per head, so
  a channel subset is an exact sub-problem), and y / the final state against
  the oracle fed the prologue's own bf16 outputs.
* The mixed continuous-batching step: three packed prefills with prefix
  states, 48 decode rows and 16 verify rows with a ragged commit, issued as
  :class:`multiplex_amd.MixedStep` (prep, then scan; the recurrent launches
  on a second stream beside the scan).  Every output is checked against the
  oracle on head subsets and is bit-identical to the same launches issued on
  one stream.
* MTP verify at B=32, Hv=32, T=4 through the unrolled MFMA verify kernel.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

import multiplex_amd as mx
from gdn_cases import STATE_TOL, Y_TOL, draw, head_errs_state, rel_err, row_errs_y, to_torch
from oracle import gdn

pytestmark = pytest.mark.gpu
DEV = "cuda"
Hk, Hv, D = 16, 32, 128
C = 2 * Hk * D + Hv * D


def _np(t):
    return t.double().cpu().numpy()


def _channels(hks, heads):
    """Mixed-projection channels of k-heads ``hks`` (q then k) and v-heads ``heads``."""
    q = [np.arange(h * D, (h + 1) * D) for h in hks]
    k = [Hk * D + np.arange(h * D, (h + 1) * D) for h in hks]
    v = [2 * Hk * D + np.arange(h * D, (h + 1) * D) for h in heads]
    return np.concatenate(q + k + v)


def _gates(r, heads):
    g = gdn.compute_g(r["A_log"][heads], r["a"][:, :, heads], r["dt_bias"][heads])
    return g, gdn.compute_beta(r["b"][:, :, heads])


def test_prefill_t4096_prologue_feeds_chunked():
    T = 4096
    gen = torch.Generator().manual_seed(1003)
    qkv = torch.randn(1, T, C, generator=gen).to(torch.bfloat16)
    w = (torch.randn(C, 4, generator=gen) * 0.1).to(torch.bfloat16)
    a = torch.randn(1, T, Hv, generator=gen).to(torch.bfloat16)
    b = torch.randn(1, T, Hv, generator=gen).to(torch.bfloat16)
    A_log = torch.rand(Hv, generator=gen) * math.log(16.0)
    dt_bias = torch.rand(Hv, generator=gen) * 2 - 1
    cs = torch.zeros(1, 3, C, dtype=torch.bfloat16)
    dq, dw, da, db, dA, ddt, dcs = (x.to(DEV) for x in (qkv, w, a, b, A_log, dt_bias, cs))
    ws = torch.empty(mx.chunk_workspace_bytes(1, T, Hv, D, D), dtype=torch.uint8, device=DEV)
    pro = mx.prepare_conv_prologue(dq, dw, Hk, Hv, D, D, dcs)
    q, k, v, cs_out = pro.outputs
    chunk = mx.prepare_chunked(q, k, v, da, db, dA, ddt, None, workspace=ws)
    pro.launch()
    chunk.launch()
    torch.cuda.synchronize()
    y, S = chunk.outputs

    hks, heads = [0, 9, 15], [0, 1, 18, 19, 30, 31]
    ch = _channels(hks, heads)
    qr, kr, vr, csr, _ = gdn.conv_prologue(_np(qkv)[:, :, ch], _np(w)[ch], len(hks), len(heads), D, D, _np(cs)[:, :, ch])
    assert rel_err(q[:, :, hks].float().cpu().numpy(), qr) <= Y_TOL
    assert rel_err(k[:, :, hks].float().cpu().numpy(), kr) <= Y_TOL
    assert rel_err(v[:, :, heads].float().cpu().numpy(), vr) <= Y_TOL
    np.testing.assert_array_equal(cs_out.float().cpu().numpy()[:, :, ch], csr)

    r = dict(a=_np(a), b=_np(b), A_log=_np(A_log), dt_bias=_np(dt_bias))
    g, beta = _gates(r, heads)
    # v-head heads[j] reads k-head heads[j] // 2, i.e. sub-head j // 2
    y_ref, S_ref = gdn.recurrent(_np(q[:, :, hks]), _np(k[:, :, hks]), _np(v[:, :, heads]), g, beta, None)
    assert row_errs_y(y[:, :, heads].float().cpu().numpy(), y_ref).max() <= Y_TOL
    assert head_errs_state(S[:, heads].cpu().numpy(), S_ref).max() <= STATE_TOL


def _mixed_inputs():
    lens = [1024, 2560, 7168]
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    pf = draw(1004, 1, int(cu[-1]), Hk, Hv, D, D, state=False)
    pf["state"] = np.random.default_rng(14).normal(0.0, 0.02, (3, Hv, D, D))
    dec = draw(1014, 48, 1, Hk, Hv, D, D)
    ver = draw(1024, 16, 4, Hk, Hv, D, D)
    n_b = np.random.default_rng(34).integers(1, 5, 16).astype(np.int32)
    return cu, pf, dec, ver, n_b


def _build_step(cu, tp, td, tv, n_b):
    ws = torch.empty(mx.chunk_workspace_bytes(3, int(cu[-1]), Hv, D, D), dtype=torch.uint8, device=DEV)
    pplan = mx.prepare_chunked(tp["q"], tp["k"], tp["v"], tp["a"], tp["b"], tp["A_log"], tp["dt_bias"], tp["state"],
                               cu_seqlens=torch.tensor(cu), workspace=ws, state_out=torch.empty_like(tp["state"]))
    dplan = mx.prepare_recurrent(td["q"], td["k"], td["v"], td["a"], td["b"], td["A_log"], td["dt_bias"],
                                 td["state"], state_out=td["state"])
    vplan = mx.prepare_recurrent(tv["q"], tv["k"], tv["v"], tv["a"], tv["b"], tv["A_log"], tv["dt_bias"],
                                 tv["state"], write_state=False)
    cplan = mx.prepare_recurrent(None, tv["k"], tv["v"], tv["a"], tv["b"], tv["A_log"], tv["dt_bias"], tv["state"],
                                 y=False, commit_len=torch.tensor(n_b, device=DEV),
                                 state_out=torch.empty_like(tv["state"]))
    # the benchmark's order: verify and commit first, the decode last
    return mx.MixedStep(pplan, [vplan, cplan, dplan]), (pplan, dplan, vplan, cplan)


def _outputs(plans):
    pplan, dplan, vplan, cplan = plans
    return [pplan.outputs[0], pplan.outputs[1], dplan.outputs[0], dplan.outputs[1], vplan.outputs[0],
            cplan.outputs[1]]


def test_mixed_step_two_streams():
    cu, pf, dec, ver, n_b = _mixed_inputs()
    (tp, rp), (td, rd), (tv, rv) = (to_torch(x, DEV) for x in (pf, dec, ver))
    dec_state0 = td["state"].clone()
    step, plans = _build_step(cu, tp, td, tv, n_b)
    step.launch_overlapped()
    torch.cuda.synchronize()
    two = [t.clone() for t in _outputs(plans)]

    # the same launches on one stream, from the same initial states
    for t in _outputs(plans):
        t.zero_()
    td["state"].copy_(dec_state0)
    step.launch_serial()
    torch.cuda.synchronize()
    for a, b in zip(two, _outputs(plans)):
        assert torch.equal(a, b)

    y_pf, S_pf, y_dec, S_dec, y_ver, S_com = two
    heads = [3, 30]
    hks = [h // 2 for h in heads]
    g, beta = _gates(rp, heads)
    y_ref, S_ref = gdn.recurrent_varlen(rp["q"][:, :, hks], rp["k"][:, :, hks], rp["v"][:, :, heads], g, beta, cu,
                                        rp["state"][:, heads])
    for n in range(3):
        sl = slice(int(cu[n]), int(cu[n + 1]))
        assert rel_err(y_pf[:, sl][:, :, heads].float().cpu().numpy(), y_ref[:, sl]) <= Y_TOL
    assert head_errs_state(S_pf[:, heads].cpu().numpy(), S_ref).max() <= STATE_TOL

    heads = [0, 7, 8, 31]
    hks = [h // 2 for h in heads]
    g, beta = _gates(rd, heads)
    y_ref, S_ref = gdn.recurrent(rd["q"][:, :, hks], rd["k"][:, :, hks], rd["v"][:, :, heads], g, beta,
                                 rd["state"][:, heads])
    assert row_errs_y(y_dec[:, :, heads].float().cpu().numpy(), y_ref).max() <= Y_TOL
    assert head_errs_state(S_dec[:, heads].cpu().numpy(), S_ref).max() <= STATE_TOL

    g, beta = _gates(rv, heads)
    args = (rv["q"][:, :, hks], rv["k"][:, :, hks], rv["v"][:, :, heads], g, beta)
    y_ref, _ = gdn.recurrent(*args, rv["state"][:, heads])
    assert row_errs_y(y_ver[:, :, heads].float().cpu().numpy(), y_ref).max() <= Y_TOL
    S_ref = gdn.commit(*args, rv["state"][:, heads], n_b)
    assert head_errs_state(S_com[:, heads].cpu().numpy(), S_ref).max() <= STATE_TOL


def test_mixed_steps_in_a_row_overlapped_equal_serial():
    """Three overlapped steps back to back (the decode rows' states carried in
    place, the prep's ordering event reused each step) against three steps on
    one stream from the same initial states: bit-identical outputs."""
    cu, pf, dec, ver, n_b = _mixed_inputs()
    (tp, _), (td, _), (tv, _) = (to_torch(x, DEV) for x in (pf, dec, ver))
    dec_state0 = td["state"].clone()
    step, plans = _build_step(cu, tp, td, tv, n_b)
    for _ in range(3):
        step.launch_overlapped()
    torch.cuda.synchronize()
    two = [t.clone() for t in _outputs(plans)]
    for t in _outputs(plans):
        t.zero_()
    td["state"].copy_(dec_state0)
    for _ in range(3):
        step.launch_serial()
    torch.cuda.synchronize()
    for a, b in zip(two, _outputs(plans)):
        assert torch.equal(a, b)


def test_verify_b32_full_heads():
    """B=32, T=4, Hv=32 with no state write: the MFMA verify kernel, all heads."""
    d = draw(1002, 32, 4, Hk, Hv, D, D)
    t, r = to_torch(d, DEV)
    y, snaps = mx.gated_delta_verify(t["q"], t["k"], t["v"], t["a"], t["b"], t["A_log"], t["dt_bias"], t["state"])
    assert snaps is None
    g, beta = gdn.compute_g(r["A_log"], r["a"], r["dt_bias"]), gdn.compute_beta(r["b"])
    y_ref, _ = gdn.recurrent(r["q"], r["k"], r["v"], g, beta, r["state"])
    assert row_errs_y(y.float().cpu().numpy(), y_ref).max() <= Y_TOL


def test_commit_verify_one_pass_b32_full_heads():
    """The bench's one-pass round at B=32: the previous round's 4 drafts with
    ragged acceptance n_b ~ U{1..4} committed and the next 4 drafts verified
    in one launch of the stepping tile kernel, all heads against the oracle."""
    d = draw(1012, 32, 8, Hk, Hv, D, D)
    t, r = to_torch(d, DEV)
    n_b = np.random.default_rng(1013).integers(1, 5, 32)
    prev = tuple(t[n][:, :4].contiguous() for n in ("q", "k", "v", "a", "b"))
    new = tuple(t[n][:, 4:].contiguous() for n in ("q", "k", "v", "a", "b"))
    y, S = mx.gated_delta_commit_verify(prev, torch.tensor(n_b, dtype=torch.int32), *new, t["A_log"], t["dt_bias"],
                                        t["state"])
    g, beta = gdn.compute_g(r["A_log"], r["a"], r["dt_bias"]), gdn.compute_beta(r["b"])
    S_ref = gdn.commit(r["q"], r["k"], r["v"], g, beta, r["state"], n_b)
    assert head_errs_state(S.cpu().numpy(), S_ref).max() <= STATE_TOL
    keep = np.concatenate([np.arange(4)[None, :] < n_b[:, None], np.ones((32, 4), dtype=bool)], axis=1)
    y_ref, _ = gdn.recurrent(r["q"], r["k"], r["v"], g, beta, r["state"], keep)
    assert row_errs_y(y.float().cpu().numpy(), y_ref[:, 4:]).max() <= Y_TOL
