"""GPU checks of the mixer prefill with the conv prologue fused into the
chunked prep (``gdn_conv_chunked`` / ``gdn_chunk_fwd_conv``).

The fused prep forms q, k and v with the conv prologue's arithmetic, so y,
the state and the new conv state must equal ``gdn_conv_prologue`` followed
by ``gated_delta_update(..., chunked=True)`` bit for bit; that pair is
itself checked against the oracle in ``tests/test_gpu_configs.py`` and
``tests/test_gpu_prologue.py``.  Cases: the benchmark's T=4096 prefill at
full width (also against the oracle on head subsets), equal-length rows with
a partial last chunk, packed sequences with lengths below the conv window
(0, 1, 2 tokens) next to long ones, fp32 taps, GQA groups of 1 and 3, qkv
and gates read as column slices of one buffer, pooled states, and rows of
no tokens.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

import multiplex_amd as mx
from gdn_cases import STATE_TOL, Y_TOL, head_errs_state, rel_err, row_errs_y
from oracle import gdn

pytestmark = pytest.mark.gpu
DEV = "cuda"
D = 128


def _inputs(seed, B, S, Hk, Hv, *, cs=True, state=True, w_dtype=torch.bfloat16, n_seqs=None):
    gen = torch.Generator().manual_seed(seed)
    C = 2 * Hk * D + Hv * D
    n = B if n_seqs is None else n_seqs
    t = dict(
        qkv=torch.randn(B, S, C, generator=gen).to(torch.bfloat16),
        w=(torch.randn(C, 4, generator=gen) * 0.3).to(w_dtype),
        a=torch.randn(B, S, Hv, generator=gen).to(torch.bfloat16),
        b=torch.randn(B, S, Hv, generator=gen).to(torch.bfloat16),
        A_log=torch.rand(Hv, generator=gen) * math.log(16.0),
        dt_bias=torch.rand(Hv, generator=gen) * 2 - 1,
        cs=(torch.randn(n, 3, C, generator=gen) * 0.5).to(torch.bfloat16) if cs else None,
        state=(torch.randn(n, Hv, D, D, generator=gen) * 0.02) if state else None,
    )
    return {k: (None if v is None else v.to(DEV)) for k, v in t.items()}


def _unfused(t, Hk, Hv, cu=None, state_index=None, pool=None):
    q, k, v, cs = mx.gdn_conv_prologue(t["qkv"], t["w"], Hk, Hv, D, D, t["cs"], cu_seqlens=cu)
    st = pool if pool is not None else t["state"]
    y, s = mx.gated_delta_update(q, k, v, t["a"], t["b"], t["A_log"], t["dt_bias"], st, cu_seqlens=cu,
                                 chunked=True, state_index=state_index)
    return y, s, cs, (q, k, v)


def _fused(t, Hk, Hv, cu=None, state_index=None, pool=None):
    st = pool if pool is not None else t["state"]
    return mx.gdn_conv_chunked(t["qkv"], t["w"], Hk, Hv, D, D, t["a"], t["b"], t["A_log"], t["dt_bias"], st,
                               t["cs"], cu_seqlens=cu, state_index=state_index)


def _assert_equal(fused, unfused):
    y, s, cs = fused
    y2, s2, cs2 = unfused[:3]
    torch.cuda.synchronize()
    assert torch.equal(y, y2), "y differs from the unfused pair"
    assert torch.equal(s, s2), "state differs from the unfused pair"
    assert torch.equal(cs, cs2), "conv state differs from the unfused pair"


def _np(t):
    return t.detach().double().cpu().numpy()


def test_t4096_full_width_equals_unfused_and_oracle():
    Hk, Hv, T = 16, 32, 4096
    t = _inputs(2001, 1, T, Hk, Hv)
    fused = _fused(t, Hk, Hv)
    unfused = _unfused(t, Hk, Hv)
    _assert_equal(fused, unfused)
    # the oracle on a subset of heads, from the raw qkv
    hks, heads = [0, 15], [0, 1, 30, 31]
    ch = np.concatenate([np.arange(h * D, (h + 1) * D) for h in hks]
                        + [np.arange((Hk + h) * D, (Hk + h + 1) * D) for h in hks]
                        + [np.arange((2 * Hk + h) * D, (2 * Hk + h + 1) * D) for h in heads])
    qr, kr, vr, csr, _ = gdn.conv_prologue(_np(t["qkv"])[:, :, ch], _np(t["w"])[ch], len(hks), len(heads), D, D,
                                           _np(t["cs"])[:, :, ch])
    np.testing.assert_array_equal(fused[2].float().cpu().numpy()[:, :, ch], csr)
    g = gdn.compute_g(_np(t["A_log"])[heads], _np(t["a"])[:, :, heads], _np(t["dt_bias"])[heads])
    beta = gdn.compute_beta(_np(t["b"])[:, :, heads])
    # the kernel's bf16 q, k, v (bit-equal to the unfused prologue's) feed the recurrent oracle
    q, k, v = unfused[3]
    y_ref, s_ref = gdn.recurrent(_np(q[:, :, hks]), _np(k[:, :, hks]), _np(v[:, :, heads]), g, beta,
                                 _np(t["state"])[:, heads])
    assert rel_err(q[:, :, hks].float().cpu().numpy(), qr) <= Y_TOL
    assert rel_err(v[:, :, heads].float().cpu().numpy(), vr) <= Y_TOL
    assert row_errs_y(fused[0][:, :, heads].float().cpu().numpy(), y_ref).max() <= Y_TOL
    assert head_errs_state(fused[1][:, heads].cpu().numpy(), s_ref).max() <= STATE_TOL


@pytest.mark.parametrize("Hk,Hv,w_dtype", [(2, 4, torch.bfloat16), (2, 2, torch.float32), (1, 3, torch.bfloat16)])
def test_rows_with_a_partial_chunk_equal_unfused(Hk, Hv, w_dtype):
    t = _inputs(2002 + Hv, 2, 200, Hk, Hv, w_dtype=w_dtype)
    _assert_equal(_fused(t, Hk, Hv), _unfused(t, Hk, Hv))


@pytest.mark.parametrize("with_cs", [True, False])
def test_packed_short_and_empty_sequences_equal_unfused(with_cs):
    """Lengths 2, 0, 68, 130, 1, 3: conv windows reaching into the conv
    state, an empty sequence (its conv state passes through), chunk edges."""
    Hk, Hv = 2, 4
    lens = [2, 0, 68, 130, 1, 3]
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    t = _inputs(2010, 1, int(cu[-1]), Hk, Hv, cs=with_cs, n_seqs=len(lens))
    for cu_arg in (cu.tolist(), torch.tensor(cu, device=DEV)):
        _assert_equal(_fused(t, Hk, Hv, cu=cu_arg), _unfused(t, Hk, Hv, cu=cu_arg))


def test_column_slices_of_one_projection_buffer():
    """qkv, a and b as column slices of one fused in_proj output."""
    Hk, Hv, S = 2, 4, 150
    t = _inputs(2020, 2, S, Hk, Hv)
    C = t["qkv"].shape[-1]
    buf = torch.zeros(2, S, C + 64 + 2 * Hv, dtype=torch.bfloat16, device=DEV)
    buf[..., :C] = t["qkv"]
    buf[..., C + 64:C + 64 + Hv] = t["a"]
    buf[..., C + 64 + Hv:] = t["b"]
    sl = dict(t, qkv=buf[..., :C], a=buf[..., C + 64:C + 64 + Hv], b=buf[..., C + 64 + Hv:])
    _assert_equal(_fused(sl, Hk, Hv), _unfused(t, Hk, Hv))


def test_pooled_states_equal_unfused():
    Hk, Hv = 2, 4
    lens = [70, 5, 130]
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    t = _inputs(2030, 1, int(cu[-1]), Hk, Hv, n_seqs=len(lens))
    gen = torch.Generator().manual_seed(2031)
    pool = (torch.randn(6, Hv, D, D, generator=gen) * 0.02).to(DEV)
    idx = torch.tensor([4, 0, 2], dtype=torch.int32, device=DEV)
    p1, p2 = pool.clone(), pool.clone()
    y, _, cs = _fused(t, Hk, Hv, cu=cu.tolist(), state_index=idx, pool=p1)
    y2, _, cs2, _ = _unfused(t, Hk, Hv, cu=cu.tolist(), state_index=idx, pool=p2)
    torch.cuda.synchronize()
    assert torch.equal(y, y2) and torch.equal(cs, cs2)
    assert torch.equal(p1, p2)


def test_rows_of_no_tokens_pass_the_conv_state_through():
    Hk, Hv = 2, 4
    t = _inputs(2040, 3, 0, Hk, Hv)
    y, s, cs = _fused(t, Hk, Hv)
    torch.cuda.synchronize()
    assert y.shape == (3, 0, Hv, D)
    assert torch.equal(cs, t["cs"])
    assert torch.equal(s, t["state"])


def test_mixer_prefill_takes_the_fused_path_and_matches_unfused():
    """The mixer's chunked prefill (fused) against the same layer with the
    prologue launched on its own."""
    m = mx.GatedDeltaNet(256, 2, 4, D, D, device=DEV)
    m.reset_parameters(torch.Generator().manual_seed(2050))
    x = torch.randn(2, 100, 256, generator=torch.Generator().manual_seed(2051)).to(torch.bfloat16).to(DEV)
    with torch.no_grad():
        c1, c2 = mx.ArraysCache(), mx.ArraysCache()
        assert m._fused_prefill(m._project(x)[0], None)
        out1 = m(x, None, c1)
        fused = m._fused_prefill
        m._fused_prefill = lambda qkv, mask: False
        try:
            out2 = m(x, None, c2)
        finally:
            m._fused_prefill = fused
        torch.cuda.synchronize()
    assert torch.equal(out1, out2)
    assert torch.equal(c1[0], c2[0]) and torch.equal(c1[1], c2[1])
