"""GPU parity of the chunked (WY/UT, bf16 MFMA) prefill kernel.

Against the float64 oracle on subsets of heads (heads are independent, so a
head subset of the full-size problem is an exact sub-problem), and against
the recurrent HIP kernel at full size.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import multiplex_amd as mx
from gdn_cases import STATE_TOL, Y_TOL, draw, head_errs_state, rel_err, row_errs_y, to_torch
from oracle import gdn

pytestmark = pytest.mark.gpu
DEV = "cuda"


def chunked(t, state, cu=None):
    return mx.gated_delta_update(t["q"], t["k"], t["v"], t["a"], t["b"], t["A_log"], t["dt_bias"], state,
                                 cu_seqlens=cu, chunked=True)


def oracle_heads(r, heads, Hv, Hk, state, cu=None):
    """Oracle on v-heads ``heads`` only (q/k heads h // (Hv/Hk) selected per v-head)."""
    grp = Hv // Hk
    hk = [h // grp for h in heads]
    g = gdn.compute_g(r["A_log"][heads], r["a"][:, :, heads], r["dt_bias"][heads])
    beta = gdn.compute_beta(r["b"][:, :, heads])
    st = None if state is None else state[:, heads]
    args = (r["q"][:, :, hk], r["k"][:, :, hk], r["v"][:, :, heads], g, beta)
    if cu is None:
        return gdn.recurrent(*args, st)
    return gdn.recurrent_varlen(*args, cu, st)


@pytest.mark.parametrize("T", [1, 37, 64, 65, 200])
def test_short_sequences_match_oracle(T):
    d = draw(300 + T, 2, T, 2, 4, 128, 128)
    t, r = to_torch(d, DEV)
    y, S = chunked(t, t["state"])
    y_ref, S_ref = oracle_heads(r, [0, 1, 2, 3], 4, 2, r["state"])
    assert row_errs_y(y.float().cpu().numpy(), y_ref).max() <= Y_TOL
    assert head_errs_state(S.cpu().numpy(), S_ref).max() <= STATE_TOL


@pytest.mark.parametrize("B,Hk,Hv", [(2, 4, 4), (2, 2, 6), (2, 1, 4), (3, 12, 12), (3, 4, 12), (3, 3, 12)])
def test_gqa_groups_match_oracle(B, Hk, Hv):
    """GQA groups of 1, 3 and 4 v-heads per k-head (the other tests use 2).
    The scan deals whole groups to an XCD and the prep writes a k-head's K, Q
    and K^T records once per group; B=3 with Hv=12 is 288 scan tiles, so K^T
    then comes from transposed LDS reads and each scan workgroup holds two
    16-row tiles."""
    d = draw(320 + 16 * B + Hk + Hv, B, 150, Hk, Hv, 128, 128)
    t, r = to_torch(d, DEV)
    y, S = chunked(t, t["state"])
    y_ref, S_ref = oracle_heads(r, list(range(Hv)), Hv, Hk, r["state"])
    assert row_errs_y(y.float().cpu().numpy(), y_ref).max() <= Y_TOL
    assert head_errs_state(S.cpu().numpy(), S_ref).max() <= STATE_TOL


def test_prefill_4096_full_heads_subset_oracle():
    # One long sequence at the prefill shape: B=1, T=4096, Hk=16, Hv=32, zero state.
    d = draw(1003, 1, 4096, 16, 32, 128, 128, state=False)
    t, r = to_torch(d, DEV)
    y, S = chunked(t, None)
    heads = [0, 1, 17, 31]
    y_ref, S_ref = oracle_heads(r, heads, 32, 16, None)
    yh = y[:, :, heads].float().cpu().numpy()
    assert row_errs_y(yh, y_ref).max() <= Y_TOL
    assert head_errs_state(S[:, heads].cpu().numpy(), S_ref).max() <= STATE_TOL
    # all heads: chunked vs the recurrent kernel (two different algorithms)
    y2, S2 = mx.gated_delta_update(t["q"], t["k"], t["v"], t["a"], t["b"], t["A_log"], t["dt_bias"], None,
                                   chunked=False)
    assert row_errs_y(y.float().cpu().numpy(), y2.float().cpu().numpy()).max() <= Y_TOL
    assert head_errs_state(S.cpu().numpy(), S2.cpu().numpy()).max() <= STATE_TOL


def test_packed_prefills_with_prefix_states():
    lens = [1024, 2560, 7168]
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    d = draw(1004, 1, int(cu[-1]), 16, 32, 128, 128, state=False)
    t, r = to_torch(d, DEV)
    S0 = np.random.default_rng(4).normal(0, 0.02, (3, 32, 128, 128)).astype(np.float32)
    y, S = chunked(t, torch.tensor(S0, device=DEV), cu=torch.tensor(cu))
    heads = [3, 30]
    y_ref, S_ref = oracle_heads(r, heads, 32, 16, S0.astype(np.float64), cu=cu)
    for n in range(3):
        sl = slice(int(cu[n]), int(cu[n + 1]))
        assert rel_err(y[:, sl][:, :, heads].float().cpu().numpy(), y_ref[:, sl]) <= Y_TOL
    assert head_errs_state(S[:, heads].cpu().numpy(), S_ref).max() <= STATE_TOL


@pytest.mark.parametrize("Hk,Hv", [(2, 4), (2, 6), (3, 12)])
def test_ragged_packed_small(Hk, Hv):
    """Five packed sequences (one empty, one of a single token); GQA groups 2,
    3 and 4 (Hv=12: 480 scan workgroups, K^T from transposed LDS reads)."""
    lens = [70, 0, 1, 128, 63]
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    d = draw(305 + Hv, 1, int(cu[-1]), Hk, Hv, 128, 128, state=False)
    t, r = to_torch(d, DEV)
    S0 = np.random.default_rng(6).normal(0, 0.02, (len(lens), Hv, 128, 128)).astype(np.float32)
    y, S = chunked(t, torch.tensor(S0, device=DEV), cu=cu)
    y_ref, S_ref = oracle_heads(r, list(range(Hv)), Hv, Hk, S0.astype(np.float64), cu=cu)
    assert rel_err(y.float().cpu().numpy(), y_ref) <= Y_TOL
    assert head_errs_state(S.cpu().numpy(), S_ref).max() <= STATE_TOL
    np.testing.assert_array_equal(S[1].cpu().numpy(), S0[1])


def test_many_ragged_packed_sequences():
    """96 packed sequences of 0-200 tokens: the prep's extra workgroup orders
    them longest first for the scan, and each sequence's chunk slots start at
    cu[n] / 64 + n; against the oracle."""
    lens = np.random.default_rng(11).integers(0, 201, 96)
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    d = draw(331, 1, int(cu[-1]), 1, 2, 128, 128, state=False)
    t, r = to_torch(d, DEV)
    S0 = np.random.default_rng(12).normal(0, 0.02, (len(lens), 2, 128, 128)).astype(np.float32)
    y, S = chunked(t, torch.tensor(S0, device=DEV), cu=cu)
    y_ref, S_ref = oracle_heads(r, [0, 1], 2, 1, S0.astype(np.float64), cu=cu)
    assert rel_err(y.float().cpu().numpy(), y_ref) <= Y_TOL
    assert head_errs_state(S.cpu().numpy(), S_ref).max() <= STATE_TOL


def test_packed_beyond_ordering_limit_matches_unpacked():
    """1100 packed sequences (above the 1024 that are ordered by length, so in
    sequence order) against the same rows unpacked: bit-identical."""
    n, L = 1100, 3
    d = draw(332, n, L, 1, 2, 128, 128)
    t, _ = to_torch(d, DEV)
    y_u, S_u = chunked(t, t["state"])
    flat = {k: (v.reshape(1, n * L, *v.shape[2:]) if k in ("q", "k", "v", "a", "b") else v) for k, v in t.items()}
    y_p, S_p = chunked(flat, t["state"], cu=torch.arange(0, n * L + 1, L, dtype=torch.int32))
    assert torch.equal(y_p.reshape(y_u.shape), y_u) and torch.equal(S_p, S_u)


def test_strong_decay_is_finite_and_exact():
    d = draw(306, 1, 256, 2, 4, 128, 128)
    d["a"][:] = 4.0
    d["A_log"][:] = np.log(15.0)
    t, r = to_torch(d, DEV)
    y, S = chunked(t, t["state"])
    assert torch.isfinite(y.float()).all() and torch.isfinite(S).all()
    y_ref, S_ref = oracle_heads(r, [0, 1, 2, 3], 4, 2, r["state"])
    assert row_errs_y(y.float().cpu().numpy(), y_ref).max() <= Y_TOL
    assert head_errs_state(S.cpu().numpy(), S_ref).max() <= STATE_TOL


@pytest.mark.parametrize("B,Hk,Hv,T,heads", [(1, 2, 4, 300, [0, 1, 2, 3]), (2, 16, 32, 200, [0, 1, 17, 31])])
def test_mixed_decays_within_chunks_match_oracle(B, Hk, Hv, T, heads):
    """Tokens alternate between almost no decay (g near 1) and strong decay
    (g near e^-60) and A_log spans its range over the heads, so inside one
    chunk the factors e^(L_t - L_i) run from 1 down to underflow while |L|
    grows large: the prep's fp64 prefix sums, its decays and the triangular
    inverse, with one scan workgroup per CU (B=1) and several (B=2, Hv=32)."""
    d = draw(315 + B, B, T, Hk, Hv, 128, 128)
    d["a"][:, 0::2] = -6.0
    d["a"][:, 1::2] = 4.0
    d["a"][:, 5::7] = 1.0
    d["A_log"][:] = np.linspace(0.0, np.log(15.0), Hv)
    t, r = to_torch(d, DEV)
    y, S = chunked(t, t["state"])
    assert torch.isfinite(y.float()).all() and torch.isfinite(S).all()
    y_ref, S_ref = oracle_heads(r, heads, Hv, Hk, r["state"])
    assert row_errs_y(y[:, :, heads].float().cpu().numpy(), y_ref).max() <= Y_TOL
    assert head_errs_state(S[:, heads].cpu().numpy(), S_ref).max() <= STATE_TOL


def test_in_place_state():
    d = draw(307, 2, 100, 2, 4, 128, 128)
    t, _ = to_torch(d, DEV)
    y1, S1 = chunked(t, t["state"])
    st = t["state"].clone()
    y2, S2 = mx.gated_delta_update(t["q"], t["k"], t["v"], t["a"], t["b"], t["A_log"], t["dt_bias"], st,
                                   state_out=st, chunked=True)
    assert S2.data_ptr() == st.data_ptr()
    assert torch.equal(S2, S1) and torch.equal(y2, y1)


def test_prepared_launch_equals_call():
    d = draw(308, 1, 300, 2, 4, 128, 128)
    t, _ = to_torch(d, DEV)
    cu = torch.tensor([0, 70, 70, 300], dtype=torch.int32)
    st = torch.tensor(np.random.default_rng(9).normal(0.0, 0.02, (3, 4, 128, 128)), dtype=torch.float32,
                      device=DEV)
    y_ref, S_ref = chunked(t, st, cu=cu)
    plan = mx.prepare_chunked(t["q"], t["k"], t["v"], t["a"], t["b"], t["A_log"], t["dt_bias"], st,
                              cu_seqlens=cu)
    for _ in range(2):  # re-issued launches recompute the same outputs
        plan.launch()
        y, S = plan.outputs
        assert torch.equal(y, y_ref) and torch.equal(S, S_ref)


def test_kt_sources_agree_bitwise():
    """With more scan tiles than CUs the scan forms K^T by transposed LDS
    reads of K and (for rows of one length) puts two 16-row tiles in each
    workgroup; with at most one tile per CU it reads the record's K^T, one
    tile per workgroup.  Two Hv=32 sequences in one call (512 tiles) against
    each alone (256): the transposes are exact and each tile's products run
    in the same order, so the results are bit-identical."""
    d = draw(309, 2, 200, 16, 32, 128, 128)
    t, _ = to_torch(d, DEV)
    y2, S2 = chunked(t, t["state"])
    for b in range(2):
        one = {k: (v[b:b + 1] if k in ("q", "k", "v", "a", "b", "state") else v) for k, v in t.items()}
        y1, S1 = chunked(one, one["state"])
        assert torch.equal(y1[0], y2[b]), f"row {b}: y"
        assert torch.equal(S1[0], S2[b]), f"row {b}: state"


def test_two_tile_workgroups_b4_match_oracle():
    """B=4 rows of 130 tokens at Hv=32 (1024 tiles, two per workgroup, two
    workgroups per CU), a partial last chunk and nonzero initial states:
    6 heads against the oracle."""
    d = draw(311, 4, 130, 16, 32, 128, 128)
    t, r = to_torch(d, DEV)
    y, S = chunked(t, t["state"])
    heads = [0, 1, 13, 14, 30, 31]
    y_ref, S_ref = oracle_heads(r, heads, 32, 16, r["state"])
    assert row_errs_y(y[:, :, heads].float().cpu().numpy(), y_ref).max() <= Y_TOL
    assert head_errs_state(S[:, heads].cpu().numpy(), S_ref).max() <= STATE_TOL


@pytest.mark.parametrize("gate_dtype,param_dtype", [("f32", "f32"), ("f16", "bf16"), ("bf16", "f16")])
def test_runtime_typed_gates(gate_dtype, param_dtype):
    """a / b and A_log / dt_bias in other dtypes than the bf16 / fp32 pair
    (runtime-typed gate loads), against the oracle."""
    d = draw(310, 2, 150, 2, 4, 128, 128)
    t, r = to_torch(d, DEV, gate_dtype=gate_dtype, param_dtype=param_dtype)
    y, S = chunked(t, t["state"])
    y_ref, S_ref = oracle_heads(r, [0, 1, 2, 3], 4, 2, r["state"])
    assert row_errs_y(y.float().cpu().numpy(), y_ref).max() <= Y_TOL
    assert head_errs_state(S.cpu().numpy(), S_ref).max() <= STATE_TOL


def test_precomputed_gates():
    """g and beta given (fp32), through a prepared chunked launch."""
    d = draw(311, 2, 150, 2, 4, 128, 128)
    t, r = to_torch(d, DEV)
    g = mx.compute_g(t["A_log"], t["a"], t["dt_bias"]).float()
    beta = mx.compute_beta(t["b"]).float()
    plan = mx.prepare_chunked(t["q"], t["k"], t["v"], g, beta, None, None, t["state"], gates_precomputed=True)
    plan.launch()
    y, S = plan.outputs
    y_ref, S_ref = oracle_heads(r, [0, 1, 2, 3], 4, 2, r["state"])
    assert row_errs_y(y.float().cpu().numpy(), y_ref).max() <= Y_TOL
    assert head_errs_state(S.cpu().numpy(), S_ref).max() <= STATE_TOL


def test_prep_and_scan_launched_apart():
    """The two phases enqueued separately (the scan on another stream, after
    an event) equal the one-call launch bit for bit."""
    d = draw(312, 1, 300, 2, 4, 128, 128)
    t, _ = to_torch(d, DEV)
    cu = torch.tensor([0, 70, 70, 300], dtype=torch.int32)
    st = torch.tensor(np.random.default_rng(10).normal(0.0, 0.02, (3, 4, 128, 128)), dtype=torch.float32,
                      device=DEV)
    y_ref, S_ref = chunked(t, st, cu=cu)
    plan = mx.prepare_chunked(t["q"], t["k"], t["v"], t["a"], t["b"], t["A_log"], t["dt_bias"], st,
                              cu_seqlens=cu)
    main, side = torch.cuda.current_stream(), torch.cuda.Stream()
    done = torch.cuda.Event()
    plan.launch_prep(main)
    done.record(main)
    side.wait_event(done)
    plan.launch_scan(side)
    main.wait_stream(side)
    torch.cuda.synchronize()
    y, S = plan.outputs
    assert torch.equal(y, y_ref) and torch.equal(S, S_ref)


def test_device_offsets_need_max_seqlen_to_pick_a_kernel():
    """One 500-token prompt packed with nine short ones (mean 51 tokens):
    a device ``cu_seqlens`` is never read back, so without ``max_seqlen``
    the call refuses to guess the kernel (the mean would step the long
    prompt through the recurrent kernel); with it, the chunked kernel runs,
    bit for bit as when forced."""
    lens = [500, 3, 5, 1, 1, 1, 1, 1, 1, 1]
    cu = torch.tensor(np.concatenate([[0], np.cumsum(lens)]), dtype=torch.int32, device=DEV)
    d = draw(313, 1, int(sum(lens)), 2, 4, 128, 128, state=False)
    t, r = to_torch(d, DEV)
    args = (t["q"], t["k"], t["v"], t["a"], t["b"], t["A_log"], t["dt_bias"], None)
    with pytest.raises(ValueError, match="max_seqlen"):
        mx.gated_delta_update(*args, cu_seqlens=cu)
    y, S = mx.gated_delta_update(*args, cu_seqlens=cu, max_seqlen=max(lens))
    y_c, S_c = chunked(t, None, cu=cu)
    assert torch.equal(y, y_c) and torch.equal(S, S_c)
    y_ref, S_ref = oracle_heads(r, [0, 1, 2, 3], 4, 2, None, cu=cu.cpu().numpy())
    assert rel_err(y.float().cpu().numpy(), y_ref) <= Y_TOL
    assert head_errs_state(S.cpu().numpy(), S_ref).max() <= STATE_TOL


def _masked(seed, B, T, kind, Hk=2, Hv=4):
    d = draw(seed, B, T, Hk, Hv, 128, 128, mask_p=0.25 if kind == "random" else None)
    if kind == "left_pad":  # batched prefills pad their rows on the left
        m = np.ones((B, T), dtype=bool)
        for b in range(B):
            m[b, : (37 * (b + 1)) % T] = False
        d["mask"] = m
    elif kind == "whole_rows":  # row 0 masked throughout, row 1 not at all
        m = np.ones((B, T), dtype=bool)
        m[0] = False
        d["mask"] = m
    return d


@pytest.mark.parametrize("T,kind", [(200, "random"), (130, "left_pad"), (64, "whole_rows"), (1, "random")])
def test_masked_rows_match_oracle(T, kind):
    """A masked token keeps the state and its y is 0 (the oracle's and the
    recurrent kernel's rule): random masks, left padding and whole rows."""
    d = _masked(910 + T, 2, T, kind)
    t, r = to_torch(d, DEV)
    y, S = mx.gated_delta_update(t["q"], t["k"], t["v"], t["a"], t["b"], t["A_log"], t["dt_bias"], t["state"],
                                 t["mask"], chunked=True)
    g = gdn.compute_g(r["A_log"], r["a"], r["dt_bias"])
    y_ref, S_ref = gdn.recurrent(r["q"][:, :, [0, 0, 1, 1]], r["k"][:, :, [0, 0, 1, 1]], r["v"], g,
                                 gdn.compute_beta(r["b"]), r["state"], r["mask"])
    yn = y.float().cpu().numpy()
    assert head_errs_state(S.cpu().numpy(), S_ref).max() <= STATE_TOL
    on = r["mask"].any(axis=1)
    if on.any():
        assert row_errs_y(yn[on], y_ref[on]).max() <= Y_TOL
    assert not yn[~r["mask"]].any(), "a masked token's y is not 0"
    if kind == "whole_rows":
        assert torch.equal(S[0], t["state"][0])
    # the recurrent kernel, which steps the same rule
    y2, S2 = mx.gated_delta_update(t["q"], t["k"], t["v"], t["a"], t["b"], t["A_log"], t["dt_bias"], t["state"],
                                   t["mask"], chunked=False)
    assert head_errs_state(S.cpu().numpy(), S2.cpu().numpy()).max() <= STATE_TOL
    if on.any():
        assert row_errs_y(yn[on], y2.float().cpu().numpy()[on]).max() <= Y_TOL


@pytest.mark.parametrize("kind", ["random", "left_pad"])
def test_masked_rows_at_full_width_match_oracle(kind):
    """Masks where the scan's tiles outnumber the CUs (B=2 at Hv=32: K^T
    from LDS, two 16-row tiles a workgroup): four heads against the oracle,
    masked tokens' y exactly 0."""
    d = _masked(940, 2, 200, kind, Hk=16, Hv=32)
    t, r = to_torch(d, DEV)
    y, S = mx.gated_delta_update(t["q"], t["k"], t["v"], t["a"], t["b"], t["A_log"], t["dt_bias"], t["state"],
                                 t["mask"], chunked=True)
    heads = [0, 1, 17, 31]
    hks = [h // 2 for h in heads]
    g = gdn.compute_g(r["A_log"][heads], r["a"][:, :, heads], r["dt_bias"][heads])
    y_ref, S_ref = gdn.recurrent(r["q"][:, :, hks], r["k"][:, :, hks], r["v"][:, :, heads], g,
                                 gdn.compute_beta(r["b"][:, :, heads]), r["state"][:, heads], r["mask"])
    yn = y[:, :, heads].float().cpu().numpy()
    assert head_errs_state(S[:, heads].cpu().numpy(), S_ref).max() <= STATE_TOL
    assert row_errs_y(yn, y_ref).max() <= Y_TOL
    assert not y.float().cpu().numpy()[~r["mask"]].any(), "a masked token's y is not 0"


def test_masked_packed_sequences_match_oracle():
    """Packed sequences with a token mask, and masked rows take the chunked
    kernel by default."""
    lens = [70, 0, 1, 128, 63]
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    d = draw(930, 1, int(cu[-1]), 2, 4, 128, 128, state=False, mask_p=0.3)
    t, r = to_torch(d, DEV)
    S0 = np.random.default_rng(9).normal(0, 0.02, (len(lens), 4, 128, 128)).astype(np.float32)
    y, S = mx.gated_delta_update(t["q"], t["k"], t["v"], t["a"], t["b"], t["A_log"], t["dt_bias"],
                                 torch.tensor(S0, device=DEV), t["mask"], cu_seqlens=cu)
    g = gdn.compute_g(r["A_log"], r["a"], r["dt_bias"])
    y_ref, S_ref = gdn.recurrent_varlen(r["q"][:, :, [0, 0, 1, 1]], r["k"][:, :, [0, 0, 1, 1]], r["v"], g,
                                        gdn.compute_beta(r["b"]), cu, S0.astype(np.float64), r["mask"])
    yn = y.float().cpu().numpy()
    assert rel_err(yn[r["mask"]], y_ref[r["mask"]]) <= Y_TOL
    assert not yn[~r["mask"]].any()
    assert head_errs_state(S.cpu().numpy(), S_ref).max() <= STATE_TOL
    assert mx.gated_delta._use_chunked(None, t["q"], t["k"], t["v"], t["mask"], 128)

