"""GPU parity of the recurrent kernel (decode / MTP verify / commit) against
the float64 oracle, through the C ABI (via the multiplex_amd wrappers).

Tolerances: see ``gdn_cases`` (2e-3 norm-wise on bf16 y per row, 1e-4
norm-wise on the fp32 state per (row, head)).
"""

from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest
import torch

import multiplex_amd as mx
from gdn_cases import STATE_TOL, Y_TOL, draw, head_errs_state, rel_err, row_errs_y, to_torch
from oracle import gdn

pytestmark = pytest.mark.gpu
DEV = "cuda"
GOLD = Path(__file__).resolve().parent / "golden"


def run_update(t, **kw):
    return mx.gated_delta_update(t["q"], t["k"], t["v"], t["a"], t["b"], t["A_log"], t["dt_bias"],
                                 t["state"], t["mask"], **kw)


def oracle_update(r):
    return gdn.gated_delta_update(r["q"], r["k"], r["v"], r["a"], r["b"], r["A_log"], r["dt_bias"],
                                  r["state"], r["mask"])


def assert_close(y, S, y_ref, S_ref, y_tol=Y_TOL, s_tol=STATE_TOL):
    y = y.float().cpu().numpy()
    S = S.cpu().numpy()
    ye = row_errs_y(y, y_ref)
    se = head_errs_state(S, S_ref)
    assert ye.max() <= y_tol, f"y rel err {ye.max():.3e}"
    assert se.max() <= s_tol, f"state rel err {se.max():.3e}"


@pytest.mark.parametrize("dtype", ["bf16", "f16", "f32"])
@pytest.mark.parametrize("Dk,Dv", [(128, 128), (64, 64), (256, 256), (128, 96), (128, 97), (64, 33)])
def test_decode_matches_oracle(dtype, Dk, Dv):
    d = draw(100 + Dk + Dv, 3, 1, 2, 4, Dk, Dv)
    t, r = to_torch(d, DEV, dtype=dtype, gate_dtype=dtype)
    y, S = run_update(t)
    assert y.dtype == t["q"].dtype and S.dtype == torch.float32
    assert_close(y, S, *oracle_update(r))


def test_decode_b64_full_heads():
    # Batched decode at the dynamic-batching shape: B=64, Hk=16, Hv=32, Dk=Dv=128.
    d = draw(1001, 64, 1, 16, 32, 128, 128)
    t, r = to_torch(d, DEV)
    y, S = run_update(t)
    assert_close(y, S, *oracle_update(r))


def test_decode_b1_full_heads():
    d = draw(1000, 1, 1, 16, 32, 128, 128)
    t, r = to_torch(d, DEV)
    y, S = run_update(t)
    assert_close(y, S, *oracle_update(r))


@pytest.mark.parametrize("mask_p", [None, 0.35])
def test_multi_token_gqa_mask(mask_p):
    d = draw(7, 3, 9, 2, 6, 128, 128, mask_p=mask_p)
    if mask_p is not None:
        d["mask"][1, :] = False
        d["mask"][2, 0] = False
    t, r = to_torch(d, DEV)
    y, S = run_update(t)
    y_ref, S_ref = oracle_update(r)
    assert_close(y, S, y_ref, S_ref)
    if mask_p is not None:
        yc = y.float().cpu().numpy()
        assert np.all(yc[~r["mask"]] == 0.0)
        np.testing.assert_array_equal(S[1].cpu().numpy(), t["state"][1].cpu().numpy())


def test_zero_state_when_none():
    d = draw(8, 2, 5, 2, 4, 128, 128, state=False)
    t, r = to_torch(d, DEV)
    y, S = run_update(t)
    assert_close(y, S, *oracle_update(r))


@pytest.mark.parametrize("name", ["recurrent_small", "recurrent_hd128"])
def test_golden_fixtures_fp32(name):
    with np.load(GOLD / f"{name}.npz") as z:
        f = {k: torch.tensor(z[k]) for k in z.files}
    if f["q"].shape[-1] not in (64, 128, 256):
        # Dk = 16 is not built; run the fixture with keys zero-padded to Dk = 64,
        # which leaves every dot product (and so y and the state) unchanged.
        pad = 64 - f["q"].shape[-1]
        for key in ("q", "k"):
            f[key] = torch.nn.functional.pad(f[key], (0, pad))
        f["state"] = torch.nn.functional.pad(f["state"], (0, pad))
        f["state_out"] = torch.nn.functional.pad(f["state_out"], (0, pad))
    t = {k: v.to(DEV) for k, v in f.items()}
    y, S = mx.gated_delta_update(t["q"], t["k"], t["v"], t["a"], t["b"], t["A_log"], t["dt_bias"], t["state"])
    assert rel_err(y.cpu().numpy(), f["y"].numpy()) < 1e-5
    assert rel_err(S.cpu().numpy(), f["state_out"].numpy()) < 1e-5


def test_kernel_with_precomputed_gates_matches_update():
    d = draw(9, 4, 3, 2, 4, 128, 128)
    t, _ = to_torch(d, DEV)
    g = mx.compute_g(t["A_log"], t["a"], t["dt_bias"])
    beta = mx.compute_beta(t["b"])
    y1, S1 = run_update(t)
    y2, S2 = mx.gated_delta_kernel(t["q"], t["k"], t["v"], g, beta, t["state"])
    assert rel_err(y2.float().cpu().numpy(), y1.float().cpu().numpy()) < 1e-3
    assert rel_err(S2.cpu().numpy(), S1.cpu().numpy()) < 1e-5


def test_functional_state_not_mutated_and_in_place():
    d = draw(10, 2, 2, 2, 4, 128, 128)
    t, r = to_torch(d, DEV)
    before = t["state"].clone()
    y, S = run_update(t)
    assert torch.equal(t["state"], before)
    y2, S2 = run_update(t, state_out=t["state"])
    assert S2.data_ptr() == t["state"].data_ptr()
    assert torch.equal(S2, S) and torch.equal(y2, y)


def test_rows_bitwise_independent():
    d = draw(11, 5, 3, 2, 4, 128, 128)
    t, _ = to_torch(d, DEV)
    y, S = run_update(t)
    for b in (0, 3):
        tb = {k: (None if v is None else (v[b:b + 1] if v.dim() >= 2 and v.shape[0] == 5 else v))
              for k, v in t.items()}
        yb, Sb = run_update(tb)
        assert torch.equal(yb, y[b:b + 1]) and torch.equal(Sb, S[b:b + 1])


def test_split_T_is_bitwise():
    d = draw(12, 2, 7, 2, 4, 128, 128)
    t, _ = to_torch(d, DEV)
    y, S = run_update(t)
    t1 = {k: (v[:, :3] if k in ("q", "k", "v", "a", "b") else v) for k, v in t.items()}
    t2 = {k: (v[:, 3:] if k in ("q", "k", "v", "a", "b") else v) for k, v in t.items()}
    y1, S1 = run_update(t1)
    t2["state"] = S1
    y2, S2 = run_update(t2)
    assert torch.equal(torch.cat([y1, y2], 1), y) and torch.equal(S2, S)


def test_verify_snapshots_and_commit():
    B, T = 32, 4
    d = draw(2002, B, T, 16, 32, 128, 128)
    t, r = to_torch(d, DEV)
    before = t["state"].clone()
    y, snaps = mx.gated_delta_verify(t["q"], t["k"], t["v"], t["a"], t["b"], t["A_log"], t["dt_bias"],
                                     t["state"], snapshots=True)
    assert torch.equal(t["state"], before)
    g, beta = gdn.compute_g(r["A_log"], r["a"], r["dt_bias"]), gdn.compute_beta(r["b"])
    y_ref, _ = gdn.recurrent(r["q"], r["k"], r["v"], g, beta, r["state"])
    assert row_errs_y(y.float().cpu().numpy(), y_ref).max() <= Y_TOL
    n = np.random.default_rng(5).integers(1, T + 1, B)
    S_ref = gdn.commit(r["q"], r["k"], r["v"], g, beta, r["state"], n)
    # snapshot n-1 is the committed state
    snap_pick = snaps[torch.arange(B), torch.tensor(n - 1)].cpu().numpy()
    assert head_errs_state(snap_pick, S_ref).max() <= STATE_TOL
    # commit kernel: re-reads the pre-verify state, writes the accepted prefix once
    S_c = mx.gated_delta_commit(t["k"], t["v"], t["a"], t["b"], t["A_log"], t["dt_bias"], t["state"],
                                torch.tensor(n, dtype=torch.int32))
    assert head_errs_state(S_c.cpu().numpy(), S_ref).max() <= STATE_TOL
    assert torch.equal(S_c, snaps[torch.arange(B), torch.tensor(n - 1)])
    # in place, with a zero and a skipped row
    n2 = n.copy()
    n2[0], n2[1] = 0, -1
    st = t["state"].clone()
    mx.gated_delta_commit(t["k"], t["v"], t["a"], t["b"], t["A_log"], t["dt_bias"], st,
                          torch.tensor(n2, dtype=torch.int32), state_out=st)
    assert torch.equal(st[0], t["state"][0]) and torch.equal(st[1], t["state"][1])
    assert torch.equal(st[2:], S_c[2:])


@pytest.mark.parametrize("T", [1, 2, 3, 4, 5, 8])
@pytest.mark.parametrize("dtype,Dk,Dv", [("bf16", 128, 128), ("f16", 64, 64), ("f32", 256, 256), ("bf16", 128, 96)])
def test_verify_without_state_write_matches_oracle(T, dtype, Dk, Dv):
    """Verify of T <= 8 tokens with no state write or snapshots runs the
    unrolled kernel; y against the oracle and against the stepping kernel
    (snapshot mode), masks included."""
    d = draw(300 + T + Dk + Dv, 3, T, 2, 4, Dk, Dv, mask_p=0.25 if T > 2 else None)
    t, r = to_torch(d, DEV, dtype=dtype, gate_dtype=dtype)
    before = t["state"].clone()
    y, none = mx.gated_delta_verify(t["q"], t["k"], t["v"], t["a"], t["b"], t["A_log"], t["dt_bias"],
                                    t["state"], t["mask"])
    assert none is None and torch.equal(t["state"], before)
    y_ref, _ = oracle_update(r)
    assert row_errs_y(y.float().cpu().numpy(), y_ref).max() <= Y_TOL
    y_step, _ = mx.gated_delta_verify(t["q"], t["k"], t["v"], t["a"], t["b"], t["A_log"], t["dt_bias"],
                                      t["state"], t["mask"], snapshots=True)
    assert row_errs_y(y.float().cpu().numpy(), y_step.float().cpu().numpy()).max() <= Y_TOL
    if t["mask"] is not None:
        off = ~t["mask"].cpu()
        assert torch.all(y.cpu()[off] == 0)


def _offset_copy(x, shift=4):
    """x in a buffer shifted by `shift` elements: 8-byte but not 16-byte aligned."""
    buf = torch.empty(x.numel() + shift, dtype=x.dtype, device=x.device)
    out = buf[shift:].view(x.shape)
    out.copy_(x)
    return out


@pytest.mark.parametrize("T", [1, 3, 4, 6, 8])
def test_verify_mfma_and_fma_kernels_agree(T):
    """bf16 q/k at Dk=128 take the MFMA verify (state split hi/lo bf16);
    q/k rows that are only 8-byte aligned take the FMA kernel.  Both against
    the oracle, and against each other."""
    d = draw(400 + T, 5, T, 2, 4, 128, 128, mask_p=0.25 if T > 2 else None)
    t, r = to_torch(d, DEV)
    args = (t["v"], t["a"], t["b"], t["A_log"], t["dt_bias"], t["state"], t["mask"])
    y_mfma, _ = mx.gated_delta_verify(t["q"], t["k"], *args)
    q8, k8 = _offset_copy(t["q"]), _offset_copy(t["k"])
    assert q8.data_ptr() % 16 != 0 and k8.data_ptr() % 16 != 0
    y_fma, _ = mx.gated_delta_verify(q8, k8, *args)
    y_ref, _ = oracle_update(r)
    assert row_errs_y(y_mfma.float().cpu().numpy(), y_ref).max() <= Y_TOL
    assert row_errs_y(y_fma.float().cpu().numpy(), y_ref).max() <= Y_TOL
    assert row_errs_y(y_mfma.float().cpu().numpy(), y_fma.float().cpu().numpy()).max() <= Y_TOL


def test_verify_with_underflowing_decay_and_precomputed_gates():
    d = draw(77, 2, 4, 2, 4, 128, 128)
    d["A_log"][:] = 12.0          # exp(A_log) softplus(.) >> 100: g underflows to 0
    t, r = to_torch(d, DEV)
    y, _ = mx.gated_delta_verify(t["q"], t["k"], t["v"], t["a"], t["b"], t["A_log"], t["dt_bias"], t["state"])
    y_ref, _ = oracle_update(r)
    assert torch.isfinite(y.float()).all()
    assert row_errs_y(y.float().cpu().numpy(), y_ref).max() <= Y_TOL
    g = mx.compute_g(t["A_log"], t["a"], t["dt_bias"])
    beta = mx.compute_beta(t["b"])
    plan = mx.prepare_recurrent(t["q"], t["k"], t["v"], g, beta, None, None, t["state"], write_state=False,
                                gates_precomputed=True)
    plan.launch()
    torch.cuda.synchronize()
    assert row_errs_y(plan.outputs[0].float().cpu().numpy(), y_ref).max() <= Y_TOL


def test_packed_ragged_rows():
    lens = [1, 4, 0, 3, 1, 7]
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    d = draw(13, 1, int(cu[-1]), 2, 4, 128, 128, state=False)
    t, r = to_torch(d, DEV)
    S0 = np.random.default_rng(3).normal(0, 0.02, (len(lens), 4, 128, 128)).astype(np.float32)
    st = torch.tensor(S0, device=DEV)
    y, S = mx.gated_delta_update(t["q"], t["k"], t["v"], t["a"], t["b"], t["A_log"], t["dt_bias"], st,
                                 cu_seqlens=torch.tensor(cu), chunked=False)
    g, beta = gdn.compute_g(r["A_log"], r["a"], r["dt_bias"]), gdn.compute_beta(r["b"])
    y_ref, S_ref = gdn.recurrent_varlen(r["q"], r["k"], r["v"], g, beta, cu, S0.astype(np.float64))
    assert rel_err(y.float().cpu().numpy(), y_ref) <= Y_TOL
    assert head_errs_state(S.cpu().numpy(), S_ref).max() <= STATE_TOL
    np.testing.assert_array_equal(S[2].cpu().numpy(), S0[2])


@pytest.mark.parametrize("Dk,Dv", [(128, 128), (64, 64), (256, 256), (128, 96), (128, 97)])
def test_decode_step_bitwise_equals_tile_step(Dk, Dv):
    """The decode kernel (one token per row, Dk/4 lanes per state row) and the
    multi-token kernel (8 lanes per row; taken here through the packed form
    with one token per sequence) sum a row's dot products in one order, so
    the same token gives bit-identical outputs and states."""
    B = 5
    d = draw(120 + Dk + Dv, B, 1, 2, 4, Dk, Dv)
    t, r = to_torch(d, DEV)
    y1, S1 = run_update(t)
    assert_close(y1, S1, *oracle_update(r))
    flat = lambda x: x.reshape(1, B, *x.shape[2:]).contiguous()
    cu = torch.arange(B + 1, dtype=torch.int32)
    y2, S2 = mx.gated_delta_update(flat(t["q"]), flat(t["k"]), flat(t["v"]), flat(t["a"]), flat(t["b"]),
                                   t["A_log"], t["dt_bias"], t["state"], cu_seqlens=cu, chunked=False)
    assert torch.equal(y2.reshape(y1.shape), y1) and torch.equal(S2, S1)


@pytest.mark.parametrize("Hk,Hv", [(4, 4), (2, 6), (3, 15)])
def test_decode_head_groups(Hk, Hv):
    """One-token steps with 1, 3 and 5 v-heads per k-head (the decode kernel
    finds a head's k-head by a multiply and shift); an odd Hv takes the
    general body (its gates are not read as dwords)."""
    d = draw(150 + Hv, 3, 1, Hk, Hv, 128, 128)
    t, r = to_torch(d, DEV)
    y, S = run_update(t)
    assert_close(y, S, *oracle_update(r))


@pytest.mark.parametrize("param_dtype,mask_p", [("bf16", None), ("bf16", 0.5), ("f32", 0.5)])
def test_decode_gate_formats_and_mask(param_dtype, mask_p):
    """One-token steps through the decode kernel's lean body (bf16 A_log /
    dt_bias: the all-bf16 gate format) and its general body (a mask), against
    the oracle and bit-identical to the multi-token kernel on the same token."""
    B = 6
    d = draw(130 + (mask_p is not None), B, 1, 2, 4, 128, 128, mask_p=mask_p)
    t, r = to_torch(d, DEV, param_dtype=param_dtype)
    y, S = run_update(t)
    assert_close(y, S, *oracle_update(r))
    if mask_p is not None:
        off = ~r["mask"][:, 0]
        assert off.any() and (~off).any()
        assert torch.equal(S[torch.tensor(off, device=DEV)], t["state"][torch.tensor(off, device=DEV)])
    flat = lambda x: x.reshape(1, B, *x.shape[2:]).contiguous()
    cu = torch.arange(B + 1, dtype=torch.int32)
    m = None if t["mask"] is None else t["mask"].reshape(1, B)
    y2, S2 = mx.gated_delta_update(flat(t["q"]), flat(t["k"]), flat(t["v"]), flat(t["a"]), flat(t["b"]),
                                   t["A_log"], t["dt_bias"], t["state"], m, cu_seqlens=cu, chunked=False)
    assert torch.equal(y2.reshape(y.shape), y) and torch.equal(S2, S)


def test_decode_snapshot_commit_and_zero_state():
    """The decode kernel's other one-token options: a verify with snapshots
    (the snapshot is the stepped state, the input state is not written), a
    commit of n in {-1, 0, 1} into a separate state, and no input state."""
    B = 5
    d = draw(140, B, 1, 2, 4, 128, 128)
    t, r = to_torch(d, DEV)
    before = t["state"].clone()
    y_ref, S_ref = oracle_update(r)
    y, snaps = mx.gated_delta_verify(t["q"], t["k"], t["v"], t["a"], t["b"], t["A_log"], t["dt_bias"],
                                     t["state"], snapshots=True)
    assert torch.equal(t["state"], before)
    assert_close(y, snaps[:, 0], y_ref, S_ref)
    n = [1, 0, -1, 1, 0]
    out = torch.full_like(t["state"], 7.0)
    S_c = mx.gated_delta_commit(t["k"], t["v"], t["a"], t["b"], t["A_log"], t["dt_bias"], t["state"], n,
                                state_out=out)
    for b_, nb in enumerate(n):
        if nb == 1:
            assert head_errs_state(S_c[b_:b_ + 1].cpu().numpy(), S_ref[b_:b_ + 1]).max() <= STATE_TOL
        else:  # 0 keeps the state; a negative n copies it unchanged into a separate state_out
            assert torch.equal(S_c[b_], before[b_])
    d0 = draw(141, B, 1, 2, 4, 128, 128, state=False)
    t0, r0 = to_torch(d0, DEV, dtype="f16", gate_dtype="f16")
    y0, S0 = run_update(t0)
    assert_close(y0, S0, *oracle_update(r0))


def test_carried_state_many_steps():
    B, steps = 4, 40
    d = draw(14, B, steps, 16, 32, 128, 128)
    t, r = to_torch(d, DEV)
    st = t["state"].clone()
    ys = []
    for s in range(steps):
        y, st = mx.gated_delta_update(t["q"][:, s:s + 1], t["k"][:, s:s + 1], t["v"][:, s:s + 1],
                                      t["a"][:, s:s + 1], t["b"][:, s:s + 1], t["A_log"], t["dt_bias"], st,
                                      state_out=st)
        ys.append(y)
    y_ref, S_ref = oracle_update(r)
    assert_close(torch.cat(ys, 1), st, y_ref, S_ref)


def test_zero_tokens_copies_state():
    d = draw(15, 3, 0, 2, 4, 128, 128)
    t, _ = to_torch(d, DEV)
    y, S = run_update(t)
    assert y.shape == (3, 0, 4, 128)
    assert torch.equal(S, t["state"])


def test_ops_path_on_device_matches_kernel():
    d = draw(16, 2, 3, 2, 4, 128, 128, mask_p=0.3)
    t, r = to_torch(d, DEV)
    y1, S1 = run_update(t)
    y2, S2 = run_update(t, use_kernel=False)
    assert y2.device.type == "cuda"
    y_ref, S_ref = oracle_update(r)
    assert_close(y2, S2, y_ref, S_ref)
    assert rel_err(S1.cpu().numpy(), S2.cpu().numpy()) < 1e-5


@pytest.mark.parametrize("T,y_from", [(8, 4), (4, 1), (16, 9)])
def test_y_from_leaves_earlier_tokens_out_and_the_rest_bit_identical(T, y_from):
    """``y_from``: tokens before it produce no y; the state and the later
    tokens' y equal the launch that forms every y, bit for bit."""
    d = draw(700 + T, 3, T, 2, 4, 128, 128, mask_p=0.25)
    t, _ = to_torch(d, DEV)
    n = torch.tensor([T // 2, T, 1], dtype=torch.int32, device=DEV)
    args = (t["q"], t["k"], t["v"], t["a"], t["b"], t["A_log"], t["dt_bias"], t["state"], t["mask"])
    full = mx.prepare_recurrent(*args, commit_len=n, state_out=torch.empty_like(t["state"]))
    part = mx.prepare_recurrent(*args, commit_len=n, state_out=torch.empty_like(t["state"]), y_from=y_from)
    full.launch()
    part.launch()
    torch.cuda.synchronize()
    assert torch.equal(part.outputs[1], full.outputs[1])
    assert torch.equal(part.outputs[0][:, y_from:], full.outputs[0][:, y_from:])


@pytest.mark.parametrize("Tp,T", [(4, 4), (3, 5), (1, 1), (4, 6)])
def test_commit_verify_is_commit_then_verify(Tp, T):
    """One pass over the state: the commit of the previous round's accepted
    drafts (n_prev clamped to [0, Tp]) and the verify of the next round's.
    The launch steps the tile kernel, as the commit does, so the committed
    state is bit-identical to the commit's."""
    d = draw(90 + Tp, 6, Tp + T, 2, 4, 128, 128)
    t, r = to_torch(d, DEV)
    part = lambda lo, hi: tuple(t[n][:, lo:hi].contiguous() for n in ("q", "k", "v", "a", "b"))
    prev, new = part(0, Tp), part(Tp, Tp + T)
    n_prev = [0, 1, Tp, 2, -1, Tp + 3]
    y, S = mx.gated_delta_commit_verify(prev, n_prev, *new, t["A_log"], t["dt_bias"], t["state"])
    S_c = mx.gated_delta_commit(*prev[1:], t["A_log"], t["dt_bias"], t["state"],
                                [min(max(n, 0), Tp) for n in n_prev])
    assert torch.equal(S, S_c)
    y_v, _ = mx.gated_delta_verify(*new, t["A_log"], t["dt_bias"], S_c)
    assert row_errs_y(y.float().cpu().numpy(), y_v.float().cpu().numpy()).max() <= Y_TOL
    # the same against the oracle: the committed prefix, then the new tokens
    g = gdn.compute_g(r["A_log"], r["a"], r["dt_bias"])
    beta = gdn.compute_beta(r["b"])
    for b_, n in enumerate(n_prev):
        n = min(max(n, 0), Tp)
        idx = list(range(n)) + list(range(Tp, Tp + T))
        hk = [h // 2 for h in range(4)]
        y_ref, S_ref = gdn.recurrent(r["q"][b_:b_ + 1, idx][:, :, hk], r["k"][b_:b_ + 1, idx][:, :, hk],
                                     r["v"][b_:b_ + 1, idx], g[b_:b_ + 1, idx], beta[b_:b_ + 1, idx],
                                     r["state"][b_:b_ + 1])
        assert row_errs_y(y[b_:b_ + 1].float().cpu().numpy(), y_ref[:, n:]).max() <= Y_TOL
    # a mask on the new drafts: masked ones leave the state alone and give y = 0
    m = torch.rand(6, T, generator=torch.Generator().manual_seed(Tp + T)) >= 0.3
    y_m, S_m = mx.gated_delta_commit_verify(prev, n_prev, *new, t["A_log"], t["dt_bias"], t["state"],
                                            m.to(DEV))
    assert torch.equal(S_m, S)
    y_vm, _ = mx.gated_delta_verify(*new, t["A_log"], t["dt_bias"], S_c, m.to(DEV))
    assert not y_m[~m.to(DEV)].any()
    assert row_errs_y(y_m.float().cpu().numpy(), y_vm.float().cpu().numpy()).max() <= Y_TOL
    st = t["state"].clone()
    y2, S2 = mx.gated_delta_commit_verify(prev, n_prev, *new, t["A_log"], t["dt_bias"], st, state_out=st)
    assert S2.data_ptr() == st.data_ptr() and torch.equal(S2, S) and torch.equal(y2, y)
    # pooled states: row b in slot idx[b], updated in place
    idx = torch.tensor([5, 0, 7, 2, 3, 6], dtype=torch.int32, device=DEV)
    pool = torch.zeros(8, *t["state"].shape[1:], device=DEV)
    pool[idx.long()] = t["state"]
    y3, _ = mx.gated_delta_commit_verify(prev, n_prev, *new, t["A_log"], t["dt_bias"], pool, state_index=idx)
    assert torch.equal(pool[idx.long()], S) and torch.equal(y3, y)
    assert not pool[[1, 4]].any()
    assert head_errs_state(S_c.cpu().numpy()[5:6], gdn.recurrent(
        r["q"][5:6, :Tp][:, :, [0, 0, 1, 1]], r["k"][5:6, :Tp][:, :, [0, 0, 1, 1]], r["v"][5:6, :Tp],
        g[5:6, :Tp], beta[5:6, :Tp], r["state"][5:6])[1]).max() <= STATE_TOL



@pytest.mark.parametrize("T,Dv,gate_dtype,param_dtype", [(2, 128, "bf16", "f32"), (4, 96, "bf16", "bf16"),
                                                         (5, 128, "f32", "f32"), (8, 80, "bf16", "f32")])
def test_ragged_commit_matches_oracle(T, Dv, gate_dtype, param_dtype):
    """Commits of 2-8 tokens: ragged n (T, 0, negative, 1, past T, T - 1)
    with a mask, Dv not a multiple of the 32-row workgroup, the typed and the
    runtime gate formats; into a fresh state, in place, into pool slots, and
    from no input state."""
    B = 6
    d = draw(300 + 10 * T + Dv, B, T, 2, 4, 128, Dv, mask_p=0.25)
    t, r = to_torch(d, DEV, gate_dtype=gate_dtype, param_dtype=param_dtype)
    g, beta = gdn.compute_g(r["A_log"], r["a"], r["dt_bias"]), gdn.compute_beta(r["b"])
    n = np.array([T, 0, -1, 1, T + 3, T - 1], dtype=np.int32)
    args = (t["k"], t["v"], t["a"], t["b"], t["A_log"], t["dt_bias"])
    S = mx.gated_delta_commit(*args, t["state"], torch.tensor(n), t["mask"])
    S_ref = gdn.commit(r["q"], r["k"], r["v"], g, beta, r["state"], np.clip(n, 0, T), r["mask"])
    assert head_errs_state(S.cpu().numpy(), S_ref).max() <= STATE_TOL
    assert torch.equal(S[1], t["state"][1]) and torch.equal(S[2], t["state"][2])
    st = t["state"].clone()
    mx.gated_delta_commit(*args, st, torch.tensor(n), t["mask"], state_out=st)
    assert torch.equal(st, S)
    idx = torch.tensor([3, 0, 5, 1, 7, 2], dtype=torch.int32, device=DEV)
    pool = torch.zeros(8, *t["state"].shape[1:], device=DEV)
    pool[idx.long()] = t["state"]
    mx.gated_delta_commit(*args, pool, torch.tensor(n), t["mask"], state_index=idx)
    assert torch.equal(pool[idx.long()], S) and not pool[[4, 6]].any()
    S0 = mx.gated_delta_commit(*args, None, torch.tensor(n), t["mask"])
    S0_ref = gdn.commit(r["q"], r["k"], r["v"], g, beta, None, np.clip(n, 0, T), r["mask"])
    assert head_errs_state(S0.cpu().numpy()[[0, 3, 4, 5]], S0_ref[[0, 3, 4, 5]]).max() <= STATE_TOL
    assert not S0[[1, 2]].any()


def test_skipped_commit_row_into_a_fresh_state():
    """A negative commit length skips the row; with no ``state_out`` (a
    fresh output tensor) the row is the unchanged input state, not
    uninitialised memory."""
    d = draw(2003, 4, 3, 2, 4, 128, 128)
    t, r = to_torch(d, DEV)
    n = np.array([2, -1, 3, -5], dtype=np.int32)
    S = mx.gated_delta_commit(t["k"], t["v"], t["a"], t["b"], t["A_log"], t["dt_bias"], t["state"],
                              torch.tensor(n))
    assert torch.equal(S[1], t["state"][1]) and torch.equal(S[3], t["state"][3])
    g, beta = gdn.compute_g(r["A_log"], r["a"], r["dt_bias"]), gdn.compute_beta(r["b"])
    S_ref = gdn.commit(r["q"], r["k"], r["v"], g, beta, r["state"], np.maximum(n, 0))
    assert head_errs_state(S.cpu().numpy(), S_ref).max() <= STATE_TOL


def test_default_path_for_shapes_the_chunked_kernel_does_not_take():
    """Long bf16 rows at Dk=128 with Dv=96, or with 8-byte aligned q/k, go to
    the recurrent kernel by default instead of failing in the chunked one."""
    d = draw(2004, 1, 80, 2, 4, 128, 96)
    t, r = to_torch(d, DEV)
    y, S = run_update(t)
    y_ref, S_ref = oracle_update(r)
    assert row_errs_y(y.float().cpu().numpy(), y_ref).max() <= Y_TOL
    assert head_errs_state(S.cpu().numpy(), S_ref).max() <= STATE_TOL
    d = draw(2005, 1, 80, 2, 4, 128, 128)
    t, r = to_torch(d, DEV)
    t["q"], t["k"] = _offset_copy(t["q"]), _offset_copy(t["k"])
    y, S = run_update(t)
    y_ref, S_ref = oracle_update(r)
    assert row_errs_y(y.float().cpu().numpy(), y_ref).max() <= Y_TOL
    assert head_errs_state(S.cpu().numpy(), S_ref).max() <= STATE_TOL
