"""Pins the float64 oracle (CPU only).

Each oracle function is checked against something other than its own
formula: closed forms, scalar brute force, the transformers library's torch
restatement (golden fixtures), torch's conv1d / rms_norm / softplus /
sigmoid, and invariants (split-T, mask = deletion, batch independence,
commit = prefix, chunked = recurrent).  ``test_planted_mistakes`` shows that
plausible mistakes in the recurrence fail those pins.
"""

from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from gdn_cases import draw, rel_err
from oracle import gdn

GOLD = Path(__file__).resolve().parent / "golden"


def load(name):
    with np.load(GOLD / f"{name}.npz") as z:
        return {k: z[k].astype(np.float64) for k in z.files}


def gates(d):
    return gdn.compute_g(d["A_log"], d["a"], d["dt_bias"]), gdn.compute_beta(d["b"])


# ------------------------------------------------------------ closed forms

def test_identity_step_keeps_state():
    d = draw(1, 2, 3, 2, 4, 8, 6)
    ones = np.ones((2, 3, 4))
    y, S = gdn.recurrent(d["q"], d["k"], d["v"], ones, np.zeros_like(ones), d["state"])
    np.testing.assert_allclose(S, d["state"], rtol=0, atol=0)
    qr = np.repeat(d["q"], 2, axis=2)
    for t in range(3):
        expect = np.einsum("bhvk,bhk->bhv", d["state"], qr[:, t])
        np.testing.assert_allclose(y[:, t], expect, rtol=1e-13, atol=1e-15)


def test_zero_decay_is_outer_product():
    d = draw(2, 1, 1, 1, 1, 5, 3)
    beta = np.full((1, 1, 1), 0.7)
    y, S = gdn.recurrent(d["q"], d["k"], d["v"], np.zeros((1, 1, 1)), beta, d["state"])
    k, q, v = d["k"][0, 0, 0], d["q"][0, 0, 0], d["v"][0, 0, 0]
    np.testing.assert_allclose(S[0, 0], 0.7 * np.outer(v, k), rtol=1e-14)
    np.testing.assert_allclose(y[0, 0, 0], 0.7 * v * (k @ q), rtol=1e-14)


def test_unit_write_stores_value():
    # g = 1, beta = 1, |k| = 1: the delta rule writes v at key k exactly.
    d = draw(3, 1, 1, 1, 2, 16, 8)
    one = np.ones((1, 1, 2))
    _, S = gdn.recurrent(d["q"], d["k"], d["v"], one, one, d["state"])
    k = d["k"][0, 0, 0]
    for h in range(2):
        np.testing.assert_allclose(S[0, h] @ k, d["v"][0, 0, h], rtol=1e-12, atol=1e-13)


def test_scalar_brute_force_tiny():
    B, T, Hk, Hv, Dk, Dv = 2, 4, 2, 4, 3, 2
    d = draw(4, B, T, Hk, Hv, Dk, Dv, mask_p=0.3)
    g, beta = gates(d)
    y, S = gdn.recurrent(d["q"], d["k"], d["v"], g, beta, d["state"], d["mask"])
    St = [[[[float(d["state"][b, h, i, j]) for j in range(Dk)] for i in range(Dv)]
           for h in range(Hv)] for b in range(B)]
    for b in range(B):
        for t in range(T):
            if not d["mask"][b, t]:
                for h in range(Hv):
                    for i in range(Dv):
                        assert y[b, t, h, i] == 0.0
                continue
            for h in range(Hv):
                hk = h // (Hv // Hk)
                M = St[b][h]
                for i in range(Dv):
                    for j in range(Dk):
                        M[i][j] *= g[b, t, h]
                for i in range(Dv):
                    kv = sum(M[i][j] * d["k"][b, t, hk, j] for j in range(Dk))
                    delta = beta[b, t, h] * (d["v"][b, t, h, i] - kv)
                    for j in range(Dk):
                        M[i][j] += delta * d["k"][b, t, hk, j]
                    yo = sum(M[i][j] * d["q"][b, t, hk, j] for j in range(Dk))
                    assert abs(yo - y[b, t, h, i]) <= 1e-12 * (1 + abs(yo))
    np.testing.assert_allclose(S, np.array(St), rtol=1e-12, atol=1e-14)


# --------------------------------------------------- library cross-checks

@pytest.mark.parametrize("name", ["recurrent_small", "recurrent_hd128"])
def test_recurrent_matches_library_fixture(name):
    d = load(name)
    y, S = gdn.gated_delta_update(d["q"], d["k"], d["v"], d["a"], d["b"], d["A_log"],
                                  d["dt_bias"], d["state"])
    assert rel_err(y, d["y"]) < 2e-6
    assert rel_err(S, d["state_out"]) < 2e-6


def test_chunked_matches_library_fixture():
    d = load("chunked_t100")
    g, beta = gates(d)
    y, S = gdn.chunked(d["q"], d["k"], d["v"], g, beta, d["state"], chunk=int(d["chunk"]))
    assert rel_err(y, d["y"]) < 2e-6
    assert rel_err(S, d["state_out"]) < 2e-6
    y2, S2 = gdn.recurrent(d["q"], d["k"], d["v"], g, beta, d["state"])
    assert rel_err(y2, d["y"]) < 2e-6


def test_gates_match_torch():
    x = np.concatenate([np.linspace(-60, 60, 241), [0.0, 1e-8, -1e-8]])
    A_log = np.linspace(0, np.log(16), x.size)
    dt = np.linspace(-1, 1, x.size)[::-1].copy()
    expect = torch.exp(-torch.exp(torch.tensor(A_log)) * F.softplus(torch.tensor(x) + torch.tensor(dt), threshold=200.0))
    np.testing.assert_allclose(gdn.compute_g(A_log, x, dt), expect.numpy(), rtol=1e-12, atol=1e-300)
    np.testing.assert_allclose(gdn.compute_beta(x), torch.sigmoid(torch.tensor(x)).numpy(), rtol=1e-12)


def test_prologue_matches_torch_fixture():
    d = load("prologue_small")
    B, S, Hk, Hv, D, Kt = (int(x) for x in d["dims"])
    q, k, v, cs, _ = gdn.conv_prologue(d["qkv"], d["weight"], Hk, Hv, D, D, conv_state=d["conv_state"],
                                       mask=d["mask"].astype(bool), eps=float(d["eps"]))
    for got, name in ((q, "q"), (k, "k"), (v, "v"), (cs, "conv_state_out")):
        np.testing.assert_allclose(got, d[name], rtol=1e-12, atol=1e-14, err_msg=name)


def test_bf16_round_matches_torch():
    x = np.random.default_rng(0).standard_normal(4096) * 10.0 ** np.random.default_rng(1).integers(-8, 8, 4096)
    x = np.concatenate([x, [0.0, -0.0, np.inf, -np.inf, 3.0e38]])
    ref = torch.tensor(x, dtype=torch.float32).to(torch.bfloat16).double().numpy()
    np.testing.assert_array_equal(gdn.bf16_round(x), ref)


def test_gated_norm_matches_library_fixture():
    d = load("gated_norm_small")
    eps = float(d["eps"])
    cases = [(gdn.bf16_round, True, "out_bf16_wbf16"), (gdn.bf16_round, False, "out_bf16_wf32"),
             (None, False, "out_f32")]
    for rnd, w_rounds, key in cases:
        got = gdn.gated_rms_norm(d["x"], d["gate"], d["weight"], eps, round_fn=rnd, weight_rounds=w_rounds)
        exp = d[key]
        if rnd is None:
            assert rel_err(got, exp) < 1e-6, key
        else:
            # float64 vs the module's float32 arithmetic: the same bf16 value
            # except where an intermediate lies next to a rounding boundary
            same = np.mean(got == exp)
            assert same > 0.999 and rel_err(got, exp) < 2e-3, (key, same)
    # a plausible mistake: the weight product left unrounded for a bf16 weight
    wrong = gdn.gated_rms_norm(d["x"], d["gate"], d["weight"], eps, round_fn=gdn.bf16_round, weight_rounds=False)
    assert np.mean(wrong == d["out_bf16_wbf16"]) < 0.95


def test_gated_norm_closed_forms():
    D = 64
    x = np.full((3, D), -2.5)
    gate = np.stack([np.zeros(D), np.full(D, 40.0), np.linspace(-3, 3, D)])
    w = np.linspace(0.5, 1.5, D)
    out = gdn.gated_rms_norm(x, gate, w, eps=0.0)
    np.testing.assert_allclose(out[0], 0.0, atol=0)                  # silu(0) = 0
    np.testing.assert_allclose(out[1], -w * 40.0, rtol=1e-15)        # rms of a constant row is |c|
    np.testing.assert_allclose(out[2], -w * gate[2] / (1 + np.exp(-gate[2])), rtol=1e-14)
    rng = np.random.default_rng(5)
    xr, gr = rng.standard_normal((4, D)), rng.standard_normal((4, D))
    np.testing.assert_allclose(gdn.gated_rms_norm(1e3 * xr, gr, w, eps=0.0), gdn.gated_rms_norm(xr, gr, w, eps=0.0),
                               rtol=1e-13)
    np.testing.assert_allclose(gdn.gated_rms_norm(xr, gr, None, eps=0.0), gdn.gated_rms_norm(xr, gr, np.ones(D), eps=0.0),
                               rtol=0)


# -------------------------------------------------------------- invariants

def test_split_T_carries_state():
    d = draw(5, 2, 9, 2, 4, 16, 8)
    g, beta = gates(d)
    y, S = gdn.recurrent(d["q"], d["k"], d["v"], g, beta, d["state"])
    y1, S1 = gdn.recurrent(d["q"][:, :4], d["k"][:, :4], d["v"][:, :4], g[:, :4], beta[:, :4], d["state"])
    y2, S2 = gdn.recurrent(d["q"][:, 4:], d["k"][:, 4:], d["v"][:, 4:], g[:, 4:], beta[:, 4:], S1)
    np.testing.assert_allclose(np.concatenate([y1, y2], axis=1), y, rtol=1e-12, atol=1e-15)
    np.testing.assert_allclose(S2, S, rtol=1e-12, atol=1e-15)


def test_mask_equals_deleting_tokens():
    d = draw(6, 1, 8, 1, 2, 8, 4, mask_p=0.4)
    d["mask"][0, 0] = False
    g, beta = gates(d)
    y, S = gdn.recurrent(d["q"], d["k"], d["v"], g, beta, d["state"], d["mask"])
    keep = np.nonzero(d["mask"][0])[0]
    yk, Sk = gdn.recurrent(d["q"][:, keep], d["k"][:, keep], d["v"][:, keep], g[:, keep], beta[:, keep],
                           d["state"])
    np.testing.assert_allclose(y[:, keep], yk, rtol=1e-12, atol=1e-15)
    np.testing.assert_allclose(S, Sk, rtol=1e-12, atol=1e-15)
    assert np.all(y[:, ~d["mask"][0]] == 0.0)


def test_rows_are_independent():
    d = draw(7, 3, 5, 2, 4, 8, 8)
    g, beta = gates(d)
    y, S = gdn.recurrent(d["q"], d["k"], d["v"], g, beta, d["state"])
    for b in range(3):
        sl = slice(b, b + 1)
        yb, Sb = gdn.recurrent(d["q"][sl], d["k"][sl], d["v"][sl], g[sl], beta[sl], d["state"][sl])
        np.testing.assert_array_equal(yb, y[sl])
        np.testing.assert_array_equal(Sb, S[sl])


def test_gqa_equals_repeated_heads():
    d = draw(8, 2, 4, 2, 6, 8, 4)
    g, beta = gates(d)
    y, S = gdn.recurrent(d["q"], d["k"], d["v"], g, beta, d["state"])
    qr, kr = np.repeat(d["q"], 3, axis=2), np.repeat(d["k"], 3, axis=2)
    y2, S2 = gdn.recurrent(qr, kr, d["v"], g, beta, d["state"])
    np.testing.assert_array_equal(y, y2)
    np.testing.assert_array_equal(S, S2)


def test_commit_equals_prefix_replay():
    d = draw(9, 4, 4, 2, 4, 8, 8)
    g, beta = gates(d)
    n = np.array([0, 1, 3, 4])
    S = gdn.commit(d["q"], d["k"], d["v"], g, beta, d["state"], n)
    np.testing.assert_array_equal(S[0], d["state"][0])
    for b in range(1, 4):
        sl = slice(b, b + 1)
        _, Sb = gdn.recurrent(d["q"][sl, : n[b]], d["k"][sl, : n[b]], d["v"][sl, : n[b]], g[sl, : n[b]],
                              beta[sl, : n[b]], d["state"][sl])
        np.testing.assert_allclose(S[b], Sb[0], rtol=1e-13, atol=1e-16)


def test_varlen_equals_separate_rows():
    lens = [3, 0, 7, 1]
    cu = np.concatenate([[0], np.cumsum(lens)])
    d = draw(10, 1, int(cu[-1]), 2, 4, 8, 8, state=False)
    g, beta = gates(d)
    S0 = np.random.default_rng(0).normal(0, 0.02, (len(lens), 4, 8, 8))
    y, S = gdn.recurrent_varlen(d["q"], d["k"], d["v"], g, beta, cu, S0)
    for n, (s, e) in enumerate(zip(cu[:-1], cu[1:])):
        yn, Sn = gdn.recurrent(d["q"][:, s:e], d["k"][:, s:e], d["v"][:, s:e], g[:, s:e], beta[:, s:e],
                               S0[n : n + 1])
        np.testing.assert_array_equal(y[:, s:e], yn)
        np.testing.assert_array_equal(S[n], Sn[0])


@pytest.mark.parametrize("T,chunk", [(1, 64), (63, 64), (64, 64), (130, 64), (50, 16)])
def test_chunked_equals_recurrent(T, chunk):
    d = draw(11 + T, 2, T, 2, 4, 16, 8)
    g, beta = gates(d)
    y, S = gdn.recurrent(d["q"], d["k"], d["v"], g, beta, d["state"])
    yc, Sc = gdn.chunked(d["q"], d["k"], d["v"], g, beta, d["state"], chunk=chunk)
    assert rel_err(yc, y) < 1e-11
    assert rel_err(Sc, S) < 1e-11


def test_chunked_survives_underflowing_decay():
    # exp(A_log) softplus(a + dt) of ~60 per token: the chunk decay underflows.
    d = draw(12, 1, 70, 1, 2, 8, 8)
    d["a"] = np.full_like(d["a"], 4.0)
    d["A_log"] = np.full_like(d["A_log"], np.log(15.0))
    g, beta = gates(d)
    assert g.max() < 1e-20
    y, S = gdn.recurrent(d["q"], d["k"], d["v"], g, beta, d["state"])
    yc, Sc = gdn.chunked(d["q"], d["k"], d["v"], g, beta, d["state"])
    assert np.isfinite(yc).all() and np.isfinite(Sc).all()
    assert rel_err(yc, y) < 1e-11 and rel_err(Sc, S) < 1e-11


def test_conv_state_commit_rule():
    d = load("prologue_small")
    B, S, Hk, Hv, D, Kt = (int(x) for x in d["dims"])
    mask = d["mask"].astype(bool)
    _, _, _, cs_full, ci = gdn.conv_prologue(d["qkv"], d["weight"], Hk, Hv, D, D,
                                             conv_state=d["conv_state"], mask=mask)
    full = gdn.conv_state_commit(ci, [S] * B, Kt)
    np.testing.assert_array_equal(full, cs_full)
    none = gdn.conv_state_commit(ci, [0] * B, Kt)
    np.testing.assert_array_equal(none, d["conv_state"])
    two = gdn.conv_state_commit(ci, [2] * B, Kt)
    np.testing.assert_array_equal(two[:, 1:], np.where(mask[:, :2, None], d["qkv"][:, :2], 0.0))


# ------------------------------------------------------ planted mistakes

def _mutant(kind):
    def run(q, k, v, g, beta, state):
        B, T, Hk, Dk = q.shape
        Hv = v.shape[2]
        r = Hv // Hk
        S = state.copy()
        y = np.zeros(v.shape)
        for t in range(T):
            for h in range(Hv):
                hk = (h % Hk) if kind == "gqa_modulo" else h // r
                kk, qq = k[:, t, hk], q[:, t, hk]
                if kind == "swap_qk":
                    kk, qq = qq, kk
                if kind == "decay_after":
                    kv = np.einsum("bvk,bk->bv", S[:, h], kk)
                    S[:, h] = g[:, t, h, None, None] * (S[:, h] + (beta[:, t, h, None] * (v[:, t, h] - kv))[..., None] * kk[:, None, :])
                else:
                    Sg = S[:, h] * g[:, t, h, None, None]
                    kv = np.einsum("bvk,bk->bv", Sg, kk)
                    sign = -1.0 if kind == "sign" else 1.0
                    S[:, h] = Sg + sign * (beta[:, t, h, None] * (v[:, t, h] - kv))[..., None] * kk[:, None, :]
                y[:, t, h] = np.einsum("bvk,bk->bv", S[:, h], qq)
        return y, S
    return run


@pytest.mark.parametrize("kind", ["gqa_modulo", "swap_qk", "decay_after", "sign"])
def test_planted_mistakes(kind):
    d = load("recurrent_small")
    g, beta = gates(d)
    y, S = _mutant("none")(d["q"], d["k"], d["v"], g, beta, d["state"])
    assert rel_err(y, d["y"]) < 2e-6 and rel_err(S, d["state_out"]) < 2e-6
    ym, Sm = _mutant(kind)(d["q"], d["k"], d["v"], g, beta, d["state"])
    assert max(rel_err(ym, d["y"]), rel_err(Sm, d["state_out"])) > 1e-2


# ------------------------------------------------------------------ mixer

def _mixer_fixture(name):
    d = load(name)
    B, S, H, Hk, Hv, D, Kt = (int(x) for x in d["dims"])
    p = {k[2:]: v for k, v in d.items() if k.startswith("p_")}
    return d, p, (Hk, Hv, D, D)


def _run_mixer(d, p, dims, round_bf16=False):
    return gdn.mixer_forward(p, d["x"], *dims, conv_state=d["conv_state"], state=d["state"],
                             eps=float(d["eps"]), round_bf16=round_bf16)


@pytest.mark.parametrize("name", ["mixer_prefill_f32", "mixer_decode_f32"])
def test_mixer_matches_library_module(name):
    """``mixer_forward`` against transformers' Qwen3_5GatedDeltaNet in float32
    (prefill through its chunked path, decode through its single-token
    update), from nonzero conv and recurrent states: output, conv state and
    state.  The remaining ~1e-6 is float32 arithmetic and the norm's epsilon
    (transformers adds 1e-6 to sum(x^2); the reference's rms_norm form adds
    Dk * 1e-6)."""
    d, p, dims = _mixer_fixture(name)
    out, cs, st = _run_mixer(d, p, dims)
    assert rel_err(out, d["out"]) < 2e-5
    assert rel_err(cs, d["conv_state_out"]) < 1e-6
    assert rel_err(st, d["state_out"]) < 2e-5


def test_mixer_bf16_module_within_rounding_distance():
    """The same module run in bfloat16 rounds at more points (after the conv,
    after SiLU, the L2 norm and beta in bf16 arithmetic) than the oracle's
    bf16 mode, which rounds where the fused kernels do (projections, q/k/v,
    y, normed y, output); the reference's own points (mlx-lm) are unknown
    here.  Two bf16 restatements agree to the size of those roundings."""
    d, p, dims = _mixer_fixture("mixer_prefill_bf16")
    out, cs, st = _run_mixer(d, p, dims, round_bf16=True)
    assert rel_err(out, d["out"]) < 2e-2 and rel_err(st, d["state_out"]) < 2e-2
    np.testing.assert_array_equal(cs, d["conv_state_out"])


def _mixer_mutant(kind, monkeypatch):
    if kind == "flipped_conv_taps":
        real = gdn.conv_prologue
        monkeypatch.setattr(gdn, "conv_prologue", lambda qkv, w, *a, **k: real(qkv, np.asarray(w)[:, ::-1], *a, **k))
    elif kind == "norm_gated_by_y":
        real = gdn.gated_rms_norm
        monkeypatch.setattr(gdn, "gated_rms_norm", lambda x, gate, *a, **k: real(x, x, *a, **k))
    elif kind == "norm_over_all_heads":
        real = gdn.gated_rms_norm

        def over_all(x, gate, weight=None, *a, **k):
            sh = np.shape(x)
            w = None if weight is None else np.tile(weight, sh[-2])
            return real(np.reshape(x, sh[:-2] + (-1,)), np.reshape(gate, sh[:-2] + (-1,)), w, *a, **k).reshape(sh)
        monkeypatch.setattr(gdn, "gated_rms_norm", over_all)
    elif kind == "q_scaled_like_k":
        real = gdn.conv_prologue

        def scaled(*a, **k):
            q, kk, v, cs, ci = real(*a, **k)
            return q * np.sqrt(q.shape[-1]), kk, v, cs, ci
        monkeypatch.setattr(gdn, "conv_prologue", scaled)


@pytest.mark.parametrize("kind", ["swap_a_b", "flipped_conv_taps", "norm_gated_by_y", "norm_over_all_heads",
                                  "q_scaled_like_k"])
def test_mixer_planted_mistakes(kind, monkeypatch):
    """Plausible wiring mistakes planted in the oracle fail the module pin."""
    d, p, dims = _mixer_fixture("mixer_prefill_f32")
    if kind == "swap_a_b":
        p = dict(p, in_proj_a=p["in_proj_b"], in_proj_b=p["in_proj_a"])
    _mixer_mutant(kind, monkeypatch)
    out, _, st = _run_mixer(d, p, dims)
    assert max(rel_err(out, d["out"]), rel_err(st, d["state_out"])) > 1e-2
