"""Float64 CPU restatement of multiplex's fused Gated DeltaNet (GDN) path.

TEST INFRASTRUCTURE ONLY.  This module is the oracle the HIP kernels are
checked against.  Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import it, and only as the checker
(or, for the baseline, as the thing timed on the host).  The product package
``multiplex_amd`` never imports it and has no CPU fallback.

What it restates (reference call sites; the arithmetic itself lives in the
third-party ``mlx-lm`` package that multiplex imports, which is absent here):

* ``gated_delta_update(q, k, v, a, b, A_log, dt_bias, state, mask)`` --
  called at ``multiplex/kernel/dflash.py:372-374`` (verify / prefill) and
  ``multiplex/kernel/dflash.py:417-422`` (rollback replay), reached through
  ``multiplex/kernel/engine.py:164-167``.
* the decay / gate transforms ``g = exp(-exp(A_log) * softplus(a + dt_bias))``
  and ``beta = sigmoid(b)`` (inputs passed at ``dflash.py:371-373``).
* the mixer prologue: mask zeroing, conv-state concat, depthwise causal
  conv1d (K taps, no bias) + SiLU, q/k RMS-norm with ``1/Dk`` and
  ``1/sqrt(Dk)`` scales, conv-state update (``dflash.py:351-370``).
* the mixer epilogue's gated RMSNorm ``norm(out, z)`` (``dflash.py:377``).
* the commit rule of a partially accepted verify: state after the first
  ``n`` tokens, ``conv_state = conv_input[:, n : n + K - 1]``
  (``dflash.py:403-426``; ``engine.py:337-359`` replays the same prefix).

Pinning (each function is checked in ``tests/test_oracle.py`` by something
other than a retyping of its own formula):

* ``recurrent``: closed forms (g=1,beta=0; g=0; delta-rule write S'k=v),
  brute-force scalar loops on tiny shapes, the transformers library's torch
  restatement ``torch_recurrent_gated_delta_rule`` (library cross-check),
  split-T / batch-independence / GQA invariants.
* ``chunked``: equality with ``recurrent`` in float64 and with transformers'
  ``torch_chunk_gated_delta_rule``.
* ``compute_g`` / ``compute_beta``: torch.nn.functional.softplus /
  torch.sigmoid.
* ``conv_prologue``: torch.nn.functional.conv1d(groups=C) and
  torch.nn.functional.rms_norm.
* ``commit``: equality with ``recurrent`` run on the accepted prefix alone.
* ``gated_rms_norm``: transformers' ``Qwen3NextRMSNormGated`` module run on
  the CPU (library cross-check), closed forms (constant rows, zero gate) and
  scale invariance.

Rounding points inside mlx-lm's Metal kernel (bf16 vs fp32 gates, reduction
order) cannot be pinned without importing mlx-lm; the tolerances
(2e-3 norm-wise on bf16 outputs, 1e-4 norm-wise on the fp32 state) absorb
them.  Masked positions: mlx-lm keeps the state (``where(mask, new, old)``);
the y value at a masked position is unspecified there and is 0 here.
"""

from __future__ import annotations

import numpy as np

__all__ = [
    "softplus",
    "sigmoid",
    "compute_g",
    "compute_beta",
    "recurrent",
    "gated_delta_update",
    "recurrent_varlen",
    "commit",
    "chunked",
    "conv_prologue",
    "conv_state_commit",
    "bf16_round",
    "gated_rms_norm",
    "mixer_forward",
]


def _f64(x):
    return None if x is None else np.asarray(x, dtype=np.float64)


def bf16_round(x) -> np.ndarray:
    """Round float values to the nearest bfloat16 (ties to even), returned as float64.

    Used to emulate the dtype of bf16 outputs; NaN/Inf are passed through.
    """
    x32 = np.asarray(x, dtype=np.float32)
    u = x32.view(np.uint32).astype(np.uint64)
    rounding = ((u >> 16) & 1) + 0x7FFF
    r = ((u + rounding) >> 16) << 16
    out = r.astype(np.uint32).view(np.float32)
    out = np.where(np.isfinite(x32), out, x32)
    return out.astype(np.float64)


def softplus(x):
    """softplus(x) = log(1 + e^x), evaluated stably."""
    x = _f64(x)
    return np.logaddexp(0.0, x)


def sigmoid(x):
    """1 / (1 + e^-x), evaluated without cancellation for either sign of x."""
    x = _f64(x)
    e = np.exp(-np.abs(x))
    return np.where(x >= 0, 1.0 / (1.0 + e), e / (1.0 + e))


def compute_g(A_log, a, dt_bias):
    """Per-token, per-v-head decay ``g = exp(-exp(A_log) * softplus(a + dt_bias))``.

    ``a`` is ``[..., Hv]``; ``A_log`` and ``dt_bias`` are ``[Hv]``.  The formula
    is the one mlx-lm's ``compute_g`` evaluates for the arguments multiplex
    passes at ``multiplex/kernel/dflash.py:372-373``.
    """
    A_log, a, dt_bias = _f64(A_log), _f64(a), _f64(dt_bias)
    return np.exp(-np.exp(A_log) * softplus(a + dt_bias))


def compute_beta(b):
    """``beta = sigmoid(b)`` (the write strength of the delta rule)."""
    return sigmoid(b)


def _expand_heads(x, Hv):
    """GQA head expansion: v-head h reads k-head ``h // (Hv // Hk)``.

    Equivalent to repeating each k-head ``Hv // Hk`` times along the head axis
    (mlx ``repeat(x, r, axis=-2)``).
    """
    Hk = x.shape[-2]
    if Hv % Hk:
        raise ValueError(f"Hv={Hv} is not a multiple of Hk={Hk}")
    return np.repeat(x, Hv // Hk, axis=-2)


def recurrent(q, k, v, g, beta, state=None, mask=None):
    """The T-step gated delta rule, sequential over T (mlx-lm ``gated_delta_ops``).

    Shapes: q, k ``[B,T,Hk,Dk]``; v ``[B,T,Hv,Dv]``; g, beta ``[B,T,Hv]``;
    state ``[B,Hv,Dv,Dk]`` (Dk innermost, mlx-lm layout) or None (zeros);
    mask ``[B,T]`` bool or None.

    Per step, for every (b, h) with S in R^{Dv x Dk}::

        S <- g S;  kv = S k;  delta = beta (v - kv);  S <- S + delta k^T;  y = S q

    A masked step (mask false) keeps S; its y is 0.
    Returns ``(y [B,T,Hv,Dv], state [B,Hv,Dv,Dk])`` in float64.
    """
    q, k, v, g, beta = (_f64(t) for t in (q, k, v, g, beta))
    B, T, Hk, Dk = q.shape
    Hv, Dv = v.shape[-2:]
    qr = _expand_heads(q, Hv)
    kr = _expand_heads(k, Hv)
    S = np.zeros((B, Hv, Dv, Dk)) if state is None else _f64(state).copy()
    y = np.zeros((B, T, Hv, Dv))
    for t in range(T):
        Sg = S * g[:, t, :, None, None]
        kv = np.einsum("bhvk,bhk->bhv", Sg, kr[:, t])
        delta = beta[:, t, :, None] * (v[:, t] - kv)
        Sn = Sg + delta[..., None] * kr[:, t][:, :, None, :]
        yt = np.einsum("bhvk,bhk->bhv", Sn, qr[:, t])
        if mask is not None:
            m = np.asarray(mask[:, t], dtype=bool)
            S = np.where(m[:, None, None, None], Sn, S)
            yt = np.where(m[:, None, None], yt, 0.0)
        else:
            S = Sn
        y[:, t] = yt
    return y, S


def gated_delta_update(q, k, v, a, b, A_log, dt_bias, state=None, mask=None):
    """Entry point semantics of ``gated_delta_update`` (``dflash.py:372-374``).

    ``beta = sigmoid(b)``, ``g = compute_g(A_log, a, dt_bias)``, zero state when
    None, then the recurrence.  Returns ``(y, new_state)`` in float64.
    """
    g = compute_g(A_log, a, dt_bias)
    beta = compute_beta(b)
    return recurrent(q, k, v, g, beta, state, mask)


def recurrent_varlen(q, k, v, g, beta, cu_seqlens, state=None, mask=None):
    """Packed ragged sequences: q ``[1,N_tok,Hk,Dk]`` etc., ``cu_seqlens [N+1]``.

    Sequence n owns tokens ``[cu[n], cu[n+1])`` and state ``state[n]``.  This is
    the same recurrence applied per sequence; it defines the varlen contract
    of the packed prefill / mixed-batch launch (continuous batching).
    """
    cu = np.asarray(cu_seqlens, dtype=np.int64)
    N = len(cu) - 1
    Hv, Dv = np.shape(v)[-2:]
    Dk = np.shape(q)[-1]
    ys = np.zeros(np.shape(v)[:-2] + (Hv, Dv))
    S_out = np.zeros((N, Hv, Dv, Dk))
    for n in range(N):
        s, e = int(cu[n]), int(cu[n + 1])
        sl = slice(s, e)
        st = None if state is None else _f64(state)[n : n + 1]
        mk = None if mask is None else np.asarray(mask)[:, sl]
        yn, Sn = recurrent(
            _f64(q)[:, sl], _f64(k)[:, sl], _f64(v)[:, sl],
            _f64(g)[:, sl], _f64(beta)[:, sl], st, mk,
        )
        ys[:, sl] = yn
        S_out[n] = Sn[0]
    return ys, S_out


def commit(q, k, v, g, beta, state, n_commit, mask=None):
    """State after each row's accepted prefix of ``n_commit[b]`` tokens.

    The rollback rule of ``dflash.py:403-426`` / ``engine.py:337-359``: re-run
    the update from the pre-verify state on ``[:, :n]``.  ``n_commit[b] = 0``
    returns the initial state.  Returns ``[B,Hv,Dv,Dk]`` float64.
    """
    B = np.shape(q)[0]
    Hv, Dv = np.shape(v)[-2:]
    Dk = np.shape(q)[-1]
    out = np.zeros((B, Hv, Dv, Dk))
    for b in range(B):
        n = int(n_commit[b])
        st = None if state is None else _f64(state)[b : b + 1]
        if n == 0:
            out[b] = 0.0 if st is None else st[0]
            continue
        mk = None if mask is None else np.asarray(mask)[b : b + 1, :n]
        _, Sb = recurrent(
            _f64(q)[b : b + 1, :n], _f64(k)[b : b + 1, :n], _f64(v)[b : b + 1, :n],
            _f64(g)[b : b + 1, :n], _f64(beta)[b : b + 1, :n], st, mk,
        )
        out[b] = Sb[0]
    return out


def chunked(q, k, v, g, beta, state=None, chunk=64):
    """WY/UT chunked form of the same recurrence (no mask), float64.

    Within a chunk of C tokens starting from state S0, with L_t the inclusive
    cumulative sum of log g and gamma_t = exp(L_t)::

        A[t,i]  = beta_t exp(L_t - L_i) (k_t . k_i)          for i < t, else 0
        U       = (I + A)^{-1} diag(beta) (V - diag(gamma) K S0^T)
        Y       = diag(gamma) Q S0^T + (exp(L_t - L_i) [i <= t] * Q K^T) U
        S_C     = gamma_C S0 + (diag(exp(L_C - L)) U)^T K

    This is the algorithm the chunked MFMA prefill kernel implements; it is
    checked against ``recurrent`` in float64.  Returns ``(y, state)``.
    """
    q, k, v, g, beta = (_f64(t) for t in (q, k, v, g, beta))
    B, T, Hk, Dk = q.shape
    Hv, Dv = v.shape[-2:]
    qr = _expand_heads(q, Hv)
    kr = _expand_heads(k, Hv)
    S = np.zeros((B, Hv, Dv, Dk)) if state is None else _f64(state).copy()
    y = np.zeros((B, T, Hv, Dv))
    with np.errstate(divide="ignore"):
        logg = np.log(g)
    for c0 in range(0, T, chunk):
        c1 = min(T, c0 + chunk)
        C = c1 - c0
        for bb in range(B):
            for h in range(Hv):
                Q = qr[bb, c0:c1, h]          # [C,Dk]
                K = kr[bb, c0:c1, h]          # [C,Dk]
                V = v[bb, c0:c1, h]           # [C,Dv]
                be = beta[bb, c0:c1, h]       # [C]
                L = np.cumsum(logg[bb, c0:c1, h])
                gam = np.exp(L)
                diff = L[:, None] - L[None, :]
                tri = np.tril(np.ones((C, C), dtype=bool))
                decay = np.where(tri, np.exp(np.where(tri, diff, 0.0)), 0.0)
                A = np.tril(be[:, None] * decay * (K @ K.T), -1)
                S0 = S[bb, h]                 # [Dv,Dk]
                R = be[:, None] * (V - gam[:, None] * (K @ S0.T))
                U = np.linalg.solve(np.eye(C) + A, R)
                Y = gam[:, None] * (Q @ S0.T) + (decay * (Q @ K.T)) @ U
                e = np.exp(L[-1] - L)
                S[bb, h] = gam[-1] * S0 + (e[:, None] * U).T @ K
                y[bb, c0:c1, h] = Y
    return y, S


def _silu(x):
    return x * sigmoid(x)


def conv_prologue(qkv, weight, Hk, Hv, Dk, Dv, conv_state=None, mask=None,
                  eps=1e-6):
    """GDN mixer prologue, following ``multiplex/kernel/dflash.py:351-370``.

    qkv: ``[B,S,C]`` with C = 2*Hk*Dk + Hv*Dv channels ordered q | k | v.
    weight: ``[C,K]`` depthwise taps (cross-correlation, no bias).
    conv_state: ``[B,K-1,C]`` or None (zeros).  mask: ``[B,S]`` or None.

    Steps: masked rows of qkv are zeroed; ``conv_input = concat(conv_state,
    qkv)``; ``out[s,c] = sum_j weight[c,j] * conv_input[s+j,c]``; SiLU;
    split into q, k, v; ``q = rms_norm(q)/Dk``, ``k = rms_norm(k)/sqrt(Dk)``
    with ``rms_norm(x) = x / sqrt(mean(x^2) + eps)``; the new conv state is
    the last K-1 rows of conv_input.

    Returns ``(q [B,S,Hk,Dk], k [B,S,Hk,Dk], v [B,S,Hv,Dv], new_conv_state,
    conv_input)`` in float64.
    """
    x = _f64(qkv)
    w = _f64(weight)
    B, S, C = x.shape
    Kt = w.shape[1]
    if C != 2 * Hk * Dk + Hv * Dv:
        raise ValueError("channel count does not match head layout")
    if conv_state is None:
        cs = np.zeros((B, Kt - 1, C))
    else:
        cs = _f64(conv_state)
    if mask is not None:
        x = np.where(np.asarray(mask, dtype=bool)[..., None], x, 0.0)
    ci = np.concatenate([cs, x], axis=1)          # [B,S+K-1,C]
    out = np.zeros((B, S, C))
    for j in range(Kt):
        out += w[None, None, :, j] * ci[:, j : j + S, :]
    out = _silu(out)
    kd = Hk * Dk
    q = out[..., :kd].reshape(B, S, Hk, Dk)
    k = out[..., kd : 2 * kd].reshape(B, S, Hk, Dk)
    v = out[..., 2 * kd :].reshape(B, S, Hv, Dv)

    def rms(z):
        return z / np.sqrt(np.mean(z * z, axis=-1, keepdims=True) + eps)

    q = rms(q) / Dk
    k = rms(k) / np.sqrt(Dk)
    new_cs = ci[:, -(Kt - 1):, :] if Kt > 1 else np.zeros((B, 0, C))
    return q, k, v, new_cs, ci


def conv_state_commit(conv_input, n_commit, Kt):
    """``conv_state = conv_input[:, n : n + K - 1]`` per row (``dflash.py:424-425``).

    conv_input: ``[B, K-1+T, C]`` (the verify's concat of old conv state and
    the T new mixed-qkv rows).  ``n_commit[b]`` counts tokens committed.
    """
    ci = _f64(conv_input)
    B = ci.shape[0]
    out = np.zeros((B, Kt - 1, ci.shape[2]))
    for b in range(B):
        n = int(n_commit[b])
        out[b] = ci[b, n : n + Kt - 1]
    return out


def gated_rms_norm(x, gate, weight=None, eps=1e-6, round_fn=None, weight_rounds=True):
    """Gated RMSNorm of the mixer epilogue, ``norm(out, z)`` at ``dflash.py:377``.

    Per row of the last dim: ``n = x / sqrt(mean(x^2) + eps)``,
    ``m = weight * n``, ``out = m * silu(gate)``.  ``round_fn`` (e.g.
    ``bf16_round``) rounds where a half-precision model materialises values,
    at the points of transformers' ``Qwen3NextRMSNormGated``
    (``models/qwen3_next/modeling_qwen3_next.py:57-74``): after the
    normalisation, after the weight product when the weight has the io dtype
    (``weight_rounds``), and at the output.
    """
    r = round_fn if round_fn is not None else (lambda t: np.asarray(t, dtype=np.float64))
    x = _f64(x)
    n = r(x / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps))
    m = n if weight is None else _f64(weight) * n
    if weight is not None and weight_rounds:
        m = r(m)
    return r(m * _silu(_f64(gate)))


def mixer_forward(params, inputs, Hk, Hv, Dk, Dv, conv_state=None, state=None, mask=None,
                  eps=1e-6, round_bf16=True):
    """GatedDeltaNet mixer (``multiplex/kernel/dflash.py:343-381``), float64.

    params: dict of float arrays ``in_proj_qkv [C,H]``, ``in_proj_z [Hv*Dv,H]``,
    ``in_proj_b [Hv,H]``, ``in_proj_a [Hv,H]``, ``conv1d [C,K]``, ``A_log``,
    ``dt_bias [Hv]``, ``norm [Dv]``, ``out_proj [H,Hv*Dv]``.  With
    ``round_bf16`` the activations are rounded to bf16 where a bf16 model
    materialises them (projection outputs, q/k/v, y, normed y, output).
    Returns ``(out, new_conv_state, new_state)``.
    """
    r = bf16_round if round_bf16 else (lambda t: np.asarray(t, dtype=np.float64))
    x = _f64(inputs)
    B, S, _ = x.shape
    qkv = r(x @ _f64(params["in_proj_qkv"]).T)
    z = r(x @ _f64(params["in_proj_z"]).T).reshape(B, S, Hv, Dv)
    b = r(x @ _f64(params["in_proj_b"]).T)
    a = r(x @ _f64(params["in_proj_a"]).T)
    q, k, v, new_cs, _ = conv_prologue(qkv, params["conv1d"], Hk, Hv, Dk, Dv, conv_state, mask, eps)
    q, k, v = r(q), r(k), r(v)
    y, new_state = gated_delta_update(q, k, v, a, b, params["A_log"], params["dt_bias"], state, mask)
    y = r(y)
    yn = gated_rms_norm(y, z, params["norm"], eps, round_fn=r if round_bf16 else None)
    out = r(yn.reshape(B, S, -1) @ _f64(params["out_proj"]).T)
    return out, new_cs, new_state
