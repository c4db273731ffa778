"""CPU port of the reference's ops path, timed as the CPU baseline.

TEST / BENCHMARK INFRASTRUCTURE ONLY: imported by ``bench.py``'s
``cpu_baseline`` leg (and tests), never by the product package.

mlx-lm's ``gated_delta_ops`` -- what the reference runs for
``gated_delta_update(..., use_kernel=...)`` off the Metal GPU, called from
``multiplex/kernel/dflash.py:372-374`` -- is a loop over T of whole-array
fp32 ops on the ``[B,Hv,Dv,Dk]`` state: decay, a reduction for ``S k``, the
rank-1 update, a reduction for ``S q``, and ``where(mask, new, old)``.  This
module restates that loop with torch CPU tensor ops in fp32, vectorised the
same way (one temporary of the state's size per op), plus the prologue
(depthwise conv1d + SiLU + RMS norm) for the prefill configurations.  It
shares the semantics of ``oracle.gdn`` (which is the float64 checker).
"""

from __future__ import annotations

import torch
import torch.nn.functional as F


def compute_g(A_log, a, dt_bias):
    return torch.exp(-torch.exp(A_log.float()) * F.softplus(a.float() + dt_bias.float()))


def gated_delta_ops(q, k, v, g, beta, state, mask=None):
    """fp32 ops-path recurrence; q,k [B,T,Hk,Dk], v [B,T,Hv,Dv], state [B,Hv,Dv,Dk]."""
    B, T, Hk, Dk = q.shape
    Hv = v.shape[2]
    r = Hv // Hk
    q = q.float().repeat_interleave(r, dim=2)
    k = k.float().repeat_interleave(r, dim=2)
    v = v.float()
    S = state.float()
    ys = []
    for t in range(T):
        old = S
        S = S * g[:, t, :, None, None]
        kv = (S * k[:, t, :, None, :]).sum(-1)
        delta = (v[:, t] - kv) * beta[:, t, :, None]
        S = S + k[:, t, :, None, :] * delta[..., None]
        y = (S * q[:, t, :, None, :]).sum(-1)
        if mask is not None:
            S = torch.where(mask[:, t, None, None, None], S, old)
        ys.append(y)
    return torch.stack(ys, dim=1), S


def gated_delta_update(q, k, v, a, b, A_log, dt_bias, state, mask=None):
    return gated_delta_ops(q, k, v, compute_g(A_log, a, dt_bias), torch.sigmoid(b.float()), state, mask)


def conv_prologue(qkv, weight, Hk, Hv, Dk, Dv, conv_state, eps=1e-6):
    """Depthwise conv1d (K taps) + SiLU + q/k RMS norm with the mixer's scales, in fp32."""
    B, S, C = qkv.shape
    Kt = weight.shape[1]
    ci = torch.cat([conv_state.float(), qkv.float()], dim=1)
    out = F.silu(F.conv1d(ci.transpose(1, 2), weight.float()[:, None, :], groups=C).transpose(1, 2))
    kd = Hk * Dk
    q = out[..., :kd].reshape(B, S, Hk, Dk)
    k = out[..., kd:2 * kd].reshape(B, S, Hk, Dk)
    v = out[..., 2 * kd:].reshape(B, S, Hv, Dv)
    q = F.rms_norm(q, (Dk,), eps=eps) / Dk
    k = F.rms_norm(k, (Dk,), eps=eps) / Dk ** 0.5
    return q, k, v, ci[:, -(Kt - 1):]
