"""Seeded GDN test inputs and the norm-wise tolerances shared by the tests.

Inputs are drawn on the CPU in float64 and rounded to the device dtypes; the
oracle is fed the rounded values, so both sides see identical inputs.

Tolerances (the contract of the path):
* bf16/fp16 outputs y: ||y - y_ref||_2 / ||y_ref||_2 <= 2e-3 per row;
* fp32 state:          ||S - S_ref||_2 / ||S_ref||_2 <= 1e-4 per (row, head).
Norm-wise, because one bf16 ulp (2^-8 relative) exceeds 2e-3 elementwise.
"""

from __future__ import annotations

import numpy as np

Y_TOL = 2e-3
STATE_TOL = 1e-4


def rel_err(x, ref, axes=None):
    """Norm-wise relative error, reduced over ``axes`` (all when None)."""
    x = np.asarray(x, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    num = np.sqrt(np.sum((x - ref) ** 2, axis=axes))
    den = np.sqrt(np.sum(ref ** 2, axis=axes))
    return num / np.maximum(den, 1e-30)


def row_errs_y(y, y_ref):
    """Per-row error of y [B,T,Hv,Dv]."""
    return rel_err(y, y_ref, axes=(1, 2, 3))


def head_errs_state(S, S_ref):
    """Per-(row, head) error of a state [B,Hv,Dv,Dk]."""
    return rel_err(S, S_ref, axes=(2, 3))


def draw(seed, B, T, Hk, Hv, Dk, Dv, state=True, mask_p=None):
    """Float64 inputs with the distributions of the benchmark configs.

    q, k ~ N(0,1) then L2-normalised per head (q also scaled by 1/sqrt(Dk)),
    v ~ N(0,1), a, b ~ N(0,1), A_log ~ U(0, ln 16), dt_bias ~ U(-1, 1),
    S0 ~ N(0, 0.02).  ``mask_p``: probability that a token is masked out.
    """
    rng = np.random.default_rng(seed)
    q = rng.standard_normal((B, T, Hk, Dk))
    k = rng.standard_normal((B, T, Hk, Dk))
    q = q / np.maximum(np.linalg.norm(q, axis=-1, keepdims=True), 1e-12) / np.sqrt(Dk)
    k = k / np.maximum(np.linalg.norm(k, axis=-1, keepdims=True), 1e-12)
    d = dict(
        q=q, k=k, v=rng.standard_normal((B, T, Hv, Dv)),
        a=rng.standard_normal((B, T, Hv)), b=rng.standard_normal((B, T, Hv)),
        A_log=rng.uniform(0.0, np.log(16.0), Hv), dt_bias=rng.uniform(-1.0, 1.0, Hv),
        state=rng.normal(0.0, 0.02, (B, Hv, Dv, Dk)) if state else None,
        mask=None,
    )
    if mask_p is not None:
        d["mask"] = rng.random((B, T)) >= mask_p
    return d


def to_torch(d, device, dtype="bf16", gate_dtype="bf16", param_dtype="f32"):
    """Device tensors for ``d`` plus the float64 values they hold (for the oracle)."""
    import torch

    dt = {"bf16": torch.bfloat16, "f16": torch.float16, "f32": torch.float32}
    out, ref = {}, {}
    for key, tdt in (("q", dtype), ("k", dtype), ("v", dtype), ("a", gate_dtype), ("b", gate_dtype),
                     ("A_log", param_dtype), ("dt_bias", param_dtype)):
        t = torch.tensor(d[key], dtype=torch.float64).to(dt[tdt])
        ref[key] = t.double().numpy()
        out[key] = t.to(device)
    if d.get("state") is not None:
        t = torch.tensor(d["state"], dtype=torch.float32)
        ref["state"] = t.double().numpy()
        out["state"] = t.to(device)
    else:
        ref["state"] = None
        out["state"] = None
    if d.get("mask") is not None:
        out["mask"] = torch.tensor(d["mask"], dtype=torch.bool).to(device)
        ref["mask"] = np.asarray(d["mask"], dtype=bool)
    else:
        out["mask"] = None
        ref["mask"] = None
    return out, ref
