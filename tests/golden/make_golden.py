"""Writes the golden fixtures in this directory.

The reference (wang1ang/multiplex) ships no GDN vectors, and its arithmetic
lives in mlx-lm, which is not installed.  The expected outputs here are
therefore computed by implementations independent of ``oracle/gdn.py``:

* the gated delta recurrence and its chunked form: the torch restatements in
  the ``transformers`` library (``torch_recurrent_gated_delta_rule`` and
  ``torch_chunk_gated_delta_rule`` of ``models/qwen3_next``), which take the
  decay in log space, the state as ``[B,H,Dk,Dv]``, scale q by 1/sqrt(Dk)
  internally and compute in float32;
* the gate transforms: ``torch.nn.functional.softplus`` / ``torch.sigmoid``;
* the prologue: ``torch.nn.functional.conv1d(groups=C)``, ``silu`` and
  ``rms_norm`` in float64;
* the epilogue's gated RMSNorm: transformers' ``Qwen3NextRMSNormGated``
  module, run in bfloat16 (bf16 and fp32 weight) and in float32.

Inputs are drawn from ``numpy.random.default_rng`` with fixed seeds.
Run: ``python tests/golden/make_golden.py [case ...]`` (needs transformers;
no argument writes every case).
"""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import torch
import torch.nn.functional as F

HERE = Path(__file__).resolve().parent


def _gdn_inputs(rng, B, T, Hk, Hv, Dk, Dv):
    q = rng.standard_normal((B, T, Hk, Dk))
    k = rng.standard_normal((B, T, Hk, Dk))
    q = q / np.linalg.norm(q, axis=-1, keepdims=True) / np.sqrt(Dk)
    k = k / np.linalg.norm(k, axis=-1, keepdims=True)
    v = rng.standard_normal((B, T, Hv, Dv))
    a = rng.standard_normal((B, T, Hv))
    b = rng.standard_normal((B, T, Hv))
    A_log = rng.uniform(0.0, np.log(16.0), Hv)
    dt_bias = rng.uniform(-1.0, 1.0, Hv)
    S0 = rng.normal(0.0, 0.02, (B, Hv, Dv, Dk))
    return dict(q=q, k=k, v=v, a=a, b=b, A_log=A_log, dt_bias=dt_bias, state=S0)


def _library_gates(d):
    A_log = torch.tensor(d["A_log"])
    a = torch.tensor(d["a"])
    dt = torch.tensor(d["dt_bias"])
    log_g = -torch.exp(A_log) * F.softplus(a + dt)
    beta = torch.sigmoid(torch.tensor(d["b"]))
    return log_g, beta


def _hf_args(d, Hv):
    Hk, Dk = d["q"].shape[2], d["q"].shape[3]
    r = Hv // Hk
    q = torch.tensor(d["q"]).repeat_interleave(r, dim=2) * np.sqrt(Dk)
    k = torch.tensor(d["k"]).repeat_interleave(r, dim=2)
    v = torch.tensor(d["v"])
    log_g, beta = _library_gates(d)
    st = torch.tensor(d["state"]).transpose(-1, -2).contiguous()
    return q, k, v, log_g, beta, st


def recurrent_case(name, seed, B, T, Hk, Hv, Dk, Dv):
    from transformers.models.qwen3_next.modeling_qwen3_next import torch_recurrent_gated_delta_rule

    d = _gdn_inputs(np.random.default_rng(seed), B, T, Hk, Hv, Dk, Dv)
    q, k, v, log_g, beta, st = _hf_args(d, Hv)
    y, S = torch_recurrent_gated_delta_rule(q, k, v, log_g, beta, st, True)
    d["y"] = y.double().numpy()
    d["state_out"] = S.double().transpose(-1, -2).numpy()
    d["g"] = torch.exp(log_g).numpy()
    d["beta"] = beta.numpy()
    np.savez_compressed(HERE / f"{name}.npz", **{kk: np.asarray(vv, dtype=np.float32) for kk, vv in d.items()})


def chunked_case(name, seed, B, T, Hk, Hv, Dk, Dv, chunk):
    from transformers.models.qwen3_next.modeling_qwen3_next import torch_chunk_gated_delta_rule

    d = _gdn_inputs(np.random.default_rng(seed), B, T, Hk, Hv, Dk, Dv)
    q, k, v, log_g, beta, st = _hf_args(d, Hv)
    y, S = torch_chunk_gated_delta_rule(q, k, v, log_g, beta, chunk_size=chunk, initial_state=st,
                                        output_final_state=True)
    d["y"] = y.double().numpy()
    d["state_out"] = S.double().transpose(-1, -2).numpy()
    d["chunk"] = np.array(chunk)
    np.savez_compressed(HERE / f"{name}.npz", **{kk: np.asarray(vv, dtype=np.float32) for kk, vv in d.items()})


def prologue_case(name, seed, B, S, Hk, Hv, D, Kt=4, eps=1e-6):
    rng = np.random.default_rng(seed)
    C = 2 * Hk * D + Hv * D
    qkv = rng.standard_normal((B, S, C))
    w = rng.normal(0.0, 0.5, (C, Kt))
    cs = rng.standard_normal((B, Kt - 1, C))
    mask = np.ones((B, S), dtype=bool)
    mask[0, S - 2] = False
    mask[-1, 0] = False
    x = torch.tensor(qkv) * torch.tensor(mask)[..., None]
    ci = torch.cat([torch.tensor(cs), x], dim=1)                    # [B, S+K-1, C]
    out = F.conv1d(ci.transpose(1, 2), torch.tensor(w)[:, None, :], groups=C)  # [B, C, S]
    out = F.silu(out.transpose(1, 2))
    kd = Hk * D
    qo = out[..., :kd].reshape(B, S, Hk, D)
    ko = out[..., kd:2 * kd].reshape(B, S, Hk, D)
    vo = out[..., 2 * kd:].reshape(B, S, Hv, D)
    qo = F.rms_norm(qo, (D,), eps=eps) / D
    ko = F.rms_norm(ko, (D,), eps=eps) / np.sqrt(D)
    np.savez_compressed(
        HERE / f"{name}.npz",
        qkv=qkv, weight=w, conv_state=cs, mask=mask.astype(np.float64),
        q=qo.numpy(), k=ko.numpy(), v=vo.numpy(), conv_state_out=ci[:, -(Kt - 1):].numpy(),
        dims=np.array([B, S, Hk, Hv, D, Kt], dtype=np.float64), eps=np.array(eps),
    )


def gated_norm_case(name, seed, rows, D, eps=1e-6):
    from transformers.models.qwen3_next.modeling_qwen3_next import Qwen3NextRMSNormGated

    rng = np.random.default_rng(seed)
    scale = 10.0 ** rng.uniform(-3, 3, (rows, 1))
    x = torch.tensor(rng.standard_normal((rows, D)) * scale, dtype=torch.float32).to(torch.bfloat16)
    gate = torch.tensor(rng.normal(0.0, 2.0, (rows, D)), dtype=torch.float32).to(torch.bfloat16)
    w = torch.tensor(rng.normal(1.0, 0.25, D), dtype=torch.float32).to(torch.bfloat16)
    x[0] = 0.75           # a constant row
    gate[1] = 0.0         # a zero gate
    outs = {}
    with torch.no_grad():
        m = Qwen3NextRMSNormGated(D, eps=eps).to(torch.bfloat16)
        m.weight.copy_(w)
        outs["out_bf16_wbf16"] = m(x, gate)
        m = Qwen3NextRMSNormGated(D, eps=eps).to(torch.float32)
        m.weight.copy_(w.float())
        outs["out_bf16_wf32"] = m(x, gate)
        outs["out_f32"] = m(x.float(), gate.float())
    np.savez_compressed(
        HERE / f"{name}.npz",
        x=x.float().numpy(), gate=gate.float().numpy(), weight=w.float().numpy(), eps=np.array(eps),
        **{k: v.float().numpy() for k, v in outs.items()},
    )


CASES = {
    "recurrent_small": lambda: recurrent_case("recurrent_small", 11, B=2, T=6, Hk=2, Hv=4, Dk=16, Dv=8),
    "recurrent_hd128": lambda: recurrent_case("recurrent_hd128", 12, B=1, T=3, Hk=2, Hv=4, Dk=128, Dv=128),
    "chunked_t100": lambda: chunked_case("chunked_t100", 13, B=1, T=100, Hk=1, Hv=2, Dk=32, Dv=16, chunk=64),
    "prologue_small": lambda: prologue_case("prologue_small", 14, B=2, S=7, Hk=2, Hv=4, D=16),
    "gated_norm_small": lambda: gated_norm_case("gated_norm_small", 15, rows=48, D=128),
}


def main():
    names = sys.argv[1:] or list(CASES)
    for n in names:
        torch.set_default_dtype(torch.float64)
        CASES[n]()
    print("wrote", names, file=sys.stderr)


if __name__ == "__main__":
    main()
