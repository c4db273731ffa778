"""GPU parity of the mixer epilogue's gated RMSNorm (``gdn_gated_rmsnorm``)
against the float64 oracle and the transformers golden fixture."""

from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest
import torch

import multiplex_amd as mx
from gdn_cases import Y_TOL, rel_err
from oracle import gdn

pytestmark = pytest.mark.gpu
DEV = "cuda"
GOLD = Path(__file__).resolve().parent / "golden"
ROUND = {torch.bfloat16: gdn.bf16_round, torch.float16: lambda t: np.asarray(t, np.float16).astype(np.float64),
         torch.float32: None}


def draw(seed, shape, dtype, w_dtype=torch.bfloat16):
    rng = np.random.default_rng(seed)
    D = shape[-1]
    scale = 10.0 ** rng.uniform(-2, 2, shape[:-1] + (1,))
    x = torch.tensor(rng.standard_normal(shape) * scale).to(dtype)
    gate = torch.tensor(rng.normal(0.0, 2.0, shape)).to(dtype)
    w = torch.tensor(rng.normal(1.0, 0.25, D)).to(w_dtype) if w_dtype is not None else None
    return x, gate, w


def oracle(x, gate, w, eps=1e-6):
    rnd = ROUND[x.dtype]
    w_np = None if w is None else w.double().numpy()
    return gdn.gated_rms_norm(x.double().numpy(), gate.double().numpy(), w_np, eps, round_fn=rnd,
                              weight_rounds=w is not None and w.dtype == x.dtype)


def run(x, gate, w, **kw):
    out = mx.gated_rms_norm(x.to(DEV), gate.to(DEV), None if w is None else w.to(DEV), 1e-6, **kw)
    torch.cuda.synchronize()
    return out.cpu()


def test_matches_library_fixture():
    z = np.load(GOLD / "gated_norm_small.npz")
    x = torch.tensor(z["x"]).to(torch.bfloat16)
    gate = torch.tensor(z["gate"]).to(torch.bfloat16)
    w = torch.tensor(z["weight"])
    got = run(x, gate, w.to(torch.bfloat16)).float().numpy()
    assert np.mean(got == z["out_bf16_wbf16"]) > 0.99 and rel_err(got, z["out_bf16_wbf16"]) <= Y_TOL
    got = run(x, gate, w).float().numpy()
    assert np.mean(got == z["out_bf16_wf32"]) > 0.99 and rel_err(got, z["out_bf16_wf32"]) <= Y_TOL
    got = run(x.float(), gate.float(), w).numpy()
    assert rel_err(got, z["out_f32"]) < 1e-5


@pytest.mark.parametrize("D", [64, 128, 256])
@pytest.mark.parametrize("dtype,w_dtype", [(torch.bfloat16, torch.bfloat16), (torch.bfloat16, torch.float32),
                                           (torch.float16, torch.float16), (torch.float32, torch.float32),
                                           (torch.bfloat16, None)])
def test_against_oracle(D, dtype, w_dtype):
    # 3 x 5 x 7 rows: not a multiple of the rows a workgroup covers
    x, gate, w = draw(40 + D, (3, 5, 7, D), dtype, w_dtype)
    got = run(x, gate, w).double().numpy()
    ref = oracle(x, gate, w)
    tol = 1e-5 if dtype == torch.float32 else Y_TOL
    assert rel_err(got, ref) <= tol
    if dtype != torch.float32:
        assert np.mean(got == ref) > 0.99


def test_mixer_shape_decode_and_prefill_rows():
    for rows in (64 * 32, 4096 * 32 + 32):
        x, gate, w = draw(rows, (rows, 128), torch.bfloat16)
        got = run(x, gate, w).double().numpy()
        ref = oracle(x, gate, w)
        assert rel_err(got, ref) <= Y_TOL and np.mean(got == ref) > 0.99


def test_in_place_and_empty():
    x, gate, w = draw(7, (33, 128), torch.bfloat16)
    ref = run(x, gate, w)
    xd = x.to(DEV)
    out = mx.gated_rms_norm(xd, gate.to(DEV), w.to(DEV), 1e-6, out=xd)
    torch.cuda.synchronize()
    assert out.data_ptr() == xd.data_ptr()
    assert torch.equal(out.cpu(), ref)
    empty = mx.gated_rms_norm(torch.empty(0, 128, dtype=torch.bfloat16, device=DEV),
                              torch.empty(0, 128, dtype=torch.bfloat16, device=DEV), w.to(DEV))
    assert empty.shape == (0, 128)


def test_rejects_bad_arguments():
    x = torch.zeros(4, 96, dtype=torch.bfloat16, device=DEV)
    with pytest.raises(ValueError):
        mx.gated_rms_norm(x, x, None)                                    # D = 96 not built
    x = torch.zeros(4, 128, dtype=torch.bfloat16, device=DEV)
    with pytest.raises(ValueError):
        mx.gated_rms_norm(x, x.float(), None)                            # dtype mismatch
    with pytest.raises(ValueError):
        mx.gated_rms_norm(x, x, torch.ones(64, device=DEV))              # weight size


def test_prepared_launch_equals_call():
    x, gate, w = draw(9, (5, 32, 128), torch.bfloat16)
    xd, gd, wd = x.to(DEV), gate.to(DEV), w.to(DEV)
    plan = mx.prepare_gated_rms_norm(xd, gd, wd)
    plan.launch()
    ref = mx.gated_rms_norm(xd, gd, wd)
    torch.cuda.synchronize()
    assert torch.equal(plan.outputs[0], ref)
    with pytest.raises(ValueError):
        mx.prepare_gated_rms_norm(xd.transpose(0, 1), gd.transpose(0, 1), wd)
