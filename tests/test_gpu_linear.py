"""GPU checks of the decode-shape projections (``gdn_linear_decode``).

* plain projections against float64 products of the same bf16 operands,
  rounded to bf16: only the fp32 accumulation order differs, which moves a
  small fraction of outputs across a bf16 rounding boundary (held to 1e-3
  norm-wise);
* the gated RMSNorm folded into out_proj against the oracle's gated norm
  (gdn_gated_rmsnorm's rounding points) and a float64 product (2e-3, the
  mixer output's contract), and against the separate norm kernel followed
  by the same projection;
* the K slices are summed by whichever workgroup of a tile finishes last,
  in slice order: 30 launches give bit-identical results, a HIP graph of
  the call replays bit for bit (the tile tickets reset themselves), and one
  workspace serves calls of different shapes.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import multiplex_amd as mx
from multiplex_amd import linear as lin
from gdn_cases import rel_err
from oracle import gdn

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _bf16(gen, *shape, scale=1.0):
    return (torch.randn(*shape, generator=gen) * scale).to(torch.bfloat16)


def _np(t):
    return t.detach().double().cpu().numpy()


@pytest.mark.parametrize("M,N,K", [(64, 2048, 4096), (64, 12352, 2048), (1, 2048, 4096), (7, 136, 1024),
                                   (33, 8, 512)])
def test_linear_decode_matches_float64(M, N, K):
    gen = torch.Generator().manual_seed(M + N + K)
    x, W = _bf16(gen, M, K), _bf16(gen, N, K, scale=K ** -0.5)
    out = mx.linear_decode(x.to(DEV), W.to(DEV))
    torch.cuda.synchronize()
    ref = gdn.bf16_round(_np(x) @ _np(W).T)
    assert rel_err(_np(out), ref) <= 1e-3


def test_linear_decode_reads_column_slices_and_writes_strided_rows():
    """x a column slice of a wider buffer, out rows inside a wider buffer."""
    gen = torch.Generator().manual_seed(91)
    M, N, K = 20, 256, 1024
    xw = _bf16(gen, M, K + 64).to(DEV)
    W = _bf16(gen, N, K, scale=K ** -0.5).to(DEV)
    ow = torch.zeros(M, N + 32, dtype=torch.bfloat16, device=DEV)
    mx.linear_decode(xw[:, 64:], W, out=ow[:, :N])
    torch.cuda.synchronize()
    ref = gdn.bf16_round(_np(xw[:, 64:]) @ _np(W).T)
    assert rel_err(_np(ow[:, :N]), ref) <= 1e-3
    assert not ow[:, N:].any()


@pytest.mark.parametrize("M", [64, 24, 5])  # the three workgroup shapes
@pytest.mark.parametrize("hd,w_dtype", [(128, torch.bfloat16), (128, torch.float32), (64, torch.bfloat16),
                                        (64, None)])
def test_gated_norm_projection_matches_oracle_and_unfused_path(hd, w_dtype, M):
    gen = torch.Generator().manual_seed(92 + hd + M)
    N, K = 2048, 4096
    y, z = _bf16(gen, M, K, scale=3.0), _bf16(gen, M, K + 128, scale=2.0)[:, 128:]
    w = None if w_dtype is None else (torch.randn(hd, generator=gen) * 0.2 + 1.0).to(w_dtype)
    W = _bf16(gen, N, K, scale=K ** -0.5)
    dy, dz, dW = y.to(DEV), z.to(DEV), W.to(DEV)
    dw = None if w is None else w.to(DEV)
    out = mx.gated_norm_linear_decode(dy, dz, dw, 1e-6, hd, dW)
    torch.cuda.synchronize()
    yn = gdn.gated_rms_norm(_np(y).reshape(M, -1, hd), _np(z).reshape(M, -1, hd),
                            None if w is None else _np(w), 1e-6, round_fn=gdn.bf16_round,
                            weight_rounds=w_dtype == torch.bfloat16)
    ref = gdn.bf16_round(yn.reshape(M, K) @ _np(W).T)
    assert rel_err(_np(out), ref) <= 2e-3
    # the separate norm kernel, then the same projection
    normed = mx.gated_rms_norm(dy.view(M, -1, hd), dz.reshape(M, -1, hd).contiguous(), dw, 1e-6)
    out2 = mx.linear_decode(normed.view(M, K), dW)
    torch.cuda.synchronize()
    assert rel_err(_np(out), _np(out2)) <= 1e-3


def test_results_do_not_depend_on_which_slice_finishes_last():
    gen = torch.Generator().manual_seed(93)
    M, N, K = 64, 2048, 4096
    y, z = _bf16(gen, M, K).to(DEV), _bf16(gen, M, K).to(DEV)
    W = _bf16(gen, N, K, scale=K ** -0.5).to(DEV)
    w = torch.ones(128, dtype=torch.bfloat16, device=DEV)
    ws = mx.DecodeWorkspace()
    first = mx.gated_norm_linear_decode(y, z, w, 1e-6, 128, W, workspace=ws)
    for _ in range(30):
        assert torch.equal(mx.gated_norm_linear_decode(y, z, w, 1e-6, 128, W, workspace=ws), first)
    # the same workspace grows for a larger problem and keeps its tickets at zero
    x2, W2 = _bf16(gen, M, 2048).to(DEV), _bf16(gen, 12352, 2048, scale=2048 ** -0.5).to(DEV)
    a = mx.linear_decode(x2, W2, workspace=ws)
    b = mx.linear_decode(x2, W2, workspace=ws)
    assert torch.equal(a, b)
    assert torch.equal(mx.gated_norm_linear_decode(y, z, w, 1e-6, 128, W, workspace=ws), first)
    torch.cuda.synchronize()
    assert not ws.buf[:16384].any()  # the ticket region


def test_graph_replays_match_eager():
    gen = torch.Generator().manual_seed(94)
    M, N, K = 48, 2048, 4096
    y, z = _bf16(gen, M, K).to(DEV), _bf16(gen, M, K).to(DEV)
    W = _bf16(gen, N, K, scale=K ** -0.5).to(DEV)
    ws = mx.DecodeWorkspace()
    out = torch.empty(M, N, dtype=torch.bfloat16, device=DEV)
    eager = mx.gated_norm_linear_decode(y, z, None, 1e-6, 128, W, workspace=ws).clone()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        mx.gated_norm_linear_decode(y, z, None, 1e-6, 128, W, out=out, workspace=ws)
    for i in range(4):
        out.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"replay {i}"
        y.mul_(1.0)  # eager work between replays


def test_rejects_shapes_it_does_not_take():
    x = torch.zeros(65, 512, dtype=torch.bfloat16, device=DEV)
    W = torch.zeros(64, 512, dtype=torch.bfloat16, device=DEV)
    with pytest.raises(ValueError, match="rows"):
        mx.linear_decode(x, W)
    with pytest.raises(ValueError, match="multiple of 512"):
        mx.linear_decode(x[:8, :500], W[:, :500].contiguous())
