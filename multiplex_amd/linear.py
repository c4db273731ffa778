"""Decode-shape projections of the GatedDeltaNet mixer (``gdn_linear_decode``).

At decode a mixer layer's GEMMs have few rows (one token per batch row)
and are bound by reading their weights: in_proj's 12352 x 2048 and
out_proj's 2048 x 4096 bf16 matrices at hidden 2048 (``dflash.py:348-350,
377-378``).  ``gdn_linear_decode`` streams each weight once, split over
64-column tiles and 512-wide K slices, for 1..64 rows, and can fold the
epilogue's gated RMSNorm (``norm(out, z)``) into out_proj's operand load,
so the norm's output is never written.

Graph-replayed against the separate norm kernel plus hipBLASLt at hidden
2048, the fused norm + out_proj takes 7.4-8.1 us against 12.6-13.4 us up to
16 rows, and loses beyond (11.4 against 10.9 us at 32 rows, 16.4 against
13.1 us at 64); the plain projection is 1-2 us slower than the library at
every row count.  So the mixer uses ``gated_norm_linear_decode`` up to
``FUSED_NORM_MAX_ROWS`` rows and the library elsewhere; ``linear_decode``
(the same kernel without the norm) is the unfused reference for tests.

The kernel sums its K slices through a workspace of fp32 partials and one
ticket per output tile; the tickets must start at zero and every call
leaves them zero, so one zero-initialised workspace serves every call of a
module on one stream (calls that overlap, on several streams, need one
each).
"""

from __future__ import annotations

from typing import Optional

import torch

from . import _lib
from .gated_delta import _dtype_code, _ptr, _require_device, _stream

__all__ = ["DECODE_MAX_ROWS", "FUSED_NORM_MAX_ROWS", "DecodeWorkspace", "linear_decode",
           "gated_norm_linear_decode", "linear_decode_workspace_bytes", "decode_shape_ok"]

DECODE_MAX_ROWS = 64
FUSED_NORM_MAX_ROWS = 16  # where the fused norm + projection beats the norm kernel plus the library GEMM
_K_SLICE = 512


def linear_decode_workspace_bytes(M: int, N: int, K: int) -> int:
    return int(_lib.load().gdn_linear_decode_workspace_bytes(M, N, K))


def decode_shape_ok(M: int, N: int, K: int) -> bool:
    """Shapes ``gdn_linear_decode`` takes: 1..64 rows, K a multiple of 512, N of 8."""
    return 1 <= M <= DECODE_MAX_ROWS and K >= _K_SLICE and K % _K_SLICE == 0 and N % 8 == 0 and N > 0


class DecodeWorkspace:
    """A zero-initialised device buffer, grown (and zeroed again) on demand.

    Growing allocates, so a call under HIP graph capture must find the
    buffer already large enough: run the step once eagerly first.
    """

    def __init__(self):
        self.buf: Optional[torch.Tensor] = None

    def get(self, nbytes: int, device: torch.device) -> torch.Tensor:
        if self.buf is None or self.buf.device != device or self.buf.numel() < nbytes:
            self.buf = torch.zeros(nbytes, dtype=torch.uint8, device=device)
        return self.buf


def _rows(t: torch.Tensor, width: int, what: str) -> int:
    """Row stride (elements) of a ``[M, width]`` matrix with contiguous,
    16-byte aligned rows (e.g. a column slice of a wider buffer)."""
    if t.dim() != 2 or t.shape[1] != width or t.stride(1) != 1:
        raise ValueError(f"{what} must be [M, {width}] with contiguous rows")
    ld = t.stride(0) if t.shape[0] > 1 else width
    if ld < width or ld % 8 != 0 or t.data_ptr() % 16 != 0:
        raise ValueError(f"{what}: rows must be 16-byte aligned and a multiple of 8 elements apart")
    return int(ld)


def _launch(x, gate, norm_weight, eps, head_dim, weight, out, workspace):
    if x.dtype != torch.bfloat16 or weight.dtype != torch.bfloat16:
        raise ValueError("gdn_linear_decode takes bf16 activations and weights")
    M, K = x.shape
    N = weight.shape[0]
    if weight.dim() != 2 or weight.shape[1] != K or not weight.is_contiguous():
        raise ValueError(f"weight must be a contiguous [N, {K}] matrix")
    if not decode_shape_ok(M, N, K):
        raise ValueError(f"gdn_linear_decode takes 1..{DECODE_MAX_ROWS} rows, K a multiple of 512 and N of 8 "
                         f"(got M={M}, N={N}, K={K})")
    dev = _require_device([x, gate, norm_weight, weight, out], ["x", "gate", "norm_weight", "weight", "out"])
    ldx = _rows(x, K, "x")
    ldg = _rows(gate, K, "gate") if gate is not None else 0
    if out is None:
        out = torch.empty(M, N, dtype=torch.bfloat16, device=dev)
    ldo = _rows(out, N, "out")
    need = linear_decode_workspace_bytes(M, N, K)
    ws = (workspace if workspace is not None else DecodeWorkspace()).get(need, dev)
    nw_dt = _dtype_code(norm_weight, "norm_weight") if norm_weight is not None else 0
    _lib.call("gdn_linear_decode", _ptr(x), ldx, _ptr(gate), ldg, _ptr(norm_weight), nw_dt, float(eps),
              int(head_dim), _ptr(weight), _ptr(out), ldo, M, N, K, _ptr(ws), ws.numel(), _stream(dev))
    return out


def linear_decode(x: torch.Tensor, weight: torch.Tensor, *, out: Optional[torch.Tensor] = None,
                  workspace: Optional[DecodeWorkspace] = None) -> torch.Tensor:
    """``x @ weight.T`` for ``x [M <= 64, K]`` (rows may be a column slice)."""
    return _launch(x, None, None, 0.0, 0, weight, out, workspace)


def gated_norm_linear_decode(y: torch.Tensor, z: torch.Tensor, norm_weight: Optional[torch.Tensor], eps: float,
                             head_dim: int, weight: torch.Tensor, *, out: Optional[torch.Tensor] = None,
                             workspace: Optional[DecodeWorkspace] = None) -> torch.Tensor:
    """``gated_rms_norm(y, z, norm_weight, eps) @ weight.T`` per head of
    ``head_dim`` (64 or 128) columns, with the norm computed inside the
    projection's operand load (gdn_gated_rmsnorm's rounding points).
    y, z ``[M, K]``."""
    if z.dtype != torch.bfloat16:
        raise ValueError("z must be bf16")
    if norm_weight is not None:
        if tuple(norm_weight.shape) != (head_dim,):
            raise ValueError(f"norm_weight must be [{head_dim}]")
        norm_weight = norm_weight.contiguous()
    return _launch(y, z, norm_weight, eps, head_dim, weight, out, workspace)
