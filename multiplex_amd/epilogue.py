"""Mixer epilogue on MI355X: the gated RMSNorm (``libgdn.so`` ``gdn_gated_rmsnorm``).

The mixer multiplex restates ends with ``out = self_layer.norm(out, z)`` and
``out = self_layer.out_proj(out.reshape(B, S, -1))``
(``multiplex/kernel/dflash.py:377-378``).  The norm runs here as one HIP
launch that reads ``out`` and ``z`` once and writes the normalised, gated
rows once, in the ``[B, S, Hv*Dv]`` layout out_proj reads.  out_proj stays a
library GEMM (hipBLASLt through ``torch.nn.functional.linear``).
"""

from __future__ import annotations

from typing import Optional

import torch

from . import _lib
from .gated_delta import PreparedCall, _dtype_code, _ptr, _require_device, _stream

__all__ = ["gated_rms_norm", "prepare_gated_rms_norm"]


def _gate_lines(gate: torch.Tensor, D: int):
    """``(gate, gate_group, gate_stride)``: a gate ``[..., G, D]`` whose rows
    are D contiguous elements, G rows per line, lines one stride apart (a
    column slice of a fused in_proj output) is read in place; anything else
    is made contiguous (group 0)."""
    if gate.is_contiguous() or gate.dim() < 3:
        return gate.contiguous(), 0, 0
    G = gate.shape[-2]
    if gate.stride(-1) != 1 or gate.stride(-2) != D:
        return gate.contiguous(), 0, 0
    lead = [i for i in range(gate.dim() - 2) if gate.shape[i] > 1]
    ld = gate.stride(lead[-1]) if lead else G * D
    expect = ld
    for i in reversed(lead):
        if gate.stride(i) != expect:
            return gate.contiguous(), 0, 0
        expect *= gate.shape[i]
    if ld < G * D or (ld * gate.element_size()) % 16 != 0 or gate.data_ptr() % 16 != 0:
        return gate.contiguous(), 0, 0
    return gate, G, ld


def _norm_args(x, gate, weight, eps, out):
    dev = _require_device([x, gate, weight, out], ["x", "gate", "weight", "out"])
    if gate.shape != x.shape:
        raise ValueError(f"gate has shape {tuple(gate.shape)}, expected {tuple(x.shape)}")
    if gate.dtype != x.dtype:
        raise ValueError(f"gate has dtype {gate.dtype}, expected {x.dtype}")
    if x.dim() < 1:
        raise ValueError("x must have a last (normalised) dimension")
    D = x.shape[-1]
    io = _dtype_code(x, "x")
    wdt = _lib.DTYPE_F32
    if weight is not None:
        if tuple(weight.shape) != (D,):
            raise ValueError(f"weight must be [{D}] (got {tuple(weight.shape)})")
        wdt = _dtype_code(weight, "weight")
        weight = weight.contiguous()
    if out is None:
        out = torch.empty(x.shape, dtype=x.dtype, device=dev)
    elif out.shape != x.shape or out.dtype != x.dtype or not out.is_contiguous():
        raise ValueError("out must be a contiguous tensor of x's shape and dtype")
    x = x.contiguous()
    gate, g_group, g_ld = _gate_lines(gate, D)
    rows = x.numel() // D if D > 0 else 0
    args = (_ptr(x), _ptr(gate), io, g_group, g_ld, _ptr(weight), wdt, _ptr(out), rows, D, float(eps), _stream(dev))
    return args, dict(x=x, gate=gate, weight=weight), out, dev


def gated_rms_norm(x: torch.Tensor, gate: torch.Tensor, weight: Optional[torch.Tensor] = None,
                   eps: float = 1e-6, *, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """``(weight * rms_norm(x)) * silu(gate)`` over the last dim.

    x and gate share shape ``[..., D]`` (D in 64, 128, 256) and dtype
    (float32, bfloat16 or float16); weight is ``[D]`` or None (ones).
    Rounding follows transformers' ``Qwen3NextRMSNormGated``
    (``models/qwen3_next/modeling_qwen3_next.py:57-74``): the normalised value
    is rounded to x's dtype, so is its product with a weight of that dtype,
    and the gate product is rounded once.  ``out`` (same shape and dtype,
    contiguous) may be x.  The gate may be a column slice of a wider buffer
    (``[..., G, D]`` rows of D contiguous channels, lines of G rows one stride
    apart, as a fused in_proj output gives); it is then read in place.
    """
    args, _, out, _ = _norm_args(x, gate, weight, eps, out)
    _lib.call("gdn_gated_rmsnorm", *args)
    return out


def prepare_gated_rms_norm(x: torch.Tensor, gate: torch.Tensor, weight: Optional[torch.Tensor] = None,
                           eps: float = 1e-6, *, out: Optional[torch.Tensor] = None) -> PreparedCall:
    """Validates :func:`gated_rms_norm` once; ``launch()`` re-issues it.

    The tensors are bound by address (x contiguous; the gate contiguous or
    lines of rows as :func:`gated_rms_norm` accepts), so the launch reads the
    caller's buffers; ``outputs`` is ``(out,)``.
    """
    if not x.is_contiguous():
        raise ValueError("prepare_gated_rms_norm binds x by address: pass a contiguous x")
    args, keep, out, dev = _norm_args(x, gate, weight, eps, out)
    if keep["gate"].data_ptr() != gate.data_ptr():
        raise ValueError("prepare_gated_rms_norm binds the gate by address: pass it contiguous or as lines of rows")
    return PreparedCall("gdn_gated_rmsnorm", args, keep, (out,), dev)
