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
    gate = gate.contiguous()
    rows = x.numel() // D if D > 0 else 0
    args = (_ptr(x), _ptr(gate), io, _ptr(weight), wdt, _ptr(out), rows, D, float(eps), _stream(dev))
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
    contiguous) may be x or gate.
    """
    args, _, out, _ = _norm_args(x, gate, weight, eps, out)
    _lib.call("gdn_gated_rmsnorm", *args)
    return out


def prepare_gated_rms_norm(x: torch.Tensor, gate: torch.Tensor, weight: Optional[torch.Tensor] = None,
                           eps: float = 1e-6, *, out: Optional[torch.Tensor] = None) -> PreparedCall:
    """Validates :func:`gated_rms_norm` once; ``launch()`` re-issues it.

    The tensors are bound by address (x and gate must already be contiguous,
    so the launch reads the caller's buffers); ``outputs`` is ``(out,)``.
    """
    if not (x.is_contiguous() and gate.is_contiguous()):
        raise ValueError("prepare_gated_rms_norm binds x and gate by address: pass contiguous tensors")
    args, keep, out, dev = _norm_args(x, gate, weight, eps, out)
    return PreparedCall("gdn_gated_rmsnorm", args, keep, (out,), dev)
