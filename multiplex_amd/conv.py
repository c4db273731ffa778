"""Fused GatedDeltaNet prologue on MI355X (``libgdn.so`` ``gdn_conv_prologue``).

Replaces the prologue of the mixer that multiplex restates at
``multiplex/kernel/dflash.py:351-370``: mask zeroing of the mixed qkv
projection, ``concat(conv_state, qkv)``, depthwise causal conv1d (4 taps, no
bias) + SiLU, the q | k | v split, ``q = rms_norm(q) / Dk`` and
``k = rms_norm(k) / sqrt(Dk)``, and the conv-state update -- in one launch
that reads each input element once.
"""

from __future__ import annotations

from typing import Optional

import torch

from . import _lib
from .gated_delta import (CHUNK, IntSeq, PreparedCall, _contig, _cu_seqlens, _dtype_code, _gate_codes, _gate_pair,
                          _int_rows, _mask_u8, _param_codes, _ptr, _require_device, _state_operands, _stream,
                          _token_rows)

__all__ = ["gdn_conv_prologue", "prepare_conv_prologue", "conv_state_commit", "gdn_conv_chunked",
           "prepare_conv_chunked", "conv_chunk_workspace_bytes"]


def _weight_2d(conv_weight: torch.Tensor, C: int) -> torch.Tensor:
    """Accepts mlx-lm's ``[C, K, 1]``, torch's ``[C, 1, K]`` or plain ``[C, K]`` taps."""
    w = conv_weight
    if w.dim() == 3:
        if w.shape[2] == 1:
            w = w[:, :, 0]
        elif w.shape[1] == 1:
            w = w[:, 0, :]
        else:
            raise ValueError(f"conv weight of shape {tuple(conv_weight.shape)} is not depthwise")
    if w.dim() != 2 or w.shape[0] != C:
        raise ValueError(f"conv weight must be [C={C}, K] (got {tuple(conv_weight.shape)})")
    return w.contiguous()


def _qkv_rows(qkv: torch.Tensor, C: int):
    """``(qkv, qkv_stride)``: a column slice of a wider row-major buffer (e.g.
    a fused in_proj output) is read in place when its rows stay 16-byte
    aligned; anything else is made contiguous (stride 0)."""
    ld = _token_rows(qkv, C)
    if ld is not None and (ld * qkv.element_size()) % 16 == 0 and qkv.data_ptr() % 16 == 0:
        return qkv, (0 if ld == C else ld)
    return qkv.contiguous(), 0


def _prologue_args(qkv, conv_weight, num_k_heads, num_v_heads, head_k_dim, head_v_dim, conv_state, mask,
                   cu_seqlens, eps, write_conv_state, conv_state_out=None):
    dev = _require_device([qkv, conv_weight, conv_state, mask], ["qkv", "conv_weight", "conv_state", "mask"])
    if qkv.dim() != 3:
        raise ValueError("qkv must be [B, S, C]")
    B, S, C = qkv.shape
    Hk, Hv, Dk, Dv = int(num_k_heads), int(num_v_heads), int(head_k_dim), int(head_v_dim)
    if C != 2 * Hk * Dk + Hv * Dv:
        raise ValueError(f"qkv has {C} channels, expected 2*{Hk}*{Dk} + {Hv}*{Dv}")
    w = _weight_2d(conv_weight, C)
    Kt = w.shape[1]
    io = _dtype_code(qkv, "qkv")
    wdt = _dtype_code(w, "conv_weight")
    cu = _cu_seqlens(cu_seqlens, S, dev) if cu_seqlens is not None else None
    if cu is not None and B != 1:
        raise ValueError("packed sequences need qkv of shape [1, N_tok, C]")
    n_rows = (cu.numel() - 1) if cu is not None else B
    in_place = conv_state_out is not None and conv_state is not None and conv_state_out is conv_state
    if conv_state is not None:
        if tuple(conv_state.shape) != (n_rows, Kt - 1, C) or conv_state.dtype != qkv.dtype:
            raise ValueError(f"conv_state must be {(n_rows, Kt - 1, C)} of dtype {qkv.dtype}")
        if in_place and not conv_state.is_contiguous():
            raise ValueError("an in-place conv state update needs a contiguous conv_state")
        conv_state = conv_state.contiguous()
    if conv_state_out is not None:
        if not write_conv_state:
            raise ValueError("conv_state_out given with write_conv_state=False")
        if (tuple(conv_state_out.shape) != (n_rows, Kt - 1, C) or conv_state_out.dtype != qkv.dtype
                or not conv_state_out.is_contiguous() or conv_state_out.device != qkv.device):
            raise ValueError(f"conv_state_out must be a contiguous {(n_rows, Kt - 1, C)} tensor of dtype {qkv.dtype}")
        if in_place and (cu is not None or S > 1):
            raise ValueError("the conv state is updated in place only for unpacked rows of one token")
    m = _mask_u8(mask, (B, S))
    qkv, ld = _qkv_rows(qkv, C)
    q = torch.empty(B, S, Hk, Dk, dtype=qkv.dtype, device=dev)
    k = torch.empty(B, S, Hk, Dk, dtype=qkv.dtype, device=dev)
    v = torch.empty(B, S, Hv, Dv, dtype=qkv.dtype, device=dev)
    if conv_state_out is not None:
        cs_out = conv_state_out
    else:
        cs_out = torch.empty(n_rows, Kt - 1, C, dtype=qkv.dtype, device=dev) if write_conv_state else None
    args = (_ptr(qkv), io, ld, _ptr(conv_state), _ptr(w), wdt, _ptr(m), _ptr(cu), _ptr(q), _ptr(k), _ptr(v),
            _ptr(cs_out), n_rows, S, Hk, Hv, Dk, Dv, Kt, float(eps), _stream(dev))
    keep = dict(qkv=qkv, conv_state=conv_state, w=w, mask=m, cu=cu)
    return args, keep, (q, k, v, cs_out), dev


def gdn_conv_prologue(qkv: torch.Tensor, conv_weight: torch.Tensor, num_k_heads: int,
                      num_v_heads: int, head_k_dim: int, head_v_dim: int,
                      conv_state: Optional[torch.Tensor] = None, mask: Optional[torch.Tensor] = None,
                      *, cu_seqlens: Optional[IntSeq] = None, eps: float = 1e-6,
                      write_conv_state: bool = True, conv_state_out: Optional[torch.Tensor] = None):
    """Returns ``(q, k, v, new_conv_state)``.

    qkv ``[B,S,C]`` (C = 2*Hk*Dk + Hv*Dv, channels q | k | v), conv_weight
    ``[C,K]`` (or ``[C,K,1]`` / ``[C,1,K]``), conv_state ``[B,K-1,C]`` or None
    (zeros), mask ``[B,S]`` or None.  q, k are ``[B,S,Hk,Dk]``, v is
    ``[B,S,Hv,Dv]``, all in qkv's dtype; the new conv state is the last K-1
    rows of ``concat(conv_state, masked qkv)`` (None if not requested).
    With ``cu_seqlens`` the rows are packed ragged sequences (``B == 1``) and
    conv_state has one row per sequence.  ``conv_state_out`` receives the
    new conv state (default: a new tensor); it may be ``conv_state`` itself
    (updated in place) for unpacked rows of one token (decode).
    """
    args, _keep, outs, dev = _prologue_args(qkv, conv_weight, num_k_heads, num_v_heads, head_k_dim, head_v_dim,
                                            conv_state, mask, cu_seqlens, eps, write_conv_state, conv_state_out)
    with torch.cuda.device(dev):
        _lib.call("gdn_conv_prologue", *args)
    return outs


def prepare_conv_prologue(qkv: torch.Tensor, conv_weight: torch.Tensor, num_k_heads: int,
                          num_v_heads: int, head_k_dim: int, head_v_dim: int,
                          conv_state: Optional[torch.Tensor] = None, mask: Optional[torch.Tensor] = None,
                          *, cu_seqlens: Optional[IntSeq] = None, eps: float = 1e-6,
                          write_conv_state: bool = True) -> PreparedCall:
    """Validates the prologue once; ``launch()`` re-issues it (``outputs`` = ``(q, k, v, conv_state)``).

    qkv must be contiguous or a column slice with one row stride (it is bound
    by address, so refill it in place).
    """
    args, keep, outs, dev = _prologue_args(qkv, conv_weight, num_k_heads, num_v_heads, head_k_dim,
                                           head_v_dim, conv_state, mask, cu_seqlens, eps, write_conv_state)
    if keep["qkv"].data_ptr() != qkv.data_ptr():
        raise ValueError("qkv must be contiguous (or a one-stride column slice) for a prepared launch")
    keep.update(q=outs[0], k=outs[1], v=outs[2], cs_out=outs[3])
    return PreparedCall("gdn_conv_prologue", args, keep, outs, dev)


def conv_state_commit(conv_state: Optional[torch.Tensor], qkv: torch.Tensor, n_commit: IntSeq,
                      mask: Optional[torch.Tensor] = None, kernel_size: int = 4) -> torch.Tensor:
    """Conv state after the accepted prefix of a verify (``dflash.py:424-425``).

    ``new[b] = concat(conv_state[b], masked qkv[b])[n : n + K - 1]`` with
    ``n = n_commit[b]``.  qkv ``[B,T,C]`` is the verify's mixed projection.
    """
    dev = _require_device([conv_state, qkv, mask], ["conv_state", "qkv", "mask"])
    B, T, C = qkv.shape
    Kt = int(kernel_size)
    if conv_state is not None:
        if tuple(conv_state.shape) != (B, Kt - 1, C) or conv_state.dtype != qkv.dtype:
            raise ValueError(f"conv_state must be {(B, Kt - 1, C)} of dtype {qkv.dtype}")
        conv_state = conv_state.contiguous()
    io = _dtype_code(qkv, "qkv")
    n = _int_rows(n_commit, B, dev, "n_commit")
    m = _mask_u8(mask, (B, T))
    out = torch.empty(B, Kt - 1, C, dtype=qkv.dtype, device=dev)
    ld = _token_rows(qkv, C)
    if ld is None:
        qkv, ld = qkv.contiguous(), C
    with torch.cuda.device(dev):
        _lib.call("gdn_conv_state_commit", _ptr(conv_state), _ptr(qkv), io, ld, _ptr(m), _ptr(n), _ptr(out),
                  B, T, C, Kt, _stream(dev))
    return out


def conv_chunk_workspace_bytes(n_seqs: int, n_tok: int, Hv: int, Dk: int, Dv: int, chunk: int = CHUNK) -> int:
    """Workspace bytes of :func:`gdn_conv_chunked` (the chunk records, then v)."""
    return int(_lib.load().gdn_chunk_conv_workspace_bytes(n_seqs, n_tok, Hv, Dk, Dv, chunk))


def _conv_chunked_args(qkv, conv_weight, num_k_heads, num_v_heads, head_k_dim, head_v_dim, a, b, A_log, dt_bias,
                       state, conv_state, cu_seqlens, eps, state_out, workspace, state_index, write_conv_state):
    dev = _require_device([qkv, conv_weight, a, b, A_log, dt_bias, state, conv_state, state_out],
                          ["qkv", "conv_weight", "a", "b", "A_log", "dt_bias", "state", "conv_state", "state_out"])
    if qkv.dim() != 3 or qkv.dtype != torch.bfloat16:
        raise ValueError("qkv must be [B, S, C] bf16")
    B, S, C = qkv.shape
    Hk, Hv, Dk, Dv = int(num_k_heads), int(num_v_heads), int(head_k_dim), int(head_v_dim)
    if C != 2 * Hk * Dk + Hv * Dv:
        raise ValueError(f"qkv has {C} channels, expected 2*{Hk}*{Dk} + {Hv}*{Dv}")
    if Hv % Hk != 0:
        raise ValueError(f"Hv={Hv} must be a multiple of Hk={Hk}")
    w = _weight_2d(conv_weight, C)
    if w.shape[1] != 4:
        raise ValueError("the fused prologue is built for 4 conv taps")
    wdt = _dtype_code(w, "conv_weight")
    for g, name in ((a, "a"), (b, "b")):
        if tuple(g.shape) != (B, S, Hv):
            raise ValueError(f"{name} has shape {tuple(g.shape)}, expected {(B, S, Hv)}")
    packed = cu_seqlens is not None
    if packed and B != 1:
        raise ValueError("packed sequences need qkv of shape [1, N_tok, C]")
    cu = _cu_seqlens(cu_seqlens, S, dev)
    n_seqs = (cu.numel() - 1) if packed else B
    if conv_state is not None:
        if tuple(conv_state.shape) != (n_seqs, 3, C) or conv_state.dtype != qkv.dtype:
            raise ValueError(f"conv_state must be {(n_seqs, 3, C)} of dtype {qkv.dtype}")
        conv_state = conv_state.contiguous()
    qkv, ld = _qkv_rows(qkv, C)
    gx, gy, g_ld = _gate_pair(a, b, Hv)
    gate_code = _gate_codes(gx, gy)
    param_code = _param_codes(A_log, dt_bias, Hv)
    A_log, dt_bias = _contig(A_log), _contig(dt_bias)
    n_tok = B * S
    state, out_state, idx, n_slots = _state_operands(state, state_out, True, n_seqs, Hv, Dv, Dk, dev, state_index)
    y = torch.empty(B, S, Hv, Dv, dtype=qkv.dtype, device=dev)
    cs_out = torch.empty(n_seqs, 3, C, dtype=qkv.dtype, device=dev) if write_conv_state else None
    ws_bytes = conv_chunk_workspace_bytes(n_seqs, n_tok, Hv, Dk, Dv, CHUNK)
    if workspace is None or workspace.numel() * workspace.element_size() < ws_bytes:
        workspace = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=dev)
    args = (_ptr(qkv), ld, _ptr(w), wdt, _ptr(conv_state), _ptr(cs_out), float(eps), _lib.GATES_RAW, _ptr(gx),
            _ptr(gy), gate_code, g_ld, _ptr(A_log), _ptr(dt_bias), param_code, _ptr(state), _ptr(y), _ptr(out_state),
            _ptr(idx), n_slots, _ptr(cu), n_seqs, n_tok, Hk, Hv, Dk, Dv, CHUNK, _ptr(workspace), ws_bytes,
            _stream(dev))
    keep = dict(qkv=qkv, w=w, conv_state=conv_state, gx=gx, gy=gy, A_log=A_log, dt_bias=dt_bias, state=state,
                cu=cu, workspace=workspace, state_index=idx, y=y, state_out=out_state, cs_out=cs_out)
    return args, keep, (y, out_state, cs_out), dev


def gdn_conv_chunked(qkv: torch.Tensor, conv_weight: torch.Tensor, num_k_heads: int, num_v_heads: int,
                     head_k_dim: int, head_v_dim: int, a: torch.Tensor, b: torch.Tensor, A_log: torch.Tensor,
                     dt_bias: torch.Tensor, state: Optional[torch.Tensor] = None,
                     conv_state: Optional[torch.Tensor] = None, *, cu_seqlens: Optional[IntSeq] = None,
                     eps: float = 1e-6, state_out: Optional[torch.Tensor] = None, workspace=None,
                     state_index=None, write_conv_state: bool = True):
    """The prefill of the mixer from its mixed projection: the conv prologue
    (``dflash.py:351-370``) fused into the chunked pass's prep
    (``gdn_chunk_fwd_conv``), then the chunked gated delta rule
    (``dflash.py:372-374``).  Returns ``(y, new_state, new_conv_state)``.

    Equal bit for bit to :func:`gdn_conv_prologue` followed by
    ``gated_delta_update(..., chunked=True)``, without writing q, k and v
    (only v, into the workspace, for the scan).  qkv ``[B, S, C]`` bf16 (or a
    one-stride column slice of a fused in_proj output), no mask; a, b
    ``[B, S, Hv]``; Dk = Dv = 128; other arguments as in those two
    functions.
    """
    args, _keep, outs, dev = _conv_chunked_args(qkv, conv_weight, num_k_heads, num_v_heads, head_k_dim,
                                                head_v_dim, a, b, A_log, dt_bias, state, conv_state, cu_seqlens,
                                                eps, state_out, workspace, state_index, write_conv_state)
    with torch.cuda.device(dev):
        _lib.call("gdn_chunk_fwd_conv", *args)
    return outs


def prepare_conv_chunked(qkv, conv_weight, num_k_heads, num_v_heads, head_k_dim, head_v_dim, a, b, A_log, dt_bias,
                         state=None, conv_state=None, *, cu_seqlens=None, eps=1e-6, state_out=None, workspace=None,
                         state_index=None, write_conv_state=True) -> PreparedCall:
    """Validates :func:`gdn_conv_chunked` once; ``launch()`` re-issues it
    (``outputs`` = ``(y, new_state, new_conv_state)``).  The inputs are bound
    by address: qkv and the gates must be contiguous or one-stride column
    slices, refilled in place."""
    args, keep, outs, dev = _conv_chunked_args(qkv, conv_weight, num_k_heads, num_v_heads, head_k_dim,
                                               head_v_dim, a, b, A_log, dt_bias, state, conv_state, cu_seqlens, eps,
                                               state_out, workspace, state_index, write_conv_state)
    for name, given in (("qkv", qkv), ("gx", a), ("gy", b)):
        if keep[name].data_ptr() != given.data_ptr():
            raise ValueError(f"{name} must be contiguous or a one-stride column slice for a prepared launch")
    return PreparedCall("gdn_chunk_fwd_conv", args, keep, outs, dev)
