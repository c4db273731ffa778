"""Gated DeltaNet update on MI355X: the torch-facing mirror of mlx-lm's
``mlx_lm.models.gated_delta`` module, backed by ``libgdn.so``.

multiplex calls ``gated_delta_update(q, k, v, a, b, A_log, dt_bias, state,
mask, use_kernel=True)`` from the GatedDeltaNet mixer
(``multiplex/kernel/dflash.py:372-374``) and from its rollback replay
(``dflash.py:417-422``); the engine reaches the mixer through
``multiplex/kernel/engine.py:164-167``.  The same positional signature and
return value ``(y, new_state)`` are kept here; new capabilities are
keyword-only with defaults so unchanged callers keep working.

Semantics (as in mlx-lm): the call is functional -- ``state`` is never
mutated and a new state tensor is returned -- unless ``state_out=`` names a
destination (which may be ``state`` itself for in-place use).  ``state=None``
means a zero state.  A masked token keeps the state; its y is 0.

Every tensor must live on one ROCm device; there is no CPU path.
"""

from __future__ import annotations

from typing import Optional, Sequence, Union

import torch

from . import _lib

__all__ = [
    "compute_g",
    "compute_beta",
    "gated_delta_ops",
    "gated_delta_kernel",
    "gated_delta_update",
    "gated_delta_verify",
    "gated_delta_commit",
    "gated_delta_commit_verify",
    "chunk_workspace_bytes",
    "prepare_recurrent",
    "prepare_chunked",
    "PreparedRecurrent",
    "PreparedCall",
    "PreparedChunked",
    "CHUNK_MIN_TOKENS",
]

# Rows of at least this many tokens (bf16, Dk = 128, no mask) use the
# chunked MFMA kernel by default; shorter rows step the recurrent kernel.
# Measured on MI355X (Hv = 32): at 64 tokens the chunked pass takes 15.7 us
# against 31.9 us at B=1 and 36.7 against 55.6 us at B=8; at 32 tokens the
# two are within 20% either way.
CHUNK_MIN_TOKENS = 64
CHUNK = 64

_DT = {torch.float32: _lib.DTYPE_F32, torch.bfloat16: _lib.DTYPE_BF16, torch.float16: _lib.DTYPE_F16}

IntSeq = Union[Sequence[int], torch.Tensor]


# ----------------------------------------------------------------- helpers

def _ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


def _dtype_code(t: torch.Tensor, what: str) -> int:
    try:
        return _DT[t.dtype]
    except KeyError:
        raise ValueError(f"{what}: unsupported dtype {t.dtype} (float32, bfloat16, float16)") from None


def _require_device(tensors, names) -> torch.device:
    dev = None
    for t, n in zip(tensors, names):
        if t is None:
            continue
        if not isinstance(t, torch.Tensor):
            raise TypeError(f"{n} must be a torch.Tensor")
        if t.device.type != "cuda":
            raise ValueError(f"{n} is on {t.device}; the GDN kernels run on a ROCm device only")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise ValueError(f"{n} is on {t.device}, expected {dev}")
    if dev is None:
        raise ValueError("no device tensor given")
    return dev


def _contig(t: Optional[torch.Tensor]) -> Optional[torch.Tensor]:
    return None if t is None else t.contiguous()


def _token_rows(t: torch.Tensor, width: int):
    """Token stride (elements) of a ``[B, T, width]`` tensor whose rows are
    ``width`` contiguous elements with one stride from token to token (a
    column slice of a wider row-major buffer), or None if it is laid out
    otherwise."""
    if t.dim() != 3 or t.shape[2] != width or (width > 1 and t.stride(2) != 1):
        return None
    B, T = t.shape[0], t.shape[1]
    ld = t.stride(1) if T > 1 else (t.stride(0) if B > 1 else width)
    if ld < width or (B > 1 and T > 1 and t.stride(0) != T * ld):
        return None
    return int(ld)


def _gate_pair(gx: torch.Tensor, gy: torch.Tensor, Hv: int):
    """``(gx, gy, gate_stride)``: the gates as given when both are column
    slices with one token stride (e.g. of a fused in_proj output), else
    contiguous copies and stride 0."""
    lx, ly = _token_rows(gx, Hv), _token_rows(gy, Hv)
    if lx is not None and lx == ly:
        return gx, gy, (0 if lx == Hv else lx)
    return gx.contiguous(), gy.contiguous(), 0


def _stream_handle(stream) -> int:
    """A ``torch.cuda.Stream`` or a raw ``hipStream_t`` value."""
    return stream.cuda_stream if hasattr(stream, "cuda_stream") else int(stream)


def _stream(dev: torch.device) -> int:
    return torch.cuda.current_stream(dev).cuda_stream


def _mask_u8(mask: Optional[torch.Tensor], shape, what="mask") -> Optional[torch.Tensor]:
    if mask is None:
        return None
    if tuple(mask.shape) != tuple(shape):
        raise ValueError(f"{what} has shape {tuple(mask.shape)}, expected {tuple(shape)}")
    if mask.dtype == torch.bool:
        return mask.contiguous().view(torch.uint8)
    if mask.dtype == torch.uint8:
        return mask.contiguous()
    return (mask != 0).contiguous().view(torch.uint8)


def _check_state(state: Optional[torch.Tensor], shape, what="state"):
    if state is None:
        return None
    if state.dtype != torch.float32:
        raise ValueError(f"{what} must be float32 (got {state.dtype})")
    if tuple(state.shape) != tuple(shape):
        raise ValueError(f"{what} has shape {tuple(state.shape)}, expected {tuple(shape)}")
    return state.contiguous()


def _out_state(state_out, shape, dev, what="state_out"):
    if state_out is None:
        return torch.empty(shape, dtype=torch.float32, device=dev)
    if state_out.dtype != torch.float32 or tuple(state_out.shape) != tuple(shape):
        raise ValueError(f"{what} must be float32 of shape {tuple(shape)}")
    if not state_out.is_contiguous():
        raise ValueError(f"{what} must be contiguous")
    return state_out


def _state_operands(state, state_out, write_state, n_rows, Hv, Dv, Dk, dev, state_index):
    """``(state_in, state_out, index, n_slots)`` of a launch.

    Dense: ``[rows, Hv, Dv, Dk]`` states, one per row.  Pooled (``state_index``
    given): ``state`` / ``state_out`` are pools ``[n_slots, Hv, Dv, Dk]`` and
    row b uses slot ``state_index[b]``; the new states go to ``state_out``, or
    into the pool itself when it is None.
    """
    if state_index is None:
        st_shape = (n_rows, Hv, Dv, Dk)
        state = _check_state(state, st_shape)
        out_state = _out_state(state_out, st_shape, dev) if write_state else None
        return state, out_state, None, 0
    pool = state if state is not None else state_out
    if pool is None:
        raise ValueError("pooled states (state_index) need the pool as state or state_out")
    st_shape = (pool.shape[0], Hv, Dv, Dk)
    if state is not None and not state.is_contiguous():
        raise ValueError("the state pool must be contiguous")
    state = _check_state(state, st_shape, "state pool")
    out_state = None
    if write_state:
        out_state = _out_state(state_out if state_out is not None else state, st_shape, dev, "state_out pool")
    idx = _int_rows(state_index, n_rows, dev, "state_index", unique_slots=write_state)
    return state, out_state, idx, st_shape[0]


def _upload_i32(host: torch.Tensor, dev) -> torch.Tensor:
    """An int32 copy of a host tensor on ``dev``, enqueued on the current
    stream through pinned memory: the host does not wait for the device."""
    t = host.to(torch.int32).contiguous()
    if t.numel() == 0:
        return torch.empty(0, dtype=torch.int32, device=dev)
    return t.pin_memory().to(dev, non_blocking=True)


def _is_device(x, dev) -> bool:
    return isinstance(x, torch.Tensor) and x.device.type == "cuda"


def _cu_seqlens(cu: Optional[IntSeq], n_tok: int, dev) -> Optional[torch.Tensor]:
    """Packed-sequence offsets on ``dev``.

    Host offsets (a list or a CPU tensor) are validated -- they must start at
    0, be non-decreasing and end at ``n_tok`` -- and uploaded asynchronously.
    A device tensor is used as it is, with no host copy and so no
    synchronisation; the kernels clamp every sequence into ``[0, n_tok]``, so
    a bad device table yields wrong rows but no access outside the buffers.
    """
    if cu is None:
        return None
    if n_tok >= 2**31:
        raise ValueError("too many packed tokens")
    if _is_device(cu, dev):
        if cu.device != dev:
            raise ValueError(f"cu_seqlens is on {cu.device}, expected {dev}")
        if cu.dim() != 1 or cu.numel() < 2:
            raise ValueError("cu_seqlens must be a 1-D sequence of at least 2 offsets")
        if cu.dtype != torch.int32 or not cu.is_contiguous():
            cu = cu.to(torch.int32).contiguous()
        return cu
    host = torch.as_tensor(cu).to("cpu", torch.int64)
    if host.dim() != 1 or host.numel() < 2:
        raise ValueError("cu_seqlens must be a 1-D sequence of at least 2 offsets")
    if int(host[0]) != 0 or int(host[-1]) != n_tok:
        raise ValueError(f"cu_seqlens must start at 0 and end at {n_tok}")
    if bool((host[1:] < host[:-1]).any()):
        raise ValueError("cu_seqlens must be non-decreasing")
    return _upload_i32(host, dev)


def _packed_max_len(cu: IntSeq, n_tok: int, max_seqlen: Optional[int]) -> int:
    """Longest packed sequence, for choosing a kernel: exact for host
    offsets.  A device table is not read back (that would synchronise): with
    one sequence its length is ``n_tok``; with several the caller must give
    ``max_seqlen`` -- a length guessed from the mean would step one long
    prompt packed with many short ones through the recurrent kernel."""
    if _is_device(cu, None):
        if max_seqlen is not None:
            return int(max_seqlen)
        if cu.numel() <= 2:
            return n_tok
        raise ValueError("a device cu_seqlens of several sequences needs max_seqlen (its longest sequence) "
                         "or an explicit chunked=True / chunked=False to choose the kernel")
    host = torch.as_tensor(cu).to("cpu", torch.int64)
    return int((host[1:] - host[:-1]).max()) if host.numel() > 1 else 0


def _int_rows(x: IntSeq, n: int, dev, what: str, unique_slots: bool = False) -> torch.Tensor:
    """An int32 ``[n]`` row table on ``dev``.  Host tables are uploaded
    asynchronously; with ``unique_slots`` (the state slots of a launch that
    writes them) a host table may not name one slot twice, since two rows
    writing one slot would race.  Device tables are used as they are."""
    if _is_device(x, dev):
        if x.device != dev:
            raise ValueError(f"{what} is on {x.device}, expected {dev}")
        if x.dim() != 1 or x.numel() != n:
            raise ValueError(f"{what} must have {n} entries")
        return x.contiguous() if x.dtype == torch.int32 else x.to(torch.int32).contiguous()
    t = torch.as_tensor(x).to("cpu", torch.int64)
    if t.dim() != 1 or t.numel() != n:
        raise ValueError(f"{what} must have {n} entries")
    if unique_slots and n > 1:
        live = t[t >= 0]
        if live.numel() != torch.unique(live).numel():
            raise ValueError(f"{what} names a state slot twice; rows that write one slot would race")
    return _upload_i32(t, dev)


class _Shapes:
    """Validated problem shape of a (q, k, v, gates) set."""

    def __init__(self, q, k, v, gx, gy, packed: bool):
        if k.dim() != 4 or v.dim() != 4:
            raise ValueError("k and v must be 4-D: [B, T, H, D]")
        B, T, Hk, Dk = k.shape
        if q is not None and tuple(q.shape) != (B, T, Hk, Dk):
            raise ValueError(f"q has shape {tuple(q.shape)}, expected {(B, T, Hk, Dk)}")
        if v.shape[0] != B or v.shape[1] != T:
            raise ValueError("v must share the [B, T] leading dims of q/k")
        Hv, Dv = v.shape[2], v.shape[3]
        if Hv % Hk != 0:
            raise ValueError(f"Hv={Hv} must be a multiple of Hk={Hk}")
        for g, name in ((gx, "a/g"), (gy, "b/beta")):
            if tuple(g.shape) != (B, T, Hv):
                raise ValueError(f"{name} has shape {tuple(g.shape)}, expected {(B, T, Hv)}")
        dt = k.dtype
        for t, name in ((q, "q"), (v, "v")):
            if t is not None and t.dtype != dt:
                raise ValueError(f"q, k and v must share one dtype (k is {dt}, {name} is {t.dtype})")
        if packed and B != 1:
            raise ValueError("packed sequences (cu_seqlens) need a leading batch dim of 1")
        self.B, self.T, self.Hk, self.Dk, self.Hv, self.Dv = B, T, Hk, Dk, Hv, Dv


def _gate_codes(gx, gy):
    if gx.dtype != gy.dtype:
        raise ValueError(f"gates must share one dtype ({gx.dtype} vs {gy.dtype})")
    return _dtype_code(gx, "gates")


def _param_codes(A_log, dt_bias, Hv):
    if A_log.shape != (Hv,) or dt_bias.shape != (Hv,):
        raise ValueError(f"A_log and dt_bias must have shape ({Hv},)")
    if A_log.dtype != dt_bias.dtype:
        raise ValueError("A_log and dt_bias must share one dtype")
    return _dtype_code(A_log, "A_log/dt_bias")


# -------------------------------------------------------- gate transforms

def compute_g(A_log: torch.Tensor, a: torch.Tensor, dt_bias: torch.Tensor) -> torch.Tensor:
    """Decay ``g = exp(-exp(A_log) * softplus(a + dt_bias))`` in float32 (mlx-lm ``compute_g``)."""
    _require_device([A_log, a, dt_bias], ["A_log", "a", "dt_bias"])
    x = a.float() + dt_bias.float()
    return torch.exp(-torch.exp(A_log.float()) * torch.nn.functional.softplus(x))


def compute_beta(b: torch.Tensor) -> torch.Tensor:
    """Write strength ``beta = sigmoid(b)`` in float32."""
    _require_device([b], ["b"])
    return torch.sigmoid(b.float())


def gated_delta_ops(q, k, v, g, beta, state=None, mask=None):
    """The ops path of mlx-lm (``use_kernel=False``), as device torch ops.

    A step-by-step loop over T built from elementwise ops and reductions; it is
    the slow reference form that mlx-lm runs when its fused kernel is not
    used, kept for API parity.  It runs on the ROCm device like everything
    else here, never silently in place of the HIP kernel.
    """
    dev = _require_device([q, k, v, g, beta, state, mask], ["q", "k", "v", "g", "beta", "state", "mask"])
    sh = _Shapes(q, k, v, g, beta, packed=False)
    r = sh.Hv // sh.Hk
    qf = q.float().repeat_interleave(r, dim=2)
    kf = k.float().repeat_interleave(r, dim=2)
    vf = v.float()
    S = (torch.zeros(sh.B, sh.Hv, sh.Dv, sh.Dk, device=dev) if state is None
         else _check_state(state, (sh.B, sh.Hv, sh.Dv, sh.Dk)).clone())
    ys = []
    for t in range(sh.T):
        Sg = S * g[:, t, :, None, None].float()
        kv = (Sg * kf[:, t, :, None, :]).sum(-1)
        delta = (vf[:, t] - kv) * beta[:, t, :, None].float()
        Sn = Sg + kf[:, t, :, None, :] * delta[..., None]
        y = (Sn * qf[:, t, :, None, :]).sum(-1)
        if mask is not None:
            m = mask[:, t].bool()
            Sn = torch.where(m[:, None, None, None], Sn, S)
            y = torch.where(m[:, None, None], y, torch.zeros_like(y))
        S = Sn
        ys.append(y)
    y = torch.stack(ys, dim=1) if ys else torch.zeros(sh.B, 0, sh.Hv, sh.Dv, device=dev)
    return y.to(q.dtype), S


# ------------------------------------------------------------ HIP launches

def _recurrent(q, k, v, gx, gy, gate_mode, A_log, dt_bias, state, mask, *,
               y=True, state_out=None, write_state=True, snapshots=False,
               cu_seqlens=None, commit_len=None, state_index=None, y_from=0):
    names = ["q", "k", "v", "a/g", "b/beta", "A_log", "dt_bias", "state", "mask", "state_out"]
    dev = _require_device([q, k, v, gx, gy, A_log, dt_bias, state, mask, state_out], names)
    packed = cu_seqlens is not None
    sh = _Shapes(q, k, v, gx, gy, packed)
    q, k, v = (_contig(t) for t in (q, k, v))
    gx, gy, g_ld = _gate_pair(gx, gy, sh.Hv)
    qkv_code = _dtype_code(k, "q/k/v")
    gate_code = _gate_codes(gx, gy)
    if gate_mode == _lib.GATES_RAW:
        if A_log is None or dt_bias is None:
            raise ValueError("A_log and dt_bias are required")
        param_code = _param_codes(A_log, dt_bias, sh.Hv)
        A_log, dt_bias = _contig(A_log), _contig(dt_bias)
    else:
        param_code = _lib.DTYPE_F32
    cu = _cu_seqlens(cu_seqlens, sh.T, dev)
    n_rows = (cu.numel() - 1) if packed else sh.B
    state, out_state, idx, n_slots = _state_operands(state, state_out, write_state, n_rows, sh.Hv, sh.Dv, sh.Dk,
                                                     dev, state_index)
    mask_u8 = _mask_u8(mask, (sh.B, sh.T))
    y_t = torch.empty(sh.B, sh.T, sh.Hv, sh.Dv, dtype=k.dtype, device=dev) if y else None
    snaps = (torch.empty(sh.B, sh.T, sh.Hv, sh.Dv, sh.Dk, dtype=torch.float32, device=dev)
             if snapshots else None)
    commit = None if commit_len is None else _int_rows(commit_len, n_rows, dev, "commit_len")
    args = _lib.RecurrentArgs(
        q=_ptr(q), k=_ptr(k), v=_ptr(v), qkv_dtype=qkv_code, gate_mode=gate_mode,
        gx=_ptr(gx), gy=_ptr(gy), gate_dtype=gate_code, param_dtype=param_code,
        A_log=_ptr(A_log), dt_bias=_ptr(dt_bias), state_in=_ptr(state),
        state_out=_ptr(out_state), snapshots=_ptr(snaps), y=_ptr(y_t), mask=_ptr(mask_u8),
        cu_seqlens=_ptr(cu), commit_len=_ptr(commit), state_index=_ptr(idx), B=n_rows, T=sh.T, Hk=sh.Hk,
        Hv=sh.Hv, Dk=sh.Dk, Dv=sh.Dv, n_slots=n_slots, gate_stride=g_ld, stream=_stream(dev),
        y_from=int(y_from),
    )
    with torch.cuda.device(dev):
        _lib.call("gdn_recurrent", _lib.ctypes.byref(args))
    return y_t, out_state, snaps


class PreparedRecurrent:
    """A validated recurrent launch that can be re-issued without re-validation.

    Holds the argument block and keeps every tensor it points to alive.  Each
    ``launch()`` enqueues the same kernel on the stream current at
    ``prepare`` time (the same work a serving loop repeats every step, e.g.
    decode with ``state_out=state``), or on ``stream`` when one is given --
    e.g. ``torch.cuda.current_stream()`` inside a ``torch.cuda.graph``
    capture.
    """

    def __init__(self, args, keep, dev):
        self._args = args
        self._keep = keep
        self.device = dev
        self._lib = _lib.load()

    def launch(self, stream=None):
        args = self._args
        if stream is not None:
            args = _lib.RecurrentArgs.from_buffer_copy(self._args)
            args.stream = _stream_handle(stream)
        st = self._lib.gdn_recurrent(_lib.ctypes.byref(args))
        if st != _lib.OK:
            _lib.check("gdn_recurrent", st)

    @property
    def outputs(self):
        return self._keep["y"], self._keep["state_out"], self._keep["snapshots"]


def prepare_recurrent(q, k, v, a, b, A_log, dt_bias, state, mask=None, *, y=True, state_out=None,
                      write_state=True, snapshots=False, commit_len=None, cu_seqlens=None,
                      gates_precomputed=False, state_index=None, y_from=0) -> PreparedRecurrent:
    """Validates once and returns a :class:`PreparedRecurrent` (same arguments as the entry points).

    ``y_from``: tokens before it produce no y (their rows of y are left unwritten).
    """
    mode = _lib.GATES_PRE if gates_precomputed else _lib.GATES_RAW
    names = ["q", "k", "v", "a/g", "b/beta", "A_log", "dt_bias", "state", "mask", "state_out"]
    dev = _require_device([q, k, v, a, b, A_log, dt_bias, state, mask, state_out], names)
    packed = cu_seqlens is not None
    sh = _Shapes(q, k, v, a, b, packed)
    for t, n in ((q, "q"), (k, "k"), (v, "v")):
        if t is not None and not t.is_contiguous():
            raise ValueError(f"{n} must be contiguous for a prepared launch")
    a_g, b_g, g_ld = _gate_pair(a, b, sh.Hv)
    if a_g is not a or b_g is not b:
        raise ValueError("a and b must be contiguous, or column slices with one token stride, for a prepared launch")
    qkv_code = _dtype_code(k, "q/k/v")
    gate_code = _gate_codes(a, b)
    param_code = _param_codes(A_log, dt_bias, sh.Hv) if mode == _lib.GATES_RAW else _lib.DTYPE_F32
    cu = _cu_seqlens(cu_seqlens, sh.T, dev)
    n_rows = (cu.numel() - 1) if packed else sh.B
    if state is not None and (not state.is_contiguous()):
        raise ValueError("state must be contiguous for a prepared launch")
    state, out_state, idx, n_slots = _state_operands(state, state_out, write_state, n_rows, sh.Hv, sh.Dv, sh.Dk,
                                                     dev, state_index)
    mask_u8 = _mask_u8(mask, (sh.B, sh.T))
    y_t = torch.empty(sh.B, sh.T, sh.Hv, sh.Dv, dtype=k.dtype, device=dev) if y else None
    snaps = (torch.empty(sh.B, sh.T, sh.Hv, sh.Dv, sh.Dk, dtype=torch.float32, device=dev)
             if snapshots else None)
    commit = None if commit_len is None else _int_rows(commit_len, n_rows, dev, "commit_len")
    args = _lib.RecurrentArgs(
        q=_ptr(q), k=_ptr(k), v=_ptr(v), qkv_dtype=qkv_code, gate_mode=mode,
        gx=_ptr(a), gy=_ptr(b), gate_dtype=gate_code, param_dtype=param_code,
        A_log=_ptr(A_log) if mode == _lib.GATES_RAW else None,
        dt_bias=_ptr(dt_bias) if mode == _lib.GATES_RAW else None, state_in=_ptr(state),
        state_out=_ptr(out_state), snapshots=_ptr(snaps), y=_ptr(y_t), mask=_ptr(mask_u8),
        cu_seqlens=_ptr(cu), commit_len=_ptr(commit), state_index=_ptr(idx), B=n_rows, T=sh.T, Hk=sh.Hk,
        Hv=sh.Hv, Dk=sh.Dk, Dv=sh.Dv, n_slots=n_slots, gate_stride=g_ld, stream=_stream(dev),
        y_from=int(y_from),
    )
    keep = dict(q=q, k=k, v=v, a=a, b=b, A_log=A_log, dt_bias=dt_bias, state=state, mask=mask_u8,
                cu=cu, commit=commit, y=y_t, state_out=out_state, snapshots=snaps, state_index=idx)
    return PreparedRecurrent(args, keep, dev)


def chunk_workspace_bytes(n_seqs: int, n_tok: int, Hv: int, Dk: int, Dv: int, chunk: int = CHUNK) -> int:
    return int(_lib.load().gdn_chunk_workspace_bytes(n_seqs, n_tok, Hv, Dk, Dv, chunk))


class PreparedCall:
    """A validated ``libgdn`` call that can be re-issued without re-validation.

    Holds the argument tuple and keeps every tensor it points to alive; each
    ``launch()`` enqueues the same work on the stream current at ``prepare``
    time (what a serving loop repeats every step), or on ``stream`` when one
    is given.  ``outputs`` are the tensors the call writes.
    """

    def __init__(self, fn: str, args: tuple, keep: dict, outputs: tuple, dev):
        self._fn_name = fn
        self._args = args
        self._keep = keep
        self.outputs = outputs
        self.device = dev
        self._fn = getattr(_lib.load(), fn)

    def launch(self, stream=None):
        args = self._args if stream is None else self._args[:-1] + (_stream_handle(stream),)
        st = self._fn(*args)
        if st != _lib.OK:
            _lib.check(self._fn_name, st)


class PreparedChunked(PreparedCall):
    """A prepared chunked prefill: ``launch()`` enqueues both phases; the
    phases can also be enqueued apart (``launch_prep`` then ``launch_scan``,
    in that order on the caller's streams), so a serving step can run
    HBM-bound launches of other rows beside the scan rather than beside the
    HBM-bound prep."""

    def __init__(self, fn: str, args: tuple, keep: dict, outputs: tuple, dev):
        super().__init__(fn, args, keep, outputs, dev)
        lib = _lib.load()
        self._prep = lib.gdn_chunk_prep
        self._scan = lib.gdn_chunk_scan

    def _issue(self, fn, name, stream):
        args = self._args if stream is None else self._args[:-1] + (_stream_handle(stream),)
        st = fn(*args)
        if st != _lib.OK:
            _lib.check(name, st)

    def launch_prep(self, stream=None):
        self._issue(self._prep, "gdn_chunk_prep", stream)

    def launch_scan(self, stream=None):
        self._issue(self._scan, "gdn_chunk_scan", stream)


def _chunk_args(q, k, v, gx, gy, gate_mode, A_log, dt_bias, state, *, cu_seqlens=None,
                state_out=None, workspace=None, state_index=None, mask=None):
    names = ["q", "k", "v", "a/g", "b/beta", "A_log", "dt_bias", "state", "state_out", "mask"]
    dev = _require_device([q, k, v, gx, gy, A_log, dt_bias, state, state_out, mask], names)
    packed = cu_seqlens is not None
    sh = _Shapes(q, k, v, gx, gy, packed)
    q, k, v = (_contig(t) for t in (q, k, v))
    gx, gy, g_ld = _gate_pair(gx, gy, sh.Hv)
    qkv_code = _dtype_code(k, "q/k/v")
    gate_code = _gate_codes(gx, gy)
    if gate_mode == _lib.GATES_RAW:
        param_code = _param_codes(A_log, dt_bias, sh.Hv)
        A_log, dt_bias = _contig(A_log), _contig(dt_bias)
    else:
        param_code = _lib.DTYPE_F32
    cu = _cu_seqlens(cu_seqlens, sh.T, dev)
    n_seqs = (cu.numel() - 1) if packed else sh.B
    n_tok = sh.B * sh.T
    state, out_state, idx, n_slots = _state_operands(state, state_out, True, n_seqs, sh.Hv, sh.Dv, sh.Dk, dev,
                                                     state_index)
    mask_u8 = _mask_u8(mask, (sh.B, sh.T))  # [B, T] row-major: one byte per token, in token order
    y_t = torch.empty(sh.B, sh.T, sh.Hv, sh.Dv, dtype=k.dtype, device=dev)
    ws_bytes = chunk_workspace_bytes(n_seqs, n_tok, sh.Hv, sh.Dk, sh.Dv, CHUNK)
    if workspace is None or workspace.numel() * workspace.element_size() < ws_bytes:
        workspace = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=dev)
    args = (_ptr(q), _ptr(k), _ptr(v), qkv_code, gate_mode, _ptr(gx), _ptr(gy), gate_code, g_ld, _ptr(A_log),
            _ptr(dt_bias), param_code, _ptr(mask_u8), _ptr(state), _ptr(y_t), _ptr(out_state), _ptr(idx), n_slots,
            _ptr(cu), n_seqs, n_tok, sh.Hk, sh.Hv, sh.Dk, sh.Dv, CHUNK, _ptr(workspace), ws_bytes, _stream(dev))
    keep = dict(q=q, k=k, v=v, gx=gx, gy=gy, A_log=A_log, dt_bias=dt_bias, state=state, cu=cu,
                workspace=workspace, state_index=idx, mask=mask_u8)
    return args, keep, y_t, out_state, dev


def _chunked(q, k, v, gx, gy, gate_mode, A_log, dt_bias, state, *, cu_seqlens=None,
             state_out=None, workspace=None, state_index=None, mask=None):
    args, _keep, y_t, out_state, dev = _chunk_args(q, k, v, gx, gy, gate_mode, A_log, dt_bias, state,
                                                   cu_seqlens=cu_seqlens, state_out=state_out,
                                                   workspace=workspace, state_index=state_index, mask=mask)
    with torch.cuda.device(dev):
        _lib.call("gdn_chunk_fwd", *args)
    return y_t, out_state


def prepare_chunked(q, k, v, a, b, A_log, dt_bias, state=None, *, cu_seqlens=None, state_out=None,
                    workspace=None, gates_precomputed=False, state_index=None, mask=None) -> "PreparedChunked":
    """Validates a chunked prefill once; ``launch()`` re-issues it.

    Same arguments as :func:`gated_delta_update` with ``chunked=True``;
    ``outputs`` is ``(y, new_state)``.  The inputs are bound by address, so a
    serving loop refills them in place between launches.
    """
    mode = _lib.GATES_PRE if gates_precomputed else _lib.GATES_RAW
    args, keep, y_t, out_state, dev = _chunk_args(q, k, v, a, b, mode, A_log, dt_bias, state,
                                                  cu_seqlens=cu_seqlens, state_out=state_out,
                                                  workspace=workspace, state_index=state_index, mask=mask)
    for name in ("q", "k", "v", "gx", "gy"):
        if keep[name].data_ptr() != {"q": q, "k": k, "v": v, "gx": a, "gy": b}[name].data_ptr():
            raise ValueError(f"{name} must be contiguous (gates: or one-stride column slices) for a prepared launch")
    keep.update(y=y_t, state_out=out_state)
    return PreparedChunked("gdn_chunk_fwd", args, keep, (y_t, out_state), dev)


def _aligned16(t: torch.Tensor) -> bool:
    # a non-contiguous operand is copied (and so aligned) before the launch
    return (not t.is_contiguous()) or t.data_ptr() % 16 == 0


def _use_chunked(chunked, q, k, v, mask, T):
    """The chunked kernel by default for long bf16 rows (masked or not) at
    Dk = Dv = 128 with 16-byte aligned q/k/v; everything else steps the
    recurrent kernel, which takes any of those."""
    if chunked is not None:
        return bool(chunked)
    if k.dtype != torch.bfloat16 or k.shape[-1] != 128 or v.shape[-1] != 128:
        return False
    if not all(_aligned16(t) for t in (q, k, v)):
        return False
    return T >= CHUNK_MIN_TOKENS


# ------------------------------------------------------------ entry points

def gated_delta_kernel(q, k, v, g, beta, state, mask=None, *, state_out=None, state_index=None):
    """mlx-lm ``gated_delta_kernel``: the fused recurrence with g and beta given.

    Returns ``(y, new_state)``.  ``state_index``: pooled states, as in
    :func:`gated_delta_update`.
    """
    y, s, _ = _recurrent(q, k, v, g, beta, _lib.GATES_PRE, None, None, state, mask,
                         state_out=state_out, state_index=state_index)
    return y, s


def gated_delta_update(q, k, v, a, b, A_log, dt_bias, state=None, mask=None, use_kernel=True, *,
                       cu_seqlens: Optional[IntSeq] = None, state_out=None,
                       chunked: Optional[bool] = None, workspace=None, state_index=None,
                       max_seqlen: Optional[int] = None):
    """mlx-lm ``gated_delta_update`` on MI355X.

    Args (as mlx-lm): q, k ``[B,T,Hk,Dk]``; v ``[B,T,Hv,Dv]``; a, b ``[B,T,Hv]``;
    A_log, dt_bias ``[Hv]``; state ``[B,Hv,Dv,Dk]`` float32 or None; mask
    ``[B,T]`` bool or None.  ``use_kernel=False`` selects the ops path
    (:func:`gated_delta_ops`) on the device.

    Keyword-only additions: ``cu_seqlens`` packs ragged sequences in a
    ``[1, N_tok, ...]`` layout (state then has one row per sequence); host
    offsets are validated, a device tensor is used without a host copy (the
    call never synchronises, so with several sequences it needs
    ``max_seqlen``, the longest one, to pick the kernel, unless ``chunked``
    picks it);
    ``state_out`` receives the new state (may be ``state``); ``chunked``
    forces the chunked MFMA prefill kernel on/off (default: long bf16 rows
    with Dk = Dv = 128, masked or not); ``workspace`` is a reusable uint8
    buffer for it.
    ``state_index`` (int32 ``[rows]``) switches to pooled states: ``state``
    (and ``state_out``) are then pools ``[n_slots, Hv, Dv, Dk]``, row b reads
    and writes slot ``state_index[b]``, and without ``state_out`` the pool is
    updated in place (see :class:`multiplex_amd.StatePool`).

    Returns ``(y [B,T,Hv,Dv] in q's dtype, new_state [rows,Hv,Dv,Dk] float32)``.
    """
    if not use_kernel:
        if cu_seqlens is not None or state_index is not None:
            raise ValueError("the ops path does not take cu_seqlens or state_index")
        y, s = gated_delta_ops(q, k, v, compute_g(A_log, a, dt_bias), compute_beta(b), state, mask)
        if state_out is not None:
            state_out.copy_(s)
            s = state_out
        return y, s
    T = k.shape[1]
    if cu_seqlens is not None and chunked is None:
        T = _packed_max_len(cu_seqlens, k.shape[1], max_seqlen)
    if _use_chunked(chunked, q, k, v, mask, T):
        return _chunked(q, k, v, a, b, _lib.GATES_RAW, A_log, dt_bias, state,
                        cu_seqlens=cu_seqlens, state_out=state_out, workspace=workspace,
                        state_index=state_index, mask=mask)
    y, s, _ = _recurrent(q, k, v, a, b, _lib.GATES_RAW, A_log, dt_bias, state, mask,
                         state_out=state_out, cu_seqlens=cu_seqlens, state_index=state_index)
    return y, s


def gated_delta_verify(q, k, v, a, b, A_log, dt_bias, state, mask=None, *, snapshots=False,
                       cu_seqlens: Optional[IntSeq] = None, state_index=None):
    """Speculative verify: y for all T draft tokens without writing the state.

    With ``snapshots=True`` also returns the float32 state after every token
    (``[B,T,Hv,Dv,Dk]``) so a rollback is an index, at T extra state writes.
    The default pairs with :func:`gated_delta_commit`, which re-reads the
    pre-verify state once and writes the accepted prefix's state once.
    Returns ``(y, snapshots or None)``.
    """
    y, _, snaps = _recurrent(q, k, v, a, b, _lib.GATES_RAW, A_log, dt_bias, state, mask,
                             write_state=False, snapshots=snapshots, cu_seqlens=cu_seqlens,
                             state_index=state_index)
    return y, snaps


def gated_delta_commit(k, v, a, b, A_log, dt_bias, state, n_commit: IntSeq, mask=None, *,
                       state_out=None, cu_seqlens: Optional[IntSeq] = None, state_index=None):
    """Commit the accepted prefix of a verify: the state after ``n_commit[b]`` tokens.

    Equivalent to the reference rollback, which re-runs ``gated_delta_update``
    on ``[:, :n]`` from the pre-verify state (``dflash.py:403-426``,
    ``engine.py:337-359``), but ragged per row and in one launch that reads
    each state once and writes it once.  ``n_commit[b]`` in ``[0, T]``
    (0 keeps the state; a negative value skips row b: in place it is not
    written, into a separate ``state_out`` its state is copied unchanged).
    ``state_out`` may be ``state`` (in place).  Returns the new state.
    """
    n_rows = (len(torch.as_tensor(cu_seqlens)) - 1) if cu_seqlens is not None else k.shape[0]
    dev = _require_device([k], ["k"])
    commit = _int_rows(n_commit, n_rows, dev, "n_commit")
    _, s, _ = _recurrent(None, k, v, a, b, _lib.GATES_RAW, A_log, dt_bias, state, mask,
                         y=False, state_out=state_out, cu_seqlens=cu_seqlens, commit_len=commit,
                         state_index=state_index)
    return s


def gated_delta_commit_verify(prev, n_prev: IntSeq, q, k, v, a, b, A_log, dt_bias, state, mask=None, *,
                              state_out=None, state_index=None):
    """Commit of the previous verify round and verify of the next, in one pass over the state.

    ``prev`` is ``(q, k, v, a, b)`` of the previous round's T_p draft tokens
    (``[B, T_p, ...]``), of which ``n_prev[b]`` were accepted (clamped to
    ``[0, T_p]``).  The result equals :func:`gated_delta_commit` of ``prev``
    with ``n_prev`` followed by :func:`gated_delta_verify` of the new tokens
    from the committed state -- the rollback replay of ``engine.py:337-359``
    folded into the next round -- but the state is read once and the committed
    state written once, where a verify and a commit read it twice.  One launch
    steps ``[prev tokens, new tokens]`` per row with the rejected previous
    tokens masked (a masked token leaves the state unchanged, the mlx-lm rule)
    and writes the state after the previous round's tokens.  ``mask``
    (``[B, T]``) masks new tokens.  ``state_out`` may be ``state``.

    Returns ``(y [B, T, Hv, Dv] of the new tokens, committed state)``.
    """
    qp, kp, vp, ap, bp = prev
    dev = _require_device([q, k, v, a, b, qp, kp, vp, ap, bp, state], ["q", "k", "v", "a", "b", "prev q",
                                                                       "prev k", "prev v", "prev a", "prev b",
                                                                       "state"])
    B, Tp = kp.shape[0], kp.shape[1]
    if k.shape[0] != B:
        raise ValueError(f"the new round has {k.shape[0]} rows, the previous one {B}")
    n = _int_rows(n_prev, B, dev, "n_prev").clamp(0, Tp)
    keep = torch.arange(Tp, device=dev)[None, :] < n[:, None]
    new = torch.ones(B, k.shape[1], dtype=torch.bool, device=dev) if mask is None else mask.to(dev, torch.bool)
    cat = [torch.cat([x0, x1], dim=1) for x0, x1 in ((qp, q), (kp, k), (vp, v), (ap, a), (bp, b))]
    commit = torch.full((B,), Tp, dtype=torch.int32, device=dev)
    # the previous tokens' y is not wanted: they are only stepped (to the
    # committed state), and the new ones take y from it unrolled
    y, s, _ = _recurrent(*cat, _lib.GATES_RAW, A_log, dt_bias, state, torch.cat([keep, new], dim=1),
                         state_out=state_out, commit_len=commit, state_index=state_index, y_from=Tp)
    return y[:, Tp:], s
