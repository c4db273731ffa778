"""Full-attention layers of the hybrid trunk and the MTP draft head on MI355X.

multiplex drafts with a native MTP head, ``MTPHead`` at
``multiplex/kernel/mtp.py:160-194``: RMSNorm of the next token's embedding and
of the trunk's hidden state, ``fc`` over their concatenation, the trunk's own
full-attention ``DecoderLayer`` (mlx-lm ``qwen3_5``) stacked
``mtp_num_hidden_layers`` times, and a final RMSNorm; each draft layer keeps
a plain KV cache that the drafter advances, trims back to the committed
length and slices by row (``mtp.py:440-668``).  The same DecoderLayer is
every fourth layer of the hybrid trunk.  This module keeps those names and
call shapes:

  KVCache        per-layer cache ``[B, Hkv, capacity, D]`` bf16 with
                 ``offset`` / ``size()`` / ``trim(n)`` / ``state`` /
                 ``filter`` / ``extract`` / ``merge`` as the drafter uses them
  Attention      Qwen3.5 gated attention: one GEMM for q|gate, k and v
                 (hipBLASLt through torch), then ``gdn_attn_qk`` (q/k RMSNorm,
                 partial rotary embedding, cache append) and ``gdn_attn_fwd``
                 (GQA flash attention on bf16 MFMA with the sigmoid gate
                 fused), then o_proj
  MLP            SwiGLU: one GEMM for gate|up, ``gdn_silu_mul``, down_proj
  DecoderLayer   pre-norm residual blocks (``gdn_rms_norm``)
  MTPHead        ``__call__(embed, hidden, cache) -> post_hidden``

Weights follow mlx's convention: a norm multiplies by its weight (mlx-lm
loads Qwen3.5's ``w - 1`` norm weights as ``w``).  Activations are bf16.
Every launch goes through ``libgdn.so``; there is no eager fallback.
"""

from __future__ import annotations

import math
from dataclasses import dataclass
from typing import List, Optional, Sequence

import torch

from . import _lib
from .gated_delta import _dtype_code, _ptr, _require_device, _stream

__all__ = [
    "AttentionArgs",
    "KVCache",
    "RMSNorm",
    "Attention",
    "MLP",
    "DecoderLayer",
    "MTPHead",
    "attn_qk",
    "attn_fwd",
    "rms_norm",
    "silu_mul",
]


@dataclass
class AttentionArgs:
    """The fields of mlx-lm's ``qwen3_5.TextModelArgs`` these layers read."""

    hidden_size: int
    num_attention_heads: int
    num_key_value_heads: int
    head_dim: int
    intermediate_size: int
    rms_norm_eps: float = 1e-6
    partial_rotary_factor: float = 0.25
    rope_theta: float = 10_000_000.0

    @property
    def rot(self) -> int:
        return int(self.head_dim * self.partial_rotary_factor)


# ------------------------------------------------------------ kernel calls

def _bf16(t: torch.Tensor, what: str):
    if t.dtype != torch.bfloat16:
        raise ValueError(f"{what} must be bfloat16 (got {t.dtype})")


def _token_stride(t: torch.Tensor, width: int, what: str) -> int:
    """Elements from one token to the next of a ``[B, T, width]`` view whose
    rows are contiguous (a column slice of a fused GEMM output)."""
    if t.dim() != 3 or t.shape[2] != width or t.stride(2) != 1:
        raise ValueError(f"{what} must be a [B, T, {width}] view with contiguous rows")
    B, T = t.shape[0], t.shape[1]
    ld = t.stride(1) if T > 1 else (t.stride(0) if B > 1 else width)
    if ld < width or (B > 1 and T > 1 and t.stride(0) != T * ld):
        raise ValueError(f"{what}: tokens must be one stride apart")
    return int(ld)


def _row_stride(t: torch.Tensor, D: int) -> int:
    """Elements between consecutive rows of a ``[..., D]`` tensor whose rows
    are contiguous and evenly spaced (a column slice of a wider buffer)."""
    if t.stride(-1) != 1:
        raise ValueError("rows must be contiguous")
    if t.dim() == 1:
        return D
    ld = t.stride(-2)
    for i in range(t.dim() - 2):
        if t.shape[i] > 1 and t.stride(i) != t.shape[i + 1] * t.stride(i + 1):
            raise ValueError("rows must be evenly spaced")
    if ld < D:
        raise ValueError("rows overlap")
    return int(ld)


def attn_qk(qg: torch.Tensor, k_new: torch.Tensor, v_new: torch.Tensor, q_norm_w: torch.Tensor,
            k_norm_w: torch.Tensor, eps: float, pos0: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
            rot: int, rope_base: float, *, q_out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """q/k norm, rotary embedding and KV-cache append (``gdn_attn_qk``).

    qg ``[B, T, Hq*2D]`` (per head: q, then the output gate); k_new, v_new
    ``[B, T, Hkv*D]`` (each may be a column slice of one GEMM output);
    caches ``[B, Hkv, cap, D]``; pos0 ``[B]`` int32 device offsets.
    Returns q ``[B, T, Hq, D]``.
    """
    dev = _require_device([qg, k_new, v_new, q_norm_w, k_norm_w, pos0, k_cache, v_cache],
                          ["qg", "k_new", "v_new", "q_norm_w", "k_norm_w", "pos0", "k_cache", "v_cache"])
    for t, n in ((qg, "qg"), (k_new, "k_new"), (v_new, "v_new"), (k_cache, "k_cache"), (v_cache, "v_cache")):
        _bf16(t, n)
    B, Hkv, cap, D = k_cache.shape
    if v_cache.shape != k_cache.shape or not k_cache.is_contiguous() or not v_cache.is_contiguous():
        raise ValueError("k_cache and v_cache must be contiguous [B, Hkv, cap, D] tensors of one shape")
    T = qg.shape[1]
    Hq = qg.shape[2] // (2 * D)
    qg_ld = _token_stride(qg, Hq * 2 * D, "qg")
    kv_ld = _token_stride(k_new, Hkv * D, "k_new")
    if _token_stride(v_new, Hkv * D, "v_new") != kv_ld:
        raise ValueError("k_new and v_new must share one token stride")
    if pos0.dtype != torch.int32 or tuple(pos0.shape) != (B,):
        raise ValueError(f"pos0 must be int32 [{B}]")
    if q_out is None:
        q_out = torch.empty(B, T, Hq, D, dtype=torch.bfloat16, device=dev)
    qn, kn = q_norm_w.contiguous(), k_norm_w.contiguous()
    _lib.call("gdn_attn_qk", _ptr(qg), qg_ld, _ptr(k_new), _ptr(v_new), kv_ld, _ptr(qn), _ptr(kn),
              _dtype_code(qn, "q_norm_w"), float(eps), _ptr(pos0), _ptr(q_out), _ptr(k_cache), _ptr(v_cache),
              B, T, Hq, Hkv, D, cap, int(rot), float(rope_base), _stream(dev))
    return q_out


def _check_attn_fwd(q, k_cache, v_cache, pos0, kv_len_max, gate, out):
    """Shapes, dtypes and layouts of :func:`attn_fwd`'s arguments, checked
    before anything is launched (a mismatch would otherwise read outside
    the caches).  Returns ``(B, T, Hq, D, Hkv, cap, gate token stride)``."""
    _bf16(q, "q")
    if q.dim() != 4:
        raise ValueError(f"q must be [B, T, Hq, D] (got {tuple(q.shape)})")
    B, T, Hq, D = q.shape
    for c, n in ((k_cache, "k_cache"), (v_cache, "v_cache")):
        _bf16(c, n)
        if c.dim() != 4 or not c.is_contiguous():
            raise ValueError(f"{n} must be a contiguous [B, Hkv, cap, D] tensor")
    if v_cache.shape != k_cache.shape:
        raise ValueError(f"v_cache {tuple(v_cache.shape)} and k_cache {tuple(k_cache.shape)} differ")
    Bc, Hkv, cap, Dc = k_cache.shape
    if Bc != B or Dc != D:
        raise ValueError(f"caches [{Bc}, {Hkv}, {cap}, {Dc}] do not match q's batch {B} and head dim {D}")
    if Hkv == 0 or Hq % Hkv != 0:
        raise ValueError(f"Hq={Hq} is not a multiple of Hkv={Hkv}")
    if not isinstance(pos0, torch.Tensor) or pos0.dtype != torch.int32 or tuple(pos0.shape) != (B,):
        raise ValueError(f"pos0 must be an int32 tensor of shape [{B}]")
    if not T <= int(kv_len_max) <= cap:
        raise ValueError(f"kv_len_max={kv_len_max} must lie in [T={T}, cap={cap}]")
    qg_ld = 0
    if gate is not None:
        _bf16(gate, "gate")
        if gate.dim() != 3 or tuple(gate.shape[:2]) != (B, T):
            raise ValueError(f"gate must be [B={B}, T={T}, {Hq * 2 * D}]")
        qg_ld = _token_stride(gate, Hq * 2 * D, "gate")
    if out is not None:
        _bf16(out, "out")
        if tuple(out.shape) != (B, T, Hq, D) or not out.is_contiguous():
            raise ValueError(f"out must be a contiguous [{B}, {T}, {Hq}, {D}] tensor")
    return B, T, Hq, D, Hkv, cap, qg_ld


def attn_fwd(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor, pos0: torch.Tensor, kv_len_max: int,
             *, gate: Optional[torch.Tensor] = None, scale: Optional[float] = None, n_split: int = 1,
             workspace: Optional[torch.Tensor] = None, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Causal GQA attention of q ``[B, T, Hq, D]`` over the caches
    (``gdn_attn_fwd``), times sigmoid of the gate half of ``gate``
    (``[B, T, Hq*2D]``, the q_proj output) when given.  ``kv_len_max`` bounds
    ``pos0[b] + T`` (host value; keys beyond it are not read)."""
    B, T, Hq, D, Hkv, cap, qg_ld = _check_attn_fwd(q, k_cache, v_cache, pos0, kv_len_max, gate, out)
    dev = _require_device([q, k_cache, v_cache, pos0, gate, out], ["q", "k_cache", "v_cache", "pos0", "gate", "out"])
    if out is None:
        out = torch.empty(B, T, Hq, D, dtype=torch.bfloat16, device=dev)
    need = int(_lib.load().gdn_attn_workspace_bytes(B, T, Hq, Hkv, D, n_split))
    if need > 0 and (workspace is None or workspace.numel() * workspace.element_size() < need):
        workspace = torch.empty(need, dtype=torch.uint8, device=dev)
    q = q.contiguous()
    scale = D ** -0.5 if scale is None else scale
    _lib.call("gdn_attn_fwd", _ptr(q), _ptr(gate), qg_ld, _ptr(k_cache), _ptr(v_cache), _ptr(pos0), _ptr(out),
              float(scale), B, T, Hq, Hkv, D, cap, int(kv_len_max), int(n_split), _ptr(workspace),
              0 if workspace is None else workspace.numel() * workspace.element_size(), _stream(dev))
    return out


def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float, *, residual: Optional[torch.Tensor] = None,
             out: Optional[torch.Tensor] = None):
    """``h / sqrt(mean(h^2) + eps) * weight`` over the last dim (bf16), with
    ``h = x`` or, given ``residual``, ``h = x + residual`` (one launch; then
    returns ``(h, y)``).  ``out`` may be a column slice of a wider buffer
    (rows one stride apart), e.g. one half of a concatenation."""
    _bf16(x, "x")
    D = x.shape[-1]
    if tuple(weight.shape) != (D,):
        raise ValueError(f"weight must be [{D}]")
    if residual is not None and residual.shape != x.shape:
        raise ValueError(f"residual {tuple(residual.shape)} must have x's shape {tuple(x.shape)}")
    dev = _require_device([x, weight, residual, out], ["x", "weight", "residual", "out"])
    x = x.contiguous()
    rows = x.numel() // D
    if out is None:
        out = torch.empty_like(x)
        y_ld = D
    else:
        if out.shape != x.shape:
            raise ValueError("out must have x's shape")
        y_ld = _row_stride(out, D)
    h = None
    if residual is not None:
        _bf16(residual, "residual")
        residual = residual.contiguous()
        h = torch.empty_like(x)
    w = weight.contiguous()
    _lib.call("gdn_rms_norm", _ptr(x), _ptr(residual), _ptr(h), _ptr(w), _dtype_code(w, "weight"), _ptr(out), y_ld,
              rows, D, float(eps), _stream(dev))
    return out if residual is None else (h, out)


def silu_mul(gate_up: torch.Tensor) -> torch.Tensor:
    """``silu(gate) * up`` of a ``[..., 2I]`` gate|up product (bf16)."""
    dev = _require_device([gate_up], ["gate_up"])
    _bf16(gate_up, "gate_up")
    I = gate_up.shape[-1] // 2
    gate_up = gate_up.contiguous()
    out = torch.empty(*gate_up.shape[:-1], I, dtype=gate_up.dtype, device=dev)
    _lib.call("gdn_silu_mul", _ptr(gate_up), _ptr(out), gate_up.numel() // (2 * I), I, _stream(dev))
    return out


# ------------------------------------------------------------------ cache

class KVCache:
    """One attention layer's KV cache, ``[B, Hkv, capacity, D]`` bf16.

    Row b holds its keys left-aligned at positions ``[0, lengths[b])``; the
    device copy of the lengths (``pos0``) is what the kernels read (a row's
    new tokens go to ``pos0[b]`` on, and it attends to keys ``[0, pos0[b] +
    T)``), so a step never reads the host value back.  Rows of a batch join
    may differ in length (:meth:`merge`), as the reference drafter's
    ``BatchKVCache.merge`` allows (``mtp.py:505-511``); ``offset`` and
    ``size()`` are the longest row's length, and :meth:`trim` drops the last
    ``n`` positions of every row.  ``capacity`` grows by reallocation (in
    steps of 256 positions) when a call would overflow it.
    """

    step = 256

    def __init__(self, batch: int, n_kv_heads: int, head_dim: int, capacity: int = 256,
                 device: Optional[torch.device] = None):
        self._alloc(batch, n_kv_heads, head_dim, capacity, device)

    def _alloc(self, batch, n_kv_heads, head_dim, capacity, device):
        capacity = max(self.step, -(-int(capacity) // self.step) * self.step)
        self.keys = torch.empty(batch, n_kv_heads, capacity, head_dim, dtype=torch.bfloat16, device=device)
        self.values = torch.empty_like(self.keys)
        self.lengths = [0] * batch
        self.pos0 = torch.zeros(batch, dtype=torch.int32, device=device)

    @property
    def batch(self) -> int:
        return self.keys.shape[0]

    @property
    def capacity(self) -> int:
        return self.keys.shape[2]

    @property
    def offset(self) -> int:
        """The longest row's length."""
        return max(self.lengths, default=0)

    def size(self) -> int:
        return self.offset

    @property
    def state(self):
        """Keys and values up to the longest row, ``[B, Hkv, offset, D]``
        views (past a shorter row's length its entries are unset)."""
        return self.keys[..., : self.offset, :], self.values[..., : self.offset, :]

    @state.setter
    def state(self, kv) -> None:
        """Replaces the contents by ``[keys, values]`` ``[B, Hkv, L, D]``: every
        row then holds L positions (a prefix-cache restore of MTP blocks,
        ``mtp.py:608``).  The cache is reallocated when its batch, head
        layout or capacity does not fit."""
        keys, values = kv
        if keys.dim() != 4 or values.shape != keys.shape:
            raise ValueError("state must be [keys, values] of one [B, Hkv, L, D] shape")
        B, Hkv, L, D = keys.shape
        if (B, Hkv, D) != (self.batch, self.keys.shape[1], self.keys.shape[3]) or L > self.capacity:
            self._alloc(B, Hkv, D, max(L, self.capacity), self.keys.device)
        self.keys[..., :L, :] = keys
        self.values[..., :L, :] = values
        self.lengths = [L] * B
        self.pos0.fill_(L)

    def reserve(self, T: int) -> None:
        need = self.offset + int(T)
        if need <= self.capacity:
            return
        cap = -(-need // self.step) * self.step
        n = self.offset
        for name in ("keys", "values"):
            old = getattr(self, name)
            new = torch.empty(*old.shape[:2], cap, old.shape[3], dtype=old.dtype, device=old.device)
            new[..., :n, :] = old[..., :n, :]
            setattr(self, name, new)

    def advance(self, T: int) -> None:
        self.lengths = [n + int(T) for n in self.lengths]
        self.pos0.add_(int(T))

    def trim(self, n: int) -> int:
        """Drops the last ``n`` positions of every row (the drafter's rollback)."""
        n = min(int(n), self.offset)
        self.lengths = [max(0, m - n) for m in self.lengths]
        self.pos0.sub_(n).clamp_(min=0)
        return n

    def filter(self, keep: Sequence[int]) -> None:
        """Keeps rows ``keep`` (a batch leave)."""
        keep = [int(i) for i in keep]
        idx = torch.as_tensor(keep, dtype=torch.long, device=self.keys.device)
        self.keys = self.keys.index_select(0, idx)
        self.values = self.values.index_select(0, idx)
        self.pos0 = self.pos0.index_select(0, idx)
        self.lengths = [self.lengths[i] for i in keep]

    def extract(self, row: int) -> "KVCache":
        """A one-row copy of row ``row``."""
        n = self.lengths[row]
        c = KVCache(1, self.keys.shape[1], self.keys.shape[3], self.capacity, self.keys.device)
        c.keys[..., :n, :] = self.keys[row : row + 1, :, :n, :]
        c.values[..., :n, :] = self.values[row : row + 1, :, :n, :]
        c.advance(n)
        return c

    @classmethod
    def merge(cls, caches: Sequence["KVCache"]) -> "KVCache":
        """Rows of several caches as one batch (a batch join); rows keep
        their own lengths."""
        first = caches[0]
        Hkv, D = first.keys.shape[1], first.keys.shape[3]
        if any(c.keys.shape[1] != Hkv or c.keys.shape[3] != D for c in caches):
            raise ValueError("caches of different head layouts cannot be merged")
        cap = max(c.capacity for c in caches)
        out = cls(sum(c.batch for c in caches), Hkv, D, cap, first.keys.device)
        r = 0
        for c in caches:
            n = c.offset
            out.keys[r : r + c.batch, :, :n, :] = c.keys[..., :n, :]
            out.values[r : r + c.batch, :, :n, :] = c.values[..., :n, :]
            r += c.batch
        out.lengths = [m for c in caches for m in c.lengths]
        out.pos0 = torch.tensor(out.lengths, dtype=torch.int32).to(first.keys.device)
        return out


# ----------------------------------------------------------------- layers

def _linear(in_f: int, out_f: int, device, dtype) -> torch.nn.Parameter:
    w = torch.empty(out_f, in_f, device=device, dtype=dtype)
    torch.nn.init.normal_(w, 0.0, in_f ** -0.5)
    return torch.nn.Parameter(w, requires_grad=False)


class RMSNorm(torch.nn.Module):
    """mlx ``nn.RMSNorm`` on ``gdn_rms_norm``."""

    def __init__(self, dim: int, eps: float = 1e-6, device=None):
        super().__init__()
        self.weight = torch.nn.Parameter(torch.ones(dim, device=device), requires_grad=False)
        self.eps = eps

    def forward(self, x: torch.Tensor, residual: Optional[torch.Tensor] = None,
                out: Optional[torch.Tensor] = None):
        """norm(x), or ``(x + residual, norm(x + residual))`` in one launch."""
        return rms_norm(x, self.weight, self.eps, residual=residual, out=out)


class Attention(torch.nn.Module):
    """Qwen3.5 gated full attention (mlx-lm ``qwen3_5`` Attention).

    ``qkv_proj`` holds q_proj (``2 * Hq * D`` rows: per head q then gate),
    k_proj and v_proj stacked, so the three projections are one GEMM;
    :meth:`load` takes them separately.
    """

    def __init__(self, args: AttentionArgs, device=None, dtype=torch.bfloat16, n_split: Optional[int] = None):
        super().__init__()
        self.args = args
        H, Hq, Hkv, D = args.hidden_size, args.num_attention_heads, args.num_key_value_heads, args.head_dim
        if Hq % Hkv != 0:
            raise ValueError("num_attention_heads must be a multiple of num_key_value_heads")
        self.Hq, self.Hkv, self.D = Hq, Hkv, D
        self.qkv_proj = _linear(H, (2 * Hq + 2 * Hkv) * D, device, dtype)
        self.o_proj = _linear(Hq * D, H, device, dtype)
        self.q_norm = RMSNorm(D, args.rms_norm_eps, device)
        self.k_norm = RMSNorm(D, args.rms_norm_eps, device)
        self.scale = D ** -0.5
        self.n_split = n_split
        self._cus = None

    @torch.no_grad()
    def load(self, q_proj, k_proj, v_proj, o_proj, q_norm, k_norm) -> None:
        self.qkv_proj.copy_(torch.cat([q_proj, k_proj, v_proj]).to(self.qkv_proj))
        self.o_proj.copy_(o_proj.to(self.o_proj))
        self.q_norm.weight.copy_(q_norm)
        self.k_norm.weight.copy_(k_norm)

    def _splits(self, B: int, T: int, L: int) -> int:
        """Key ranges per row for decode and draft verify: about one
        workgroup per CU (measured best: one 68 KB-LDS workgroup per CU
        streams the cache faster than two), ranges of at least 512 keys."""
        if self.n_split is not None:
            return self.n_split
        if T * (self.Hq // self.Hkv) > 16:
            return 1
        if self._cus is None:
            self._cus = torch.cuda.get_device_properties(self.qkv_proj.device).multi_processor_count
        return int(max(1, min(round(self._cus / (B * self.Hkv)), L // 512)))

    def forward(self, x: torch.Tensor, cache: KVCache) -> torch.Tensor:
        B, T, _ = x.shape
        Hq, Hkv, D = self.Hq, self.Hkv, self.D
        qkv = torch.nn.functional.linear(x, self.qkv_proj)
        qg = qkv[..., : 2 * Hq * D]
        k = qkv[..., 2 * Hq * D : (2 * Hq + Hkv) * D]
        v = qkv[..., (2 * Hq + Hkv) * D :]
        cache.reserve(T)
        q = attn_qk(qg, k, v, self.q_norm.weight, self.k_norm.weight, self.args.rms_norm_eps, cache.pos0,
                    cache.keys, cache.values, self.args.rot, self.args.rope_theta)
        L = cache.offset + T
        o = attn_fwd(q, cache.keys, cache.values, cache.pos0, L, gate=qg, scale=self.scale,
                     n_split=self._splits(B, T, L))
        cache.advance(T)
        return torch.nn.functional.linear(o.view(B, T, Hq * D), self.o_proj)


class MLP(torch.nn.Module):
    """SwiGLU ``down(silu(gate(x)) * up(x))`` with gate|up as one GEMM."""

    def __init__(self, hidden: int, inter: int, device=None, dtype=torch.bfloat16):
        super().__init__()
        self.gate_up_proj = _linear(hidden, 2 * inter, device, dtype)
        self.down_proj = _linear(inter, hidden, device, dtype)

    @torch.no_grad()
    def load(self, gate_proj, up_proj, down_proj) -> None:
        self.gate_up_proj.copy_(torch.cat([gate_proj, up_proj]).to(self.gate_up_proj))
        self.down_proj.copy_(down_proj.to(self.down_proj))

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return torch.nn.functional.linear(silu_mul(torch.nn.functional.linear(x, self.gate_up_proj)), self.down_proj)


class DecoderLayer(torch.nn.Module):
    """mlx-lm ``qwen3_5.DecoderLayer`` at a full-attention index (dense MLP)."""

    def __init__(self, args: AttentionArgs, device=None, dtype=torch.bfloat16):
        super().__init__()
        self.self_attn = Attention(args, device, dtype)
        self.mlp = MLP(args.hidden_size, args.intermediate_size, device, dtype)
        self.input_layernorm = RMSNorm(args.hidden_size, args.rms_norm_eps, device)
        self.post_attention_layernorm = RMSNorm(args.hidden_size, args.rms_norm_eps, device)

    def forward(self, x: torch.Tensor, cache: KVCache) -> torch.Tensor:
        h, m = self.forward_parts(x, None, cache)
        return h + m

    def forward_parts(self, x: torch.Tensor, residual: Optional[torch.Tensor], cache: KVCache):
        """The layer on ``x + residual`` (or ``x``), returning ``(h, m)`` whose
        sum is its output: the caller adds them inside the next norm
        (``gdn_rms_norm`` with a residual, the same bf16 rounding point), so no
        residual add runs as a launch of its own."""
        if residual is None:
            xin, y0 = x, self.input_layernorm(x)
        else:
            xin, y0 = self.input_layernorm(x, residual=residual)
        # the residual add in front of the second norm is fused into it
        h, y = self.post_attention_layernorm(xin, residual=self.self_attn(y0, cache))
        return h, self.mlp(y)


class MTPHead(torch.nn.Module):
    """The MTP draft stack (``mtp.py:160-194``): reuses the trunk's embedding
    and output projection, which the caller applies; this module maps
    ``(embed, hidden)`` to the post-norm hidden of the drafted positions."""

    def __init__(self, args: AttentionArgs, n_layers: int = 1, device=None, dtype=torch.bfloat16):
        super().__init__()
        H, eps = args.hidden_size, args.rms_norm_eps
        self.args = args
        self.pre_fc_norm_embedding = RMSNorm(H, eps, device)
        self.pre_fc_norm_hidden = RMSNorm(H, eps, device)
        self.fc = _linear(2 * H, H, device, dtype)
        self.layers = torch.nn.ModuleList(DecoderLayer(args, device, dtype) for _ in range(max(int(n_layers), 1)))
        self.norm = RMSNorm(H, eps, device)

    def make_cache(self, batch: int, capacity: int = 256) -> List[KVCache]:
        dev = self.fc.device
        a = self.args
        return [KVCache(batch, a.num_key_value_heads, a.head_dim, capacity, dev) for _ in self.layers]

    def forward(self, embed: torch.Tensor, hidden: torch.Tensor, cache: Sequence[KVCache]) -> torch.Tensor:
        """Post-norm hidden ``[B, L, H]``; each draft layer's cache advances by L."""
        if len(cache) != len(self.layers):
            raise ValueError(f"expected {len(self.layers)} draft caches, got {len(cache)}")
        # both norms write their halves of fc's input in place of a concatenation
        H = embed.shape[-1]
        eh = torch.empty(*embed.shape[:-1], 2 * H, dtype=embed.dtype, device=embed.device)
        self.pre_fc_norm_embedding(embed, out=eh[..., :H])
        self.pre_fc_norm_hidden(hidden, out=eh[..., H:])
        x = torch.nn.functional.linear(eh, self.fc)
        res = None  # the pending residual: each layer's output is x + res
        for layer, c in zip(self.layers, cache):
            x, res = layer.forward_parts(x, res, c)
        # the last layer's residual add happens inside the final norm
        return self.norm(res, residual=x)[1]

    @staticmethod
    def trim_cache_to(cache: Sequence[KVCache], size: int) -> None:
        """``Drafter.trim_cache_to`` (mtp.py:497-503)."""
        target = max(0, int(size))
        for c in cache:
            if c.size() > target:
                c.trim(c.size() - target)
