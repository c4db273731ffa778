"""GatedDeltaNet mixer on MI355X, callable like the one multiplex drives.

The reference restates the mixer at ``multiplex/kernel/dflash.py:343-381``
and the engine calls it as ``mixer(inputs, mask=None, cache=None)`` through
``_GDNMixerProxy`` (``engine.py:151-170``), finding it by class name
``GatedDeltaNet`` on ``layer.linear_attn`` (``engine.py:330-335``).  This
module keeps that class name and call signature, with ``cache[0]`` the conv
state and ``cache[1]`` the recurrent state -- a dense ``[B, Hv, Dv, Dk]``
array, or a :class:`~multiplex_amd.state_pool.PooledBatch` whose slots the
kernels update in place.  With pooled states a decode step (one token per
row) also updates the conv state ``cache[0]`` in place.

Data path per call:
  in_proj_qkv / z / b / a      one library GEMM (hipBLASLt through torch); the
                               kernels below read its column slices in place
  gdn_conv_prologue            fused conv1d + SiLU + q/k norm (HIP)
  gated_delta_update           recurrent or chunked kernel (HIP); where the
                               chunked kernel runs (long unmasked rows) the
                               prologue is fused into its prep instead
                               (``gdn_conv_chunked``)
  norm(out, z) + out_proj      up to 16 rows (decode of up to 16 rows) one
                               ``gdn_linear_decode`` launch with the gated
                               RMSNorm in its operand load (HIP); else the
                               gated RMSNorm kernel (HIP) and the library GEMM

Speculative rounds: ``mixer(inputs, mask, cache, verify=True)`` computes the
outputs of all T draft tokens without touching ``cache`` and remembers what
a commit needs; ``mixer.commit(cache, n_commit)`` then advances each row by
its accepted length in one pass over the state.  This replaces the
reference's snapshot -> verify -> restore -> replay sequence
(``engine.py:300-359``, ``dflash.py:403-426``), which moves the state about
four times as often.
"""

from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Optional, Sequence

import torch

from .cache import ArraysCache
from .conv import conv_state_commit, gdn_conv_chunked, gdn_conv_prologue
from .epilogue import gated_rms_norm
from .state_pool import PooledBatch
from .gated_delta import CHUNK_MIN_TOKENS, IntSeq, gated_delta_commit, gated_delta_update, gated_delta_verify
from .linear import FUSED_NORM_MAX_ROWS, DecodeWorkspace, decode_shape_ok, gated_norm_linear_decode

__all__ = ["GatedDeltaNet", "gated_rms_norm", "commit_verified"]


@dataclass
class _Pending:
    qkv: torch.Tensor
    k: torch.Tensor
    v: torch.Tensor
    a: torch.Tensor
    b: torch.Tensor
    mask: Optional[torch.Tensor]
    conv_state: Optional[torch.Tensor]
    cache: ArraysCache


class GatedDeltaNet(torch.nn.Module):
    """Gated DeltaNet mixer (Qwen3.5 / Qwen3-Next layout)."""

    def __init__(self, hidden_size: int, num_k_heads: int = 16, num_v_heads: int = 32, head_k_dim: int = 128,
                 head_v_dim: int = 128, conv_kernel_size: int = 4, rms_norm_eps: float = 1e-6,
                 dtype: torch.dtype = torch.bfloat16, device=None):
        super().__init__()
        self.hidden_size = hidden_size
        self.num_k_heads, self.num_v_heads = num_k_heads, num_v_heads
        self.head_k_dim, self.head_v_dim = head_k_dim, head_v_dim
        self.key_dim = num_k_heads * head_k_dim
        self.value_dim = num_v_heads * head_v_dim
        self.conv_dim = 2 * self.key_dim + self.value_dim
        self.conv_kernel_size = conv_kernel_size
        self.rms_norm_eps = rms_norm_eps
        self.sharding_group = None
        kw = dict(dtype=dtype, device=device)
        self.in_proj_qkv = torch.nn.Linear(hidden_size, self.conv_dim, bias=False, **kw)
        self.in_proj_z = torch.nn.Linear(hidden_size, self.value_dim, bias=False, **kw)
        self.in_proj_b = torch.nn.Linear(hidden_size, num_v_heads, bias=False, **kw)
        self.in_proj_a = torch.nn.Linear(hidden_size, num_v_heads, bias=False, **kw)
        # The four in_proj weights live in one [conv_dim + value_dim + 2 Hv,
        # hidden] buffer (qkv | z | b | a), each module's weight a row slice
        # of it, so the projections run as one GEMM whose output the
        # prologue, the GDN kernel and the norm read in place as column
        # slices.  The parameter names stay the reference's.
        self._splits = (self.conv_dim, self.conv_dim + self.value_dim, self.conv_dim + self.value_dim + num_v_heads)
        fused = torch.empty(self._splits[2] + num_v_heads, hidden_size, **kw)
        bounds = (0,) + self._splits + (fused.shape[0],)
        for lin, lo, hi in zip(self._in_projs(), bounds[:-1], bounds[1:]):
            lin.weight = torch.nn.Parameter(fused[lo:hi])
        self._in_proj_fused = fused
        self.conv1d_weight = torch.nn.Parameter(torch.empty(self.conv_dim, conv_kernel_size, **kw))
        self.A_log = torch.nn.Parameter(torch.empty(num_v_heads, dtype=torch.float32, device=device))
        self.dt_bias = torch.nn.Parameter(torch.empty(num_v_heads, dtype=torch.float32, device=device))
        self.norm_weight = torch.nn.Parameter(torch.ones(head_v_dim, **kw))
        self.out_proj = torch.nn.Linear(self.value_dim, hidden_size, bias=False, **kw)
        self._pending: Optional[_Pending] = None
        # the fused norm + out_proj runs up to this many rows (0: never), with
        # its workspace (zeroed once, left zeroed by every call)
        self.fused_norm_max_rows = FUSED_NORM_MAX_ROWS
        self._ws_out = DecodeWorkspace()
        self.reset_parameters()

    @torch.no_grad()
    def reset_parameters(self, generator: Optional[torch.Generator] = None) -> None:
        """Random init with the benchmark's distributions (no checkpoints here)."""
        for lin in (self.in_proj_qkv, self.in_proj_z, self.in_proj_b, self.in_proj_a, self.out_proj):
            w = torch.randn(lin.weight.shape, generator=generator) / math.sqrt(lin.weight.shape[1])
            lin.weight.copy_(w)
        self.conv1d_weight.copy_(torch.randn(self.conv1d_weight.shape, generator=generator) * 0.1)
        self.A_log.copy_(torch.rand(self.num_v_heads, generator=generator) * math.log(16.0))
        self.dt_bias.copy_(torch.rand(self.num_v_heads, generator=generator) * 2 - 1)
        self.norm_weight.fill_(1.0)

    def _in_projs(self):
        return (self.in_proj_qkv, self.in_proj_z, self.in_proj_b, self.in_proj_a)

    def _apply(self, fn, *args, **kwargs):
        # .to() / .cuda() move each parameter on its own: stack the in_proj
        # weights into one buffer again afterwards
        out = super()._apply(fn, *args, **kwargs)
        with torch.no_grad():
            fused = torch.cat([lin.weight for lin in self._in_projs()], dim=0)
            bounds = (0,) + self._splits + (fused.shape[0],)
            for lin, lo, hi in zip(self._in_projs(), bounds[:-1], bounds[1:]):
                lin.weight = torch.nn.Parameter(fused[lo:hi], requires_grad=lin.weight.requires_grad)
        self._in_proj_fused = fused
        return out

    def _fused_in_proj_weight(self) -> torch.Tensor:
        """The stacked in_proj weight; rebuilt (a copy) if a module's weight
        was replaced by a tensor outside the shared buffer."""
        f = self._in_proj_fused
        row = f.stride(0) * f.element_size()
        bounds = (0,) + self._splits
        if all(lin.weight.data_ptr() == f.data_ptr() + lo * row for lin, lo in zip(self._in_projs(), bounds)):
            return f
        return torch.cat([lin.weight for lin in self._in_projs()], dim=0)

    def _project(self, inputs):
        """in_proj_qkv / z / b / a as column slices of fused GEMM outputs.

        Up to 256 tokens the GEMM reads the weights once and is bound by
        that: one launch for all four.  Beyond, the library's tiling favours
        [qkv | z] (a multiple of 256 columns) and [b | a] as two GEMMs.
        """
        B, S, _ = inputs.shape
        w = self._fused_in_proj_weight()
        c1, c2, c3 = self._splits
        if B * S <= 256:
            out = torch.nn.functional.linear(inputs, w)
            qkv, z, ba = out[..., :c1], out[..., c1:c2], out[..., c2:]
        else:
            out = torch.nn.functional.linear(inputs, w[:c2])
            ba = torch.nn.functional.linear(inputs, w[c2:])
            qkv, z = out[..., :c1], out[..., c1:]
        z = z.unflatten(-1, (self.num_v_heads, self.head_v_dim))
        hv = self.num_v_heads
        return qkv, z, ba[..., hv:], ba[..., :hv]

    def _epilogue(self, y, z):
        B, S = y.shape[:2]
        M = B * S
        W = self.out_proj.weight
        if (M <= self.fused_norm_max_rows and y.dtype == torch.bfloat16 and self.out_proj.bias is None
                and self.head_v_dim in (64, 128) and decode_shape_ok(M, W.shape[0], W.shape[1])
                and z.stride(-2) == self.head_v_dim and (B == 1 or S == 1 or z.stride(0) == S * z.stride(1))):
            # z [B, S, Hv, Dv] is a column slice of the in_proj output: rows one token stride apart
            z_rows = z.as_strided((M, self.value_dim), (z.stride(1) if S > 1 else z.stride(0), 1))
            out = gated_norm_linear_decode(y.reshape(M, -1), z_rows, self.norm_weight, self.rms_norm_eps,
                                           self.head_v_dim, W, workspace=self._ws_out)
            return out.view(B, S, -1)
        # y is this call's own buffer: normalise it in place
        out = gated_rms_norm(y, z, self.norm_weight, self.rms_norm_eps, out=y)
        return self.out_proj(out.reshape(B, S, -1))

    def _fused_prefill(self, qkv: torch.Tensor, mask) -> bool:
        """Whether a call takes the chunked kernel (``gated_delta_update``'s
        default rule: unmasked bf16 rows of at least ``CHUNK_MIN_TOKENS``
        tokens at 128-wide heads), with a 4-tap conv to fuse into it."""
        return (mask is None and qkv.dtype == torch.bfloat16 and qkv.shape[1] >= CHUNK_MIN_TOKENS
                and self.head_k_dim == 128 and self.head_v_dim == 128 and self.conv_kernel_size == 4
                and self.conv1d_weight.dtype in (torch.bfloat16, torch.float32))

    def forward(self, inputs: torch.Tensor, mask: Optional[torch.Tensor] = None,
                cache: Optional[ArraysCache] = None, *, verify: bool = False) -> torch.Tensor:
        """``inputs [B, S, hidden]`` -> ``[B, S, hidden]``; updates ``cache`` unless ``verify``."""
        if self.sharding_group is not None:
            raise NotImplementedError("tensor-parallel sharding of the mixer is not built")
        qkv, z, a, b = self._project(inputs)
        conv_state = cache[0] if cache is not None else None
        state = cache[1] if cache is not None else None
        pooled = isinstance(state, PooledBatch)
        if not verify and self._fused_prefill(qkv, mask):
            # long unmasked rows: the conv prologue runs inside the chunked
            # pass's prep (bit-identical to the two launches below)
            pool = state.pool.states if pooled else state
            y, new_state, new_cs = gdn_conv_chunked(
                qkv, self.conv1d_weight, self.num_k_heads, self.num_v_heads, self.head_k_dim, self.head_v_dim,
                a, b, self.A_log, self.dt_bias, pool, conv_state, eps=self.rms_norm_eps,
                state_index=state.index if pooled else None)
            if cache is not None:
                cache[0] = new_cs
                if not pooled:
                    cache[1] = new_state
            return self._epilogue(y, z)
        # pooled decode advances the conv state in place too, as its states
        # advance in their pool slots (no new tensor per step)
        cs_in_place = (pooled and not verify and qkv.shape[1] == 1 and conv_state is not None
                       and conv_state.is_contiguous())
        q, k, v, new_cs = gdn_conv_prologue(
            qkv, self.conv1d_weight, self.num_k_heads, self.num_v_heads, self.head_k_dim, self.head_v_dim,
            conv_state, mask, eps=self.rms_norm_eps, write_conv_state=not verify,
            conv_state_out=conv_state if cs_in_place else None)
        if verify:
            if cache is None:
                raise ValueError("verify needs the cache the round will be committed into")
            if pooled:
                y, _ = gated_delta_verify(q, k, v, a, b, self.A_log, self.dt_bias, state.pool.states, mask,
                                          state_index=state.index)
            else:
                y, _ = gated_delta_verify(q, k, v, a, b, self.A_log, self.dt_bias, state, mask)
            self._pending = _Pending(qkv, k, v, a, b, mask, conv_state, cache)
        elif pooled:
            # the rows' states advance in their pool slots
            y, _ = gated_delta_update(q, k, v, a, b, self.A_log, self.dt_bias, state.pool.states, mask,
                                      state_index=state.index)
            cache[0] = new_cs
        else:
            y, new_state = gated_delta_update(q, k, v, a, b, self.A_log, self.dt_bias, state, mask)
            if cache is not None:
                cache[0] = new_cs
                cache[1] = new_state
        return self._epilogue(y, z)

    def commit(self, cache: ArraysCache, n_commit: IntSeq) -> None:
        """Advance every row of ``cache`` by its first ``n_commit[b]`` verified tokens.

        State: one read and one in-place write per row (rows with a zero state
        get a new tensor).  Conv state: ``concat(conv_state, qkv)[n : n+K-1]``.
        """
        p = self._pending
        if p is None or p.cache is not cache:
            raise ValueError("commit() must follow verify on the same cache")
        state = cache[1]
        if isinstance(state, PooledBatch):
            gated_delta_commit(p.k, p.v, p.a, p.b, self.A_log, self.dt_bias, state.pool.states, n_commit, p.mask,
                               state_index=state.index)
            new_state = state
        elif state is None:
            new_state = gated_delta_commit(p.k, p.v, p.a, p.b, self.A_log, self.dt_bias, None, n_commit, p.mask)
        else:
            new_state = gated_delta_commit(p.k, p.v, p.a, p.b, self.A_log, self.dt_bias, state, n_commit, p.mask,
                                           state_out=state)
        cache[1] = new_state
        cache[0] = conv_state_commit(p.conv_state, p.qkv, n_commit, p.mask, self.conv_kernel_size)
        self._pending = None


def commit_verified(mixers: Sequence[GatedDeltaNet], caches: Sequence[ArraysCache], n_commit: IntSeq) -> None:
    """Engine-level rollback of a partially accepted round for every GDN layer.

    The counterpart of ``Engine.rollback_ssm_replay`` (``engine.py:337-359``):
    each layer commits its verified prefix instead of restore + replay.
    """
    for m, c in zip(mixers, caches):
        m.commit(c, n_commit)
