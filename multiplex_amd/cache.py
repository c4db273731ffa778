"""Per-layer GDN recurrent state and the state-movement verbs the engine,
scheduler and prefix cache apply to it.

``ArraysCache`` mirrors the container multiplex keeps for every
GatedDeltaNet layer (mlx-lm's ``ArraysCache``): ``cache[0]`` is the conv
state ``[B, K-1, conv_dim]`` in the activation dtype, ``cache[1]`` the
recurrent state ``[B, Hv, Dv, Dk]`` float32 (``multiplex/kernel/engine.py:
309-320, 424-432``; ``dflash.py:351-376``).  It is not trimmable: rolling
back a speculative round needs the verify/commit pair of the mixer, or a
snapshot.

The verbs are the engine's (``engine.py:300-320`` snapshot/restore,
``:383-393`` filter/extract, ``:424-432`` batch merge) and the prefix
cache's (``prefixcache/state.py:65-78`` clone, ``:122-140`` restore).  They
move whole rows of device tensors; a copy is always a fresh tensor, so later
in-place kernel writes never reach a snapshot (the reference's ``v + 0``).

``cache[1]`` may also be a :class:`~multiplex_amd.state_pool.PooledBatch`
(pool slots instead of a dense array): filter and merge then move slot
indices only, and the copies (extract, clone, snapshot) copy slots.
"""

from __future__ import annotations

from typing import List, Optional, Sequence

import torch

from .state_pool import PooledBatch

__all__ = [
    "ArraysCache",
    "snapshot_ssm",
    "restore_ssm",
    "merge_layer",
    "clone_ssm",
    "restore_ssm_snapshot",
]


def _copy(v):
    """An independent copy: a fresh tensor, or fresh pool slots."""
    if v is None:
        return None
    if isinstance(v, PooledBatch):
        return v.snapshot()
    return v.clone()


class ArraysCache:
    """A fixed-size list of per-row state arrays (``[conv_state, ssm_state]``)."""

    def __init__(self, size: int = 2):
        self.cache: List[Optional[torch.Tensor]] = [None] * size

    def __getitem__(self, i: int) -> Optional[torch.Tensor]:
        return self.cache[i]

    def __setitem__(self, i: int, v: Optional[torch.Tensor]) -> None:
        self.cache[i] = v

    def __len__(self) -> int:
        return len(self.cache)

    @property
    def state(self) -> List[Optional[torch.Tensor]]:
        return self.cache

    @state.setter
    def state(self, v: Sequence[Optional[torch.Tensor]]) -> None:
        self.cache = list(v)

    def is_trimmable(self) -> bool:
        return False

    @property
    def batch_size(self) -> int:
        for v in self.cache:
            if v is not None:
                return int(v.shape[0])
        return 0

    @property
    def nbytes(self) -> int:
        total = 0
        for v in self.cache:
            if isinstance(v, PooledBatch):
                total += len(v) * v.pool.states[0].numel() * v.pool.states.element_size()
            elif v is not None:
                total += v.numel() * v.element_size()
        return total

    def filter(self, batch_indices) -> None:
        """Keep only rows ``batch_indices`` (in that order), in place (``engine.py:383-387``)."""
        for i, v in enumerate(self.cache):
            if isinstance(v, PooledBatch):
                v.filter([int(j) for j in batch_indices])
            elif v is not None:
                idx = torch.as_tensor(batch_indices, dtype=torch.long, device=v.device)
                self.cache[i] = v.index_select(0, idx)

    def extract(self, idx: int) -> "ArraysCache":
        """Row ``idx`` as its own single-row cache, leaving this one unchanged (``engine.py:389-393``)."""
        out = ArraysCache(len(self.cache))
        out.cache = [None if v is None else (v.extract(idx) if isinstance(v, PooledBatch) else v[idx:idx + 1].clone())
                     for v in self.cache]
        return out

    def clone(self) -> "ArraysCache":
        out = ArraysCache(len(self.cache))
        out.cache = [_copy(v) for v in self.cache]
        return out

    @staticmethod
    def merge(caches: Sequence["ArraysCache"]) -> "ArraysCache":
        return merge_layer(caches)


def snapshot_ssm(caches: Sequence[object]) -> list:
    """Copies of every ArraysCache's arrays; None for other layer caches (``engine.py:300-314``)."""
    return [[_copy(v) for v in c.cache] if isinstance(c, ArraysCache) else None for c in caches]


def restore_ssm(caches: Sequence[object], snap: Sequence[Optional[list]]) -> None:
    """Writes a :func:`snapshot_ssm` result back (as copies) (``engine.py:316-320``)."""
    for c, s in zip(caches, snap):
        if s is not None:
            c.cache = [_copy(v) for v in s]


def merge_layer(caches: Sequence[ArraysCache]) -> ArraysCache:
    """Stacks single- or multi-row caches along the batch axis (``engine.py:424-432``).

    Pooled entries are joined without moving states (the merged cache takes
    over the parts' slots).
    """
    out = ArraysCache(len(caches[0].cache))

    def join(i):
        first = caches[0].cache[i]
        if first is None:
            return None
        if isinstance(first, PooledBatch):
            return PooledBatch.merge([c.cache[i] for c in caches])
        return torch.cat([c.cache[i] for c in caches], dim=0)

    out.cache = [join(i) for i in range(len(caches[0].cache))]
    return out


def clone_ssm(caches: Sequence[object]) -> list:
    """Prefix-cache snapshot at a reusable boundary (``prefixcache/state.py:65-78``)."""
    return snapshot_ssm(caches)


def restore_ssm_snapshot(caches: Sequence[object], ssm_snapshot: Sequence[Optional[list]]) -> None:
    """Seeds fresh caches from a prefix-cache snapshot (``prefixcache/state.py:122-129``)."""
    restore_ssm(caches, ssm_snapshot)
