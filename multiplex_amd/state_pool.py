"""Pooled recurrent states: batch membership moves slot indices, not states.

multiplex keeps each GDN layer's recurrent state as one dense
``[B, Hv, Dv, Dk]`` float32 array per running batch and rebuilds it whenever
the batch changes: ``filter`` / ``extract_row`` slice it
(``multiplex/kernel/engine.py:383-393``), a join concatenates
(``engine.py:424-432``), and snapshots copy it (``engine.py:300-320``,
``prefixcache/state.py:65-78``).  Every such step copies 2 MiB per row and
layer at Hv=32, Dk=Dv=128.

Here the states of all rows live in one pool ``[n_slots, Hv, Dv, Dk]`` per
layer, and a batch is a list of slots.  The kernels read and write
``pool[slot[b]]`` through the ``state_index`` argument of
:func:`gated_delta_update`, :func:`gated_delta_verify`,
:func:`gated_delta_commit` and the chunked prefill, so filter and merge
change only the slot list (an int32 tensor of B entries).  Copies remain
where the reference semantics need an independent state: extracting a row,
a snapshot (:meth:`PooledBatch.snapshot`) and export to a dense array
(:meth:`StatePool.gather`).

Slots are managed on the host (one engine thread drives the scheduler,
``multiplex/kernel/hub.py:7-13``), so the index tensors are valid by
construction; the kernels also skip any row whose slot lies outside the
pool rather than touch memory beyond it.
"""

from __future__ import annotations

from typing import Iterable, List, Optional, Sequence

import torch

__all__ = ["StatePool", "PooledBatch"]


class StatePool:
    """``n_slots`` float32 GDN states ``[Hv, Dv, Dk]`` in one device tensor."""

    def __init__(self, n_slots: int, num_v_heads: int, head_v_dim: int, head_k_dim: int, device=None):
        if n_slots <= 0:
            raise ValueError("a pool needs at least one slot")
        self.states = torch.zeros(n_slots, num_v_heads, head_v_dim, head_k_dim, dtype=torch.float32,
                                  device=device)
        self._free: List[int] = list(range(n_slots - 1, -1, -1))  # pop() hands out the lowest slot first
        self._used = set()

    @property
    def n_slots(self) -> int:
        return int(self.states.shape[0])

    @property
    def n_free(self) -> int:
        return len(self._free)

    @property
    def device(self) -> torch.device:
        return self.states.device

    def alloc(self, n: int = 1, *, zero: bool = True) -> List[int]:
        """Takes ``n`` free slots (zeroed unless ``zero=False``, e.g. when a prefill writes them whole)."""
        if n < 0:
            raise ValueError("n must be >= 0")
        if n > len(self._free):
            raise RuntimeError(f"state pool exhausted: {n} slots asked, {len(self._free)} free")
        slots = [self._free.pop() for _ in range(n)]
        self._used.update(slots)
        if zero and slots:
            self.states.index_fill_(0, self.index(slots).long(), 0.0)
        return slots

    def release(self, slots: Iterable[int]) -> None:
        """Returns slots to the pool; their contents are left as they are."""
        slots = [int(s) for s in slots]
        for s in slots:
            if s not in self._used:
                raise ValueError(f"slot {s} is not allocated")
        for s in slots:
            self._used.discard(s)
            self._free.append(s)
        self._free.sort(reverse=True)

    def index(self, slots: Sequence[int]) -> torch.Tensor:
        """The int32 device tensor the kernels take as ``state_index``.

        On a GPU the slot list goes through pinned host memory and an
        asynchronous copy on the current stream, so no launch waits for it.
        """
        host = torch.tensor([int(s) for s in slots], dtype=torch.int32)
        if self.device.type != "cuda":
            return host
        return host.pin_memory().to(self.device, non_blocking=True)

    def gather(self, slots: Sequence[int]) -> torch.Tensor:
        """A dense copy ``[len(slots), Hv, Dv, Dk]`` (export, e.g. to a dense ArraysCache)."""
        return self.states.index_select(0, self.index(slots).long())

    def scatter(self, slots: Sequence[int], states: torch.Tensor) -> None:
        """Writes dense states into ``slots`` (import, e.g. a prefix-cache restore)."""
        if states.shape[0] != len(slots) or states.shape[1:] != self.states.shape[1:]:
            raise ValueError(f"states must be [{len(slots)}, {', '.join(map(str, self.states.shape[1:]))}]")
        self.states.index_copy_(0, self.index(slots).long(), states.to(self.states.dtype))

    def copy_slots(self, src: Sequence[int], dst: Sequence[int]) -> None:
        """``pool[dst[i]] = pool[src[i]]`` (a device copy of 64 KiB per head)."""
        if len(src) != len(dst):
            raise ValueError("src and dst must have the same length")
        if src:
            self.states.index_copy_(0, self.index(dst).long(), self.states.index_select(0, self.index(src).long()))


class PooledBatch:
    """The rows of one running batch as pool slots (row b -> ``slots[b]``).

    The pooled counterpart of ``cache[1]`` of multiplex's per-layer
    ArraysCache (an ArraysCache and the GatedDeltaNet mixer accept one in
    that place); pass ``pool.states`` as the state and :attr:`index` as
    ``state_index``.

    A batch owns its slots: they return to the pool when the batch is
    released or garbage-collected (as the reference's arrays are freed).
    ``merge`` hands the parts' slots to the merged batch; ``extract``,
    ``snapshot`` and ``clone`` copy into fresh slots, as the reference's
    ``extract`` and ``v + 0`` copies do.
    """

    def __init__(self, pool: StatePool, slots: Sequence[int]):
        self.pool = pool
        self.slots = [int(s) for s in slots]
        if len(set(self.slots)) != len(self.slots):
            raise ValueError("a batch cannot hold one slot twice")
        self._index: Optional[torch.Tensor] = None

    def __del__(self):
        try:
            if self.slots:
                self.pool.release(self.slots)
                self.slots = []
        except Exception:  # interpreter shutdown or an already-released slot
            pass

    @property
    def shape(self):
        """``[rows, Hv, Dv, Dk]``, like the dense state it stands for."""
        return (len(self.slots),) + tuple(self.pool.states.shape[1:])

    @classmethod
    def new(cls, pool: StatePool, rows: int) -> "PooledBatch":
        """``rows`` fresh rows with zero states."""
        return cls(pool, pool.alloc(rows))

    def __len__(self) -> int:
        return len(self.slots)

    @property
    def index(self) -> torch.Tensor:
        if self._index is None:
            self._index = self.pool.index(self.slots)
        return self._index

    def _set(self, slots: List[int]) -> None:
        self.slots = slots
        self._index = None

    def filter(self, keep: Sequence[int]) -> None:
        """Keeps rows ``keep`` in that order (``engine.py:383-387``); dropped rows' slots are released."""
        keep = [int(i) for i in keep]
        if len(set(keep)) != len(keep):
            raise ValueError("filter cannot keep a row twice (two rows would share one state)")
        kept = [self.slots[i] for i in keep]
        dropped = set(self.slots) - set(kept)
        self.pool.release(sorted(dropped))
        self._set(kept)

    def extract(self, b: int) -> "PooledBatch":
        """A copy of row ``b`` as its own batch, this one unchanged (``engine.py:389-393``)."""
        dst = self.pool.alloc(1, zero=False)
        self.pool.copy_slots([self.slots[b]], dst)
        return PooledBatch(self.pool, dst)

    @staticmethod
    def merge(batches: Sequence["PooledBatch"]) -> "PooledBatch":
        """Concatenates batches of one pool along the rows (``engine.py:424-432``).

        No state moves: the merged batch takes over the parts' slots and the
        parts are left empty.
        """
        pool = batches[0].pool
        if any(b.pool is not pool for b in batches):
            raise ValueError("batches of different pools cannot be merged")
        slots = [s for b in batches for s in b.slots]
        for b in batches:
            b._set([])
        return PooledBatch(pool, slots)

    def snapshot(self) -> "PooledBatch":
        """Independent copies of every row's state in fresh slots (``prefixcache/state.py:65-78``)."""
        dst = self.pool.alloc(len(self.slots), zero=False)
        self.pool.copy_slots(self.slots, dst)
        return PooledBatch(self.pool, dst)

    clone = snapshot

    def restore(self, snap: "PooledBatch") -> None:
        """Writes ``snap``'s states back into this batch's slots (``engine.py:316-320``)."""
        if len(snap) != len(self):
            raise ValueError("snapshot and batch differ in rows")
        self.pool.copy_slots(snap.slots, self.slots)

    def release(self) -> None:
        self.pool.release(self.slots)
        self._set([])
