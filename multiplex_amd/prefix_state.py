"""Prefix-cache records of GDN state on disk, with an asynchronous
device -> host -> disk path and its reverse.

multiplex keeps, at every reusable prefix boundary, each GDN layer's
``[conv_state, ssm_state]`` (``multiplex/kernel/prefixcache/state.py:65-78``)
and persists it through its disk store (``prefixcache/disk.py``).  This
module reads and writes that store's format, version 1, for torch tensors,
so records written on either side load on the other.  The format is an
interface; it is restated here (and is the contract the tests check bytes
against):

Spec nodes, JSON objects whose ``"k"`` names the kind:

* ``{"k": "none"}``; ``{"k": "int", "v": n}`` (bools are ints);
  ``{"k": "tuple" | "list", "v": [node, ...]}``;
* ``{"k": "tensor", "sha": hex, "dtype": name, "shape": [...], "nbytes": n}``;
* ``{"k": "blocks", "dtype", "shape", "axis": 2, "block_size": b,
  "blocks": [{"sha", "start", "end", "shape", "nbytes"}, ...]}`` for an array
  of rank >= 3 with ``shape[2] >= 2 b``: block i holds ``[i b, min((i+1) b,
  shape[2]))`` of axis 2.  ``b`` defaults to 256.

``dtype`` is one of bool, uint8/16/32/64, int8/16/32/64, float16/32/64 and
bfloat16.  A blob is the C-order little-endian bytes of one (block) array,
bfloat16 as its 16-bit pattern, named by the lowercase SHA-256 hex digest of
those bytes and stored at ``blobs/<sha[:2]>/<sha>.bin``.  A record is
``records/<key[:2]>/<key>.json``: one compact JSON object with ``version``
(1), ``key``, ``parent``, ``tokens``, ``start``, ``pos``, ``pool``,
``source``, ``touch``, ``attn``, ``ssm`` and ``cached_h``.  Blobs and
records are each written whole under a temporary name and renamed into
place, blobs first, so a reader never sees a record whose blobs are missing
or a partial file.

Device side: :func:`stage_to_host` queues device -> pinned-host copies on a
side stream behind the current stream's work and returns at once;
:class:`AsyncStateWriter` waits for them on a worker thread, encodes, and
writes.  :func:`load_tree` decodes a spec and uploads it asynchronously.
"""

from __future__ import annotations

import hashlib
import itertools
import json
import os
import sys
import threading
from concurrent.futures import Future, ThreadPoolExecutor
from dataclasses import dataclass, field
from pathlib import Path
from typing import Any, Callable, Dict, Iterator, List, Optional, Sequence, Tuple

import numpy as np
import torch

__all__ = [
    "RECORD_FORMAT_VERSION",
    "axis2_blocks",
    "encode_tree",
    "decode_tree",
    "spec_nbytes",
    "ContentStore",
    "StateRecord",
    "write_json_atomic",
    "stage_to_host",
    "StagedTree",
    "AsyncStateWriter",
    "load_tree",
]

RECORD_FORMAT_VERSION = 1
DEFAULT_BLOCK_SIZE = 256

if sys.byteorder != "little":  # blobs are the little-endian bytes as they lie in host memory
    raise ImportError("prefix_state needs a little-endian host")

# format dtype name -> (torch dtype, torch dtype whose bits are stored)
_DTYPES: Dict[str, Tuple[torch.dtype, torch.dtype]] = {
    "bool": (torch.bool, torch.bool),
    "uint8": (torch.uint8, torch.uint8),
    "uint16": (torch.uint16, torch.uint16),
    "uint32": (torch.uint32, torch.uint32),
    "uint64": (torch.uint64, torch.uint64),
    "int8": (torch.int8, torch.int8),
    "int16": (torch.int16, torch.int16),
    "int32": (torch.int32, torch.int32),
    "int64": (torch.int64, torch.int64),
    "float16": (torch.float16, torch.float16),
    "float32": (torch.float32, torch.float32),
    "float64": (torch.float64, torch.float64),
    "bfloat16": (torch.bfloat16, torch.int16),
}
_NAMES = {dt: name for name, (dt, _) in _DTYPES.items()}


def _format_dtype(t: torch.Tensor) -> str:
    name = _NAMES.get(t.dtype)
    if name is None:
        raise TypeError(f"{t.dtype} has no prefix-cache blob encoding")
    return name


def axis2_blocks(shape: Sequence[int], block_size: int = DEFAULT_BLOCK_SIZE) -> Optional[List[Tuple[int, int]]]:
    """The ``[start, end)`` ranges of axis 2 an array of ``shape`` is cut
    into, or None when it is stored whole (rank < 3 or fewer than two
    blocks' worth of axis 2)."""
    b = max(1, int(block_size))
    if len(shape) < 3 or shape[2] < 2 * b:
        return None
    n = int(shape[2])
    return [(s, min(n, s + b)) for s in range(0, n, b)]


def _blob_bytes(t: torch.Tensor) -> bytes:
    """C-order bytes of a host tensor in the format's encoding."""
    stored = _DTYPES[_format_dtype(t)][1]
    host = t.detach().to("cpu").contiguous()
    if stored != host.dtype:
        host = host.view(stored)
    return host.numpy().tobytes() if host.numel() else b""


# ------------------------------------------------------------------ encode

class _Encoder:
    """Builds a spec tree and the blobs it names (deduplicated by digest)."""

    def __init__(self, block_size: int):
        self.block_size = max(1, int(block_size))
        self.blobs: Dict[str, bytes] = {}

    def _intern(self, raw: bytes) -> str:
        sha = hashlib.sha256(raw).hexdigest()
        if sha not in self.blobs:
            self.blobs[sha] = raw
        return sha

    def node(self, value: Any) -> Dict[str, Any]:
        if value is None:
            return {"k": "none"}
        if isinstance(value, torch.Tensor):
            return self._array(value)
        if isinstance(value, (bool, int, np.integer)):
            return {"k": "int", "v": int(value)}
        if isinstance(value, (tuple, list)):
            return {"k": "tuple" if isinstance(value, tuple) else "list", "v": [self.node(x) for x in value]}
        raise TypeError(f"a prefix-cache tree holds None, ints, tensors, tuples and lists, not {type(value)!r}")

    def _array(self, t: torch.Tensor) -> Dict[str, Any]:
        dtype = _format_dtype(t)
        shape = [int(d) for d in t.shape]
        cuts = axis2_blocks(shape, self.block_size)
        if cuts is None:
            raw = _blob_bytes(t)
            return {"k": "tensor", "sha": self._intern(raw), "dtype": dtype, "shape": shape, "nbytes": len(raw)}
        blocks = []
        for start, end in cuts:
            raw = _blob_bytes(t[:, :, start:end])
            blocks.append({"sha": self._intern(raw), "start": start, "end": end,
                           "shape": [shape[0], shape[1], end - start, *shape[3:]], "nbytes": len(raw)})
        return {"k": "blocks", "dtype": dtype, "shape": shape, "axis": 2, "block_size": self.block_size,
                "blocks": blocks}


def encode_tree(value: Any, *, block_size: int = DEFAULT_BLOCK_SIZE) -> Tuple[Dict[str, Any], Dict[str, bytes]]:
    """``(spec, blobs)`` of a snapshot tree (None, ints, tensors, tuples,
    lists).  Device tensors are copied to the host synchronously; stage them
    with :func:`stage_to_host` for the asynchronous path."""
    enc = _Encoder(block_size)
    return enc.node(value), enc.blobs


# ------------------------------------------------------------------ decode

class _Decoder:
    def __init__(self, read_blob: Callable[[str], bytes]):
        self.read_blob = read_blob

    def node(self, spec: Any) -> Any:
        kind = spec.get("k") if isinstance(spec, dict) else None
        handler = {"none": self._none, "int": self._int, "tuple": self._seq, "list": self._seq,
                   "tensor": self._tensor, "blocks": self._blocks}.get(kind)
        if handler is None:
            raise ValueError(f"not a prefix-cache spec node (kind {kind!r})")
        return handler(spec)

    def _none(self, spec):
        return None

    def _int(self, spec):
        return int(spec["v"])

    def _seq(self, spec):
        items = [self.node(x) for x in spec.get("v", [])]
        return tuple(items) if spec["k"] == "tuple" else items

    def _fill(self, dst: torch.Tensor, sha: str, dtype: str) -> None:
        """Copies blob ``sha`` into ``dst`` (a host tensor of its shape)."""
        raw = self.read_blob(str(sha))
        stored = _DTYPES[dtype][1]
        want = dst.numel() * dst.element_size()
        if len(raw) != want:
            raise ValueError(f"blob {sha}: {len(raw)} bytes where a {dtype} {list(dst.shape)} takes {want}")
        if want:
            src = torch.frombuffer(bytearray(raw), dtype=stored).reshape(dst.shape)
            dst.copy_(src.view(dst.dtype) if stored != dst.dtype else src)

    def _tensor(self, spec):
        dtype = str(spec["dtype"])
        out = torch.empty([int(d) for d in spec["shape"]], dtype=_DTYPES[dtype][0])
        self._fill(out, spec["sha"], dtype)
        return out

    def _blocks(self, spec):
        dtype = str(spec["dtype"])
        out = torch.zeros([int(d) for d in spec.get("shape") or []], dtype=_DTYPES[dtype][0])
        axis = int(spec.get("axis", 2))
        for blk in spec.get("blocks", []):
            self._fill(out.narrow(axis, int(blk["start"]), int(blk["end"]) - int(blk["start"])), blk["sha"], dtype)
        return out


def decode_tree(spec: Any, read_blob: Callable[[str], bytes]) -> Any:
    """The host tree a spec describes; ``read_blob(sha)`` returns a blob's bytes."""
    return _Decoder(read_blob).node(spec)


def _walk_specs(spec: Any) -> Iterator[Dict[str, Any]]:
    stack = [spec]
    while stack:
        x = stack.pop()
        if isinstance(x, dict):
            yield x
            stack.extend(v for v in x.values() if isinstance(v, (dict, list)))
        elif isinstance(x, list):
            stack.extend(x)


def spec_nbytes(spec: Any) -> int:
    """Array bytes a spec accounts for (every tensor node and block)."""
    total = 0
    for node in _walk_specs(spec):
        if node.get("k") == "tensor":
            total += int(node.get("nbytes", 0))
        elif node.get("k") == "blocks":
            total += sum(int(b.get("nbytes", 0)) for b in node.get("blocks", []))
    return total


# ------------------------------------------------------------------- files

_tmp_seq = itertools.count()
_tmp_lock = threading.Lock()


def _replace_into(path: Path, data: bytes) -> None:
    """Writes ``data`` to ``path`` whole: a uniquely named sibling, then a rename."""
    path.parent.mkdir(parents=True, exist_ok=True)
    with _tmp_lock:
        n = next(_tmp_seq)
    tmp = path.parent / f".{path.name}.{os.getpid()}.{threading.get_ident()}.{n}.part"
    try:
        with open(tmp, "xb") as f:
            f.write(data)
        os.replace(tmp, path)
    except BaseException:
        tmp.unlink(missing_ok=True)
        raise


def write_json_atomic(path, data: Any) -> None:
    """Compact UTF-8 JSON at ``path``, replaced whole."""
    text = json.dumps(data, ensure_ascii=False, separators=(",", ":"))
    _replace_into(Path(path), text.encode("utf-8"))


class ContentStore:
    """Blobs by content under ``<root>/blobs/<sha[:2]>/<sha>.bin``."""

    def __init__(self, root):
        self.root = Path(root).expanduser()

    def blob_path(self, sha: str) -> Path:
        return self.root / "blobs" / sha[:2] / f"{sha}.bin"

    def put_many(self, blobs: Dict[str, bytes]) -> Tuple[int, int]:
        """Stores the blobs not yet present; returns ``(written, present)``."""
        written = 0
        for sha, raw in blobs.items():
            p = self.blob_path(sha)
            if not p.exists():
                _replace_into(p, raw)
                written += 1
        return written, len(blobs) - written

    def get(self, sha: str) -> bytes:
        return self.blob_path(sha).read_bytes()


@dataclass
class StateRecord:
    """One record file of the store (the format's record object)."""

    key: str
    ssm: Any
    parent: Optional[str] = None
    tokens: List[int] = field(default_factory=list)
    start: int = 0
    pos: int = 0
    pool: str = "default"
    source: Optional[str] = None
    touch: int = 0
    attn: Any = None
    cached_h: Any = None

    def to_json(self) -> Dict[str, Any]:
        return {"version": RECORD_FORMAT_VERSION, "key": self.key, "parent": self.parent,
                "tokens": [int(t) for t in self.tokens], "start": int(self.start), "pos": int(self.pos),
                "pool": self.pool, "source": self.source, "touch": int(self.touch), "attn": self.attn,
                "ssm": self.ssm, "cached_h": self.cached_h}

    @classmethod
    def from_json(cls, obj: Dict[str, Any]) -> "StateRecord":
        if obj.get("version") != RECORD_FORMAT_VERSION:
            raise ValueError(f"record format version {obj.get('version')!r}; this reader knows "
                             f"{RECORD_FORMAT_VERSION}")
        return cls(key=obj["key"], ssm=obj.get("ssm"), parent=obj.get("parent"), tokens=list(obj.get("tokens", [])),
                   start=obj.get("start", 0), pos=obj.get("pos", 0), pool=obj.get("pool", "default"),
                   source=obj.get("source"), touch=obj.get("touch", 0), attn=obj.get("attn"),
                   cached_h=obj.get("cached_h"))


# ------------------------------------------------------------- device side

def _tensors(tree: Any) -> List[torch.Tensor]:
    out: List[torch.Tensor] = []
    stack = [tree]
    while stack:
        x = stack.pop()
        if isinstance(x, torch.Tensor):
            out.append(x)
        elif isinstance(x, (list, tuple)):
            stack.extend(x)
    return out


def _rebuild(tree: Any, fn: Callable[[torch.Tensor], torch.Tensor]) -> Any:
    if isinstance(tree, torch.Tensor):
        return fn(tree)
    if isinstance(tree, (list, tuple)):
        items = [_rebuild(x, fn) for x in tree]
        return tuple(items) if isinstance(tree, tuple) else items
    return tree


class StagedTree:
    """A snapshot on its way to pinned host memory (from :func:`stage_to_host`)."""

    def __init__(self, host: Any, done: Optional["torch.cuda.Event"]):
        self._host = host
        self._done = done

    def ready(self) -> bool:
        return self._done is None or self._done.query()

    def wait(self) -> Any:
        """The host tree, once every copy has landed."""
        if self._done is not None:
            self._done.synchronize()
            self._done = None
        return self._host


def stage_to_host(tree: Any, stream: Optional["torch.cuda.Stream"] = None) -> StagedTree:
    """Queues device -> pinned-host copies of every device tensor in
    ``tree`` and returns at once.

    The copies run on ``stream`` (a new side stream of default priority when
    None), behind the work already queued on the current stream, so the
    snapshot holds the state the preceding kernels wrote.  Work queued on
    the current stream *after* this call may run before the copies: a
    caller that snapshots live state it is about to update in place (e.g.
    decode with ``state_out=state``) must not queue that update before
    :meth:`StagedTree.ready` (or clone first, as ``clone_ssm`` does).  Each
    source tensor is marked as used on the side stream, so its memory is not
    reused while a copy is pending even if the caller drops it.
    """
    cuda = [t for t in _tensors(tree) if t.device.type == "cuda"]
    if not cuda:
        return StagedTree(_rebuild(tree, lambda t: t.detach().clone()), None)
    dev = cuda[0].device
    side = stream if stream is not None else torch.cuda.Stream(dev)
    side.wait_stream(torch.cuda.current_stream(dev))

    def copy(t: torch.Tensor) -> torch.Tensor:
        if t.device.type != "cuda":
            return t.detach().clone()
        h = torch.empty(t.shape, dtype=t.dtype, pin_memory=True)
        t.record_stream(side)
        h.copy_(t, non_blocking=True)
        return h

    with torch.cuda.stream(side):
        host = _rebuild(tree, copy)
        done = torch.cuda.Event()
        done.record(side)
    return StagedTree(host, done)


def load_tree(spec: Any, read_blob: Callable[[str], bytes], device=None) -> Any:
    """Decodes a spec; with a ROCm ``device``, uploads every tensor through
    pinned memory with asynchronous copies on the current stream (ahead of
    any kernel queued after this call)."""
    host = decode_tree(spec, read_blob)
    if device is None or torch.device(device).type != "cuda":
        return host
    return _rebuild(host, lambda t: t.pin_memory().to(device, non_blocking=True))


class AsyncStateWriter:
    """Writes state records in the background (the GDN-state part of
    multiplex's ``AsyncPrefixDiskStore``, ``disk.py:305-573``).

    :meth:`submit` hands a :class:`StagedTree` (or a host tree) and the
    record fields to a single worker thread, which waits for the staged
    copies, encodes the tree, stores its blobs and then the record.
    """

    def __init__(self, base_dir, *, block_size: int = DEFAULT_BLOCK_SIZE):
        self.base_dir = Path(base_dir).expanduser()
        self.blobs = ContentStore(self.base_dir)
        self.block_size = int(block_size)
        self._pool = ThreadPoolExecutor(max_workers=1, thread_name_prefix="gdn-state-writer")
        self._pending: List[Future] = []
        self.written = 0

    def record_path(self, key: str) -> Path:
        return self.base_dir / "records" / key[:2] / f"{key}.json"

    def submit(self, key: str, ssm, **fields) -> Future:
        """Queues one record; ``fields`` are the other :class:`StateRecord` fields."""
        rec = StateRecord(key=str(key), ssm=None, **fields)
        fut = self._pool.submit(self._write, rec, ssm)
        self._pending.append(fut)
        return fut

    def _write(self, rec: StateRecord, ssm) -> None:
        tree = ssm.wait() if isinstance(ssm, StagedTree) else ssm
        rec.ssm, blobs = encode_tree(tree, block_size=self.block_size)
        self.blobs.put_many(blobs)
        write_json_atomic(self.record_path(rec.key), rec.to_json())
        self.written += 1

    def flush(self) -> None:
        """Waits for every queued record; raises the first failure."""
        pending, self._pending = self._pending, []
        errors = [f.exception() for f in pending]
        errors = [e for e in errors if e is not None]
        if errors:
            raise RuntimeError(f"{len(errors)} state record(s) failed to write") from errors[0]

    def read_record(self, key: str) -> StateRecord:
        return StateRecord.from_json(json.loads(self.record_path(key).read_text(encoding="utf-8")))

    def load_ssm(self, key: str, device=None) -> Any:
        return load_tree(self.read_record(key).ssm, self.blobs.get, device)

    def close(self) -> None:
        self.flush()
        self._pool.shutdown(wait=True)
