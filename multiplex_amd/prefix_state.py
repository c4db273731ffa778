"""Prefix-cache records of GDN state, in multiplex's on-disk format, with an
asynchronous device -> host -> disk path and its reverse.

multiplex snapshots every GDN layer's ``[conv_state, ssm_state]`` at a
reusable prefix boundary (``multiplex/kernel/prefixcache/state.py:65-78``)
and its disk store persists the snapshot as a tree spec in a JSON record
plus content-addressed blobs (``multiplex/kernel/prefixcache/disk.py``):

* ``encode_tree`` (``disk.py:106-163``): ``None`` -> ``{"k": "none"}``, ints
  -> ``{"k": "int", "v": n}``, tuples / lists -> ``{"k": "tuple"|"list",
  "v": [...]}``, an array -> ``{"k": "tensor", "sha", "dtype", "shape",
  "nbytes"}``; an array of rank >= 3 whose axis 2 holds at least two blocks
  (``block_size``, default 256) is cut along axis 2 into ``{"k": "blocks",
  "dtype", "shape", "axis": 2, "block_size", "blocks": [{"sha", "start",
  "end", "shape", "nbytes"}, ...]}``.
* a blob is the array's C-order little-endian bytes (bfloat16 as its 16-bit
  pattern, ``disk.py:715-722``), named by the SHA-256 hex digest of those
  bytes and stored at ``blobs/<digest[:2]>/<digest>.bin``, written to a
  temporary file and renamed (``disk.py:192-225``).
* a record is ``records/<key[:2]>/<key>.json`` with ``version`` =
  ``RECORD_FORMAT_VERSION`` (1), written last and atomically
  (``disk.py:24, 272-302, 543-573, 601-605, 691-697``).

The same spec and bytes come out here for torch tensors, so either side can
read the other's store.  The GPU part: :func:`stage_to_host` copies a
device snapshot into pinned host memory on a side stream and returns at
once; the :class:`AsyncStateWriter` thread waits for that copy, hashes and
writes.  :func:`load_tree` reads a spec back and uploads it asynchronously.
"""

from __future__ import annotations

import hashlib
import json
import os
import queue
import sys
import tempfile
import threading
from pathlib import Path
from typing import Any, Callable, Dict, Optional, Tuple

import numpy as np
import torch

__all__ = [
    "RECORD_FORMAT_VERSION",
    "encode_tree",
    "decode_tree",
    "spec_nbytes",
    "BlobStore",
    "write_json_atomic",
    "stage_to_host",
    "StagedTree",
    "AsyncStateWriter",
    "load_tree",
]

RECORD_FORMAT_VERSION = 1
DEFAULT_BLOCK_SIZE = 256

# dtype names of the format (MLX's names) <-> torch dtypes
_TORCH_BY_NAME = {
    "bool": torch.bool, "uint8": torch.uint8, "int8": torch.int8, "int16": torch.int16,
    "int32": torch.int32, "int64": torch.int64, "float16": torch.float16, "float32": torch.float32,
    "float64": torch.float64, "bfloat16": torch.bfloat16,
}
_NAME_BY_TORCH = {v: k for k, v in _TORCH_BY_NAME.items()}

if sys.byteorder != "little":  # the format stores little-endian bytes as they lie in memory
    raise ImportError("prefix_state needs a little-endian host")


def _dtype_name(t: torch.Tensor) -> str:
    try:
        return _NAME_BY_TORCH[t.dtype]
    except KeyError:
        raise TypeError(f"unsupported dtype for a prefix-cache blob: {t.dtype}") from None


def _raw_bytes(t: torch.Tensor) -> bytes:
    """C-order little-endian bytes of a host tensor (bfloat16 as its bit pattern)."""
    t = t.detach()
    if t.device.type != "cpu":
        t = t.cpu()
    t = t.contiguous()
    if t.dtype == torch.bfloat16:
        t = t.view(torch.int16)
    return t.numpy().tobytes()


def encode_tree(value: Any, *, block_size: int = DEFAULT_BLOCK_SIZE) -> Tuple[Any, Dict[str, bytes]]:
    """``(spec, blobs)`` of a snapshot tree, as multiplex's ``encode_tree``.

    Leaves are None, ints and tensors (host tensors; a device tensor is
    copied to the host synchronously -- stage it first for the async path).
    """
    blobs: Dict[str, bytes] = {}
    block_size = max(1, int(block_size))

    def put(raw: bytes) -> str:
        digest = hashlib.sha256(raw).hexdigest()
        blobs.setdefault(digest, raw)
        return digest

    def tensor(t: torch.Tensor) -> Any:
        shape = [int(d) for d in t.shape]
        dtype = _dtype_name(t)
        if len(shape) >= 3 and shape[2] >= 2 * block_size:
            blocks = []
            for start in range(0, shape[2], block_size):
                end = min(shape[2], start + block_size)
                raw = _raw_bytes(t[:, :, start:end])
                blocks.append({"sha": put(raw), "start": start, "end": end,
                               "shape": shape[:2] + [end - start] + shape[3:], "nbytes": len(raw)})
            return {"k": "blocks", "dtype": dtype, "shape": shape, "axis": 2, "block_size": block_size,
                    "blocks": blocks}
        raw = _raw_bytes(t)
        return {"k": "tensor", "sha": put(raw), "dtype": dtype, "shape": shape, "nbytes": len(raw)}

    def enc(v: Any) -> Any:
        if v is None:
            return {"k": "none"}
        if isinstance(v, (int, np.integer)):  # Python bools are ints here too
            return {"k": "int", "v": int(v)}
        if isinstance(v, torch.Tensor):
            return tensor(v)
        if isinstance(v, tuple):
            return {"k": "tuple", "v": [enc(x) for x in v]}
        if isinstance(v, list):
            return {"k": "list", "v": [enc(x) for x in v]}
        raise TypeError(f"unsupported prefix cache leaf: {type(v)!r}")

    return enc(value), blobs


def _decode_tensor(spec: Dict[str, Any], read_blob: Callable[[str], bytes]) -> torch.Tensor:
    dtype = _TORCH_BY_NAME[str(spec["dtype"])]
    raw = bytearray(read_blob(str(spec["sha"])))
    shape = tuple(int(d) for d in spec["shape"])
    if len(raw) != int(np.prod(shape, dtype=np.int64)) * torch.empty(0, dtype=dtype).element_size():
        raise ValueError(f"blob {spec['sha']} holds {len(raw)} bytes, not a {spec['dtype']} {list(shape)}")
    if len(raw) == 0:
        return torch.empty(shape, dtype=dtype)
    return torch.frombuffer(raw, dtype=dtype).reshape(shape)


def decode_tree(spec: Any, read_blob: Callable[[str], bytes]) -> Any:
    """The host tensors of a spec (multiplex's ``decode_tree``)."""
    kind = spec.get("k") if isinstance(spec, dict) else None
    if kind == "none":
        return None
    if kind == "int":
        return int(spec["v"])
    if kind == "tuple":
        return tuple(decode_tree(x, read_blob) for x in spec.get("v", []))
    if kind == "list":
        return [decode_tree(x, read_blob) for x in spec.get("v", [])]
    if kind == "tensor":
        return _decode_tensor(spec, read_blob)
    if kind == "blocks":
        shape = tuple(int(d) for d in spec.get("shape") or [])
        parts = [_decode_tensor({**b, "dtype": spec["dtype"]}, read_blob) for b in spec.get("blocks", [])]
        if not parts:
            return torch.zeros(shape, dtype=_TORCH_BY_NAME[str(spec["dtype"])])
        return torch.cat(parts, dim=int(spec.get("axis", 2))).reshape(shape)
    raise ValueError(f"unsupported prefix cache spec kind: {kind!r}")


def spec_nbytes(spec: Any) -> int:
    """Tensor bytes a spec accounts for (multiplex's ``spec_nbytes``)."""
    if isinstance(spec, dict):
        kind = spec.get("k")
        if kind == "tensor":
            return int(spec.get("nbytes", 0))
        if kind == "blocks":
            return sum(int(b.get("nbytes", 0)) for b in spec.get("blocks", []))
        return sum(spec_nbytes(v) for v in spec.values())
    if isinstance(spec, list):
        return sum(spec_nbytes(v) for v in spec)
    return 0


class BlobStore:
    """Content-addressed blobs under ``<base>/blobs/<digest[:2]>/<digest>.bin``."""

    def __init__(self, base_dir):
        self.base_dir = Path(base_dir).expanduser()

    def path(self, digest: str) -> Path:
        return self.base_dir / "blobs" / digest[:2] / f"{digest}.bin"

    def write_blobs(self, blobs: Dict[str, bytes]) -> Tuple[int, int]:
        """Writes missing blobs (temporary file + rename); returns ``(wrote, deduped)``."""
        wrote = deduped = 0
        for digest, raw in blobs.items():
            p = self.path(digest)
            if p.exists():
                deduped += 1
                continue
            p.parent.mkdir(parents=True, exist_ok=True)
            fd, tmp = tempfile.mkstemp(prefix=f".{p.name}.tmp-", dir=str(p.parent))
            try:
                with os.fdopen(fd, "wb") as f:
                    f.write(raw)
                os.replace(tmp, p)
                wrote += 1
            except BaseException:
                try:
                    os.unlink(tmp)
                except OSError:
                    pass
                raise
        return wrote, deduped

    def read_blob(self, digest: str) -> bytes:
        return self.path(digest).read_bytes()


def write_json_atomic(path, data: Any) -> None:
    path = Path(path)
    path.parent.mkdir(parents=True, exist_ok=True)
    tmp = path.with_suffix(path.suffix + ".tmp")
    tmp.write_text(json.dumps(data, ensure_ascii=False, separators=(",", ":")), encoding="utf-8")
    os.replace(tmp, path)


# ------------------------------------------------------------- device side

def _map(tree: Any, fn: Callable[[torch.Tensor], torch.Tensor]) -> Any:
    if isinstance(tree, torch.Tensor):
        return fn(tree)
    if isinstance(tree, list):
        return [_map(x, fn) for x in tree]
    if isinstance(tree, tuple):
        return tuple(_map(x, fn) for x in tree)
    return tree


class StagedTree:
    """A snapshot tree on its way to pinned host memory."""

    def __init__(self, host: Any, event: Optional["torch.cuda.Event"], keep: Any):
        self._host = host
        self._event = event
        self._keep = keep  # the device tensors stay alive until the copy is done

    def ready(self) -> bool:
        return self._event is None or self._event.query()

    def wait(self) -> Any:
        """The host tree, once the copies have landed."""
        if self._event is not None:
            self._event.synchronize()
            self._event = None
            self._keep = None
        return self._host


def stage_to_host(tree: Any, stream: Optional["torch.cuda.Stream"] = None) -> StagedTree:
    """Starts device -> pinned-host copies of every tensor in ``tree``; returns at once.

    The copies run on ``stream`` (a side stream of default priority by
    default) after the work already queued on the current stream, so a
    snapshot taken right after a kernel sees its result.
    """
    dev_tensors = []
    _map(tree, lambda t: dev_tensors.append(t) or t)
    cuda = [t for t in dev_tensors if t.device.type == "cuda"]
    if not cuda:
        return StagedTree(_map(tree, lambda t: t.detach().clone()), None, None)
    dev = cuda[0].device
    cur = torch.cuda.current_stream(dev)
    side = stream if stream is not None else torch.cuda.Stream(dev)
    side.wait_stream(cur)
    with torch.cuda.stream(side):
        def copy(t: torch.Tensor) -> torch.Tensor:
            h = torch.empty(t.shape, dtype=t.dtype, pin_memory=True)
            h.copy_(t, non_blocking=True)
            return h
        host = _map(tree, copy)
        ev = torch.cuda.Event()
        ev.record(side)
    return StagedTree(host, ev, tree)


def load_tree(spec: Any, read_blob: Callable[[str], bytes], device=None) -> Any:
    """Decodes a spec and, with a device, uploads it through pinned memory
    with asynchronous copies on the current stream (ordered before any kernel
    queued after this call)."""
    host = decode_tree(spec, read_blob)
    if device is None or torch.device(device).type != "cuda":
        return host
    return _map(host, lambda t: t.pin_memory().to(device, non_blocking=True))


class AsyncStateWriter:
    """Background writer of GDN state records (the SSM part of multiplex's
    ``AsyncPrefixDiskStore``, ``disk.py:305-573``).

    ``submit`` takes a :class:`StagedTree` (or a host tree) and the record's
    metadata; the writer thread waits for the staged copy, encodes it, writes
    the blobs and then the record.
    """

    def __init__(self, base_dir, *, block_size: int = DEFAULT_BLOCK_SIZE):
        self.base_dir = Path(base_dir).expanduser()
        self.blobs = BlobStore(self.base_dir)
        self.block_size = int(block_size)
        self._queue: "queue.Queue" = queue.Queue()
        self._errors = []
        self.written = 0
        self._thread = threading.Thread(target=self._loop, name="gdn-state-writer", daemon=True)
        self._thread.start()

    def record_path(self, key: str) -> Path:
        return self.base_dir / "records" / key[:2] / f"{key}.json"

    def submit(self, key: str, ssm, *, parent: Optional[str] = None, tokens=(), start: int = 0, pos: int = 0,
               pool: str = "default", source: Optional[str] = None, touch: int = 0, attn_spec: Any = None) -> None:
        meta = dict(key=str(key), parent=parent, tokens=[int(t) for t in tokens], start=int(start), pos=int(pos),
                    pool=str(pool), source=source, touch=int(touch), attn=attn_spec)
        self._queue.put((meta, ssm))

    def _loop(self) -> None:
        while True:
            item = self._queue.get()
            try:
                if item is None:
                    return
                meta, ssm = item
                tree = ssm.wait() if isinstance(ssm, StagedTree) else ssm
                spec, blobs = encode_tree(tree, block_size=self.block_size)
                self.blobs.write_blobs(blobs)
                record = {"version": RECORD_FORMAT_VERSION, "key": meta["key"], "parent": meta["parent"],
                          "tokens": meta["tokens"], "start": meta["start"], "pos": meta["pos"],
                          "pool": meta["pool"], "source": meta["source"], "touch": meta["touch"],
                          "attn": meta["attn"], "ssm": spec, "cached_h": None}
                write_json_atomic(self.record_path(meta["key"]), record)
                self.written += 1
            except Exception as e:  # noqa: BLE001 - reported by flush()
                self._errors.append(e)
            finally:
                self._queue.task_done()

    def flush(self) -> None:
        """Waits for every submitted record; raises the first write error."""
        self._queue.join()
        if self._errors:
            raise RuntimeError(f"{len(self._errors)} state record(s) failed") from self._errors[0]

    def read_record(self, key: str) -> Dict[str, Any]:
        data = json.loads(self.record_path(key).read_text(encoding="utf-8"))
        if int(data.get("version", 0)) != RECORD_FORMAT_VERSION:
            raise ValueError(f"bad prefix-cache record version: {data.get('version')!r}")
        return data

    def load_ssm(self, key: str, device=None) -> Any:
        return load_tree(self.read_record(key)["ssm"], self.blobs.read_blob, device)

    def close(self) -> None:
        self._queue.put(None)
        self._thread.join()
