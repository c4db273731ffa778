"""The prefix-cache state format on the host (no GPU): spec shapes, blob
bytes and digests computed independently with numpy/hashlib, the axis-2
block rule, dedup, atomic records, and bit-exact round trips."""

from __future__ import annotations

import hashlib
import json

import numpy as np
import pytest
import torch

from multiplex_amd import prefix_state as ps


def snapshot(seed=0, layers=3):
    g = torch.Generator().manual_seed(seed)
    out = []
    for i in range(layers):
        if i == 1:
            out.append(None)  # a non-GDN layer
            continue
        conv = torch.randn(1, 3, 8192, generator=g).to(torch.bfloat16)
        ssm = torch.randn(1, 32, 128, 128, generator=g) * 0.02
        out.append([conv, ssm])
    return out


def test_spec_bytes_match_tensor_bytes():
    spec, blobs = ps.encode_tree([[torch.ones(1024)]])
    assert ps.spec_nbytes(spec) == 4096 and len(blobs) == 1
    spec, _ = ps.encode_tree([[torch.zeros(1, 1, 2048, 4)]], block_size=256)
    assert spec["v"][0]["v"][0]["k"] == "blocks"
    assert ps.spec_nbytes(spec) == 1 * 1 * 2048 * 4 * 4


def test_blob_bytes_and_digests_are_little_endian_c_order():
    snap = snapshot()
    spec, blobs = ps.encode_tree(snap)
    ssm = snap[0][1]
    leaf = spec["v"][0]["v"][1]
    raw = np.ascontiguousarray(ssm.numpy()).astype("<f4").tobytes()
    assert leaf == {"k": "tensor", "sha": hashlib.sha256(raw).hexdigest(), "dtype": "float32",
                    "shape": [1, 32, 128, 128], "nbytes": len(raw)}
    assert blobs[leaf["sha"]] == raw
    # bf16 conv state: 8192 channels on axis 2 -> 32 blocks of 256, each the
    # bf16 bit patterns (upper half of the exact fp32 value) of a [1, 3, 256] slice
    conv = snap[0][0]
    blk = spec["v"][0]["v"][0]
    assert blk["k"] == "blocks" and blk["dtype"] == "bfloat16" and blk["axis"] == 2 and blk["block_size"] == 256
    assert blk["shape"] == [1, 3, 8192] and len(blk["blocks"]) == 32
    bits = (conv.float().numpy().view(np.uint32) >> 16).astype("<u2")
    for j, b in enumerate(blk["blocks"]):
        raw = np.ascontiguousarray(bits[:, :, 256 * j:256 * (j + 1)]).tobytes()
        assert (b["start"], b["end"], b["shape"], b["nbytes"]) == (256 * j, 256 * (j + 1), [1, 3, 256], len(raw))
        assert b["sha"] == hashlib.sha256(raw).hexdigest() and blobs[b["sha"]] == raw
    assert spec["v"][1] == {"k": "none"}


@pytest.mark.parametrize("n,blocked", [(511, False), (512, True), (700, True)])
def test_axis2_block_rule(n, blocked):
    t = torch.arange(2 * 3 * n, dtype=torch.float32).reshape(2, 3, n)
    spec, blobs = ps.encode_tree(t, block_size=256)
    assert (spec["k"] == "blocks") == blocked
    if blocked:
        ends = [b["end"] for b in spec["blocks"]]
        assert ends[-1] == n and all(e - s <= 256 for s, e in ((b["start"], b["end"]) for b in spec["blocks"]))
    back = ps.decode_tree(spec, blobs.__getitem__)
    assert torch.equal(back, t)


def test_round_trip_through_the_blob_store(tmp_path):
    snap = snapshot(1)
    tree = (7, snap, [None, True])
    spec, blobs = ps.encode_tree(tree)
    store = ps.ContentStore(tmp_path)
    wrote, present = store.put_many(blobs)
    assert wrote == len(blobs) and present == 0
    assert store.put_many(blobs) == (0, len(blobs))
    assert not [p for p in tmp_path.rglob("*") if p.name.startswith(".")]
    for d in blobs:
        assert store.blob_path(d) == tmp_path / "blobs" / d[:2] / f"{d}.bin"
        assert hashlib.sha256(store.blob_path(d).read_bytes()).hexdigest() == d
    back = ps.decode_tree(json.loads(json.dumps(spec)), store.get)
    assert back[0] == 7 and back[2] == [None, 1]
    for a, b in zip(back[1], snap):
        if b is None:
            assert a is None
        else:
            assert a[0].dtype == torch.bfloat16 and torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])


def test_identical_tensors_share_one_blob():
    t = torch.full((4, 4), 3.0)
    spec, blobs = ps.encode_tree([t, t.clone()])
    assert len(blobs) == 1 and spec["v"][0]["sha"] == spec["v"][1]["sha"]


def test_decode_rejects_a_short_blob():
    spec, blobs = ps.encode_tree(torch.ones(8))
    with pytest.raises(ValueError):
        ps.decode_tree(spec, lambda d: blobs[d][:-4])


def test_writer_records_host_snapshots(tmp_path):
    snap = snapshot(2)
    w = ps.AsyncStateWriter(tmp_path)
    try:
        w.submit("ab" * 32, snap, parent=None, tokens=[1, 2, 3], start=0, pos=3, touch=5).result()
        w.flush()
        path = w.record_path("ab" * 32)
        assert path == tmp_path / "records" / "ab" / f"{'ab' * 32}.json"
        rec = json.loads(path.read_text(encoding="utf-8"))
        assert list(rec) == ["version", "key", "parent", "tokens", "start", "pos", "pool", "source", "touch",
                             "attn", "ssm", "cached_h"]
        assert rec["version"] == ps.RECORD_FORMAT_VERSION == 1
        assert (rec["key"], rec["tokens"], rec["pos"], rec["touch"], rec["pool"]) == ("ab" * 32, [1, 2, 3], 3, 5,
                                                                                       "default")
        assert path.read_text(encoding="utf-8") == json.dumps(rec, ensure_ascii=False, separators=(",", ":"))
        # every blob the record names is in the store, under its own digest
        shas = []
        stack = [rec["ssm"]]
        while stack:
            x = stack.pop()
            if isinstance(x, dict):
                shas += [x["sha"]] if "sha" in x else []
                stack += list(x.values())
            elif isinstance(x, list):
                stack += x
        for d in shas:
            assert hashlib.sha256((tmp_path / "blobs" / d[:2] / f"{d}.bin").read_bytes()).hexdigest() == d
        back = w.load_ssm("ab" * 32)
        assert torch.equal(back[0][1], snap[0][1]) and back[1] is None
        assert back[0][0].dtype == torch.bfloat16 and torch.equal(back[0][0], snap[0][0])
        assert ps.spec_nbytes(rec["ssm"]) == 2 * (3 * 8192 * 2 + 32 * 128 * 128 * 4)
    finally:
        w.close()


@pytest.mark.parametrize("dtype", [torch.bool, torch.uint8, torch.int16, torch.int32, torch.int64, torch.float16,
                                   torch.float64, torch.bfloat16])
def test_every_dtype_round_trips_with_numpy_bytes(dtype):
    g = torch.Generator().manual_seed(5)
    t = (torch.randn(2, 3, 600, generator=g) * 100).to(dtype)
    spec, blobs = ps.encode_tree(t, block_size=256)
    assert spec["k"] == "blocks" and [(b["start"], b["end"]) for b in spec["blocks"]] == [(0, 256), (256, 512),
                                                                                           (512, 600)]
    for b in spec["blocks"]:
        part = t[:, :, b["start"]:b["end"]]
        ref = (part.view(torch.int16) if dtype == torch.bfloat16 else part).numpy()
        raw = np.ascontiguousarray(ref).tobytes()
        assert blobs[b["sha"]] == raw and b["sha"] == hashlib.sha256(raw).hexdigest()
    assert torch.equal(ps.decode_tree(spec, blobs.__getitem__), t)


def test_record_reader_checks_the_version(tmp_path):
    w = ps.AsyncStateWriter(tmp_path)
    try:
        w.submit("cd" * 32, [None]).result()
        p = w.record_path("cd" * 32)
        obj = json.loads(p.read_text())
        obj["version"] = 2
        p.write_text(json.dumps(obj))
        with pytest.raises(ValueError):
            w.read_record("cd" * 32)
    finally:
        w.close()


def test_writer_reports_failures_on_flush(tmp_path):
    w = ps.AsyncStateWriter(tmp_path)
    try:
        w.submit("ef" * 32, [object()])
        with pytest.raises(RuntimeError):
            w.flush()
        w.submit("ef" * 32, [None]).result()
        w.flush()
    finally:
        w.close()
