"""C-ABI checks that need no GPU: the library loads, exports every symbol
``include/gdn.h`` declares, and rejects bad arguments before any HIP call
(fake, never-dereferenced pointers are enough for that)."""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest
import torch

from multiplex_amd import _lib

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "gdn.h"

FAKE = 0x10000  # 64 KiB-aligned dummy address; only ever compared, never read


def header_functions():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b(gdn_[a-z0-9_]+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    return _lib.load()


def test_exports_match_header(lib):
    names = header_functions()
    assert names == sorted(_lib.EXPORTS)
    for n in names:
        assert hasattr(lib, n), n


def test_abi_version(lib):
    assert lib.gdn_abi_version() == _lib.GDN_ABI_VERSION == 4


def test_struct_layout_matches_header():
    # gdn_recurrent_args: 29 fields; pointers 8 B, int32 fields packed in pairs.
    assert ctypes.sizeof(_lib.RecurrentArgs) == 8 * 3 + 4 * 2 + 8 * 2 + 4 * 2 + 8 * 10 + 8 * 6 + 8 + 8 + 8 + 8
    assert _lib.RecurrentArgs.state_index.offset == _lib.RecurrentArgs.commit_len.offset + 8
    assert _lib.RecurrentArgs.n_slots.offset == _lib.RecurrentArgs.Dv.offset + 8
    assert _lib.RecurrentArgs.gate_stride.offset == _lib.RecurrentArgs.n_slots.offset + 8
    assert _lib.RecurrentArgs.y_from.offset == _lib.RecurrentArgs.stream.offset + 8


def _update(lib, **kw):
    args = dict(q=FAKE, k=FAKE, v=FAKE, qkv=_lib.DTYPE_BF16, a=FAKE, b=FAKE, ab=_lib.DTYPE_BF16,
                A_log=FAKE, dt_bias=FAKE, pdt=_lib.DTYPE_F32, state_in=FAKE, mask=None, y=FAKE,
                state_out=FAKE, B=2, T=1, Hk=16, Hv=32, Dk=128, Dv=128)
    args.update(kw)
    return lib.gdn_gated_delta_update(
        args["q"], args["k"], args["v"], args["qkv"], args["a"], args["b"], args["ab"], args["A_log"],
        args["dt_bias"], args["pdt"], args["state_in"], args["mask"], args["y"], args["state_out"],
        args["B"], args["T"], args["Hk"], args["Hv"], args["Dk"], args["Dv"], None)


@pytest.mark.parametrize(
    "kw,status",
    [
        (dict(y=None), _lib.ERR_INVALID),
        (dict(state_out=None), _lib.ERR_INVALID),
        (dict(Dk=100), _lib.ERR_UNSUPPORTED),
        (dict(Hv=30), _lib.ERR_INVALID),
        (dict(qkv=7), _lib.ERR_INVALID),
        (dict(A_log=None), _lib.ERR_INVALID),
        (dict(B=-1), _lib.ERR_INVALID),
        (dict(q=FAKE + 2), _lib.ERR_INVALID),
        (dict(state_out=FAKE + 4), _lib.ERR_INVALID),
    ],
)
def test_update_rejects_bad_arguments(lib, kw, status):
    assert _update(lib, **kw) == status
    assert _lib.last_error()


def test_empty_batch_is_a_no_op(lib):
    assert _update(lib, B=0) == _lib.OK


def test_recurrent_null_args(lib):
    assert lib.gdn_recurrent(None) == _lib.ERR_INVALID
    a = _lib.RecurrentArgs(k=FAKE, v=FAKE, gx=FAKE, gy=FAKE, gate_mode=5, B=1, T=1, Hk=1, Hv=1, Dk=128, Dv=128)
    assert lib.gdn_recurrent(ctypes.byref(a)) == _lib.ERR_INVALID
    a.gate_mode = _lib.GATES_PRE
    a.y = FAKE  # y without q
    assert lib.gdn_recurrent(ctypes.byref(a)) == _lib.ERR_INVALID


def test_prologue_rejects_bad_arguments(lib):
    def call(**kw):
        args = dict(qkv=FAKE, io=_lib.DTYPE_BF16, ld=0, cs=None, w=FAKE, wdt=_lib.DTYPE_BF16, mask=None,
                    cu=None, q=FAKE, k=FAKE, v=FAKE, cso=FAKE, B=1, S=4, Hk=16, Hv=32, Dk=128, Dv=128,
                    Kt=4, eps=1e-6)
        args.update(kw)
        return lib.gdn_conv_prologue(args["qkv"], args["io"], args["ld"], args["cs"], args["w"], args["wdt"], args["mask"],
                                     args["cu"], args["q"], args["k"], args["v"], args["cso"], args["B"],
                                     args["S"], args["Hk"], args["Hv"], args["Dk"], args["Dv"], args["Kt"],
                                     args["eps"], None)

    assert call(Dk=64) == _lib.ERR_UNSUPPORTED
    assert call(Kt=3) == _lib.ERR_UNSUPPORTED
    assert call(cs=FAKE, cso=FAKE) == _lib.ERR_INVALID           # in place over 4-token rows
    assert call(cs=FAKE, cso=FAKE, S=1, cu=FAKE) == _lib.ERR_INVALID  # in place over packed rows
    assert call(cs=FAKE, cso=FAKE, S=1, B=0) == _lib.OK          # in place over one-token rows
    assert call(q=None) == _lib.ERR_INVALID
    assert call(eps=-1.0) == _lib.ERR_INVALID
    assert call(B=0) == _lib.OK
    assert call(ld=100) == _lib.ERR_INVALID        # below C
    assert call(ld=8192 + 4) == _lib.ERR_INVALID   # rows not 16-byte aligned


def test_conv_commit_rejects_bad_arguments(lib):
    assert lib.gdn_conv_state_commit(FAKE, FAKE, _lib.DTYPE_BF16, 0, None, None, FAKE, 2, 4, 8192, 4, None) == _lib.ERR_INVALID
    assert lib.gdn_conv_state_commit(FAKE, FAKE, _lib.DTYPE_BF16, 0, None, FAKE, FAKE, 2, 4, 8192, 1, None) == _lib.ERR_INVALID
    assert lib.gdn_conv_state_commit(FAKE, FAKE, _lib.DTYPE_BF16, 0, None, FAKE, 2 * FAKE, 0, 4, 8192, 4, None) == _lib.OK
    assert lib.gdn_conv_state_commit(FAKE, FAKE, _lib.DTYPE_BF16, 0, None, FAKE, FAKE, 2, 4, 8192, 4, None) == _lib.ERR_INVALID
    assert lib.gdn_conv_state_commit(FAKE, FAKE, _lib.DTYPE_BF16, 100, None, FAKE, 2 * FAKE, 2, 4, 8192, 4, None) == _lib.ERR_INVALID


def test_chunk_rejects_bad_arguments(lib):
    def call(**kw):
        args = dict(q=FAKE, k=FAKE, v=FAKE, qkv=_lib.DTYPE_BF16, mode=_lib.GATES_RAW, gx=FAKE, gy=FAKE,
                    gdt=_lib.DTYPE_BF16, g_ld=0, A_log=FAKE, dt_bias=FAKE, pdt=_lib.DTYPE_F32, mask=None, s_in=None, y=FAKE,
                    s_out=FAKE, index=None, n_slots=0, cu=None, n_seqs=1, n_tok=4096, Hk=16, Hv=32, Dk=128, Dv=128, chunk=64,
                    ws=FAKE, ws_bytes=1 << 40)
        args.update(kw)
        return lib.gdn_chunk_fwd(*args.values(), None)

    assert call(chunk=32) == _lib.ERR_UNSUPPORTED
    assert call(qkv=_lib.DTYPE_F32) == _lib.ERR_UNSUPPORTED
    assert call(Dk=64) == _lib.ERR_UNSUPPORTED
    assert call(ws_bytes=0) == _lib.ERR_INVALID
    assert call(y=None) == _lib.ERR_INVALID
    assert call(n_seqs=2, n_tok=4095) == _lib.ERR_INVALID  # not n_seqs rows of equal length
    assert call(n_seqs=0, n_tok=0) == _lib.OK
    assert call(index=FAKE, n_slots=-1) == _lib.ERR_INVALID
    assert call(g_ld=16) == _lib.ERR_INVALID       # below Hv
    # packed sequences: the workspace must also hold their order after the records
    need = lib.gdn_chunk_workspace_bytes(3, 4096, 32, 128, 128, 64)
    assert call(cu=FAKE, n_seqs=3, ws_bytes=need - 256) == _lib.ERR_INVALID
    assert "workspace" in _lib.last_error()


def test_recurrent_rejects_bad_pool_size(lib):
    a = _lib.RecurrentArgs(q=FAKE, k=FAKE, v=FAKE, gx=FAKE, gy=FAKE, gate_mode=_lib.GATES_PRE, y=FAKE,
                           state_out=FAKE, state_index=FAKE, n_slots=-3, B=1, T=1, Hk=1, Hv=1, Dk=128, Dv=128)
    assert lib.gdn_recurrent(ctypes.byref(a)) == _lib.ERR_INVALID
    assert "n_slots" in _lib.last_error()


def test_recurrent_rejects_bad_y_from(lib):
    base = dict(q=FAKE, k=FAKE, v=FAKE, gx=FAKE, gy=FAKE, gate_mode=_lib.GATES_PRE, B=1, T=4, Hk=1, Hv=1, Dk=128,
                Dv=128)
    for bad in (dict(y=FAKE, y_from=5), dict(y=FAKE, y_from=-1), dict(y_from=2)):  # past T, negative, no y
        a = _lib.RecurrentArgs(**base, **bad)
        assert lib.gdn_recurrent(ctypes.byref(a)) == _lib.ERR_INVALID
        assert "y_from" in _lib.last_error()


def test_workspace_size_is_monotone(lib):
    small = lib.gdn_chunk_workspace_bytes(1, 64, 32, 128, 128, 64)
    big = lib.gdn_chunk_workspace_bytes(1, 4096, 32, 128, 128, 64)
    assert 0 < small < big
    assert lib.gdn_chunk_workspace_bytes(1, 64, 32, 128, 128, 32) == 0  # unsupported chunk


def test_workspace_holds_records_and_sequence_order(lib):
    """One record per (chunk slot, v-head): a packed call numbers sequence n's
    slots from cu[n] / 64 + n, so n_tok / 64 + n_seqs slots bound every
    packing.  2..1024 packed sequences add their longest-first order (int32,
    rounded up to 256 B) after the records."""
    rec = lib.gdn_chunk_workspace_bytes(1, 64, 4, 128, 128, 64) // (4 * 2)  # 1 + 1 slots
    assert rec % 256 == 0

    def slots(n_seqs, n_tok):
        return -(-n_tok // 64) + n_seqs

    assert lib.gdn_chunk_workspace_bytes(1, 4096, 4, 128, 128, 64) == slots(1, 4096) * 4 * rec
    assert lib.gdn_chunk_workspace_bytes(3, 300, 4, 128, 128, 64) == slots(3, 300) * 4 * rec + 256
    assert lib.gdn_chunk_workspace_bytes(100, 300, 4, 128, 128, 64) == slots(100, 300) * 4 * rec + 512
    assert lib.gdn_chunk_workspace_bytes(1024, 2048, 4, 128, 128, 64) == slots(1024, 2048) * 4 * rec + 4096
    assert lib.gdn_chunk_workspace_bytes(1025, 2048, 4, 128, 128, 64) == slots(1025, 2048) * 4 * rec


def test_python_rejects_host_tensors():
    import multiplex_amd as mx

    q = torch.zeros(1, 1, 16, 128, dtype=torch.bfloat16)
    v = torch.zeros(1, 1, 32, 128, dtype=torch.bfloat16)
    g = torch.zeros(1, 1, 32)
    p = torch.zeros(32)
    with pytest.raises(ValueError, match="ROCm device"):
        mx.gated_delta_update(q, q, v, g, g, p, p)
    with pytest.raises(ValueError, match="ROCm device"):
        mx.gated_delta_ops(q, q, v, g, g)
    with pytest.raises(ValueError, match="ROCm device"):
        mx.gdn_conv_prologue(torch.zeros(1, 1, 8192), torch.zeros(8192, 4), 16, 32, 128, 128)


def test_noalloc_chunk_rejects_calls_beyond_its_scratch(lib):
    """gdn_chunk_fwd_noalloc refuses, before any HIP call, a call whose chunk
    records exceed its 64 MiB static scratch (2048 tokens at Hv=32 need
    (32 + 1) * 32 records of 82,688 B), and takes no workspace argument."""
    P, I = FAKE, _lib.DTYPE_BF16
    st = lib.gdn_chunk_fwd_noalloc(P, P, P, I, _lib.GATES_RAW, P, P, I, 0, P, P, _lib.DTYPE_F32, None, P, P, P,
                                   None, 0, None, 1, 2048, 16, 32, 128, 128, 64, None)
    assert st == _lib.ERR_UNSUPPORTED
    msg = lib.gdn_last_error().decode()
    assert "static scratch" in msg and "67108864" in msg
    assert lib.gdn_chunk_workspace_bytes(1, 2048, 32, 128, 128, 64) > 64 << 20
    assert lib.gdn_chunk_workspace_bytes(1, 1536, 32, 128, 128, 64) <= 64 << 20


def test_attention_entry_points_reject_bad_arguments(lib):
    """gdn_attn_qk / gdn_attn_fwd / gdn_rms_norm / gdn_silu_mul validate
    before any HIP call."""
    def qk(**kw):
        a = dict(qg=FAKE, qg_ld=0, k=FAKE, v=FAKE, kv_ld=0, qw=FAKE, kw=FAKE, wdt=_lib.DTYPE_F32, eps=1e-6,
                 pos=FAKE, q=FAKE, kc=FAKE, vc=FAKE, B=2, T=3, Hq=16, Hkv=4, D=256, cap=64, rot=64, base=1e7)
        a.update(kw)
        return lib.gdn_attn_qk(*a.values(), None)

    assert qk(D=96) == _lib.ERR_UNSUPPORTED
    assert qk(rot=6) == _lib.ERR_UNSUPPORTED          # not whole lane groups
    assert qk(Hkv=3) == _lib.ERR_INVALID              # Hq not a multiple of Hkv
    assert qk(cap=2) == _lib.ERR_INVALID              # T new tokens cannot fit
    assert qk(qg_ld=100) == _lib.ERR_INVALID          # token stride below the row
    assert qk(pos=None) == _lib.ERR_INVALID
    assert qk(base=0.0) == _lib.ERR_INVALID
    assert qk(B=0) == _lib.OK                         # nothing to do

    def fwd(**kw):
        a = dict(q=FAKE, qg=FAKE, qg_ld=0, kc=FAKE, vc=FAKE, pos=FAKE, out=FAKE, scale=0.0625, B=2, T=1, Hq=16,
                 Hkv=4, D=256, cap=64, kvmax=64, n_split=1, ws=None, ws_bytes=0)
        a.update(kw)
        return lib.gdn_attn_fwd(*a.values(), None)

    assert fwd(D=64) == _lib.ERR_UNSUPPORTED
    assert fwd(kvmax=0) == _lib.ERR_INVALID           # below T
    assert fwd(kvmax=65) == _lib.ERR_INVALID          # beyond the cache
    assert fwd(scale=0.0) == _lib.ERR_INVALID
    assert fwd(n_split=4) == _lib.ERR_INVALID         # split partials need a workspace
    assert fwd(q=FAKE + 2) == _lib.ERR_INVALID        # misaligned
    assert fwd(qg_ld=6) == _lib.ERR_INVALID
    need = lib.gdn_attn_workspace_bytes(2, 1, 16, 4, 256, 4)
    assert need == 2 * 4 * 16 * 4 * (256 + 2) * 4     # rows padded to one 16-row tile
    assert lib.gdn_attn_workspace_bytes(2, 1, 16, 4, 256, 1) == 0

    assert lib.gdn_rms_norm(FAKE, None, None, FAKE, _lib.DTYPE_F32, FAKE, 0, 4, 100, 1e-6, None) == _lib.ERR_INVALID
    assert lib.gdn_rms_norm(FAKE, None, None, FAKE, _lib.DTYPE_F32, FAKE, 8, 4, 16, 1e-6, None) == _lib.ERR_INVALID
    assert lib.gdn_rms_norm(FAKE, None, None, None, _lib.DTYPE_F32, FAKE, 0, 4, 16, 1e-6, None) == _lib.ERR_INVALID
    assert lib.gdn_silu_mul(FAKE, FAKE, 4, 12, None) == _lib.ERR_INVALID
    assert lib.gdn_silu_mul(FAKE, FAKE, 0, 16, None) == _lib.OK
