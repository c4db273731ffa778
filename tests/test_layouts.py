"""Host-side layout checks: which column slices the kernels read in place
(row strides passed to the C ABI) and which are copied first."""

from __future__ import annotations

import torch

from multiplex_amd.conv import _qkv_rows
from multiplex_amd.epilogue import _gate_lines
from multiplex_amd.gated_delta import _gate_pair, _token_rows


def test_token_rows():
    buf = torch.zeros(3, 5, 40)
    assert _token_rows(buf[..., 8:16], 8) == 40                 # column slice: token stride 40
    assert _token_rows(buf[..., :8].contiguous(), 8) == 8      # contiguous
    assert _token_rows(buf[:, :1, 8:16], 8) == 200             # T = 1: row stride = batch stride
    assert _token_rows(buf.transpose(0, 1)[..., :8], 8) is None  # batch stride != T * token stride
    assert _token_rows(buf[..., ::2][..., :8], 8) is None       # channels not contiguous
    _token_rows(torch.zeros(2, 0, 8), 8)                        # no tokens: any answer is safe


def test_gate_pair_needs_one_stride():
    buf = torch.zeros(2, 4, 16)
    a, b = buf[..., :4], buf[..., 4:8]
    ga, gb, ld = _gate_pair(a, b, 4)
    assert ga is a and gb is b and ld == 16
    ga, gb, ld = _gate_pair(a, torch.zeros(2, 4, 4), 4)
    assert ga.is_contiguous() and gb.is_contiguous() and ld == 0
    c = torch.zeros(2, 4, 4)
    ga, gb, ld = _gate_pair(c, c.clone(), 4)
    assert ga is c and ld == 0


def test_qkv_rows_keep_16_byte_rows():
    buf = torch.zeros(2, 3, 1024 + 64, dtype=torch.bfloat16)
    q, ld = _qkv_rows(buf[..., :1024], 1024)
    assert ld == 1088 and q.data_ptr() == buf.data_ptr()
    buf = torch.zeros(2, 3, 1024 + 4, dtype=torch.bfloat16)   # 2056-byte rows: copied
    q, ld = _qkv_rows(buf[..., :1024], 1024)
    assert ld == 0 and q.is_contiguous()


def test_gate_lines():
    buf = torch.zeros(3, 5, 4 * 128 + 64, dtype=torch.bfloat16)
    z = buf[..., :512].unflatten(-1, (4, 128))
    g, group, ld = _gate_lines(z, 128)
    assert g is z and (group, ld) == (4, 576)
    g, group, ld = _gate_lines(z.contiguous(), 128)
    assert (group, ld) == (0, 0)
    zt = z.transpose(0, 1)                                     # lines not in row-major order
    g, group, ld = _gate_lines(zt, 128)
    assert (group, ld) == (0, 0) and g.is_contiguous()
    one = buf[:1, :1, :512].unflatten(-1, (4, 128))            # a single line
    g, group, ld = _gate_lines(one, 128)
    assert g.is_contiguous()
