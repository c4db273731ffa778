"""Host-side logic of the attention module on CPU tensors: KV-cache row
bookkeeping (ragged batch joins, trims, state restore) and the argument
checks that ``attn_fwd`` and ``rms_norm`` run before any launch."""

from __future__ import annotations

import pytest
import torch

from multiplex_amd import attention as att
from multiplex_amd.attention import KVCache


def _filled(batch, length, cap, seed):
    g = torch.Generator().manual_seed(seed)
    c = KVCache(batch, 2, 8, cap, "cpu")
    c.keys.copy_(torch.randn(c.keys.shape, generator=g).to(torch.bfloat16))
    c.values.copy_(torch.randn(c.values.shape, generator=g).to(torch.bfloat16))
    c.advance(length)
    return c


def test_merge_keeps_each_rows_length():
    a, b = _filled(2, 5, 16, 1), _filled(1, 9, 300, 2)
    m = KVCache.merge([a, b])
    assert m.lengths == [5, 5, 9] and m.pos0.tolist() == [5, 5, 9]
    assert m.size() == 9 and m.capacity >= 300
    assert torch.equal(m.keys[:2, :, :5], a.keys[:, :, :5])
    assert torch.equal(m.values[2, :, :9], b.values[0, :, :9])


def test_trim_extract_filter_on_ragged_rows():
    m = KVCache.merge([_filled(2, 5, 16, 3), _filled(1, 9, 16, 4)])
    assert m.trim(6) == 6
    assert m.lengths == [0, 0, 3] and m.pos0.tolist() == [0, 0, 3]
    e = m.extract(2)
    assert e.lengths == [3] and torch.equal(e.keys[0, :, :3], m.keys[2, :, :3])
    m.filter([2, 0])
    assert m.lengths == [3, 0] and m.pos0.tolist() == [3, 0]
    m.advance(2)
    assert m.lengths == [5, 2] and m.pos0.tolist() == [5, 2]


def test_state_setter_resizes_and_sets_lengths():
    c = KVCache(1, 2, 8, 16, "cpu")
    k = torch.randn(2, 2, 300, 8).to(torch.bfloat16)
    v = torch.randn(2, 2, 300, 8).to(torch.bfloat16)
    c.state = [k, v]
    assert c.batch == 2 and c.capacity >= 300 and c.lengths == [300, 300] and c.pos0.tolist() == [300, 300]
    keys, values = c.state
    assert torch.equal(keys, k) and torch.equal(values, v)
    with pytest.raises(ValueError):
        c.state = [k, v[:, :, :10]]


def _attn_args(B=2, T=1, Hq=4, Hkv=2, D=16, cap=32):
    bf = torch.bfloat16
    return dict(q=torch.zeros(B, T, Hq, D, dtype=bf), k_cache=torch.zeros(B, Hkv, cap, D, dtype=bf),
                v_cache=torch.zeros(B, Hkv, cap, D, dtype=bf), pos0=torch.zeros(B, dtype=torch.int32),
                kv_len_max=T)


@pytest.mark.parametrize("change,match", [
    (lambda a: a.update(k_cache=a["k_cache"].float()), "k_cache must be bfloat16"),
    (lambda a: a.update(v_cache=a["v_cache"][:, :, :16].contiguous()), "differ"),
    (lambda a: a.update(k_cache=a["k_cache"][:1], v_cache=a["v_cache"][:1]), "do not match"),
    (lambda a: a.update(k_cache=a["k_cache"].transpose(2, 3).contiguous().transpose(2, 3)), "contiguous"),
    (lambda a: a.update(pos0=a["pos0"].long()), "pos0"),
    (lambda a: a.update(pos0=a["pos0"][:1]), "pos0"),
    (lambda a: a.update(kv_len_max=33), "kv_len_max"),
    (lambda a: a.update(gate=torch.zeros(1, 1, 4 * 2 * 16, dtype=torch.bfloat16)), "gate"),
    (lambda a: a.update(gate=torch.zeros(2, 1, 8, dtype=torch.bfloat16)), "gate"),
    (lambda a: a.update(out=torch.zeros(2, 1, 4, 8, dtype=torch.bfloat16)), "out"),
    (lambda a: a.update(q=a["q"][:, :, :3]), "multiple"),
])
def test_attn_fwd_rejects_mismatched_arguments(change, match):
    a = _attn_args()
    change(a)
    kv_len_max = a.pop("kv_len_max")
    q, kc, vc, pos0 = a.pop("q"), a.pop("k_cache"), a.pop("v_cache"), a.pop("pos0")
    with pytest.raises(ValueError, match=match):
        att.attn_fwd(q, kc, vc, pos0, kv_len_max, **a)


def test_rms_norm_rejects_residual_of_another_shape():
    x = torch.zeros(3, 8, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="residual"):
        att.rms_norm(x, torch.ones(8), 1e-6, residual=torch.zeros(2, 8, dtype=torch.bfloat16))
