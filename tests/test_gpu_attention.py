"""GPU parity of the full-attention path (trunk attention layers and the MTP
draft head) against the float64 oracle in ``oracle/attention.py``, which
``tests/test_oracle_attention.py`` pins to transformers' Qwen3.5 modules.

Tolerances (norm-wise relative, per output row unless stated).  With u =
2^-8 the unit roundoff of bf16 (round to nearest even):

* attention rows: ATT_TOL = 5e-3.  Two independent roundings separate the
  kernel from the float64 oracle: the output's own rounding to bf16, and the
  rounding of the softmax weights p_j to bf16 for the P.V product (the
  normaliser sums them in fp32).  Each relative element error lies in
  [-u, u] with an RMS of about u/sqrt(3) = 2.3e-3 (uniform over the half
  ulp and the mantissa), so norm-wise the output rounding contributes about
  u/sqrt(3) and the weights, for near-uniform attention over random values,
  at most about u/sqrt(3) as well (sum_j w_j delta_j v_j against
  sum_j w_j v_j; the largest weight, exactly 1, is not rounded at all).
  Their linear sum with a 10% allowance is 2 (u / sqrt 3) 1.1 = 5.0e-3.
  Measured (deterministic, seeded inputs): rounding the float64 reference
  itself to bf16 gives 1.5-2.5e-3 per row, the kernel 1.8-4.0e-3.
* whole layers and the MTP head: LAYER_TOL = 1e-2.  The oracle rounds at
  the same points (GEMM outputs, residual adds, norms) in its bf16 mode,
  so what remains is the attention error above carried through o_proj and
  the MLP, plus rounding-boundary flips where the library GEMMs accumulate
  in another order: twice the attention bound.  Measured: 2.4-4.3e-3.
* the cache append is exact for v and within one bf16 rounding for k.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import multiplex_amd as mx
from multiplex_amd import attention as att
from oracle import attention as oa
from oracle.gdn import bf16_round

pytestmark = pytest.mark.gpu
DEV = "cuda"
ATT_TOL = 5e-3
LAYER_TOL = 1e-2


def _bf16(gen, *shape, scale=1.0):
    return (torch.randn(*shape, generator=gen) * scale).to(torch.bfloat16)


def _np(t):
    return t.double().cpu().numpy()


def _row_errs(y, ref):
    """Norm-wise relative error of each last-axis row."""
    y, ref = np.asarray(y, np.float64), np.asarray(ref, np.float64)
    num = np.linalg.norm((y - ref).reshape(-1, y.shape[-1]), axis=-1)
    den = np.linalg.norm(ref.reshape(-1, y.shape[-1]), axis=-1)
    return num / np.maximum(den, 1e-30)


def test_qk_prep_matches_oracle():
    """Norms, rotary embedding and cache append at per-row offsets, reading
    q|gate and k|v as column slices of fused projection outputs."""
    gen = torch.Generator().manual_seed(71)
    B, T, Hq, Hkv, D, rot, base, cap = 3, 5, 16, 4, 256, 64, 1.0e7, 64
    pos0 = [0, 17, 40]
    qg_wide = _bf16(gen, B, T, Hq * 2 * D + 32)
    qg = qg_wide[..., :Hq * 2 * D]
    kv = _bf16(gen, B, T, 2 * Hkv * D)
    qw = torch.randn(D, generator=gen) * 0.2 + 1.0
    kw = torch.randn(D, generator=gen) * 0.2 + 1.0
    kc = torch.zeros(B, Hkv, cap, D, dtype=torch.bfloat16, device=DEV)
    vc = torch.zeros_like(kc)
    dqg, dkv = qg_wide.to(DEV)[..., :Hq * 2 * D], kv.to(DEV)
    q = att.attn_qk(dqg, dkv[..., :Hkv * D], dkv[..., Hkv * D:], qw.to(DEV), kw.to(DEV), 1e-6,
                    torch.tensor(pos0, dtype=torch.int32, device=DEV), kc, vc, rot, base)
    torch.cuda.synchronize()
    rq, _, rk, rv = oa.qk_prep(_np(qg), _np(kv[..., :Hkv * D]), _np(kv[..., Hkv * D:]), _np(qw), _np(kw), 1e-6,
                               pos0, rot, base, Hq, Hkv, D, round_fn=bf16_round)
    assert _row_errs(_np(q), rq).max() < 4e-3
    kc_n, vc_n = _np(kc), _np(vc)
    for b in range(B):
        sl = slice(pos0[b], pos0[b] + T)
        assert _row_errs(kc_n[b, :, sl], rk[b].transpose(1, 0, 2)).max() < 4e-3
        np.testing.assert_array_equal(vc_n[b, :, sl], rv[b].transpose(1, 0, 2))
        untouched = np.ones(cap, dtype=bool)
        untouched[sl] = False
        assert not kc_n[b, :, untouched].any() and not vc_n[b, :, untouched].any()


def test_rms_norm_residual_and_strided_output():
    """``gdn_rms_norm`` with a fused residual add (h = bf16(x + r), written
    out) and its output in one half of a concatenation buffer, against
    torch.nn.functional.rms_norm in float64."""
    gen = torch.Generator().manual_seed(77)
    rows, H = 37, 4096
    x, r = _bf16(gen, rows, H, scale=3.0), _bf16(gen, rows, H)
    w = torch.randn(H, generator=gen) * 0.2 + 1.0
    buf = torch.zeros(rows, 2 * H, dtype=torch.bfloat16, device=DEV)
    h, y = att.rms_norm(x.to(DEV), w.to(DEV), 1e-6, residual=r.to(DEV), out=buf[:, H:])
    torch.cuda.synchronize()
    h_ref = (x.float() + r.float()).to(torch.bfloat16)
    assert torch.equal(h.cpu(), h_ref)
    ref = torch.nn.functional.rms_norm(h_ref.double(), (H,), w.double(), 1e-6).numpy()
    assert _row_errs(_np(buf[:, H:]), ref).max() < 4e-3
    assert not buf[:, :H].any()


CASES = {
    # name: (B, T, pos0, n_split, gate[, (Hq, Hkv, D)]); heads default to 16, 4, 256
    "decode": (8, 1, [0, 1, 63, 64, 65, 300, 511, 700], 1, True),
    "decode_split": (8, 1, [0, 1, 63, 64, 65, 300, 511, 700], 4, True),
    "verify_t4": (4, 4, [3, 100, 257, 0], 1, True),
    "verify_t4_split": (4, 4, [3, 100, 257, 0], 3, False),
    "prefill": (2, 150, [0, 33], 1, True),
    "prefill_nogate": (1, 70, [5], 1, False),
    "prefill_long": (2, 611, [0, 77], 1, True),
    "prefill_d128": (2, 300, [20, 0], 1, True, (16, 4, 128)),
    "prefill_g8": (1, 97, [130], 1, False, (16, 2, 256)),
    "prefill_mha": (1, 520, [3], 1, True, (4, 4, 128)),
    "prefill_g2": (3, 300, [0, 260, 41], 1, True, (8, 4, 256)),
    "prefill_g3": (1, 200, [17], 1, True, (12, 4, 128)),
    "prefill_512_rows": (2, 128, [0, 5], 1, False),
    "prefill_508_rows": (1, 127, [9], 1, True),
    # 32-row tiles (4 per workgroup) with keys split over workgroups
    "rt4_split": (2, 8, [5, 300], 3, True),
    # head dim 128 on the decode / verify / short-prefill kernels and their combine
    "decode_d128": (8, 1, [0, 1, 63, 64, 65, 300, 511, 700], 1, True, (16, 4, 128)),
    "decode_split_d128": (8, 1, [0, 1, 63, 64, 65, 300, 511, 700], 4, False, (16, 4, 128)),
    "verify_t4_split_d128": (4, 4, [3, 100, 257, 0], 3, True, (16, 4, 128)),
    "rt4_split_d128": (2, 8, [5, 300], 3, False, (16, 4, 128)),
    "prefill_short_d128": (2, 40, [0, 17], 1, True, (16, 4, 128)),
}


@pytest.mark.parametrize("name", list(CASES))
def test_attention_matches_oracle(name):
    """Causal GQA attention over per-row cache lengths: decode and 4-token
    verify (one 16-row tile, keys split over the waves and optionally over
    workgroups), short prefills (64-row tiles, below 512 rows per kv-head)
    and long ones (128-row workgroups with double-buffered K/V blocks, from
    512 rows: T=150 and up at 4 heads per group), at head dims 256 and 128.
    Cache positions past each row's keys hold NaN, which must not leak."""
    B, T, pos0, n_split, use_gate = CASES[name][:5]
    Hq, Hkv, D = CASES[name][5] if len(CASES[name]) > 5 else (16, 4, 256)
    gen = torch.Generator().manual_seed(72)
    L = max(pos0) + T
    cap = L + 40
    kc = _bf16(gen, B, Hkv, cap, D)
    vc = _bf16(gen, B, Hkv, cap, D)
    for b in range(B):
        kc[b, :, pos0[b] + T:] = float("nan")
        vc[b, :, pos0[b] + T:] = float("nan")
    q = _bf16(gen, B, T, Hq, D)
    gate = _bf16(gen, B, T, Hq * 2 * D, scale=2.0) if use_gate else None
    out = att.attn_fwd(q.to(DEV), kc.to(DEV), vc.to(DEV), torch.tensor(pos0, dtype=torch.int32, device=DEV), L,
                       gate=None if gate is None else gate.to(DEV), n_split=n_split)
    torch.cuda.synchronize()
    ref = oa.attention(_np(q), np.nan_to_num(_np(kc)), np.nan_to_num(_np(vc)), pos0, D ** -0.5)
    if gate is not None:
        g = _np(gate).reshape(B, T, Hq, 2 * D)[..., D:]
        ref = ref * (1.0 / (1.0 + np.exp(-g)))
    got = _np(out)
    assert np.isfinite(got).all()
    assert _row_errs(got, ref).max() < ATT_TOL


def test_split_keys_agree_with_one_range():
    """A 2000-key decode split over 1 and 5 workgroups per row."""
    gen = torch.Generator().manual_seed(73)
    B, Hq, Hkv, D, L = 4, 16, 4, 256, 2000
    kc = _bf16(gen, B, Hkv, L, D).to(DEV)
    vc = _bf16(gen, B, Hkv, L, D).to(DEV)
    q = _bf16(gen, B, 1, Hq, D).to(DEV)
    pos0 = torch.full((B,), L - 1, dtype=torch.int32, device=DEV)
    a = att.attn_fwd(q, kc, vc, pos0, L, n_split=1)
    b = att.attn_fwd(q, kc, vc, pos0, L, n_split=5)
    torch.cuda.synchronize()
    assert _row_errs(_np(b), _np(a)).max() < 4e-3


ARGS = mx.AttentionArgs(hidden_size=512, num_attention_heads=8, num_key_value_heads=2, head_dim=256,
                        intermediate_size=768, rms_norm_eps=1e-6, partial_rotary_factor=0.25, rope_theta=1.0e7)


def _oracle_layer_params(layer: mx.DecoderLayer):
    a = layer.self_attn
    Hq, Hkv, D = a.Hq, a.Hkv, a.D
    w = _np(a.qkv_proj)
    I = layer.mlp.down_proj.shape[1]
    gu = _np(layer.mlp.gate_up_proj)
    return dict(
        self_attn=dict(q_proj=w[:2 * Hq * D], k_proj=w[2 * Hq * D:(2 * Hq + Hkv) * D], v_proj=w[(2 * Hq + Hkv) * D:],
                       o_proj=_np(a.o_proj), q_norm=_np(a.q_norm.weight), k_norm=_np(a.k_norm.weight)),
        mlp=dict(gate_proj=gu[:I], up_proj=gu[I:], down_proj=_np(layer.mlp.down_proj)),
        input_layernorm=_np(layer.input_layernorm.weight),
        post_attention_layernorm=_np(layer.post_attention_layernorm.weight))


def _oracle_args(a: mx.AttentionArgs):
    return dict(Hq=a.num_attention_heads, Hkv=a.num_key_value_heads, D=a.head_dim, eps=a.rms_norm_eps, rot=a.rot,
                base=a.rope_theta)


def _randomise_norms(module, gen):
    with torch.no_grad():
        for n, p in module.named_parameters():
            if n.endswith("weight") and p.dim() == 1:
                p.copy_(torch.randn(p.shape, generator=gen) * 0.2 + 1.0)


def test_decoder_layer_matches_oracle():
    """A trunk full-attention DecoderLayer: a 37-token prefill of two rows,
    then two decode steps over the cache."""
    torch.manual_seed(74)
    gen = torch.Generator().manual_seed(74)
    layer = mx.DecoderLayer(ARGS, device=DEV)
    _randomise_norms(layer, gen)
    lp = _oracle_layer_params(layer)
    B = 2
    cache = mx.KVCache(B, ARGS.num_key_value_heads, ARGS.head_dim, 64, DEV)
    oc = oa.empty_cache(B, ARGS.num_key_value_heads, 64, ARGS.head_dim)
    for T in (37, 1, 1):
        x = _bf16(gen, B, T, ARGS.hidden_size)
        y = layer(x.to(DEV), cache)
        torch.cuda.synchronize()
        ref = oa.decoder_layer(lp, _np(x), oc, _oracle_args(ARGS), round_fn=bf16_round)
        assert _row_errs(_np(y), ref).max() < LAYER_TOL
    assert cache.size() == 39 and cache.pos0.tolist() == [39, 39]


def test_mtp_head_matches_oracle_and_rolls_back():
    """MTPHead (mtp.py:181-194): a 4-position call from an empty draft cache,
    two draft steps, then a trim back to the committed length and the same
    draft step again, which reproduces the first one bit for bit."""
    gen = torch.Generator().manual_seed(75)
    torch.manual_seed(75)
    head = mx.MTPHead(ARGS, n_layers=1, device=DEV)
    _randomise_norms(head, gen)
    hp = dict(pre_fc_norm_embedding=_np(head.pre_fc_norm_embedding.weight),
              pre_fc_norm_hidden=_np(head.pre_fc_norm_hidden.weight), fc=_np(head.fc), norm=_np(head.norm.weight),
              layers=[_oracle_layer_params(head.layers[0])])
    B, H = 3, ARGS.hidden_size
    cache = head.make_cache(B, 16)
    oc = [oa.empty_cache(B, ARGS.num_key_value_heads, 16, ARGS.head_dim)]
    steps = [(_bf16(gen, B, L, H), _bf16(gen, B, L, H)) for L in (4, 1, 1)]
    outs = []
    for e, h in steps:
        y = head(e.to(DEV), h.to(DEV), cache)
        torch.cuda.synchronize()
        outs.append(y.clone())
        ref = oa.mtp_head(hp, _np(e), _np(h), oc, _oracle_args(ARGS), round_fn=bf16_round)
        assert _row_errs(_np(y), ref).max() < LAYER_TOL
    head.trim_cache_to(cache, 5)
    assert cache[0].size() == 5
    y = head(steps[2][0].to(DEV), steps[2][1].to(DEV), cache)
    torch.cuda.synchronize()
    assert torch.equal(y, outs[2])


def test_kv_cache_rows_extract_filter_merge():
    """Row bookkeeping: a row extracted (or kept by filter, or merged back)
    decodes as it does inside the full batch; a cache grows past its
    capacity without losing rows."""
    gen = torch.Generator().manual_seed(76)
    torch.manual_seed(76)
    attn = mx.Attention(ARGS, device=DEV, n_split=1)
    B, H = 3, ARGS.hidden_size
    cache = mx.KVCache(B, ARGS.num_key_value_heads, ARGS.head_dim, 32, DEV)
    attn(_bf16(gen, B, 9, H).to(DEV), cache)
    x = _bf16(gen, B, 1, H).to(DEV)
    one = cache.extract(1)
    kept = mx.KVCache.merge([cache.extract(0), cache.extract(2)])
    full = attn(x, cache)
    # the projections of 1, 2 and 3 rows may take different GEMM kernels, so
    # rows are compared to the layer's tolerance (a mixed-up row is off by ~1)
    assert _row_errs(_np(attn(x[1:2], one)), _np(full[1:2])).max() < 1e-2
    assert _row_errs(_np(attn(x[0::2].contiguous(), kept)), _np(full[0::2])).max() < 1e-2
    cache.trim(1)
    cache.filter([2, 0])
    assert _row_errs(_np(attn(x[[2, 0]].contiguous(), cache)), _np(full[[2, 0]])).max() < 1e-2
    # growth past the capacity keeps the cached rows
    big = mx.KVCache(1, ARGS.num_key_value_heads, ARGS.head_dim, 1, DEV)
    xs = _bf16(gen, 1, 300, H).to(DEV)
    y_grow = torch.cat([attn(xs[:, :200], big), attn(xs[:, 200:], big)], dim=1)
    assert big.capacity == 512
    ref = attn(xs, mx.KVCache(1, ARGS.num_key_value_heads, ARGS.head_dim, 300, DEV))
    assert _row_errs(_np(y_grow), _np(ref)).max() < 1e-2


def test_kv_cache_merge_of_different_lengths_and_state_restore():
    """A batch join of rows of different lengths (9 and 20 positions, as
    ``BatchKVCache.merge`` allows at ``mtp.py:505-511``): each row keeps its
    own length in ``pos0``, appends at its own end and attends to its own
    keys only, so a decode step of the merged batch matches each cache
    alone.  Then ``state`` assignment (``mtp.py:608``) restores one row's
    keys into a fresh cache, which decodes bit for bit like the source."""
    gen = torch.Generator().manual_seed(77)
    torch.manual_seed(77)
    attn = mx.Attention(ARGS, device=DEV, n_split=1)
    Hkv, D, H = ARGS.num_key_value_heads, ARGS.head_dim, ARGS.hidden_size
    a = mx.KVCache(1, Hkv, D, 32, DEV)
    b = mx.KVCache(2, Hkv, D, 300, DEV)
    attn(_bf16(gen, 1, 9, H).to(DEV), a)
    attn(_bf16(gen, 2, 20, H).to(DEV), b)
    m = mx.KVCache.merge([a, b])
    assert m.lengths == [9, 20, 20] and m.pos0.tolist() == [9, 20, 20] and m.size() == 20
    x = _bf16(gen, 3, 1, H).to(DEV)
    y = attn(x, m)
    assert m.pos0.tolist() == [10, 21, 21]
    ya, yb = attn(x[0:1], a), attn(x[1:].contiguous(), b)
    # 1-, 2- and 3-row projections may take different GEMM kernels: rows are
    # compared to the layer's tolerance (a row attending to another row's
    # keys, or to unset positions, is off by order 1)
    assert _row_errs(_np(y[0:1]), _np(ya)).max() < 1e-2
    assert _row_errs(_np(y[1:]), _np(yb)).max() < 1e-2
    # the merged row 0 appended at position 9, not at the batch's longest length
    assert _row_errs(_np(m.keys[0, :, 9]), _np(a.keys[0, :, 9])).max() < 1e-2
    # state restore of row 1 into a fresh one-row cache
    r = mx.KVCache(1, Hkv, D, 16, DEV)
    keys, values = m.state
    r.state = [keys[1:2, :, :21].clone(), values[1:2, :, :21].clone()]
    assert r.size() == 21 and r.pos0.tolist() == [21] and r.capacity >= 21
    src = m.extract(1)
    x1 = _bf16(gen, 1, 1, H).to(DEV)
    assert torch.equal(attn(x1, r), attn(x1, src))
