"""Pins the float64 restatement of the full-attention layer and the MTP head
(``oracle/attention.py``), CPU only.

The expected values come from transformers' Qwen3.5 modules
(``tests/golden/make_golden.py``: ``Qwen3_5Attention`` and
``Qwen3_5DecoderLayer`` in float32, a prefill and then more tokens over the
KV cache; the MTP head composed from them as ``mtp.py:181-194`` composes
it), from torch's ``rms_norm`` and ``apply_rotary_pos_emb``, and from closed
forms.  Planted wiring mistakes fail those pins.
"""

from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from gdn_cases import rel_err
from oracle import attention as oa

GOLD = Path(__file__).resolve().parent / "golden"


def load(name):
    with np.load(GOLD / f"{name}.npz") as z:
        return {k: z[k].astype(np.float64) for k in z.files}


def _layer_params(d):
    P = lambda n: d["p_" + n.replace(".", "__")]
    attn = {k: P(f"self_attn.{k}.weight") for k in ("q_proj", "k_proj", "v_proj", "o_proj", "q_norm", "k_norm")}
    return dict(self_attn=attn, mlp={k: P(f"mlp.{k}.weight") for k in ("gate_proj", "up_proj", "down_proj")},
                input_layernorm=P("input_layernorm.weight"),
                post_attention_layernorm=P("post_attention_layernorm.weight"))


def _layer_fixture():
    d = load("attention_layer_f32")
    B, T0, T1, H, Hq, Hkv, D, I = (int(x) for x in d["dims"])
    args = dict(Hq=Hq, Hkv=Hkv, D=D, eps=float(d["eps"]), rot=int(d["rot"]), base=float(d["base"]))
    return d, _layer_params(d), args, (B, T0, T1, Hkv, D)


def _run_layer(d, lp, args, dims, tag):
    B, T0, T1, Hkv, D = dims
    c = oa.empty_cache(B, Hkv, T0 + T1, D)
    outs = []
    for x in (d["x0"], d["x1"]):
        outs.append(oa.attention_layer(lp["self_attn"], x, c, args) if tag == "attn"
                    else oa.decoder_layer(lp, x, c, args))
    return outs


@pytest.mark.parametrize("tag", ["attn", "layer"])
def test_attention_matches_library_module(tag):
    """Qwen3_5Attention alone and the whole Qwen3_5DecoderLayer (float32):
    5 prompt tokens from an empty cache, then 2 more over it."""
    d, lp, args, dims = _layer_fixture()
    for i, y in enumerate(_run_layer(d, lp, args, dims, tag)):
        assert rel_err(y, d[f"{tag}_out{i}"]) < 2e-6


def _mtp_fixture():
    m = load("mtp_head_f32")
    B, L0, H, Hq, Hkv, D, I = (int(x) for x in m["dims"])
    args = dict(Hq=Hq, Hkv=Hkv, D=D, eps=float(m["eps"]), rot=int(m["rot"]), base=float(m["base"]))
    hp = dict(pre_fc_norm_embedding=m["h_pre_fc_norm_embedding"], pre_fc_norm_hidden=m["h_pre_fc_norm_hidden"],
              fc=m["h_fc"], norm=m["h_norm"], layers=[_layer_params(m)])
    return m, hp, args, (B, L0, Hkv, D)


def test_mtp_head_matches_composed_modules():
    """MTPHead: a 3-position call from an empty draft cache, then one draft step."""
    m, hp, args, (B, L0, Hkv, D) = _mtp_fixture()
    c = [oa.empty_cache(B, Hkv, L0 + 1, D)]
    for i in range(2):
        y = oa.mtp_head(hp, m[f"embed{i}"], m[f"hidden{i}"], c, args)
        assert rel_err(y, m[f"out{i}"]) < 2e-6
    assert list(c[0]["offset"]) == [L0 + 1] * B


def test_rms_norm_matches_torch():
    x = np.random.default_rng(0).standard_normal((5, 64)) * 3
    w = np.random.default_rng(1).normal(1.0, 0.3, 64)
    ref = F.rms_norm(torch.tensor(x), (64,), torch.tensor(w), 1e-6).numpy()
    assert rel_err(oa.rms_norm(x, w, 1e-6), ref) < 1e-12


def test_rope_matches_library():
    """transformers' rotary embedding (default rope, partial factor) and
    apply_rotary_pos_emb, in float64, at positions up to 40000."""
    from transformers.models.qwen3_5.configuration_qwen3_5 import Qwen3_5TextConfig
    from transformers.models.qwen3_5.modeling_qwen3_5 import Qwen3_5TextRotaryEmbedding, apply_rotary_pos_emb

    D, rot, base = 32, 16, 1.0e7
    cfg = Qwen3_5TextConfig(hidden_size=64, num_attention_heads=2, num_key_value_heads=1, head_dim=D,
                            rope_parameters={"rope_type": "default", "rope_theta": base,
                                             "partial_rotary_factor": rot / D})
    rng = np.random.default_rng(2)
    x = rng.standard_normal((1, 4, 2, D))
    pos = np.array([[0, 7, 513, 40000]])
    emb = Qwen3_5TextRotaryEmbedding(cfg)
    emb.inv_freq = emb.inv_freq.double()
    xt = torch.tensor(x)
    cos, sin = emb(xt, torch.tensor(pos))
    ref, _ = apply_rotary_pos_emb(xt.transpose(1, 2), xt.transpose(1, 2), cos.double(), sin.double())
    got = oa.rope(x, pos, rot, base)
    ref = ref.transpose(1, 2).numpy()
    # transformers forms the angles pos * inv_freq in float32: ~1e-7 relative
    # up to position 513, 2e-5 at 40000
    assert rel_err(got[:, :3], ref[:, :3]) < 1e-6
    assert rel_err(got, ref) < 5e-5
    np.testing.assert_array_equal(got[..., rot:], x[..., rot:])


def test_attention_closed_forms():
    """One visible key returns its value (token 0 of an empty cache); keys
    equal to each other average the values; GQA heads of one kv-head see the
    same keys."""
    rng = np.random.default_rng(3)
    B, Hq, Hkv, D, L = 2, 4, 2, 8, 6
    kc = rng.standard_normal((B, Hkv, L, D))
    vc = rng.standard_normal((B, Hkv, L, D))
    q = rng.standard_normal((B, 1, Hq, D))
    out = oa.attention(q, kc, vc, [0, 0], 0.5)
    for h in range(Hq):
        np.testing.assert_allclose(out[:, 0, h], vc[:, h // 2, 0], rtol=1e-12)
    kc[:] = kc[:, :, :1]
    out = oa.attention(q, kc, vc, [L - 1, 3], 0.5)
    np.testing.assert_allclose(out[0, 0, 1], vc[0, 0].mean(0), rtol=1e-12)
    np.testing.assert_allclose(out[1, 0, 3], vc[1, 1, :4].mean(0), rtol=1e-12)


def _mutant(kind, monkeypatch):
    if kind == "norm_one_plus_w":
        real = oa.rms_norm
        monkeypatch.setattr(oa, "rms_norm", lambda x, w, eps: real(x, 1.0 + np.asarray(w), eps))
    elif kind == "rope_on_last_dims":
        real = oa.rope

        def last(x, pos, rot, base):
            return real(np.asarray(x)[..., ::-1], pos, rot, base)[..., ::-1]
        monkeypatch.setattr(oa, "rope", last)
    elif kind == "no_causal_mask":
        real = oa.attention
        monkeypatch.setattr(oa, "attention", lambda q, kc, vc, pos0, s: real(
            q, kc, vc, np.asarray(pos0) + np.asarray(q).shape[1] - 1, s))
    elif kind == "gate_not_applied":
        monkeypatch.setattr(oa, "sigmoid", lambda g: np.ones_like(g))
    elif kind == "gqa_heads_interleaved":
        real = oa.attention

        def inter(q, kc, vc, pos0, s):
            q = np.asarray(q)
            Hq, Hkv = q.shape[2], np.asarray(kc).shape[1]
            perm = np.arange(Hq).reshape(Hq // Hkv, Hkv).T.reshape(-1)  # head h -> kv-head h % Hkv
            return real(q[:, :, perm], kc, vc, pos0, s)[:, :, np.argsort(perm)]
        monkeypatch.setattr(oa, "attention", inter)


@pytest.mark.parametrize("kind", ["norm_one_plus_w", "rope_on_last_dims", "no_causal_mask", "gate_not_applied",
                                  "gqa_heads_interleaved"])
def test_planted_mistakes(kind, monkeypatch):
    """Plausible mistakes planted in the oracle fail the module pin."""
    d, lp, args, dims = _layer_fixture()
    _mutant(kind, monkeypatch)
    outs = _run_layer(d, lp, args, dims, "attn")
    assert max(rel_err(y, d[f"attn_out{i}"]) for i, y in enumerate(outs)) > 1e-2
