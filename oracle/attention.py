"""Float64 CPU restatement of the full-attention layers multiplex runs beside
the GDN mixers: the hybrid trunk's attention DecoderLayers and the MTP draft
head.

TEST INFRASTRUCTURE ONLY.  Only ``tests/``, ``__graft_entry__.smoke()`` and
``bench.py``'s ``cpu_baseline`` leg may import this module, and only as the
checker.  The product package ``multiplex_amd`` never imports it.

What it restates (the arithmetic lives in mlx-lm's ``qwen3_5`` model, absent
here; multiplex reaches it through these call sites):

* ``MTPHead.__call__`` -- ``multiplex/kernel/mtp.py:181-194``: RMSNorm of the
  token embedding and of the trunk hidden, ``fc`` over their concatenation,
  the stacked full-attention DecoderLayers with a causal mask from the first
  draft cache's offset, and a final RMSNorm.  The head's norms are mlx
  ``nn.RMSNorm`` (``mtp.py:173-179``): ``x / sqrt(mean(x^2) + eps) * w``.
* ``q5.DecoderLayer(targs, fa_idx)`` (``mtp.py:178``) -- mlx-lm's Qwen3.5
  layer at a full-attention index: pre-norm residual blocks around the gated
  attention and the SwiGLU MLP.
* the gated attention: ``q_proj`` emits, per head, q then an output gate;
  q_norm / k_norm are RMSNorms over the head dim; the rotary embedding covers
  the first ``partial_rotary_factor * head_dim`` dims in rotate-half form
  with angle ``pos * base^(-2i/rot)``; scaled dot-product attention over the
  KV cache (causal from the cache offset, ``mtp.py:190``); the output is
  multiplied by ``sigmoid(gate)`` before ``o_proj``.
* the draft cache's bookkeeping (``mtp.py:479-503``): one KV cache per draft
  layer, advanced by each call, trimmed back to the committed length.

Weights use mlx's convention (norms multiply by ``w``).  transformers'
Qwen3.5 modules keep ``w - 1`` and multiply by ``1 + w``; the fixtures in
``tests/golden/make_golden.py`` convert.

Pinning (``tests/test_oracle.py``): ``rms_norm`` against
``torch.nn.functional.rms_norm``; ``rope`` against transformers'
``apply_rotary_pos_emb`` with the model's rotary embedding; ``attention``,
``attention_layer`` and ``decoder_layer`` against transformers'
``Qwen3_5Attention`` / ``Qwen3_5DecoderLayer`` (float32 fixtures: a prefill
from an empty cache, then decode steps over the cache); ``mtp_head`` against
the same modules composed as ``mtp.py:181-194`` composes them; closed forms
(one visible key returns its value; equal keys average the values) and
planted mistakes.
"""

from __future__ import annotations

import numpy as np

from .gdn import bf16_round, sigmoid


def _f64(x):
    return np.asarray(x, dtype=np.float64)


def rms_norm(x, w, eps):
    """mlx ``nn.RMSNorm`` / ``mx.fast.rms_norm``: normalise the last axis, scale by w."""
    x = _f64(x)
    return x / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps) * _f64(w)


def silu(x):
    x = _f64(x)
    return x * sigmoid(x)


def rope(x, pos, rot, base):
    """Rotary embedding of the first ``rot`` dims of ``x`` [..., T, H, D] at
    positions ``pos`` [..., T] (rotate-half pairs d and d + rot/2)."""
    x = _f64(x).copy()
    if rot == 0:
        return x
    half = rot // 2
    inv_freq = base ** (-np.arange(half, dtype=np.float64) * 2.0 / rot)
    ang = _f64(pos)[..., None] * inv_freq  # [..., T, half]
    cos, sin = np.cos(ang)[..., None, :], np.sin(ang)[..., None, :]  # broadcast over heads
    x1, x2 = x[..., :half].copy(), x[..., half:rot].copy()
    x[..., :half] = x1 * cos - x2 * sin
    x[..., half:rot] = x2 * cos + x1 * sin
    return x


def attention(q, k_cache, v_cache, pos0, scale):
    """Causal GQA attention of T new tokens per row over the cache.

    q [B,T,Hq,D]; k_cache, v_cache [B,Hkv,L,D] (valid up to pos0[b] + T);
    token t of row b sees keys 0 .. pos0[b] + t.  Returns [B,T,Hq,D].
    """
    q, kc, vc = _f64(q), _f64(k_cache), _f64(v_cache)
    B, T, Hq, D = q.shape
    Hkv = kc.shape[1]
    g = Hq // Hkv
    out = np.zeros((B, T, Hq, D))
    for b in range(B):
        for t in range(T):
            n = int(pos0[b]) + t + 1
            for h in range(Hq):
                s = kc[b, h // g, :n] @ q[b, t, h] * scale
                p = np.exp(s - s.max())
                out[b, t, h] = (p / p.sum()) @ vc[b, h // g, :n]
    return out


def qk_prep(qg, k_new, v_new, q_norm_w, k_norm_w, eps, pos0, rot, base, Hq, Hkv, D, round_fn=None):
    """Split q / gate, q and k norms, rotary embedding; returns (q, gate, k, v)
    with shapes [B,T,H,D].  ``round_fn`` (e.g. bf16_round) is applied where
    the layer's activations are rounded: after each norm and after the
    rotation."""
    r = round_fn or (lambda a: a)
    qg = _f64(qg)
    B, T = qg.shape[:2]
    qg = qg.reshape(B, T, Hq, 2 * D)
    q, gate = qg[..., :D], qg[..., D:]
    k = _f64(k_new).reshape(B, T, Hkv, D)
    v = _f64(v_new).reshape(B, T, Hkv, D)
    pos = np.asarray(pos0, dtype=np.int64)[:, None] + np.arange(T)[None, :]
    q = r(rope(r(rms_norm(q, q_norm_w, eps)), pos, rot, base))
    k = r(rope(r(rms_norm(k, k_norm_w, eps)), pos, rot, base))
    return q, gate, k, v


def attention_layer(p, x, cache, args, round_fn=None):
    """The gated full-attention mixer on x [B,T,H] with a KV cache.

    ``p``: q_proj [2*Hq*D, H], k_proj / v_proj [Hkv*D, H], o_proj [H, Hq*D],
    q_norm / k_norm [D].  ``cache``: dict(k=[B,Hkv,L,D], v=..., offset=[B]),
    updated in place (the new keys appended, offset advanced).
    """
    r = round_fn or (lambda a: a)
    x = _f64(x)
    B, T, _ = x.shape
    Hq, Hkv, D = args["Hq"], args["Hkv"], args["D"]
    qg = r(x @ _f64(p["q_proj"]).T)
    kn = r(x @ _f64(p["k_proj"]).T)
    vn = r(x @ _f64(p["v_proj"]).T)
    pos0 = np.asarray(cache["offset"], dtype=np.int64)
    q, gate, k, v = qk_prep(qg, kn, vn, p["q_norm"], p["k_norm"], args["eps"], pos0, args["rot"],
                            args["base"], Hq, Hkv, D, round_fn)
    for b in range(B):
        o = int(pos0[b])
        cache["k"][b, :, o:o + T] = k[b].transpose(1, 0, 2)
        cache["v"][b, :, o:o + T] = v[b].transpose(1, 0, 2)
    a = r(attention(q, cache["k"], cache["v"], pos0, D ** -0.5) * sigmoid(gate))
    cache["offset"] = pos0 + T
    return r(a.reshape(B, T, Hq * D) @ _f64(p["o_proj"]).T)


def mlp(p, x, round_fn=None):
    """SwiGLU: down(silu(gate(x)) * up(x))."""
    r = round_fn or (lambda a: a)
    x = _f64(x)
    h = r(silu(r(x @ _f64(p["gate_proj"]).T)) * r(x @ _f64(p["up_proj"]).T))
    return r(h @ _f64(p["down_proj"]).T)


def decoder_layer(p, x, cache, args, round_fn=None):
    """Pre-norm residual blocks: x + attn(norm(x)), then h + mlp(norm(h))."""
    r = round_fn or (lambda a: a)
    x = _f64(x)
    h = r(x + attention_layer(p["self_attn"], r(rms_norm(x, p["input_layernorm"], args["eps"])), cache, args,
                              round_fn))
    return r(h + mlp(p["mlp"], r(rms_norm(h, p["post_attention_layernorm"], args["eps"])), round_fn))


def mtp_head(p, embed, hidden, caches, args, round_fn=None):
    """``MTPHead.__call__`` (mtp.py:181-194): post-norm hidden [B,L,H]."""
    r = round_fn or (lambda a: a)
    e = r(rms_norm(embed, p["pre_fc_norm_embedding"], args["eps"]))
    h = r(rms_norm(hidden, p["pre_fc_norm_hidden"], args["eps"]))
    x = r(np.concatenate([e, h], axis=-1) @ _f64(p["fc"]).T)
    for lp, c in zip(p["layers"], caches):
        x = decoder_layer(lp, x, c, args, round_fn)
    return r(rms_norm(x, p["norm"], args["eps"]))


def empty_cache(B, Hkv, L, D):
    return {"k": np.zeros((B, Hkv, L, D)), "v": np.zeros((B, Hkv, L, D)), "offset": np.zeros(B, dtype=np.int64)}


__all__ = ["rms_norm", "silu", "rope", "attention", "qk_prep", "attention_layer", "mlp", "decoder_layer",
           "mtp_head", "empty_cache", "bf16_round"]
