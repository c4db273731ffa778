"""Writes the golden fixtures in this directory.

The reference (wang1ang/multiplex) ships no GDN vectors, and its arithmetic
lives in mlx-lm, which is not installed.  The expected outputs here are
therefore computed by implementations independent of ``oracle/gdn.py``:

* the gated delta recurrence and its chunked form: the torch restatements in
  the ``transformers`` library (``torch_recurrent_gated_delta_rule`` and
  ``torch_chunk_gated_delta_rule`` of ``models/qwen3_next``), which take the
  decay in log space, the state as ``[B,H,Dk,Dv]``, scale q by 1/sqrt(Dk)
  internally and compute in float32;
* the gate transforms: ``torch.nn.functional.softplus`` / ``torch.sigmoid``;
* the prologue: ``torch.nn.functional.conv1d(groups=C)``, ``silu`` and
  ``rms_norm`` in float64;
* the epilogue's gated RMSNorm: transformers' ``Qwen3NextRMSNormGated``
  module, run in bfloat16 (bf16 and fp32 weight) and in float32;
* the whole mixer: transformers' ``Qwen3_5GatedDeltaNet`` module, run from
  given conv and recurrent states in float32 (prefill and single-token
  decode) and in bfloat16;
* the full-attention layer of the hybrid trunk: transformers'
  ``Qwen3_5DecoderLayer`` and ``Qwen3_5Attention`` (float32, a prefill then
  more tokens over its KV cache), and the MTP draft head composed from it as
  ``multiplex/kernel/mtp.py:181-194`` composes it.

Inputs are drawn from ``numpy.random.default_rng`` with fixed seeds.
Run: ``python tests/golden/make_golden.py [case ...]`` (needs transformers;
no argument writes every case).
"""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import torch
import torch.nn.functional as F

HERE = Path(__file__).resolve().parent


def _gdn_inputs(rng, B, T, Hk, Hv, Dk, Dv):
    q = rng.standard_normal((B, T, Hk, Dk))
    k = rng.standard_normal((B, T, Hk, Dk))
    q = q / np.linalg.norm(q, axis=-1, keepdims=True) / np.sqrt(Dk)
    k = k / np.linalg.norm(k, axis=-1, keepdims=True)
    v = rng.standard_normal((B, T, Hv, Dv))
    a = rng.standard_normal((B, T, Hv))
    b = rng.standard_normal((B, T, Hv))
    A_log = rng.uniform(0.0, np.log(16.0), Hv)
    dt_bias = rng.uniform(-1.0, 1.0, Hv)
    S0 = rng.normal(0.0, 0.02, (B, Hv, Dv, Dk))
    return dict(q=q, k=k, v=v, a=a, b=b, A_log=A_log, dt_bias=dt_bias, state=S0)


def _library_gates(d):
    A_log = torch.tensor(d["A_log"])
    a = torch.tensor(d["a"])
    dt = torch.tensor(d["dt_bias"])
    log_g = -torch.exp(A_log) * F.softplus(a + dt)
    beta = torch.sigmoid(torch.tensor(d["b"]))
    return log_g, beta


def _hf_args(d, Hv):
    Hk, Dk = d["q"].shape[2], d["q"].shape[3]
    r = Hv // Hk
    q = torch.tensor(d["q"]).repeat_interleave(r, dim=2) * np.sqrt(Dk)
    k = torch.tensor(d["k"]).repeat_interleave(r, dim=2)
    v = torch.tensor(d["v"])
    log_g, beta = _library_gates(d)
    st = torch.tensor(d["state"]).transpose(-1, -2).contiguous()
    return q, k, v, log_g, beta, st


def recurrent_case(name, seed, B, T, Hk, Hv, Dk, Dv):
    from transformers.models.qwen3_next.modeling_qwen3_next import torch_recurrent_gated_delta_rule

    d = _gdn_inputs(np.random.default_rng(seed), B, T, Hk, Hv, Dk, Dv)
    q, k, v, log_g, beta, st = _hf_args(d, Hv)
    y, S = torch_recurrent_gated_delta_rule(q, k, v, log_g, beta, st, True)
    d["y"] = y.double().numpy()
    d["state_out"] = S.double().transpose(-1, -2).numpy()
    d["g"] = torch.exp(log_g).numpy()
    d["beta"] = beta.numpy()
    np.savez_compressed(HERE / f"{name}.npz", **{kk: np.asarray(vv, dtype=np.float32) for kk, vv in d.items()})


def chunked_case(name, seed, B, T, Hk, Hv, Dk, Dv, chunk):
    from transformers.models.qwen3_next.modeling_qwen3_next import torch_chunk_gated_delta_rule

    d = _gdn_inputs(np.random.default_rng(seed), B, T, Hk, Hv, Dk, Dv)
    q, k, v, log_g, beta, st = _hf_args(d, Hv)
    y, S = torch_chunk_gated_delta_rule(q, k, v, log_g, beta, chunk_size=chunk, initial_state=st,
                                        output_final_state=True)
    d["y"] = y.double().numpy()
    d["state_out"] = S.double().transpose(-1, -2).numpy()
    d["chunk"] = np.array(chunk)
    np.savez_compressed(HERE / f"{name}.npz", **{kk: np.asarray(vv, dtype=np.float32) for kk, vv in d.items()})


def prologue_case(name, seed, B, S, Hk, Hv, D, Kt=4, eps=1e-6):
    rng = np.random.default_rng(seed)
    C = 2 * Hk * D + Hv * D
    qkv = rng.standard_normal((B, S, C))
    w = rng.normal(0.0, 0.5, (C, Kt))
    cs = rng.standard_normal((B, Kt - 1, C))
    mask = np.ones((B, S), dtype=bool)
    mask[0, S - 2] = False
    mask[-1, 0] = False
    x = torch.tensor(qkv) * torch.tensor(mask)[..., None]
    ci = torch.cat([torch.tensor(cs), x], dim=1)                    # [B, S+K-1, C]
    out = F.conv1d(ci.transpose(1, 2), torch.tensor(w)[:, None, :], groups=C)  # [B, C, S]
    out = F.silu(out.transpose(1, 2))
    kd = Hk * D
    qo = out[..., :kd].reshape(B, S, Hk, D)
    ko = out[..., kd:2 * kd].reshape(B, S, Hk, D)
    vo = out[..., 2 * kd:].reshape(B, S, Hv, D)
    qo = F.rms_norm(qo, (D,), eps=eps) / D
    ko = F.rms_norm(ko, (D,), eps=eps) / np.sqrt(D)
    np.savez_compressed(
        HERE / f"{name}.npz",
        qkv=qkv, weight=w, conv_state=cs, mask=mask.astype(np.float64),
        q=qo.numpy(), k=ko.numpy(), v=vo.numpy(), conv_state_out=ci[:, -(Kt - 1):].numpy(),
        dims=np.array([B, S, Hk, Hv, D, Kt], dtype=np.float64), eps=np.array(eps),
    )


def gated_norm_case(name, seed, rows, D, eps=1e-6):
    from transformers.models.qwen3_next.modeling_qwen3_next import Qwen3NextRMSNormGated

    rng = np.random.default_rng(seed)
    scale = 10.0 ** rng.uniform(-3, 3, (rows, 1))
    x = torch.tensor(rng.standard_normal((rows, D)) * scale, dtype=torch.float32).to(torch.bfloat16)
    gate = torch.tensor(rng.normal(0.0, 2.0, (rows, D)), dtype=torch.float32).to(torch.bfloat16)
    w = torch.tensor(rng.normal(1.0, 0.25, D), dtype=torch.float32).to(torch.bfloat16)
    x[0] = 0.75           # a constant row
    gate[1] = 0.0         # a zero gate
    outs = {}
    with torch.no_grad():
        m = Qwen3NextRMSNormGated(D, eps=eps).to(torch.bfloat16)
        m.weight.copy_(w)
        outs["out_bf16_wbf16"] = m(x, gate)
        m = Qwen3NextRMSNormGated(D, eps=eps).to(torch.float32)
        m.weight.copy_(w.float())
        outs["out_bf16_wf32"] = m(x, gate)
        outs["out_f32"] = m(x.float(), gate.float())
    np.savez_compressed(
        HERE / f"{name}.npz",
        x=x.float().numpy(), gate=gate.float().numpy(), weight=w.float().numpy(), eps=np.array(eps),
        **{k: v.float().numpy() for k, v in outs.items()},
    )


class _OneLayerCache:
    """The part of a transformers ``Cache`` that ``Qwen3_5GatedDeltaNet.forward``
    uses, for layer 0: a conv state ``[B, C, K]`` (transformers keeps K
    columns; the last K-1 are the previous inputs) and a recurrent state
    ``[B, H, Dk, Dv]``, both present (a continued sequence)."""

    def __init__(self, conv, rec):
        import types

        self.layers = [types.SimpleNamespace(conv_states={0: conv}, recurrent_states={0: rec}, record_past=False)]

    def has_previous_state(self, idx):
        return True

    def update_conv_state(self, x, idx, conv_kernel_size):
        layer = self.layers[idx]
        full = torch.cat([layer.conv_states[0], x], dim=-1)
        layer.conv_states[0] = full[..., -conv_kernel_size:].clone()
        return full

    def update_recurrent_state(self, st, idx):
        self.layers[idx].recurrent_states[0] = st.clone()


def mixer_case(name, seed, B, S, hidden, Hk, Hv, D, dtype, Kt=4, eps=1e-6):
    """transformers' ``Qwen3_5GatedDeltaNet`` (the GatedDeltaNet mixer of the
    Qwen3.5 family, whose layout -- in_proj_qkv / in_proj_z / in_proj_b /
    in_proj_a, depthwise conv1d, gated RMSNorm, out_proj -- is the one
    ``multiplex/kernel/dflash.py:343-381`` restates), run on the CPU from
    given conv and recurrent states: with S > 1 through its chunked path,
    with S = 1 through its single-token update."""
    import types

    from transformers.models.qwen3_5.modeling_qwen3_5 import Qwen3_5GatedDeltaNet

    rng = np.random.default_rng(seed)
    C = 2 * Hk * D + Hv * D
    cfg = types.SimpleNamespace(hidden_size=hidden, linear_num_value_heads=Hv, linear_num_key_heads=Hk,
                                linear_key_head_dim=D, linear_value_head_dim=D, linear_conv_kernel_dim=Kt,
                                hidden_act="silu", rms_norm_eps=eps, layer_types=["linear_attention"])
    prm = {
        "in_proj_qkv": rng.normal(0.0, hidden ** -0.5, (C, hidden)),
        "in_proj_z": rng.normal(0.0, hidden ** -0.5, (Hv * D, hidden)),
        "in_proj_b": rng.normal(0.0, hidden ** -0.5, (Hv, hidden)),
        "in_proj_a": rng.normal(0.0, hidden ** -0.5, (Hv, hidden)),
        "conv1d": rng.normal(0.0, 0.3, (C, Kt)),
        "A_log": rng.uniform(0.0, np.log(16.0), Hv),
        "dt_bias": rng.uniform(-1.0, 1.0, Hv),
        "norm": rng.normal(1.0, 0.2, D),
        "out_proj": rng.normal(0.0, (Hv * D) ** -0.5, (hidden, Hv * D)),
    }
    x = rng.standard_normal((B, S, hidden))
    conv_state = rng.standard_normal((B, Kt - 1, C))
    state = rng.normal(0.0, 0.05, (B, Hv, D, D))                 # [B, Hv, Dv, Dk]
    tdt = {"f32": torch.float32, "bf16": torch.bfloat16}[dtype]
    with torch.no_grad():
        m = Qwen3_5GatedDeltaNet(cfg, 0).to(tdt)
        for n, w in (("in_proj_qkv", "in_proj_qkv"), ("in_proj_z", "in_proj_z"), ("in_proj_b", "in_proj_b"),
                     ("in_proj_a", "in_proj_a"), ("out_proj", "out_proj")):
            getattr(m, n).weight.copy_(torch.tensor(prm[w]))
        m.conv1d.weight.copy_(torch.tensor(prm["conv1d"])[:, None, :])
        m.A_log.copy_(torch.tensor(prm["A_log"]))
        m.dt_bias.copy_(torch.tensor(prm["dt_bias"]))
        m.norm.weight.copy_(torch.tensor(prm["norm"]))
        # round every parameter / input to the module's dtype, and store the rounded values
        prm = {"in_proj_qkv": m.in_proj_qkv.weight, "in_proj_z": m.in_proj_z.weight, "in_proj_b": m.in_proj_b.weight,
               "in_proj_a": m.in_proj_a.weight, "conv1d": m.conv1d.weight[:, 0, :], "A_log": m.A_log,
               "dt_bias": m.dt_bias, "norm": m.norm.weight, "out_proj": m.out_proj.weight}
        prm = {k: v.double().numpy() for k, v in prm.items()}
        xt = torch.tensor(x).to(tdt)
        cst = torch.tensor(conv_state).to(tdt)
        conv_hf = torch.cat([torch.zeros(B, 1, C, dtype=tdt), cst], dim=1).transpose(1, 2).contiguous()
        st = torch.tensor(state, dtype=torch.float32)
        cache = _OneLayerCache(conv_hf, st.transpose(-1, -2).contiguous())
        out = m(xt, cache_params=cache)
        cs_out = cache.layers[0].conv_states[0][..., 1:].transpose(1, 2)
        st_out = cache.layers[0].recurrent_states[0].transpose(-1, -2)
    np.savez_compressed(
        HERE / f"{name}.npz",
        x=xt.double().numpy(), conv_state=cst.double().numpy(), state=st.double().numpy(),
        out=out.double().numpy(), conv_state_out=cs_out.double().numpy(), state_out=st_out.double().numpy(),
        dims=np.array([B, S, hidden, Hk, Hv, D, Kt], dtype=np.float64), eps=np.array(eps),
        **{f"p_{k}": v for k, v in prm.items()},
    )


def _attn_config(hidden, Hq, Hkv, D, rot_factor, base, inter, eps):
    from transformers.models.qwen3_5.configuration_qwen3_5 import Qwen3_5TextConfig

    cfg = Qwen3_5TextConfig(hidden_size=hidden, num_attention_heads=Hq, num_key_value_heads=Hkv, head_dim=D,
                            intermediate_size=inter, rms_norm_eps=eps, num_hidden_layers=1,
                            layer_types=["full_attention"], attention_bias=False,
                            rope_parameters={"rope_type": "default", "rope_theta": base,
                                             "partial_rotary_factor": rot_factor})
    cfg._attn_implementation = "eager"
    return cfg


def _causal_mask(B, T, offset, dtype):
    """Additive mask [B,1,T,offset+T]: token t sees keys 0 .. offset + t."""
    L = offset + T
    keep = torch.arange(L)[None, :] <= (offset + torch.arange(T))[:, None]
    m = torch.zeros(T, L, dtype=dtype).masked_fill(~keep, torch.finfo(dtype).min)
    return m[None, None].expand(B, 1, T, L)


def _decoder_layer(cfg, rng, hidden, Hq, Hkv, D, inter):
    """transformers' Qwen3_5DecoderLayer at a full-attention index with random
    weights; returns the module and its weights in mlx's convention (norm
    weights w with y = x / rms * w; transformers keeps w - 1)."""
    from transformers.models.qwen3_5.modeling_qwen3_5 import Qwen3_5DecoderLayer

    layer = Qwen3_5DecoderLayer(cfg, 0).to(torch.float32)
    sd = {
        "self_attn.q_proj.weight": rng.normal(0.0, hidden ** -0.5, (2 * Hq * D, hidden)),
        "self_attn.k_proj.weight": rng.normal(0.0, hidden ** -0.5, (Hkv * D, hidden)),
        "self_attn.v_proj.weight": rng.normal(0.0, hidden ** -0.5, (Hkv * D, hidden)),
        "self_attn.o_proj.weight": rng.normal(0.0, (Hq * D) ** -0.5, (hidden, Hq * D)),
        "self_attn.q_norm.weight": rng.normal(0.0, 0.2, D),
        "self_attn.k_norm.weight": rng.normal(0.0, 0.2, D),
        "mlp.gate_proj.weight": rng.normal(0.0, hidden ** -0.5, (inter, hidden)),
        "mlp.up_proj.weight": rng.normal(0.0, hidden ** -0.5, (inter, hidden)),
        "mlp.down_proj.weight": rng.normal(0.0, inter ** -0.5, (hidden, inter)),
        "input_layernorm.weight": rng.normal(0.0, 0.2, hidden),
        "post_attention_layernorm.weight": rng.normal(0.0, 0.2, hidden),
    }
    with torch.no_grad():
        for n, w in sd.items():
            layer.get_parameter(n).copy_(torch.tensor(w, dtype=torch.float32))
    mlx = {}
    for n, prm in layer.named_parameters():
        w = prm.detach().double().numpy()
        mlx[n] = w + 1.0 if n.endswith("norm.weight") else w
    return layer, mlx


def attention_case(name, seed, B, T0, T1, hidden, Hq, Hkv, D, rot_factor, base, inter, eps=1e-6):
    """transformers' Qwen3_5DecoderLayer (full attention: gated q_proj,
    q/k RMSNorm, partial rotary embedding, GQA, SwiGLU MLP) and its
    Qwen3_5Attention alone, in float32: a prefill of T0 tokens from an empty
    cache, then T1 more tokens over that cache."""
    from transformers import DynamicCache
    from transformers.models.qwen3_5.modeling_qwen3_5 import Qwen3_5TextRotaryEmbedding

    rng = np.random.default_rng(seed)
    cfg = _attn_config(hidden, Hq, Hkv, D, rot_factor, base, inter, eps)
    layer, mlx = _decoder_layer(cfg, rng, hidden, Hq, Hkv, D, inter)
    rotary = Qwen3_5TextRotaryEmbedding(cfg)
    x0 = rng.standard_normal((B, T0, hidden))
    x1 = rng.standard_normal((B, T1, hidden))
    out = {}
    with torch.no_grad():
        for tag, run in (("layer", lambda x, **kw: layer(x, **kw)),
                         ("attn", lambda x, **kw: layer.self_attn(x, **kw)[0])):
            cache = DynamicCache(config=cfg)
            off = 0
            for i, x in enumerate((x0, x1)):
                xt = torch.tensor(x, dtype=torch.float32)
                T = x.shape[1]
                pos = torch.arange(off, off + T)[None].expand(B, T)
                cos, sin = rotary(xt, pos)
                y = run(xt, position_embeddings=(cos, sin), attention_mask=_causal_mask(B, T, off, torch.float32),
                        position_ids=pos, past_key_values=cache)
                out[f"{tag}_out{i}"] = y.double().numpy()
                off += T
    np.savez_compressed(
        HERE / f"{name}.npz", x0=x0, x1=x1, dims=np.array([B, T0, T1, hidden, Hq, Hkv, D, inter], dtype=np.float64),
        rot=np.array(int(D * rot_factor)), base=np.array(base), eps=np.array(eps), **out,
        **{"p_" + k.replace(".", "__"): v for k, v in mlx.items()},
    )


def mtp_case(name, seed, B, L0, hidden, Hq, Hkv, D, rot_factor, base, inter, eps=1e-6):
    """The MTP draft head as ``multiplex/kernel/mtp.py:181-194`` composes it:
    plain RMSNorms (mlx ``nn.RMSNorm``, here torch.nn.functional.rms_norm) of
    the embedding and of the trunk hidden, ``fc`` over their concatenation,
    one transformers Qwen3_5DecoderLayer at a full-attention index, and a final
    RMSNorm; float32.  A first call over L0 positions from an empty draft
    cache, then one draft step over that cache."""
    from transformers import DynamicCache
    from transformers.models.qwen3_5.modeling_qwen3_5 import Qwen3_5TextRotaryEmbedding

    rng = np.random.default_rng(seed)
    cfg = _attn_config(hidden, Hq, Hkv, D, rot_factor, base, inter, eps)
    layer, mlx = _decoder_layer(cfg, rng, hidden, Hq, Hkv, D, inter)
    rotary = Qwen3_5TextRotaryEmbedding(cfg)
    head = {
        "pre_fc_norm_embedding": rng.normal(1.0, 0.2, hidden),
        "pre_fc_norm_hidden": rng.normal(1.0, 0.2, hidden),
        "fc": rng.normal(0.0, (2 * hidden) ** -0.5, (hidden, 2 * hidden)),
        "norm": rng.normal(1.0, 0.2, hidden),
    }
    ht = {k: torch.tensor(v, dtype=torch.float32) for k, v in head.items()}
    calls = [(rng.standard_normal((B, L, hidden)), rng.standard_normal((B, L, hidden))) for L in (L0, 1)]
    out = {}
    with torch.no_grad():
        cache = DynamicCache(config=cfg)
        off = 0
        for i, (emb, hid) in enumerate(calls):
            e = F.rms_norm(torch.tensor(emb, dtype=torch.float32), (hidden,), ht["pre_fc_norm_embedding"], eps)
            h = F.rms_norm(torch.tensor(hid, dtype=torch.float32), (hidden,), ht["pre_fc_norm_hidden"], eps)
            x = torch.cat([e, h], dim=-1) @ ht["fc"].T
            T = x.shape[1]
            pos = torch.arange(off, off + T)[None].expand(B, T)
            x = layer(x, position_embeddings=rotary(x, pos), attention_mask=_causal_mask(B, T, off, torch.float32),
                      position_ids=pos, past_key_values=cache)
            out[f"out{i}"] = F.rms_norm(x, (hidden,), ht["norm"], eps).double().numpy()
            out[f"embed{i}"], out[f"hidden{i}"] = emb, hid
            off += T
    np.savez_compressed(
        HERE / f"{name}.npz", dims=np.array([B, L0, hidden, Hq, Hkv, D, inter], dtype=np.float64),
        rot=np.array(int(D * rot_factor)), base=np.array(base), eps=np.array(eps), **out,
        **{"h_" + k: v for k, v in head.items()}, **{"p_" + k.replace(".", "__"): v for k, v in mlx.items()},
    )


CASES = {
    "recurrent_small": lambda: recurrent_case("recurrent_small", 11, B=2, T=6, Hk=2, Hv=4, Dk=16, Dv=8),
    "recurrent_hd128": lambda: recurrent_case("recurrent_hd128", 12, B=1, T=3, Hk=2, Hv=4, Dk=128, Dv=128),
    "chunked_t100": lambda: chunked_case("chunked_t100", 13, B=1, T=100, Hk=1, Hv=2, Dk=32, Dv=16, chunk=64),
    "prologue_small": lambda: prologue_case("prologue_small", 14, B=2, S=7, Hk=2, Hv=4, D=16),
    "gated_norm_small": lambda: gated_norm_case("gated_norm_small", 15, rows=48, D=128),
    "mixer_prefill_f32": lambda: mixer_case("mixer_prefill_f32", 16, B=2, S=6, hidden=48, Hk=2, Hv=4, D=16,
                                            dtype="f32"),
    "mixer_decode_f32": lambda: mixer_case("mixer_decode_f32", 17, B=3, S=1, hidden=48, Hk=2, Hv=4, D=16,
                                           dtype="f32"),
    "mixer_prefill_bf16": lambda: mixer_case("mixer_prefill_bf16", 18, B=2, S=6, hidden=48, Hk=2, Hv=4, D=16,
                                             dtype="bf16"),
    "attention_layer_f32": lambda: attention_case("attention_layer_f32", 19, B=2, T0=5, T1=2, hidden=48, Hq=4,
                                                  Hkv=2, D=16, rot_factor=0.5, base=1000.0, inter=40),
    "mtp_head_f32": lambda: mtp_case("mtp_head_f32", 20, B=2, L0=3, hidden=48, Hq=4, Hkv=2, D=16, rot_factor=0.25,
                                     base=10000.0, inter=40),
}


def main():
    names = sys.argv[1:] or list(CASES)
    for n in names:
        torch.set_default_dtype(torch.float64)
        CASES[n]()
    print("wrote", names, file=sys.stderr)


if __name__ == "__main__":
    main()
