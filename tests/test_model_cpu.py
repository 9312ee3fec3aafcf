"""CPU checks of the model-level oracle and of the synthetic model files (no GPU).

The oracle's whole-model forward is pinned against an independent numpy forward of the same
MLX-format files, read by the test-side reader `qfix.read_safetensors` (numpy over the raw header and
buffer; independent of the oracle's C reader) and dequantized with numpy bit arrays: embedding row, RMSNorm, q/k-norm, half-split RoPE, GQA attention with a
bf16 KV cache, SwiGLU, tied / untied lm_head (Transformer.swift:1323-1584).
"""
import json
import os

import numpy as np
import pytest

import configs
import mlxr
import oracle
from qfix import bf16_round, bf16_to_f32, read_safetensors, unpack_codes


def load_dequant(d):
    t = read_safetensors(os.path.join(d, "model.safetensors"))
    cfg = json.load(open(os.path.join(d, "config.json")))
    bits, gs = cfg["quantization"]["bits"], cfg["quantization"]["group_size"]

    def lin(p):
        w = t[p + ".weight"]
        O = w.shape[0]
        K = w.shape[1] * 32 // bits
        packed = w.view(np.uint8).reshape(O, -1)
        codes = np.stack([unpack_codes(packed[r], K, bits) for r in range(O)]).astype(np.float32)
        s = bf16_to_f32(t[p + ".scales"])
        b = bf16_to_f32(t[p + ".biases"])
        g = np.repeat(np.arange(K // gs), gs)
        W = codes * s[:, g] + b[:, g]
        bias = bf16_to_f32(t[p + ".bias"]) if p + ".bias" in t else None
        return W.astype(np.float32), bias

    def vec(n):
        return bf16_to_f32(t[n]) if n in t else None
    return cfg, t, lin, vec


def numpy_forward(d, tokens):
    cfg, t, lin, vec = load_dequant(d)
    H, L, nH, nKV, D, eps = cfg["hidden_size"], cfg["num_hidden_layers"], cfg["num_attention_heads"], cfg["num_key_value_heads"], cfg["head_dim"], cfg["rms_norm_eps"]
    theta = float(np.float32(cfg["rope_theta"]))
    invf = (1.0 / theta ** (np.arange(0, D, 2, dtype=np.float64) / D)).astype(np.float32)
    E, _ = lin("model.embed_tokens")
    T = len(tokens)
    h = E[tokens].astype(np.float64)

    def rms(x, w):
        return x / np.sqrt((x ** 2).mean(-1, keepdims=True) + eps) * (w if w is not None else 1.0)

    def rope(x, pos):   # x [..., D], half-split
        a = np.float32(pos) * invf
        c, s = np.cos(a.astype(np.float64)), np.sin(a.astype(np.float64))
        x1, x2 = x[..., :D // 2], x[..., D // 2:]
        return np.concatenate([x1 * c - x2 * s, x2 * c + x1 * s], -1)

    for li in range(L):
        p = f"model.layers.{li}"
        xn = rms(h, vec(p + ".input_layernorm.weight"))
        outs = []
        for n in ("q", "k", "v"):
            W, b = lin(f"{p}.self_attn.{n}_proj")
            y = xn @ W.T.astype(np.float64)
            outs.append(y + b if b is not None else y)
        q = outs[0].reshape(T, nH, D); k = outs[1].reshape(T, nKV, D); v = outs[2].reshape(T, nKV, D)
        qn, kn = vec(p + ".self_attn.q_norm.weight"), vec(p + ".self_attn.k_norm.weight")
        if qn is not None:
            q = rms(q, qn); k = rms(k, kn)
        pos = np.arange(T)
        q = np.stack([rope(q[i], pos[i]) for i in range(T)])
        k = np.stack([rope(k[i], pos[i]) for i in range(T)])
        k = bf16_to_f32(bf16_round(k.astype(np.float32))).astype(np.float64)
        v = bf16_to_f32(bf16_round(v.astype(np.float32))).astype(np.float64)
        att = np.zeros((T, nH, D))
        for i in range(T):
            for hh in range(nH):
                kv = hh // (nH // nKV)
                sc = (q[i, hh] / np.sqrt(D)) @ k[:i + 1, kv].T
                w = np.exp(sc - sc.max()); w /= w.sum()
                att[i, hh] = w @ v[:i + 1, kv]
        Wo, _ = lin(p + ".self_attn.o_proj")
        h = h + att.reshape(T, -1) @ Wo.T
        xn = rms(h, vec(p + ".post_attention_layernorm.weight"))
        Wg, _ = lin(p + ".mlp.gate_proj"); Wu, _ = lin(p + ".mlp.up_proj"); Wd, _ = lin(p + ".mlp.down_proj")
        g = xn @ Wg.T; u = xn @ Wu.T
        h = h + (g / (1 + np.exp(-g)) * u) @ Wd.T
    xn = rms(h, vec("model.norm.weight"))
    Wh = lin("lm_head")[0] if "lm_head.weight" in t else E
    return xn[-1] @ Wh.T


@pytest.mark.parametrize("family", ["qwen3", "qwen2", "llama"])
def test_oracle_forward_matches_numpy(tmp_path, family):
    cfg = configs.tiny(family, layers=1, hidden=128, heads=2, kv_heads=1, inter=256, vocab=200, tie=family == "qwen3")
    d = str(tmp_path / family)
    mlxr.synth_write(cfg, seed=99, directory=d)
    toks = np.array([3, 17, 150, 42, 7, 99], np.int32)
    ref = numpy_forward(d, toks)
    m = oracle.Model(d, 256)
    got = m.forward(toks, 0, small_t=8)            # fp32 decode-precision path for 6 tokens
    assert np.max(np.abs(got - ref)) < 2e-4
    m2 = oracle.Model(d, 256)
    inc = None
    for i, t in enumerate(toks):                    # token by token == all at once
        inc = m2.forward(np.array([t], np.int32), i)
    assert np.max(np.abs(inc - got)) < 1e-5


def test_synth_is_deterministic_and_valid(tmp_path):
    cfg = configs.tiny("qwen2", layers=1, hidden=128, heads=2, kv_heads=1, inter=256, vocab=64, tie=False)
    a, b, c = (str(tmp_path / n) for n in "abc")
    mlxr.synth_write(cfg, seed=5, directory=a)
    mlxr.synth_write(cfg, seed=5, directory=b)
    mlxr.synth_write(cfg, seed=6, directory=c)
    fa = open(os.path.join(a, "model.safetensors"), "rb").read()
    assert fa == open(os.path.join(b, "model.safetensors"), "rb").read()
    assert fa != open(os.path.join(c, "model.safetensors"), "rb").read()
    t = read_safetensors(os.path.join(a, "model.safetensors"))
    assert t["model.layers.0.self_attn.q_proj.weight"].shape == (256, 128 * 4 // 32)
    assert t["model.layers.0.self_attn.q_proj.scales"].shape == (256, 2)
    assert "model.layers.0.self_attn.q_proj.bias" in t and "lm_head.weight" in t
    # weights ~ N(0, 0.02): dequantized statistics
    cfgj, _, lin, _ = load_dequant(a)
    W, _ = lin("model.layers.0.mlp.up_proj")
    assert abs(W.mean()) < 2e-3 and 0.017 < W.std() < 0.023


def test_quantize_row_bounds():
    rng = np.random.default_rng(1)
    for bits, gs in ((4, 64), (3, 32), (6, 128), (8, 64), (2, 32)):
        w = rng.normal(0, 0.02, 1024).astype(np.float32)
        codes, s, b = mlxr.quantize_row(w, bits, gs)
        q = unpack_codes(codes, 1024, bits)
        assert q.max() < (1 << bits)
        sf, bf = bf16_to_f32(s), bf16_to_f32(b)
        g = np.repeat(np.arange(1024 // gs), gs)
        deq = q * sf[g] + bf[g]
        # rounding to the nearest level: error <= half a step (plus the bf16 rounding of scale / bias)
        span = np.array([w[i * gs:(i + 1) * gs].max() - w[i * gs:(i + 1) * gs].min() for i in range(1024 // gs)])
        assert np.all(np.abs(deq - w) <= (sf[g] / 2 + span[g] * 2 ** -7 + 1e-7))
