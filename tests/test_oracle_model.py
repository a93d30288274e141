"""Pins of the oracle's RMSNorm, per-head norm, RoPE, GQA attention and SwiGLU.

1. The reference's HF fixture (tests/golden/qwen3_tiny, from crates/aien-inference-abi/fixtures):
   a dense Qwen3 forward composed from the oracle's primitives must give transformers' float32
   last-position logits within 1e-4 absolute (tests/qwen3_forward_parity.rs:19-22). Dropping the
   q/k norm or using the interleaved RoPE pairing moves the logits far outside it (checked).
2. Closed forms for attention and RoPE at head_dim 128.
"""
import json
import os
import struct

import numpy as np
import pytest

from conftest import GOLDEN

TINY = os.path.join(GOLDEN, "qwen3_tiny")


def load_safetensors_bf16(path):
    b = open(path, "rb").read()
    n = struct.unpack("<Q", b[:8])[0]
    hdr = json.loads(b[8:8 + n])
    base = 8 + n
    out = {}
    for name, meta in hdr.items():
        if name == "__metadata__":
            continue
        assert meta["dtype"] == "BF16"
        s, e = meta["data_offsets"]
        bits = np.frombuffer(b[base + s:base + e], dtype="<u2").reshape(meta["shape"])
        out[name] = bits
    return out


def tiny_forward(oracle, ids, qk_norm=True, rope="half"):
    cfg = json.load(open(os.path.join(TINY, "config.json")))
    t = load_safetensors_bf16(os.path.join(TINY, "model.safetensors"))
    f = {k: oracle.bf16_to_f32(v).astype(np.float32) for k, v in t.items()}
    H, hd, qh, kvh = cfg["hidden_size"], cfg["head_dim"], cfg["num_attention_heads"], \
        cfg["num_key_value_heads"]
    eps, theta = cfg["rms_norm_eps"], float(cfg["rope_theta"])
    emb = f["model.embed_tokens.weight"]
    keys = [[] for _ in range(cfg["num_hidden_layers"])]
    vals = [[] for _ in range(cfg["num_hidden_layers"])]
    for pos, tok in enumerate(ids):
        x = emb[tok].copy()
        for l in range(cfg["num_hidden_layers"]):
            p = f"model.layers.{l}."
            xn = oracle.rmsnorm(x, f[p + "input_layernorm.weight"], eps)
            q = (f[p + "self_attn.q_proj.weight"] @ xn).astype(np.float32)
            k = (f[p + "self_attn.k_proj.weight"] @ xn).astype(np.float32)
            v = (f[p + "self_attn.v_proj.weight"] @ xn).astype(np.float32)
            if qk_norm:
                q = oracle.rmsnorm_per_head(q, f[p + "self_attn.q_norm.weight"], eps, qh, hd)
                k = oracle.rmsnorm_per_head(k, f[p + "self_attn.k_norm.weight"], eps, kvh, hd)
            if rope == "half":
                q, k = oracle.apply_rope(q, k, pos, qh, kvh, hd, theta)
            else:  # planted mistake: interleaved pairs (2i, 2i+1)
                c, s = oracle.rope_cos_sin(theta, hd, pos)
                for arr, nh in ((q, qh), (k, kvh)):
                    a = arr.reshape(nh, hd // 2, 2)
                    a0, a1 = a[..., 0].copy(), a[..., 1].copy()
                    a[..., 0] = a0 * c - a1 * s
                    a[..., 1] = a0 * s + a1 * c
            keys[l].append(k)
            vals[l].append(v)
            att = oracle.sdpa(q, np.stack(keys[l]), np.stack(vals[l]), qh, kvh, hd)
            x = x + (f[p + "self_attn.o_proj.weight"] @ att).astype(np.float32)
            post = oracle.rmsnorm(x, f[p + "post_attention_layernorm.weight"], eps)
            g = (f[p + "mlp.gate_proj.weight"] @ post).astype(np.float32)
            u = (f[p + "mlp.up_proj.weight"] @ post).astype(np.float32)
            act = oracle.swiglu(np.concatenate([g, u]), g.size)
            x = x + (f[p + "mlp.down_proj.weight"] @ act).astype(np.float32)
    hid = oracle.rmsnorm(x, f["model.norm.weight"], eps)
    return (emb @ hid).astype(np.float32)     # tied lm_head


def test_tiny_qwen3_matches_transformers_float32(oracle):
    ref = json.load(open(os.path.join(TINY, "forward_reference.json")))
    logits = tiny_forward(oracle, ref["ids"])
    want = np.array(ref["logits"], np.float32)
    assert np.abs(logits - want).max() < 1e-4
    assert oracle.argmax(logits) == ref["argmax"]


def test_tiny_qwen3_negative_controls_move_far_outside_the_tolerance(oracle):
    ref = json.load(open(os.path.join(TINY, "forward_reference.json")))
    want = np.array(ref["logits"], np.float32)
    assert np.abs(tiny_forward(oracle, ref["ids"], qk_norm=False) - want).max() > 1e-2
    assert np.abs(tiny_forward(oracle, ref["ids"], rope="interleaved") - want).max() > 1e-3


def test_attention_closed_forms(oracle):
    qh, kvh, hd = 32, 4, 128
    rng = np.random.default_rng(0)
    q = rng.standard_normal(qh * hd).astype(np.float32)
    # one position: every head returns its KV head's V row (GQA group of 8)
    K = rng.standard_normal((1, kvh * hd)).astype(np.float32)
    V = rng.standard_normal((1, kvh * hd)).astype(np.float32)
    out = oracle.sdpa(q, K, V, qh, kvh, hd).reshape(qh, hd)
    for h in range(qh):
        np.testing.assert_array_equal(out[h], V[0, (h // 8) * hd:(h // 8 + 1) * hd])
    # identical keys: uniform softmax, the mean of V
    ctx = 37
    K = np.tile(rng.standard_normal((1, kvh * hd)).astype(np.float32), (ctx, 1))
    V = rng.standard_normal((ctx, kvh * hd)).astype(np.float32)
    out = oracle.sdpa(q, K, V, qh, kvh, hd).reshape(qh, hd)
    mean = V.astype(np.float64).mean(0)
    for h in range(qh):
        assert np.abs(out[h] - mean[(h // 8) * hd:(h // 8 + 1) * hd]).max() < 1e-6
    # brute force against an independent float64 softmax
    K = rng.standard_normal((ctx, kvh * hd)).astype(np.float32)
    out = oracle.sdpa(q, K, V, qh, kvh, hd).reshape(qh, hd)
    for h in range(qh):
        kv = h // 8
        kk = K[:, kv * hd:(kv + 1) * hd].astype(np.float64)
        s = kk @ q[h * hd:(h + 1) * hd].astype(np.float64) / np.sqrt(hd)
        p = np.exp(s - s.max())
        p /= p.sum()
        want = p @ V[:, kv * hd:(kv + 1) * hd].astype(np.float64)
        assert np.abs(out[h] - want).max() < 1e-6


def test_rope_closed_forms(oracle):
    qh, kvh, hd, theta = 32, 4, 128, 1e6
    rng = np.random.default_rng(1)
    q = rng.standard_normal(qh * hd).astype(np.float32)
    k = rng.standard_normal(kvh * hd).astype(np.float32)
    q0, k0 = oracle.apply_rope(q, k, 0, qh, kvh, hd, theta)
    np.testing.assert_array_equal(q0, q)          # position 0 is the identity
    np.testing.assert_array_equal(k0, k)
    pos = 517
    q1, k1 = oracle.apply_rope(q, k, pos, qh, kvh, hd, theta)
    c, s = oracle.rope_cos_sin(theta, hd, pos)
    i = np.arange(hd // 2)
    ang = pos * (1.0 / theta ** (2 * i / hd))
    assert np.abs(c - np.cos(ang)).max() < 1e-7 and np.abs(s - np.sin(ang)).max() < 1e-7
    for h in range(qh):
        a, b = q[h * hd:h * hd + 64], q[h * hd + 64:(h + 1) * hd]
        np.testing.assert_allclose(q1[h * hd:h * hd + 64], a * c - b * s, rtol=0, atol=1e-6)
        np.testing.assert_allclose(q1[h * hd + 64:(h + 1) * hd], a * s + b * c, rtol=0, atol=1e-6)
    # rotations keep each pair's length
    for v0, v1 in ((q, q1), (k, k1)):
        r0 = v0.reshape(-1, 2, 64)
        r1 = v1.reshape(-1, 2, 64)
        np.testing.assert_allclose((r0 ** 2).sum(1), (r1 ** 2).sum(1), rtol=1e-5)


def test_rmsnorm_closed_form(oracle):
    x = np.full(2048, 3.0, np.float32)
    w = np.linspace(0.5, 1.5, 2048).astype(np.float32)
    out = oracle.rmsnorm(x, w, 1e-6)
    want = 3.0 / np.sqrt(9.0 + 1e-6) * w.astype(np.float64)
    assert np.abs(out - want).max() < 1e-6
    heads = oracle.rmsnorm_per_head(np.arange(256, dtype=np.float32), np.ones(128, np.float32),
                                    1e-6, 2, 128)
    for h in range(2):
        v = np.arange(h * 128, (h + 1) * 128, dtype=np.float64)
        assert np.abs(heads[h * 128:(h + 1) * 128] - v / np.sqrt((v ** 2).mean() + 1e-6)).max() < 1e-5


def test_layer_subset_holds_the_full_models_layers(oracle):
    # oref_model_synth_layers: layer i of the subset is layer ids[i] of the whole model, every
    # tensor kind bit for bit (the full-size layer trace checks hold three of 48 layers this way)
    cfg = dict(layers=4, hidden=256, q_heads=2, kv_heads=1, head_dim=128, experts=4, top_k=2,
               inter=128, vocab=64, eps=1e-6, rope_theta=1e6)
    whole = oracle.Model(cfg, 77, sigma=0.02, norm_sigma=0.1, threads=8)
    ids = [3, 0, 2]
    part = oracle.Model(cfg, 77, sigma=0.02, norm_sigma=0.1, threads=8, layer_ids=ids)
    assert part.cfg.layers == 3
    for i, l in enumerate(ids):
        for kind in range(9):
            a, b = part.tensor(i, kind), whole.tensor(l, kind)
            for u, v in zip(a if kind < 4 else (a,), b if kind < 4 else (b,)):
                np.testing.assert_array_equal(u, v)
    # different layers really differ (the map is not the identity by accident)
    assert not np.array_equal(part.tensor(0, 2)[0], whole.tensor(0, 2)[0])
    np.testing.assert_array_equal(part.embed(), whole.embed())
    with pytest.raises(ValueError):
        oracle.Model(cfg, 77, layer_ids=[4])
