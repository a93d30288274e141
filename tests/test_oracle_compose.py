"""Pins of the oracle's compositions: the whole engine step, the fused decode attention and the
paged attention, each against a restatement that shares no code with the oracle.

1. The engine step (oracle/oracle.c oref_engine_step + oref_engine_logits, the restatement of
   Qwen3MoeOmegaEngine::step / logits, qwen3_moe_omega.rs:4096-4368) against an independent
   numpy forward modelled on the reference's naive_forward (qwen3_moe_omega.rs:4598-4718):
   dequantised weights, f64 arithmetic, its own e4m3 decoding, norms, RoPE, attention loop,
   top-k and experts. The bar is the reference's own test
   engine_forward_matches_a_naive_reference_at_every_position (:5311-5331): logits cosine
   > 0.9999 and the same argmax at every position, over 2 layers of the real layer shape (hidden
   2048, 32 / 4 heads of 128, 128 experts top-8, intermediate 768). Three wiring mistakes planted
   in the oracle (oref_set_mutant) must each break the bar: the input and post-attention norms
   swapped, q rotated one position late, the K/V row appended one slot late.
2. oref_dattn_attend by closed forms: at position 0 every head returns its KV head's (bf16) V
   row; with one key repeated at every position the output is the mean of V; out_scale scales
   linearly; the K row it appends is the bf16 of the RMSNormed, rotated k.
3. oref_paged_attention against a gather that walks the page table by hand (independent offset
   arithmetic) and an f64 softmax.
"""
import ctypes as C

import numpy as np
import pytest

SEED, VOCAB = 4711, 8192
L, H, QH, KVH, HD, E, TOPK, I = 2, 2048, 32, 4, 128, 128, 8, 768
EPS, THETA = 1e-6, 1e6


def e4m3_decode(code):
    """OCP e4m3fn from the bit fields: bias 7, 3 mantissa bits, subnormals at 2^-6 * m/8,
    S.1111.111 NaN."""
    c = code.astype(np.int64)
    s = np.where(c & 0x80, -1.0, 1.0)
    e = (c >> 3) & 0xF
    m = c & 0x7
    v = np.where(e == 0, m / 8.0 * 2.0 ** -6, (1.0 + m / 8.0) * 2.0 ** (e - 7.0))
    v = np.where((c & 0x7F) == 0x7F, np.nan, v)
    return s * v


E4M3 = e4m3_decode(np.arange(256))


def bf16(bits):
    return (bits.astype(np.uint32) << 16).view(np.float32).astype(np.float64)


def dequant(w, s):
    """[n][k] e4m3 codes times their 128 x 128 block's bf16 scale, f64."""
    sc = np.repeat(np.repeat(bf16(s), 128, axis=0), 128, axis=1)
    return E4M3[w] * sc


def rms(x, w):
    return x / np.sqrt(np.mean(x * x) + EPS) * w


def rope(v, heads, pos):
    i = np.arange(HD // 2)
    ang = pos * THETA ** (-2.0 * i / HD)
    c, s = np.cos(ang), np.sin(ang)
    v = v.reshape(heads, HD)
    a, b = v[:, :64], v[:, 64:]
    return np.concatenate([a * c - b * s, a * s + b * c], axis=1).reshape(-1)


class Naive:
    """Plain f64 forward over the oracle model's raw tensors (nothing of the oracle is called)."""

    def __init__(self, m):
        self.m = m
        self.w = []
        for l in range(L):
            qkv = dequant(*[a[0] for a in m.tensor(l, 0)])
            o = dequant(*[a[0] for a in m.tensor(l, 1)])
            norms = [m.tensor(l, k).astype(np.float64) for k in (5, 6, 7, 8)]
            self.w.append((qkv, o, bf16(m.tensor(l, 4)), norms))
        self.gu, self.dn = [m.tensor(l, 2) for l in range(L)], [m.tensor(l, 3) for l in range(L)]
        self.embed, self.lm = m.embed(), m.lm_head()
        self.final = m.final_norm().astype(np.float64)
        self.keys = [[] for _ in range(L)]
        self.vals = [[] for _ in range(L)]

    def step(self, tok, pos):
        x = bf16(self.embed[tok])
        for l in range(L):
            qkv_w, o_w, gate, (n_in, n_post, n_q, n_k) = self.w[l]
            y = qkv_w @ rms(x, n_in)
            q = np.concatenate([rms(h, n_q) for h in y[:QH * HD].reshape(QH, HD)])
            k = np.concatenate([rms(h, n_k) for h in y[QH * HD:(QH + KVH) * HD].reshape(KVH, HD)])
            v = y[(QH + KVH) * HD:]
            q, k = rope(q, QH, pos), rope(k, KVH, pos)
            self.keys[l].append(k.reshape(KVH, HD))
            self.vals[l].append(v.reshape(KVH, HD))
            K, V = np.stack(self.keys[l]), np.stack(self.vals[l])  # [ctx][KVH][HD]
            att = np.empty((QH, HD))
            for h in range(QH):
                sc = K[:, h // 8] @ q[h * HD:(h + 1) * HD] / np.sqrt(HD)
                p = np.exp(sc - sc.max())
                att[h] = (p / p.sum()) @ V[:, h // 8]
            x = x + o_w @ att.reshape(-1)
            post = rms(x, n_post)
            logits = gate @ post
            ids = np.argsort(-logits, kind="stable")[:TOPK]
            wts = np.exp(logits[ids] - logits[ids[0]])
            wts /= wts.sum()
            for e, wt in zip(ids, wts):
                gu = dequant(self.gu[l][0][e], self.gu[l][1][e]) @ post
                g, u = gu[:I], gu[I:]
                act = g / (1.0 + np.exp(-g)) * u
                x = x + wt * (dequant(self.dn[l][0][e], self.dn[l][1][e]) @ act)
        return bf16(self.lm) @ rms(x, self.final)


def cosine(a, b):
    a, b = a.astype(np.float64), b.astype(np.float64)
    return float(a @ b / np.sqrt((a @ a) * (b @ b)))


@pytest.fixture(scope="module")
def model(oracle):
    cfg = dict(layers=L, hidden=H, q_heads=QH, kv_heads=KVH, head_dim=HD, experts=E, top_k=TOPK,
               inter=I, vocab=VOCAB, eps=EPS, rope_theta=THETA)
    return oracle.Model(cfg, SEED, sigma=0.02, norm_sigma=0.1, threads=8)


@pytest.fixture(scope="module")
def naive_logits(model):
    nv = Naive(model)
    return [nv.step(t, pos) for pos, t in enumerate(TOKENS)]


TOKENS = [5, 17, 42, 3, 9, 60]  # the reference test's tokens


def engine_logits(oracle, model):
    eng = oracle.Engine(model, 64, refined_router=True, threads=8)
    return [eng.logits(eng.step(t)) for t in TOKENS]


def test_engine_step_matches_an_independent_forward(oracle, model, naive_logits):
    got = engine_logits(oracle, model)
    for pos, (g, w) in enumerate(zip(got, naive_logits)):
        c = cosine(g, w)
        assert c > 0.9999, (pos, c)
        assert int(np.argmax(g)) == int(np.argmax(w)), pos


@pytest.mark.parametrize("mutant", [1, 2, 3])
def test_planted_wiring_mistakes_break_the_bar(oracle, model, naive_logits, mutant):
    oracle.lib().oref_set_mutant(mutant)
    try:
        got = engine_logits(oracle, model)
    finally:
        oracle.lib().oref_set_mutant(0)
    worst = min(cosine(g, w) for g, w in zip(got, naive_logits))
    same_argmax = all(int(np.argmax(g)) == int(np.argmax(w)) for g, w in zip(got, naive_logits))
    assert worst < 0.9999 or not same_argmax, (mutant, worst)


def test_fused_attention_closed_forms(oracle):
    rng = np.random.default_rng(3)
    d = oracle.Dattn(1, 256, THETA)
    qn = (1 + 0.1 * rng.standard_normal(HD)).astype(np.float32)
    kn = (1 + 0.1 * rng.standard_normal(HD)).astype(np.float32)
    d.set_norms(0, qn, kn)
    qkv = (2 * rng.standard_normal(5120)).astype(np.float32)
    out = d.attend(0, 0, qkv, EPS).reshape(QH, HD)
    v_row = oracle.bf16_to_f32(oracle.f32_to_bf16(qkv[4608:])).reshape(KVH, HD)
    for h in range(QH):
        np.testing.assert_array_equal(out[h], v_row[h // 8])
    # the appended K row: bf16 of the per-head RMSNorm then RoPE at the position
    pos = 37
    qkv = (2 * rng.standard_normal(5120)).astype(np.float32)
    d.attend(0, pos, qkv, EPS)
    k = np.concatenate([rms(h.astype(np.float64), kn.astype(np.float64))
                        for h in qkv[4096:4608].reshape(KVH, HD)])
    k = rope(k, KVH, pos).reshape(KVH, HD)
    for h in range(KVH):
        got_k, got_v = d.read_row(0, h, pos)
        assert np.abs(oracle.bf16_to_f32(got_k) - k[h]).max() <= 2.0 ** -7 * np.abs(k[h]).max()
        np.testing.assert_array_equal(got_v, oracle.f32_to_bf16(qkv[4608 + h * HD:4608 + (h + 1) * HD]))
    # one key at positions 0 .. ctx - 2 (arbitrary V rows there), then the token at ctx - 1 with
    # its own row: two distinct scores, so the output is the closed-form two-key mixture
    # ((ctx - 1) w_rep mean(V_rep) + w_cur v_cur) / ((ctx - 1) w_rep + w_cur)
    ctx = 40
    key = oracle.f32_to_bf16(rng.standard_normal((KVH, HD)).astype(np.float32))
    vals = oracle.f32_to_bf16(rng.standard_normal((ctx, KVH, HD)).astype(np.float32))
    e = oracle.Dattn(1, 256, THETA)
    e.set_norms(0, np.ones(HD, np.float32), np.ones(HD, np.float32))
    for h in range(KVH):
        e.write_rows(0, h, 0, np.tile(key[h], (ctx - 1, 1)), vals[:ctx - 1, h])
    qkv = (2 * rng.standard_normal(5120)).astype(np.float32)
    out = e.attend(0, ctx - 1, qkv, EPS).reshape(QH, HD)
    q = np.concatenate([rms(h.astype(np.float64), np.ones(HD)) for h in qkv[:4096].reshape(QH, HD)])
    q = rope(q, QH, ctx - 1).reshape(QH, HD)
    for h in range(QH):
        g = h // 8
        k_cur, v_cur = (bf16(r) for r in e.read_row(0, g, ctx - 1))  # the row it appended
        s_rep = q[h] @ bf16(key[g]) / np.sqrt(HD)
        s_cur = q[h] @ k_cur / np.sqrt(HD)
        m = max(s_rep, s_cur)
        w_rep, w_cur = np.exp(s_rep - m), np.exp(s_cur - m)
        mean_v = bf16(vals[:ctx - 1, g]).mean(0)
        want = ((ctx - 1) * w_rep * mean_v + w_cur * v_cur) / ((ctx - 1) * w_rep + w_cur)
        assert np.abs(out[h] - want).max() <= 1e-5 * np.abs(want).max(), h
    # out_scale is a plain factor
    a = e.attend(0, 45, qkv, EPS, 1.0)
    b = e.attend(0, 45, qkv, EPS, 2.0 ** 64)
    np.testing.assert_allclose(b / 2.0 ** 64, a, rtol=1e-6)


def test_paged_attention_against_a_hand_walked_gather(oracle):
    rng = np.random.default_rng(5)
    blocks, layers, layer = 64, 3, 2
    lay = oracle.kv_layout(blocks, 16, layers, KVH, HD)
    pool = oracle.f32_to_bf16(rng.standard_normal(lay.pool_bytes // 2).astype(np.float32)).view(np.uint8)
    ctx = 16 * 9 + 5
    table = rng.permutation(blocks)[:10].astype(np.int32)
    q = rng.standard_normal(QH * HD).astype(np.float32)
    got = np.zeros(QH * HD, np.float32)
    oracle.lib().oref_paged_attention(oracle.ptr(q), oracle.ptr(pool), C.byref(lay), oracle.ptr(table), ctx,
                                      layer, QH, KVH, HD, oracle.ptr(got))
    # aien-kv-cache layout by hand: block * BS + layer * LS + plane * PS + token * TS + head * HS
    HS, TS = HD * 2, KVH * HD * 2
    PS = 16 * TS
    LS = 2 * PS
    BS = layers * LS
    words = pool.view(np.uint16)
    K = np.empty((ctx, KVH, HD))
    V = np.empty((ctx, KVH, HD))
    for t in range(ctx):
        blk, tok = int(table[t // 16]), t % 16
        for h in range(KVH):
            ko = (blk * BS + layer * LS + tok * TS + h * HS) // 2
            vo = (blk * BS + layer * LS + PS + tok * TS + h * HS) // 2
            K[t, h] = bf16(words[ko:ko + HD])
            V[t, h] = bf16(words[vo:vo + HD])
    want = np.empty((QH, HD))
    for h in range(QH):
        s = K[:, h // 8] @ q[h * HD:(h + 1) * HD].astype(np.float64) / np.sqrt(HD)
        p = np.exp(s - s.max())
        want[h] = (p / p.sum()) @ V[:, h // 8]
    assert np.abs(got - want.reshape(-1)).max() <= 1e-6 * np.abs(want).max()
    # a transposed table (the pages in another order) gives a different answer
    alt = np.zeros(QH * HD, np.float32)
    oracle.lib().oref_paged_attention(oracle.ptr(q), oracle.ptr(pool), C.byref(lay),
                                      oracle.ptr(table[::-1].copy()), ctx, layer, QH, KVH, HD, oracle.ptr(alt))
    assert np.abs(alt - want.reshape(-1)).max() > 1e-3


def test_paged_step_equals_the_engine_step(oracle, model):
    """pyoracle.paged_step (the engine step with the paged pool as its KV store, the oracle of the
    batched serving step) against oref_engine_step (the fused-cache store): the same arithmetic on
    the same bf16 rows, so hidden rows and routes are bit-identical at every position, whatever
    pages the table names."""
    rng = np.random.default_rng(6)
    blocks = 64
    lay = oracle.kv_layout(blocks, 16, L, KVH, HD)
    pool = np.zeros(lay.pool_bytes, np.uint8)
    table = rng.permutation(blocks)[:4].astype(np.int32)
    eng = oracle.Engine(model, 64, refined_router=True, threads=8)
    for pos, tok in enumerate([5, 17, 42, 3, 9, 60, 1, 8191, 600, 77, 5, 5, 13, 21, 34, 55, 89, 144]):
        want = eng.step(tok)
        got, routes, _ = oracle.paged_step(model, pool, lay, table, pos, tok, threads=8)
        np.testing.assert_array_equal(got, want)
        np.testing.assert_array_equal(routes, eng.last_routes()[0])
