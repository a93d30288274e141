"""Pins of the prefill oracle's composition (oracle/pyoracle.py prefill_w8a8), CPU only.

The whole-prompt prefill runs every GEMM on W8A8 operands. The reference defines the arithmetic
that its prefill is checked against as the decode step with every GEMV input put through the
same activation quantiser (fake_quant_row: e4m3 with a power-of-two scale per 128-block) at four
points (Qwen3MoeOmegaEngine::control_step, crates/aien-inference-abi/src/qwen3_moe_omega/
w8a8_control.rs:17-30, 55-207): the input-normed row before q|k|v, the attention output before
o, the post-normed row before gate|up (after the routing, which reads the unquantised row), and
the SwiGLU activation before down, rounded to bf16 first.

1. With the quantiser switched off, prefill_w8a8 is the oracle's decode step (oref_engine_step,
   the restatement of Qwen3MoeOmegaEngine::step) token by token up to the GEMV primitive: the
   prefill's q|k|v and o products sum in dequant_matvec's order, the engine's in fp8_grouped's
   (both pinned against an f64 brute force in test_oracle_moe.py). A token-major restatement of
   the step (below) equals the engine bit for bit with fp8_grouped and prefill_w8a8 bit for bit
   with dequant_matvec, so the two differ in nothing but that order; directly, their residual
   rows agree within 1e-3 relative (the order's 1e-7 differences move a bf16 K / V rounding now
   and then) and the routes agree away from near ties, while the W8A8 prefill is far outside
   that bar.
2. The W8A8 arm of the MoE block (oref_moe_block) equals a restatement composed from the pinned
   primitives in control_step's order (quantise the post row, grouped gate|up, SwiGLU, bf16
   round, quantise, grouped down, slot-order combine) bit for bit; with the quantisers taken out
   the same restatement equals the f32 arm bit for bit, so the two arms differ only by the
   quantisers. On rows whose 128-blocks are exactly e4m3 at power-of-two scales the quantiser is
   the identity.
3. prefill_w8a8 over a prompt equals a token-major restatement of control_step bit for bit
   (layer-major and token-major orders compute the same values: a token's attention at a layer
   reads only earlier tokens' K/V of that layer). Two plausible wiring mistakes planted in the
   restatement break the equality: the activation not rounded to bf16 before its quantiser, and
   the attention output not quantised before o. The restatement uses the same GEMV primitive as
   prefill_w8a8 (dequant_matvec, pinned against an f64 brute force in test_oracle_moe.py) so that
   the comparison is exact; it does not share prefill_w8a8's wiring.
"""
import numpy as np
import pytest

SEED = 9091
L, H, E, TOPK, I, VOCAB = 2, 2048, 128, 8, 768, 512


def model_config():
    return dict(layers=L, hidden=H, q_heads=32, kv_heads=4, head_dim=128, experts=E, top_k=TOPK,
                inter=I, vocab=VOCAB, eps=1e-6, rope_theta=1e6)


@pytest.fixture(scope="module")
def model(oracle):
    return oracle.Model(model_config(), SEED, sigma=0.02, norm_sigma=0.1, threads=8)


PROMPT = [5, 77, 301, 12, 450, 9]


def moe_restated(oracle, gw, gs, dw, ds, ids, wts, post, quant_post=True, round_act=True,
                 quant_act=True):
    """control_step's expert arm (w8a8_control.rs:160-190) from the primitives."""
    x = oracle.fake_quant(post) if quant_post else post
    gu = oracle.fp8_grouped(gw, gs, ids, x, threads=8)
    acts = []
    for s in range(len(ids)):
        a = oracle.swiglu(gu[s], I)
        if round_act:
            a = oracle.bf16_round(a)
        if quant_act:
            a = oracle.fake_quant(a)
        acts.append(a)
    dn = oracle.fp8_grouped(dw, ds, ids, np.stack(acts), threads=8)
    moe = np.zeros(H, np.float32)
    for s in range(len(ids)):
        moe = (moe + np.float32(wts[s]) * dn[s]).astype(np.float32)
    return moe


def test_w8a8_moe_arm_against_its_restatement(oracle, model):
    rng = np.random.default_rng(3)
    gw, gs = model.tensor(0, 2)
    dw, ds = model.tensor(0, 3)
    post = rng.standard_normal(H).astype(np.float32)
    logits = oracle.router_logits(model.tensor(0, 4), post)
    plan = oracle.moe_plan(logits, 1, E, TOPK)
    ids, wts = plan["topk_experts"], plan["topk_weights"]
    want = oracle.moe_block(gw, gs, dw, ds, ids, wts, post, w8a8=True)
    np.testing.assert_array_equal(moe_restated(oracle, gw, gs, dw, ds, ids, wts, post), want)
    # without the quantisers the restatement is the f32 arm
    f32 = oracle.moe_block(gw, gs, dw, ds, ids, wts, post, w8a8=False)
    np.testing.assert_array_equal(
        moe_restated(oracle, gw, gs, dw, ds, ids, wts, post, False, False, False), f32)
    assert not np.array_equal(f32, want)
    # planted mistakes break the equality
    for kw in (dict(round_act=False), dict(quant_post=False), dict(quant_act=False)):
        assert not np.array_equal(moe_restated(oracle, gw, gs, dw, ds, ids, wts, post, **kw), want), kw


def test_quantiser_is_the_identity_on_exact_blocks(oracle):
    # each 128-block: e4m3 values times a power of two, the block's largest magnitude in
    # [256, 448] so that the block scale the quantiser picks (fake_quant.rs:85-104) is that power
    rng = np.random.default_rng(8)
    table = oracle.e4m3_table()
    codes = np.concatenate([np.arange(0x00, 0x7F), np.arange(0x80, 0xFF)])
    vals = table[codes].astype(np.float32)
    row = []
    for b in range(16):
        blk = rng.choice(vals[np.abs(vals) <= 448], 128)
        blk[rng.integers(0, 128)] = 448.0 if b % 2 else -320.0
        row.append(blk * np.float32(2.0 ** (b - 12)))
    row = np.concatenate(row).astype(np.float32)
    np.testing.assert_array_equal(oracle.fake_quant(row), row)
    # and a value off the e4m3 grid is not kept
    bent = row.copy()
    bent[5] = np.nextafter(np.float32(bent[5] if bent[5] != 0 else 1.0), np.float32(np.inf))
    assert not np.array_equal(oracle.fake_quant(bent), bent)


def control_prefill_restated(oracle, model, tokens, round_act=True, quant_attn=True, w8a8=True,
                             gemv="matvec"):
    """Qwen3MoeOmegaEngine::control_step in W8A8 mode (w8a8_control.rs:55-207), token by token.
    With w8a8 False every quantiser and the act's bf16 rounding are left out (the decode step,
    qwen3_moe_omega.rs:4096-4345); gemv picks the q|k|v and o product's summation order."""
    c = model.cfg
    eps = c.eps
    fq = oracle.fake_quant if w8a8 else (lambda v: v)
    if gemv == "matvec":
        mv = lambda w, s, v: oracle.dequant_matvec(w[0], s[0], v)
    else:
        mv = lambda w, s, v: oracle.fp8_grouped(w, s, [0], v, threads=8)[0]
    cache = oracle.Dattn(L, 64, c.rope_theta)
    for l in range(L):
        cache.set_norms(l, model.tensor(l, 7), model.tensor(l, 8))
    emb = model.embed()
    x_out = [[None] * len(tokens) for _ in range(L)]
    ids_out = [[None] * len(tokens) for _ in range(L)]
    hidden = []
    for t, tok in enumerate(tokens):
        x = oracle.bf16_to_f32(emb[tok]).astype(np.float32)
        for l in range(L):
            qw, qs = model.tensor(l, 0)
            ow, os_ = model.tensor(l, 1)
            gw, gs = model.tensor(l, 2)
            dw, ds = model.tensor(l, 3)
            gate, in_norm, post_norm = model.tensor(l, 4), model.tensor(l, 5), model.tensor(l, 6)
            x_norm = fq(oracle.rmsnorm(x, in_norm, eps))                        # point 1
            qkv = mv(qw, qs, x_norm)
            attn = cache.attend(l, t, qkv, eps)
            if quant_attn:
                attn = fq(attn)                                                 # point 2
            x = (x + mv(ow, os_, attn)).astype(np.float32)
            post = oracle.rmsnorm(x, post_norm, eps)
            logits = oracle.router_logits(gate, post)                           # unquantised row
            plan = oracle.moe_plan(logits, 1, E, TOPK)
            moe = moe_restated(oracle, gw, gs, dw, ds, plan["topk_experts"], plan["topk_weights"],
                               post, quant_post=w8a8, round_act=round_act and w8a8,
                               quant_act=w8a8)                                  # points 3, 4
            x = (x + moe).astype(np.float32)
            x_out[l][t] = x.copy()
            ids_out[l][t] = plan["topk_experts"].copy()
        hidden.append(oracle.rmsnorm(x, model.final_norm(), eps))
    return hidden, x_out, ids_out


def test_prefill_without_quantiser_is_the_engine_step(oracle, model):
    eng = oracle.Engine(model, 64, refined_router=False, threads=8)
    want_hid, want_x, want_ids = control_prefill_restated(oracle, model, PROMPT, w8a8=False,
                                                          gemv="grouped")
    hid_eng, x_eng, ids_eng, margins = [], [], [], []
    for tok in PROMPT:
        hid_eng.append(eng.step(tok))
        ids, _, m = eng.last_routes()
        ids_eng.append(ids.copy())
        margins.append(m.copy())
        x_eng.append(eng.last_x().copy())
    # the restatement with the engine's GEMV is the engine, bit for bit
    for t in range(len(PROMPT)):
        np.testing.assert_array_equal(want_hid[t], hid_eng[t])
        np.testing.assert_array_equal(want_x[L - 1][t], x_eng[t])
        for l in range(L):
            np.testing.assert_array_equal(want_ids[l][t], ids_eng[t][l])
    # with the prefill's GEMV it is prefill_w8a8 without the quantiser, bit for bit
    hid, out = oracle.prefill_w8a8(model, PROMPT, max_pos=64, w8a8=False)
    m_hid, m_x, _ = control_prefill_restated(oracle, model, PROMPT, w8a8=False, gemv="matvec")
    np.testing.assert_array_equal(hid, m_hid[-1])
    for l in range(L):
        for t in range(len(PROMPT)):
            np.testing.assert_array_equal(out["x_out"][l][t], m_x[l][t])
    # directly: the two orders agree closely, the W8A8 prefill does not
    _, out8 = oracle.prefill_w8a8(model, PROMPT, max_pos=64)

    def worst(rows):
        return max(float(np.abs(rows[t] - x_eng[t]).max() / np.abs(x_eng[t]).max())
                   for t in range(len(PROMPT)))

    assert worst(out["x_out"][L - 1]) <= 1e-3
    assert worst(out8["x_out"][L - 1]) > 1e-2
    for t in range(len(PROMPT)):
        for l in range(L):
            if margins[t][l] > 1e-4:  # away from a near tie of ranks 8 and 9
                np.testing.assert_array_equal(out["ids"][l][t], ids_eng[t][l])


def test_prefill_is_the_control_step_restated(oracle, model):
    hid, out = oracle.prefill_w8a8(model, PROMPT, max_pos=64)
    want_hid, want_x, _ = control_prefill_restated(oracle, model, PROMPT)
    np.testing.assert_array_equal(hid, want_hid[-1])
    for l in range(L):
        for t in range(len(PROMPT)):
            np.testing.assert_array_equal(out["x_out"][l][t], want_x[l][t])
    # two plausible wiring mistakes, planted in the restatement, each break the equality
    for kw in (dict(round_act=False), dict(quant_attn=False)):
        h2, _, _ = control_prefill_restated(oracle, model, PROMPT, **kw)
        assert not np.array_equal(h2[-1], hid), kw
