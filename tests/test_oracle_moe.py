"""Pins of the oracle's GEMV, routing plan and MoE block.

Reference tests restated: moe_plan.rs:248-307 (plan invariants, inverse permutation, histogram,
refusals), qwen3_moe.rs:983-1014 (hand-computed identity expert). GEMV orders are pinned against
an independent float64 brute force and against each other.
"""
import math

import numpy as np
import pytest

E, K = 128, 8


def test_plan_groups_and_restores_all_assignments(oracle):
    # moe_plan.rs:253-275
    logits = np.full(3 * E, -20.0, dtype=np.float32)
    for t in range(3):
        for s in range(K):
            logits[t * E + (t * 11 + s)] = s + 1
    p = oracle.moe_plan(logits, 3, E, K)
    assert p["expert_offsets"][E] == 24
    for a in range(24):
        g = int(p["assignment_to_grouped"][a])
        assert p["grouped_to_assignment"][g] == a
        assert p["grouped_token_ids"][g] == a // 8
        e = int(p["topk_experts"][a])
        assert p["expert_offsets"][e] <= g < p["expert_offsets"][e + 1]
    for w in p["topk_weights"].reshape(-1, 8):
        assert abs(float(w.sum()) - 1.0) < 1e-6
    # descending logit order: slot 0 holds the largest (token t, slot 7 -> id t*11+7)
    for t in range(3):
        assert list(p["topk_experts"][t * 8:(t + 1) * 8]) == [t * 11 + 7 - s for s in range(8)]


def test_weighted_inverse_permutation_preserves_token_values(oracle):
    # moe_plan.rs:277-289
    p = oracle.moe_plan(np.array([4.0, 2.0, 1.0, 2.0, 4.0, 1.0], np.float32), 2, 3, 2)
    grouped = np.zeros(4 * 2, dtype=np.float32)
    for pos, tok in enumerate(p["grouped_token_ids"]):
        grouped[pos * 2] = tok + 1
        grouped[pos * 2 + 1] = (tok + 1) * 3.0
    out = np.zeros(4, dtype=np.float32)
    oracle.lib().oref_reduce_grouped(oracle.ptr(p["assignment_to_grouped"]),
                                     oracle.ptr(p["topk_weights"]), 2, 2, oracle.ptr(grouped), 2,
                                     oracle.ptr(out))
    np.testing.assert_allclose(out, [1.0, 3.0, 2.0, 6.0], atol=1e-6)


def test_five_hundred_branch_batch_histogram(oracle):
    # moe_plan.rs:291-301
    idx = np.arange(500 * E)
    logits = (((idx * 37 + idx // 128 * 19) % 257) / 32.0).astype(np.float32)
    p = oracle.moe_plan(logits, 500, E, K)
    counts = np.diff(p["expert_offsets"].astype(np.int64))
    assert counts.sum() == 4000
    assert (counts > 0).sum() > 100
    pr = counts[counts > 0] / 4000.0
    assert float(-(pr * np.log2(pr)).sum()) > 6.0


def test_plan_refuses_corrupt_values_and_shapes(oracle):
    # moe_plan.rs:303-307
    L = oracle.lib()
    te = np.zeros(4, np.uint32)
    tw = np.zeros(4, np.float32)
    nan = np.array([np.nan], np.float32)
    assert L.oref_moe_plan(oracle.ptr(nan), 1, 1, 1, oracle.ptr(te), oracle.ptr(tw), None, None,
                           None, None) <= -2
    assert L.oref_moe_plan(oracle.ptr(nan), 1, 1, 2, oracle.ptr(te), oracle.ptr(tw), None, None,
                           None, None) == -1


def test_plan_ties_go_to_the_lower_id_and_weights_follow_the_softmax(oracle):
    logits = np.zeros(E, np.float32)
    logits[[5, 9, 100, 3]] = [2.0, 2.0, 2.0, 1.0]
    p = oracle.moe_plan(logits, 1, E, K)
    assert list(p["topk_experts"][:4]) == [5, 9, 100, 3]
    assert list(p["topk_experts"][4:]) == [0, 1, 2, 4]   # the zeros, lowest ids first
    # weight = exp(l - max) / sum over the selected (the full denominator cancels)
    sel = np.array([2, 2, 2, 1, 0, 0, 0, 0], np.float64)
    want = np.exp(sel - 2) / np.exp(sel - 2).sum()
    np.testing.assert_allclose(p["topk_weights"], want, rtol=1e-6)
    # -0.0 ranks below +0.0 under total_cmp
    l2 = np.full(E, -1.0, np.float32)
    l2[7] = -0.0
    l2[3] = 0.0
    p2 = oracle.moe_plan(l2, 1, E, 2)
    assert list(p2["topk_experts"][:2]) == [3, 7]


def test_identity_expert_closed_form(oracle):
    # qwen3_moe.rs:983-1014: gate = I, up = 2I, down = I (h = i = 128), x = 1
    h = i = 128
    gu = np.zeros((E, 2 * i, h), np.uint8)
    dn = np.zeros((E, h, i), np.uint8)
    for c in range(128):
        gu[:, c, c] = 0x38
        gu[:, i + c, c] = 0x40
        dn[:, c, c] = 0x38
    gus = np.full((E, 2, 1), 0x3F80, np.uint16)
    dns = np.full((E, 1, 1), 0x3F80, np.uint16)
    x = np.ones(h, np.float32)
    router = np.zeros((E, h), np.uint16)
    logits = oracle.router_logits(router, x)
    p = oracle.moe_plan(logits, 1, E, K)
    out = np.zeros(h, np.float32)
    oracle.lib().oref_moe_forward(oracle.ptr(gu), oracle.ptr(gus), oracle.ptr(dn), oracle.ptr(dns),
                                  h, i, 1, K, oracle.ptr(p["topk_experts"]),
                                  oracle.ptr(p["topk_weights"]), oracle.ptr(x), 0, oracle.ptr(out))
    expected = 2.0 / (1.0 + math.exp(-1.0))
    assert np.abs(out - expected).max() < 1e-5
    # the engine's MoE block (grouped GEMV order) gives the same closed form
    moe = np.zeros(h, np.float32)
    oracle.lib().oref_moe_block(oracle.ptr(gu), oracle.ptr(gus), oracle.ptr(dn), oracle.ptr(dns),
                                E, h, i, K, oracle.ptr(p["topk_experts"]),
                                oracle.ptr(p["topk_weights"]), oracle.ptr(x), 0, oracle.ptr(moe))
    assert np.abs(moe - expected).max() < 1e-5


def _f64_gemv(w, s, x, table, bf):
    n, k = w.shape
    deq = table[w].astype(np.float64) * np.repeat(np.repeat(bf(s).astype(np.float64), 128, 0), 128, 1)
    return deq @ x.astype(np.float64)


@pytest.mark.parametrize("n,k", [(128, 128), (256, 768), (384, 2048)])
def test_fp8_gemv_orders_agree_with_a_float64_brute_force(oracle, n, k):
    w, s = oracle.synth_fp8(3, n + k, 1, n, k)
    rng = np.random.default_rng(n * k)
    x = rng.standard_normal(k).astype(np.float32)
    t = oracle.e4m3_table()
    want = _f64_gemv(w[0], s[0], x, t, oracle.bf16_to_f32)
    got = oracle.fp8_grouped(w, s, [0], x)[0]
    got_blk = oracle.dequant_matvec(w[0], s[0], x)
    scale = np.abs(want).max()
    assert np.abs(got - want).max() <= 1e-5 * scale
    assert np.abs(got_blk - want).max() <= 1e-5 * scale


def test_fp8_grouped_ids_and_row_modes(oracle):
    # grouped = the single GEMV per id; x shared or one row per group
    w, s = oracle.synth_fp8(4, 1, 6, 256, 256)
    rng = np.random.default_rng(2)
    ids = np.array([5, 0, 3, 3], np.uint32)
    x1 = rng.standard_normal(256).astype(np.float32)
    xg = rng.standard_normal((4, 256)).astype(np.float32)
    y1 = oracle.fp8_grouped(w, s, ids, x1)
    yg = oracle.fp8_grouped(w, s, ids, xg)
    for g, e in enumerate(ids):
        np.testing.assert_array_equal(y1[g], oracle.fp8_grouped(w[e:e + 1], s[e:e + 1], [0], x1)[0])
        np.testing.assert_array_equal(yg[g], oracle.fp8_grouped(w[e:e + 1], s[e:e + 1], [0], xg[g])[0])
    # a transposed scale (block index swapped) is caught by the brute force
    t = oracle.e4m3_table()
    want = _f64_gemv(w[5], s[5].T.copy() if s.shape[1] == s.shape[2] else s[5], x1, t,
                     oracle.bf16_to_f32)
    assert np.abs(y1[0] - want).max() > 1e-3 * np.abs(want).max()


def test_bf16_gemv_and_argmax(oracle):
    rng = np.random.default_rng(9)
    wf = (rng.standard_normal((300, 256)) * 0.02).astype(np.float32)
    w = oracle.f32_to_bf16(wf)
    x = rng.standard_normal(256).astype(np.float32)
    want = oracle.bf16_to_f32(w).astype(np.float64) @ x.astype(np.float64)
    got = oracle.bf16_gemv(w, x)
    assert np.abs(got - want).max() < 1e-5
    np.testing.assert_array_equal(oracle.bf16_gemv(w, x, threads=4), got)
    # argmax: lowest index of the max
    l = np.array([0.0, 3.0, -1.0, 3.0, 2.0], np.float32)
    assert oracle.argmax(l) == 1
    assert oracle.argmax(np.array([-5.0], np.float32)) == 0


def test_router_refinement_agrees_with_the_sequential_f32_router(oracle):
    # The f64-accumulated logits differ from the reference's sequential f32 sums by rounding
    # only, so top-8 agrees whenever the rank-8 / rank-9 margin is above that rounding.
    rng = np.random.default_rng(21)
    gate = oracle.f32_to_bf16((rng.standard_normal((E, 2048)) * 0.02).astype(np.float32))
    norm = np.ones(2048, np.float32)
    for t in range(40):
        x = rng.standard_normal(2048).astype(np.float32)
        ids_a, w_a, post_a, la = oracle.route(gate, norm, x, 1e-6, refined=False)
        ids_b, w_b, post_b, lb = oracle.route(gate, norm, x, 1e-6, refined=True)
        np.testing.assert_array_equal(post_a, post_b)
        assert np.abs(la - lb).max() < 1e-5
        srt = np.sort(lb)[::-1]
        if srt[7] - srt[8] > 1e-4:
            np.testing.assert_array_equal(ids_a, ids_b)
            np.testing.assert_allclose(w_a, w_b, rtol=1e-5)


def test_router_post_row_is_the_rmsnorm(oracle):
    rng = np.random.default_rng(4)
    gate = oracle.f32_to_bf16((rng.standard_normal((E, 2048)) * 0.02).astype(np.float32))
    nw = (1 + 0.1 * rng.standard_normal(2048)).astype(np.float32)
    x = rng.standard_normal(2048).astype(np.float32) * 3
    ids, w, post, logits = oracle.route(gate, nw, x, 1e-6)
    ref = x.astype(np.float64) / np.sqrt((x.astype(np.float64) ** 2).mean() + 1e-6) * nw
    assert np.abs(post - ref).max() < 1e-5
    want = oracle.bf16_to_f32(gate).astype(np.float64) @ post.astype(np.float64)
    assert np.abs(logits - want).max() < 1e-6
    order = np.argsort(-want, kind="stable")[:8]
    np.testing.assert_array_equal(ids, order)


def test_moe_block_w8a8_is_within_activation_rounding(oracle):
    # The W8A8 control differs from the f32-activation block by e4m3 activation rounding only
    # (about 2-3% rms); a dropped quantisation step would make them equal.
    rng = np.random.default_rng(5)
    h, i = 256, 128
    gu_w, gu_s = oracle.synth_fp8(6, 1, 4, 2 * i, h)
    dn_w, dn_s = oracle.synth_fp8(6, 2, 4, h, i)
    post = rng.standard_normal(h).astype(np.float32)
    ids = np.array([2, 0], np.uint32)
    wts = np.array([0.6, 0.4], np.float32)
    outs = []
    for q in (0, 1):
        o = np.zeros(h, np.float32)
        oracle.lib().oref_moe_block(oracle.ptr(gu_w), oracle.ptr(gu_s), oracle.ptr(dn_w),
                                    oracle.ptr(dn_s), 4, h, i, 2, oracle.ptr(ids), oracle.ptr(wts),
                                    oracle.ptr(post), q, oracle.ptr(o))
        outs.append(o)
    rel = np.linalg.norm(outs[0] - outs[1]) / np.linalg.norm(outs[0])
    assert 0.003 < rel < 0.1
