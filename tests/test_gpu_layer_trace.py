"""Layer parity of the decode graph at configuration 4's full size, on the reference's own bar.

The reference's full-size check (own30b_check, crates/aien-inference-abi/src/bin/own30b_check.rs:
632-700) traces a few layers of the engine's decode (LayerTrace, qwen3_moe_omega.rs:3227-3243)
over a short prompt and replays each traced layer on the host from the chip's own inputs:
attention from the traced residual rows entering the layer (replay_attention,
qwen3_moe_omega.rs:5520-5572), the MoE from the host's RMSNorm of the traced residual after the
attention (replay_moe, :5584-5618). Per traced layer it requires attention and MoE cosine >= 0.999
(parity_stats, qwen3_moe.rs:699-735), the chip's expert set equal to the host's, routing weights
within 1e-4 of the host's (an expert the host did not pick counts as its whole weight), and the
device router's x' within 1e-4 of the host's (|d - p| / (1 + |p|)). Its negative controls must be
caught (own30b_check.rs:686-840): a routing mutant (every expert shifted to (e + 1) % experts)
and FP8 block scales dropped move the MoE cosine below 0.99; the decode attention without RoPE
moves the attention cosine below 0.99; router kernel mutants make the MoE replay disagree.

Here: the full 48-layer model synthesised on the device (the seed of tests/golden/
config4_greedy.npz), layers 0, 23 and 47 traced at every processed position of configuration 4's
decode: the 512 prompt tokens, then 63 greedy tokens the device chooses (575 positions); on the
host the oracle holds just those three layers (oref_model_synth_layers, the same generator) and
replays them: q|k|v and o with fp8_grouped (oref_fp8_grouped), the decode
attention over the layer's own bf16 K/V (oref_dattn_attend), the router (oref_router_logits_f64),
the plan (oref_moe_plan) and the FP8 MoE arm (oref_moe_block). Router mutant 1 (norm weight
ignored) is the identity on this model's unit norm weights and router mutant 3 moves only the
group tables, which the chain form does not read; the controls use router mutants 2 and 4.
"""
import os

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

FIXTURE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "config4_greedy.npz")
LAYERS = [0, 23, 47]
GENERATED = 63
CONTROL_TOKENS = 4
MAX_POS = 1024
THREADS = 16


def cosine(a, e):
    a = np.asarray(a, np.float64)
    e = np.asarray(e, np.float64)
    return float(a @ e / (np.sqrt(a @ a) * np.sqrt(e @ e)))


@pytest.fixture(scope="module")
def setup(omega, oracle):
    z = np.load(FIXTURE)  # numpy arrays only (allow_pickle off)
    seed = int(z["seed"])
    prompt = [int(t) for t in z["prompt"]]
    dev = omega.SynthDecodeModel(seed, MAX_POS)
    cfg = dict(dev.cfg)
    host = oracle.Model(dict(layers=cfg["layers"], hidden=cfg["hidden"], q_heads=cfg["q_heads"],
                             kv_heads=cfg["kv_heads"], head_dim=cfg["head_dim"],
                             experts=cfg["experts"], top_k=cfg["top_k"], inter=cfg["inter"],
                             vocab=16, eps=cfg["eps"], rope_theta=cfg["rope_theta"]),
                        seed, sigma=0.02, norm_sigma=0.0, threads=THREADS, layer_ids=LAYERS)
    yield dev, host, prompt
    dev.free()


def run_traced(dev, tokens, layers, generate=0):
    """Trace the given layers over the tokens, then `generate` greedy tokens; returns the records
    per layer and the token fed at every position."""
    g = dev.graph
    g.set_trace(layers)
    recs = [[] for _ in layers]
    fed = []
    try:
        tok = None
        for pos in range(len(tokens) + generate):
            if pos % 64 == 0:
                print(f"traced token pos {pos}", flush=True)
            tok_in = tokens[pos] if pos < len(tokens) else tok
            fed.append(tok_in)
            tok, _ = g.token_id(tok_in, pos)
            for i in range(len(layers)):
                recs[i].append(g.read_trace(i))
    finally:
        g.set_trace(None)
    return recs, fed


def replay(oracle, host, i, recs, eps, theta):
    """The host replay of subset layer i over consecutive traced positions 0..n-1: per position
    the attention cosine, the MoE cosine, whether the expert sets agree, the weight error and the
    router x' error. The attention runs position by position (its K/V cache grows); the MoE of
    every position is independent and runs on a pool of host threads."""
    from concurrent.futures import ThreadPoolExecutor

    qw, qs = host.tensor(i, 0)
    ow, os_ = host.tensor(i, 1)
    gw, gs = host.tensor(i, 2)
    dw, ds = host.tensor(i, 3)
    gate, in_norm, post_norm = host.tensor(i, 4), host.tensor(i, 5), host.tensor(i, 6)
    cache = oracle.Dattn(1, MAX_POS, theta)
    cache.set_norms(0, host.tensor(i, 7), host.tensor(i, 8))
    attn = []
    for t, r in enumerate(recs):
        xn = oracle.rmsnorm(r["x_in"], in_norm, eps)
        qkv = oracle.fp8_grouped(qw, qs, [0], xn, THREADS)[0]
        att = cache.attend(0, t, qkv, eps)
        attn.append(cosine(r["attn_proj"], oracle.fp8_grouped(ow, os_, [0], att, THREADS)[0]))

    def moe(t):
        r = recs[t]
        post = oracle.rmsnorm(r["x_mid"], post_norm, eps)
        xprime = float(np.max(np.abs(r["post"] - post) / (1.0 + np.abs(post))))
        logits = oracle.router_logits(gate, post, refined=True)
        plan = oracle.moe_plan(logits, 1, gate.shape[0], 8)
        ids, wts = plan["topk_experts"], plan["topk_weights"]
        want = oracle.moe_block(gw, gs, dw, ds, ids, wts, post)
        host_w = dict(zip(ids.tolist(), wts.tolist()))
        wt_err = max(abs(float(w) - host_w.get(int(e), 0.0)) for e, w in zip(r["experts"], r["weights"]))
        return dict(attn=attn[t], moe=cosine(r["moe_out"], want),
                    routing=sorted(r["experts"].tolist()) == sorted(ids.tolist()), wt_err=wt_err,
                    xprime=xprime)

    with ThreadPoolExecutor(THREADS) as ex:
        return list(ex.map(moe, range(len(recs))))


def summary(rows):
    return dict(attn=min(r["attn"] for r in rows), moe=min(r["moe"] for r in rows),
                routing=all(r["routing"] for r in rows), wt_err=max(r["wt_err"] for r in rows),
                xprime=max(r["xprime"] for r in rows))


def test_traced_layers_replay_on_the_reference_bar(oracle, setup):
    dev, host, prompt = setup
    c = dev.cfg
    recs, fed = run_traced(dev, prompt, LAYERS, GENERATED)
    assert len(recs[0]) == len(prompt) + GENERATED
    g = dev.graph
    for i, l in enumerate(LAYERS):
        for t, r in enumerate(recs[i]):
            # the record is one layer's arithmetic as the chain ran it: x' = x_in + attn_proj and
            # x_out = x' + moe_out (one f32 rounding each), ids / weights as the route log holds
            np.testing.assert_array_equal(r["x_mid"], (r["x_in"] + r["attn_proj"]).astype(np.float32))
            np.testing.assert_array_equal(r["x_out"], (r["x_mid"] + r["moe_out"]).astype(np.float32))
            if i + 1 < len(LAYERS) and LAYERS[i + 1] == l + 1:
                np.testing.assert_array_equal(recs[i + 1][t]["x_in"], r["x_out"])
        s = summary(replay(oracle, host, i, recs[i], c["eps"], c["rope_theta"]))
        print(f"PARITY layer {l} over {len(recs[i])} positions: attention cosine(min) {s['attn']:.6f} "
              f"moe cosine(min) {s['moe']:.6f} routing_agrees={s['routing']} routing weights "
              f"err(max) {s['wt_err']:.2e} router x' rel(max) {s['xprime']:.2e}", flush=True)
        assert s["attn"] >= 0.999 and s["moe"] >= 0.999, (l, s)
        assert s["routing"], (l, s)
        assert s["wt_err"] <= 1e-4 and s["xprime"] <= 1e-4, (l, s)
    ids, w = g.read_routes()
    last = recs[-1][-1]
    np.testing.assert_array_equal(ids[LAYERS[-1]], last["experts"])
    np.testing.assert_array_equal(w[LAYERS[-1]].view(np.uint32), last["weights"].view(np.uint32))
    # the trace does not change the arithmetic: the same tokens replayed by the graph (no trace)
    # end on the same residual row and the same logits
    xa, _, la = g.read(x=True, logits=True)
    for pos, tok in enumerate(fed):
        g.token_id(tok, pos)
    xb, _, lb = g.read(x=True, logits=True)
    np.testing.assert_array_equal(xa.view(np.uint32), xb.view(np.uint32))
    np.testing.assert_array_equal(la.view(np.uint32), lb.view(np.uint32))


@pytest.mark.parametrize("name", ["routing-mutant", "fp8-scales-dropped", "attention-mutant-1",
                                  "router-mutant-2", "router-mutant-4"])
def test_negative_controls_are_caught(omega, oracle, setup, name):
    dev, host, prompt = setup
    c = dev.cfg
    g = dev.graph
    lib = omega.lib()
    sets = {
        "routing-mutant": (lambda: g.test_set_mutant(4), lambda: g.test_set_mutant(0)),
        "fp8-scales-dropped": (lambda: g.test_set_mutant(5), lambda: g.test_set_mutant(0)),
        "attention-mutant-1": (lambda: lib.omega_gpu_decode_attn_test_set_mutant(1),
                               lambda: lib.omega_gpu_decode_attn_test_set_mutant(0)),
        "router-mutant-2": (lambda: lib.omega_gpu_router_test_set_mutant(2),
                            lambda: lib.omega_gpu_router_test_set_mutant(0)),
        "router-mutant-4": (lambda: lib.omega_gpu_router_test_set_mutant(4),
                            lambda: lib.omega_gpu_router_test_set_mutant(0)),
    }
    on, off = sets[name]
    on()  # the traced tokens run as direct launches: each launch reads the mutant it is given
    try:
        recs = run_traced(dev, prompt[:CONTROL_TOKENS], [LAYERS[0]])[0][0]
    finally:
        off()
    s = summary(replay(oracle, host, 0, recs, c["eps"], c["rope_theta"]))
    if name == "attention-mutant-1":
        caught = s["attn"] < 0.99
    elif name.startswith("router-mutant"):
        caught = s["moe"] < 0.99 or not s["routing"] or s["wt_err"] > 1e-3 or s["xprime"] > 1e-4
    else:
        caught = s["moe"] < 0.99
    print(f"CONTROL {name}: layer {LAYERS[0]} {s} -> {'CAUGHT' if caught else 'NOT CAUGHT'}", flush=True)
    assert caught, (name, s)
