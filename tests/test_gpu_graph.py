"""GPU parity of the whole decode step (one hipGraph per token) against the oracle engine.

The model is the real Qwen3-30B-A3B layer shape (hidden 2048, 32/4 heads of 128, 128 experts
top-8, intermediate 768) with fewer layers and a smaller vocabulary so the CPU oracle runs in
seconds; seeded random-init weights from the shared generator, norm weights 1 + N(0, 0.1).
Bars: greedy tokens identical at every step; logits within 2e-3 relative; routed experts of
every layer identical to the oracle's.
Reference: crates/aien-omega-dgraph (ABI), qwen3_moe_omega.rs:4096-4368 (step + logits).
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu
TOL = 2e-3


def rel_err(a, e):
    return float(np.abs(a - e).max() / max(np.abs(e).max(), 1e-30))


def model_config(layers, vocab):
    return dict(layers=layers, hidden=2048, q_heads=32, kv_heads=4, head_dim=128, experts=128,
                top_k=8, inter=768, vocab=vocab, eps=1e-6, rope_theta=1e6)


class GpuModel:
    """Uploads an oracle model through the C ABI, the way OmegaModelUploader does
    (qwen3_moe_omega.rs:1231-1598): FP8 projections, router layers and directories, the fused
    decode cache with its norms, the bf16 lm_head, and the decode graph over them."""

    def __init__(self, omega, m, max_pos):
        c = m.cfg
        self.omega, self.m = omega, m
        self.layers = []
        self.router = omega.Router(c.layers)
        self.cache = omega.DecodeAttnCache(c.layers, max_pos, c.rope_theta)
        for l in range(c.layers):
            ts = []
            for kind in range(4):
                w, s = m.tensor(l, kind)
                ts.append(omega.Fp8Tensor.upload(w.shape[0], w.shape[1], w.shape[2], w, s))
            self.layers.append(ts)
            self.router.set_layer(l, m.tensor(l, 4), m.tensor(l, 6))
            gu = np.array([ts[2].entry(e) for e in range(c.experts)], np.uint64)
            dn = np.array([ts[3].entry(e) for e in range(c.experts)], np.uint64)
            self.router.set_directory(l, gu, dn)
            self.cache.set_norms(l, m.tensor(l, 7), m.tensor(l, 8))
        self.lm = omega.Bf16Tensor.upload(c.vocab, c.hidden, m.lm_head())
        self.graph = omega.DecodeGraph(c.layers, c.vocab, c.eps, self.router, self.cache, self.lm)
        for l in range(c.layers):
            q, o, g, d = self.layers[l]
            self.graph.set_layer(l, q, o, g, d, m.tensor(l, 5))
        self.graph.set_final_norm(m.final_norm())
        self.embed = m.embed()

    def x_embed(self, token):
        return (self.embed[token % self.m.cfg.vocab].astype(np.uint32) << 16).view(np.float32)

    def free(self):
        self.graph.free()
        for ts in self.layers:
            for t in ts:
                t.free()
        self.router.free()
        self.cache.free()
        self.lm.free()


@pytest.fixture(scope="module")
def small(omega, oracle):
    m = oracle.Model(model_config(2, 8192), seed=2026, sigma=0.02, norm_sigma=0.1, threads=16)
    g = GpuModel(omega, m, 256)
    yield m, g
    g.free()


def run_both(oracle, m, g, prompt, new_tokens, max_pos=256, log=None):
    """Steps the graph and the oracle engine side by side. Returns the tokens, the per-step top-2
    logit margins, the worst logit error over the steps whose history has identical routing,
    and the steps where a layer routed differently (with the oracle's rank-8/9 margin there)."""
    eng = oracle.Engine(m, max_pos, refined_router=True, threads=16)
    toks, margins, flips = [], [], []
    tok = prompt[0]
    pos = 0
    seq = list(prompt)
    worst = 0.0
    diverged = False
    while pos < len(prompt) + new_tokens - 1:
        gt, st = g.graph.token(g.x_embed(tok), pos)
        hidden = eng.step(tok)
        logits = eng.logits(hidden)
        want = oracle.argmax(logits)
        _, _, gl = g.graph.read(logits=True)
        g_ids, g_w = g.graph.read_routes()
        o_ids, o_w, o_margin = eng.last_routes()
        same = np.array_equal(g_ids, o_ids)
        if not same:
            bad = [l for l in range(m.cfg.layers) if not np.array_equal(g_ids[l], o_ids[l])]
            flips.append((pos, bad, [float(o_margin[l]) for l in bad]))
            diverged = True
        err = rel_err(gl, logits)
        if not diverged:
            worst = max(worst, err)
        top2 = np.sort(logits)[-2:]
        margins.append(float(top2[1] - top2[0]))
        if log is not None:
            log.append((pos, gt, want, err, margins[-1], float(o_margin.min()), same))
        assert gt == want, (pos, gt, want, margins[-1])
        pos += 1
        tok = seq[pos] if pos < len(prompt) else gt
        if pos >= len(prompt):
            seq.append(gt)
        toks.append(gt)
        # one submission per token: the persistent launch + the lm_head, or the six-launch chain
        assert st.launches in (2, 6 * m.cfg.layers + 1) and st.submits == 1
    return toks, margins, worst, flips


def test_greedy_tokens_match_the_oracle(omega, oracle, small):
    m, g = small
    prompt = [5, 1000, 77, 4096, 8191, 3]
    log = []
    toks, margins, worst, flips = run_both(oracle, m, g, prompt, 40, log=log)
    for row in log:
        print("pos %3d tok %5d/%5d err %.2e top2 %.4f route-margin %.2e same %s" % row)
    # the first layer that ever routes differently must be at a near tie of its rank-8 / rank-9
    # logits; after it the two KV histories differ, so later differences are consequences
    if flips:
        pos, layers, mg = flips[0]
        assert mg[0] < 1e-3, (pos, layers, mg)
    assert worst <= TOL, worst
    print(f"min top-2 margin {min(margins):.4f}, worst logit rel err {worst:.2e}, flips {flips}")


def test_eager_submission_is_bit_identical_to_the_graph(omega, oracle, small):
    m, g = small
    outs = []
    for flush in (False, True):
        g.graph.set_flush_each(flush)
        toks = []
        for pos, t in enumerate([11, 12, 13, 14]):
            toks.append(g.graph.token(g.x_embed(t), pos)[0])
        outs.append((toks, g.graph.read(x=True, hidden=True, logits=True)))
    g.graph.set_flush_each(False)
    assert outs[0][0] == outs[1][0]
    for a, b in zip(outs[0][1], outs[1][1]):
        np.testing.assert_array_equal(a, b)


def test_stamps_time_every_launch(omega, small):
    m, g = small
    g.graph.set_stamps(True)
    g.graph.token(g.x_embed(9), 0)
    st, kinds = g.graph.stamps()
    ns = g.graph.kernel_ns()
    g.graph.set_stamps(False)
    # every launch's own duration, inside the token's span
    assert len(ns) == len(kinds) and (ns > 0).all() and ns.sum() <= st[-1]
    assert len(kinds) == 6 * m.cfg.layers + 1
    assert (np.diff(st.astype(np.int64)) >= 0).all()
    names = [omega.kind_name(int(k)) for k in kinds[:6]]
    # the attention merges its splits in the same launch
    assert names == ["qkv", "attn", "o_proj", "router", "gate_up", "down"]
    assert omega.kind_name(int(kinds[-1])) == "lm_head"


@pytest.mark.parametrize("mutant", [1, 2, 3])
def test_graph_mutants_are_caught(omega, oracle, small, mutant):
    # crates/aien-omega-dgraph/src/lib.rs:469-480
    m, g = small
    eng = oracle.Engine(m, 256, refined_router=True, threads=16)
    g.graph.test_set_mutant(mutant)
    try:
        worst = 0.0
        for pos, t in enumerate([21, 22, 23]):
            g.graph.token(g.x_embed(t), pos)
            want = eng.logits(eng.step(t))
            worst = max(worst, rel_err(g.graph.read(logits=True)[2], want))
    finally:
        g.graph.test_set_mutant(0)
    assert worst > 0.01


def test_chain_merge_wait_that_runs_out_is_reported_and_the_next_token_recovers(omega, small):
    # test mutant 9 on the chain: every attention split merge gives up at once (no poll); the token
    # reports CHIP_FAIL with the count, the flags are cleared and the epochs restart, and the
    # same positions run again give the bits they gave before the failure
    m, g = small
    graph = g.graph
    rng = np.random.default_rng(31)
    toks = [int(t) for t in rng.integers(0, m.cfg.vocab, 12)]
    before = []
    for pos, tok in enumerate(toks):
        graph.token(g.x_embed(tok), pos)
        if pos >= 10:
            before.append(graph.read(x=True, logits=True))
    graph.test_set_mutant(9)
    try:
        with pytest.raises(omega.OmegaGpuError, match=r"waits ran out \(chain form\)"):
            graph.token(g.x_embed(toks[11]), 11)
    finally:
        graph.test_set_mutant(0)
    for i, pos in enumerate((10, 11)):
        graph.token(g.x_embed(toks[pos]), pos)
        x, _, lg = graph.read(x=True, logits=True)
        np.testing.assert_array_equal(x.view(np.uint32), before[i][0].view(np.uint32))
        np.testing.assert_array_equal(lg.view(np.uint32), before[i][2].view(np.uint32))


def test_routes_match_per_layer(omega, oracle, small):
    # the router's device state after a token holds the last layer's routing
    m, g = small
    eng = oracle.Engine(m, 256, refined_router=True, threads=16)
    for pos, t in enumerate([31, 32, 33, 34, 35]):
        g.graph.token(g.x_embed(t), pos)
        eng.step(t)
    ids, w, margins = eng.last_routes()
    xout, tab_gu, _ = g.router.read_back()
    last = m.cfg.layers - 1
    gu_entries = np.array([g.layers[last][2].entry(int(e)) for e in ids[last]], np.uint64)
    np.testing.assert_array_equal(tab_gu.reshape(8, 2), gu_entries)
    x_gpu = g.graph.read(x=True)[0]
    assert rel_err(x_gpu, eng.last_x()) <= TOL


def test_token_id_gathers_the_embedding_on_the_device(omega, oracle, small):
    m, g = small
    c = m.cfg
    emb = omega.Bf16Tensor.upload(c.vocab, c.hidden, m.embed())
    g.graph.set_embedding(emb)
    seq = [41, 42, c.vocab + 5, 44]          # ids past the vocabulary wrap (embed_row)
    outs = []
    for use_id in (False, True):
        toks, logits = [], []
        for pos, t in enumerate(seq):
            r = g.graph.token_id(t, pos) if use_id else g.graph.token(g.x_embed(t), pos)
            toks.append(r[0])
            logits.append(g.graph.read(logits=True)[2])
        outs.append((toks, logits))
    assert outs[0][0] == outs[1][0]
    for a, b in zip(outs[0][1], outs[1][1]):
        np.testing.assert_array_equal(a, b)
    # the device generator's embedding equals the oracle model's (same seed, tensor id 1)
    emb2 = omega.Bf16Tensor.synth(c.vocab, c.hidden, 2026, 1, 0.02)
    g.graph.set_embedding(emb2)
    for pos, t in enumerate(seq):
        assert g.graph.token_id(t, pos)[0] == outs[0][0][pos]
    g.graph.set_embedding(emb)
    emb2.free()


def test_argmax_ties_go_to_the_lowest_index(omega, oracle):
    """The graph's greedy token is the lowest index of the maximum (crates/aien-omega-dgraph/src/
    lib.rs:347-349, sample_argmax tensor.rs:299-318). Four lm_head rows (3, 100, 5000, 8000) are
    the same bf16 vector u = bf16(0.05 h), h the oracle's final hidden of the first step, so their
    logits are exactly tied and far above every other row (u . h is about 0.05 |h|^2, the other
    logits are about N(0, 1)); two rows hold -u. Identical rows give bit-identical logits on the
    device (a row's arithmetic does not depend on where it sits), so the token must be 3."""
    m = oracle.Model(model_config(2, 8192), seed=77, sigma=0.02, norm_sigma=0.1, threads=16)
    eng = oracle.Engine(m, 256, refined_router=True, threads=16)
    h0 = eng.step(11)
    lm = m.lm_head()  # a writable view of the oracle model's buffer, uploaded below
    u = oracle.f32_to_bf16((0.05 * h0).astype(np.float32))
    for r in (3, 100, 5000, 8000):
        lm[r] = u
    for r in (5, 9):
        lm[r] = u ^ np.uint16(0x8000)
    want_logits = eng.logits(h0)
    assert oracle.argmax(want_logits) == 3
    g = GpuModel(omega, m, 256)
    try:
        tok, _ = g.graph.token(g.x_embed(11), 0)
        _, _, logits = g.graph.read(logits=True)
        tied = logits[[3, 100, 5000, 8000]]
        assert (tied == tied[0]).all(), tied
        assert logits.max() == tied[0] and np.flatnonzero(logits == logits.max())[0] == 3
        assert tok == 3, tok
        assert rel_err(logits, want_logits) <= TOL
    finally:
        g.free()
