"""The decode graph's persistent form (every layer in one launch) against its six-launch chain.

Both forms compute every value with the same lane split, reduction order and rounding, so the
bar is bit identity: greedy token, logits, final residual, final hidden, every layer's routed ids
and weights, and the router's device state, token by token, on two independent models (each form
writes its own KV cache). Positions run past 1024 so the splits take two pages each (both forms cut
a kv head's pages into at most 64 splits). The oracle comparison of the persistent
form rests on these tests: they pin the two forms to each
other, the stage stamps, and the failure path of its bounded waits; test_gpu_graph.py runs the
default form (the chain) against the oracle.
Reference: crates/aien-omega-dgraph/src/lib.rs:16-30 (one submission per token).
"""
import numpy as np
import pytest

from test_gpu_graph import GpuModel, model_config, rel_err

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def pair(omega, oracle):
    m = oracle.Model(model_config(2, 8192), seed=2027, sigma=0.02, norm_sigma=0.1, threads=16)
    a = GpuModel(omega, m, 1280)
    b = GpuModel(omega, m, 1280)
    if not a.graph.set_persistent(True):
        a.free()
        b.free()
        pytest.skip("this device cannot hold the persistent launch")
    assert b.graph.set_persistent(False) is False
    emb = omega.Bf16Tensor.upload(m.cfg.vocab, m.cfg.hidden, m.embed())
    a.graph.set_embedding(emb)
    b.graph.set_embedding(emb)
    yield m, a, b
    a.free()
    b.free()
    emb.free()


def step_both(a, b, tok, pos):
    ta, sa = a.graph.token_id(tok, pos)
    tb, sb = b.graph.token_id(tok, pos)
    assert sa.launches == 2 and sb.launches == 6 * a.m.cfg.layers + 1
    ra = a.graph.read(x=True, hidden=True, logits=True)
    rb = b.graph.read(x=True, hidden=True, logits=True)
    return ta, tb, ra, rb


def assert_same(a, b, ta, tb, ra, rb, pos):
    assert ta == tb, (pos, ta, tb)
    for name, u, v in zip(("x", "hidden", "logits"), ra, rb):
        assert np.array_equal(u.view(np.uint32), v.view(np.uint32)), (pos, name, rel_err(u, v))
    ia, wa = a.graph.read_routes()
    ib, wb = b.graph.read_routes()
    np.testing.assert_array_equal(ia, ib)
    np.testing.assert_array_equal(wa.view(np.uint32), wb.view(np.uint32))


def test_persistent_is_bit_identical_to_the_chain(pair):
    m, a, b = pair
    rng = np.random.default_rng(5)
    prompt = [int(t) for t in rng.integers(0, m.cfg.vocab, 24)]
    tok = prompt[0]
    for pos in range(40):
        ta, tb, ra, rb = step_both(a, b, tok, pos)
        assert_same(a, b, ta, tb, ra, rb, pos)
        tok = prompt[pos + 1] if pos + 1 < len(prompt) else ta
    # the router's device state after the token: the last layer's x' and route (the group
    # tables hold each model's own expert addresses)
    xa, tga, tda = a.router.read_back()
    xb, tgb, tdb = b.router.read_back()
    np.testing.assert_array_equal(xa.view(np.uint32), xb.view(np.uint32))
    last = m.cfg.layers - 1
    ids = a.graph.read_routes()[0][last]
    for g, tg, td in ((a, tga, tda), (b, tgb, tdb)):
        np.testing.assert_array_equal(tg.reshape(8, 2), [g.layers[last][2].entry(int(e)) for e in ids])
        np.testing.assert_array_equal(td.reshape(8, 2), [g.layers[last][3].entry(int(e)) for e in ids])


def test_persistent_long_context_matches_the_chain(pair):
    # positions 40..1100: from 1025 on a kv head's 65..69 pages take two per split
    m, a, b = pair
    rng = np.random.default_rng(6)
    toks = [int(t) for t in rng.integers(0, m.cfg.vocab, 1100)]
    for pos in range(40, 1100):
        ta, tb, ra, rb = step_both(a, b, toks[pos], pos)
        if pos % 37 == 0 or pos in (511, 512, 513, 1023, 1024, 1025, 1040, 1041, 1099):
            assert_same(a, b, ta, tb, ra, rb, pos)
        else:
            assert ta == tb, pos


def test_stage_stamps_are_ordered(pair):
    m, a, b = pair
    a.graph.set_stage_stamps(True)
    try:
        ta, tb, ra, rb = step_both(a, b, 7, 1100)
        ns = a.graph.stage_ns()
    finally:
        a.graph.set_stage_stamps(False)
    assert_same(a, b, ta, tb, ra, rb, 1100)
    assert ns.shape == (m.cfg.layers, 5)
    flat = ns.reshape(-1).astype(np.int64)
    assert (np.diff(flat) >= 0).all() and flat[-1] > 0, ns
    print("stage ns per layer:", ns.tolist())


def test_a_wait_that_runs_out_is_reported_and_the_next_token_recovers(omega, pair):
    # test mutant 9: every wait that is not already satisfied gives up at once; each gives up by
    # counting and setting the abort word, so the launch ends and the token is reported failed
    m, a, b = pair
    a.graph.test_set_mutant(9)
    try:
        with pytest.raises(omega.OmegaGpuError) as e:
            a.graph.token_id(11, 1101)
        assert "waits ran out" in str(e.value)
    finally:
        a.graph.test_set_mutant(0)
    # the same position again, now complete: bit-identical to the chain at that position
    ta, tb, ra, rb = step_both(a, b, 11, 1101)
    assert_same(a, b, ta, tb, ra, rb, 1101)
    ta, tb, ra, rb = step_both(a, b, ta, 1102)
    assert_same(a, b, ta, tb, ra, rb, 1102)
