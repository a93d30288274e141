"""GPU tests of the beat scheduler (omega_amd.serve): many conversations over one batched decode.

The model is the 2-layer real-shape Qwen3-30B-A3B of test_gpu_batch (vocabulary 8192). Bars: each
request's generated tokens equal the oracle engine's greedy tokens for its prompt and the tokens
the same request gets alone through the scheduler, bit for bit, with requests joining at
different beats, leaving at different lengths and waiting while every slot is taken; a stop
token ends a request after it is emitted; a cancelled request leaves at the next beat; every page
comes back to the free list."""
import numpy as np
import pytest

from test_gpu_batch import SEED, BatchModel, model_config

pytestmark = pytest.mark.gpu
BLOCKS, MAX_BLOCKS = 256, 8


@pytest.fixture(scope="module")
def served(omega, oracle):
    m = oracle.Model(model_config(2, 8192), seed=SEED, sigma=0.02, norm_sigma=0.1, threads=16)
    bm = BatchModel(omega, oracle, m, max_seqs=8, blocks=BLOCKS, max_blocks=MAX_BLOCKS)
    yield m, bm
    bm.free()


def scheduler(bm, slots):
    from omega_amd import serve
    return serve.BeatScheduler(bm.bd, BLOCKS, MAX_BLOCKS, slots=slots)


def oracle_greedy(oracle, m, prompt, n):
    eng = oracle.Engine(m, 256, refined_router=True, threads=16)
    for t in prompt:
        h = eng.step(t)
    out = []
    for _ in range(n):
        out.append(int(oracle.argmax(eng.logits(h))))
        h = eng.step(out[-1])
    return out


def test_staggered_requests_match_the_oracle_and_their_solo_runs(oracle, served):
    m, bm = served
    rng = np.random.default_rng(11)
    reqs = {k: (list(rng.integers(0, 8192, n)), new) for k, (n, new) in
            {"a": (5, 10), "b": (20, 6), "c": (3, 12), "d": (9, 4), "e": (14, 7), "f": (1, 9)}.items()}
    arrivals = {0: [("a", *reqs["a"], ()), ("b", *reqs["b"], ())], 4: [("c", *reqs["c"], ())],
                7: [("d", *reqs["d"], ()), ("e", *reqs["e"], ()), ("f", *reqs["f"], ())]}
    sch = scheduler(bm, slots=4)                      # "f" waits for a free slot
    got = sch.run(arrivals)
    assert len(sch.free_pages) == BLOCKS
    assert got["f"].joined_beat > 7
    for k, (prompt, new) in reqs.items():
        r = got[k]
        assert r.finish == "length" and len(r.tokens) == new
        assert r.tokens == oracle_greedy(oracle, m, prompt, new), k
        solo = scheduler(bm, slots=1).run({0: [(k, prompt, new, ())]})[k]
        assert solo.tokens == r.tokens, k


def test_stop_cancel_and_refusals(omega, served):
    from omega_amd import serve
    m, bm = served
    prompt = [7, 300, 4000, 12]
    alone = scheduler(bm, 1).run({0: [("x", prompt, 8, ())]})["x"].tokens
    j = alone.index(alone[2])                         # the first occurrence of the third token
    r = scheduler(bm, 1).run({0: [("x", prompt, 8, (alone[2],))]})["x"]
    assert r.finish == "stop" and r.tokens == alone[:j + 1]
    sch = scheduler(bm, 2)
    a = sch.submit(prompt, 20)
    b = sch.submit([1, 2, 3], 20)
    with pytest.raises(serve.SchedulerBusy):
        sch.submit([5], 3)                            # both slots taken
    with pytest.raises(omega.OmegaGpuError):
        scheduler(bm, 2).submit(list(range(100)), 40)  # 140 positions > 8 pages of 16
    for _ in range(6):
        sch.beat()
    sch.cancel(a)
    sch.beat()
    assert a.finish == "cancelled" and not a.pages
    while sch.live:
        sch.beat()
    assert b.finish == "length" and len(b.tokens) == 20
    assert len(sch.free_pages) == BLOCKS


@pytest.fixture(scope="module")
def prefill_join(omega, oracle, served):
    from omega_amd import prefill as pf
    from omega_amd import serve
    m, bm = served
    c = m.cfg
    layers = [dict(qkv=q, o=o, gate_up=g, down=d, input_norm=m.tensor(l, 5), post_norm=m.tensor(l, 6),
                   router=oracle.bf16_to_f32(m.tensor(l, 4))) for l, (q, o, g, d) in enumerate(bm.tensors)]
    cache = omega.DecodeAttnCache(c.layers, 256, c.rope_theta)
    for l in range(c.layers):
        cache.set_norms(l, m.tensor(l, 7), m.tensor(l, 8))
    emb = m.embed()
    wp = pf.WholePromptPrefill(layers, m.final_norm(), lambda t: oracle.bf16_to_f32(emb[t]), cache, c.eps)
    pp = serve.PromptPrefill(wp, cache, bm.pool.ptr, 128, min_tokens=4)
    yield pp
    pp.free()
    wp.free()
    cache.free()


def test_whole_prompt_joins(omega, oracle, served, prefill_join):
    from omega_amd import serve
    m, bm = served
    rng = np.random.default_rng(12)
    reqs = {k: (list(rng.integers(0, 8192, n)), new) for k, (n, new) in
            {"a": (37, 6), "b": (3, 8), "c": (20, 5), "d": (64, 4)}.items()}   # "b" is fed per beat
    arrivals = {0: [("a", *reqs["a"], ()), ("b", *reqs["b"], ())], 3: [("c", *reqs["c"], ()), ("d", *reqs["d"], ())]}
    got = serve.BeatScheduler(bm.bd, BLOCKS, MAX_BLOCKS, slots=4, prefill=prefill_join).run(arrivals)
    for k, (prompt, new) in reqs.items():
        r = got[k]
        assert r.finish == "length" and len(r.tokens) == new
        solo = serve.BeatScheduler(bm.bd, BLOCKS, MAX_BLOCKS, slots=1, prefill=prefill_join).run(
            {0: [(k, prompt, new, ())]})[k]
        assert solo.tokens == r.tokens, k
    # the joined generation against the oracle engine: the prompt's K / V rows as the prefill
    # left them (the payload the join copied into the request's pages) written into the oracle's
    # cache, then the last prompt token at position n - 1 and greedy steps (pins the position and
    # token of the last prompt step and the page order; the rows themselves are pinned against the
    # W8A8 oracle stage by stage in test_gpu_prefill)
    c = m.cfg
    geo = oracle.PoolBlockGeometry(c.layers, c.kv_heads, c.head_dim, 16)
    for k in ("a", "c", "d"):
        prompt, new = reqs[k]
        n = len(prompt)
        prefill_join.wp.run(prompt[:-1], 0)
        payload, _ = prefill_join.cache.export_kv(0, n - 1)
        eng = oracle.Engine(m, 256, refined_router=True, threads=16)
        oracle.kv_blocks_to_rows(geo, 0, n - 1, payload,
                                 lambda layer, head, kr, vr: eng.write_kv_rows(layer, head, 0, kr, vr))
        eng.seek(n - 1)
        h = eng.step(prompt[-1])
        want = []
        for _ in range(new):
            want.append(int(oracle.argmax(eng.logits(h))))
            h = eng.step(want[-1])
        assert got[k].tokens == want, k
    # the pages of a whole-prompt join hold the fused cache's rows byte for byte
    prompt = reqs["d"][0]
    sch = serve.BeatScheduler(bm.bd, BLOCKS, MAX_BLOCKS, slots=1, prefill=prefill_join)
    r = sch.submit(prompt, 4)
    sch.beat()                                        # the join runs the prefill, then one step
    want, _ = prefill_join.cache.export_kv(0, len(prompt) - 1)
    bb = prefill_join.block_bytes
    pool = bm.pool.download(np.uint8, BLOCKS * bb)
    for j in range(len(want) // bb - 1):              # whole pages (the last one now holds the step's row)
        np.testing.assert_array_equal(pool[r.pages[j] * bb:(r.pages[j] + 1) * bb], want[j * bb:(j + 1) * bb])
    while sch.live:
        sch.beat()
