"""Configuration 4 at its stated size on the GPU, against the CPU oracle's recorded decode.

The full 48-layer, vocab-151936 random-init Qwen3-30B-A3B FP8 model (the tensors the oracle's
generator makes, synthesised on the device), the seeded 512-token prompt through the decode
graph one token per step, then 64 greedy tokens: the workload bench.py times. The expected
values are tests/golden/config4_greedy.npz, written by tests/golden/make_config4.py from the
oracle engine (oref_engine_step: qwen3_moe_omega.rs:4096-4345 restated).

The device and the oracle sum their f32 products in different orders, so their rows differ by
about 1e-6 relative; K and V are stored as bf16 (the reference's KV format), and now and then an
element lands on the other side of a bf16 rounding boundary, a whole bf16 step (2^-8) apart. The
first such V element (layer 5 of the first token here) moves the residual by about 1e-4, and from
there the two runs' router logits differ by up to about 1e-3 in the deeper layers (measured:
1e-6 through layer 4, 2e-4 at layer 8, 1.4e-3 at layer 20), so a layer whose consecutive routing
ranks sit closer than that can order or pick its experts differently, and from there the two
histories are different computations. Hence two tests:

1. Free-running, the reference's own full-size bar (own30b_check,
   crates/aien-inference-abi/src/bin/own30b_check.rs:181-193, 986-1006): the 512 prompt tokens
   and 64 greedy tokens with nothing forced; every generated token equals the oracle's, or the
   first divergence sits at an oracle top-2 margin below the 1e-3 floor. Up to the first token
   at which any layer routes to another expert set than the oracle (the two histories are the
   same computation until then; here that is processed token 4), the prompt positions' logits
   are held to test 2's prompt bar. (The random-init model's greedy stream repeats a few ids;
   test 2's 512 prompt positions each read a different context.)
2. Routing forced only near ties: at every processed token, each layer whose oracle
   consecutive-rank gap of the top 9 (rank-8 / rank-9 logit margin and ln(w_k / w_k+1) inside the
   top 8) is below 1e-2, ten times the measured drift, takes the oracle's expert ids (teacher
   forcing through omega_gpu_decode_graph_test_force_routes; the weights stay the device's own
   softmax over that set); every other layer ranks its own logits and must route exactly as the
   oracle did (ids bit-exact in slot order, every layer of all 575 processed tokens). Both runs
   then compute the same function over the same history: all 64 greedy tokens identical (a
   divergence passes only at an oracle top-2 margin below 1e-3), logits within 2e-3 relative (max
   |gpu - cpu| over max |cpu|) at 1024 seeded vocabulary indices plus the oracle's top 16 at every
   step and over the whole vocabulary at the first generated step, top-2 margins within 2 x 2e-3
   of max |logit|. The logits of all 512 prompt positions (each a different context) are held to
   the same bar at 256 seeded indices and the oracle's top 16, except positions 0..3 at 4e-3: they
   attend over at most four bf16 V rows, so one rounding flip weighs up to a quarter of the
   attention output (measured 2.8e-3 at position 0, 1.8e-3 at most from position 4, 8.2e-4 from
   64). A prompt position's argmax may differ from the oracle's only where the oracle's top-2
   margin is within twice the measured absolute error of the top 16 (the most that error can
   move a margin).
"""
import os

import numpy as np
import pytest

pytestmark = pytest.mark.gpu
TOL = 2e-3
NEAR_TIE = 1e-3        # the reference's top-2 margin floor
ROUTE_NEAR = 1e-2      # routing gaps forced in test 2: ten times the measured drift
FIXTURE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "config4_greedy.npz")


def rel_err(a, e):
    return float(np.abs(a - e).max() / max(np.abs(e).max(), 1e-30))


def top2(logits):
    o = np.argsort(-logits, kind="stable")
    return int(o[0]), float(logits[o[0]] - logits[o[1]])


@pytest.fixture(scope="module")
def golden():
    z = np.load(FIXTURE)  # numpy arrays only (allow_pickle off)
    return {k: z[k] for k in z.files}


@pytest.fixture(scope="module")
def model(omega, golden):
    m = omega.SynthDecodeModel(int(golden["seed"]), omega.round_max_pos(len(golden["prompt"]) + 72))
    yield m
    m.free()


class StepCheck:
    """The bars of one generated step against the fixture."""

    def __init__(self, golden):
        self.z = golden
        self.worst = 0.0
        self.worst_margin = 0.0
        self.compared = 0

    def check(self, s, tok, logits):
        z = self.z
        got_tok, got_margin = top2(logits)
        assert got_tok == tok, (s, got_tok, tok)  # the graph's argmax is the lowest index of the max
        e = max(rel_err(logits[z["subset"]], z["sub_val"][s]),
                rel_err(logits[z["top_idx"][s]], z["top_val"][s]))
        if s == 0:
            e = max(e, rel_err(logits, z["first_logits"]))
        self.worst = max(self.worst, e)
        scale = float(np.abs(z["sub_val"][s]).max())
        self.worst_margin = max(self.worst_margin, abs(got_margin - float(z["margins"][s])) / scale)
        assert e <= TOL, f"step {s}: logits rel err {e:.2e}"
        assert self.worst_margin <= 2 * TOL, f"step {s}: top-2 margin off by {self.worst_margin:.2e} of max |logit|"
        if tok != int(z["tokens"][s]):
            m = float(z["margins"][s])
            assert m < NEAR_TIE, (f"greedy token {s} is {tok}, oracle {int(z['tokens'][s])} at oracle "
                                  f"top-2 margin {m:.4f} (>= {NEAR_TIE})")
            return False
        self.compared += 1
        return True


def prompt_bar(t):
    return 4e-3 if t < 4 else TOL


def check_prompt_position(golden, t, logits):
    """Prompt position t's logits against the fixture: 256 seeded indices and the oracle's top 16
    within prompt_bar(t); the argmax equal unless the oracle's top-2 margin is within twice the
    measured absolute error of the top 16. Returns the relative error."""
    ti, tv = golden["prompt_top_idx"][t], golden["prompt_top_val"][t]
    e = max(rel_err(logits[golden["prompt_subset"]], golden["prompt_sub_val"][t]), rel_err(logits[ti], tv))
    assert e <= prompt_bar(t), f"prompt position {t}: logits rel err {e:.2e}"
    top, want = int(np.argmax(logits)), int(golden["prompt_top1"][t])
    if top != want:
        abs_err = float(np.abs(logits[ti] - tv).max())
        m = float(golden["prompt_margin"][t])
        assert m <= 2 * abs_err, (f"prompt position {t}: argmax {top}, oracle {want} at margin {m:.2e} "
                                  f"(measured abs error {abs_err:.2e})")
    return e


def decode(g, golden, forced, on_step):
    """The 512 prompt tokens, then the first 63 generated tokens, one decode step each (575
    processed tokens); on_step(t, tok) after processed token t with the greedy token it produced
    (generated step t - 511 from t = 511 on) returns whether to go on."""
    prompt, routes = golden["prompt"], golden["step_routes"].astype(np.uint32)
    n_gen = len(golden["tokens"])
    pos, tok = 0, None
    steps = len(prompt) + n_gen - 1
    for t in range(steps):
        if forced:
            g.force_routes(routes[t])
        tok_in = int(prompt[t]) if t < len(prompt) else tok
        tok, _ = g.token_id(tok_in, pos)
        pos += 1
        if not on_step(t, tok):
            return


def test_config4_routes_match_except_at_near_ties(omega, golden, model):
    g = model.graph
    chk = StepCheck(golden)
    npr = len(golden["prompt"])
    n_gen = len(golden["tokens"])
    routes = golden["step_routes"].astype(np.uint32)
    near = golden["step_gap"] < ROUTE_NEAR                  # [steps][layers]
    state = {"diverged": None, "ranked": 0, "forced": int(near.sum()), "prompt_worst": 0.0}
    prompt = golden["prompt"]
    pos, tok = 0, None
    try:
        for t in range(npr + n_gen - 1):
            sel = routes[t].copy()
            sel[~near[t], 0] = omega.DGRAPH_RANK                 # these layers rank their own logits
            g.force_routes(sel)
            tok_in = int(prompt[t]) if t < npr else tok
            tok, _ = g.token_id(tok_in, pos)
            pos += 1
            ids, _ = g.read_routes()
            for l in np.flatnonzero(~near[t]):
                assert ids[l].tolist() == routes[t, l].tolist(), \
                    f"step {t} layer {l}: routed {ids[l].tolist()}, oracle {routes[t, l].tolist()} " \
                    f"(oracle gap {float(golden['step_gap'][t, l]):.2e})"
                state["ranked"] += 1
            if t < npr:
                _, _, logits = g.read(logits=True)
                state["prompt_worst"] = max(state["prompt_worst"], check_prompt_position(golden, t, logits))
            if t >= npr - 1:
                s = t - (npr - 1)
                _, _, logits = g.read(logits=True)
                if not chk.check(s, tok, logits):
                    state["diverged"] = s
                    break
    finally:
        g.force_routes(None)
    print(f"routing forced at {state['forced']} near-tie (step, layer) points, {state['ranked']} ranked "
          f"by the device and equal to the oracle; prompt logits rel err <= {state['prompt_worst']:.2e} "
          f"over {npr} positions; {chk.compared} of {n_gen} greedy tokens identical "
          f"(divergence at {state['diverged']}), logits rel err <= {chk.worst:.2e}, margins within "
          f"{chk.worst_margin:.2e} of max |logit|")
    assert state["diverged"] is not None or chk.compared == n_gen


def test_config4_free_running_greedy_tokens(omega, golden, model):
    g = model.graph
    g.force_routes(None)
    npr, n_gen = len(golden["prompt"]), len(golden["tokens"])
    routes = golden["step_routes"].astype(np.uint32)
    state = {"diverged": None, "worst": 0.0, "route_apart": None, "prompt_worst": 0.0, "prompt_checked": 0}
    got = []

    def on_step(t, tok):
        ids, _ = g.read_routes()
        # the expert sets (an order swap inside the top 8 only reorders the combine's sum)
        if state["route_apart"] is None and not np.array_equal(np.sort(ids, axis=1), np.sort(routes[t], axis=1)):
            state["route_apart"] = t
        if t < npr and state["route_apart"] is None:
            # the same history so far: this prompt position's logits on the prompt bar
            _, _, logits = g.read(logits=True)
            state["prompt_worst"] = max(state["prompt_worst"], check_prompt_position(golden, t, logits))
            state["prompt_checked"] += 1
        if t < npr - 1:
            return True
        s = t - (npr - 1)
        got.append(tok)
        _, _, logits = g.read(logits=True)
        e = rel_err(logits[golden["subset"]], golden["sub_val"][s])
        state["worst"] = max(state["worst"], e)
        if state["route_apart"] is None:
            assert e <= TOL, f"generated step {s}: logits rel err {e:.2e}"
        if tok != int(golden["tokens"][s]):
            m = float(golden["margins"][s])
            assert m < NEAR_TIE, (f"greedy token {s} is {tok}, oracle {int(golden['tokens'][s])} at oracle "
                                  f"top-2 margin {m:.4f} (>= {NEAR_TIE})")
            state["diverged"] = s
            return False
        return True

    decode(g, golden, False, on_step)
    print(f"free-running: routing first apart at processed token {state['route_apart']}; "
          f"{state['prompt_checked']} prompt positions on the logit bar (rel err <= "
          f"{state['prompt_worst']:.2e}); {len(got) - (state['diverged'] is not None)} of {n_gen} greedy "
          f"tokens identical (divergence at {state['diverged']}); generated logits rel err <= "
          f"{state['worst']:.2e}")
    assert state["diverged"] is not None or len(got) == n_gen
