"""Writes tests/golden/config4_greedy.npz: the CPU oracle's greedy decode of configuration 4.

Configuration 4: the full 48-layer random-init Qwen3-30B-A3B FP8 model
(hidden 2048, 32 q / 4 kv heads of 128, 128 experts top-8 with intermediate 768, vocab 151936,
RMSNorm eps 1e-6, RoPE theta 1e6, norm weights 1.0, FP8 projections N(0, 0.02) block-quantised,
bf16 embedding and lm_head N(0, 0.02)), the seeded 512-token prompt, then 64 greedy tokens.
Weights come from the oracle's counter-based generator with seed 20261201 and the tensor ids
1000 + 16 * layer + kind (the device generator makes the same values), the prompt from
numpy.random.default_rng(20261201).integers(0, 151936, 512): the workload bench.py times.

The oracle engine (oracle/oracle.c oref_engine_step: qwen3_moe_omega.rs:4096-4345 restated, the
refined f64 router) runs every prompt token and every generated token one step at a time; the
first generated token is the argmax after the last prompt token. Recorded per generated step:
the token, the top-2 margin (own30b_check.rs:181-193), the top 16 (index, value) pairs, the
logits at 1024 seeded vocabulary indices, the smallest rank-8 / rank-9 routing margin over the
48 layers and its layer; plus the full logits of the first generated step. Recorded at every
prompt position too (each reads a different context, so the stream is not a greedy repetition):
the argmax, the top-2 margin, the top 16 (index, value) pairs and the logits at 256 of the seeded
indices (every fourth). Recorded per processed
token (the 512 prompt tokens, then the first 63 generated ones), per layer: the routed expert ids
in slot order and the smallest logit gap between consecutive ranks of the top 9 (the rank-8 /
rank-9 margin, and ln(w_k / w_k+1) inside the top 8), which bounds how close the routing was to
changing. About 15 minutes on 8 host threads and 32 GB of memory.

Run from the repository root:  python tests/golden/make_config4.py [--threads 8]
"""
import argparse
import os
import sys
import time

import numpy as np

REPO = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, os.path.join(REPO, "oracle"))

import pyoracle as orc  # noqa: E402

SEED = 20261201
L, H, QH, KVH, HD, E, TOPK, I, V = 48, 2048, 32, 4, 128, 128, 8, 768, 151936
PROMPT, NEW = 512, 64
SUBSET = 1024


def route_record(eng):
    """(ids uint8 [48][8], smallest consecutive-rank gap of the top 9 per layer)"""
    ids, w, m89 = eng.last_routes()
    with np.errstate(divide="ignore"):
        inner = np.log(w[:, :-1].astype(np.float64) / w[:, 1:].astype(np.float64)).min(axis=1)
    return ids.astype(np.uint8), np.minimum(inner, m89.astype(np.float64)).astype(np.float32)


def top2(logits):
    order = np.argsort(-logits, kind="stable")
    return int(order[0]), float(logits[order[0]] - logits[order[1]]), order[:16]


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--threads", type=int, default=os.cpu_count() or 1)
    ap.add_argument("--out", default=os.path.join(REPO, "tests", "golden", "config4_greedy.npz"))
    args = ap.parse_args()
    cfg = dict(layers=L, hidden=H, q_heads=QH, kv_heads=KVH, head_dim=HD, experts=E, top_k=TOPK,
               inter=I, vocab=V, eps=1e-6, rope_theta=1e6)
    t0 = time.time()
    model = orc.Model(cfg, SEED, sigma=0.02, norm_sigma=0.0, threads=args.threads)
    print(f"model synthesised in {time.time() - t0:.0f} s", flush=True)
    eng = orc.Engine(model, 1024, refined_router=True, threads=args.threads)
    prompt = np.random.default_rng(SEED).integers(0, V, PROMPT)
    subset = np.sort(np.random.default_rng(SEED + 1).choice(V, SUBSET, replace=False)).astype(np.int64)
    prompt_margin = np.empty((PROMPT, L), np.float32)
    steps = PROMPT + NEW - 1
    step_routes = np.zeros((steps, L, TOPK), np.uint8)
    step_gap = np.zeros((steps, L), np.float32)
    psub = subset[::4]
    p_top1 = np.empty(PROMPT, np.int64)
    p_margin = np.empty(PROMPT, np.float32)
    p_top_idx = np.empty((PROMPT, 16), np.int64)
    p_top_val = np.empty((PROMPT, 16), np.float32)
    p_sub_val = np.empty((PROMPT, psub.size), np.float32)
    t1 = time.time()
    hidden = None
    for p, tok in enumerate(prompt.tolist()):
        hidden = eng.step(int(tok))
        prompt_margin[p] = eng.last_routes()[2]
        step_routes[p], step_gap[p] = route_record(eng)
        logits = eng.logits(hidden)
        p_top1[p], p_margin[p], order = top2(logits)
        p_top_idx[p] = order
        p_top_val[p] = logits[order]
        p_sub_val[p] = logits[psub]
        if p % 64 == 63:
            print(f"prompt {p + 1}/{PROMPT}, {(time.time() - t1) / (p + 1):.2f} s/step", flush=True)
    tokens = np.empty(NEW, np.int64)
    margins = np.empty(NEW, np.float32)
    top_idx = np.empty((NEW, 16), np.int64)
    top_val = np.empty((NEW, 16), np.float32)
    sub_val = np.empty((NEW, SUBSET), np.float32)
    route_min = np.empty(NEW, np.float32)
    route_layer = np.empty(NEW, np.int64)
    first_logits = None
    gen_margin = np.empty((NEW, L), np.float32)
    for s in range(NEW):
        logits = eng.logits(hidden)
        if s == 0:
            first_logits = logits.copy()
        tok, m, order = top2(logits)
        tokens[s] = tok
        margins[s] = m
        top_idx[s] = order
        top_val[s] = logits[order]
        sub_val[s] = logits[subset]
        if s + 1 < NEW:
            hidden = eng.step(tok)
            rm = eng.last_routes()[2]
            step_routes[PROMPT + s], step_gap[PROMPT + s] = route_record(eng)
            gen_margin[s] = rm
            route_min[s] = rm.min()
            route_layer[s] = int(rm.argmin())
        else:
            gen_margin[s] = np.nan
            route_min[s] = np.nan
            route_layer[s] = -1
        print(f"gen {s}: token {tok} margin {m:.4f}", flush=True)
    np.savez_compressed(args.out, seed=SEED, prompt=prompt.astype(np.int64), tokens=tokens,
                        margins=margins, top_idx=top_idx, top_val=top_val, subset=subset,
                        sub_val=sub_val, first_logits=first_logits.astype(np.float32),
                        prompt_route_margin=prompt_margin, gen_route_margin=gen_margin,
                        route_min=route_min, route_layer=route_layer, step_routes=step_routes,
                        step_gap=step_gap, prompt_top1=p_top1, prompt_margin=p_margin,
                        prompt_top_idx=p_top_idx, prompt_top_val=p_top_val,
                        prompt_subset=psub, prompt_sub_val=p_sub_val)
    print(f"wrote {args.out} in {time.time() - t0:.0f} s", flush=True)


if __name__ == "__main__":
    main()
