"""Benchmark of the Qwen3-30B-A3B FP8 decode step on one MI355X.

Workload (the configuration the headline metric is quoted on): the full 48-layer random-init
Qwen3-30B-A3B FP8 model (hidden 2048, 32 q / 4 kv heads of 128, 128 experts top-8 with
intermediate 768, vocab 151936, RMSNorm eps 1e-6, RoPE theta 1e6, bf16 embedding and lm_head
N(0, 0.02), FP8 projections N(0, 0.02) block-quantised, norm weights 1.0), weights synthesised
on the device by the library's counter-based generator (the same values the CPU oracle
generates). A seeded 512-token prompt runs through the decode graph first (untimed), then
`warmup` greedy tokens, then exactly `steps` timed greedy tokens at bs=1, each one
hipGraph replay (token id in, greedy token out). value = tokens / second.

The JSON line also carries:
  roofline: the dominant launch's algorithmic bytes over its average duration. The timed form
            is the default chain of launches per layer (the router rows inside the gate|up launch:
            five per layer; or, with --persistent, every layer in one persistent launch,
            "decode_layers", then the lm_head). The durations come from
            further decode steps made as direct launches, each launch's start and end recorded by
            its own dispatch (hipExtLaunchKernel events on the library stream); peak 8 TB/s.
            traffic comes from the committed rocprofv3 PMC summary for that kernel when one exists
            (profiles/), else null.
  other_form: the same step in the other form (tok/s).
  persistent_stage_us_per_layer: the persistent launch's own stage stamps (the GPU's constant
            clock), the mean time per layer of each stage: input row handoff, q|k|v + attention,
            o + residual, router and route, expert FFN (gate|up and down).
  top2_margins: the top-2 logit margin of each untimed stamped token.
  cpu_baseline: the C oracle engine (the CPU restatement of the reference's host step) on the
            host cores at the GPU run's context: 4 of the 48 layers over a cache holding the
            same number of positions, plus the full-vocab lm_head, scaled to the 48-layer step;
            timed on one thread and on every core this process may use (nproc reported beside
            it), about 15 s of CPU work. value is the all-cores figure.
  bs32:     the metric's batch-32 figure, measured after the bs=1 model is freed: configuration
            5's batched step (32 sequences, contexts log-uniform in [1k, 128k], one hipGraph per
            step) for --bs32-steps steps; --no-bs32 skips it. --workload serve prints the full
            line for that configuration.
"""
import argparse
import json
import os
import sys
import time

REPO = os.path.dirname(os.path.abspath(__file__))
sys.path[:0] = [os.path.join(REPO, "aien-sovereign-core-mv_amd"), os.path.join(REPO, "oracle")]

import numpy as np  # noqa: E402

METRIC = "Qwen3-30B-A3B FP8 decode tok/s at bs1/bs32; achieved HBM TB/s vs peak"
L, H, QH, KVH, HD, E, TOPK, I, V = 48, 2048, 32, 4, 128, 128, 8, 768, 151936
SEED = 20261201
PEAK_GBS = 8000.0


def tid(layer, kind):
    # tensor ids of the generator, shared with the CPU oracle's synthetic model
    return 1000 + layer * 16 + kind


def algorithmic_bytes(kind, ctx):
    """HBM bytes one launch of a decode-graph kernel must move at context `ctx` (weights,
    scales, activations in and out; the KV rows the attention must read)."""
    if kind == "qkv":          # 5120 x 2048 e4m3 + scales + x + norm weights + q|k|v out
        return 5120 * 2048 + 40 * 16 * 4 + 2 * H * 4 + 5120 * 4
    # the decode graph cuts a kv head's pages into at most 64 splits
    pages = max(1, -(-(ctx - 1) // 16))
    splits = -(-pages // -(-pages // 64))
    if kind == "attn":         # K and V of 4 heads over ctx positions + q|k|v in + the split
        # partials out and back in for the merge + the attention row out
        return 2 * KVH * ctx * HD * 2 + 5120 * 4 + 2 * QH * splits * 132 * 4 + 4096 * 4
    if kind == "o_proj":       # 2048 x 4096 e4m3 + scales + attention row + residual read/write
        return 2048 * 4096 + 16 * 32 * 4 + 4096 * 4 + 2 * H * 4
    if kind == "router":       # bf16 gate + norm weights + x in + x' out + logits
        return E * H * 2 + 3 * H * 4 + E * 4
    if kind == "gate_up":      # 8 experts x 1536 x 2048 e4m3 + scales + logits + x' + activations
        return TOPK * (1536 * 2048 + 12 * 16 * 4) + E * 4 + H * 4 + TOPK * I * 4
    if kind == "down":         # 8 experts x 2048 x 768 e4m3 + scales + activations + residual
        return TOPK * (2048 * 768 + 16 * 6 * 4) + TOPK * I * 4 + 2 * H * 4
    if kind == "lm_head":      # 151936 x 2048 bf16 + x + final norm + logits
        return V * H * 2 + 2 * H * 4 + V * 4
    if kind == "route_gate_up":  # the router rows and gate|up in one launch
        return algorithmic_bytes("router", ctx) + algorithmic_bytes("gate_up", ctx)
    return 0


# the decode graph's kernels of one layer (the router rows in their own launch or in gate|up's),
# then the lm_head
LAYER_KINDS = ["qkv", "attn", "o_proj", "router", "gate_up", "down"]
# launch kinds the graph records per launch (include/omega_gpu.h OMEGA_GPU_DGRAPH_K_*)
KIND_NAMES = {1: "qkv", 2: "attn", 3: "o_proj", 5: "router", 6: "gate_up", 8: "down", 10: "lm_head"}


def launch_names(kinds):
    """Names of a token's launches from the kinds the graph recorded; a gate|up launch with no
    router launch in the token carries the router rows too."""
    names = [KIND_NAMES.get(int(k), f"kind{int(k)}") for k in kinds]
    if "router" not in names:
        names = ["route_gate_up" if n == "gate_up" else n for n in names]
    return names


def build_model(om, max_pos):
    """The full 48-layer model synthesised on the device (omega_amd.SynthDecodeModel)."""
    t0 = time.time()
    m = om.SynthDecodeModel(SEED, max_pos)
    om.sync()
    return dict(model=m, graph=m.graph, seconds=time.time() - t0)


def host_cores():
    """(nproc, cores this process may use): the second is the affinity set, capped by
    OMP_NUM_THREADS where the box sets it (one GPU's share of the host)."""
    nproc = os.cpu_count() or 1
    usable = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else nproc
    cap = os.environ.get("OMP_NUM_THREADS", "")
    if cap.isdigit() and int(cap) > 0:
        usable = min(usable, int(cap))
    return nproc, usable


def cpu_baseline(threads, ctx):
    """The oracle engine (oref_engine_step, the C restatement of the reference's host step) on a
    bounded sample at the GPU run's context: 4 of the 48 layers with the cache holding `ctx`
    positions, timed on one host thread and on `threads` threads (per-output-row parallel GEMVs,
    as the reference's rayon loops), plus the 151936-row lm_head each way; scaled to 48 layers."""
    import pyoracle as orc

    layers = 4
    nproc, _ = host_cores()
    cfg = dict(layers=layers, hidden=H, q_heads=QH, kv_heads=KVH, head_dim=HD, experts=E,
               top_k=TOPK, inter=I, vocab=V, eps=1e-6, rope_theta=1e6)
    m = orc.Model(cfg, SEED, sigma=0.02, norm_sigma=0.0, threads=threads)

    def timed(nthreads, tokens, heads):
        eng = orc.Engine(m, ctx + tokens + 2, refined_router=True, threads=nthreads)
        eng.fill_random(ctx, seed=SEED)
        hid = eng.step(1)   # first touch of every weight page
        t0 = time.perf_counter()
        for t in range(tokens):
            hid = eng.step(2 + t)
        t_layer = (time.perf_counter() - t0) / tokens / layers
        t1 = time.perf_counter()
        for _ in range(heads):
            eng.logits(hid)
        t_lm = (time.perf_counter() - t1) / heads
        del eng
        step = t_layer * L + t_lm
        return dict(s_per_token=round(step, 4), tok_s=round(1.0 / step, 4),
                    ms_per_layer=round(t_layer * 1e3, 2), ms_lm_head=round(t_lm * 1e3, 1),
                    sample=f"{tokens} tokens x {layers} layers, {heads} lm_heads")

    one = timed(1, 3, 1)
    many = timed(threads, 32, 4)
    return {"value": many["tok_s"], "unit": "tok/s", "cores": threads, "kind": "port",
            "nproc": nproc, "context": ctx,
            "extrapolated": f"from {layers} of {L} layers (per-layer time x {L} + the full lm_head)",
            "single_thread": one, "all_cores": many,
            "sample": f"C oracle engine (oracle/oracle.c oref_engine_step + oref_engine_logits), "
                      f"{layers} of 48 layers with {ctx} cached positions, scaled to 48 layers; "
                      f"all cores = {threads} threads of nproc {nproc} (this process's share): "
                      f"{many['ms_per_layer']} ms/layer, lm_head {many['ms_lm_head']} ms, "
                      f"{many['s_per_token']} s/token; one thread: {one['ms_per_layer']} ms/layer, "
                      f"lm_head {one['ms_lm_head']} ms, {one['s_per_token']} s/token"}


def committed_traffic(kind, summary=None):
    """HBM bytes per launch of `kind` from the committed rocprofv3 PMC summary (profiles/
    <kind>_traffic.md, or the file `summary` there), if any."""
    p = os.path.join(REPO, "profiles", summary or f"{kind}_traffic.md")
    if not os.path.exists(p):
        return None
    for line in open(p):
        if line.startswith("traffic_bytes_per_launch:"):
            return int(float(line.split(":", 1)[1]))
    return None


def copy_probe(nbytes):
    """One device-to-device copy of `nbytes` (the runtime's copy kernel): the calibration run of
    the HBM byte counters, whose FETCH_SIZE / WRITE_SIZE should read nbytes each."""
    import ctypes as C

    hip = C.CDLL("libamdhip64.so")
    src, dst = C.c_void_p(), C.c_void_p()
    assert hip.hipMalloc(C.byref(src), C.c_size_t(nbytes)) == 0
    assert hip.hipMalloc(C.byref(dst), C.c_size_t(nbytes)) == 0
    assert hip.hipMemset(src, 1, C.c_size_t(nbytes)) == 0
    for _ in range(3):
        assert hip.hipMemcpy(dst, src, C.c_size_t(nbytes), 3) == 0  # hipMemcpyDeviceToDevice
    assert hip.hipDeviceSynchronize() == 0
    hip.hipFree(src)
    hip.hipFree(dst)
    print(json.dumps({"copy_probe_bytes": nbytes, "copies": 3}))


# ---------------------------------------------------------------- configuration 1: the q|k|v FP8 GEMV
GEMV_COPIES = 48


def gemv_bytes():
    """Algorithmic HBM bytes of one configuration-1 GEMV: 5120 x 2048 e4m3 weights, 40 x 16 f32
    block scales, the f32 activation row in and the f32 output row out."""
    return 5120 * 2048 + 40 * 16 * 4 + H * 4 + 5120 * 4


def gemv_cpu_baseline():
    """The oracle's FP8 GEMV (oref_fp8_grouped: one group, in-order f32 accumulation) on one host
    thread, for about 10 s."""
    import pyoracle as orc

    w, s_ = orc.synth_fp8(SEED, 3000, 1, 5120, 2048)
    x = orc.bf16_to_f32(orc.synth_bf16(SEED, 7, (H,), 1.0))
    reps = 0
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < 10.0:
        orc.fp8_grouped(w, s_, np.zeros(1, np.uint32), x, threads=1)
        reps += 1
    us = (time.perf_counter() - t0) / reps * 1e6
    return {"value": round(us, 1), "unit": "us/GEMV", "cores": 1, "kind": "port",
            "sample": f"oracle oref_fp8_grouped (oracle/oracle.c), one 5120 x 2048 GEMV, {reps} calls "
                      f"in about 10 s on one host thread"}


def bench_gemv(om, args):
    """Configuration 1: the fused q|k|v FP8 GEMV (5120 x 2048 e4m3 N(0, 0.02) block-quantised,
    x a bf16 N(0, 1) row) as device-pointer GEMVs rotating over 48 distinct weight copies (504 MB,
    about twice the 256 MB Infinity Cache), captured once as a hipGraph of 48 launches and replayed;
    the time per GEMV includes the graph's launch gap between dependent kernels."""
    import ctypes as C

    h = om.hip()
    lib = om.lib()
    ts = [om.Fp8Tensor.synth(1, 5120, 2048, SEED, 3000 + c) for c in range(GEMV_COPIES)]
    x = om.DeviceBuffer.from_array(om.synth_bf16_host(SEED, 7, (H,), 1.0).astype(np.uint32) << 16)
    y = om.DeviceBuffer(5120 * 4)
    om.sync()
    stream = lib.omega_gpu_stream()
    graph, exe = C.c_void_p(), C.c_void_p()

    def direct():
        for t in ts:
            assert lib.omega_gpu_fp8_gemv_dev(t.as_raw(), 0, x.ptr, y.ptr) == 0

    if args.eager:  # the same launches made directly (a kernel trace cannot follow a graph replay)
        run = direct
    else:
        assert h.hipStreamBeginCapture(C.c_void_p(stream), 1) == 0   # hipStreamCaptureModeThreadLocal
        direct()
        assert h.hipStreamEndCapture(C.c_void_p(stream), C.byref(graph)) == 0
        assert h.hipGraphInstantiate(C.byref(exe), graph, None, None, C.c_size_t(0)) == 0

        def run():
            assert h.hipGraphLaunch(exe, C.c_void_p(stream)) == 0
    timer = om.StreamTimer()
    reps = args.gemv_reps
    for _ in range(2):
        run()
    timer.start()
    for _ in range(reps):
        run()
    timer.stop()
    ms = timer.ms()
    us = ms * 1e3 / (reps * GEMV_COPIES)
    b = gemv_bytes()
    gbs = b / (us * 1e3)
    if not args.eager:
        h.hipGraphExecDestroy(exe)
        h.hipGraphDestroy(graph)
    cpu = None if args.no_cpu else gemv_cpu_baseline()
    print(json.dumps({
        "metric": "FP8 block-scaled GEMV 5120 x 2048 (configuration 1), achieved HBM GB/s vs peak",
        "value": round(gbs, 1), "unit": "GB/s", "n_gpus": 1, "higher_is_better": True,
        "us_per_gemv": round(us, 3), "gemvs": reps * GEMV_COPIES,
        "dtype": "fp8 (e4m3 weights, f32 activations, fp32 accumulate)",
        "data": "synthetic N(0, 0.02) weights block-quantised to e4m3, bf16 N(0,1) row",
        "config": {"workload": "q|k|v GEMV 5120 x 2048, 48 weight copies, "
                               + ("48 direct launches" if args.eager else "hipGraph of 48 launches")},
        "roofline": {"bound": "hbm", "kernel": "k_fp8_rows1", "achieved": round(gbs, 1), "peak": PEAK_GBS,
                     "unit": "GB/s", "frac": round(gbs / PEAK_GBS, 4),
                     "traffic": committed_traffic(None, "gemv_config1_kernel_trace.md")},
        "cpu_baseline": cpu}), flush=True)
    for t in ts:
        t.free()
    x.free()
    y.free()


# ---------------------------------------------------------------- whole-prompt prefill (time to first token)
def bench_prefill(om, args):
    """The whole-prompt prefill of the full 48-layer model (the reference's prefill boundary:
    W8A8 quantiser + grouped GEMM + prefill attention, host RMSNorms / routing plan as in the
    reference driver) for a seeded prompt of each length in --prefill-lengths, then the lm_head
    and argmax of the last token: time to first token (wall, host included) and the chip time of
    the prefill launches. The decode-graph alternative (every prompt token one decode step) is
    printed beside it from the bs=1 step time when --prefill-decode-ms is given."""
    from omega_amd import prefill as pf

    lengths = [int(v) for v in args.prefill_lengths.split(",")]
    max_pos = om.round_max_pos(max(lengths) + 8)
    t0 = time.time()
    layers, tensors = [], []
    ones = np.ones(H, np.float32)
    for l in range(L):
        qkv = om.Fp8Tensor.synth(1, 5120, 2048, SEED, tid(l, 0))
        o = om.Fp8Tensor.synth(1, 2048, 4096, SEED, tid(l, 1))
        gu = om.Fp8Tensor.synth(E, 1536, 2048, SEED, tid(l, 2))
        dn = om.Fp8Tensor.synth(E, 2048, 768, SEED, tid(l, 3))
        tensors += [qkv, o, gu, dn]
        gate = om.synth_bf16_host(SEED, tid(l, 8), (E, H), 0.02)
        layers.append(dict(qkv=qkv, o=o, gate_up=gu, down=dn, input_norm=ones, post_norm=ones,
                           router=(gate.astype(np.uint32) << 16).view(np.float32)))
    cache = om.DecodeAttnCache(L, max_pos, 1e6)
    for l in range(L):
        cache.set_norms(l, np.ones(HD, np.float32), np.ones(HD, np.float32))
    lm = om.Bf16Tensor.synth(V, H, SEED, 2, 0.02)
    embed_host = om.synth_bf16_host(SEED, 1, (V, H), 0.02)
    wp = pf.WholePromptPrefill(layers, ones, lambda t: (embed_host[t].astype(np.uint32) << 16).view(np.float32),
                               cache, 1e-6)
    om.sync()
    build_s = time.time() - t0
    rng = np.random.default_rng(SEED)
    points = []
    for m in lengths:
        prompt = rng.integers(0, V, m).tolist()
        wp.run(prompt, 0)  # warm at the same length: buffers sized, code paths touched
        pf.stats_reset()
        t1 = time.perf_counter()
        hidden = wp.run(prompt, 0)
        logits, _ = lm.gemv_f32(hidden)
        tok = int(np.argmax(logits))
        ttft = time.perf_counter() - t1
        chip_ns, launches = pf.stats()
        line = {"workload": "whole_prompt_prefill", "tokens": m, "ttft_s": round(ttft, 4),
                "chip_ms": round(wp.stats["chip_ns"] / 1e6, 2), "pf_launch_ms": round(chip_ns / 1e6, 2),
                "pf_launches": launches, "prompt_tok_s": round(m / ttft, 1), "first_token": tok}
        if args.prefill_decode_ms:
            line["decode_graph_prompt_s"] = round(m * args.prefill_decode_ms / 1e3, 3)
        print(json.dumps(line), flush=True)
        points.append(line)
    print(json.dumps({
        "metric": "Qwen3-30B-A3B FP8 whole-prompt prefill, time to first token",
        "value": points[0]["ttft_s"], "unit": "s", "n_gpus": 1, "higher_is_better": False,
        "dtype": "fp8 (W8A8: e4m3 weights and activations, fp32 accumulate)",
        "data": "synthetic random-init weights, seeded prompt",
        "config": {"workload": "whole-prompt prefill through the omega_gpu_pf_* boundary and the host "
                               "driver mirror", "lengths": lengths},
        "points": points, "extra": {"build_s": round(build_s, 1)}}), flush=True)
    wp.free()
    cache.free()
    lm.free()
    for t in tensors:
        t.free()


def bench_schedule(om, args):
    """The beat scheduler (omega_amd.serve) over the batched step of the full 48-layer model: 32
    slots, --schedule-requests requests arriving two per beat from beat 0 (each waits while every
    slot is taken), prompts of 32..512 seeded tokens fed one per beat, 128 greedy tokens each.
    With --schedule-prefill a joining prompt goes in whole (the whole-prompt prefill into a fused
    cache, then its payload blocks into the request's pages). Reports generated tokens / s, all
    fed tokens / s and the time to first token in beats."""
    from omega_amd import serve

    slots, new, nreq = SERVE_SEQS, 128, args.schedule_requests
    rng = np.random.default_rng(SEED + 5)
    prompts = [rng.integers(0, V, int(n)).tolist() for n in rng.integers(32, 513, nreq)]
    max_blocks = -(-(512 + new) // 16)
    blocks = slots * max_blocks
    lay = om.kv_layout(blocks, 16, L, KVH, HD)
    pool = om.DeviceBuffer(lay.pool_bytes)
    router = om.Router(L)
    ones = np.ones(H, np.float32)
    layers = []
    for l in range(L):
        qkv = om.Fp8Tensor.synth(1, 5120, 2048, SEED, tid(l, 0))
        o = om.Fp8Tensor.synth(1, 2048, 4096, SEED, tid(l, 1))
        gu = om.Fp8Tensor.synth(E, 1536, 2048, SEED, tid(l, 2))
        dn = om.Fp8Tensor.synth(E, 2048, 768, SEED, tid(l, 3))
        layers.append((qkv, o, gu, dn))
        router.set_layer(l, om.synth_bf16_host(SEED, tid(l, 8), (E, H), 0.02), ones)
        router.set_directory(l, np.zeros(2 * E, np.uint64), np.zeros(2 * E, np.uint64))
    lm = om.Bf16Tensor.synth(V, H, SEED, 2, 0.02)
    embed = om.Bf16Tensor.synth(V, H, SEED, 1, 0.02)
    bd = om.BatchDecode(L, V, slots, max_blocks, max_blocks * 16, 1e-6, 1e6, router, lm, embed, pool.ptr, lay)
    hd1 = np.ones(HD, np.float32)
    for l, (qkv, o, gu, dn) in enumerate(layers):
        bd.set_layer(l, qkv, o, gu, dn, ones, hd1, hd1)
    bd.set_final_norm(ones)
    pp = fused = wp = None
    if args.schedule_prefill:
        from omega_amd import prefill as pf

        fused = om.DecodeAttnCache(L, om.round_max_pos(512), 1e6)
        for l in range(L):
            fused.set_norms(l, hd1, hd1)
        embed_host = om.synth_bf16_host(SEED, 1, (V, H), 0.02)
        wp = pf.WholePromptPrefill(
            [dict(qkv=q, o=o, gate_up=g, down=d, input_norm=ones, post_norm=ones,
                  router=(om.synth_bf16_host(SEED, tid(l, 8), (E, H), 0.02).astype(np.uint32) << 16).view(np.float32))
             for l, (q, o, g, d) in enumerate(layers)],
            ones, lambda t: (embed_host[t].astype(np.uint32) << 16).view(np.float32), fused, 1e-6)
        pp = serve.PromptPrefill(wp, fused, pool.ptr, 512)
        wp.run(prompts[0], 0)  # buffers sized for the longest prompt
    serve.BeatScheduler(bd, blocks, max_blocks, slots=slots, prefill=pp).run(
        {0: [("warm", prompts[0][:40], 4, ())]})
    om.sync()
    arrivals = {}
    for i, p in enumerate(prompts):
        arrivals.setdefault(i // 2, []).append((i, p, new, ()))
    sch = serve.BeatScheduler(bd, blocks, max_blocks, slots=slots, prefill=pp)
    t0 = time.perf_counter()
    done = sch.run(arrivals)
    om.sync()
    elapsed = time.perf_counter() - t0
    gen = sum(len(r.tokens) for r in done.values())
    ttft = np.array([r.first_token_beat - r.joined_beat for r in done.values()])
    wait = np.array([r.joined_beat - i // 2 for i, r in done.items()])
    print(json.dumps({
        "metric": "Qwen3-30B-A3B FP8 serving mode (beat scheduler over the batched step): generated tok/s",
        "value": round(gen / elapsed, 1), "unit": "tok/s", "n_gpus": 1, "higher_is_better": True,
        "dtype": "fp8", "data": "synthetic random-init weights, seeded prompts",
        "config": {"workload": f"{nreq} requests, 2 arriving per beat, prompts 32..512 tokens "
                               + ("through the whole-prompt prefill at join" if pp else "fed one per beat")
                               + f", {new} greedy tokens each, {slots} slots",
                   "slots": slots},
        "beats": sch.beats, "ms_per_beat": round(elapsed * 1e3 / sch.beats, 3),
        "fed_tok_s": round(sch.fed_tokens / elapsed, 1), "generated": gen, "elapsed_s": round(elapsed, 2),
        "mean_rows_per_beat": round(sch.fed_tokens / sch.beats, 2),
        "first_token_beats_mean": round(float(ttft.mean()), 1), "wait_beats_mean": round(float(wait.mean()), 1)}),
        flush=True)
    if pp:
        pp.free()
        wp.free()
        fused.free()
    bd.free()
    for t in layers:
        for x in t:
            x.free()
    router.free()
    lm.free()
    embed.free()
    pool.free()


def bench_kvio(om, args):
    """KV park / restore of the fused 48-layer cache (the HostPagedPoolV1 payload of
    qwen3_moe_omega_kvio.rs): export and import of --kvio-positions positions between the cache
    and a device payload buffer (both resident in HBM; each moves the payload's bytes in and out),
    then one export and one import through pageable host memory (the PCIe-inclusive rate)."""
    n = args.kvio_positions
    cache = om.DecodeAttnCache(L, om.round_max_pos(n), 1e6)
    nbytes = cache.payload_len(n)
    buf = om.DeviceBuffer(nbytes)
    for _ in range(2):
        cache.export_kv_dev(0, n, buf.ptr, nbytes)
        cache.import_kv_dev(0, n, buf.ptr, nbytes)
    ex = [cache.export_kv_dev(0, n, buf.ptr, nbytes) for _ in range(args.kvio_reps)]
    im = [cache.import_kv_dev(0, n, buf.ptr, nbytes) for _ in range(args.kvio_reps)]
    t0 = time.perf_counter()
    host, _ = cache.export_kv(0, n)
    t_host_ex = time.perf_counter() - t0
    t0 = time.perf_counter()
    cache.import_kv(0, n, host)
    t_host_im = time.perf_counter() - t0
    ex_us, im_us = np.mean(ex) / 1e3, np.mean(im) / 1e3
    moved = 2 * nbytes  # payload bytes read and written
    gbs = moved / (ex_us * 1e3)
    print(json.dumps({
        "metric": "KV park / restore of the fused cache (HostPagedPoolV1 payload), achieved HBM GB/s vs peak",
        "value": round(gbs, 1), "unit": "GB/s", "n_gpus": 1, "higher_is_better": True,
        "dtype": "bf16 bytes (moved, not converted)",
        "data": "an allocated 48-layer fused cache (contents as allocated)",
        "config": {"workload": f"export / import of {n} positions x 48 layers x 4 kv heads x 128 dims",
                   "payload_bytes": nbytes},
        "roofline": {"bound": "hbm", "kernel": "k_kv_export", "achieved": round(gbs, 1), "peak": PEAK_GBS,
                     "unit": "GB/s", "frac": round(gbs / PEAK_GBS, 4), "traffic": None},
        "export_us": round(ex_us, 1), "import_us": round(im_us, 1),
        "import_GBs": round(moved / (im_us * 1e3), 1),
        "host_export_s": round(t_host_ex, 3), "host_import_s": round(t_host_im, 3),
        "host_export_GBs": round(nbytes / t_host_ex / 1e9, 2), "host_import_GBs": round(nbytes / t_host_im / 1e9, 2),
        "reps": args.kvio_reps}), flush=True)
    buf.free()
    cache.free()


# ---------------------------------------------------------------- configuration 3: paged attention
PAGED_POINTS = [(b, l) for b in (1, 8, 32) for l in (2048, 8192, 32768)]


def paged_bytes(seqs, ctx):
    """Algorithmic HBM bytes of one paged-attention call: the K and V rows of the 4 kv heads over
    every context token (2 x 4 x 256 B per token), q and out f32, the page tables and lengths."""
    return seqs * ctx * 2 * KVH * HD * 2 + 2 * seqs * QH * HD * 4 + seqs * (ctx // 16) * 4 + seqs * 4


def paged_cpu_baseline(om_unused=None):
    """The oracle's paged attention (f64 SDPA over the bf16 rows) on one host thread, batch 1 at
    context 2048, on a host pool of the same layout."""
    import ctypes as C

    import pyoracle as orc

    rng = np.random.default_rng(1)
    lay = orc.kv_layout(128, 16, 1, KVH, HD)
    pool = orc.f32_to_bf16(rng.standard_normal(lay.pool_bytes // 2).astype(np.float32)).view(np.uint8)
    tab = rng.permutation(128).astype(np.int32)
    q = rng.standard_normal(QH * HD).astype(np.float32)
    out = np.zeros(QH * HD, np.float32)
    reps = 0
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < 10.0:
        orc.lib().oref_paged_attention(orc.ptr(q), orc.ptr(pool), C.byref(lay), orc.ptr(tab), 2048, 0,
                                       QH, KVH, HD, orc.ptr(out))
        reps += 1
    us = (time.perf_counter() - t0) / reps * 1e6
    return {"value": round(us, 1), "unit": "us/call", "cores": 1, "kind": "port",
            "sample": f"oracle oref_paged_attention (oracle/oracle.c), batch 1 at context 2048, "
                      f"{reps} calls in about 10 s on one host thread"}


def bench_paged(om, args):
    """Configuration 3: GQA 32/4 x 128 decode attention over 16-token pages of the 30B pool
    geometry (48 layers, one layer read), page tables random permutations of the free pages,
    bf16 K/V ~ N(0,1); each point timed cold (the Infinity Cache and L2 flushed by a 1 GiB fill
    before every call) with HIP events on the library stream: one launch per call where the
    split workgroups all fit the device at once (the splits merged in the same launch, every point
    here), else the split launch and the combine launch. Each point is also timed back to back:
    one call per layer of the pool (48 calls in a row, each on K/V the row has not read before,
    the caches flushed once before the row), the way a decode step issues them; that figure is the
    row's event span / 48, so one call's event and launch overhead is not charged to it alone."""
    import ctypes as C

    max_pages = max(b * l // 16 for b, l in PAGED_POINTS)
    L_ = om.kv_layout(max_pages, 16, L, KVH, HD)
    pool = om.DeviceBuffer(L_.pool_bytes)
    om.synth_bf16_dev(pool, L_.pool_bytes // 2, SEED, 77, 1.0)
    flush = om.DeviceBuffer(1 << 30)
    om.sync()
    lib = om.lib()
    hip = om.hip()
    stream = lib.omega_gpu_stream()
    timer = om.StreamTimer()
    rng = np.random.default_rng(SEED)
    layer = 7
    lines = []
    points = PAGED_POINTS
    if args.paged_points:
        points = [tuple(int(v) for v in p.split("x")) for p in args.paged_points.split(",")]
        assert all(pt in PAGED_POINTS for pt in points), f"points must come from {PAGED_POINTS}"
    for seqs, ctx in points:
        pages = ctx // 16
        perm = rng.permutation(max_pages)[: seqs * pages].astype(np.int32).reshape(seqs, pages)
        q = rng.standard_normal((seqs, QH * HD)).astype(np.float32)
        qd = om.DeviceBuffer.from_array(q)
        td = om.DeviceBuffer.from_array(perm)
        ld = om.DeviceBuffer.from_array(np.full(seqs, ctx, np.int32))
        od = om.DeviceBuffer(q.nbytes)

        def call(lay=layer):
            rc = lib.omega_gpu_paged_attention_batch_dev(qd.ptr, pool.ptr, C.byref(L_), td.ptr, ld.ptr,
                                                         pages, seqs, ctx, lay, QH, KVH, HD, od.ptr)
            assert rc == 0, om._s(lib.omega_gpu_attention_last_error())

        for _ in range(2):
            call()
        times = []
        for _ in range(args.paged_reps):
            assert hip.hipMemsetAsync(flush.ptr, 1, C.c_size_t(flush.nbytes), stream) == 0
            timer.start()
            call()
            timer.stop()
            times.append(timer.ms() * 1e3)
        us = float(np.median(times))
        # back to back: the 48 layers' calls in a row on the stream (as a decode step makes them),
        # each reading K/V no earlier call of the row touched, after one flush; per call = row / 48
        chained = []
        for _ in range(max(3, args.paged_reps // 3)):
            assert hip.hipMemsetAsync(flush.ptr, 1, C.c_size_t(flush.nbytes), stream) == 0
            timer.start()
            for lay in range(L):
                call(lay)
            timer.stop()
            chained.append(timer.ms() * 1e3 / L)
        us_b2b = float(np.median(chained))
        b = paged_bytes(seqs, ctx)
        line = {"workload": "paged_attention", "seqs": seqs, "ctx": ctx, "us_per_call": round(us, 2),
                "algorithmic_bytes": b, "GBs": round(b / (us * 1e3), 1),
                "frac": round(b / (us * 1e3) / PEAK_GBS, 4), "reps": len(times),
                "us_per_call_back_to_back": round(us_b2b, 2),
                "GBs_back_to_back": round(b / (us_b2b * 1e3), 1)}
        print(json.dumps(line), flush=True)
        lines.append(line)
        for buf in (qd, td, ld, od):
            buf.free()
    cpu = None if args.no_cpu else paged_cpu_baseline()
    big = lines[-1]
    print(json.dumps({
        "metric": "paged GQA decode attention (configuration 3), achieved HBM GB/s vs peak",
        "value": big["GBs"], "unit": "GB/s", "n_gpus": 1, "higher_is_better": True,
        "dtype": "bf16 KV, f32 q/out, fp32 accumulate", "data": "synthetic N(0,1) K/V, random page tables",
        "config": {"workload": "paged attention 32q/4kv x 128, 16-token pages, 48-layer pool geometry",
                   "points": [[p["seqs"], p["ctx"]] for p in lines]},
        "roofline": {"bound": "hbm", "kernel": "k_paged4f (splits merged in the launch)", "achieved": big["GBs"],
                     "peak": PEAK_GBS, "unit": "GB/s", "frac": big["frac"],
                     "traffic": (committed_traffic(None, "paged_attention_traffic.md")
                                 if (big["seqs"], big["ctx"]) == PAGED_POINTS[-1] else None)},
        "points": lines, "cpu_baseline": cpu}), flush=True)


# ---------------------------------------------------------------- configuration 2: batched MoE block
def moe_bytes(T, distinct):
    """Algorithmic HBM bytes of one MoE block: the bf16 router, the e4m3 gate|up and down weights
    and block scales of every distinct routed expert, h in, ids / weights / moe_out out."""
    per_expert = 1536 * 2048 + 12 * 16 * 4 + 2048 * 768 + 16 * 6 * 4
    return E * H * 2 + H * 4 + distinct * per_expert + T * H * 4 * 2 + T * TOPK * 8


def moe_cpu_baseline(T, threads):
    """The oracle's per-token route + FP8 MoE arm over T tokens (synthetic weights)."""
    import pyoracle as orc

    rng = np.random.default_rng(3)
    gu_w, gu_s = orc.synth_fp8(SEED, 2, E, 2 * I, H)
    dn_w, dn_s = orc.synth_fp8(SEED, 3, E, H, I)
    gate = orc.f32_to_bf16((rng.standard_normal((E, H)) * 0.02).astype(np.float32))
    norm = np.ones(H, np.float32)
    h = rng.standard_normal((T, H)).astype(np.float32)
    t0 = time.perf_counter()
    for t in range(T):
        ids, w, post, _ = orc.route(gate, norm, h[t], 1e-6)
        orc.moe_block(gu_w, gu_s, dn_w, dn_s, ids, w, post)
    ms = (time.perf_counter() - t0) * 1e3
    return {"value": round(ms, 2), "unit": "ms/block", "cores": 1, "kind": "port",
            "sample": f"oracle route + oref_moe_block (oracle/oracle.c) for {T} tokens, one host "
                      f"thread, synthetic weights of the same shapes"}


def bench_moe(om, args):
    """Configuration 2: one Qwen3-30B-A3B MoE block at token batch 1 and 32 (h ~ N(0,1) bf16,
    router N(0, 0.02) bf16, experts e4m3 with 128x128 block scales), timed with HIP events on the
    library stream over `moe_reps` calls with fresh inputs each (so the routed experts change)."""
    import ctypes as C

    router = om.Router(1)
    rng = np.random.default_rng(SEED)
    gate = om.synth_bf16_host(SEED, 9, (E, H), 0.02)
    router.set_layer(0, gate, np.ones(H, np.float32))
    router.set_directory(0, np.zeros(2 * E, np.uint64), np.zeros(2 * E, np.uint64))
    gu = om.Fp8Tensor.synth(E, 2 * I, H, SEED, 2)
    dn = om.Fp8Tensor.synth(E, H, I, SEED, 3)
    lib = om.lib()
    timer = om.StreamTimer()
    lines = []
    for T in (1, 32):
        reps = args.moe_reps
        hs = [om.DeviceBuffer.from_array(
            om.synth_bf16_host(SEED, 500 + r, (T, H), 1.0).astype(np.uint32) << 16) for r in range(reps + 2)]
        od = om.DeviceBuffer(T * H * 4)
        idd = om.DeviceBuffer(T * TOPK * 4)
        wd = om.DeviceBuffer(T * TOPK * 4)
        times, distinct = [], []
        for r in range(reps + 2):
            timer.start()
            rc = lib.omega_gpu_moe_batch_dev(router.as_raw(), 0, gu.as_raw(), dn.as_raw(), T, hs[r].ptr,
                                             1e-6, 1, None, idd.ptr, wd.ptr, od.ptr)
            assert rc == 0, om._s(lib.omega_gpu_fp8gemm_last_error())
            timer.stop()
            ms = timer.ms()
            if r >= 2:
                times.append(ms * 1e3)
                distinct.append(len(np.unique(idd.download(np.uint32, T * TOPK))))
        us = float(np.median(times))
        d = float(np.mean(distinct))
        b = moe_bytes(T, d)
        line = {"workload": "moe_block", "tokens": T, "us_per_block": round(us, 2),
                "distinct_experts": d, "algorithmic_bytes": int(b), "GBs": round(b / (us * 1e3), 1),
                "frac": round(b / (us * 1e3) / PEAK_GBS, 4), "reps": len(times),
                "launches": 3 if T == 1 else 6,
                "expert_path": ("decode-step GEMVs (router logits, gate|up with the ranking, down with the combine)"
                                if T == 1 else "grouped GEMV" if T < 16 else "FP8 MFMA")}
        print(json.dumps(line), flush=True)
        lines.append(line)
        for buf in hs + [od, idd, wd]:
            buf.free()
    # the reference's own grouped-GEMM entry (omega_gpu_fp8gemm_f32, what its batched-row path
    # calls) over the T = 32 row table of each expert projection: one launch, each segment's
    # weights read once; elapsed is the launch between HIP events on the library stream
    gemm = []
    for name, t, k in (("gate_up", gu, H), ("down", dn, I)):
        eids = np.concatenate([rng.choice(E, TOPK, replace=False) for _ in range(32)]).astype(np.uint32)
        toks = np.repeat(np.arange(32, dtype=np.uint32), TOPK)
        order = np.argsort(eids, kind="stable")
        x = rng.standard_normal((32, k)).astype(np.float32)
        el = []
        for r in range(args.moe_reps + 2):
            _, info = t.gemm_f32(eids[order], toks[order], x)
            if r >= 2:
                el.append(info.elapsed_ns / 1e3)
        us = float(np.median(el))
        g = {"workload": "fp8gemm_f32", "tensor": name, "rows": 256, "segments": int(info.segments),
             "us": round(us, 2), "weight_bytes": int(info.weight_bytes),
             "streamed_bytes": int(info.streamed_bytes), "GBs": round(info.weight_bytes / (us * 1e3), 1),
             "frac": round(info.weight_bytes / (us * 1e3) / PEAK_GBS, 4)}
        print(json.dumps(g), flush=True)
        gemm.append(g)
    cpu = None if args.no_cpu else moe_cpu_baseline(32, 1)
    big = lines[-1]
    print(json.dumps({
        "metric": "Qwen3-30B-A3B MoE block (configuration 2) at token batch 32, achieved HBM GB/s vs peak",
        "value": big["GBs"], "unit": "GB/s", "n_gpus": 1, "higher_is_better": True,
        "dtype": "fp8 (e4m3 weights, 4-term e4m3 activations, fp32 accumulate)",
        "data": "synthetic random-init weights and bf16 N(0,1) rows",
        "config": {"workload": "MoE block, 128 experts top-8, hidden 2048, intermediate 768",
                   "tokens": [1, 32]},
        "roofline": {"bound": "hbm", "kernel": "moe block (6 launches)", "achieved": big["GBs"],
                     "peak": PEAK_GBS, "unit": "GB/s", "frac": big["frac"], "traffic": None},
        "points": lines, "gemm_entry": gemm, "cpu_baseline": cpu}), flush=True)


# ---------------------------------------------------------------- configuration 5: batched serving decode
SERVE_SEQS = 32
KV_BYTES_PER_TOKEN = L * 2 * KVH * HD * 2                         # 98,304: K and V of 48 layers
DENSE_BYTES_PER_LAYER = 5120 * 2048 + 2048 * 4096 + E * H * 2     # q|k|v + o (e4m3) + router (bf16)
EXPERT_BYTES = 1536 * 2048 + 2048 * 768                           # gate|up + down of one expert (e4m3)


def serve_contexts():
    """32 context lengths drawn log-uniform in [1024, 131072] (seeded)."""
    rng = np.random.default_rng(SEED + 5)
    return np.exp(rng.uniform(np.log(1024), np.log(131072), SERVE_SEQS)).astype(np.int64)


def serve_cpu_baseline(threads, mean_ctx):
    """The oracle engine per token at a short context (4 of 48 layers, scaled) plus the oracle's
    paged attention of one layer at the mean context (times 48) plus one lm_head, times 32
    sequences: the CPU restatement serving the same step one sequence at a time."""
    import ctypes as C

    import pyoracle as orc

    cfg = dict(layers=4, hidden=H, q_heads=QH, kv_heads=KVH, head_dim=HD, experts=E, top_k=TOPK,
               inter=I, vocab=V, eps=1e-6, rope_theta=1e6)
    m = orc.Model(cfg, SEED, sigma=0.02, norm_sigma=0.0, threads=threads)
    eng = orc.Engine(m, 256, refined_router=True, threads=threads)
    hid = eng.step(1)
    t0 = time.perf_counter()
    for t in range(16):
        hid = eng.step(2 + t)
    t_layer = (time.perf_counter() - t0) / 16 / 4
    t1 = time.perf_counter()
    eng.logits(hid)
    t_lm = time.perf_counter() - t1
    rng = np.random.default_rng(1)
    pages = (mean_ctx + 15) // 16
    lay = orc.kv_layout(pages, 16, 1, KVH, HD)
    pool = orc.f32_to_bf16(rng.standard_normal(lay.pool_bytes // 2).astype(np.float32)).view(np.uint8)
    tab = np.arange(pages, dtype=np.int32)
    q = rng.standard_normal(QH * HD).astype(np.float32)
    out = np.zeros(QH * HD, np.float32)
    t2 = time.perf_counter()
    orc.lib().oref_paged_attention(orc.ptr(q), orc.ptr(pool), C.byref(lay), orc.ptr(tab), int(mean_ctx), 0,
                                   QH, KVH, HD, orc.ptr(out))
    t_attn = time.perf_counter() - t2
    per_token = t_layer * L + t_attn * L + t_lm
    return {"value": round(SERVE_SEQS / (per_token * SERVE_SEQS), 4), "unit": "tok/s", "cores": threads,
            "kind": "port",
            "sample": f"oracle engine (oracle/oracle.c, {threads} threads): 4 of 48 layers x 16 tokens "
                      f"({t_layer * 1e3:.1f} ms/layer) + oref_paged_attention of one layer at the mean "
                      f"context {int(mean_ctx)} ({t_attn * 1e3:.0f} ms, one thread) + one 151936-row "
                      f"lm_head ({t_lm * 1e3:.0f} ms), scaled to 48 layers: {per_token:.2f} s per token, "
                      f"the 32 sequences served one after another"}


def bench_serve(om, args, emit=True):
    """Configuration 5: 32 concurrent sequences of the random-init 48-layer model, contexts
    log-uniform in [1k, 128k] already resident as bf16 KV (N(0,1)) in 16-token pages of the pool
    (pages of every sequence a random permutation of the pool), `serve_steps` greedy steps of all
    32 sequences timed after `serve_warmup`, each step one hipGraph replay."""
    ctx = serve_contexts()
    steps, warmup = args.serve_steps, args.serve_warmup
    need = ctx + warmup + steps + 1
    pages = (need + 15) // 16
    max_blocks = int(pages.max())
    total = int(pages.sum())
    lay = om.kv_layout(total, 16, L, KVH, HD)
    t_build = time.time()
    pool = om.DeviceBuffer(lay.pool_bytes)
    om.synth_bf16_dev(pool, lay.pool_bytes // 2, SEED, 78, 1.0)
    rng = np.random.default_rng(SEED)
    perm = rng.permutation(total).astype(np.int32)
    tables = np.full((SERVE_SEQS, max_blocks), -1, np.int32)
    off = 0
    for s in range(SERVE_SEQS):
        tables[s, :pages[s]] = perm[off:off + pages[s]]
        off += pages[s]
    router = om.Router(L)
    ones = np.ones(H, np.float32)
    layers = []
    for l in range(L):
        qkv = om.Fp8Tensor.synth(1, 5120, 2048, SEED, tid(l, 0))
        o = om.Fp8Tensor.synth(1, 2048, 4096, SEED, tid(l, 1))
        gu = om.Fp8Tensor.synth(E, 1536, 2048, SEED, tid(l, 2))
        dn = om.Fp8Tensor.synth(E, 2048, 768, SEED, tid(l, 3))
        layers.append((qkv, o, gu, dn))
        router.set_layer(l, om.synth_bf16_host(SEED, tid(l, 8), (E, H), 0.02), ones)
        router.set_directory(l, np.zeros(2 * E, np.uint64), np.zeros(2 * E, np.uint64))
    lm = om.Bf16Tensor.synth(V, H, SEED, 2, 0.02)
    embed = om.Bf16Tensor.synth(V, H, SEED, 1, 0.02)
    bd = om.BatchDecode(L, V, SERVE_SEQS, max_blocks, max_blocks * 16, 1e-6, 1e6, router, lm, embed,
                        pool.ptr, lay)
    hd1 = np.ones(HD, np.float32)
    for l, (qkv, o, gu, dn) in enumerate(layers):
        bd.set_layer(l, qkv, o, gu, dn, ones, hd1, hd1)
    bd.set_final_norm(ones)
    bd.set_tables(tables)
    if args.eager:
        bd.set_eager(True)
    om.sync()
    t_build = time.time() - t_build
    tok = rng.integers(0, V, SERVE_SEQS).astype(np.uint32)
    pos = ctx.astype(np.uint32).copy()
    for _ in range(warmup):
        tok = bd.step(tok, pos)
        pos += 1
    om.sync()
    ctx_mid = pos.astype(np.int64) + steps // 2 + 1
    t0 = time.perf_counter()
    for _ in range(steps):
        tok = bd.step(tok, pos)
        pos += 1
    om.sync()
    elapsed = time.perf_counter() - t0
    _, _, _, routes = bd.read(SERVE_SEQS, routes=True)
    distinct = [len(np.unique(routes[l])) for l in range(L)]
    step_bytes = int(ctx_mid.sum() * KV_BYTES_PER_TOKEN + sum(distinct) * EXPERT_BYTES +
                     L * DENSE_BYTES_PER_LAYER + V * H * 2)
    ms = elapsed * 1e3 / steps
    tok_s = SERVE_SEQS * steps / elapsed
    gbs = step_bytes / (ms * 1e6)
    cpu = None if args.no_cpu else serve_cpu_baseline(args.cpu_threads, int(ctx_mid.mean()))
    line = {
        "metric": "Qwen3-30B-A3B FP8 batched serving decode (configuration 5): 32 sequences, tok/s",
        "value": round(tok_s, 2), "unit": "tok/s", "n_gpus": 1, "steps": steps, "warmup": warmup,
        "ms_per_step": round(ms, 3), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "fp8", "data": "synthetic random-init weights, N(0,1) bf16 KV of the drawn contexts",
        "config": {"workload": "Qwen3-30B-A3B FP8 batched decode, 32 sequences, contexts log-uniform "
                               "in [1k, 128k], bf16 KV in 16-token pages, "
                               + ("direct launches" if args.eager else "one hipGraph per step"),
                   "global_batch": SERVE_SEQS, "context_mean": int(ctx_mid.mean()),
                   "context_min": int(ctx_mid.min()), "context_max": int(ctx_mid.max()),
                   "kv_pool_GB": round(lay.pool_bytes / 1e9, 1), "parallelism": "single GPU"},
        "step_roofline": {"bound": "hbm", "algorithmic_bytes_per_step": step_bytes,
                          "achieved_GBs": round(gbs, 1), "peak": PEAK_GBS, "frac": round(gbs / PEAK_GBS, 4),
                          "distinct_experts_mean": round(float(np.mean(distinct)), 1),
                          "kv_bytes_per_step": int(ctx_mid.sum() * KV_BYTES_PER_TOKEN)},
        "cpu_baseline": cpu,
        "extra": {"build_s": round(t_build, 1), "last_tokens_head": tok[:4].tolist()}}
    if emit:
        print(json.dumps(line), flush=True)
    bd.free()
    pool.free()
    for ts in layers:
        for t in ts:
            t.free()
    router.free()
    lm.free()
    embed.free()
    return line


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=64)
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--prompt", type=int, default=512)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--eager", action="store_true",
                    help="launch the step's kernels directly instead of replaying the hipGraph "
                         "(for profilers that cannot follow graph capture)")
    ap.add_argument("--cpu-threads", type=int, default=host_cores()[1])
    ap.add_argument("--persistent", action="store_true",
                    help="decode: time the persistent form (every layer in one launch) instead of the "
                         "default six-launch chain")
    ap.add_argument("--no-other", action="store_true",
                    help="decode: skip timing the other form beside the headline")
    ap.add_argument("--other-steps", type=int, default=32)
    ap.add_argument("--workload", choices=["decode", "gemv", "paged", "moe", "serve", "prefill", "kvio", "schedule"],
                    default="decode",
                    help="decode: the bs=1 decode step (configuration 4, the headline line); "
                         "gemv: the q|k|v FP8 GEMV (configuration 1); prefill: whole-prompt prefill "
                         "time to first token; "
                         "paged: the paged-attention sweep (configuration 3); moe: the MoE block "
                         "at token batch 1 and 32 (configuration 2); serve: 32 sequences of batched "
                         "decode over long contexts (configuration 5); kvio: KV park / restore of a "
                         "fused cache in the HostPagedPoolV1 payload; schedule: the beat scheduler "
                         "serving staggered requests over the batched step")
    ap.add_argument("--serve-steps", type=int, default=128)
    ap.add_argument("--serve-warmup", type=int, default=4)
    ap.add_argument("--paged-reps", type=int, default=10)
    ap.add_argument("--paged-points", default="",
                    help="paged workload: a comma-separated subset of the sweep as SEQSxCTX, e.g. 32x32768")
    ap.add_argument("--moe-reps", type=int, default=20)
    ap.add_argument("--gemv-reps", type=int, default=200)
    ap.add_argument("--prefill-lengths", default="512,2048")
    ap.add_argument("--kvio-positions", type=int, default=32768)
    ap.add_argument("--schedule-requests", type=int, default=96)
    ap.add_argument("--schedule-prefill", action="store_true",
                    help="schedule: prompts go in through the whole-prompt prefill at join")
    ap.add_argument("--kvio-reps", type=int, default=10)
    ap.add_argument("--prefill-decode-ms", type=float, default=0.0,
                    help="bs=1 decode step time, for the token-by-token prompt time beside the prefill")
    ap.add_argument("--no-bs32", action="store_true",
                    help="decode workload: skip the 32-sequence batched figure (configuration 5)")
    ap.add_argument("--bs32-steps", type=int, default=64)
    ap.add_argument("--copy-probe", type=int, default=0, metavar="BYTES",
                    help="only run device-to-device copies of BYTES (byte-counter calibration)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: the decode step runs on a single MI355X and this build "
              "has no multi-GPU path (--gpus 1)", file=sys.stderr)
        sys.exit(2)

    import omega_amd as om

    if om.gpu_count() == 0:
        print("bench.py needs an MI355X", file=sys.stderr)
        sys.exit(3)
    if args.copy_probe:
        copy_probe(args.copy_probe)
        return
    if args.workload == "gemv":
        bench_gemv(om, args)
        return
    if args.workload == "prefill":
        bench_prefill(om, args)
        return
    if args.workload == "kvio":
        bench_kvio(om, args)
        return
    if args.workload == "schedule":
        bench_schedule(om, args)
        return
    if args.workload == "paged":
        bench_paged(om, args)
        return
    if args.workload == "moe":
        bench_moe(om, args)
        return
    if args.workload == "serve":
        bench_serve(om, args)
        return
    total = args.prompt + args.warmup + args.steps + 8
    max_pos = om.round_max_pos(total)
    model = build_model(om, max_pos)
    g = model["graph"]
    persistent = g.set_persistent(args.persistent)
    if args.eager:
        g.set_flush_each(3 if persistent else 2)
    rng = np.random.default_rng(SEED)
    prompt = rng.integers(0, V, args.prompt).tolist()
    pos = 0
    tok = prompt[0]
    t_prompt = time.perf_counter()
    for p in range(args.prompt):
        nxt, _ = g.token_id(prompt[p], pos)
        pos += 1
        tok = nxt
    t_prompt = time.perf_counter() - t_prompt
    for _ in range(args.warmup):
        tok, _ = g.token_id(tok, pos)
        pos += 1
    om.sync()
    t0 = time.perf_counter()
    generated = []
    for _ in range(args.steps):
        tok, st = g.token_id(tok, pos)
        generated.append(tok)
        pos += 1
    om.sync()
    elapsed = time.perf_counter() - t0
    launches = int(st.launches)
    ms_per_step = elapsed * 1e3 / args.steps
    tok_s = args.steps / elapsed

    # Where the time goes, on further (untimed) decode steps:
    # (1) dispatch durations of the timed form's launches, each timed by its own dispatch
    #     (hipExtLaunchKernel events on the library stream; the same launches made directly):
    #     the roofline of the dominant launch and per-kind GB/s;
    # (2) the chain's graph spans per kind: its replayed graph with an event-record node before the
    #     first kernel and after every kernel (each kernel's share of the replayed token, its launch
    #     gap included; the event nodes' own cost is subtracted);
    # (3) the other form of the same step: tok/s, and for the persistent form its own stage stamps
    #     (the GPU's constant clock at the end of each stage of each layer).
    stamp_tokens = 8
    ctx_mid = pos + stamp_tokens
    margins = []

    def top2(lg):
        t2 = np.sort(lg)[-2:]
        margins.append(float(t2[1] - t2[0]))

    def kind_names(n):
        if persistent:
            return ["decode_layers", "lm_head"]
        return launch_names(g.stamps()[1])[:n]

    dispatch = {}
    g.set_stamps(True)
    g.set_flush_each(3 if persistent else 2)
    for _ in range(stamp_tokens):
        tok, _ = g.token_id(tok, pos)
        pos += 1
        top2(g.read(logits=True)[2])
        ns = g.kernel_ns()
        for n_, dt in zip(kind_names(len(ns)), ns):
            dispatch.setdefault(n_, []).append(int(dt))
    g.set_flush_each(0)
    layer_bytes = sum(algorithmic_bytes(k, ctx_mid) for k in LAYER_KINDS)
    kernels = {}
    for name, ds in dispatch.items():
        n_launch = len(ds) // stamp_tokens
        d_us = float(np.mean(ds)) / 1e3
        b = L * layer_bytes if name == "decode_layers" else algorithmic_bytes(name, ctx_mid)
        kernels[name] = dict(launches_per_token=n_launch, dispatch_us=round(d_us, 3),
                             dispatch_us_per_token=round(d_us * n_launch, 2),
                             algorithmic_bytes=b, dispatch_gbs=round(b / (d_us * 1e3), 1))
    spans = {}
    g.set_persistent(False)
    for _ in range(4):
        tok, _ = g.token_id(tok, pos)
        pos += 1
        top2(g.read(logits=True)[2])
        st_, kinds_ = g.stamps()
        for k, dt in zip(launch_names(kinds_), g.kernel_ns()):
            spans.setdefault(k, []).append(int(dt))
        spans.setdefault("_token", []).append(int(st_[-1]))
        n_nodes = len(kinds_) + 1
    g.set_stamps(False)
    dom = max(kernels, key=lambda k: kernels[k]["dispatch_us_per_token"])
    dk = kernels[dom]
    achieved = dk["algorithmic_bytes"] / (dk["dispatch_us"] * 1e3)
    step_bytes = L * layer_bytes + algorithmic_bytes("lm_head", ctx_mid)
    # (3) the other form
    other = None
    if not args.no_other:
        want_p = not persistent
        got_p = g.set_persistent(want_p)
        if got_p == want_p:
            for _ in range(4):
                tok, _ = g.token_id(tok, pos)
                pos += 1
            om.sync()
            t1 = time.perf_counter()
            for _ in range(args.other_steps):
                tok, _ = g.token_id(tok, pos)
                pos += 1
            om.sync()
            o_ms = (time.perf_counter() - t1) * 1e3 / args.other_steps
            other = {"form": "persistent" if got_p else "chain", "tok_s": round(1e3 / o_ms, 2),
                     "ms_per_step": round(o_ms, 4),
                     "step_roofline_frac": round(step_bytes / (o_ms * 1e6) / PEAK_GBS, 4)}
        g.set_persistent(persistent)
    # the chain's spans less the event-record nodes' own cost (the stamped token's time beyond the
    # plain chain token's, spread over its nodes)
    chain_ms = ms_per_step if not persistent else (other["ms_per_step"] if other else None)
    ev_ns = 0.0
    if chain_ms:
        ev_ns = max(0.0, float(np.mean(spans["_token"])) - chain_ms * 1e6) / n_nodes
    chain_graph_us = {k: round(max(0.0, float(np.mean(v)) - ev_ns) / 1e3, 3)
                      for k, v in spans.items() if k != "_token"}
    stage_us = None
    if g.set_persistent(True):
        g.set_stage_stamps(True)
        sts = []
        for _ in range(4):
            tok, _ = g.token_id(tok, pos)
            pos += 1
            ends = g.stage_ns().astype(np.int64).reshape(-1)
            sts.append((ends - np.concatenate([[0], ends[:-1]])).reshape(L, 5))
        g.set_stage_stamps(False)
        st_all = np.stack(sts)
        per = st_all[:, 1:, :].mean(axis=(0, 1)) / 1e3  # layer 0 also holds the launch's start
        stage_us = {n: round(float(v), 3) for n, v in zip(["input", "qkv_attn", "o_proj", "route", "moe"], per)}
        stage_us["layer"] = round(float(per.sum()), 3)
    g.set_persistent(persistent)

    cpu = None if args.no_cpu else cpu_baseline(args.cpu_threads, ctx_mid)
    line = {
        "metric": METRIC,
        "value": round(tok_s, 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp8",
        "data": "synthetic (random-init weights from the seeded counter-based generator, "
                "seeded 512-token prompt)",
        "config": {
            "workload": "Qwen3-30B-A3B FP8 decode step, bs=1, "
                        + ("direct kernel launches" if args.eager else "one hipGraph per token")
                        + (" (every layer in one persistent launch)" if persistent
                           else f" ({(launches - 1) // L} launches per layer)")
                        + f", {args.prompt}-token prompt then greedy decode",
            "layers": L, "hidden": H, "q_heads": QH, "kv_heads": KVH, "head_dim": HD,
            "experts": E, "top_k": TOPK, "moe_intermediate": I, "vocab": V,
            "global_batch": 1, "context": f"{args.prompt + args.warmup}-{pos}",
            "parallelism": "single GPU",
        },
        "roofline": {
            "bound": "hbm",
            "kernel": dom,
            "duration_us": dk["dispatch_us"],
            "achieved": round(achieved, 1),
            "peak": PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / PEAK_GBS, 4),
            "traffic": committed_traffic(dom),
        },
        "step_roofline": {
            "algorithmic_bytes_per_token": step_bytes,
            "achieved_GBs": round(step_bytes / (ms_per_step * 1e6), 1),
            "frac": round(step_bytes / (ms_per_step * 1e6) / PEAK_GBS, 4),
            "launches_per_token": launches,
            "form": "persistent (every layer in one launch) + lm_head" if persistent
                    else f"chain of {(launches - 1) // L} launches per layer + lm_head",
            "chain_graph_span_us": chain_graph_us,
        },
        "kernels": kernels,
        "other_form": other,
        "persistent_stage_us_per_layer": stage_us,
        "top2_margins": {"tokens": len(margins), "min": round(min(margins), 5),
                         "median": round(float(np.median(margins)), 5),
                         "values": [round(m_, 5) for m_ in margins]},
        "cpu_baseline": cpu,
        "extra": {"model_build_s": round(model["seconds"], 1),
                  "prompt_s": round(t_prompt, 2),
                  "generated_head": generated[:8]},
    }
    if not args.no_bs32:
        # the metric's bs32 figure: configuration 5's batched step over the same architecture
        # (its own model build; the bs=1 model is freed first)
        model["model"].free()
        sargs = argparse.Namespace(serve_steps=args.bs32_steps, serve_warmup=4, no_cpu=True, eager=False,
                                   cpu_threads=args.cpu_threads)
        sl = bench_serve(om, sargs, emit=False)
        line["bs32"] = {"metric": sl["metric"], "value": sl["value"], "unit": "tok/s",
                        "ms_per_step": sl["ms_per_step"], "steps": sl["steps"],
                        "context_mean": sl["config"]["context_mean"],
                        "step_roofline_frac": sl["step_roofline"]["frac"],
                        "achieved_GBs": sl["step_roofline"]["achieved_GBs"],
                        "workload": sl["config"]["workload"]}
    print(json.dumps(line))


if __name__ == "__main__":
    main()
