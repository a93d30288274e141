// The whole decode token as one hipGraph launch (omega_gpu_decode_graph_*).
//
// Contract: crates/aien-omega-dgraph/src/lib.rs:16-30 — per layer: input norm, q|k|v FP8, decode
// attention, o FP8, residual add, router, gate|up FP8, SwiGLU, down FP8, combine; then the final
// norm, the bf16 lm_head and the argmax; the greedy token is the lowest index of the max. The
// residual row stays on the device for the whole token.
//
// MI355X shape: six kernels per layer, each fusing what the reference runs as separate launches —
//   1. q|k|v GEMV with the input RMSNorm as its prologue and q/k RMSNorm + RoPE + bf16 K/V
//      append as its epilogue,
//   2. paged flash-decoding attention over the cache (identity page table),
//   3. o GEMV whose epilogue adds into the residual row,
//   4. router (RMSNorm, logits, top-8, weights, group tables),
//   5. gate|up grouped GEMV whose epilogue is the SwiGLU,
//   6. down grouped GEMV whose epilogue is the weighted combine plus the residual add,
// plus the final RMSNorm and the lm_head GEMV with a fused two-level argmax: 6 * layers + 2
// launches, captured once as a hipGraph and replayed per token. The position lives in device
// memory, so the same graph serves every token; the host copies the embedding row in and the
// token out.
#include <cstdio>
#include <vector>

#include "kernels.hpp"
#include "runtime.hpp"

namespace omega {
RouterArgs router_args(const OmegaGpuRouter *r, uint32_t layer, const float *x, float eps,
                       int norm_topk, float out_scale);
uint32_t router_layers(const OmegaGpuRouter *r);
uint32_t router_rows(const OmegaGpuRouter *r);
HeadPrep cache_prep(OmegaGpuDecodeAttnCache *c, uint32_t layer, float eps, float *q_out);
AttnArgs cache_attn(OmegaGpuDecodeAttnCache *c, uint32_t layer, const float *q);
uint32_t cache_layers(const OmegaGpuDecodeAttnCache *c);
uint32_t cache_max_pos(const OmegaGpuDecodeAttnCache *c);
}  // namespace omega

using namespace omega;

namespace {

// x = bf16 row `*tok` of the embedding (tiled bf16 layout of the GEMV tensors), widened to f32
// (Qwen3MoeOmegaWeights::embed_row, qwen3_moe_omega.rs:1108-1115: token modulo the vocabulary)
__global__ __launch_bounds__(256) void k_embed_gather(const uint16_t *w, uint32_t n, uint32_t k,
                                                      const uint32_t *tok, float *x) {
    const uint32_t r = *tok % n;
    const uint32_t ksteps = k >> 3;
    for (uint32_t c = threadIdx.x; c < k; c += 256) {
        const uint16_t b = w[((size_t)(r >> 6) * ksteps + (c >> 3)) * 512 + (r & 63) * 8 + (c & 7)];
        x[c] = __uint_as_float((uint32_t)b << 16);
    }
}

constexpr uint32_t kAttnSplits = 64;
constexpr size_t kPartialFloats = 256 * 1024;

struct GLayer {
    const OmegaGpuFp8Tensor *qkv = nullptr, *o = nullptr, *gu = nullptr, *dn = nullptr;
    float *input_norm = nullptr;  // device [2048]
};

const char *kKindNames[12] = {"norm", "qkv", "attn", "o_proj", "res_add", "router",
                              "gate_up", "swiglu", "down", "combine_norm", "lm_head", "argmax"};

}  // namespace

struct OmegaGpuDecodeGraph {
    OmegaGpuDecodeGraphConfig cfg{};
    OmegaGpuRouter *router = nullptr;
    OmegaGpuDecodeAttnCache *cache = nullptr;
    const OmegaGpuBf16Tensor *lm = nullptr;
    std::vector<GLayer> layers;
    float *final_norm = nullptr;
    bool final_set = false;
    // device state
    float *x = nullptr, *q = nullptr, *attn = nullptr, *act = nullptr, *hidden = nullptr;
    float *logits = nullptr, *partial = nullptr, *attn_part = nullptr, *arg_val = nullptr;
    uint32_t *arg_idx = nullptr, *token = nullptr, *pos = nullptr, *counters = nullptr;
    uint32_t *route_log = nullptr;  // [layers][8] routed ids of the last token
    float *route_log_w = nullptr;   // [layers][8] their weights
    // pinned io
    uint8_t *pin = nullptr;
    const OmegaGpuBf16Tensor *embed = nullptr;  // optional: device embedding (token-id entry)
    uint32_t *tok_in = nullptr;                 // device token id the gather reads
    // graphs: [0] x from the host, [1] x gathered from the embedding by token id
    hipGraph_t graph_v[2] = {nullptr, nullptr};
    hipGraphExec_t exec_v[2] = {nullptr, nullptr};
    bool dirty_v[2] = {true, true};
    void mark_dirty() { dirty_v[0] = dirty_v[1] = true; }
    int mutant = 0;
    bool stamps = false;
    int flush_each = 0;  // 1: synchronise after every launch; 2: direct launches, no graph
    std::vector<uint8_t> kinds;
    std::vector<hipEvent_t> events;
    bool stamps_valid = false;
};

namespace {

// Enqueues one token's kernels on `st`. With `ev` (stamps), records an event before the first
// launch and after each one.
int enqueue_token(OmegaGpuDecodeGraph *g, hipStream_t st, std::vector<uint8_t> &kinds,
                  std::vector<hipEvent_t> *ev, bool sync_each, bool gather) {
    kinds.clear();
    if (gather) {
        hipLaunchKernelGGL(k_embed_gather, dim3(1), dim3(256), 0, st, g->embed->w, g->embed->n,
                           g->embed->k, g->tok_in, g->x);
        OMEGA_HIP(F_SESSION, hipGetLastError());
        kinds.push_back(OMEGA_GPU_DGRAPH_K_NORM);
    }
    const float eps = g->cfg.eps;
    size_t e_i = 0;
    auto mark = [&](uint8_t kind) -> hipError_t {
        kinds.push_back(kind);
        if (ev && e_i < ev->size()) {
            hipError_t r = hipEventRecord((*ev)[e_i++], st);
            if (r != hipSuccess) return r;
        }
        if (sync_each) return hipStreamSynchronize(st);
        return hipSuccess;
    };
    if (ev && !ev->empty()) {
        OMEGA_HIP(F_SESSION, hipEventRecord((*ev)[0], st));
        e_i = 1;
    }
    for (uint32_t l = 0; l < g->cfg.layers; ++l) {
        const GLayer &L = g->layers[l];
        // 1. q|k|v with the input norm prologue and the q/k norm + RoPE + KV append epilogue
        Fp8GemvArgs a;
        a.w = L.qkv->w;
        a.s = L.qkv->s;
        a.n = L.qkv->n;
        a.k = L.qkv->k;
        a.groups = 1;
        a.x = g->x;
        a.norm_w = L.input_norm;
        a.eps = eps;
        a.partial = g->partial;
        a.counters = g->counters;
        a.prep = cache_prep(g->cache, l, eps, g->q);
        a.pos_dev = g->pos;
        int steps = fp8_gemv_plan(a, EPI_QKV);
        OMEGA_HIP(F_SESSION, launch_fp8_gemv_epi(a, steps, EPI_QKV, st));
        OMEGA_HIP(F_SESSION, mark(OMEGA_GPU_DGRAPH_K_QKV));
        // 2. attention
        AttnArgs at = cache_attn(g->cache, l, g->q);
        at.pos_dev = g->pos;
        at.splits = kAttnSplits;
        at.out_scale = g->mutant == 3 ? 2.0f : 1.0f;
        at.part = g->attn_part;
        at.counters = g->counters + 64;
        at.out = g->attn;
        OMEGA_HIP(F_SESSION, launch_attention(at, st));
        OMEGA_HIP(F_SESSION, mark(OMEGA_GPU_DGRAPH_K_ATTN));
        // 3. o projection into the residual
        Fp8GemvArgs o;
        o.w = L.o->w;
        o.s = L.o->s;
        o.n = L.o->n;
        o.k = L.o->k;
        o.groups = 1;
        o.x = g->attn;
        o.y = g->x;
        o.partial = g->partial;
        o.counters = g->counters + 128;
        steps = fp8_gemv_plan(o, EPI_RESID);
        OMEGA_HIP(F_SESSION, launch_fp8_gemv_epi(o, steps, EPI_RESID, st));
        OMEGA_HIP(F_SESSION, mark(OMEGA_GPU_DGRAPH_K_O_PROJ));
        // 4. router: x' * 2^64 and the group tables stay on the device
        RouterArgs ra = router_args(g->router, l, g->x, eps, g->cfg.norm_topk, 0x1p64f);
        ra.route_log = g->route_log + (size_t)l * 8;
        ra.route_log_w = g->route_log_w + (size_t)l * 8;
        OMEGA_HIP(F_SESSION, launch_router(ra, st));
        OMEGA_HIP(F_SESSION, mark(OMEGA_GPU_DGRAPH_K_ROUTER));
        // 5. gate|up of the 8 routed experts, SwiGLU epilogue
        Fp8GemvArgs gu;
        gu.tab = ra.tab_gu;
        gu.x = ra.xout;
        gu.x_scale = 0x1p-64f;
        gu.n = L.gu->n;
        gu.k = L.gu->k;
        gu.groups = 8;
        gu.y = g->act;
        gu.partial = g->partial;
        gu.counters = g->counters + 256;
        gu.graph_mutant = g->mutant;
        steps = fp8_gemv_plan(gu, EPI_SWIGLU);
        OMEGA_HIP(F_SESSION, launch_fp8_gemv_epi(gu, steps, EPI_SWIGLU, st));
        OMEGA_HIP(F_SESSION, mark(OMEGA_GPU_DGRAPH_K_GATE_UP));
        // 6. down of the 8 experts, weighted combine + residual epilogue
        Fp8GemvArgs dn;
        dn.tab = ra.tab_dn;
        dn.x = g->act;
        dn.x_stride = L.dn->k;
        dn.n = L.dn->n;
        dn.k = L.dn->k;
        dn.groups = 8;
        dn.y = g->x;
        dn.partial = g->partial;
        dn.counters = g->counters + 512;
        dn.comb_w = ra.weights;
        dn.graph_mutant = g->mutant;
        steps = fp8_gemv_plan(dn, EPI_COMBINE);
        OMEGA_HIP(F_SESSION, launch_fp8_gemv_epi(dn, steps, EPI_COMBINE, st));
        OMEGA_HIP(F_SESSION, mark(OMEGA_GPU_DGRAPH_K_DOWN));
    }
    // final norm + lm_head + argmax
    Bf16GemvArgs b;
    b.w = g->lm->w;
    b.x = g->x;
    b.norm_w = g->final_norm;
    b.eps = eps;
    b.n = g->lm->n;
    b.n_pad = g->lm->n_pad;
    b.k = g->lm->k;
    b.y = g->logits;
    b.hidden_out = g->hidden;
    b.arg_val = g->arg_val;
    b.arg_idx = g->arg_idx;
    b.token = g->token;
    b.counter = g->counters + 1024;
    OMEGA_HIP(F_SESSION, launch_bf16_gemv(b, st));
    // launch_bf16_gemv enqueues the norm and the GEMV: two launches
    kinds.push_back(OMEGA_GPU_DGRAPH_K_NORM);
    OMEGA_HIP(F_SESSION, mark(OMEGA_GPU_DGRAPH_K_LM_HEAD));
    return OMEGA_GPU_OK;
}

int ensure_events(OmegaGpuDecodeGraph *g, size_t n) {
    while (g->events.size() < n) {
        hipEvent_t e;
        OMEGA_HIP(F_SESSION, hipEventCreate(&e));
        g->events.push_back(e);
    }
    return OMEGA_GPU_OK;
}

int rebuild(OmegaGpuDecodeGraph *g, Ctx *c, int v) {
    if (g->exec_v[v]) {
        (void)hipGraphExecDestroy(g->exec_v[v]);
        g->exec_v[v] = nullptr;
    }
    if (g->graph_v[v]) {
        (void)hipGraphDestroy(g->graph_v[v]);
        g->graph_v[v] = nullptr;
    }
    OMEGA_HIP(F_SESSION, hipStreamBeginCapture(c->stream, hipStreamCaptureModeThreadLocal));
    int rc = enqueue_token(g, c->stream, g->kinds, nullptr, false, v == 1);
    hipGraph_t graph = nullptr;
    hipError_t e = hipStreamEndCapture(c->stream, &graph);
    if (rc) {
        if (graph) (void)hipGraphDestroy(graph);
        return rc;
    }
    if (e != hipSuccess) {
        set_error(F_SESSION, "decode graph capture: %s", hipGetErrorString(e));
        return OMEGA_GPU_CODEGEN_FAIL;
    }
    g->graph_v[v] = graph;
    e = hipGraphInstantiate(&g->exec_v[v], graph, nullptr, nullptr, 0);
    if (e != hipSuccess) {
        set_error(F_SESSION, "decode graph instantiate: %s", hipGetErrorString(e));
        return OMEGA_GPU_CODEGEN_FAIL;
    }
    g->dirty_v[v] = false;
    return OMEGA_GPU_OK;
}

bool check_fp8(const OmegaGpuFp8Tensor *t, uint32_t experts, uint32_t n, uint32_t k) {
    return t && t->experts == experts && t->n == n && t->k == k;
}

}  // namespace

extern "C" {

int omega_gpu_decode_graph_create(const OmegaGpuDecodeGraphConfig *cfg, OmegaGpuDecodeGraph **out) {
    std::lock_guard<std::recursive_mutex> lk(big_lock());
    clear_error(F_SESSION);
    if (out) *out = nullptr;
    if (!cfg || !out) {
        set_error(F_SESSION, "decode graph create: NULL pointer");
        return OMEGA_GPU_BAD_ARGS;
    }
    if (cfg->layers == 0 || cfg->layers > OMEGA_GPU_DGRAPH_MAX_LAYERS) {
        set_error(F_SESSION, "decode graph: %u layers, 1..=64 supported", cfg->layers);
        return OMEGA_GPU_BAD_ARGS;
    }
    if (cfg->vocab == 0 || cfg->vocab > OMEGA_GPU_DGRAPH_MAX_VOCAB) {
        set_error(F_SESSION, "decode graph: vocab %u outside 1..=%u", cfg->vocab,
                  OMEGA_GPU_DGRAPH_MAX_VOCAB);
        return OMEGA_GPU_BAD_ARGS;
    }
    if (!cfg->router || !cfg->attn || !cfg->lm_head) {
        set_error(F_SESSION,
                  "decode graph: the router, the KV cache and the lm_head must all be device objects");
        return OMEGA_GPU_BAD_ARGS;
    }
    OmegaGpuRouter *r = static_cast<OmegaGpuRouter *>(cfg->router);
    OmegaGpuDecodeAttnCache *ca = static_cast<OmegaGpuDecodeAttnCache *>(cfg->attn);
    const OmegaGpuBf16Tensor *lm = static_cast<const OmegaGpuBf16Tensor *>(cfg->lm_head);
    if (router_layers(r) < cfg->layers || cache_layers(ca) < cfg->layers) {
        set_error(F_SESSION, "decode graph: the router or the cache holds fewer than %u layers",
                  cfg->layers);
        return OMEGA_GPU_BAD_ARGS;
    }
    if (router_rows(r) != 128) {
        set_error(F_SESSION, "decode graph: the router must be the 128-expert shape");
        return OMEGA_GPU_BAD_ARGS;
    }
    if (lm->n != cfg->vocab || lm->k != OMEGA_GPU_DGRAPH_HIDDEN) {
        set_error(F_SESSION, "decode graph: lm_head is %u x %u, want %u x 2048", lm->n, lm->k, cfg->vocab);
        return OMEGA_GPU_BAD_ARGS;
    }
    Ctx *c = ctx(F_SESSION);
    if (!c) return OMEGA_GPU_CHIP_FAIL;
    OmegaGpuDecodeGraph *g = new OmegaGpuDecodeGraph();
    g->cfg = *cfg;
    g->router = r;
    g->cache = ca;
    g->lm = lm;
    g->layers.resize(cfg->layers);
    const uint32_t tiles = lm->n_pad / 64;
    hipError_t e = hipSuccess;
    auto M = [&](void **p, size_t bytes) {
        if (e == hipSuccess) e = hipMalloc(p, bytes);
        if (e == hipSuccess) e = hipMemset(*p, 0, bytes);
    };
    M((void **)&g->x, 2048 * 4);
    M((void **)&g->q, 4096 * 4);
    M((void **)&g->attn, 4096 * 4);
    M((void **)&g->act, 8 * 768 * 4);
    M((void **)&g->hidden, 2048 * 4);
    M((void **)&g->logits, (size_t)lm->n_pad * 4);
    M((void **)&g->partial, kPartialFloats * 4);
    M((void **)&g->attn_part, (size_t)32 * kAttnSplits * 132 * 4);
    M((void **)&g->arg_val, (size_t)tiles * 4);
    M((void **)&g->arg_idx, (size_t)tiles * 4);
    M((void **)&g->token, 4);
    M((void **)&g->pos, 8);
    M((void **)&g->counters, 2048 * 4);
    M((void **)&g->final_norm, 2048 * 4);
    M((void **)&g->route_log, (size_t)cfg->layers * 8 * 4);
    M((void **)&g->route_log_w, (size_t)cfg->layers * 8 * 4);
    for (auto &L : g->layers) M((void **)&L.input_norm, 2048 * 4);
    g->tok_in = g->pos + 1;
    if (e == hipSuccess) e = hipHostMalloc((void **)&g->pin, 2048 * 4 + 256, hipHostMallocDefault);
    if (e == hipSuccess) e = hipDeviceSynchronize();
    if (e != hipSuccess) {
        set_error(F_SESSION, "decode graph create: %s", hipGetErrorString(e));
        omega_gpu_decode_graph_free(g);
        return OMEGA_GPU_CHIP_FAIL;
    }
    *out = g;
    return OMEGA_GPU_OK;
}

void omega_gpu_decode_graph_free(OmegaGpuDecodeGraph *g) {
    if (!g) return;
    std::lock_guard<std::recursive_mutex> lk(big_lock());
    Ctx *c = ctx(F_SESSION);
    if (c) (void)hipStreamSynchronize(c->stream);
    for (int v = 0; v < 2; ++v) {
        if (g->exec_v[v]) (void)hipGraphExecDestroy(g->exec_v[v]);
        if (g->graph_v[v]) (void)hipGraphDestroy(g->graph_v[v]);
    }
    for (hipEvent_t e : g->events) (void)hipEventDestroy(e);
    void *ps[] = {g->x, g->q, g->attn, g->act, g->hidden, g->logits, g->partial, g->attn_part,
                  g->arg_val, g->arg_idx, g->token, g->pos, g->counters, g->final_norm,
                  g->route_log, g->route_log_w};
    for (void *p : ps)
        if (p) (void)hipFree(p);
    for (auto &L : g->layers)
        if (L.input_norm) (void)hipFree(L.input_norm);
    if (g->pin) (void)hipHostFree(g->pin);
    delete g;
}

int omega_gpu_decode_graph_set_layer(OmegaGpuDecodeGraph *g, uint32_t layer, const void *qkv,
                                     const void *o, const void *gate_up, const void *down,
                                     const float *input_norm) {
    std::lock_guard<std::recursive_mutex> lk(big_lock());
    clear_error(F_SESSION);
    if (!g || !input_norm) {
        set_error(F_SESSION, "decode graph set_layer: NULL pointer");
        return OMEGA_GPU_BAD_ARGS;
    }
    if (layer >= g->cfg.layers) {
        set_error(F_SESSION, "decode graph: layer %u of %u", layer, g->cfg.layers);
        return OMEGA_GPU_BAD_ARGS;
    }
    auto tq = static_cast<const OmegaGpuFp8Tensor *>(qkv);
    auto to = static_cast<const OmegaGpuFp8Tensor *>(o);
    auto tg = static_cast<const OmegaGpuFp8Tensor *>(gate_up);
    auto td = static_cast<const OmegaGpuFp8Tensor *>(down);
    if (!check_fp8(tq, 1, 5120, 2048) || !check_fp8(to, 1, 2048, 4096) ||
        !check_fp8(tg, 128, 1536, 2048) || !check_fp8(td, 128, 2048, 768)) {
        set_error(F_SESSION,
                  "decode graph layer %u: projections must be q|k|v 1x5120x2048, o 1x2048x4096, "
                  "gate|up 128x1536x2048, down 128x2048x768",
                  layer);
        return OMEGA_GPU_BAD_ARGS;
    }
    GLayer &L = g->layers[layer];
    L.qkv = tq;
    L.o = to;
    L.gu = tg;
    L.dn = td;
    OMEGA_HIP(F_SESSION, hipMemcpy(L.input_norm, input_norm, 2048 * 4, hipMemcpyHostToDevice));
    g->mark_dirty();
    return OMEGA_GPU_OK;
}

int omega_gpu_decode_graph_set_final_norm(OmegaGpuDecodeGraph *g, const float *final_norm) {
    std::lock_guard<std::recursive_mutex> lk(big_lock());
    clear_error(F_SESSION);
    if (!g || !final_norm) {
        set_error(F_SESSION, "decode graph set_final_norm: NULL pointer");
        return OMEGA_GPU_BAD_ARGS;
    }
    OMEGA_HIP(F_SESSION, hipMemcpy(g->final_norm, final_norm, 2048 * 4, hipMemcpyHostToDevice));
    g->final_set = true;
    return OMEGA_GPU_OK;
}

}  // extern "C"

namespace {

// One token: x from the host (x_embed) or gathered on the device from the embedding by token id.
int run_token(OmegaGpuDecodeGraph *g, const float *x_embed, uint32_t token_in, uint32_t pos,
              uint32_t *token, OmegaGpuDecodeGraphStats *st) {
    const uint64_t t0 = now_ns();
    for (uint32_t l = 0; l < g->cfg.layers; ++l)
        if (!g->layers[l].qkv) {
            set_error(F_SESSION, "decode graph: layer %u has no projections", l);
            return OMEGA_GPU_BAD_ARGS;
        }
    if (pos >= cache_max_pos(g->cache)) {
        set_error(F_SESSION, "decode graph: pos %u >= cache max_pos %u", pos, cache_max_pos(g->cache));
        return OMEGA_GPU_BAD_ARGS;
    }
    Ctx *c = ctx(F_SESSION);
    if (!c) return OMEGA_GPU_CHIP_FAIL;
    const int v = x_embed ? 0 : 1;
    g->stamps_valid = false;
    uint64_t record_ns = 0;
    // stamps and flush_each run the same kernels as direct launches (events between them for
    // the timeline); otherwise the captured graph is replayed
    const bool eager = g->flush_each != 0 || g->stamps;
    if (!eager && (g->dirty_v[v] || !g->exec_v[v])) {
        const uint64_t r0 = now_ns();
        int rc = rebuild(g, c, v);
        if (rc) return rc;
        record_ns = now_ns() - r0;
    }
    uint8_t *pin = g->pin;
    memcpy(pin + 2048 * 4, &pos, 4);
    memcpy(pin + 2048 * 4 + 4, &token_in, 4);
    if (x_embed) {
        memcpy(pin, x_embed, 2048 * 4);
        OMEGA_HIP(F_SESSION, hipMemcpyAsync(g->x, pin, 2048 * 4, hipMemcpyHostToDevice, c->stream));
        OMEGA_HIP(F_SESSION, hipMemcpyAsync(g->pos, pin + 2048 * 4, 4, hipMemcpyHostToDevice, c->stream));
    } else {
        // pos and the token id sit next to each other: one 8-byte copy
        OMEGA_HIP(F_SESSION, hipMemcpyAsync(g->pos, pin + 2048 * 4, 8, hipMemcpyHostToDevice, c->stream));
    }
    OMEGA_HIP(F_SESSION, hipEventRecord(c->ev0, c->stream));
    if (eager) {
        std::vector<hipEvent_t> *ev = nullptr;
        if (g->stamps) {
            int rc = ensure_events(g, 6 * (size_t)g->cfg.layers + 2);
            if (rc) return rc;
            ev = &g->events;
        }
        int rc = enqueue_token(g, c->stream, g->kinds, ev, g->flush_each == 1, v == 1);
        if (rc) return rc;
    } else {
        OMEGA_HIP(F_SESSION, hipGraphLaunch(g->exec_v[v], c->stream));
    }
    const uint32_t launches = (uint32_t)g->kinds.size();
    OMEGA_HIP(F_SESSION, hipEventRecord(c->ev1, c->stream));
    OMEGA_HIP(F_SESSION, hipMemcpyAsync(pin + 2048 * 4 + 64, g->token, 4, hipMemcpyDeviceToHost, c->stream));
    OMEGA_HIP(F_SESSION, hipStreamSynchronize(c->stream));
    memcpy(token, pin + 2048 * 4 + 64, 4);
    g->stamps_valid = g->stamps;
    if (st) {
        memset(st, 0, sizeof(*st));
        st->launches = launches;
        st->submits = eager ? launches : 1;
        st->chip_ns = event_ns(c);
        st->record_ns = record_ns;
        st->total_ns = now_ns() - t0;
        st->sems_done = launches;
    }
    return OMEGA_GPU_OK;
}

}  // namespace

extern "C" {

int omega_gpu_decode_graph_token(OmegaGpuDecodeGraph *g, const float *x_embed, uint32_t pos,
                                 uint32_t *token, OmegaGpuDecodeGraphStats *st) {
    std::lock_guard<std::recursive_mutex> lk(big_lock());
    clear_error(F_SESSION);
    if (!g || !x_embed || !token) {
        set_error(F_SESSION, "decode graph token: NULL pointer");
        return OMEGA_GPU_BAD_ARGS;
    }
    return run_token(g, x_embed, 0, pos, token, st);
}

int omega_gpu_decode_graph_set_embedding(OmegaGpuDecodeGraph *g, const void *embed_bf16) {
    std::lock_guard<std::recursive_mutex> lk(big_lock());
    clear_error(F_SESSION);
    auto e = static_cast<const OmegaGpuBf16Tensor *>(embed_bf16);
    if (!g || !e || e->k != OMEGA_GPU_DGRAPH_HIDDEN || e->n != g->cfg.vocab) {
        set_error(F_SESSION, "decode graph embedding: a [vocab][2048] bf16 tensor is required");
        return OMEGA_GPU_BAD_ARGS;
    }
    g->embed = e;
    g->dirty_v[1] = true;
    return OMEGA_GPU_OK;
}

int omega_gpu_decode_graph_token_id(OmegaGpuDecodeGraph *g, uint32_t token_in, uint32_t pos,
                                    uint32_t *token, OmegaGpuDecodeGraphStats *st) {
    std::lock_guard<std::recursive_mutex> lk(big_lock());
    clear_error(F_SESSION);
    if (!g || !token) {
        set_error(F_SESSION, "decode graph token_id: NULL pointer");
        return OMEGA_GPU_BAD_ARGS;
    }
    if (!g->embed) {
        set_error(F_SESSION, "decode graph token_id: no embedding set");
        return OMEGA_GPU_BAD_ARGS;
    }
    return run_token(g, nullptr, token_in, pos, token, st);
}

int omega_gpu_decode_graph_read(OmegaGpuDecodeGraph *g, float *x, float *hidden, float *logits) {
    std::lock_guard<std::recursive_mutex> lk(big_lock());
    clear_error(F_SESSION);
    if (!g) {
        set_error(F_SESSION, "decode graph read: NULL graph");
        return OMEGA_GPU_BAD_ARGS;
    }
    Ctx *c = ctx(F_SESSION);
    if (!c) return OMEGA_GPU_CHIP_FAIL;
    OMEGA_HIP(F_SESSION, hipStreamSynchronize(c->stream));
    if (x) OMEGA_HIP(F_SESSION, hipMemcpy(x, g->x, 2048 * 4, hipMemcpyDeviceToHost));
    if (hidden) OMEGA_HIP(F_SESSION, hipMemcpy(hidden, g->hidden, 2048 * 4, hipMemcpyDeviceToHost));
    if (logits) OMEGA_HIP(F_SESSION, hipMemcpy(logits, g->logits, (size_t)g->cfg.vocab * 4, hipMemcpyDeviceToHost));
    return OMEGA_GPU_OK;
}

void omega_gpu_decode_graph_set_flush_each(OmegaGpuDecodeGraph *g, int on) {
    if (!g) return;
    std::lock_guard<std::recursive_mutex> lk(big_lock());
    // 1 (any non-zero but 2): submit and wait after every launch (the batching comparison);
    // 2: direct launches without the graph and without waits (profilers that cannot follow
    // graph capture)
    g->flush_each = on == 2 ? 2 : (on != 0 ? 1 : 0);
}

void omega_gpu_decode_graph_test_set_mutant(OmegaGpuDecodeGraph *g, int mutant) {
    if (!g) return;
    std::lock_guard<std::recursive_mutex> lk(big_lock());
    g->mutant = mutant;
    g->mark_dirty();
}

void omega_gpu_decode_graph_set_stamps(OmegaGpuDecodeGraph *g, int on) {
    if (!g) return;
    std::lock_guard<std::recursive_mutex> lk(big_lock());
    if (g->stamps != (on != 0)) g->mark_dirty();
    g->stamps = on != 0;
    g->stamps_valid = false;
}

int omega_gpu_decode_graph_stamps(const OmegaGpuDecodeGraph *g, uint64_t *stamps, uint8_t *kinds,
                                  uint32_t cap) {
    std::lock_guard<std::recursive_mutex> lk(big_lock());
    clear_error(F_SESSION);
    if (!g || !stamps || !kinds) return OMEGA_GPU_BAD_ARGS;
    if (!g->stamps || !g->stamps_valid) {
        set_error(F_SESSION, "decode graph stamps: off, or no token since they were switched on");
        return OMEGA_GPU_BAD_ARGS;
    }
    // one event per recorded point: the first before any launch, then one per mark; the norm
    // of the lm_head tail shares the lm_head's mark
    const uint32_t marks = (uint32_t)g->events.size();
    const uint32_t n = marks - 1;
    if (cap < marks) {
        set_error(F_SESSION, "decode graph stamps: capacity %u < %u", cap, marks);
        return OMEGA_GPU_TOO_LARGE;
    }
    stamps[0] = 0;
    for (uint32_t i = 1; i < marks; ++i) {
        float ms = 0.f;
        hipError_t e = hipEventElapsedTime(&ms, g->events[0], g->events[i]);
        if (e != hipSuccess) {
            set_error(F_SESSION, "decode graph stamps: %s", hipGetErrorString(e));
            return OMEGA_GPU_CHIP_FAIL;
        }
        stamps[i] = (uint64_t)((double)ms * 1e6);
    }
    // kinds per mark (the norm launch folds into the lm_head interval)
    uint32_t j = 0;
    for (size_t i = 0; i < g->kinds.size() && j < n; ++i) {
        if (g->kinds[i] == OMEGA_GPU_DGRAPH_K_NORM) continue;
        kinds[j++] = g->kinds[i];
    }
    return (int)n;
}

int omega_gpu_decode_graph_read_routes(OmegaGpuDecodeGraph *g, uint32_t *ids, float *weights) {
    std::lock_guard<std::recursive_mutex> lk(big_lock());
    clear_error(F_SESSION);
    if (!g) return OMEGA_GPU_BAD_ARGS;
    Ctx *c = ctx(F_SESSION);
    if (!c) return OMEGA_GPU_CHIP_FAIL;
    OMEGA_HIP(F_SESSION, hipStreamSynchronize(c->stream));
    const size_t n = (size_t)g->cfg.layers * 8;
    if (ids) OMEGA_HIP(F_SESSION, hipMemcpy(ids, g->route_log, n * 4, hipMemcpyDeviceToHost));
    if (weights) OMEGA_HIP(F_SESSION, hipMemcpy(weights, g->route_log_w, n * 4, hipMemcpyDeviceToHost));
    return OMEGA_GPU_OK;
}

const char *omega_gpu_decode_graph_kind_name(uint8_t kind) {
    return kind < 12 ? kKindNames[kind] : "?";
}

}  // extern "C"
