// The whole decode token as one hipGraph launch (omega_gpu_decode_graph_*).
//
// Contract: crates/aien-omega-dgraph/src/lib.rs:16-30 — per layer: input norm, q|k|v FP8, decode
// attention, o FP8, residual add, router, gate|up FP8, SwiGLU, down FP8, combine; then the final
// norm, the bf16 lm_head and the argmax; the greedy token is the lowest index of the max. The
// residual row stays on the device for the whole token.
//
// MI355X shape: six launches per layer. Every cross-workgroup reduction sits at a launch
// boundary, except the attention's split merge: eight split workgroups of each kv head wait
// (bounded) for that head's splits to flag their partials, all splits being resident at once:
//   1. q|k|v GEMV, the input RMSNorm in its prologue (layer 0 in token-id mode also gathers the
//      embedding row and publishes it as the residual),
//   2. matrix-core flash-decoding over the cache: q/k RMSNorm + RoPE in its prologue, this
//      token's K/V append, one wavefront per (16-token page range, kv head), then the split merge,
//   3. o GEMV whose epilogue adds into the residual row,
//   4. router logits (post-attention RMSNorm, exact f64 dot products),
//   5. gate|up GEMV of the 8 routed experts: the top-8 ranking in its prologue (one wavefront
//      per workgroup ranks, LDS shares), SwiGLU in its epilogue,
//   6. down GEMV: one workgroup = the 8 experts' wavefronts for 8 rows, combined in slot order
//      in LDS and added into the residual,
// then the lm_head with the final RMSNorm in its prologue and the argmax folded in: 6L + 1
// launches built once as a hipGraph (kernel nodes in a chain) and replayed per token. The
// position, token id and epoch live in device memory, so one graph serves every token.
#include <cstddef>
#include <cstdio>
#include <vector>

#include "kernels.hpp"
#include "route.hpp"
#include "rows.hpp"
#include "runtime.hpp"

namespace omega {
RouterArgs router_args(const OmegaGpuRouter *r, uint32_t layer, const float *x, float eps,
                       int norm_topk, float out_scale);
uint32_t router_layers(const OmegaGpuRouter *r);
uint32_t router_rows(const OmegaGpuRouter *r);
DattnArgs cache_dattn(OmegaGpuDecodeAttnCache *c, uint32_t layer, float eps, const float *qkv,
                      float *part);
uint32_t cache_layers(const OmegaGpuDecodeAttnCache *c);
uint32_t cache_max_pos(const OmegaGpuDecodeAttnCache *c);

constexpr uint32_t kHidden = 2048, kInter = 768, kExperts = 128;
constexpr uint32_t kLaunchesPerLayer = 6;

// ---------------------------------------------------------------- gate|up + SwiGLU
struct GateUpArgs {
    const uint8_t *w = nullptr;  // [128][1536][2048] e4m3, gate rows then up rows
    const float *s = nullptr;    // [128][12][16]
    const float *logits = nullptr;
    int norm_topk = 1;
    int route_mutant = 0;
    const float *xn = nullptr;   // post-attention normed row x'
    float *act = nullptr;        // [8][768]
    // workgroup 0 publishes the route: ids / weights for the down launch, the group tables
    // from the layer's directories, and the per-layer log
    uint32_t *ids = nullptr;
    float *weights = nullptr;
    const uint64_t *dir_gu = nullptr, *dir_dn = nullptr;
    uint64_t *tab_gu = nullptr, *tab_dn = nullptr;
    uint32_t *log_ids = nullptr;
    float *log_w = nullptr;
    const uint32_t *forced = nullptr;  // parity tests: the layer's 8 expert ids instead of the ranking
    int graph_mutant = 0;        // 1: gate and up swapped; 4: every routed id e computed and
                                 // reported as (e + 1) % 128; 5: expert block scales read as 1
};

constexpr uint32_t kGuPairs = 2;  // gate/up row pairs per wavefront

// The logits and the normed row come in as leading scalar arguments (preloaded into SGPRs), so
// the two loads every workgroup waits on go out at the first instruction. FORCED: the parity
// tests' forced routes (a.forced set), decided at launch.
template <bool FORCED>
__global__ __launch_bounds__(256) void k_gate_up(const float *logits, const float *xn, const GateUpArgs a) {
    using S = Fp8Slab<kHidden, kGuPairs>;
    constexpr int P = S::P;
    __shared__ uint32_t sh_id[kTopK];
    __shared__ float sh_w[kTopK];
    __shared__ __align__(16) float xs[kHidden];  // the normed row, staged once per workgroup
    const uint32_t lane = lane_id(), wid = threadIdx.x >> 6;
    const uint32_t item = blockIdx.x * 4 + wid;
    const uint32_t slot = item / (kInter / kGuPairs), j0 = (item % (kInter / kGuPairs)) * kGuPairs;
    static_assert(kHidden == 8 * 256, "two float4 of the row per thread");
    const f32x4 xt0 = *as_global_f32x4(xn + 4 * threadIdx.x);
    const f32x4 xt1 = *as_global_f32x4(xn + 1024 + 4 * threadIdx.x);
    // wavefront 0 ranks the logits for the workgroup (its logits load goes out right behind the
    // row's: the row is written to LDS after the ranking). Workgroup 0 ranks all 8 slots and
    // weighs them (it publishes the route); every other workgroup needs its own slot's id only,
    // which the first slot + 1 rounds decide, so its stream starts that many rounds in.
    if (wid == 0) {
        // parity tests: the layer's forced ids, unless its row asks for the ranking
        const bool forced = FORCED && *as_global_u32(a.forced) != OMEGA_GPU_DGRAPH_RANK;
        if (forced || blockIdx.x == 0) {
            Route r;
            if (forced) route_forced(logits, a.forced, r);
            else route_topk<kExperts / 64>(logits, 0, a.norm_topk, a.route_mutant, r);
            if (lane == 0) {
#pragma unroll
                for (int s = 0; s < kTopK; ++s) {
                    sh_id[s] = a.graph_mutant == 4 ? (r.id[s] + 1) % kExperts : r.id[s];
                    sh_w[s] = r.w[s];
                }
            }
        } else {
            const uint32_t id = route_slot_id<kExperts / 64>(logits, slot + 1, a.route_mutant);
            if (lane == 0) sh_id[slot] = a.graph_mutant == 4 ? (id + 1) % kExperts : id;
        }
    }
    reinterpret_cast<f32x4 *>(xs)[threadIdx.x] = xt0;
    reinterpret_cast<f32x4 *>(xs)[threadIdx.x + 256] = xt1;
    __syncthreads();  // route and staged row complete
    float xr[P][16];
    S::load_x_lds(xs, lane, xr);
    const uint32_t e = sh_id[slot];
    const uint8_t *we = a.w + (size_t)e * 2 * kInter * kHidden;
    const float *se = a.s + (size_t)e * (2 * kInter / 128) * (kHidden / 128);
    // block scales ahead of the weight stream: waits complete in issue order
    float scg[P], scu[P];
    const int scale_mutant = a.graph_mutant == 5 ? 1 : 0;
    S::load_scales(se + (size_t)(j0 >> 7) * (kHidden / 128), lane, 1.0f, scale_mutant, scg);
    S::load_scales(se + (size_t)((kInter + j0) >> 7) * (kHidden / 128), lane, 1.0f, scale_mutant, scu);
    S gate, up;
    gate.load(we + (size_t)j0 * kHidden, lane);
    up.load(we + (size_t)(kInter + j0) * kHidden, lane);
    __builtin_amdgcn_sched_barrier(0);
    // workgroup 0 publishes the route once its own weight stream is in flight
    if (blockIdx.x == 0 && wid == 0 && lane < (uint32_t)kTopK) {
        const uint32_t id = sh_id[lane];
        const float wt = sh_w[lane];
        a.ids[lane] = id;
        a.weights[lane] = wt;
        if (a.log_ids) a.log_ids[lane] = id;
        if (a.log_w) a.log_w[lane] = wt;
        if (a.tab_gu) {  // the group tables (the MoE block's one-token form has none)
            const uint64_t gu0 = a.dir_gu[2 * id], gu1 = a.dir_gu[2 * id + 1];
            const uint64_t dn0 = a.dir_dn[2 * id], dn1 = a.dir_dn[2 * id + 1];
            a.tab_gu[2 * lane] = gu0;
            a.tab_gu[2 * lane + 1] = gu1;
            a.tab_dn[2 * lane] = dn0;
            a.tab_dn[2 * lane + 1] = dn1;
        }
    }
    float ag[kGuPairs], au[kGuPairs];
#pragma unroll
    for (uint32_t j = 0; j < kGuPairs; ++j) ag[j] = au[j] = 0.f;
    gate.dot(xr, scg, ag, lane);
    up.dot(xr, scu, au, lane);
    float gv = reduce_rows(ag, lane);
    float uv = reduce_rows(au, lane);
    if (a.graph_mutant == 1) {
        const float t = gv;
        gv = uv;
        uv = t;
    }
    if (lane < kGuPairs) a.act[slot * kInter + j0 + lane] = gv / (1.0f + expf(-gv)) * uv;
}

// ---------------------------------------------------------------- down + combine + residual
struct DownArgs {
    const uint8_t *w = nullptr;  // [128][2048][768] e4m3
    const float *s = nullptr;    // [128][16][6]
    const uint32_t *ids = nullptr;
    const float *weights = nullptr;
    const float *act = nullptr;  // [8][768]
    const float *xin = nullptr;  // residual read [2048] (null: the combine alone is written)
    float *x = nullptr;          // out [2048]: xin + the combine (the decode step: xin == x)
    int graph_mutant = 0;        // 2: slot 7 dropped from the combine; 5: block scales read as 1
};

constexpr uint32_t kDnRows = 8;  // output rows per workgroup (one wavefront per slot)

// The route, the SwiGLU rows, the route weights, the residual row and the test mutant come in as
// leading scalar arguments (preloaded into SGPRs): the route load, which every weight address
// waits on, goes out at the first instruction.
__global__ __launch_bounds__(512) void k_down(const uint32_t *ids, const float *act, const float *weights,
                                              const float *xin, int graph_mutant, const DownArgs a) {
    using S = Fp8Slab<kInter, kDnRows>;
    constexpr int P = S::P;
    __shared__ float red[kTopK][kDnRows];
    const uint32_t lane = lane_id();
    const uint32_t slot = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // scalar: e by s_load
    const uint32_t row0 = blockIdx.x * kDnRows;
    // every small load goes ahead of the weight stream (the route weights and the residual rows
    // of the epilogue included), so no round trip is left after the dot
    const uint32_t e = ids[slot];
    float xr[P][16];
    S::load_x(act + slot * kInter, lane, xr);
    const float wraw = *as_global_f32(weights + (lane & (kTopK - 1)));  // lane s: slot s's weight
    const float xres = xin ? *as_global_f32(xin + row0 + (lane & (kDnRows - 1))) : 0.f;
    float sc[P];
    S::load_scales(a.s + ((size_t)e * (kHidden / 128) + (row0 >> 7)) * (kInter / 128), lane, 1.0f,
                   graph_mutant == 5 ? 1 : 0, sc);
    S slab;
    slab.load(a.w + ((size_t)e * kHidden + row0) * kInter, lane);
    __builtin_amdgcn_sched_barrier(0);
    // graph mutant 2 drops slot 7 from the combine (decided here, not after the dot)
    const float wgt = (graph_mutant == 2 && (lane & (kTopK - 1)) == 7) ? 0.f : wraw;
    float acc[kDnRows];
#pragma unroll
    for (uint32_t j = 0; j < kDnRows; ++j) acc[j] = 0.f;
    slab.dot(xr, sc, acc, lane);
    const float v = reduce_rows(acc, lane);
    if (lane < kDnRows) red[slot][lane] = v;
    __syncthreads();
    if (threadIdx.x < kDnRows) {
        float moe = 0.f;
#pragma unroll
        for (int s = 0; s < kTopK; ++s) {
            moe += readlane_f32(wgt, s) * red[s][threadIdx.x];
        }
        a.x[row0 + threadIdx.x] = xres + moe;
    }
}

static hipError_t launch_gate_up(const GateUpArgs &gu, hipStream_t st) {
    const dim3 grid(kTopK * (kInter / kGuPairs) / 4);
    if (gu.forced) OMEGA_LAUNCH(k_gate_up<true>, grid, dim3(256), 0, st, gu.logits, gu.xn, gu);
    else OMEGA_LAUNCH(k_gate_up<false>, grid, dim3(256), 0, st, gu.logits, gu.xn, gu);
    return hipGetLastError();
}

static hipError_t launch_down(const DownArgs &dn, hipStream_t st) {
    OMEGA_LAUNCH(k_down, dim3(kHidden / kDnRows), dim3(512), 0, st, dn.ids, dn.act, dn.weights, dn.xin,
                 dn.graph_mutant, dn);
    return hipGetLastError();
}

// The MoE block of one token as the decode step runs it: router logits and x' (ra), then gate|up
// with the top-8 ranking in its prologue and SwiGLU, then down with the slot-order combine into
// out (plus resid when given). ra.ids / ra.weights receive the route; act holds [8][768].
hipError_t launch_moe_one_token(const RouterArgs &ra, const uint8_t *gu_w, const float *gu_s,
                                const uint8_t *dn_w, const float *dn_s, float *act, const float *resid,
                                float *out, hipStream_t st) {
    hipError_t e = launch_router_logits(ra, st);
    if (e != hipSuccess) return e;
    GateUpArgs gu;
    gu.w = gu_w;
    gu.s = gu_s;
    gu.logits = ra.logits;
    gu.norm_topk = ra.norm_topk;
    gu.route_mutant = ra.mutant;
    gu.xn = ra.xout;
    gu.act = act;
    gu.ids = ra.ids;
    gu.weights = ra.weights;
    e = launch_gate_up(gu, st);
    if (e != hipSuccess) return e;
    DownArgs dn;
    dn.w = dn_w;
    dn.s = dn_s;
    dn.ids = ra.ids;
    dn.weights = ra.weights;
    dn.act = act;
    dn.xin = resid;
    dn.x = out;
    return launch_down(dn, st);
}

}  // namespace omega

using namespace omega;

namespace {

struct GLayer {
    const OmegaGpuFp8Tensor *qkv = nullptr, *o = nullptr, *gu = nullptr, *dn = nullptr;
    float *input_norm = nullptr;  // device [2048]
};

const char *kKindNames[12] = {"norm", "qkv", "attn", "o_proj", "res_add", "router",
                              "gate_up", "swiglu", "down", "combine_norm", "lm_head", "argmax"};

// device words the host writes before every token: pos, token id, the token's epoch (the
// attention's split flags), then the words it reads back: the count of attention waits that ran
// out, the argmax slots
struct GraphIo {
    uint32_t pos;
    uint32_t tok;
    uint32_t epoch;
    uint32_t merge_err;
    uint32_t pad[12];
    unsigned long long argmax[kArgmaxSlots];
};

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
    float *x = nullptr, *qkv = nullptr, *attn = nullptr, *part = nullptr, *act = nullptr;
    float *hidden = nullptr, *logits = nullptr;
    GraphIo *io = nullptr;
    uint32_t *route_log = nullptr;  // [layers][8] routed ids of the last token
    uint32_t *forced = nullptr;     // [layers][8] forced expert ids (parity tests), when force_on
    uint32_t *flags = nullptr;      // [4][64] the attention's split flags (epochs)
    uint32_t epoch = 0;             // of the last token
    bool sync_stale = false;        // a token failed after its epoch was taken: clear the flags
    bool force_on = false;
    float *route_log_w = nullptr;   // [layers][8] their weights
    GraphIo *pin = nullptr;         // pinned host twin of io
    const OmegaGpuBf16Tensor *embed = nullptr;  // optional: device embedding (token-id entry)
    // graphs: [0] x from the host, [1] x gathered from the embedding by token id; [2], [3] the
    // same with an event-record node before the first kernel and after every kernel (stamps);
    // [4], [5] the persistent form (one launch of every layer, then the lm_head) of [0], [1]
    static constexpr int kVariants = 6;
    hipGraph_t graph_v[kVariants] = {};
    hipGraphExec_t exec_v[kVariants] = {};
    bool dirty_v[kVariants] = {true, true, true, true, true, true};
    void mark_dirty() {
        for (bool &d : dirty_v) d = true;
        players_dirty = true;
    }
    // the persistent form: per-layer descriptors, words (f32 | epoch) per (layer, stage), the
    // attention's split flags per layer, stage stamps
    bool persistent = false;        // chosen at create when the device holds the whole launch
    bool players_dirty = true;
    PLayer *players = nullptr;      // [layers]
    uint64_t *words = nullptr;
    size_t words_bytes = 0;
    uint32_t *pflags = nullptr;     // [layers][4][kDattnSplits]
    unsigned long long *pstamps = nullptr;  // [1 + layers * kTokStampsPerLayer]
    bool stage_stamps = false;
    bool stage_valid = false;
    std::vector<unsigned long long> stage_host;
    bool stamps_graph = false;  // the last stamped token ran as the stamped graph
    int mutant = 0;
    bool stamps = false;
    int flush_each = 0;  // 1: synchronise after every launch; 2: direct launches, no graph
    std::vector<uint8_t> kinds;
    std::vector<hipEvent_t> events;   // one before the first launch, one after each launch
    std::vector<hipEvent_t> kevents;  // start / stop pair per launch, recorded by the dispatch
    bool stamps_valid = false;
    // test-only layer trace: the traced layers and one record of kTrWords floats per layer
    std::vector<uint32_t> trace_layers;
    float *trace = nullptr;
};

namespace {

// one traced layer's record: the residual entering the layer, the o projection's output, the
// residual after the attention (x'), the router's normed row, the MoE output (no residual), the
// residual leaving the layer, then the routed ids (u32) and weights in slot order
constexpr size_t kTrX = 0, kTrAttn = 2048, kTrMid = 4096, kTrPost = 6144, kTrMoe = 8192,
                 kTrOut = 10240, kTrIds = 12288, kTrW = 12296, kTrWords = 12304;
constexpr uint32_t kTrMaxLayers = 8;

// the trace record of layer l, or null (not traced, or a graph is being recorded)
float *trace_record(const OmegaGpuDecodeGraph *g, uint32_t l) {
    if (!g->trace || graph_recorder()) return nullptr;
    for (size_t i = 0; i < g->trace_layers.size(); ++i)
        if (g->trace_layers[i] == l) return g->trace + i * kTrWords;
    return nullptr;
}

// Enqueues one token's kernels on `st`. With `ev` (stamps), records an event before the first
// launch and after each one.
int enqueue_token(OmegaGpuDecodeGraph *g, hipStream_t st, std::vector<uint8_t> &kinds,
                  std::vector<hipEvent_t> *ev, std::vector<hipEvent_t> *kev, bool sync_each,
                  bool gather) {
    kinds.clear();
    const float eps = g->cfg.eps;
    size_t e_i = 0, k_i = 0;
    // the next launch records its own start / stop (stamp mode)
    auto arm = [&]() {
        if (kev && k_i + 1 < kev->size()) {
            launch_stamp().start = (*kev)[k_i];
            launch_stamp().stop = (*kev)[k_i + 1];
            k_i += 2;
        }
    };
    // an event after the launch: a stream record, or an event-record node while a graph is built
    auto record = [&](hipEvent_t e) -> hipError_t {
        return graph_recorder() ? record_event_node(e) : hipEventRecord(e, st);
    };
    auto mark = [&](uint8_t kind) -> hipError_t {
        kinds.push_back(kind);
        if (ev && e_i < ev->size()) {
            hipError_t r = record((*ev)[e_i++]);
            if (r != hipSuccess) return r;
        }
        if (sync_each) return hipStreamSynchronize(st);
        return hipSuccess;
    };
    if (ev && !ev->empty()) {
        OMEGA_HIP(F_SESSION, record((*ev)[0]));
        e_i = 1;
    }
    const uint32_t *pos_dev = &g->io->pos;
    for (uint32_t l = 0; l < g->cfg.layers; ++l) {
        const GLayer &L = g->layers[l];
        // 1. q|k|v with the input norm prologue
        Fp8RowsArgs a;
        a.w = L.qkv->w;
        a.s = L.qkv->s;
        a.n = L.qkv->n;
        a.k = L.qkv->k;
        a.groups = 1;
        a.x = g->x;
        a.norm_w = L.input_norm;
        a.eps = eps;
        a.y = g->qkv;
        int xsrc = XS_NORM;
        if (gather && l == 0) {
            xsrc = XS_EMBED_NORM;
            a.embed = g->embed->w;
            a.embed_tok = &g->io->tok;
            a.embed_rows = g->embed->n;
            a.x_out = g->x;
        }
        float *tr = trace_record(g, l);
        auto trace_copy = [&](size_t at, const void *src, size_t bytes) -> hipError_t {
            return hipMemcpyAsync(tr + at, src, bytes, hipMemcpyDeviceToDevice, st);
        };
        arm();
        OMEGA_HIP(F_SESSION, launch_fp8_rows(a, EPI_STORE, xsrc, st));
        OMEGA_HIP(F_SESSION, mark(OMEGA_GPU_DGRAPH_K_QKV));
        if (tr) OMEGA_HIP(F_SESSION, trace_copy(kTrX, g->x, kHidden * 4));
        // 2. attention (q/k norm + RoPE, K/V append) with the split merge in the same launch
        DattnArgs da = cache_dattn(g->cache, l, eps, g->qkv, g->part);
        da.splits = kGraphSplits;
        da.pos_dev = pos_dev;
        da.flags = g->flags;
        da.errc = &g->io->merge_err;
        da.epoch_dev = &g->io->epoch;
        da.out = g->attn;
        da.out_scale = g->mutant == 3 ? 2.0f : 1.0f;
        if (g->mutant == 9) da.merge_spins = 0;  // every merge gives up at once (counted)
        arm();
        OMEGA_HIP(F_SESSION, launch_dattn(da, st));
        OMEGA_HIP(F_SESSION, mark(OMEGA_GPU_DGRAPH_K_ATTN));
        // 4. o projection into the residual
        Fp8RowsArgs o;
        o.w = L.o->w;
        o.s = L.o->s;
        o.n = L.o->n;
        o.k = L.o->k;
        o.groups = 1;
        o.x = g->attn;
        o.y = g->x;
        arm();
        OMEGA_HIP(F_SESSION, launch_fp8_rows(o, EPI_RESID, XS_F32, st));
        OMEGA_HIP(F_SESSION, mark(OMEGA_GPU_DGRAPH_K_O_PROJ));
        if (tr) {
            // the same launch shape stored on its own: the o projection's output as added
            Fp8RowsArgs o2 = o;
            o2.y = tr + kTrAttn;
            OMEGA_HIP(F_SESSION, launch_fp8_rows(o2, EPI_STORE, XS_F32, st));
            OMEGA_HIP(F_SESSION, trace_copy(kTrMid, g->x, kHidden * 4));
        }
        // 5. router logits and x'
        RouterArgs ra = router_args(g->router, l, g->x, eps, g->cfg.norm_topk, 1.0f);
        arm();
        OMEGA_HIP(F_SESSION, launch_router_logits(ra, st));
        OMEGA_HIP(F_SESSION, mark(OMEGA_GPU_DGRAPH_K_ROUTER));
        if (tr) OMEGA_HIP(F_SESSION, trace_copy(kTrPost, ra.xout, kHidden * 4));
        // 6. ranking + gate|up of the 8 routed experts + SwiGLU
        GateUpArgs gu;
        gu.w = L.gu->w;
        gu.s = L.gu->s;
        gu.logits = ra.logits;
        gu.norm_topk = ra.norm_topk;
        gu.route_mutant = ra.mutant;
        gu.xn = ra.xout;
        gu.act = g->act;
        gu.ids = ra.ids;
        gu.weights = ra.weights;
        gu.dir_gu = ra.dir_gu;
        gu.dir_dn = ra.dir_dn;
        gu.tab_gu = ra.tab_gu;
        gu.tab_dn = ra.tab_dn;
        gu.log_ids = g->route_log + (size_t)l * 8;
        gu.log_w = g->route_log_w + (size_t)l * 8;
        gu.forced = g->force_on ? g->forced + (size_t)l * 8 : nullptr;
        gu.graph_mutant = g->mutant;
        arm();
        OMEGA_HIP(F_SESSION, launch_gate_up(gu, st));
        OMEGA_HIP(F_SESSION, mark(OMEGA_GPU_DGRAPH_K_GATE_UP));
        // 7. down of the 8 experts, weighted combine + residual
        DownArgs dn;
        dn.w = L.dn->w;
        dn.s = L.dn->s;
        dn.ids = ra.ids;
        dn.weights = ra.weights;
        dn.act = g->act;
        dn.xin = g->x;
        dn.x = g->x;
        dn.graph_mutant = g->mutant;
        arm();
        OMEGA_HIP(F_SESSION, launch_down(dn, st));
        OMEGA_HIP(F_SESSION, mark(OMEGA_GPU_DGRAPH_K_DOWN));
        if (tr) {
            // the combine alone (no residual read) is the sum the fused launch added
            DownArgs d2 = dn;
            d2.xin = nullptr;
            d2.x = tr + kTrMoe;
            OMEGA_HIP(F_SESSION, launch_down(d2, st));
            OMEGA_HIP(F_SESSION, trace_copy(kTrIds, ra.ids, kTopK * 4));
            OMEGA_HIP(F_SESSION, trace_copy(kTrW, ra.weights, kTopK * 4));
            OMEGA_HIP(F_SESSION, trace_copy(kTrOut, g->x, kHidden * 4));
        }
    }
    // final norm + lm_head + argmax
    Bf16RowsArgs b;
    b.w = g->lm->w;
    b.n = g->lm->n;
    b.k = g->lm->k;
    b.x = g->x;
    b.norm_w = g->final_norm;
    b.eps = eps;
    b.hidden_out = g->hidden;
    b.y = g->logits;
    b.argmax = g->io->argmax;
    arm();
    OMEGA_HIP(F_SESSION, launch_bf16_rows(b, st));
    OMEGA_HIP(F_SESSION, mark(OMEGA_GPU_DGRAPH_K_LM_HEAD));
    return OMEGA_GPU_OK;
}

// words of one (layer, stage) buffer set, carved from g->words in this order
struct WordLayout {
    size_t x, qkv, att, xn, log, xp, act, total;
};
WordLayout word_layout(uint32_t layers) {
    WordLayout w{};
    size_t o = 0;
    w.x = o;
    o += (size_t)(layers + 1) * kHidden;
    w.qkv = o;
    o += (size_t)layers * 5120;
    w.att = o;
    o += (size_t)layers * 4096;
    w.xn = o;
    o += (size_t)layers * kHidden;
    w.log = o;
    o += (size_t)layers * kExperts;
    w.xp = o;
    o += (size_t)layers * kHidden;
    w.act = o;
    o += (size_t)layers * kTopK * kInter;
    w.total = o;
    return w;
}

// the per-layer descriptors of the persistent form, rebuilt after set_layer / force_routes
int upload_players(OmegaGpuDecodeGraph *g) {
    std::vector<PLayer> h(g->cfg.layers);
    for (uint32_t l = 0; l < g->cfg.layers; ++l) {
        const GLayer &L = g->layers[l];
        RouterArgs ra = router_args(g->router, l, g->x, g->cfg.eps, g->cfg.norm_topk, 1.0f);
        DattnArgs da = cache_dattn(g->cache, l, g->cfg.eps, g->qkv, g->part);
        PLayer &p = h[l];
        p.qkv_w = L.qkv->w;
        p.qkv_s = L.qkv->s;
        p.o_w = L.o->w;
        p.o_s = L.o->s;
        p.gu_w = L.gu->w;
        p.gu_s = L.gu->s;
        p.dn_w = L.dn->w;
        p.dn_s = L.dn->s;
        p.in_norm = L.input_norm;
        p.rgate = ra.gate;
        p.rnorm = ra.norm_w;
        p.dir_gu = ra.dir_gu;
        p.dir_dn = ra.dir_dn;
        p.q_norm = da.q_norm;
        p.k_norm = da.k_norm;
        p.forced = g->force_on ? g->forced + (size_t)l * 8 : nullptr;
        p.log_ids = g->route_log + (size_t)l * 8;
        p.log_w = g->route_log_w + (size_t)l * 8;
    }
    OMEGA_HIP(F_SESSION, hipMemcpy(g->players, h.data(), h.size() * sizeof(PLayer), hipMemcpyHostToDevice));
    g->players_dirty = false;
    return OMEGA_GPU_OK;
}

// One token in the persistent form: every layer in one launch, then the final norm, lm_head and
// argmax as in the chain.
int enqueue_token_persistent(OmegaGpuDecodeGraph *g, hipStream_t st, std::vector<uint8_t> &kinds, bool gather,
                             std::vector<hipEvent_t> *kev = nullptr) {
    kinds.clear();
    size_t k_i = 0;
    // direct launches in stamp mode: each launch records its own start / stop
    auto arm = [&]() {
        if (kev && k_i + 1 < kev->size()) {
            launch_stamp().start = (*kev)[k_i];
            launch_stamp().stop = (*kev)[k_i + 1];
            k_i += 2;
        }
    };
    const WordLayout wl = word_layout(g->cfg.layers);
    RouterArgs ra = router_args(g->router, 0, g->x, g->cfg.eps, g->cfg.norm_topk, 1.0f);
    DattnArgs da = cache_dattn(g->cache, 0, g->cfg.eps, g->qkv, g->part);
    PTokenArgs a;
    a.layers = g->players;
    a.nlayers = g->cfg.layers;
    a.io = &g->io->pos;
    a.errc = &g->io->merge_err;
    a.abort = &g->io->pad[0];
    a.embed = gather ? g->embed->w : nullptr;
    a.embed_rows = gather ? g->embed->n : 0;
    a.x = g->x;
    a.pool = da.pool;
    a.g = da.g;
    a.max_pos = da.max_pos;
    a.rope_cos = da.rope_cos;
    a.rope_sin = da.rope_sin;
    a.eps = g->cfg.eps;
    a.norm_topk = g->cfg.norm_topk;
    a.w_x = g->words + wl.x;
    a.w_qkv = g->words + wl.qkv;
    a.w_att = g->words + wl.att;
    a.w_xn = g->words + wl.xn;
    a.w_log = g->words + wl.log;
    a.w_xp = g->words + wl.xp;
    a.w_act = g->words + wl.act;
    a.part = g->part;
    a.aflags = g->pflags;
    a.r_xout = ra.xout;
    a.r_logits = ra.logits;
    a.r_weights = ra.weights;
    a.r_ids = ra.ids;
    a.r_tab_gu = ra.tab_gu;
    a.r_tab_dn = ra.tab_dn;
    a.graph_mutant = g->mutant;
    // a wait runs out after 10 ms of the 100 MHz clock; test mutant 9: at once (every wait that
    // is not already satisfied gives up, the token is reported failed, every kernel exits)
    a.wait_ticks = g->mutant == 9 ? 0 : 1000000;
    a.dattn_mutant = da.mutant;
    a.router_mutant = ra.mutant;
    a.tiles_per_split = da.tiles_per_split;
    a.attn_out_scale = g->mutant == 3 ? 2.0f : 1.0f;
    a.stamps = g->stage_stamps ? g->pstamps : nullptr;
    arm();
    OMEGA_HIP(F_SESSION, launch_token(a, st));
    kinds.push_back(OMEGA_GPU_DGRAPH_K_QKV);
    Bf16RowsArgs b;
    b.w = g->lm->w;
    b.n = g->lm->n;
    b.k = g->lm->k;
    b.x = g->x;
    b.norm_w = g->final_norm;
    b.eps = g->cfg.eps;
    b.hidden_out = g->hidden;
    b.y = g->logits;
    b.argmax = g->io->argmax;
    arm();
    OMEGA_HIP(F_SESSION, launch_bf16_rows(b, st));
    kinds.push_back(OMEGA_GPU_DGRAPH_K_LM_HEAD);
    return OMEGA_GPU_OK;
}

int ensure_events(std::vector<hipEvent_t> &v, size_t n) {
    while (v.size() < n) {
        hipEvent_t e;
        OMEGA_HIP(F_SESSION, hipEventCreate(&e));
        v.push_back(e);
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
    // the graph is built node by node (no stream capture): a chain of the token's kernels, with
    // event-record nodes between them in the stamped variants
    std::vector<hipEvent_t> *ev = nullptr;
    if (v >= 2) {
        const int rc = ensure_events(g->events, (size_t)kLaunchesPerLayer * g->cfg.layers + 2);
        if (rc) return rc;
        ev = &g->events;
    }
    if (v >= 4 && g->players_dirty) {
        const int rc = upload_players(g);
        if (rc) return rc;
    }
    const int rc = build_graph(F_SESSION, "decode graph", &g->graph_v[v], &g->exec_v[v], [&]() {
        if (v >= 4) return enqueue_token_persistent(g, c->stream, g->kinds, (v & 1) == 1);
        return enqueue_token(g, c->stream, g->kinds, ev, nullptr, false, (v & 1) == 1);
    });
    if (rc) return rc;
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
    if (router_rows(r) != kExperts) {
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
    hipError_t e = hipSuccess;
    auto M = [&](void **p, size_t bytes) {
        if (e == hipSuccess) e = dev_malloc(p, bytes);
        if (e == hipSuccess) e = hipMemset(*p, 0, bytes);
    };
    M((void **)&g->x, kHidden * 4);
    M((void **)&g->qkv, 5120 * 4);
    M((void **)&g->attn, 4096 * 4);
    M((void **)&g->part, (size_t)32 * kDattnSplits * kPartStride * 4);
    M((void **)&g->act, kTopK * kInter * 4);
    M((void **)&g->hidden, kHidden * 4);
    M((void **)&g->logits, (size_t)lm->n * 4);
    M((void **)&g->io, sizeof(GraphIo));
    M((void **)&g->final_norm, kHidden * 4);
    M((void **)&g->route_log, (size_t)cfg->layers * 8 * 4);
    M((void **)&g->route_log_w, (size_t)cfg->layers * 8 * 4);
    M((void **)&g->forced, (size_t)cfg->layers * 8 * 4);
    M((void **)&g->flags, 4 * kDattnSplits * 4);
    for (auto &L : g->layers) M((void **)&L.input_norm, kHidden * 4);
    // the persistent form's state (words start at epoch 0, which no token uses)
    g->words_bytes = word_layout(cfg->layers).total * 8;
    M((void **)&g->players, (size_t)cfg->layers * sizeof(PLayer));
    M((void **)&g->words, g->words_bytes);
    M((void **)&g->pflags, (size_t)cfg->layers * 4 * kDattnSplits * 4);
    M((void **)&g->pstamps, (size_t)(1 + cfg->layers * kTokStampsPerLayer) * 8);
    if (e == hipSuccess) e = host_malloc((void **)&g->pin, sizeof(GraphIo) + kHidden * 4, hipHostMallocDefault);
    if (e == hipSuccess) e = hipDeviceSynchronize();
    if (e != hipSuccess) {
        set_error(F_SESSION, "decode graph create: %s", hipGetErrorString(e));
        omega_gpu_decode_graph_free(g);
        return OMEGA_GPU_CHIP_FAIL;
    }
    memset(g->pin, 0, sizeof(GraphIo));
    // the chain is the default form: on the MI355X it measured faster (1.65 against 1.86 ms a
    // token); omega_gpu_decode_graph_set_persistent switches
    g->persistent = false;
    *out = g;
    return OMEGA_GPU_OK;
}

void omega_gpu_decode_graph_free(OmegaGpuDecodeGraph *g) {
    if (!g) return;
    std::lock_guard<std::recursive_mutex> lk(big_lock());
    Ctx *c = ctx(F_SESSION);
    if (c) (void)hipStreamSynchronize(c->stream);
    for (int v = 0; v < OmegaGpuDecodeGraph::kVariants; ++v) {
        if (g->exec_v[v]) (void)hipGraphExecDestroy(g->exec_v[v]);
        if (g->graph_v[v]) (void)hipGraphDestroy(g->graph_v[v]);
    }
    for (hipEvent_t e : g->events) (void)hipEventDestroy(e);
    for (hipEvent_t e : g->kevents) (void)hipEventDestroy(e);
    void *ps[] = {g->x, g->qkv, g->attn, g->part, g->act, g->hidden, g->logits, g->io,
                  g->final_norm, g->route_log, g->route_log_w, g->forced, g->flags,
                  g->players, g->words, g->pflags, g->pstamps, g->trace};
    for (void *p : ps)
        if (p) (void)dev_free(p);
    for (auto &L : g->layers)
        if (L.input_norm) (void)dev_free(L.input_norm);
    if (g->pin) (void)host_free(g->pin);
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
    OMEGA_HIP(F_SESSION, hipMemcpy(L.input_norm, input_norm, kHidden * 4, hipMemcpyHostToDevice));
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
    OMEGA_HIP(F_SESSION, hipMemcpy(g->final_norm, final_norm, kHidden * 4, hipMemcpyHostToDevice));
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
    // graph variant: x from the host or by token id; stamped (event nodes between kernels) or not;
    // the persistent form unless stamps or direct launches ask for the chain
    // a layer trace runs the chain as direct launches
    const bool tracing = g->trace != nullptr;
    const bool pers = g->persistent && !tracing && ((!g->stamps && g->flush_each == 0) || g->flush_each == 3);
    const int v = pers ? 4 + (x_embed ? 0 : 1) : (x_embed ? 0 : 1) + (g->stamps ? 2 : 0);
    g->stamps_valid = false;
    g->stage_valid = false;
    uint64_t record_ns = 0;
    // flush_each runs the same kernels as direct launches (with stamps: events between them and
    // each launch timed by its dispatch); otherwise the graph is replayed
    const bool eager = g->flush_each != 0 || tracing;
    if (!eager && (g->dirty_v[v] || !g->exec_v[v])) {
        const uint64_t r0 = now_ns();
        int rc = rebuild(g, c, v);
        if (rc) return rc;
        record_ns = now_ns() - r0;
    }
    // pos, token id and cleared argmax slots in one copy; the embedding row in another
    GraphIo *pin = g->pin;
    memset(pin, 0, sizeof(GraphIo));
    pin->pos = pos;
    pin->tok = token_in;
    // The attention's split flags hold epoch * 64 + layer. Before the epoch wraps, or after a token
    // that failed once its epoch was taken, the flags are cleared and the epochs start again from 1.
    // The persistent form's words and split flags hold the epoch itself, so they are cleared
    // whenever the epochs start again.
    if (++g->epoch >= (1u << 26) || g->sync_stale) {
        OMEGA_HIP(F_SESSION, hipMemsetAsync(g->flags, 0, 4 * kDattnSplits * 4, c->stream));
        OMEGA_HIP(F_SESSION, hipMemsetAsync(g->words, 0, g->words_bytes, c->stream));
        OMEGA_HIP(F_SESSION, hipMemsetAsync(g->pflags, 0, (size_t)g->cfg.layers * 4 * kDattnSplits * 4, c->stream));
        g->epoch = 1;
    }
    g->sync_stale = true;  // until this token has completed
    pin->epoch = g->epoch;
    float *xin = reinterpret_cast<float *>(pin + 1);
    OMEGA_HIP(F_SESSION, hipMemcpyAsync(g->io, pin, sizeof(GraphIo), hipMemcpyHostToDevice, c->stream));
    if (x_embed) {
        memcpy(xin, x_embed, kHidden * 4);
        OMEGA_HIP(F_SESSION, hipMemcpyAsync(g->x, xin, kHidden * 4, hipMemcpyHostToDevice, c->stream));
    }
    OMEGA_HIP(F_SESSION, hipEventRecord(c->ev0, c->stream));
    if (eager && pers) {
        // the persistent form as direct launches (flush_each 3), each timed by its dispatch in
        // stamp mode
        std::vector<hipEvent_t> *kev = nullptr;
        if (g->stamps) {
            int rc = ensure_events(g->kevents, 4);
            if (!rc) rc = ensure_events(g->events, 3);
            if (rc) return rc;
            kev = &g->kevents;
        }
        if (g->players_dirty) {
            const int rc = upload_players(g);
            if (rc) return rc;
        }
        int rc = enqueue_token_persistent(g, c->stream, g->kinds, (v & 1) == 1, kev);
        if (rc) return rc;
    } else if (eager) {
        std::vector<hipEvent_t> *ev = nullptr, *kev = nullptr;
        if (g->stamps) {
            const size_t launches = (size_t)kLaunchesPerLayer * g->cfg.layers + 1;
            int rc = ensure_events(g->events, launches + 1);
            if (!rc) rc = ensure_events(g->kevents, 2 * launches);
            if (rc) return rc;
            ev = &g->events;
            kev = &g->kevents;
        }
        int rc = enqueue_token(g, c->stream, g->kinds, ev, kev, g->flush_each == 1, (v & 1) == 1);
        if (rc) return rc;
    } else {
        OMEGA_HIP(F_SESSION, hipGraphLaunch(g->exec_v[v], c->stream));
    }
    const uint32_t launches = (uint32_t)g->kinds.size();
    OMEGA_HIP(F_SESSION, hipEventRecord(c->ev1, c->stream));
    OMEGA_HIP(F_SESSION, hipMemcpyAsync(&pin->merge_err, &g->io->merge_err,
                                        sizeof(GraphIo) - offsetof(GraphIo, merge_err), hipMemcpyDeviceToHost,
                                        c->stream));
    OMEGA_HIP(F_SESSION, hipStreamSynchronize(c->stream));
    if (pin->merge_err) {
        set_error(F_SESSION, "decode graph: %u in-launch waits ran out (%s form)", pin->merge_err,
                  pers ? "persistent" : "chain");
        return OMEGA_GPU_CHIP_FAIL;
    }
    g->sync_stale = false;
    if (pers && g->stage_stamps) {
        g->stage_host.resize(1 + (size_t)g->cfg.layers * kTokStampsPerLayer);
        OMEGA_HIP(F_SESSION, hipMemcpy(g->stage_host.data(), g->pstamps, g->stage_host.size() * 8,
                                       hipMemcpyDeviceToHost));
        g->stage_valid = true;
    }
    *token = argmax_from_slots(pin->argmax);
    g->stamps_valid = g->stamps;
    g->stamps_graph = g->stamps && !eager;
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
    g->dirty_v[1] = g->dirty_v[3] = true;
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
    if (x) OMEGA_HIP(F_SESSION, hipMemcpy(x, g->x, kHidden * 4, hipMemcpyDeviceToHost));
    if (hidden) OMEGA_HIP(F_SESSION, hipMemcpy(hidden, g->hidden, kHidden * 4, hipMemcpyDeviceToHost));
    if (logits) OMEGA_HIP(F_SESSION, hipMemcpy(logits, g->logits, (size_t)g->cfg.vocab * 4, hipMemcpyDeviceToHost));
    return OMEGA_GPU_OK;
}

void omega_gpu_decode_graph_set_flush_each(OmegaGpuDecodeGraph *g, int on) {
    if (!g) return;
    std::lock_guard<std::recursive_mutex> lk(big_lock());
    // 1 (any non-zero but 2): submit and wait after every launch (the batching comparison);
    // 2: direct launches without the graph and without waits (profilers that cannot follow
    // graph capture)
    // 3: the persistent form as direct launches (each dispatch timed in stamp mode); the chain
    // where the persistent form is off
    g->flush_each = on == 2 ? 2 : on == 3 ? (g->persistent ? 3 : 2) : (on != 0 ? 1 : 0);
}

int omega_gpu_decode_graph_test_set_trace(OmegaGpuDecodeGraph *g, const uint32_t *layers, uint32_t n) {
    std::lock_guard<std::recursive_mutex> lk(big_lock());
    clear_error(F_SESSION);
    if (!g || (n && !layers) || n > kTrMaxLayers) {
        set_error(F_SESSION, "decode graph trace: a graph and at most %u layers", kTrMaxLayers);
        return OMEGA_GPU_BAD_ARGS;
    }
    for (uint32_t i = 0; i < n; ++i) {
        bool repeat = false;
        for (uint32_t j = 0; j < i; ++j) repeat |= layers[j] == layers[i];
        if (layers[i] >= g->cfg.layers || repeat) {
            set_error(F_SESSION, "decode graph trace: layer %u outside 0..%u or repeated", layers[i],
                      g->cfg.layers - 1);
            return OMEGA_GPU_BAD_ARGS;
        }
    }
    Ctx *c = ctx(F_SESSION);
    if (!c) return OMEGA_GPU_CHIP_FAIL;
    OMEGA_HIP(F_SESSION, hipStreamSynchronize(c->stream));
    if (g->trace) OMEGA_HIP(F_SESSION, dev_free(g->trace));
    g->trace = nullptr;
    g->trace_layers.assign(layers, layers + n);
    if (n) {
        OMEGA_HIP(F_SESSION, dev_malloc(&g->trace, (size_t)n * kTrWords * 4));
        OMEGA_HIP(F_SESSION, hipMemset(g->trace, 0, (size_t)n * kTrWords * 4));
    }
    return OMEGA_GPU_OK;
}

int omega_gpu_decode_graph_test_read_trace(OmegaGpuDecodeGraph *g, uint32_t i, float *x_in,
                                           float *attn_proj, float *x_mid, float *post,
                                           uint32_t *experts, float *weights, float *moe_out,
                                           float *x_out) {
    std::lock_guard<std::recursive_mutex> lk(big_lock());
    clear_error(F_SESSION);
    if (!g || !g->trace || i >= g->trace_layers.size()) {
        set_error(F_SESSION, "decode graph trace read: no trace record %u", i);
        return OMEGA_GPU_BAD_ARGS;
    }
    Ctx *c = ctx(F_SESSION);
    if (!c) return OMEGA_GPU_CHIP_FAIL;
    std::vector<float> rec(kTrWords);
    OMEGA_HIP(F_SESSION, hipStreamSynchronize(c->stream));
    OMEGA_HIP(F_SESSION, hipMemcpy(rec.data(), g->trace + (size_t)i * kTrWords, kTrWords * 4,
                                   hipMemcpyDeviceToHost));
    const struct {
        void *dst;
        size_t at, n;
    } parts[] = {{x_in, kTrX, kHidden},     {attn_proj, kTrAttn, kHidden}, {x_mid, kTrMid, kHidden},
                 {post, kTrPost, kHidden},  {moe_out, kTrMoe, kHidden},    {x_out, kTrOut, kHidden},
                 {experts, kTrIds, kTopK},  {weights, kTrW, kTopK}};
    for (const auto &p : parts)
        if (p.dst) memcpy(p.dst, rec.data() + p.at, p.n * 4);
    return OMEGA_GPU_OK;
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
    // one event before the first launch, then one after each launch
    const uint32_t n = (uint32_t)g->kinds.size();
    if (cap < n + 1) {
        set_error(F_SESSION, "decode graph stamps: capacity %u < %u", cap, n + 1);
        return OMEGA_GPU_TOO_LARGE;
    }
    stamps[0] = 0;
    for (uint32_t i = 1; i <= n; ++i) {
        float ms = 0.f;
        hipError_t e = hipEventElapsedTime(&ms, g->events[0], g->events[i]);
        if (e != hipSuccess) {
            set_error(F_SESSION, "decode graph stamps: %s", hipGetErrorString(e));
            return OMEGA_GPU_CHIP_FAIL;
        }
        stamps[i] = (uint64_t)((double)ms * 1e6);
    }
    for (uint32_t i = 0; i < n; ++i) kinds[i] = g->kinds[i];
    return (int)n;
}

int omega_gpu_decode_graph_kernel_ns(const OmegaGpuDecodeGraph *g, uint64_t *ns, uint32_t cap) {
    std::lock_guard<std::recursive_mutex> lk(big_lock());
    clear_error(F_SESSION);
    if (!g || !ns) return OMEGA_GPU_BAD_ARGS;
    if (!g->stamps || !g->stamps_valid) {
        set_error(F_SESSION, "decode graph kernel_ns: off, or no token since stamps were switched on");
        return OMEGA_GPU_BAD_ARGS;
    }
    const uint32_t n = (uint32_t)g->kinds.size();
    if (cap < n || (!g->stamps_graph && g->kevents.size() < 2 * (size_t)n) || g->events.size() < (size_t)n + 1) {
        set_error(F_SESSION, "decode graph kernel_ns: capacity %u < %u", cap, n);
        return OMEGA_GPU_TOO_LARGE;
    }
    for (uint32_t i = 0; i < n; ++i) {
        // graph replay: the span between the event nodes around launch i (its launch gap and its
        // run in the replayed graph); direct launches: the dispatch's own start and end
        float ms = 0.f;
        hipError_t e = g->stamps_graph ? hipEventElapsedTime(&ms, g->events[i], g->events[i + 1])
                                       : hipEventElapsedTime(&ms, g->kevents[2 * i], g->kevents[2 * i + 1]);
        if (e != hipSuccess) {
            set_error(F_SESSION, "decode graph kernel_ns: %s", hipGetErrorString(e));
            return OMEGA_GPU_CHIP_FAIL;
        }
        ns[i] = (uint64_t)((double)ms * 1e6);
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

int omega_gpu_decode_graph_test_force_routes(OmegaGpuDecodeGraph *g, const uint32_t *ids) {
    std::lock_guard<std::recursive_mutex> lk(big_lock());
    clear_error(F_SESSION);
    if (!g) return OMEGA_GPU_BAD_ARGS;
    if (ids) {
        for (uint32_t l = 0; l < g->cfg.layers; ++l) {
            if (ids[l * 8] == OMEGA_GPU_DGRAPH_RANK) continue;  // this layer ranks its own logits
            for (uint32_t i = l * 8; i < l * 8 + 8; ++i)
                if (ids[i] >= kExperts) {
                    set_error(F_SESSION, "decode graph force_routes: expert id %u >= %u", ids[i], kExperts);
                    return OMEGA_GPU_BAD_ARGS;
                }
        }
        Ctx *c = ctx(F_SESSION);
        if (!c) return OMEGA_GPU_CHIP_FAIL;
        OMEGA_HIP(F_SESSION, hipStreamSynchronize(c->stream));
        OMEGA_HIP(F_SESSION, hipMemcpy(g->forced, ids, (size_t)g->cfg.layers * 8 * 4, hipMemcpyHostToDevice));
    }
    if (g->force_on != (ids != nullptr)) g->mark_dirty();
    g->force_on = ids != nullptr;
    return OMEGA_GPU_OK;
}

const char *omega_gpu_decode_graph_kind_name(uint8_t kind) {
    return kind < 12 ? kKindNames[kind] : "?";
}

int omega_gpu_decode_graph_set_persistent(OmegaGpuDecodeGraph *g, int on) {
    std::lock_guard<std::recursive_mutex> lk(big_lock());
    clear_error(F_SESSION);
    if (!g) return OMEGA_GPU_BAD_ARGS;
    int dev = 0;
    const bool want = on != 0 && hipGetDevice(&dev) == hipSuccess && token_fits(dev);
    g->persistent = want;
    return want ? 1 : 0;
}

void omega_gpu_decode_graph_set_stage_stamps(OmegaGpuDecodeGraph *g, int on) {
    if (!g) return;
    std::lock_guard<std::recursive_mutex> lk(big_lock());
    if (g->stage_stamps != (on != 0)) g->dirty_v[4] = g->dirty_v[5] = true;
    g->stage_stamps = on != 0;
    g->stage_valid = false;
}

int omega_gpu_decode_graph_stage_ns(const OmegaGpuDecodeGraph *g, uint64_t *ns, uint32_t cap) {
    std::lock_guard<std::recursive_mutex> lk(big_lock());
    clear_error(F_SESSION);
    if (!g || !ns) return OMEGA_GPU_BAD_ARGS;
    if (!g->stage_valid) {
        set_error(F_SESSION, "decode graph stage_ns: stage stamps off, or the last token ran as the chain");
        return OMEGA_GPU_BAD_ARGS;
    }
    const uint32_t n = g->cfg.layers * kTokStampsPerLayer;
    if (cap < n) {
        set_error(F_SESSION, "decode graph stage_ns: capacity %u < %u", cap, n);
        return OMEGA_GPU_TOO_LARGE;
    }
    // the constant clock runs at 100 MHz: 10 ns a tick
    const unsigned long long t0 = g->stage_host[0];
    for (uint32_t i = 0; i < n; ++i) ns[i] = (uint64_t)(g->stage_host[1 + i] - t0) * 10u;
    return (int)n;
}

}  // extern "C"
