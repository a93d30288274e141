// MoE router for gfx950 (RMSNorm, router logits, softmax, top-k, renormalised weights, the
// normed row and both grouped-GEMV group tables) and the omega_gpu_router_* entry points.
//
// Contract: crates/aien-omega-router/src/lib.rs:16-28. Host oracle: FakeRouter::route
// (crates/aien-inference-abi/src/qwen3_moe_omega.rs:1943-1998) and MoeBatchPlan::from_logits
// (moe_plan.rs:86-171).
//
// Two launches: k_router_logits gives one gate row to each wavefront (bf16, 4 KiB, the normed
// row's phases in registers — each lane normalises with the f64 sum of squares over the whole
// row, rows.hpp). Each logit accumulates the exact f32 products in f64 and rounds once, so its
// value does not depend on the summation order and equals the CPU oracle's. Workgroup 0 also
// writes x' * out_scale. k_router_topk ranks the logits on one wavefront (route.hpp) and fills
// the ids, weights and group tables. The decode graph runs the ranking inside its gate|up
// kernel instead.
#include <cmath>
#include <vector>

#include "kernels.hpp"
#include "route.hpp"
#include "rows.hpp"
#include "runtime.hpp"

namespace omega {

constexpr uint32_t kRouterHidden = 2048;

// x, the norm weights and the gate rows come in as leading scalar arguments (preloaded into
// SGPRs), so their loads go out at the first instruction. One wavefront per workgroup: each gate
// row, and the residual row and norm weights it needs (16 KiB), arrive on a CU of their own
// instead of four rows' worth through one CU's load path (measured 24 us a token faster).
// Workgroup 0 also writes x'.
__global__ __launch_bounds__(64) void k_router_logits(const float *x, const float *norm_w, const uint16_t *gate,
                                                      const RouterArgs a) {
    using S = Bf16Slab<kRouterHidden, 1>;
    constexpr int P = S::P;
    const uint32_t lane = lane_id(), wid = 0;
    const uint32_t row = blockIdx.x;
    const uint32_t rows = a.experts + a.shared;
    float xr[P][8], nw[P][8];
    S::load_x(x, lane, xr);
    S::load_x(norm_w, lane, nw);
    S slab;
    if (row < rows) slab.load(gate + (size_t)row * kRouterHidden, lane);
    const float scale = rms_scale(phases_sumsq(xr), kRouterHidden, a.eps);
#pragma unroll
    for (int ph = 0; ph < P; ++ph)
#pragma unroll
        for (int i = 0; i < 8; ++i) xr[ph][i] = xr[ph][i] * scale * (a.mutant == 1 ? 1.0f : nw[ph][i]);
    if (blockIdx.x == 0 && wid == 0) {
#pragma unroll
        for (int ph = 0; ph < P; ++ph) {
            float *o = a.xout + S::col(ph, lane);
#pragma unroll
            for (int i = 0; i < 8; ++i) o[i] = xr[ph][i] * a.out_scale;
        }
    }
    if (row >= rows) return;
    double acc = 0.0;
#pragma unroll
    for (int c = 0; c < S::CH; ++c) {
        const u32x4 w = slab.v[c];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            acc += (double)bf16_lo(w[q]) * (double)xr[c][2 * q];
            acc += (double)bf16_hi(w[q]) * (double)xr[c][2 * q + 1];
        }
    }
    acc = wave_sum_f64(acc);
    if (lane == 0) a.logits[row] = (float)acc;
}

__global__ __launch_bounds__(64) void k_router_topk(const RouterArgs a) {
    Route r;
    if (a.experts == 256) route_topk<4>(a.logits, a.shared, a.norm_topk, a.mutant, r);
    else route_topk<2>(a.logits, a.shared, a.norm_topk, a.mutant, r);
    const uint32_t lane = lane_id();
    const uint32_t slots = kTopK + (a.shared ? 1 : 0);
#pragma unroll
    for (uint32_t s = 0; s < kTopK + 1; ++s) {
        if (lane != s || s >= slots) continue;
        const uint32_t id = r.id[s];
        a.ids[s] = id;
        a.weights[s] = r.w[s];
        if (a.route_log) a.route_log[s] = id;
        if (a.route_log_w) a.route_log_w[s] = r.w[s];
        const uint32_t did = (a.mutant == 3 && s < (uint32_t)kTopK) ? (id ^ 1u) : id;
        a.tab_gu[2 * s] = a.dir_gu[2 * did];
        a.tab_gu[2 * s + 1] = a.dir_gu[2 * did + 1];
        a.tab_dn[2 * s] = a.dir_dn[2 * did];
        a.tab_dn[2 * s + 1] = a.dir_dn[2 * did + 1];
    }
}

hipError_t launch_router_logits(const RouterArgs &a, hipStream_t st) {
    const uint32_t rows = a.experts + a.shared;
    OMEGA_LAUNCH(k_router_logits, dim3(rows), dim3(64), 0, st, a.x, a.norm_w, a.gate, a);
    return hipGetLastError();
}

hipError_t launch_router_topk(const RouterArgs &a, hipStream_t st) {
    OMEGA_LAUNCH(k_router_topk, dim3(1), dim3(64), 0, st, a);
    return hipGetLastError();
}

}  // namespace omega

struct OmegaGpuRouter {
    uint32_t layers = 0, experts = 128, shared = 0, rows = 128, slots = 8;
    uint16_t *gate = nullptr;       // [layers][rows][2048]
    float *norm = nullptr;          // [layers][2048]
    uint64_t *dir_gu = nullptr;     // [layers][rows][2]
    uint64_t *dir_dn = nullptr;
    // launch buffers (fixed addresses for the router's life)
    float *xin = nullptr, *xout = nullptr, *logits = nullptr, *weights = nullptr;
    uint32_t *ids = nullptr;
    uint64_t *tab_gu = nullptr, *tab_dn = nullptr;
};

using namespace omega;

namespace omega {
// for the decode graph: the device buffers and per-layer tensors of a router
RouterArgs router_args(const OmegaGpuRouter *r, uint32_t layer, const float *x, float eps,
                       int norm_topk, float out_scale) {
    RouterArgs a;
    a.x = x;
    a.gate = r->gate + (size_t)layer * r->rows * 2048;
    a.norm_w = r->norm + (size_t)layer * 2048;
    a.dir_gu = r->dir_gu + (size_t)layer * r->rows * 2;
    a.dir_dn = r->dir_dn + (size_t)layer * r->rows * 2;
    a.eps = eps;
    a.norm_topk = norm_topk;
    a.out_scale = out_scale;
    a.experts = r->experts;
    a.shared = r->shared;
    a.logits = r->logits;
    a.xout = r->xout;
    a.ids = r->ids;
    a.weights = r->weights;
    a.tab_gu = r->tab_gu;
    a.tab_dn = r->tab_dn;
    a.mutant = knobs().router_mutant;
    return a;
}
uint32_t router_layers(const OmegaGpuRouter *r) { return r->layers; }
uint32_t router_rows(const OmegaGpuRouter *r) { return r->rows; }
}  // namespace omega

extern "C" {

int omega_gpu_router_alloc_shape(uint32_t layers, uint32_t experts, uint32_t shared,
                                 OmegaGpuRouter **out) {
    std::lock_guard<std::recursive_mutex> lk(big_lock());
    clear_error(F_ROUTER);
    if (!out) return OMEGA_GPU_BAD_ARGS;
    *out = nullptr;
    if (layers == 0 || layers > 64) {
        set_error(F_ROUTER, "router layers=%u refused: 1 <= layers <= 64", layers);
        return OMEGA_GPU_BAD_ARGS;
    }
    if (!(experts == 128 || experts == 256) || shared > 1) {
        set_error(F_ROUTER, "router shape experts %u shared %u: 128 or 256, 0 or 1", experts, shared);
        return OMEGA_GPU_BAD_ARGS;
    }
    Ctx *c = ctx(F_ROUTER);
    if (!c) return OMEGA_GPU_CHIP_FAIL;
    OmegaGpuRouter *r = new OmegaGpuRouter();
    r->layers = layers;
    r->experts = experts;
    r->shared = shared;
    r->rows = experts + shared;
    r->slots = 8 + shared;
    hipError_t e = dev_malloc(&r->gate, (size_t)layers * r->rows * 2048 * 2);
    if (e == hipSuccess) e = dev_malloc(&r->norm, (size_t)layers * 2048 * 4);
    if (e == hipSuccess) e = dev_malloc(&r->dir_gu, (size_t)layers * r->rows * 16);
    if (e == hipSuccess) e = dev_malloc(&r->dir_dn, (size_t)layers * r->rows * 16);
    if (e == hipSuccess) e = dev_malloc(&r->xin, 2048 * 4);
    if (e == hipSuccess) e = dev_malloc(&r->xout, 2048 * 4);
    if (e == hipSuccess) e = dev_malloc(&r->logits, 512 * 4);
    if (e == hipSuccess) e = dev_malloc(&r->weights, 16 * 4);
    if (e == hipSuccess) e = dev_malloc(&r->ids, 16 * 4);
    if (e == hipSuccess) e = dev_malloc(&r->tab_gu, 16 * 16);
    if (e == hipSuccess) e = dev_malloc(&r->tab_dn, 16 * 16);
    if (e == hipSuccess) e = hipMemset(r->gate, 0, (size_t)layers * r->rows * 2048 * 2);
    if (e == hipSuccess) e = hipMemset(r->norm, 0, (size_t)layers * 2048 * 4);
    if (e == hipSuccess) e = hipMemset(r->dir_gu, 0, (size_t)layers * r->rows * 16);
    if (e == hipSuccess) e = hipMemset(r->dir_dn, 0, (size_t)layers * r->rows * 16);
    if (e == hipSuccess) e = hipMemset(r->xout, 0, 2048 * 4);
    if (e == hipSuccess) e = hipMemset(r->tab_gu, 0, 256);
    if (e == hipSuccess) e = hipMemset(r->tab_dn, 0, 256);
    if (e == hipSuccess) e = hipDeviceSynchronize();
    if (e != hipSuccess) {
        set_error(F_ROUTER, "router alloc: %s", hipGetErrorString(e));
        omega_gpu_router_free(r);
        return OMEGA_GPU_CHIP_FAIL;
    }
    *out = r;
    return OMEGA_GPU_OK;
}

void omega_gpu_router_free(OmegaGpuRouter *r) {
    if (!r) return;
    std::lock_guard<std::recursive_mutex> lk(big_lock());
    Ctx *c = ctx(F_ROUTER);
    if (c) (void)hipStreamSynchronize(c->stream);
    void *ps[] = {r->gate, r->norm, r->dir_gu, r->dir_dn, r->xin, r->xout, r->logits,
                  r->weights, r->ids, r->tab_gu, r->tab_dn};
    for (void *p : ps)
        if (p) (void)dev_free(p);
    delete r;
}

int omega_gpu_router_set_layer(OmegaGpuRouter *r, uint32_t layer, const uint16_t *gate_bf16,
                               const float *norm_w) {
    std::lock_guard<std::recursive_mutex> lk(big_lock());
    clear_error(F_ROUTER);
    if (!r || !gate_bf16 || !norm_w) {
        set_error(F_ROUTER, "router set_layer: NULL pointer");
        return OMEGA_GPU_BAD_ARGS;
    }
    if (layer >= r->layers) {
        set_error(F_ROUTER, "router layer %u >= layers %u", layer, r->layers);
        return OMEGA_GPU_BAD_ARGS;
    }
    OMEGA_HIP(F_ROUTER, hipMemcpy(r->gate + (size_t)layer * r->rows * 2048, gate_bf16,
                                  (size_t)r->rows * 2048 * 2, hipMemcpyHostToDevice));
    OMEGA_HIP(F_ROUTER, hipMemcpy(r->norm + (size_t)layer * 2048, norm_w, 2048 * 4,
                                  hipMemcpyHostToDevice));
    return OMEGA_GPU_OK;
}

int omega_gpu_router_set_directory(OmegaGpuRouter *r, uint32_t layer, const uint64_t *gu,
                                   const uint64_t *dn) {
    std::lock_guard<std::recursive_mutex> lk(big_lock());
    clear_error(F_ROUTER);
    if (!r || !gu || !dn) {
        set_error(F_ROUTER, "router set_directory: NULL pointer");
        return OMEGA_GPU_BAD_ARGS;
    }
    if (layer >= r->layers) {
        set_error(F_ROUTER, "router layer %u >= layers %u", layer, r->layers);
        return OMEGA_GPU_BAD_ARGS;
    }
    OMEGA_HIP(F_ROUTER, hipMemcpy(r->dir_gu + (size_t)layer * r->rows * 2, gu, (size_t)r->rows * 16,
                                  hipMemcpyHostToDevice));
    OMEGA_HIP(F_ROUTER, hipMemcpy(r->dir_dn + (size_t)layer * r->rows * 2, dn, (size_t)r->rows * 16,
                                  hipMemcpyHostToDevice));
    return OMEGA_GPU_OK;
}

int omega_gpu_router(OmegaGpuRouter *r, uint32_t layer, const float *x, float eps, int norm_topk,
                     float out_scale, uint32_t *ids, float *weights, OmegaGpuRouterInfo *info) {
    std::lock_guard<std::recursive_mutex> lk(big_lock());
    const uint64_t t0 = now_ns();
    clear_error(F_ROUTER);
    if (!r || !x || !ids || !weights) {
        set_error(F_ROUTER, "router: NULL pointer");
        return OMEGA_GPU_BAD_ARGS;
    }
    if (layer >= r->layers) {
        set_error(F_ROUTER, "router layer %u >= layers %u", layer, r->layers);
        return OMEGA_GPU_BAD_ARGS;
    }
    Ctx *c = ctx(F_ROUTER);
    if (!c) return OMEGA_GPU_CHIP_FAIL;
    if (!ensure_pinned(F_ROUTER, c, 2048 * 4 + 256)) return OMEGA_GPU_CHIP_FAIL;
    uint8_t *pin = static_cast<uint8_t *>(c->pin);
    memcpy(pin, x, 2048 * 4);
    OMEGA_HIP(F_ROUTER, hipMemcpyAsync(r->xin, pin, 2048 * 4, hipMemcpyHostToDevice, c->stream));
    RouterArgs a = router_args(r, layer, r->xin, eps, norm_topk, out_scale);
    OMEGA_HIP(F_ROUTER, hipEventRecord(c->ev0, c->stream));
    OMEGA_HIP(F_ROUTER, launch_router_logits(a, c->stream));
    OMEGA_HIP(F_ROUTER, launch_router_topk(a, c->stream));
    OMEGA_HIP(F_ROUTER, hipEventRecord(c->ev1, c->stream));
    OMEGA_HIP(F_ROUTER, hipMemcpyAsync(pin, r->ids, 16 * 4, hipMemcpyDeviceToHost, c->stream));
    OMEGA_HIP(F_ROUTER, hipMemcpyAsync(pin + 64, r->weights, 16 * 4, hipMemcpyDeviceToHost, c->stream));
    OMEGA_HIP(F_ROUTER, hipStreamSynchronize(c->stream));
    memcpy(ids, pin, r->slots * 4);
    memcpy(weights, pin + 64, r->slots * 4);
    if (info) {
        memset(info, 0, sizeof(*info));
        info->layer = layer;
        info->warps = r->rows + 1;
        info->depth = 1;
        info->threads = 256;
        info->weight_bytes = (uint64_t)r->rows * 2048 * 2;
        info->elapsed_ns = event_ns(c);
        info->call_ns = now_ns() - t0;
        info->completion_marker = 1;
        info->kernel_cache_hit = 1;
    }
    return OMEGA_GPU_OK;
}

void omega_gpu_router_device_outputs(const OmegaGpuRouter *r, uint64_t *xout_va,
                                     uint64_t *tab_gu_va, uint64_t *tab_dn_va) {
    if (!r) return;
    if (xout_va) *xout_va = (uint64_t)(uintptr_t)r->xout;
    if (tab_gu_va) *tab_gu_va = (uint64_t)(uintptr_t)r->tab_gu;
    if (tab_dn_va) *tab_dn_va = (uint64_t)(uintptr_t)r->tab_dn;
}

int omega_gpu_router_read_back(OmegaGpuRouter *r, float *xout, uint64_t *tab_gu, uint64_t *tab_dn) {
    std::lock_guard<std::recursive_mutex> lk(big_lock());
    clear_error(F_ROUTER);
    if (!r) {
        set_error(F_ROUTER, "router read_back: NULL router");
        return OMEGA_GPU_BAD_ARGS;
    }
    Ctx *c = ctx(F_ROUTER);
    if (!c) return OMEGA_GPU_CHIP_FAIL;
    OMEGA_HIP(F_ROUTER, hipStreamSynchronize(c->stream));
    if (xout) OMEGA_HIP(F_ROUTER, hipMemcpy(xout, r->xout, 2048 * 4, hipMemcpyDeviceToHost));
    if (tab_gu) OMEGA_HIP(F_ROUTER, hipMemcpy(tab_gu, r->tab_gu, (size_t)r->slots * 16, hipMemcpyDeviceToHost));
    if (tab_dn) OMEGA_HIP(F_ROUTER, hipMemcpy(tab_dn, r->tab_dn, (size_t)r->slots * 16, hipMemcpyDeviceToHost));
    return OMEGA_GPU_OK;
}

const char *omega_gpu_router_last_error(void) { return last_error(F_ROUTER); }
const char *omega_gpu_router_rc_name(int rc) { return rc_name(rc); }
void omega_gpu_router_test_set_mutant(int mutant) { knobs().router_mutant = mutant; }

}  // extern "C"
