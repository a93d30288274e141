// One-launch MoE router for gfx950 (RMSNorm, router logits, softmax, top-k, renormalised
// weights, the normed row and both grouped-GEMV group tables) and the omega_gpu_router_* entry
// points.
//
// Contract: crates/aien-omega-router/src/lib.rs:16-28. Host oracle: FakeRouter::route
// (crates/aien-inference-abi/src/qwen3_moe_omega.rs:1943-1998) and MoeBatchPlan::from_logits
// (moe_plan.rs:86-171): rank by total order descending, ties to the lower id, weight =
// exp(l - max) / sum over the selected of exp(l - max).
//
// Kernel shape: ROUTER_WGS workgroups of four wavefronts. Every workgroup normalises the row
// itself (f64 sum of squares, the RMSNorm of tensor.rs:94-110) into LDS, scores its share of the
// gate rows — each logit accumulates the exact f32 products in f64 and rounds once, so the value
// does not depend on the summation order and equals the CPU oracle's — and writes its slice of
// x' * out_scale. The last workgroup to finish runs the top-k on one wavefront with shuffles.
#include <cmath>
#include <vector>

#include "kernels.hpp"
#include "runtime.hpp"

namespace omega {

constexpr int ROUTER_WGS = 32;

__device__ __forceinline__ int32_t total_key(float f) {
    int32_t b = __float_as_int(f);
    return b < 0 ? (b ^ 0x7fffffff) : b;
}

__global__ __launch_bounds__(256) void k_router(const RouterArgs a) {
    __shared__ float post[2048];
    __shared__ double red[4];
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t H = a.hidden;
    // RMSNorm of the residual row
    double ss = 0.0;
    for (uint32_t c = tid; c < H; c += 256) ss += (double)a.x[c] * (double)a.x[c];
    for (int o = 32; o > 0; o >>= 1) ss += __shfl_xor(ss, o, 64);
    if (lane == 0) red[wave] = ss;
    __syncthreads();
    ss = (red[0] + red[1]) + (red[2] + red[3]);
    const float scale = (float)(1.0 / sqrt(ss / (double)H + (double)a.eps));
    for (uint32_t c = tid; c < H; c += 256) {
        const float wn = a.mutant == 1 ? 1.0f : a.norm_w[c];
        post[c] = a.x[c] * scale * wn;
    }
    __syncthreads();
    // this workgroup's slice of x' * out_scale
    const uint32_t per = H / gridDim.x;
    for (uint32_t c = blockIdx.x * per + tid; c < (blockIdx.x + 1) * per; c += 256)
        a.xout[c] = post[c] * a.out_scale;
    // logits of rows blockIdx.x + gridDim.x * (4 * i + wave)
    const uint32_t rows = a.experts + a.shared;
    for (uint32_t row = blockIdx.x + gridDim.x * wave; row < rows; row += gridDim.x * 4) {
        const uint16_t *g = a.gate + (size_t)row * H;
        double acc = 0.0;
        for (uint32_t c = lane * 8; c < H; c += 512) {
            const uint4 v = *reinterpret_cast<const uint4 *>(g + c);
            const uint32_t w4[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                acc += (double)__uint_as_float(w4[q] << 16) * (double)post[c + 2 * q];
                acc += (double)__uint_as_float(w4[q] & 0xffff0000u) * (double)post[c + 2 * q + 1];
            }
        }
        for (int o = 32; o > 0; o >>= 1) acc += __shfl_xor(acc, o, 64);
        if (lane == 0) a.logits[row] = (float)acc;
    }
    // the last workgroup ranks
    __threadfence();
    __shared__ uint32_t last;
    if (tid == 0) last = atomicAdd(a.counter, 1u) == gridDim.x - 1;
    __syncthreads();
    if (!last || wave != 0) return;
    __threadfence();
    const uint32_t E = a.experts;  // 128 or 256: E / 64 candidates per lane
    float lv[4];
    int32_t key[4];
    bool taken[4];
    for (int q = 0; q < 4; ++q) {
        const uint32_t id = lane + 64 * q;
        taken[q] = id >= E;
        lv[q] = taken[q] ? 0.f : __builtin_nontemporal_load(&a.logits[id]);
        key[q] = total_key(lv[q]);
    }
    uint32_t sel_id[8];
    float sel_v[8];
    for (uint32_t s = 0; s < a.top_k; ++s) {
        int32_t bk = INT32_MIN;
        uint32_t bi = 0xffffffffu;
        float bv = 0.f;
        for (int q = 0; q < 4; ++q) {
            const uint32_t id = lane + 64 * q;
            if (!taken[q] && (bi == 0xffffffffu || key[q] > bk)) {
                bk = key[q];
                bi = id;
                bv = lv[q];
            }
        }
        for (int o = 32; o > 0; o >>= 1) {
            const int32_t ok = __shfl_xor(bk, o, 64);
            const uint32_t oi = __shfl_xor(bi, o, 64);
            const float ov = __shfl_xor(bv, o, 64);
            const bool take = oi != 0xffffffffu &&
                              (bi == 0xffffffffu || ok > bk || (ok == bk && oi < bi));
            if (take) {
                bk = ok;
                bi = oi;
                bv = ov;
            }
        }
        sel_id[s] = bi;
        sel_v[s] = bv;
        const uint32_t mask_id = a.mutant == 2 ? (bi ^ 1u) : bi;
        for (int q = 0; q < 4; ++q)
            if (lane + 64 * q == mask_id) taken[q] = true;
    }
    if (lane == 0) {
        const float mx = sel_v[0];
        float p[8];
        float sum = 0.f;
        for (uint32_t s = 0; s < a.top_k; ++s) {
            p[s] = expf(sel_v[s] - mx);
            sum += p[s];
        }
        if (!a.norm_topk) {
            sum = 0.f;
            for (uint32_t id = 0; id < E; ++id) sum += expf(__builtin_nontemporal_load(&a.logits[id]) - mx);
        }
        for (uint32_t s = 0; s < a.top_k; ++s) {
            const uint32_t id = sel_id[s];
            a.ids[s] = id;
            a.weights[s] = a.mutant == 4 ? p[s] : p[s] / sum;
            if (a.route_log) a.route_log[s] = id;
            if (a.route_log_w) a.route_log_w[s] = a.weights[s];
            const uint32_t did = a.mutant == 3 ? (id ^ 1u) : id;
            a.tab_gu[2 * s] = a.dir_gu[2 * did];
            a.tab_gu[2 * s + 1] = a.dir_gu[2 * did + 1];
            a.tab_dn[2 * s] = a.dir_dn[2 * did];
            a.tab_dn[2 * s + 1] = a.dir_dn[2 * did + 1];
        }
        if (a.shared) {
            const uint32_t s = a.top_k;
            const float ls = __builtin_nontemporal_load(&a.logits[E]);
            a.ids[s] = E;
            a.weights[s] = 1.0f / (1.0f + expf(-ls));
            a.tab_gu[2 * s] = a.dir_gu[2 * E];
            a.tab_gu[2 * s + 1] = a.dir_gu[2 * E + 1];
            a.tab_dn[2 * s] = a.dir_dn[2 * E];
            a.tab_dn[2 * s + 1] = a.dir_dn[2 * E + 1];
        }
        atomicExch(a.counter, 0u);
    }
}

hipError_t launch_router(const RouterArgs &a, hipStream_t st) {
    hipLaunchKernelGGL(k_router, dim3(ROUTER_WGS), dim3(256), 0, st, a);
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
    uint32_t *ids = nullptr, *counter = nullptr;
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
    a.counter = r->counter;
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
    hipError_t e = hipMalloc(&r->gate, (size_t)layers * r->rows * 2048 * 2);
    if (e == hipSuccess) e = hipMalloc(&r->norm, (size_t)layers * 2048 * 4);
    if (e == hipSuccess) e = hipMalloc(&r->dir_gu, (size_t)layers * r->rows * 16);
    if (e == hipSuccess) e = hipMalloc(&r->dir_dn, (size_t)layers * r->rows * 16);
    if (e == hipSuccess) e = hipMalloc(&r->xin, 2048 * 4);
    if (e == hipSuccess) e = hipMalloc(&r->xout, 2048 * 4);
    if (e == hipSuccess) e = hipMalloc(&r->logits, 512 * 4);
    if (e == hipSuccess) e = hipMalloc(&r->weights, 16 * 4);
    if (e == hipSuccess) e = hipMalloc(&r->ids, 16 * 4);
    if (e == hipSuccess) e = hipMalloc(&r->counter, 4);
    if (e == hipSuccess) e = hipMalloc(&r->tab_gu, 16 * 16);
    if (e == hipSuccess) e = hipMalloc(&r->tab_dn, 16 * 16);
    if (e == hipSuccess) e = hipMemset(r->gate, 0, (size_t)layers * r->rows * 2048 * 2);
    if (e == hipSuccess) e = hipMemset(r->norm, 0, (size_t)layers * 2048 * 4);
    if (e == hipSuccess) e = hipMemset(r->dir_gu, 0, (size_t)layers * r->rows * 16);
    if (e == hipSuccess) e = hipMemset(r->dir_dn, 0, (size_t)layers * r->rows * 16);
    if (e == hipSuccess) e = hipMemset(r->xout, 0, 2048 * 4);
    if (e == hipSuccess) e = hipMemset(r->tab_gu, 0, 256);
    if (e == hipSuccess) e = hipMemset(r->tab_dn, 0, 256);
    if (e == hipSuccess) e = hipMemset(r->counter, 0, 4);
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
                  r->weights, r->ids, r->counter, r->tab_gu, r->tab_dn};
    for (void *p : ps)
        if (p) (void)hipFree(p);
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
    OMEGA_HIP(F_ROUTER, launch_router(a, c->stream));
    OMEGA_HIP(F_ROUTER, hipEventRecord(c->ev1, c->stream));
    OMEGA_HIP(F_ROUTER, hipMemcpyAsync(pin, r->ids, 16 * 4, hipMemcpyDeviceToHost, c->stream));
    OMEGA_HIP(F_ROUTER, hipMemcpyAsync(pin + 64, r->weights, 16 * 4, hipMemcpyDeviceToHost, c->stream));
    OMEGA_HIP(F_ROUTER, hipStreamSynchronize(c->stream));
    memcpy(ids, pin, r->slots * 4);
    memcpy(weights, pin + 64, r->slots * 4);
    if (info) {
        memset(info, 0, sizeof(*info));
        info->layer = layer;
        info->warps = ROUTER_WGS * 4;
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
