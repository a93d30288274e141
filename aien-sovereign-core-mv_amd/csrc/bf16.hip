// bf16 streaming GEMV (the lm_head) for gfx950 with an optional fused RMSNorm prologue and a
// fused two-level argmax, plus the omega_gpu_bf16_* entry points.
//
// Contract: crates/aien-omega-bf16/src/lib.rs:15-24 — y[r] = sum_c W[r][c] * x[c] over an
// [n][k] bf16 matrix, f32, deterministic summation order. The greedy token is the lowest index
// of the max (crates/aien-omega-dgraph/src/lib.rs:347-349, tensor.rs:299-318).
//
// Kernel shape: one wavefront per 64-row tile (lane l owns row 64*tile + l) streaming 1 KiB per
// 8-column step, 16 steps in flight per batch; the activation row is wave-uniform (scalar loads).
// Each tile writes its (max, index); the last tile to finish reduces the tile maxima in order.
#include <cmath>
#include <vector>

#include "device.hpp"
#include "kernels.hpp"
#include "runtime.hpp"

namespace omega {

__device__ __forceinline__ void dot8_bf16(u32x4 v, const float *xx, float &p0, float &p1) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const uint32_t w = v[q];
        p0 = fmaf(__uint_as_float(w << 16), xx[2 * q], p0);
        p1 = fmaf(__uint_as_float(w & 0xffff0000u), xx[2 * q + 1], p1);
    }
}

// better(a, b): a strictly greater, or equal with the lower index
__device__ __forceinline__ bool better(float va, uint32_t ia, float vb, uint32_t ib) {
    return va > vb || (va == vb && ia < ib);
}

__device__ __forceinline__ void wave_argmax(float &v, uint32_t &i) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const float ov = __shfl_xor(v, o, 64);
        const uint32_t oi = __shfl_xor(i, o, 64);
        if (better(ov, oi, v, i)) {
            v = ov;
            i = oi;
        }
    }
}

// RMSNorm prologue kernel (final norm): hidden = x * scale * w with the f64 sum of squares
__global__ __launch_bounds__(256) void k_rmsnorm_row(const float *x, const float *w, float eps,
                                                     uint32_t k, float *out) {
    __shared__ double red[4];
    double ss = 0.0;
    for (uint32_t c = threadIdx.x; c < k; c += 256) ss += (double)x[c] * (double)x[c];
    for (int o = 32; o > 0; o >>= 1) ss += __shfl_xor(ss, o, 64);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
    __syncthreads();
    ss = (red[0] + red[1]) + (red[2] + red[3]);
    const float scale = (float)(1.0 / sqrt(ss / (double)k + (double)eps));
    for (uint32_t c = threadIdx.x; c < k; c += 256) out[c] = x[c] * scale * w[c];
}

constexpr int BF16_BATCH = 16;

__global__ __launch_bounds__(64) void k_bf16_gemv(const Bf16GemvArgs a) {
    const uint32_t lane = threadIdx.x;
    const uint32_t t = blockIdx.x;
    const uint32_t ksteps = a.k >> 3;
    const gu32x4 *p = as_global(a.w + (size_t)t * ksteps * 512) + lane;
    float p0 = 0.f, p1 = 0.f, p2 = 0.f, p3 = 0.f;
    for (uint32_t j = 0; j < ksteps; j += BF16_BATCH) {
        u32x4 wv[BF16_BATCH];
#pragma unroll
        for (int i = 0; i < BF16_BATCH; ++i) wv[i] = __builtin_nontemporal_load(p + (size_t)(j + i) * 64);
#pragma unroll
        for (int i = 0; i < BF16_BATCH; i += 2) {
            dot8_bf16(wv[i], a.x + (j + i) * 8, p0, p1);
            dot8_bf16(wv[i + 1], a.x + (j + i + 1) * 8, p2, p3);
        }
    }
    float v = (p0 + p1) + (p2 + p3);
    if (a.mutant == 1) v = -v;
    const uint32_t r = t * 64 + lane;
    if (r < a.n) a.y[r] = v;
    if (!a.token) return;
    float best = r < a.n ? v : -INFINITY;
    uint32_t bi = r < a.n ? r : 0xffffffffu;
    wave_argmax(best, bi);
    if (lane == 0) {
        a.arg_val[t] = best;
        a.arg_idx[t] = bi;
    }
    __threadfence();
    uint32_t last = 0;
    if (lane == 0) last = atomicAdd(a.counter, 1u) == gridDim.x - 1;
    last = __shfl(last, 0, 64);
    if (!last) return;
    __threadfence();
    const uint32_t tiles = gridDim.x;
    float bv = -INFINITY;
    uint32_t bidx = 0xffffffffu;
    for (uint32_t q = lane; q < tiles; q += 64) {
        const float qv = __builtin_nontemporal_load(&a.arg_val[q]);
        const uint32_t qi = __builtin_nontemporal_load(&a.arg_idx[q]);
        if (better(qv, qi, bv, bidx)) {
            bv = qv;
            bidx = qi;
        }
    }
    wave_argmax(bv, bidx);
    if (lane == 0) {
        *a.token = bidx;
        atomicExch(a.counter, 0u);
    }
}

hipError_t launch_bf16_gemv(const Bf16GemvArgs &a, hipStream_t st) {
    Bf16GemvArgs b = a;
    if (a.norm_w) {
        hipLaunchKernelGGL(k_rmsnorm_row, dim3(1), dim3(256), 0, st, a.x, a.norm_w, a.eps, a.k,
                           a.hidden_out);
        b.x = a.hidden_out;
    }
    hipLaunchKernelGGL(k_bf16_gemv, dim3(a.n_pad / 64), dim3(64), 0, st, b);
    return hipGetLastError();
}

__global__ void k_bf16_relayout(const uint16_t *__restrict__ src, uint16_t *__restrict__ dst,
                                uint32_t n, uint32_t n_pad, uint32_t k, uint32_t *bad) {
    const uint32_t ksteps = k >> 3;
    const size_t chunks = (size_t)n_pad * ksteps;
    for (size_t c = blockIdx.x * (size_t)blockDim.x + threadIdx.x; c < chunks;
         c += (size_t)gridDim.x * blockDim.x) {
        const uint32_t r = (uint32_t)(c / ksteps), j = (uint32_t)(c % ksteps);
        u32x4 v = {0u, 0u, 0u, 0u};
        if (r < n) {
            v = *reinterpret_cast<const u32x4 *>(src + (size_t)r * k + j * 8);
            uint32_t bad_here = 0;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                // exponent all ones: inf or NaN
                bad_here |= ((v[q] & 0x7f80u) == 0x7f80u) | ((v[q] & 0x7f800000u) == 0x7f800000u);
            }
            if (bad_here) atomicOr(bad, 1u);
        }
        *reinterpret_cast<u32x4 *>(dst + ((size_t)(r >> 6) * ksteps + j) * 512 + (r & 63) * 8) = v;
    }
}

hipError_t launch_bf16_relayout(const uint16_t *src, uint16_t *dst, uint32_t n, uint32_t n_pad,
                                uint32_t k, uint32_t *bad_flag, hipStream_t st) {
    hipLaunchKernelGGL(k_bf16_relayout, dim3(4096), dim3(256), 0, st, src, dst, n, n_pad, k,
                       bad_flag);
    return hipGetLastError();
}

static int check_bf16_shape(uint32_t n, uint32_t k) {
    if (n == 0 || k % 256 != 0 || k < 256 || k > 16384) {
        set_error(F_BF16,
                  "bf16 gemv shape n=%u k=%u refused: n >= 1, k a multiple of 256 in 256..=16384",
                  n, k);
        return OMEGA_GPU_BAD_ARGS;
    }
    return OMEGA_GPU_OK;
}

static int bf16_run(const OmegaGpuBf16Tensor *t, const float *x, float *y, OmegaGpuBf16Info *info) {
    const uint64_t t0 = now_ns();
    Ctx *c = ctx(F_BF16);
    if (!c) return OMEGA_GPU_CHIP_FAIL;
    const size_t xb = ((size_t)t->k * 4 + 255) & ~(size_t)255;
    const size_t yb = ((size_t)t->n_pad * 4 + 255) & ~(size_t)255;
    if (!ensure_scratch(F_BF16, c, xb + yb) || !ensure_pinned(F_BF16, c, xb + yb))
        return OMEGA_GPU_CHIP_FAIL;
    uint8_t *dev = static_cast<uint8_t *>(c->scratch);
    uint8_t *pin = static_cast<uint8_t *>(c->pin);
    memcpy(pin, x, (size_t)t->k * 4);
    OMEGA_HIP(F_BF16, hipMemcpyAsync(dev, pin, (size_t)t->k * 4, hipMemcpyHostToDevice, c->stream));
    Bf16GemvArgs a;
    a.w = t->w;
    a.x = reinterpret_cast<const float *>(dev);
    a.n = t->n;
    a.n_pad = t->n_pad;
    a.k = t->k;
    a.y = reinterpret_cast<float *>(dev + xb);
    a.mutant = knobs().bf16_mutant;
    OMEGA_HIP(F_BF16, hipEventRecord(c->ev0, c->stream));
    OMEGA_HIP(F_BF16, launch_bf16_gemv(a, c->stream));
    OMEGA_HIP(F_BF16, hipEventRecord(c->ev1, c->stream));
    OMEGA_HIP(F_BF16, hipMemcpyAsync(pin + xb, a.y, (size_t)t->n * 4, hipMemcpyDeviceToHost, c->stream));
    OMEGA_HIP(F_BF16, hipStreamSynchronize(c->stream));
    memcpy(y, pin + xb, (size_t)t->n * 4);
    if (info) {
        memset(info, 0, sizeof(*info));
        info->n = t->n;
        info->k = t->k;
        info->rows_per_warp = 64;
        info->warps_per_cta = 1;
        info->depth = BF16_BATCH;
        info->grid_x = t->n_pad / 64;
        info->steps = t->k / 8;
        info->weight_bytes = (uint64_t)t->n * t->k * 2;
        info->elapsed_ns = event_ns(c);
        info->call_ns = now_ns() - t0;
        info->completion_marker = 1;
        info->kernel_cache_hit = true;
        fill_chip(info->target_chip, &info->sm_architecture, c);
    }
    return OMEGA_GPU_OK;
}

}  // namespace omega

using namespace omega;

extern "C" {

int omega_gpu_bf16_tensor_upload(uint32_t n, uint32_t k, const uint16_t *w_bf16,
                                 OmegaGpuBf16Tensor **out) {
    std::lock_guard<std::recursive_mutex> lk(big_lock());
    clear_error(F_BF16);
    if (!out || !w_bf16) {
        set_error(F_BF16, "bf16 upload: NULL pointer");
        return OMEGA_GPU_BAD_ARGS;
    }
    *out = nullptr;
    int rc = check_bf16_shape(n, k);
    if (rc) return rc;
    Ctx *c = ctx(F_BF16);
    if (!c) return OMEGA_GPU_CHIP_FAIL;
    OmegaGpuBf16Tensor *t = new OmegaGpuBf16Tensor();
    t->n = n;
    t->k = k;
    t->n_pad = (n + 63) / 64 * 64;
    const size_t bytes = (size_t)n * k * 2, pbytes = (size_t)t->n_pad * k * 2;
    uint16_t *raw = nullptr;
    uint32_t *flag = nullptr;
    uint32_t bad = 0;
    hipError_t e = hipMalloc(&t->w, pbytes);
    if (e == hipSuccess) e = hipMalloc(&raw, bytes);
    if (e == hipSuccess) e = hipMalloc(&flag, 4);
    if (e == hipSuccess) e = hipMemsetAsync(flag, 0, 4, c->stream);
    if (e == hipSuccess) e = hipMemcpyAsync(raw, w_bf16, bytes, hipMemcpyHostToDevice, c->stream);
    if (e == hipSuccess) e = launch_bf16_relayout(raw, t->w, n, t->n_pad, k, flag, c->stream);
    if (e == hipSuccess) e = hipMemcpyAsync(&bad, flag, 4, hipMemcpyDeviceToHost, c->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(c->stream);
    if (raw) (void)hipFree(raw);
    if (flag) (void)hipFree(flag);
    if (e != hipSuccess || bad) {
        if (e != hipSuccess) set_error(F_BF16, "bf16 upload: %s", hipGetErrorString(e));
        else set_error(F_BF16, "bf16 upload: a NaN or infinite weight");
        if (t->w) (void)hipFree(t->w);
        delete t;
        return e != hipSuccess ? OMEGA_GPU_CHIP_FAIL : OMEGA_GPU_BAD_ARGS;
    }
    *out = t;
    return OMEGA_GPU_OK;
}

int omega_gpu_bf16_tensor_synth(uint32_t n, uint32_t k, uint64_t seed, uint64_t tensor_id,
                                float sigma, OmegaGpuBf16Tensor **out) {
    std::lock_guard<std::recursive_mutex> lk(big_lock());
    clear_error(F_BF16);
    if (!out) return OMEGA_GPU_BAD_ARGS;
    *out = nullptr;
    int rc = check_bf16_shape(n, k);
    if (rc) return rc;
    Ctx *c = ctx(F_BF16);
    if (!c) return OMEGA_GPU_CHIP_FAIL;
    OmegaGpuBf16Tensor *t = new OmegaGpuBf16Tensor();
    t->n = n;
    t->k = k;
    t->n_pad = (n + 63) / 64 * 64;
    hipError_t e = hipMalloc(&t->w, (size_t)t->n_pad * k * 2);
    if (e == hipSuccess) e = launch_bf16_synth(t->w, n, t->n_pad, k, seed, tensor_id, sigma, c->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(c->stream);
    if (e != hipSuccess) {
        set_error(F_BF16, "bf16 synth: %s", hipGetErrorString(e));
        if (t->w) (void)hipFree(t->w);
        delete t;
        return OMEGA_GPU_CHIP_FAIL;
    }
    *out = t;
    return OMEGA_GPU_OK;
}

void omega_gpu_bf16_tensor_free(OmegaGpuBf16Tensor *t) {
    if (!t) return;
    std::lock_guard<std::recursive_mutex> lk(big_lock());
    Ctx *c = ctx(F_BF16);
    if (c) (void)hipStreamSynchronize(c->stream);
    if (t->w) (void)hipFree(t->w);
    delete t;
}

int omega_gpu_bf16_gemv_f32(const OmegaGpuBf16Tensor *t, const float *x, float *y,
                            OmegaGpuBf16Info *info) {
    std::lock_guard<std::recursive_mutex> lk(big_lock());
    clear_error(F_BF16);
    if (!t || !x || !y) {
        set_error(F_BF16, "bf16 gemv: NULL pointer");
        return OMEGA_GPU_BAD_ARGS;
    }
    return bf16_run(t, x, y, info);
}

int omega_gpu_bf16_gemv_bf16(const OmegaGpuBf16Tensor *t, const uint16_t *x, float *y,
                             OmegaGpuBf16Info *info) {
    std::lock_guard<std::recursive_mutex> lk(big_lock());
    clear_error(F_BF16);
    if (!t || !x || !y) {
        set_error(F_BF16, "bf16 gemv: NULL pointer");
        return OMEGA_GPU_BAD_ARGS;
    }
    std::vector<float> xf(t->k);
    for (uint32_t i = 0; i < t->k; ++i) {
        uint32_t u = (uint32_t)x[i] << 16;
        memcpy(&xf[i], &u, 4);
    }
    return bf16_run(t, xf.data(), y, info);
}

int omega_gpu_bf16_prepare(uint32_t k) {
    clear_error(F_BF16);
    return check_bf16_shape(1, k);
}
const char *omega_gpu_bf16_rc_name(int rc) { return rc_name(rc); }
const char *omega_gpu_bf16_last_error(void) { return last_error(F_BF16); }
// 0 off; 1 every logit negated; 2, 3 reserved (accepted, no effect)
void omega_gpu_bf16_test_set_mutant(int mutant) { knobs().bf16_mutant = mutant; }

}  // extern "C"
