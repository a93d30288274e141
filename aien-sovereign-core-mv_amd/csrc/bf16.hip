// bf16 streaming GEMV (the lm_head) for gfx950 with an optional fused RMSNorm prologue and a
// fused argmax, plus the omega_gpu_bf16_* entry points.
//
// Contract: crates/aien-omega-bf16/src/lib.rs:15-24 — y[r] = sum_c W[r][c] * x[c] over an
// [n][k] bf16 matrix, f32, deterministic summation order. The greedy token is the lowest index
// of the max (crates/aien-omega-dgraph/src/lib.rs:347-349, tensor.rs:299-318).
//
// Kernel shape (rows.hpp): row-major rows, two per wavefront (8 KiB, eight 1 KiB chunks), the
// activation phases in registers; one workgroup of 16 wavefronts per CU loops over the rows, with
// the activation row and the norm weights staged once per workgroup in LDS (read per wavefront,
// they crossed each CU's load path 16 to 20 times at the start of the stream), so the norm
// prologue runs once per wavefront from LDS. The argmax packs
// (value, ~index) into one 64-bit key whose integer maximum is the greedy token; each
// workgroup issues one fire-and-forget atomicMax into one of kArgmaxSlots slots and the host
// takes the maximum of the slots (no ordering between workgroups is involved).
#include <cmath>
#include <vector>

#include "kernels.hpp"
#include "rows.hpp"
#include "runtime.hpp"

namespace omega {


uint32_t argmax_from_slots(const unsigned long long *slots) {
    unsigned long long best = 0;
    for (uint32_t i = 0; i < kArgmaxSlots; ++i)
        if (slots[i] > best) best = slots[i];
    return 0xffffffffu - (uint32_t)(best & 0xffffffffu);
}

constexpr int kLmK = 2048;
constexpr int kLmRows = 2;
constexpr uint32_t kLmBlocks = 256;  // one 16-wavefront workgroup per CU
constexpr uint32_t kAnyBlocks = 2048;

template <bool NORM, bool ARGMAX>
__global__ __launch_bounds__(1024) void k_bf16_lm(const Bf16RowsArgs a) {
    using S = Bf16Slab<kLmK, kLmRows>;
    constexpr int P = S::P;
    constexpr uint32_t W = 16;  // wavefronts per workgroup: one workgroup per CU
    static_assert(!NORM || P * 8 * 64 == kLmK, "the phases must partition the row");
    __shared__ unsigned long long best_w[W];
    __shared__ __align__(16) float xs[kLmK];
    __shared__ __align__(16) float ws[NORM ? kLmK : 4];
    const uint32_t lane = lane_id(), wid = threadIdx.x >> 6;
    // the row and the norm weights staged once per workgroup
    if (threadIdx.x < kLmK / 4) {
        reinterpret_cast<f32x4 *>(xs)[threadIdx.x] = *as_global_f32x4(a.x + 4 * threadIdx.x);
        if (NORM) reinterpret_cast<f32x4 *>(ws)[threadIdx.x] = *as_global_f32x4(a.norm_w + 4 * threadIdx.x);
    }
    __syncthreads();
    float xr[P][8];
    float nw[P][8];
#pragma unroll
    for (int ph = 0; ph < P; ++ph) {
        const f32x4 *q = reinterpret_cast<const f32x4 *>(xs + S::col(ph, lane));
        const f32x4 *r = reinterpret_cast<const f32x4 *>(ws + (NORM ? S::col(ph, lane) : 0));
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const f32x4 t = q[i];
            xr[ph][4 * i] = t.x;
            xr[ph][4 * i + 1] = t.y;
            xr[ph][4 * i + 2] = t.z;
            xr[ph][4 * i + 3] = t.w;
            if (NORM) {
                const f32x4 u = r[i];
                nw[ph][4 * i] = u.x;
                nw[ph][4 * i + 1] = u.y;
                nw[ph][4 * i + 2] = u.z;
                nw[ph][4 * i + 3] = u.w;
            }
        }
    }
    // the final RMSNorm as one scale on the row sums (the sum of squares runs beside the stream)
    float scale = 1.0f;
    if (NORM) {
        const double ss = phases_sumsq(xr);
#pragma unroll
        for (int ph = 0; ph < P; ++ph)
#pragma unroll
            for (int i = 0; i < 8; ++i) xr[ph][i] = xr[ph][i] * nw[ph][i];
        scale = rms_scale(ss, kLmK, a.eps);
        if (a.hidden_out && blockIdx.x == 0 && wid == 0) {
#pragma unroll
            for (int ph = 0; ph < P; ++ph) {
                float4 *o = reinterpret_cast<float4 *>(a.hidden_out + S::col(ph, lane));
                o[0] = make_float4(xr[ph][0] * scale, xr[ph][1] * scale, xr[ph][2] * scale, xr[ph][3] * scale);
                o[1] = make_float4(xr[ph][4] * scale, xr[ph][5] * scale, xr[ph][6] * scale, xr[ph][7] * scale);
            }
        }
    }
    const uint32_t items = (a.n + kLmRows - 1) / kLmRows;
    const uint32_t stride = gridDim.x * W;
    unsigned long long best = 0;
    for (uint32_t item = blockIdx.x * W + wid; item < items; item += stride) {
        const uint32_t r0 = item * kLmRows;
        const bool two = r0 + 1 < a.n;
        S slab;
        const gu32x4 *p = as_global(a.w + (size_t)r0 * kLmK) + lane;
#pragma unroll
        for (int c = 0; c < S::CH; ++c)
            slab.v[c] = (two || c < S::CH / 2) ? __builtin_nontemporal_load(p + c * 64) : u32x4{0u, 0u, 0u, 0u};
        float acc[kLmRows] = {0.f, 0.f};
        slab.dot(xr, acc, lane);
        float v = reduce_rows(acc, lane) * scale;
        acc[0] *= scale;
        acc[1] *= scale;
        if (a.mutant == 1) {
            v = -v;
            acc[0] = -acc[0];
            acc[1] = -acc[1];
        }
        if (lane < (two ? 2u : 1u)) a.y[r0 + lane] = v;
        if (ARGMAX) {
            const unsigned long long k0 = argmax_key(acc[0], r0);
            if (k0 > best) best = k0;
            if (two) {
                const unsigned long long k1 = argmax_key(acc[1], r0 + 1);
                if (k1 > best) best = k1;
            }
        }
    }
    if (ARGMAX) {
        if (lane == 0) best_w[wid] = best;
        __syncthreads();
        if (threadIdx.x == 0) {
            unsigned long long b = best_w[0];
            for (uint32_t w = 1; w < W; ++w) b = best_w[w] > b ? best_w[w] : b;
            if (b) atomicMax(&a.argmax[blockIdx.x % kArgmaxSlots], b);
        }
    }
}

// any k (a multiple of 256 up to 16384): the row staged in LDS, one or two rows per wavefront
__global__ __launch_bounds__(256) void k_bf16_any(const Bf16RowsArgs a, uint32_t rpw) {
    extern __shared__ float xs[];
    const uint32_t lane = lane_id(), wid = threadIdx.x >> 6;
    const uint32_t k = a.k;
    for (uint32_t c = threadIdx.x; c < k; c += 256) xs[c] = a.x[c];
    __syncthreads();
    const uint32_t kb = 2 * k;
    const uint32_t ch = rpw * kb / 1024;
    const uint32_t items = (a.n + rpw - 1) / rpw;
    for (uint32_t item = blockIdx.x * 4 + wid; item < items; item += gridDim.x * 4) {
        const uint32_t r0 = item * rpw;
        const uint32_t rows = min(rpw, a.n - r0);
        const gu32x4 *base = as_global(a.w + (size_t)r0 * k) + lane;
        float acc[2] = {0.f, 0.f};
        for (uint32_t c0 = 0; c0 < ch; c0 += 8) {
            u32x4 v[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const uint32_t c = c0 + i;
                const uint32_t rl = (c * 1024 + 16 * lane) / kb;
                v[i] = (c < ch && rl < rows) ? __builtin_nontemporal_load(base + (size_t)c * 64)
                                             : u32x4{0u, 0u, 0u, 0u};
            }
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const uint32_t c = c0 + i;
                if (c >= ch) break;
                const uint32_t o = c * 1024 + 16 * lane;
                const uint32_t rl = o / kb, col = (o % kb) / 2;
                const float p = bf16_dot8(v[i], xs + col);
                acc[0] += rl == 0 ? p : 0.f;
                acc[1] += rl == 1 ? p : 0.f;
            }
        }
        float v = reduce_rows(acc, lane);
        if (a.mutant == 1) v = -v;
        if (lane < rows) a.y[r0 + lane] = v;
    }
}

hipError_t launch_bf16_rows(const Bf16RowsArgs &a, hipStream_t st) {
    if (a.k == (uint32_t)kLmK) {
        const uint32_t items = (a.n + kLmRows - 1) / kLmRows;
        uint32_t blocks = (items + 15) / 16;
        if (blocks > kLmBlocks) blocks = kLmBlocks;
        if (a.norm_w && a.argmax)
            OMEGA_LAUNCH((k_bf16_lm<true, true>), dim3(blocks), dim3(1024), 0, st, a);
        else if (a.norm_w)
            OMEGA_LAUNCH((k_bf16_lm<true, false>), dim3(blocks), dim3(1024), 0, st, a);
        else if (a.argmax)
            OMEGA_LAUNCH((k_bf16_lm<false, true>), dim3(blocks), dim3(1024), 0, st, a);
        else
            OMEGA_LAUNCH((k_bf16_lm<false, false>), dim3(blocks), dim3(1024), 0, st, a);
        return hipGetLastError();
    }
    if (a.norm_w || a.argmax) return hipErrorInvalidValue;
    const uint32_t rpw = (2 * a.k) % 1024 == 0 ? 1 : 2;
    const uint32_t items = (a.n + rpw - 1) / rpw;
    uint32_t blocks = (items + 3) / 4;
    if (blocks > kAnyBlocks) blocks = kAnyBlocks;
    OMEGA_LAUNCH(k_bf16_any, dim3(blocks), dim3(256), a.k * 4, st, a, rpw);
    return hipGetLastError();
}

__global__ void k_bf16_scan(const uint16_t *__restrict__ w, size_t chunks, uint32_t *bad) {
    uint32_t b = 0;
    for (size_t c = blockIdx.x * (size_t)blockDim.x + threadIdx.x; c < chunks;
         c += (size_t)gridDim.x * blockDim.x) {
        const u32x4 v = __builtin_nontemporal_load(as_global(w) + c);
#pragma unroll
        for (int q = 0; q < 4; ++q)  // exponent all ones: inf or NaN
            b |= ((v[q] & 0x7f80u) == 0x7f80u) | ((v[q] & 0x7f800000u) == 0x7f800000u);
    }
    if (b) atomicOr(bad, 1u);
}

hipError_t launch_bf16_scan(const uint16_t *w, size_t count, uint32_t *flag, hipStream_t st) {
    hipLaunchKernelGGL(k_bf16_scan, dim3(2048), dim3(256), 0, st, w, count / 8, flag);
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
    const size_t yb = ((size_t)t->n * 4 + 255) & ~(size_t)255;
    if (!ensure_scratch(F_BF16, c, xb + yb) || !ensure_pinned(F_BF16, c, xb + yb))
        return OMEGA_GPU_CHIP_FAIL;
    uint8_t *dev = static_cast<uint8_t *>(c->scratch);
    uint8_t *pin = static_cast<uint8_t *>(c->pin);
    memcpy(pin, x, (size_t)t->k * 4);
    OMEGA_HIP(F_BF16, hipMemcpyAsync(dev, pin, (size_t)t->k * 4, hipMemcpyHostToDevice, c->stream));
    Bf16RowsArgs a;
    a.w = t->w;
    a.x = reinterpret_cast<const float *>(dev);
    a.n = t->n;
    a.k = t->k;
    a.y = reinterpret_cast<float *>(dev + xb);
    a.mutant = knobs().bf16_mutant;
    OMEGA_HIP(F_BF16, hipEventRecord(c->ev0, c->stream));
    OMEGA_HIP(F_BF16, launch_bf16_rows(a, c->stream));
    OMEGA_HIP(F_BF16, hipEventRecord(c->ev1, c->stream));
    OMEGA_HIP(F_BF16, hipMemcpyAsync(pin + xb, a.y, (size_t)t->n * 4, hipMemcpyDeviceToHost, c->stream));
    OMEGA_HIP(F_BF16, hipStreamSynchronize(c->stream));
    memcpy(y, pin + xb, (size_t)t->n * 4);
    if (info) {
        memset(info, 0, sizeof(*info));
        info->n = t->n;
        info->k = t->k;
        info->rows_per_warp = t->k == (uint32_t)kLmK ? kLmRows : ((2 * t->k) % 1024 == 0 ? 1 : 2);
        info->warps_per_cta = t->k == (uint32_t)kLmK ? 16 : 4;
        info->depth = 8;
        info->grid_x = t->k == (uint32_t)kLmK ? kLmBlocks : kAnyBlocks;
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

namespace omega {
// row-major bf16 -> the tiled twin (runtime.hpp): one thread per 16 output bytes (8 elements)
__global__ __launch_bounds__(256) void k_bf16_tile(const uint16_t *w, uint16_t *wt, uint32_t n, uint32_t k,
                                                   size_t pieces) {
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= pieces) return;
    const size_t b = i >> 6;  // 64 pieces of 16 B per 1 KiB block
    const uint32_t l = (uint32_t)i & 63u, r = l & 15u, gq = l >> 4;
    const uint32_t kbs = k / 32;
    const size_t rt = b / kbs;
    const uint32_t kb = (uint32_t)(b % kbs);
    const size_t row = rt * 16 + r;
    const u32x4 v = *as_global(w + row * k + (size_t)kb * 32 + 8 * gq);
    *reinterpret_cast<u32x4 *>(wt + i * 8) = v;
}

int bf16_ensure_tiled(Family f, OmegaGpuBf16Tensor *t) {
    if (t->wt) return OMEGA_GPU_OK;
    if (t->n % 16 != 0 || t->k % 32 != 0) {
        set_error(f, "bf16 tiled twin: %u x %u is not whole 16 x 32 blocks", t->n, t->k);
        return OMEGA_GPU_BAD_ARGS;
    }
    Ctx *c = ctx(f);
    if (!c) return OMEGA_GPU_CHIP_FAIL;
    const size_t elems = (size_t)t->n * t->k, pieces = elems / 8;
    if (seal_refuses(f, "bf16 tiled weight twin", elems * 2)) return OMEGA_GPU_TOO_LARGE;
    OMEGA_HIP(f, dev_malloc(&t->wt, elems * 2));
    hipLaunchKernelGGL(k_bf16_tile, dim3((unsigned)((pieces + 255) / 256)), dim3(256), 0, c->stream, t->w, t->wt,
                       t->n, t->k, pieces);
    hipError_t e = hipGetLastError();
    if (e == hipSuccess) e = hipStreamSynchronize(c->stream);
    if (e != hipSuccess) {
        (void)dev_free(t->wt);
        t->wt = nullptr;
        set_error(f, "bf16 tiled twin: %s", hipGetErrorString(e));
        return OMEGA_GPU_CHIP_FAIL;
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
    t->n_pad = n;
    const size_t count = (size_t)n * k;
    uint32_t *flag = nullptr;
    uint32_t bad = 0;
    hipError_t e = dev_malloc(&t->w, count * 2);
    if (e == hipSuccess) e = dev_malloc(&flag, 4);
    if (e == hipSuccess) e = hipMemsetAsync(flag, 0, 4, c->stream);
    if (e == hipSuccess) e = hipMemcpyAsync(t->w, w_bf16, count * 2, hipMemcpyHostToDevice, c->stream);
    if (e == hipSuccess) e = launch_bf16_scan(t->w, count, flag, c->stream);
    if (e == hipSuccess) e = hipMemcpyAsync(&bad, flag, 4, hipMemcpyDeviceToHost, c->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(c->stream);
    if (flag) (void)dev_free(flag);
    if (e != hipSuccess || bad) {
        if (e != hipSuccess) set_error(F_BF16, "bf16 upload: %s", hipGetErrorString(e));
        else set_error(F_BF16, "bf16 upload: a NaN or infinite weight");
        if (t->w) (void)dev_free(t->w);
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
    t->n_pad = n;
    hipError_t e = dev_malloc(&t->w, (size_t)n * k * 2);
    if (e == hipSuccess) e = launch_bf16_synth(t->w, n, k, seed, tensor_id, sigma, c->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(c->stream);
    if (e != hipSuccess) {
        set_error(F_BF16, "bf16 synth: %s", hipGetErrorString(e));
        if (t->w) (void)dev_free(t->w);
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
    if (t->w) (void)dev_free(t->w);
    if (t->wt) (void)dev_free(t->wt);
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
