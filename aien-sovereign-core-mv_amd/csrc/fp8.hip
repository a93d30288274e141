// FP8 e4m3 block-scaled GEMV for gfx950: upload (re-layout to the row-per-lane tiling), the
// GEMV kernel with its four epilogues, the device-side synthetic generator, and the
// omega_gpu_fp8_* / omega_gpu_fp8gemm_* entry points.
//
// Contract: crates/aien-omega-fp8/src/lib.rs:16-29 — y[g][r] = sum_c e4m3(W[id_g][r][c]) *
// x[row(g)][c] * bf16(scale[id_g][r/128][c/128]) in f32.
//
// Kernel shape: one wavefront per work item = (group, 64-row tile, k-split). Lane l owns row
// 64*tile + l; the wave streams 1 KiB per 16-column step (fully coalesced, non-temporal), the
// 16 activation values of a step are wave-uniform (scalar loads or an LDS broadcast), each
// byte pair is widened by the native OCP-fp8 convert (v_cvt_pk_f32_fp8) and accumulated with
// f32 FMAs; per 128-column block the partial dot is multiplied by the block scale (the
// dequant_matvec order of qwen3_moe.rs:595-619). Splits along k meet in a deterministic
// last-arriver reduction (fixed split order), so results never depend on timing.
#include <cmath>
#include <cstdio>
#include <vector>

#include "device.hpp"
#include "kernels.hpp"
#include "runtime.hpp"

namespace omega {

typedef float f32x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ void dot4_fp8(uint32_t w, const float *xx, float &p) {
    f32x2 lo = __builtin_amdgcn_cvt_pk_f32_fp8((int)w, false);
    f32x2 hi = __builtin_amdgcn_cvt_pk_f32_fp8((int)w, true);
    p = fmaf(lo.x, xx[0], p);
    p = fmaf(lo.y, xx[1], p);
    p = fmaf(hi.x, xx[2], p);
    p = fmaf(hi.y, xx[3], p);
}

__device__ __forceinline__ float silu_mul(float g, float u) { return g / (1.0f + expf(-g)) * u; }

__device__ __forceinline__ double wave_sum_f64(double v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

// RMSNorm scale of a [k] row, f64 sum of squares (tensor.rs:94-110), every lane gets it.
__device__ __forceinline__ float row_rms_scale(const float *x, uint32_t k, float eps) {
    const int lane = threadIdx.x & 63;
    double ss = 0.0;
    for (uint32_t c = lane * 4; c < k; c += 256) {
        float4 v = *reinterpret_cast<const float4 *>(x + c);
        ss += (double)v.x * (double)v.x;
        ss += (double)v.y * (double)v.y;
        ss += (double)v.z * (double)v.z;
        ss += (double)v.w * (double)v.w;
    }
    ss = wave_sum_f64(ss);
    return (float)(1.0 / sqrt(ss / (double)k + (double)eps));
}

template <int STEPS, int EPI, bool NORM>
__global__ __launch_bounds__(64) void k_fp8_gemv(const Fp8GemvArgs a) {
    static_assert(STEPS % 8 == 0, "a split covers whole 128-column blocks");
    constexpr int ROWSETS = EPI == EPI_SWIGLU ? 2 : 1;
    __shared__ float xs[NORM ? STEPS * 16 : 1];

    const uint32_t lane = threadIdx.x;
    const uint32_t S = a.splits;
    const uint32_t ksteps = a.k >> 4;
    const uint32_t kb = a.k >> 7;
    const uint32_t tiles = (EPI == EPI_SWIGLU) ? (a.n >> 7) : (a.n >> 6);
    uint32_t item = blockIdx.x;
    const uint32_t s = item % S;
    item /= S;
    const uint32_t t = item % tiles;
    const uint32_t g = item / tiles;

    // the expert of this group
    uint32_t gsel = g;
    if (a.mutant == 3 && a.groups > 1) gsel = (g + 1) % a.groups;
    const uint8_t *wexp;
    const float *sexp;
    if (a.tab) {
        wexp = reinterpret_cast<const uint8_t *>(a.tab[2 * gsel]);
        sexp = reinterpret_cast<const float *>(a.tab[2 * g + 1]);
    } else {
        const size_t e = a.ids[gsel];
        wexp = a.w + e * (size_t)a.n * a.k;
        sexp = a.s + e * (size_t)(a.n >> 7) * kb;
    }

    const uint32_t j0 = s * STEPS;
    uint32_t rows0[ROWSETS];
    rows0[0] = t * 64;
    if (EPI == EPI_SWIGLU) rows0[ROWSETS - 1] = (a.n >> 1) + t * 64;

    // issue every weight load of the item first (STEPS x 16 B per lane per row set)
    u32x4 wv[ROWSETS][STEPS];
#pragma unroll
    for (int r = 0; r < ROWSETS; ++r) {
        const gu32x4 *p = as_global(wexp + ((size_t)(rows0[r] >> 6) * ksteps + j0) * 1024 + lane * 16);
#pragma unroll
        for (int i = 0; i < STEPS; ++i) wv[r][i] = __builtin_nontemporal_load(p + i * 64);
    }

    const float *xg = a.x + (size_t)g * a.x_stride;
    const float *xp;
    if (NORM) {
        const float scale = row_rms_scale(xg, a.k, a.eps);
        for (uint32_t c = lane; c < STEPS * 16; c += 64) {
            const uint32_t col = j0 * 16 + c;
            xs[c] = xg[col] * scale * a.norm_w[col];
        }
        __syncthreads();
        xp = xs;
    } else {
        xp = xg + j0 * 16;
    }

    float acc[ROWSETS];
#pragma unroll
    for (int r = 0; r < ROWSETS; ++r) {
        const uint32_t rb = rows0[r] >> 7;
        acc[r] = 0.0f;
#pragma unroll
        for (int b = 0; b < STEPS / 8; ++b) {
            float p0 = 0.f, p1 = 0.f, p2 = 0.f, p3 = 0.f;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const u32x4 v = wv[r][b * 8 + i];
                const float *xx = xp + (b * 8 + i) * 16;
                dot4_fp8(v.x, xx + 0, p0);
                dot4_fp8(v.y, xx + 4, p1);
                dot4_fp8(v.z, xx + 8, p2);
                dot4_fp8(v.w, xx + 12, p3);
                // LDS operands: read each step's 16 values when they are used (keeps the
                // normalised row out of registers)
                if (NORM) __asm__ volatile("" : "+v"(p0), "+v"(p1), "+v"(p2), "+v"(p3)::"memory");
            }
            const uint32_t cb = (a.mutant == 2) ? 0 : (j0 >> 3) + b;
            float sc = (a.mutant == 1) ? 1.0f : sexp[rb * kb + cb];
            sc *= a.x_scale;
            acc[r] = fmaf((p0 + p1) + (p2 + p3), sc, acc[r]);
        }
    }

    const uint32_t n = a.n;
    // ---------------------------------------------------------------- epilogues
    if (EPI == EPI_STORE || EPI == EPI_RESID) {
        const size_t row = (size_t)g * n + t * 64 + lane;
        if (S == 1) {
            if (EPI == EPI_STORE) a.y[row] = acc[0];
            else a.y[row] += acc[0];
            return;
        }
        a.partial[(size_t)s * a.groups * n + row] = acc[0];
        __threadfence();
        uint32_t last = 0;
        const uint32_t cidx = g * tiles + t;
        if (lane == 0) last = atomicAdd(&a.counters[cidx], 1u) == S - 1;
        last = __shfl(last, 0, 64);
        if (!last) return;
        __threadfence();
        float sum = 0.f;
        for (uint32_t s2 = 0; s2 < S; ++s2) sum += __builtin_nontemporal_load(&a.partial[(size_t)s2 * a.groups * n + row]);
        if (lane == 0) atomicExch(&a.counters[cidx], 0u);
        if (EPI == EPI_STORE) a.y[row] = sum;
        else a.y[row] += sum;
        return;
    }
    if (EPI == EPI_SWIGLU) {
        const uint32_t half = n >> 1;
        const size_t jrow = t * 64 + lane;
        float gv = acc[0], uv = acc[ROWSETS - 1];
        if (S > 1) {
            float *pg = a.partial + (size_t)s * a.groups * n + (size_t)g * n;
            pg[jrow] = gv;
            pg[half + jrow] = uv;
            __threadfence();
            uint32_t last = 0;
            const uint32_t cidx = g * tiles + t;
            if (lane == 0) last = atomicAdd(&a.counters[cidx], 1u) == S - 1;
            last = __shfl(last, 0, 64);
            if (!last) return;
            __threadfence();
            gv = 0.f;
            uv = 0.f;
            for (uint32_t s2 = 0; s2 < S; ++s2) {
                const float *q = a.partial + (size_t)s2 * a.groups * n + (size_t)g * n;
                gv += __builtin_nontemporal_load(&q[jrow]);
                uv += __builtin_nontemporal_load(&q[half + jrow]);
            }
            if (lane == 0) atomicExch(&a.counters[cidx], 0u);
        }
        if (a.graph_mutant == 1) {
            const float tmp = gv;
            gv = uv;
            uv = tmp;
        }
        a.y[(size_t)g * half + jrow] = silu_mul(gv, uv);
        return;
    }
    if (EPI == EPI_QKV) {
        // 128-row heads: the last of the head's two tiles x splits prepares it
        const size_t r = t * 64 + lane;
        a.partial[(size_t)s * n + r] = acc[0];
        __threadfence();
        uint32_t last = 0;
        const uint32_t head = t >> 1;
        if (lane == 0) last = atomicAdd(&a.counters[head], 1u) == 2 * S - 1;
        last = __shfl(last, 0, 64);
        if (!last) return;
        __threadfence();
        float v0 = 0.f, v1 = 0.f;
        for (uint32_t s2 = 0; s2 < S; ++s2) {
            v0 += __builtin_nontemporal_load(&a.partial[(size_t)s2 * n + head * 128 + lane]);
            v1 += __builtin_nontemporal_load(&a.partial[(size_t)s2 * n + head * 128 + 64 + lane]);
        }
        if (lane == 0) atomicExch(&a.counters[head], 0u);
        const uint32_t pos = a.pos_dev ? *a.pos_dev : a.pos_host;
        prep_head(a.prep, head, pos, v0, v1);
        return;
    }
    if (EPI == EPI_COMBINE) {
        // partial [s][g][n]; the last of all groups x splits of this tile combines
        const size_t r = t * 64 + lane;
        a.partial[((size_t)s * a.groups + g) * n + r] = acc[0];
        __threadfence();
        uint32_t last = 0;
        if (lane == 0) last = atomicAdd(&a.counters[t], 1u) == S * a.groups - 1;
        last = __shfl(last, 0, 64);
        if (!last) return;
        __threadfence();
        float moe = 0.f;
        for (uint32_t gg = 0; gg < a.groups; ++gg) {
            float d = 0.f;
            for (uint32_t s2 = 0; s2 < S; ++s2)
                d += __builtin_nontemporal_load(&a.partial[((size_t)s2 * a.groups + gg) * n + r]);
            const float wgt = (a.graph_mutant == 2 && gg == 7) ? 0.f : a.comb_w[gg];
            moe += wgt * d;
        }
        if (lane == 0) atomicExch(&a.counters[t], 0u);
        a.y[r] += moe;
    }
}

uint32_t fp8_gemv_items(const Fp8GemvArgs &a, int steps) {
    (void)steps;
    return a.groups * a.splits * (a.n >> 6);
}

int fp8_gemv_plan(Fp8GemvArgs &a, int epi) {
    const uint32_t ksteps = a.k >> 4;
    int steps = (epi == EPI_SWIGLU) ? 8 : 16;
    if (ksteps % steps != 0) steps = 8;
    a.splits = ksteps / steps;
    return steps;
}

template <int STEPS, int EPI>
static hipError_t launch_t(const Fp8GemvArgs &a, hipStream_t st) {
    uint32_t items = a.groups * a.splits * ((EPI == EPI_SWIGLU) ? (a.n >> 7) : (a.n >> 6));
    if (a.norm_w)
        hipLaunchKernelGGL((k_fp8_gemv<STEPS, EPI, true>), dim3(items), dim3(64), 0, st, a);
    else
        hipLaunchKernelGGL((k_fp8_gemv<STEPS, EPI, false>), dim3(items), dim3(64), 0, st, a);
    return hipGetLastError();
}

hipError_t launch_fp8_gemv_epi(const Fp8GemvArgs &a, int steps, int epi, hipStream_t st) {
    if (steps == 16) {
        switch (epi) {
        case EPI_STORE: return launch_t<16, EPI_STORE>(a, st);
        case EPI_RESID: return launch_t<16, EPI_RESID>(a, st);
        case EPI_SWIGLU: return launch_t<16, EPI_SWIGLU>(a, st);
        case EPI_COMBINE: return launch_t<16, EPI_COMBINE>(a, st);
        case EPI_QKV: return launch_t<16, EPI_QKV>(a, st);
        }
    } else {
        switch (epi) {
        case EPI_STORE: return launch_t<8, EPI_STORE>(a, st);
        case EPI_RESID: return launch_t<8, EPI_RESID>(a, st);
        case EPI_SWIGLU: return launch_t<8, EPI_SWIGLU>(a, st);
        case EPI_COMBINE: return launch_t<8, EPI_COMBINE>(a, st);
        case EPI_QKV: return launch_t<8, EPI_QKV>(a, st);
        }
    }
    return hipErrorInvalidValue;
}

hipError_t launch_fp8_gemv(const Fp8GemvArgs &a, int steps, hipStream_t st) {
    return launch_fp8_gemv_epi(a, steps, EPI_STORE, st);
}

// ---------------------------------------------------------------- upload re-layout
__global__ void k_fp8_relayout(const uint8_t *__restrict__ src, uint8_t *__restrict__ dst,
                               uint32_t experts, uint32_t n, uint32_t k, uint32_t *nan_flag) {
    const uint32_t ksteps = k >> 4;
    const size_t chunks = (size_t)experts * n * ksteps;
    for (size_t c = blockIdx.x * (size_t)blockDim.x + threadIdx.x; c < chunks;
         c += (size_t)gridDim.x * blockDim.x) {
        const size_t e = c / ((size_t)n * ksteps);
        const size_t rem = c % ((size_t)n * ksteps);
        const uint32_t r = (uint32_t)(rem / ksteps), j = (uint32_t)(rem % ksteps);
        const u32x4 v = *reinterpret_cast<const u32x4 *>(src + e * (size_t)n * k + (size_t)r * k + j * 16);
        // e4m3 NaN: S.1111.111 in any byte
        uint32_t bad = 0;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const uint32_t x = v[q] & 0x7f7f7f7fu;
            const uint32_t m = ~(x ^ 0x7f7f7f7fu);  // bytes equal to 0x7f have all 8 bits set
            bad |= (m & (m >> 1) & (m >> 2) & (m >> 3) & (m >> 4) & (m >> 5) & (m >> 6) & 0x01010101u);
        }
        if (bad) atomicOr(nan_flag, 1u);
        uint8_t *d = dst + e * (size_t)n * k + ((size_t)(r >> 6) * ksteps + j) * 1024 + (r & 63) * 16;
        *reinterpret_cast<u32x4 *>(d) = v;
    }
}

hipError_t launch_fp8_relayout(const uint8_t *src, uint8_t *dst, uint32_t experts, uint32_t n,
                               uint32_t k, uint32_t *nan_flag, hipStream_t st) {
    hipLaunchKernelGGL(k_fp8_relayout, dim3(4096), dim3(256), 0, st, src, dst, experts, n, k,
                       nan_flag);
    return hipGetLastError();
}

// ---------------------------------------------------------------- synthetic generator
// Identical arithmetic to the tests' CPU generator: splitmix64 counters, twelve 16-bit
// uniforms (Irwin-Hall), one f32 rounding; per-block bf16(absmax/448) scale; RNE e4m3.
__device__ __forceinline__ uint64_t splitmix64(uint64_t x) {
    uint64_t z = x + 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

__device__ __forceinline__ float synth_normal(uint64_t base, uint64_t idx, float c) {
    uint64_t b = base + idx * 3;
    int32_t sum = 0;
#pragma unroll
    for (int j = 0; j < 3; ++j) {
        uint64_t h = splitmix64(b + (uint64_t)j);
        sum += (int32_t)(h & 0xffff) + (int32_t)((h >> 16) & 0xffff) +
               (int32_t)((h >> 32) & 0xffff) + (int32_t)((h >> 48) & 0xffff);
    }
    return (float)(sum - 393210) * c;
}

__device__ __forceinline__ uint16_t f32_to_bf16_rne(float v) {
    uint32_t u = __float_as_uint(v);
    return (uint16_t)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}

__device__ __forceinline__ uint8_t f32_to_e4m3_rne(float value) {
    uint32_t u = __float_as_uint(value);
    uint8_t sign = (u >> 31) ? 0x80 : 0;
    uint32_t a = u & 0x7fffffffu;
    if (a >= 0x43e00000u) return sign | 0x7e;
    if (a < 0x3c800000u) return sign | (uint8_t)rintf(__uint_as_float(a) * 512.0f);
    uint32_t e = (a >> 23) - 127 + 7;
    uint32_t mant = a & 0x7fffffu;
    uint32_t r = mant + 0x7ffffu + ((mant >> 20) & 1u);
    uint32_t code = (e << 3) + (r >> 20);
    if (code > 0x7e) code = 0x7e;
    return sign | (uint8_t)code;
}

// one workgroup of 256 threads per 128x128 block
__global__ __launch_bounds__(256) void k_fp8_synth(uint8_t *w, float *s, uint32_t n, uint32_t k,
                                                   uint64_t base, float c) {
    const uint32_t nb = n >> 7, kbk = k >> 7;
    const uint32_t e = blockIdx.z, rb = blockIdx.y, cb = blockIdx.x;
    const size_t ebase = (size_t)e * n * k;
    __shared__ float red[8];
    float amax = 0.f;
    for (uint32_t i = threadIdx.x; i < 128 * 128; i += 256) {
        const uint32_t r = rb * 128 + (i >> 7), col = cb * 128 + (i & 127);
        amax = fmaxf(amax, fabsf(synth_normal(base, ebase + (size_t)r * k + col, c)));
    }
    for (int o = 32; o > 0; o >>= 1) amax = fmaxf(amax, __shfl_xor(amax, o, 64));
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = amax;
    __syncthreads();
    amax = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    const uint16_t sb = f32_to_bf16_rne(amax / 448.0f);
    const float sv = __uint_as_float((uint32_t)sb << 16);
    if (threadIdx.x == 0) s[((size_t)e * nb + rb) * kbk + cb] = sv;
    const uint32_t ksteps = k >> 4;
    for (uint32_t i = threadIdx.x; i < 128 * 128; i += 256) {
        const uint32_t r = rb * 128 + (i >> 7), col = cb * 128 + (i & 127);
        const float v = synth_normal(base, ebase + (size_t)r * k + col, c);
        w[ebase + ((size_t)(r >> 6) * ksteps + (col >> 4)) * 1024 + (r & 63) * 16 + (col & 15)] =
            f32_to_e4m3_rne(v / sv);
    }
}

static uint64_t synth_base(uint64_t seed, uint64_t tensor) {
    // host twin of the device base: splitmix64(seed ^ tensor * K) (same constant as the tests)
    uint64_t x = seed ^ (tensor * 0xD1B54A32D192ED03ull);
    uint64_t z = x + 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

hipError_t launch_fp8_synth(uint8_t *w, float *s, uint32_t experts, uint32_t n, uint32_t k,
                            uint64_t seed, uint64_t tensor, float sigma, hipStream_t st) {
    const float c = sigma * (1.0f / 65536.0f);
    hipLaunchKernelGGL(k_fp8_synth, dim3(k >> 7, n >> 7, experts), dim3(256), 0, st, w, s, n, k,
                       synth_base(seed, tensor), c);
    return hipGetLastError();
}

// bf16 synthetic rows (tiled layout of the bf16 GEMV): element (r, c) of [n][k] N(0, sigma)
__global__ void k_bf16_synth(uint16_t *w, uint32_t n, uint32_t n_pad, uint32_t k, uint64_t base,
                             float c) {
    const uint32_t ksteps = k >> 3;
    const size_t total = (size_t)n_pad * k;
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < total;
         i += (size_t)gridDim.x * blockDim.x) {
        const uint32_t r = (uint32_t)(i / k), col = (uint32_t)(i % k);
        const uint16_t v = r < n ? f32_to_bf16_rne(synth_normal(base, i, c)) : 0;
        w[((size_t)(r >> 6) * ksteps + (col >> 3)) * 512 + (r & 63) * 8 + (col & 7)] = v;
    }
}

hipError_t launch_bf16_synth(uint16_t *w, uint32_t n, uint32_t n_pad, uint32_t k, uint64_t seed,
                             uint64_t tensor, float sigma, hipStream_t st) {
    const float c = sigma * (1.0f / 65536.0f);
    hipLaunchKernelGGL(k_bf16_synth, dim3(8192), dim3(256), 0, st, w, n, n_pad, k,
                       synth_base(seed, tensor), c);
    return hipGetLastError();
}

// ---------------------------------------------------------------- host-side checks
static int check_tensor_shape(Family f, uint32_t experts, uint32_t n, uint32_t k) {
    if (experts == 0 || n == 0 || n % 128 != 0 || k % 128 != 0 || k < 128 || k > 32768) {
        set_error(f,
                  "fp8 shape experts=%u n=%u k=%u refused: experts >= 1, n and k multiples of "
                  "128, 128 <= k <= 32768",
                  experts, n, k);
        return OMEGA_GPU_BAD_ARGS;
    }
    return OMEGA_GPU_OK;
}

static void fill_info(OmegaGpuFp8Info *info, const OmegaGpuFp8Tensor *t, uint32_t groups,
                      const Fp8GemvArgs &a, int steps, uint64_t elapsed, uint64_t t0, Ctx *c) {
    if (!info) return;
    memset(info, 0, sizeof(*info));
    info->experts = t->experts;
    info->n = t->n;
    info->k = t->k;
    info->groups = groups;
    info->lane_bytes = 16;
    info->rows_per_warp = 64;
    info->warps_per_cta = 1;
    info->depth = (uint32_t)steps;
    info->grid_x = fp8_gemv_items(a, steps);
    info->grid_y = 1;
    info->steps = (uint32_t)steps;
    info->weight_bytes = (uint64_t)groups * t->n * t->k;
    info->scale_bytes = (uint64_t)groups * (t->n / 128) * (t->k / 128) * 4;
    info->elapsed_ns = elapsed;
    info->call_ns = now_ns() - t0;
    info->completion_marker = 1;
    info->kernel_cache_hit = true;
    fill_chip(info->target_chip, &info->sm_architecture, c);
}

// Runs one GEMV launch with host x/y (the staging path of the standalone entries).
static bool counters_fit(Ctx *c, const Fp8GemvArgs &a) {
    if ((size_t)a.groups * (a.n / 64) <= c->n_counters) return true;
    set_error(F_FP8, "fp8 gemv: %u groups x %u rows need more tile counters than the pool holds",
              a.groups, a.n);
    return false;
}

static int run_gemv_host(Ctx *c, const OmegaGpuFp8Tensor *t, Fp8GemvArgs &a, const float *x,
                         size_t x_floats, float *y, uint64_t *elapsed, int *steps_out) {
    const int steps = fp8_gemv_plan(a, EPI_STORE);
    if (!counters_fit(c, a)) return OMEGA_GPU_TOO_LARGE;
    const size_t y_floats = (size_t)a.groups * t->n;
    const size_t part_floats = a.splits > 1 ? (size_t)a.splits * y_floats : 0;
    const size_t x_bytes = (x_floats * 4 + 255) & ~(size_t)255;
    const size_t y_bytes = (y_floats * 4 + 255) & ~(size_t)255;
    if (!ensure_scratch(F_FP8, c, x_bytes + y_bytes + part_floats * 4)) return OMEGA_GPU_CHIP_FAIL;
    if (!ensure_pinned(F_FP8, c, x_bytes + y_bytes)) return OMEGA_GPU_CHIP_FAIL;
    uint8_t *dev = static_cast<uint8_t *>(c->scratch);
    float *xd = reinterpret_cast<float *>(dev);
    float *yd = reinterpret_cast<float *>(dev + x_bytes);
    float *pd = reinterpret_cast<float *>(dev + x_bytes + y_bytes);
    uint8_t *pin = static_cast<uint8_t *>(c->pin);
    memcpy(pin, x, x_floats * 4);
    OMEGA_HIP(F_FP8, hipMemcpyAsync(xd, pin, x_floats * 4, hipMemcpyHostToDevice, c->stream));
    a.x = xd;
    a.y = yd;
    a.partial = pd;
    a.counters = counters(c);
    OMEGA_HIP(F_FP8, hipEventRecord(c->ev0, c->stream));
    OMEGA_HIP(F_FP8, launch_fp8_gemv(a, steps, c->stream));
    OMEGA_HIP(F_FP8, hipEventRecord(c->ev1, c->stream));
    OMEGA_HIP(F_FP8, hipMemcpyAsync(pin + x_bytes, yd, y_floats * 4, hipMemcpyDeviceToHost, c->stream));
    OMEGA_HIP(F_FP8, hipStreamSynchronize(c->stream));
    memcpy(y, pin + x_bytes, y_floats * 4);
    *elapsed = event_ns(c);
    *steps_out = steps;
    return OMEGA_GPU_OK;
}

}  // namespace omega

using namespace omega;

extern "C" {

int omega_gpu_fp8_tensor_upload(uint32_t experts, uint32_t n, uint32_t k, const uint8_t *w,
                                const uint16_t *scale_inv_bf16, OmegaGpuFp8Tensor **out) {
    std::lock_guard<std::recursive_mutex> lk(big_lock());
    clear_error(F_FP8);
    if (!out || !w || !scale_inv_bf16) {
        set_error(F_FP8, "fp8 upload: NULL pointer");
        return OMEGA_GPU_BAD_ARGS;
    }
    *out = nullptr;
    int rc = check_tensor_shape(F_FP8, experts, n, k);
    if (rc) return rc;
    Ctx *c = ctx(F_FP8);
    if (!c) return OMEGA_GPU_CHIP_FAIL;
    const size_t wbytes = (size_t)experts * n * k;
    const size_t ns = (size_t)experts * (n / 128) * (k / 128);
    std::vector<float> sf(ns);
    const float fold = knobs().fp8_no_fold ? 0x1p-56f : 1.0f;
    for (size_t i = 0; i < ns; ++i) {
        uint32_t u = (uint32_t)scale_inv_bf16[i] << 16;
        float v;
        memcpy(&v, &u, 4);
        sf[i] = v * fold;
    }
    OmegaGpuFp8Tensor *t = new OmegaGpuFp8Tensor();
    t->experts = experts;
    t->n = n;
    t->k = k;
    uint8_t *raw = nullptr;
    uint32_t *flag = nullptr;
    hipError_t e = hipMalloc(&t->w, wbytes);
    if (e == hipSuccess) e = hipMalloc(&t->s, ns * 4);
    if (e == hipSuccess) e = hipMalloc(&raw, wbytes);
    if (e == hipSuccess) e = hipMalloc(&flag, 4);
    if (e == hipSuccess) e = hipMemsetAsync(flag, 0, 4, c->stream);
    if (e == hipSuccess) e = hipMemcpyAsync(raw, w, wbytes, hipMemcpyHostToDevice, c->stream);
    if (e == hipSuccess) e = hipMemcpyAsync(t->s, sf.data(), ns * 4, hipMemcpyHostToDevice, c->stream);
    if (e == hipSuccess) e = launch_fp8_relayout(raw, t->w, experts, n, k, flag, c->stream);
    uint32_t nan_seen = 0;
    if (e == hipSuccess) e = hipMemcpyAsync(&nan_seen, flag, 4, hipMemcpyDeviceToHost, c->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(c->stream);
    if (raw) (void)hipFree(raw);
    if (flag) (void)hipFree(flag);
    if (e != hipSuccess) {
        set_error(F_FP8, "fp8 upload of %zu bytes: %s", wbytes, hipGetErrorString(e));
        if (t->w) (void)hipFree(t->w);
        if (t->s) (void)hipFree(t->s);
        delete t;
        return e == hipErrorOutOfMemory ? OMEGA_GPU_TOO_LARGE : OMEGA_GPU_CHIP_FAIL;
    }
    if (nan_seen) {
        set_error(F_FP8, "NAN_WEIGHT: an e4m3 NaN code (0x7f/0xff) in the weights");
        (void)hipFree(t->w);
        (void)hipFree(t->s);
        delete t;
        return OMEGA_GPU_BAD_ARGS;
    }
    *out = t;
    return OMEGA_GPU_OK;
}

void omega_gpu_synth_bf16_host(uint64_t seed, uint64_t tensor_id, size_t count, float sigma,
                               int one_plus, uint16_t *out) {
    // the host twin of the device generator (k_bf16_synth / synth_normal)
    const uint64_t base = synth_base(seed, tensor_id);
    const float c = sigma * (1.0f / 65536.0f);
    for (size_t i = 0; i < count; ++i) {
        uint64_t b = base + (uint64_t)i * 3;
        int32_t sum = 0;
        for (int j = 0; j < 3; ++j) {
            uint64_t z = b + (uint64_t)j + 0x9E3779B97F4A7C15ull;
            z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
            z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
            z ^= z >> 31;
            sum += (int32_t)(z & 0xffff) + (int32_t)((z >> 16) & 0xffff) +
                   (int32_t)((z >> 32) & 0xffff) + (int32_t)((z >> 48) & 0xffff);
        }
        float v = (float)(sum - 393210) * c;
        if (one_plus) v = 1.0f + v;
        uint32_t u;
        memcpy(&u, &v, 4);
        out[i] = (uint16_t)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
    }
}

int omega_gpu_fp8_tensor_synth(uint32_t experts, uint32_t n, uint32_t k, uint64_t seed,
                               uint64_t tensor_id, float sigma, OmegaGpuFp8Tensor **out) {
    std::lock_guard<std::recursive_mutex> lk(big_lock());
    clear_error(F_FP8);
    if (!out) return OMEGA_GPU_BAD_ARGS;
    *out = nullptr;
    int rc = check_tensor_shape(F_FP8, experts, n, k);
    if (rc) return rc;
    Ctx *c = ctx(F_FP8);
    if (!c) return OMEGA_GPU_CHIP_FAIL;
    OmegaGpuFp8Tensor *t = new OmegaGpuFp8Tensor();
    t->experts = experts;
    t->n = n;
    t->k = k;
    const size_t wbytes = (size_t)experts * n * k;
    const size_t ns = (size_t)experts * (n / 128) * (k / 128);
    hipError_t e = hipMalloc(&t->w, wbytes);
    if (e == hipSuccess) e = hipMalloc(&t->s, ns * 4);
    if (e == hipSuccess) e = launch_fp8_synth(t->w, t->s, experts, n, k, seed, tensor_id, sigma, c->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(c->stream);
    if (e != hipSuccess) {
        set_error(F_FP8, "fp8 synth: %s", hipGetErrorString(e));
        if (t->w) (void)hipFree(t->w);
        if (t->s) (void)hipFree(t->s);
        delete t;
        return e == hipErrorOutOfMemory ? OMEGA_GPU_TOO_LARGE : OMEGA_GPU_CHIP_FAIL;
    }
    *out = t;
    return OMEGA_GPU_OK;
}

void omega_gpu_fp8_tensor_free(OmegaGpuFp8Tensor *t) {
    if (!t) return;
    std::lock_guard<std::recursive_mutex> lk(big_lock());
    Ctx *c = ctx(F_FP8);
    if (c) (void)hipStreamSynchronize(c->stream);
    if (t->w) (void)hipFree(t->w);
    if (t->s) (void)hipFree(t->s);
    delete t;
}

int omega_gpu_fp8_tensor_entry(const OmegaGpuFp8Tensor *t, uint32_t expert, uint64_t *w_va,
                               uint64_t *s_va) {
    clear_error(F_FP8);
    if (!t || !w_va || !s_va) {
        set_error(F_FP8, "fp8 entry: NULL pointer");
        return OMEGA_GPU_BAD_ARGS;
    }
    if (expert >= t->experts) {
        set_error(F_FP8, "fp8 expert %u >= experts %u", expert, t->experts);
        return OMEGA_GPU_BAD_ARGS;
    }
    *w_va = (uint64_t)(uintptr_t)(t->w + (size_t)expert * t->n * t->k);
    *s_va = (uint64_t)(uintptr_t)(t->s + (size_t)expert * (t->n / 128) * (t->k / 128));
    return OMEGA_GPU_OK;
}

int omega_gpu_fp8_gemv_f32(const OmegaGpuFp8Tensor *t, uint32_t expert, const float *x, float *y,
                           OmegaGpuFp8Info *info) {
    return omega_gpu_fp8_gemv_grouped_f32(t, 1, &expert, x, 1, y, info);
}

int omega_gpu_fp8_gemv_grouped_f32(const OmegaGpuFp8Tensor *t, uint32_t groups,
                                   const uint32_t *expert_ids, const float *x, uint32_t x_rows,
                                   float *y, OmegaGpuFp8Info *info) {
    std::lock_guard<std::recursive_mutex> lk(big_lock());
    const uint64_t t0 = now_ns();
    clear_error(F_FP8);
    if (!t || !expert_ids || !x || !y) {
        set_error(F_FP8, "fp8 gemv: NULL pointer");
        return OMEGA_GPU_BAD_ARGS;
    }
    if (groups == 0 || groups > 64) {
        set_error(F_FP8, "fp8 groups %u outside 1..=64", groups);
        return OMEGA_GPU_BAD_ARGS;
    }
    if (!(x_rows == 1 || x_rows == groups)) {
        set_error(F_FP8, "fp8 x_rows %u must be 1 or groups (%u)", x_rows, groups);
        return OMEGA_GPU_BAD_ARGS;
    }
    for (uint32_t g = 0; g < groups; ++g)
        if (expert_ids[g] >= t->experts) {
            set_error(F_FP8, "fp8 expert id %u >= experts %u", expert_ids[g], t->experts);
            return OMEGA_GPU_BAD_ARGS;
        }
    Ctx *c = ctx(F_FP8);
    if (!c) return OMEGA_GPU_CHIP_FAIL;
    Fp8GemvArgs a;
    a.w = t->w;
    a.s = t->s;
    a.n = t->n;
    a.k = t->k;
    a.groups = groups;
    a.x_stride = x_rows == 1 ? 0 : t->k;
    a.mutant = knobs().fp8_mutant;
    for (uint32_t g = 0; g < groups; ++g) a.ids[g] = expert_ids[g];
    uint64_t el = 0;
    int steps = 0;
    int rc = run_gemv_host(c, t, a, x, (size_t)x_rows * t->k, y, &el, &steps);
    if (rc) return rc;
    fill_info(info, t, groups, a, steps, el, t0, c);
    return OMEGA_GPU_OK;
}

int omega_gpu_fp8_gemv_grouped_dev(const OmegaGpuFp8Tensor *t, uint32_t groups, uint64_t tab_va,
                                   uint64_t x_va, float *y, OmegaGpuFp8Info *info) {
    std::lock_guard<std::recursive_mutex> lk(big_lock());
    const uint64_t t0 = now_ns();
    clear_error(F_FP8);
    if (!t || !y) {
        set_error(F_FP8, "fp8 gemv dev: NULL pointer");
        return OMEGA_GPU_BAD_ARGS;
    }
    if (groups == 0 || groups > 64) {
        set_error(F_FP8, "fp8 groups %u outside 1..=64", groups);
        return OMEGA_GPU_BAD_ARGS;
    }
    if (tab_va == 0 || x_va == 0) {
        set_error(F_FP8, "fp8 device table or row address is 0");
        return OMEGA_GPU_BAD_ARGS;
    }
    Ctx *c = ctx(F_FP8);
    if (!c) return OMEGA_GPU_CHIP_FAIL;
    Fp8GemvArgs a;
    a.tab = reinterpret_cast<const uint64_t *>((uintptr_t)tab_va);
    a.x = reinterpret_cast<const float *>((uintptr_t)x_va);
    a.x_scale = 0x1p-64f;  // the router's row carries x' * 2^64
    a.n = t->n;
    a.k = t->k;
    a.groups = groups;
    a.mutant = knobs().fp8_mutant;
    const int steps = fp8_gemv_plan(a, EPI_STORE);
    if (!counters_fit(c, a)) return OMEGA_GPU_TOO_LARGE;
    const size_t y_floats = (size_t)groups * t->n;
    const size_t y_bytes = (y_floats * 4 + 255) & ~(size_t)255;
    const size_t part = a.splits > 1 ? (size_t)a.splits * y_floats * 4 : 0;
    if (!ensure_scratch(F_FP8, c, y_bytes + part) || !ensure_pinned(F_FP8, c, y_bytes))
        return OMEGA_GPU_CHIP_FAIL;
    uint8_t *dev = static_cast<uint8_t *>(c->scratch);
    a.y = reinterpret_cast<float *>(dev);
    a.partial = reinterpret_cast<float *>(dev + y_bytes);
    a.counters = counters(c);
    OMEGA_HIP(F_FP8, hipEventRecord(c->ev0, c->stream));
    OMEGA_HIP(F_FP8, launch_fp8_gemv(a, steps, c->stream));
    OMEGA_HIP(F_FP8, hipEventRecord(c->ev1, c->stream));
    OMEGA_HIP(F_FP8, hipMemcpyAsync(c->pin, a.y, y_floats * 4, hipMemcpyDeviceToHost, c->stream));
    OMEGA_HIP(F_FP8, hipStreamSynchronize(c->stream));
    memcpy(y, c->pin, y_floats * 4);
    fill_info(info, t, groups, a, steps, event_ns(c), t0, c);
    return OMEGA_GPU_OK;
}

int omega_gpu_fp8_gemv_dev(const OmegaGpuFp8Tensor *t, uint32_t expert, const float *x_dev,
                           float *y_dev) {
    std::lock_guard<std::recursive_mutex> lk(big_lock());
    clear_error(F_FP8);
    if (!t || !x_dev || !y_dev || expert >= t->experts) {
        set_error(F_FP8, "fp8 gemv_dev: bad arguments");
        return OMEGA_GPU_BAD_ARGS;
    }
    Ctx *c = ctx(F_FP8);
    if (!c) return OMEGA_GPU_CHIP_FAIL;
    Fp8GemvArgs a;
    a.w = t->w;
    a.s = t->s;
    a.n = t->n;
    a.k = t->k;
    a.groups = 1;
    a.ids[0] = expert;
    a.x = x_dev;
    a.y = y_dev;
    a.mutant = knobs().fp8_mutant;
    const int steps = fp8_gemv_plan(a, EPI_STORE);
    if (!counters_fit(c, a)) return OMEGA_GPU_TOO_LARGE;
    if (a.splits > 1) {
        if (!ensure_scratch(F_FP8, c, (size_t)a.splits * t->n * 4)) return OMEGA_GPU_CHIP_FAIL;
        a.partial = static_cast<float *>(c->scratch);
    }
    a.counters = counters(c);
    OMEGA_HIP(F_FP8, launch_fp8_gemv(a, steps, c->stream));
    return OMEGA_GPU_OK;
}

int omega_gpu_fp8_prepare(uint32_t k) {
    clear_error(F_FP8);
    if (k % 128 != 0 || k < 128 || k > 32768) {
        set_error(F_FP8, "fp8 prepare k=%u outside 128..=32768 in steps of 128", k);
        return OMEGA_GPU_BAD_ARGS;
    }
    return OMEGA_GPU_OK;  // kernels are compiled ahead of time: nothing to build or pin
}
void omega_gpu_fp8_seal(int on) { knobs().fp8_sealed = on != 0; }
const char *omega_gpu_fp8_rc_name(int rc) { return rc_name(rc); }
const char *omega_gpu_fp8_last_error(void) { return last_error(F_FP8); }
void omega_gpu_fp8_cache_clear(void) {}
void omega_gpu_fp8_set_shape(uint32_t, uint32_t, uint32_t) {}
void omega_gpu_fp8_set_cta_budget(uint32_t ctas) { knobs().fp8_cta_budget = ctas; }
uint32_t omega_gpu_fp8_grouped_ctas_auto(uint32_t groups) {
    // workgroups per group of a 2048 x 1536 grouped launch (64-row tiles x k-splits)
    (void)groups;
    return (1536 / 64) * (2048 / 16 / 16);
}
void omega_gpu_fp8_test_set_mutant(int mutant) { knobs().fp8_mutant = mutant; }
void omega_gpu_fp8_test_set_no_fold(int on) { knobs().fp8_no_fold = on != 0; }

}  // extern "C"
