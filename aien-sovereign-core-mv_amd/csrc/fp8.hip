// FP8 e4m3 block-scaled GEMV for gfx950: upload (row-major, NaN scan), the streaming GEMV
// kernels, the device-side synthetic generator, and the omega_gpu_fp8_* entry points.
//
// Contract: crates/aien-omega-fp8/src/lib.rs:16-29 — y[g][r] = sum_c e4m3(W[id_g][r][c]) *
// x[row(g)][c] * bf16(scale[id_g][r/128][c/128]) in f32.
//
// Kernel shape (rows.hpp): one wavefront per RPW consecutive rows of one group, workgroups of
// four independent wavefronts, no split along k and so no reduction between workgroups. For the
// model's k (768, 2048, 4096) the shape is compiled in: each lane keeps its P activation phases
// and their block scales in registers, streams RPW*k/1024 chunks of 1 KiB, widens bytes with
// the native OCP-fp8 convert (v_cvt_pk_f32_fp8) and accumulates 16-column dots in f32, each
// scaled by its 128x128 block scale. Other k take a runtime-shaped kernel with the same
// arithmetic. Optional prologue: the input RMSNorm (f64 sum of squares of the lane phases,
// which partition the row) and the embedding gather; optional epilogue: add into the residual.
#include <cmath>
#include <cstdio>
#include <vector>

#include "kernels.hpp"
#include "rows.hpp"
#include "runtime.hpp"

namespace omega {

// expert weights and scales of group g (mutant 3 reads the next group's weights)
__device__ __forceinline__ void group_tensor(const Fp8RowsArgs &a, uint32_t g, uint32_t k,
                                             const uint8_t *&wexp, const float *&sexp) {
    uint32_t gsel = g;
    if (a.mutant == 3 && a.groups > 1) gsel = (g + 1) % a.groups;
    if (a.tab) {
        wexp = reinterpret_cast<const uint8_t *>(a.tab[2 * gsel]);
        sexp = reinterpret_cast<const float *>(a.tab[2 * g + 1]);
    } else {
        const size_t e = a.ids[gsel];
        wexp = a.w + e * (size_t)a.n * k;
        sexp = a.s + e * (size_t)(a.n >> 7) * (k >> 7);
    }
}

// XL: the workgroup's four wavefronts share one group (groups == 1 or n / RPW a multiple of 4),
// so the activation row (and the norm weights) is staged once per workgroup in LDS instead of
// once per wavefront — a CU's loads share one path, and the replicated activation bytes would
// otherwise double its traffic.
//
// ONE: one group, no group table, n / RPW a multiple of 4 (the decode projections): the
// expert's weight and scale pointers, the activation row, the norm weights, the output row and
// the test mutant come in as leading scalar kernel arguments, which gfx950 preloads into SGPRs
// before the wave starts (-amdgpu-kernarg-preload-count), so the loads ahead of the weight
// stream wait on no scalar round trip; every wavefront is live. The general form reads the
// group's expert id, then its table entry, from the arguments: a chain of dependent scalar
// loads (0.29 us per q|k|v launch, measured) ahead of the stream.
template <int K, int RPW, int EPI, int XSRC, bool XL, bool ONE>
__device__ __forceinline__ void fp8_rows_body(const Fp8RowsArgs &a, const uint8_t *w1, const float *s1,
                                              const float *x1, const float *nw1, float *y1,
                                              int mut1) {
    using S = Fp8Slab<K, RPW>;
    constexpr int P = S::P;
    constexpr int NX = (K / 4 + 255) / 256;  // float4 of the row per thread when staged
    __shared__ __align__(16) float xs[XL ? K : 4];
    __shared__ __align__(16) float ws[XL && XSRC != XS_F32 ? K : 4];
    const uint32_t lane = lane_id();
    // wave-uniform (scalar registers): the group's weight pointer then comes from a scalar
    // kernel-argument load instead of a vector round trip ahead of the weight stream
    const uint32_t wave = __builtin_amdgcn_readfirstlane(blockIdx.x * 4 + (threadIdx.x >> 6));
    const uint32_t per_group = ONE ? 0 : a.n / RPW;
    const bool live = ONE || wave < a.groups * per_group;
    if (!XL && !live) return;  // with XL every thread takes part in the staging and its barrier
    const uint32_t wv = live ? wave : 0;  // a wavefront past the end streams row 0, unused
    const uint32_t g = ONE ? 0 : wv / per_group, row0 = (ONE ? wv : wv % per_group) * RPW;
    const uint8_t *wexp = w1;
    const float *sexp = s1;
    if constexpr (!ONE) group_tensor(a, g, K, wexp, sexp);
    const float *xrow = ONE ? x1 : a.x + (size_t)g * a.x_stride;
    const float *norm_w = ONE ? nw1 : a.norm_w;
    float *y = ONE ? y1 : a.y;
    const int mutant = ONE ? mut1 : a.mutant;

    // every small load (activation row or phases, norm weights, block scales) goes ahead of the
    // weight stream: vector-memory waits complete in issue order, so waiting on any of them then
    // never waits on the weights
    float xr[P][16];
    float nw[P][16];
    f32x4 xt[NX], wt[NX];
    u32x4 et;
    if constexpr (XL) {
        if (XSRC == XS_EMBED_NORM) {
            static_assert(XSRC != XS_EMBED_NORM || K == 2048, "one 8-value piece of the row per thread");
            const uint32_t tok = *as_global_u32(a.embed_tok) % a.embed_rows;
            et = *as_global(a.embed + (size_t)tok * K + 8 * threadIdx.x);
        } else {
#pragma unroll
            for (int i = 0; i < NX; ++i)
                xt[i] = *as_global_f32x4(xrow + 4 * min(threadIdx.x + 256 * i, (uint32_t)K / 4 - 1));
        }
        if (XSRC != XS_F32) {
#pragma unroll
            for (int i = 0; i < NX; ++i)
                wt[i] = *as_global_f32x4(norm_w + 4 * min(threadIdx.x + 256 * i, (uint32_t)K / 4 - 1));
        }
    } else {
        if (XSRC == XS_EMBED_NORM) {
            const uint32_t tok = *as_global_u32(a.embed_tok) % a.embed_rows;
            S::load_x_bf16(a.embed + (size_t)tok * K, lane, xr);
        } else {
            S::load_x(xrow, lane, xr);
        }
        if (XSRC != XS_F32) S::load_x(norm_w, lane, nw);
    }
    __builtin_amdgcn_sched_barrier(0);  // the activation loads stay ahead of everything below
    // block scales of row0's 128-row block, and of the last row's when RPW does not divide 128
    float sc[2][P];
    S::load_scales(sexp + (size_t)(row0 >> 7) * (K >> 7), lane, 1.0f, mutant, sc[0]);
    if constexpr (!S::kOneBlock)
        S::load_scales(sexp + (size_t)((row0 + RPW - 1) >> 7) * (K >> 7), lane, 1.0f, mutant, sc[1]);
    // the residual row of the epilogue, read now rather than after the dot
    const size_t yrow = (ONE ? 0 : (size_t)g * a.n) + row0 + min(lane, (uint32_t)RPW - 1);
    const float yres = EPI == EPI_RESID ? *as_global_f32(y + yrow) : 0.f;
    S slab;
    slab.load(wexp + (size_t)row0 * K, lane);
    // every load is issued before any arithmetic (the scheduler would otherwise sink the weight
    // loads between the dots, one round trip each)
    __builtin_amdgcn_sched_barrier(0);

    if constexpr (XL) {
        if (XSRC == XS_EMBED_NORM) {
            f32x4 *d = reinterpret_cast<f32x4 *>(xs + 8 * threadIdx.x);
            d[0] = f32x4{bf16_lo(et[0]), bf16_hi(et[0]), bf16_lo(et[1]), bf16_hi(et[1])};
            d[1] = f32x4{bf16_lo(et[2]), bf16_hi(et[2]), bf16_lo(et[3]), bf16_hi(et[3])};
        } else {
#pragma unroll
            for (int i = 0; i < NX; ++i)
                if (threadIdx.x + 256 * i < (uint32_t)K / 4) reinterpret_cast<f32x4 *>(xs)[threadIdx.x + 256 * i] = xt[i];
        }
        if (XSRC != XS_F32) {
#pragma unroll
            for (int i = 0; i < NX; ++i)
                if (threadIdx.x + 256 * i < (uint32_t)K / 4) reinterpret_cast<f32x4 *>(ws)[threadIdx.x + 256 * i] = wt[i];
        }
        __syncthreads();  // LDS only: the weight stream stays in flight
        S::load_x_lds(xs, lane, xr);
        if (XSRC != XS_F32) S::load_x_lds(ws, lane, nw);
    }

    // RMSNorm is one scale per row: dot with x * w and scale the row sums at the end, so the
    // f64 sum of squares runs beside the weight stream instead of ahead of it
    float scale = a.x_scale;
    if (XSRC != XS_F32) {
        static_assert(XSRC == XS_F32 || P * 16 * 64 == K, "the phases must partition the row");
        if (XSRC == XS_EMBED_NORM && blockIdx.x == 0 && threadIdx.x < 64) {
#pragma unroll
            for (int ph = 0; ph < P; ++ph) {
                float4 *o = reinterpret_cast<float4 *>(a.x_out + S::col_bytes(ph, lane));
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    o[i] = make_float4(xr[ph][4 * i], xr[ph][4 * i + 1], xr[ph][4 * i + 2], xr[ph][4 * i + 3]);
            }
        }
        const double ss = phases_sumsq(xr);
#pragma unroll
        for (int ph = 0; ph < P; ++ph)
#pragma unroll
            for (int i = 0; i < 16; ++i) xr[ph][i] = xr[ph][i] * nw[ph][i];
        scale *= rms_scale(ss, K, a.eps);
    }
    float acc[RPW];
#pragma unroll
    for (int j = 0; j < RPW; ++j) acc[j] = 0.f;
    if constexpr (S::kOneBlock) slab.dot(xr, sc[0], acc, lane);
    else slab.dot2(xr, sc, row0, acc);
    const float v = reduce_rows(acc, lane) * scale;
    if (live && lane < (uint32_t)RPW) y[yrow] = EPI == EPI_STORE ? v : yres + v;
}

template <int K, int RPW, int EPI, int XSRC, bool XL>
__global__ __launch_bounds__(256) void k_fp8_rows(const Fp8RowsArgs a) {
    fp8_rows_body<K, RPW, EPI, XSRC, XL, false>(a, nullptr, nullptr, nullptr, nullptr, nullptr, 0);
}

// w and s point at the expert's own rows (the host adds the group's expert offset)
template <int K, int RPW, int EPI, int XSRC>
__global__ __launch_bounds__(256) void k_fp8_rows1(const uint8_t *w, const float *s, const float *x,
                                                  const float *norm_w, float *y, int mutant,
                                                  const Fp8RowsArgs a) {
    fp8_rows_body<K, RPW, EPI, XSRC, true, true>(a, w, s, x, norm_w, y, mutant);
}

// Any k (a multiple of 128 up to 32768): rows per wavefront rpw = 1024 / gcd(k, 1024) <= 8,
// activations read per chunk, the chunk's row found per lane.
constexpr uint32_t kAnyRows = 8;

__global__ __launch_bounds__(256) void k_fp8_rows_any(const Fp8RowsArgs a, uint32_t rpw) {
    const uint32_t lane = lane_id();
    const uint32_t wave = __builtin_amdgcn_readfirstlane(blockIdx.x * 4 + (threadIdx.x >> 6));
    const uint32_t per_group = a.n / rpw;
    if (wave >= a.groups * per_group) return;
    const uint32_t g = wave / per_group, row0 = (wave % per_group) * rpw;
    const uint32_t k = a.k;
    const uint8_t *wexp;
    const float *sexp;
    group_tensor(a, g, k, wexp, sexp);
    const float *xg = a.x + (size_t)g * a.x_stride;
    const gu32x4 *base = as_global(wexp + (size_t)row0 * k) + lane;
    const float *srow = sexp + (size_t)(row0 >> 7) * (k >> 7);
    const uint32_t ch = rpw * k / 1024;
    float acc[kAnyRows];
#pragma unroll
    for (int j = 0; j < (int)kAnyRows; ++j) acc[j] = 0.f;
    for (uint32_t c0 = 0; c0 < ch; c0 += 8) {
        u32x4 v[8];
#pragma unroll
        for (int i = 0; i < 8; ++i)
            if (c0 + i < ch) v[i] = __builtin_nontemporal_load(base + (size_t)(c0 + i) * 64);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            if (c0 + i >= ch) break;
            const uint32_t o = (c0 + i) * 1024 + 16 * lane;
            const uint32_t rl = o / k, col = o % k;
            float xx[16];
            const gf32x4 *xq = as_global_f32x4(xg + col);
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const f32x4 t = xq[q];
                xx[4 * q] = t.x;
                xx[4 * q + 1] = t.y;
                xx[4 * q + 2] = t.z;
                xx[4 * q + 3] = t.w;
            }
            const uint32_t cb = a.mutant == 2 ? 0u : col >> 7;
            const float sc = (a.mutant == 1 ? 1.0f : *as_global_f32(srow + cb)) * a.x_scale;
            const float p = fp8_dot16(v[i], xx);
#pragma unroll
            for (int j = 0; j < (int)kAnyRows; ++j) acc[j] = (rl == (uint32_t)j) ? fmaf(p, sc, acc[j]) : acc[j];
        }
    }
    const float v = reduce_rows(acc, lane);
    if (lane < rpw) a.y[(size_t)g * a.n + row0 + lane] = v;
}

uint32_t fp8_rows_per_wave(uint32_t k) {
    switch (k) {
    case 768: return 8;
    case 2048: return 4;
    case 4096: return 2;
    default: {
        uint32_t a = k, b = 1024;
        while (b) {
            const uint32_t t = a % b;
            a = b;
            b = t;
        }
        return 1024 / a;
    }
    }
}

uint32_t fp8_rows_blocks(const Fp8RowsArgs &a) {
    const uint32_t waves = a.groups * (a.n / fp8_rows_per_wave(a.k));
    return (waves + 3) / 4;
}

template <int K, int RPW, int EPI, int XSRC>
static hipError_t launch_k(const Fp8RowsArgs &a, hipStream_t st) {
    const uint32_t waves = a.groups * (a.n / RPW);
    // the activation row is staged per workgroup when the workgroup's wavefronts share a group
    const bool xl = a.groups == 1 || (a.n / RPW) % 4 == 0;
    if (a.groups == 1 && !a.tab && waves % 4 == 0) {
        const size_t e = a.ids[0];
        OMEGA_LAUNCH((k_fp8_rows1<K, RPW, EPI, XSRC>), dim3(waves / 4), dim3(256), 0, st,
                     a.w + e * a.n * K, a.s + e * (a.n >> 7) * (K >> 7), a.x, a.norm_w, a.y, a.mutant, a);
    } else if (xl) {
        OMEGA_LAUNCH((k_fp8_rows<K, RPW, EPI, XSRC, true>), dim3((waves + 3) / 4), dim3(256), 0, st, a);
    } else {
        OMEGA_LAUNCH((k_fp8_rows<K, RPW, EPI, XSRC, false>), dim3((waves + 3) / 4), dim3(256), 0, st, a);
    }
    return hipGetLastError();
}

hipError_t launch_fp8_rows(const Fp8RowsArgs &a, int epi, int xsrc, hipStream_t st) {
    if (xsrc != XS_F32 && a.k != 2048) return hipErrorInvalidValue;
    if (epi == EPI_STORE && xsrc == XS_F32) {
        switch (a.k) {
        case 768: return launch_k<768, 8, EPI_STORE, XS_F32>(a, st);
        case 2048: return launch_k<2048, 4, EPI_STORE, XS_F32>(a, st);
        case 4096: return launch_k<4096, 2, EPI_STORE, XS_F32>(a, st);
        default:
            OMEGA_LAUNCH(k_fp8_rows_any, dim3(fp8_rows_blocks(a)), dim3(256), 0, st, a,
                         fp8_rows_per_wave(a.k));
            return hipGetLastError();
        }
    }
    // the normed GEMVs are the q|k|v projection (n = 5120): 5 rows per wavefront make 1024
    // wavefronts, one per SIMD, where 4 rows would leave a quarter of the SIMDs with two
    if (epi == EPI_STORE && xsrc == XS_NORM)
        return a.n % 5 == 0 && a.groups == 1 ? launch_k<2048, 5, EPI_STORE, XS_NORM>(a, st)
                                              : launch_k<2048, 4, EPI_STORE, XS_NORM>(a, st);
    if (epi == EPI_STORE && xsrc == XS_EMBED_NORM)
        return a.n % 5 == 0 && a.groups == 1 ? launch_k<2048, 5, EPI_STORE, XS_EMBED_NORM>(a, st)
                                              : launch_k<2048, 4, EPI_STORE, XS_EMBED_NORM>(a, st);
    if (epi == EPI_RESID && xsrc == XS_F32 && a.k == 4096) return launch_k<4096, 2, EPI_RESID, XS_F32>(a, st);
    return hipErrorInvalidValue;
}

// ---------------------------------------------------------------- upload check
__global__ void k_fp8_nan_scan(const uint8_t *__restrict__ w, size_t chunks, uint32_t *flag) {
    uint32_t bad = 0;
    for (size_t c = blockIdx.x * (size_t)blockDim.x + threadIdx.x; c < chunks;
         c += (size_t)gridDim.x * blockDim.x) {
        const u32x4 v = __builtin_nontemporal_load(as_global(w) + c);
        // e4m3 NaN: S.1111.111 in any byte
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const uint32_t x = v[q] & 0x7f7f7f7fu;
            const uint32_t m = ~(x ^ 0x7f7f7f7fu);  // bytes equal to 0x7f have all 8 bits set
            bad |= (m & (m >> 1) & (m >> 2) & (m >> 3) & (m >> 4) & (m >> 5) & (m >> 6) & 0x01010101u);
        }
    }
    if (bad) atomicOr(flag, 1u);
}

hipError_t launch_fp8_nan_scan(const uint8_t *w, size_t bytes, uint32_t *flag, hipStream_t st) {
    hipLaunchKernelGGL(k_fp8_nan_scan, dim3(2048), dim3(256), 0, st, w, bytes / 16, flag);
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
    __shared__ float red[4];
    float amax = 0.f;
    for (uint32_t i = threadIdx.x; i < 128 * 128; i += 256) {
        const uint32_t r = rb * 128 + (i >> 7), col = cb * 128 + (i & 127);
        amax = fmaxf(amax, fabsf(synth_normal(base, ebase + (size_t)r * k + col, c)));
    }
    for (int o = 32; o > 0; o >>= 1) amax = fmaxf(amax, __shfl_xor(amax, o, 64));
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = amax;
    __syncthreads();
    amax = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    const uint16_t sb = bf16_rne(amax / 448.0f);
    const float sv = bf16_to_f32(sb);
    if (threadIdx.x == 0) s[((size_t)e * nb + rb) * kbk + cb] = sv;
    for (uint32_t i = threadIdx.x; i < 128 * 128; i += 256) {
        const uint32_t r = rb * 128 + (i >> 7), col = cb * 128 + (i & 127);
        const float v = synth_normal(base, ebase + (size_t)r * k + col, c);
        w[ebase + (size_t)r * k + col] = f32_to_e4m3_rne(v / sv);
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

// bf16 synthetic rows, row-major: element (r, c) of [n][k] is N(0, sigma)
__global__ void k_bf16_synth(uint16_t *w, size_t total, uint64_t base, float c) {
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < total;
         i += (size_t)gridDim.x * blockDim.x)
        w[i] = bf16_rne(synth_normal(base, i, c));
}

hipError_t launch_bf16_synth(uint16_t *w, uint32_t n, uint32_t k, uint64_t seed, uint64_t tensor,
                             float sigma, hipStream_t st) {
    const float c = sigma * (1.0f / 65536.0f);
    hipLaunchKernelGGL(k_bf16_synth, dim3(8192), dim3(256), 0, st, w, (size_t)n * k,
                       synth_base(seed, tensor), c);
    return hipGetLastError();
}

hipError_t launch_bf16_synth_count(uint16_t *w, size_t count, uint64_t seed, uint64_t tensor, float sigma,
                                   hipStream_t st) {
    const float c = sigma * (1.0f / 65536.0f);
    hipLaunchKernelGGL(k_bf16_synth, dim3(8192), dim3(256), 0, st, w, count, synth_base(seed, tensor), c);
    return hipGetLastError();
}

// row-major e4m3 -> the tiled twin (runtime.hpp): one thread per 16 output bytes
__global__ __launch_bounds__(256) void k_fp8_tile(const uint8_t *w, uint8_t *wt, uint32_t n, uint32_t k,
                                                  size_t pieces) {
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= pieces) return;
    // output piece i: block b = i / 128, lane slot l = i % 64, half h = (i / 64) % 2
    const size_t b = i >> 7;
    const uint32_t h = (uint32_t)(i >> 6) & 1u, l = (uint32_t)i & 63u;
    const uint32_t kbs = k / 128, rts = n / 16;
    const uint32_t kb = (uint32_t)(b % kbs);
    const size_t rt_all = b / kbs;  // expert * rts + rt
    const uint32_t r = l & 15u, gq = l >> 4;
    const size_t row = (rt_all / rts) * n + (rt_all % rts) * 16 + r;  // expert * n + 16 rt + r
    const u32x4 v = *as_global(w + row * k + (size_t)kb * 128 + 64 * h + 16 * gq);
    *reinterpret_cast<u32x4 *>(wt + i * 16) = v;
}

hipError_t launch_fp8_tile(const uint8_t *w, uint8_t *wt, uint32_t experts, uint32_t n, uint32_t k,
                           hipStream_t st) {
    const size_t pieces = (size_t)experts * n * k / 16;
    hipLaunchKernelGGL(k_fp8_tile, dim3((unsigned)((pieces + 255) / 256)), dim3(256), 0, st, w, wt, n, k, pieces);
    return hipGetLastError();
}

// the tiled twin of t, built on first use (not while a graph is being captured: callers build
// it before capture)
int fp8_ensure_tiled(Family f, OmegaGpuFp8Tensor *t) {
    if (t->wt) return OMEGA_GPU_OK;
    Ctx *c = ctx(f);
    if (!c) return OMEGA_GPU_CHIP_FAIL;
    const size_t bytes = (size_t)t->experts * t->n * t->k;
    if (seal_refuses(f, "fp8 tiled weight twin", bytes)) return OMEGA_GPU_TOO_LARGE;
    OMEGA_HIP(f, dev_malloc(&t->wt, bytes));
    hipError_t e = launch_fp8_tile(t->w, t->wt, t->experts, t->n, t->k, c->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(c->stream);
    if (e != hipSuccess) {
        (void)dev_free(t->wt);
        t->wt = nullptr;
        set_error(f, "fp8 tiled twin: %s", hipGetErrorString(e));
        return OMEGA_GPU_CHIP_FAIL;
    }
    return OMEGA_GPU_OK;
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
                      const Fp8RowsArgs &a, uint64_t elapsed, uint64_t t0, Ctx *c) {
    if (!info) return;
    memset(info, 0, sizeof(*info));
    const uint32_t rpw = fp8_rows_per_wave(t->k);
    info->experts = t->experts;
    info->n = t->n;
    info->k = t->k;
    info->groups = groups;
    info->lane_bytes = 16;
    info->rows_per_warp = rpw;
    info->warps_per_cta = 4;
    info->depth = rpw * t->k / 1024;
    info->grid_x = fp8_rows_blocks(a);
    info->grid_y = 1;
    info->steps = t->k / 16;
    info->weight_bytes = (uint64_t)groups * t->n * t->k;
    info->scale_bytes = (uint64_t)groups * (t->n / 128) * (t->k / 128) * 4;
    info->elapsed_ns = elapsed;
    info->call_ns = now_ns() - t0;
    info->completion_marker = 1;
    info->kernel_cache_hit = true;
    fill_chip(info->target_chip, &info->sm_architecture, c);
}

// Runs one GEMV launch with host x/y (the staging path of the standalone entries).
static int run_gemv_host(Ctx *c, const OmegaGpuFp8Tensor *t, Fp8RowsArgs &a, const float *x,
                         size_t x_floats, float *y, uint64_t *elapsed) {
    const size_t y_floats = (size_t)a.groups * t->n;
    const size_t x_bytes = (x_floats * 4 + 255) & ~(size_t)255;
    const size_t y_bytes = (y_floats * 4 + 255) & ~(size_t)255;
    if (!ensure_scratch(F_FP8, c, x_bytes + y_bytes)) return OMEGA_GPU_CHIP_FAIL;
    if (!ensure_pinned(F_FP8, c, x_bytes + y_bytes)) return OMEGA_GPU_CHIP_FAIL;
    uint8_t *dev = static_cast<uint8_t *>(c->scratch);
    float *xd = reinterpret_cast<float *>(dev);
    float *yd = reinterpret_cast<float *>(dev + x_bytes);
    uint8_t *pin = static_cast<uint8_t *>(c->pin);
    memcpy(pin, x, x_floats * 4);
    OMEGA_HIP(F_FP8, hipMemcpyAsync(xd, pin, x_floats * 4, hipMemcpyHostToDevice, c->stream));
    a.x = xd;
    a.y = yd;
    OMEGA_HIP(F_FP8, hipEventRecord(c->ev0, c->stream));
    OMEGA_HIP(F_FP8, launch_fp8_rows(a, EPI_STORE, XS_F32, c->stream));
    OMEGA_HIP(F_FP8, hipEventRecord(c->ev1, c->stream));
    OMEGA_HIP(F_FP8, hipMemcpyAsync(pin + x_bytes, yd, y_floats * 4, hipMemcpyDeviceToHost, c->stream));
    OMEGA_HIP(F_FP8, hipStreamSynchronize(c->stream));
    memcpy(y, pin + x_bytes, y_floats * 4);
    *elapsed = event_ns(c);
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
    uint32_t *flag = nullptr;
    hipError_t e = dev_malloc(&t->w, wbytes);
    if (e == hipSuccess) e = dev_malloc(&t->s, ns * 4);
    if (e == hipSuccess) e = dev_malloc(&flag, 4);
    if (e == hipSuccess) e = hipMemsetAsync(flag, 0, 4, c->stream);
    if (e == hipSuccess) e = hipMemcpyAsync(t->w, w, wbytes, hipMemcpyHostToDevice, c->stream);
    if (e == hipSuccess) e = hipMemcpyAsync(t->s, sf.data(), ns * 4, hipMemcpyHostToDevice, c->stream);
    if (e == hipSuccess) e = launch_fp8_nan_scan(t->w, wbytes, flag, c->stream);
    uint32_t nan_seen = 0;
    if (e == hipSuccess) e = hipMemcpyAsync(&nan_seen, flag, 4, hipMemcpyDeviceToHost, c->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(c->stream);
    if (flag) (void)dev_free(flag);
    if (e != hipSuccess) {
        set_error(F_FP8, "fp8 upload of %zu bytes: %s", wbytes, hipGetErrorString(e));
        if (t->w) (void)dev_free(t->w);
        if (t->s) (void)dev_free(t->s);
        delete t;
        return e == hipErrorOutOfMemory ? OMEGA_GPU_TOO_LARGE : OMEGA_GPU_CHIP_FAIL;
    }
    if (nan_seen) {
        set_error(F_FP8, "NAN_WEIGHT: an e4m3 NaN code (0x7f/0xff) in the weights");
        (void)dev_free(t->w);
        (void)dev_free(t->s);
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

int omega_gpu_synth_bf16_dev(void *dst, uint64_t count, uint64_t seed, uint64_t tensor_id, float sigma) {
    std::lock_guard<std::recursive_mutex> lk(big_lock());
    clear_error(F_BF16);
    if (!dst) {
        set_error(F_BF16, "bf16 synth dev: NULL buffer");
        return OMEGA_GPU_BAD_ARGS;
    }
    Ctx *c = ctx(F_BF16);
    if (!c) return OMEGA_GPU_CHIP_FAIL;
    if (count == 0) return OMEGA_GPU_OK;
    OMEGA_HIP(F_BF16, launch_bf16_synth_count(static_cast<uint16_t *>(dst), count, seed, tensor_id, sigma, c->stream));
    return OMEGA_GPU_OK;
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
    hipError_t e = dev_malloc(&t->w, wbytes);
    if (e == hipSuccess) e = dev_malloc(&t->s, ns * 4);
    if (e == hipSuccess) e = launch_fp8_synth(t->w, t->s, experts, n, k, seed, tensor_id, sigma, c->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(c->stream);
    if (e != hipSuccess) {
        set_error(F_FP8, "fp8 synth: %s", hipGetErrorString(e));
        if (t->w) (void)dev_free(t->w);
        if (t->s) (void)dev_free(t->s);
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
    if (t->w) (void)dev_free(t->w);
    if (t->s) (void)dev_free(t->s);
    if (t->wt) (void)dev_free(t->wt);
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
    Fp8RowsArgs a;
    a.w = t->w;
    a.s = t->s;
    a.n = t->n;
    a.k = t->k;
    a.groups = groups;
    a.x_stride = x_rows == 1 ? 0 : t->k;
    a.mutant = knobs().fp8_mutant;
    for (uint32_t g = 0; g < groups; ++g) a.ids[g] = expert_ids[g];
    uint64_t el = 0;
    int rc = run_gemv_host(c, t, a, x, (size_t)x_rows * t->k, y, &el);
    if (rc) return rc;
    fill_info(info, t, groups, a, el, t0, c);
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
    Fp8RowsArgs a;
    a.tab = reinterpret_cast<const uint64_t *>((uintptr_t)tab_va);
    a.x = reinterpret_cast<const float *>((uintptr_t)x_va);
    a.x_scale = 0x1p-64f;  // the router's row carries x' * 2^64
    a.n = t->n;
    a.k = t->k;
    a.groups = groups;
    a.mutant = knobs().fp8_mutant;
    const size_t y_floats = (size_t)groups * t->n;
    const size_t y_bytes = (y_floats * 4 + 255) & ~(size_t)255;
    if (!ensure_scratch(F_FP8, c, y_bytes) || !ensure_pinned(F_FP8, c, y_bytes)) return OMEGA_GPU_CHIP_FAIL;
    a.y = static_cast<float *>(c->scratch);
    OMEGA_HIP(F_FP8, hipEventRecord(c->ev0, c->stream));
    OMEGA_HIP(F_FP8, launch_fp8_rows(a, EPI_STORE, XS_F32, c->stream));
    OMEGA_HIP(F_FP8, hipEventRecord(c->ev1, c->stream));
    OMEGA_HIP(F_FP8, hipMemcpyAsync(c->pin, a.y, y_floats * 4, hipMemcpyDeviceToHost, c->stream));
    OMEGA_HIP(F_FP8, hipStreamSynchronize(c->stream));
    memcpy(y, c->pin, y_floats * 4);
    fill_info(info, t, groups, a, event_ns(c), t0, c);
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
    Fp8RowsArgs a;
    a.w = t->w;
    a.s = t->s;
    a.n = t->n;
    a.k = t->k;
    a.groups = 1;
    a.ids[0] = expert;
    a.x = x_dev;
    a.y = y_dev;
    a.mutant = knobs().fp8_mutant;
    OMEGA_HIP(F_FP8, launch_fp8_rows(a, EPI_STORE, XS_F32, c->stream));
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
    // workgroups per group of a 1536 x 2048 grouped launch (four wavefronts of 4 rows each)
    (void)groups;
    return 1536 / (4 * 4);
}
void omega_gpu_fp8_test_set_mutant(int mutant) { knobs().fp8_mutant = mutant; }
void omega_gpu_fp8_test_set_no_fold(int on) { knobs().fp8_no_fold = on != 0; }

}  // extern "C"
