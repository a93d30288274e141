// Grouped FP8 GEMM over a row table sorted by expert (omega_gpu_fp8gemm_*).
//
// Contract: crates/aien-omega-fp8/src/lib.rs:514-593 — row i computes expert expert_ids[i] on
// activation row x[token_rows[i]]; expert_ids non-decreasing; y is m*n in row-table order and
// bit-identical to calling the GEMV once per row. m <= 1024 rows, <= 256 segments (runs of one
// expert). GemmInfo (lib.rs:68-91): weight_bytes = the distinct experts' bytes once each,
// streamed_bytes = the sum over segments of passes x n x k.
//
// One launch. For the model's widths (k = 768, 2048, 4096) a wavefront owns RPW weight rows of
// one segment, the same RPW rows and the same lane layout as the GEMV kernel k_fp8_rows. It loads
// them (and their block scales) into registers once, then walks the segment's activation rows:
// the four wavefronts of a workgroup share the segment (n / RPW is a multiple of 4), so each
// activation row is staged once per workgroup in LDS (double-buffered, the next row's loads in
// flight during the current dot), and every output row is the GEMV's own arithmetic on the held
// weights (same phases, same fmaf order, same wavefront reduction), hence bit-identical. One pass
// per segment: streamed_bytes == weight_bytes. Other widths take the same plan over the GEMV's
// runtime-shaped kernel (k_fp8_rows_any), whose weights stream through registers chunk by chunk:
// a pass there covers up to 8 activation rows of a segment, and a longer segment takes more passes.
#include <vector>

#include "kernels.hpp"
#include "rows.hpp"
#include "runtime.hpp"

namespace omega {

struct Fp8GemmArgs {
    const uint8_t *w = nullptr;  // tensor base, [experts][n][k] e4m3
    const float *s = nullptr;    // [experts][n/128][k/128]
    uint32_t n = 0, k = 0, m = 0;
    const float *x = nullptr;    // [m][k] activation rows in row-table order
    float *y = nullptr;          // [m][n]
    const u32x4 *pass = nullptr; // [passes] {expert, first row, rows, 0}
    uint32_t passes = 0;
    int mutant = 0;              // 1 scale dropped; 2 scale block never advances; 3 neighbour row's x
};

// activation row of row-table entry r (mutant 3: the next entry's)
__device__ __forceinline__ const float *gemm_xrow(const Fp8GemmArgs &a, uint32_t r, uint32_t k) {
    if (a.mutant == 3) r = (r + 1) % a.m;
    return a.x + (size_t)r * k;
}

template <int K, int RPW>
__global__ __launch_bounds__(256) void k_fp8_gemm(const Fp8GemmArgs a) {
    using S = Fp8Slab<K, RPW>;
    constexpr int P = S::P;
    static_assert(S::kOneBlock, "RPW divides the 128-row scale block");
    constexpr int NX = (K / 4 + 255) / 256;  // float4 of an activation row per thread
    __shared__ __align__(16) float xs[2][K];
    const uint32_t lane = lane_id();
    const uint32_t wave = __builtin_amdgcn_readfirstlane(blockIdx.x * 4 + (threadIdx.x >> 6));
    const uint32_t per_pass = a.n / RPW;  // a multiple of 4: the workgroup shares its pass
    const uint32_t pi = wave / per_pass, row0 = (wave % per_pass) * RPW;
    const u32x4 d = a.pass[pi];
    const uint32_t e = __builtin_amdgcn_readfirstlane(d.x);
    const uint32_t first = __builtin_amdgcn_readfirstlane(d.y);
    const uint32_t rows = __builtin_amdgcn_readfirstlane(d.z);
    const uint8_t *wexp = a.w + (size_t)e * a.n * K;
    const float *sexp = a.s + (size_t)e * (a.n >> 7) * (K >> 7);

    // the first activation row, then the scales and the held weights (issue order = wait order)
    f32x4 xt[NX];
    {
        const float *xr0 = gemm_xrow(a, first, K);
#pragma unroll
        for (int i = 0; i < NX; ++i) xt[i] = *as_global_f32x4(xr0 + 4 * min(threadIdx.x + 256 * i, (uint32_t)K / 4 - 1));
    }
    __builtin_amdgcn_sched_barrier(0);
    float sc[P];
    S::load_scales(sexp + (size_t)(row0 >> 7) * (K >> 7), lane, 1.0f, a.mutant, sc);
    S slab;
    slab.load(wexp + (size_t)row0 * K, lane);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < NX; ++i)
        if (threadIdx.x + 256 * i < (uint32_t)K / 4) reinterpret_cast<f32x4 *>(xs[0])[threadIdx.x + 256 * i] = xt[i];

    for (uint32_t r = 0; r < rows; ++r) {
        // row r is staged; every wavefront is done with the buffer the next row goes to
        lds_sync();
        const bool more = r + 1 < rows;
        if (more) {
            const float *xn = gemm_xrow(a, first + r + 1, K);
#pragma unroll
            for (int i = 0; i < NX; ++i) xt[i] = *as_global_f32x4(xn + 4 * min(threadIdx.x + 256 * i, (uint32_t)K / 4 - 1));
        }
        float xr[P][16];
        S::load_x_lds(xs[r & 1], lane, xr);
        float acc[RPW];
#pragma unroll
        for (int j = 0; j < RPW; ++j) acc[j] = 0.f;
        slab.dot(xr, sc, acc, lane);
        const float v = reduce_rows(acc, lane) * 1.0f;  // the GEMV's x_scale
        if (lane < (uint32_t)RPW) a.y[(size_t)(first + r) * a.n + row0 + lane] = v;
        if (more) {
#pragma unroll
            for (int i = 0; i < NX; ++i)
                if (threadIdx.x + 256 * i < (uint32_t)K / 4)
                    reinterpret_cast<f32x4 *>(xs[(r + 1) & 1])[threadIdx.x + 256 * i] = xt[i];
        }
    }
}

constexpr uint32_t kGemmAnyRows = 8;  // activation rows per pass of the runtime-shaped kernel
constexpr uint32_t kAnyRowsW = 8;     // weight rows per wavefront at most (1024 / gcd(k, 1024))

// k_fp8_rows_any's arithmetic for up to 8 activation rows on one pass over the weights
__global__ __launch_bounds__(256) void k_fp8_gemm_any(const Fp8GemmArgs a, uint32_t rpw) {
    const uint32_t lane = lane_id();
    const uint32_t wave = __builtin_amdgcn_readfirstlane(blockIdx.x * 4 + (threadIdx.x >> 6));
    const uint32_t per_pass = a.n / rpw;
    if (wave >= a.passes * per_pass) return;
    const uint32_t pi = wave / per_pass, row0 = (wave % per_pass) * rpw;
    const u32x4 d = a.pass[pi];
    const uint32_t e = __builtin_amdgcn_readfirstlane(d.x);
    const uint32_t first = __builtin_amdgcn_readfirstlane(d.y);
    const uint32_t rows = __builtin_amdgcn_readfirstlane(d.z);  // 1 ..= 8
    const uint32_t k = a.k;
    const uint8_t *wexp = a.w + (size_t)e * a.n * k;
    const float *sexp = a.s + (size_t)e * (a.n >> 7) * (k >> 7);
    const gu32x4 *base = as_global(wexp + (size_t)row0 * k) + lane;
    const float *srow = sexp + (size_t)(row0 >> 7) * (k >> 7);
    const float *xg[kGemmAnyRows];
#pragma unroll
    for (uint32_t t = 0; t < kGemmAnyRows; ++t) xg[t] = gemm_xrow(a, first + min(t, rows - 1), k);
    const uint32_t ch = rpw * k / 1024;
    float acc[kGemmAnyRows][kAnyRowsW];
#pragma unroll
    for (uint32_t t = 0; t < kGemmAnyRows; ++t)
#pragma unroll
        for (uint32_t j = 0; j < kAnyRowsW; ++j) acc[t][j] = 0.f;
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
            const uint32_t cb = a.mutant == 2 ? 0u : col >> 7;
            const float sc = (a.mutant == 1 ? 1.0f : *as_global_f32(srow + cb)) * 1.0f;
#pragma unroll
            for (uint32_t t = 0; t < kGemmAnyRows; ++t) {
                if (t >= rows) break;
                float xx[16];
                const gf32x4 *xq = as_global_f32x4(xg[t] + col);
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const f32x4 u = xq[q];
                    xx[4 * q] = u.x;
                    xx[4 * q + 1] = u.y;
                    xx[4 * q + 2] = u.z;
                    xx[4 * q + 3] = u.w;
                }
                const float p = fp8_dot16(v[i], xx);
#pragma unroll
                for (uint32_t j = 0; j < kAnyRowsW; ++j) acc[t][j] = (rl == j) ? fmaf(p, sc, acc[t][j]) : acc[t][j];
            }
        }
    }
#pragma unroll
    for (uint32_t t = 0; t < kGemmAnyRows; ++t) {
        if (t >= rows) break;
        const float v = reduce_rows(acc[t], lane);
        if (lane < rpw) a.y[(size_t)(first + t) * a.n + row0 + lane] = v;
    }
}

template <int K, int RPW>
static hipError_t launch_gemm_k(const Fp8GemmArgs &a, hipStream_t st) {
    const uint32_t waves = a.passes * (a.n / RPW);
    OMEGA_LAUNCH((k_fp8_gemm<K, RPW>), dim3(waves / 4), dim3(256), 0, st, a);
    return hipGetLastError();
}

// the compiled-in widths hold the weights for a whole segment
static bool gemm_holds(uint32_t k) { return k == 768 || k == 2048 || k == 4096; }

static hipError_t launch_gemm(const Fp8GemmArgs &a, hipStream_t st) {
    switch (a.k) {
    case 768: return launch_gemm_k<768, 8>(a, st);
    case 2048: return launch_gemm_k<2048, 4>(a, st);
    case 4096: return launch_gemm_k<4096, 2>(a, st);
    default: {
        const uint32_t rpw = fp8_rows_per_wave(a.k);
        const uint32_t waves = a.passes * (a.n / rpw);
        OMEGA_LAUNCH(k_fp8_gemm_any, dim3((waves + 3) / 4), dim3(256), 0, st, a, rpw);
        return hipGetLastError();
    }
    }
}

}  // namespace omega

using namespace omega;

extern "C" {

int omega_gpu_fp8gemm_f32(const OmegaGpuFp8Tensor *t, uint32_t m, const uint32_t *expert_ids,
                          const uint32_t *token_rows, const float *x, uint32_t x_rows, float *y,
                          OmegaGpuFp8GemmInfo *info) {
    std::lock_guard<std::recursive_mutex> lk(big_lock());
    const uint64_t t0 = now_ns();
    clear_error(F_GEMM);
    if (!t || !expert_ids || !token_rows || !x || !y) {
        set_error(F_GEMM, "fp8 gemm: NULL pointer");
        return OMEGA_GPU_BAD_ARGS;
    }
    if (m == 0 || m > OMEGA_GPU_FP8GEMM_MAX_ROWS) {
        set_error(F_GEMM, "fp8 gemm rows %u outside 1..=1024", m);
        return OMEGA_GPU_BAD_ARGS;
    }
    if (x_rows == 0) {
        set_error(F_GEMM, "fp8 gemm x has no rows");
        return OMEGA_GPU_BAD_ARGS;
    }
    uint32_t segments = 1;
    for (uint32_t i = 0; i < m; ++i) {
        if (expert_ids[i] >= t->experts) {
            set_error(F_GEMM, "fp8 gemm expert id %u >= experts %u", expert_ids[i], t->experts);
            return OMEGA_GPU_BAD_ARGS;
        }
        if (token_rows[i] >= x_rows) {
            set_error(F_GEMM, "fp8 gemm token row %u >= x rows %u", token_rows[i], x_rows);
            return OMEGA_GPU_BAD_ARGS;
        }
        if (i > 0 && expert_ids[i] < expert_ids[i - 1]) {
            set_error(F_GEMM, "fp8 gemm expert ids must be sorted (non-decreasing)");
            return OMEGA_GPU_BAD_ARGS;
        }
        if (i > 0 && expert_ids[i] != expert_ids[i - 1]) ++segments;
    }
    if (segments > OMEGA_GPU_FP8GEMM_MAX_SEGMENTS) {
        set_error(F_GEMM, "fp8 gemm segments %u > 256", segments);
        return OMEGA_GPU_BAD_ARGS;
    }
    if (t->n % 128 != 0 || t->k % 128 != 0) {  // the upload's own rule; the kernels rely on it
        set_error(F_GEMM, "fp8 gemm tensor %ux%u is not in 128-blocks", t->n, t->k);
        return OMEGA_GPU_BAD_ARGS;
    }
    Ctx *c = ctx(F_GEMM);
    if (!c) return OMEGA_GPU_CHIP_FAIL;
    const size_t k = t->k, n = t->n;
    // passes: one per segment where the weights are held, else runs of up to 8 rows
    const bool holds = gemm_holds(t->k);
    std::vector<u32x4> pass;
    uint32_t passes_max = 0, mt = 0;
    uint64_t streamed = 0;
    for (uint32_t i = 0; i < m;) {
        uint32_t j = i;
        while (j < m && expert_ids[j] == expert_ids[i]) ++j;
        const uint32_t len = j - i, step = holds ? len : kGemmAnyRows;
        uint32_t np = 0;
        for (uint32_t r = i; r < j; r += step, ++np) {
            const uint32_t cnt = j - r < step ? j - r : step;
            pass.push_back(u32x4{expert_ids[i], r, cnt, 0u});
            mt = mt > cnt ? mt : cnt;
        }
        passes_max = passes_max > np ? passes_max : np;
        streamed += (uint64_t)np * n * k;
        i = j;
    }
    const size_t xb = ((size_t)m * k * 4 + 255) & ~(size_t)255;
    const size_t pb = (pass.size() * sizeof(u32x4) + 255) & ~(size_t)255;
    const size_t yb = ((size_t)m * n * 4 + 255) & ~(size_t)255;
    if (!ensure_scratch(F_GEMM, c, xb + pb + yb) || !ensure_pinned(F_GEMM, c, xb + pb + yb))
        return OMEGA_GPU_CHIP_FAIL;
    uint8_t *dev = static_cast<uint8_t *>(c->scratch);
    uint8_t *pin = static_cast<uint8_t *>(c->pin);
    for (uint32_t i = 0; i < m; ++i) memcpy(pin + (size_t)i * k * 4, x + (size_t)token_rows[i] * k, k * 4);
    memcpy(pin + xb, pass.data(), pass.size() * sizeof(u32x4));
    OMEGA_HIP(F_GEMM, hipMemcpyAsync(dev, pin, xb + pb, hipMemcpyHostToDevice, c->stream));
    Fp8GemmArgs a;
    a.w = t->w;
    a.s = t->s;
    a.n = t->n;
    a.k = t->k;
    a.m = m;
    a.x = reinterpret_cast<const float *>(dev);
    a.pass = reinterpret_cast<const u32x4 *>(dev + xb);
    a.passes = (uint32_t)pass.size();
    a.y = reinterpret_cast<float *>(dev + xb + pb);
    a.mutant = knobs().gemm_mutant;
    OMEGA_HIP(F_GEMM, hipEventRecord(c->ev0, c->stream));
    OMEGA_HIP(F_GEMM, launch_gemm(a, c->stream));
    OMEGA_HIP(F_GEMM, hipEventRecord(c->ev1, c->stream));
    OMEGA_HIP(F_GEMM, hipMemcpyAsync(pin + xb + pb, dev + xb + pb, (size_t)m * n * 4, hipMemcpyDeviceToHost, c->stream));
    OMEGA_HIP(F_GEMM, hipStreamSynchronize(c->stream));
    memcpy(y, pin + xb + pb, (size_t)m * n * 4);
    if (info) {
        const uint32_t rpw = fp8_rows_per_wave(t->k);
        memset(info, 0, sizeof(*info));
        info->rows = m;
        info->segments = segments;
        info->n = t->n;
        info->k = t->k;
        info->mt = mt;
        info->warps_per_cta = 4;
        info->lane_bytes = 16;
        info->grid_x = (a.passes * (t->n / rpw) + 3) / 4;
        info->grid_y = 1;
        info->passes_max = passes_max;
        info->weight_bytes = (uint64_t)segments * n * k;
        info->streamed_bytes = streamed;
        info->elapsed_ns = event_ns(c);
        info->call_ns = now_ns() - t0;
        info->completion_marker = 1;
        info->kernel_cache_hit = true;
    }
    return OMEGA_GPU_OK;
}

int omega_gpu_fp8gemm_prepare(uint32_t k) {
    clear_error(F_GEMM);
    if (k % 128 != 0 || k < 128 || k > 32768) {
        set_error(F_GEMM, "fp8 gemm prepare k=%u outside 128..=32768 in steps of 128", k);
        return OMEGA_GPU_BAD_ARGS;
    }
    return OMEGA_GPU_OK;
}
const char *omega_gpu_fp8gemm_rc_name(int rc) { return rc_name(rc); }
const char *omega_gpu_fp8gemm_last_error(void) { return last_error(F_GEMM); }
// 0 off; 1 scale dropped; 2 scale block never advances; 3 neighbour row's x
void omega_gpu_fp8gemm_test_set_mutant(int mutant) { knobs().gemm_mutant = mutant; }

}  // extern "C"
