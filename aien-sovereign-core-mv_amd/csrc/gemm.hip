// Grouped FP8 GEMM over a row table sorted by expert (omega_gpu_fp8gemm_*).
//
// Contract: crates/aien-omega-fp8/src/lib.rs:514-593 — row i computes expert expert_ids[i] on
// activation row x[token_rows[i]]; expert_ids non-decreasing; y is m*n in row-table order and
// bit-identical to calling the GEMV once per row. m <= 1024 rows, <= 256 segments.
//
// This cut runs the rows through the GEMV kernel in launches of up to 64 rows (the row table
// becomes the group table; every output row is computed by the same wavefront program as the
// single GEMV, hence bit-identical results).
#include <vector>

#include "kernels.hpp"
#include "runtime.hpp"

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
    Ctx *c = ctx(F_GEMM);
    if (!c) return OMEGA_GPU_CHIP_FAIL;
    const size_t k = t->k, n = t->n;
    Fp8RowsArgs a;
    a.w = t->w;
    a.s = t->s;
    a.n = t->n;
    a.k = t->k;
    a.mutant = knobs().gemm_mutant;
    a.groups = 64;
    const size_t xb = ((size_t)m * k * 4 + 255) & ~(size_t)255;
    const size_t yb = ((size_t)m * n * 4 + 255) & ~(size_t)255;
    if (!ensure_scratch(F_GEMM, c, xb + yb) || !ensure_pinned(F_GEMM, c, xb + yb))
        return OMEGA_GPU_CHIP_FAIL;
    uint8_t *dev = static_cast<uint8_t *>(c->scratch);
    uint8_t *pin = static_cast<uint8_t *>(c->pin);
    for (uint32_t i = 0; i < m; ++i) memcpy(pin + (size_t)i * k * 4, x + (size_t)token_rows[i] * k, k * 4);
    OMEGA_HIP(F_GEMM, hipMemcpyAsync(dev, pin, (size_t)m * k * 4, hipMemcpyHostToDevice, c->stream));
    OMEGA_HIP(F_GEMM, hipEventRecord(c->ev0, c->stream));
    uint64_t streamed = 0;
    for (uint32_t r0 = 0; r0 < m; r0 += 64) {
        const uint32_t g = m - r0 < 64 ? m - r0 : 64;
        a.groups = g;
        for (uint32_t i = 0; i < g; ++i) a.ids[i] = expert_ids[r0 + i];
        a.x = reinterpret_cast<const float *>(dev) + (size_t)r0 * k;
        a.x_stride = (uint32_t)k;
        a.y = reinterpret_cast<float *>(dev + xb) + (size_t)r0 * n;
        OMEGA_HIP(F_GEMM, launch_fp8_rows(a, EPI_STORE, XS_F32, c->stream));
        streamed += (uint64_t)g * n * k;
    }
    OMEGA_HIP(F_GEMM, hipEventRecord(c->ev1, c->stream));
    OMEGA_HIP(F_GEMM, hipMemcpyAsync(pin + xb, dev + xb, (size_t)m * n * 4, hipMemcpyDeviceToHost, c->stream));
    OMEGA_HIP(F_GEMM, hipStreamSynchronize(c->stream));
    memcpy(y, pin + xb, (size_t)m * n * 4);
    if (info) {
        memset(info, 0, sizeof(*info));
        info->rows = m;
        info->segments = segments;
        info->n = t->n;
        info->k = t->k;
        info->mt = 1;
        info->warps_per_cta = 4;
        info->lane_bytes = 16;
        a.groups = m < 64 ? m : 64;
        info->grid_x = fp8_rows_blocks(a);
        info->grid_y = (m + 63) / 64;
        info->passes_max = 1;
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
// 0 off; 1 scale dropped; 2 scale block never advances; 3 neighbour row's x (as the group
// table skew of the GEMV)
void omega_gpu_fp8gemm_test_set_mutant(int mutant) { knobs().gemm_mutant = mutant; }

}  // extern "C"
