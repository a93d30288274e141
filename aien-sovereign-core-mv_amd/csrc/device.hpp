// Device helpers shared by the kernels: wave reductions, bf16 rounding, and the per-head
// preparation of the fused decode attention (per-head RMSNorm of q and k, RoPE from the table,
// bf16 append of K and V into the page pool).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "kernels.hpp"

namespace omega {

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef const __attribute__((address_space(1))) u32x4 gu32x4;
typedef const __attribute__((address_space(1))) uint32_t gu32;
typedef const __attribute__((address_space(1))) float gf32;

// Buffers reached through argument structs are global memory: give their loads the global
// address space (global_load, not flat_load).
__device__ __forceinline__ const gu32x4 *as_global(const void *p) {
    return (const gu32x4 *)(uintptr_t)p;
}
__device__ __forceinline__ const gu32 *as_global_u32(const void *p) {
    return (const gu32 *)(uintptr_t)p;
}
__device__ __forceinline__ const gf32 *as_global_f32(const void *p) {
    return (const gf32 *)(uintptr_t)p;
}

__device__ __forceinline__ double wave_sum_f64x(double v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

__device__ __forceinline__ uint16_t bf16_rne(float v) {
    // crates/aien-kv-cache/src/lib.rs:116-121 (finite values)
    uint32_t u = __float_as_uint(v);
    return (uint16_t)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}

__device__ __forceinline__ uint64_t kv_row_offset(const KvGeom &g, uint32_t block, uint32_t layer,
                                                  uint32_t plane, uint32_t token, uint32_t head) {
    return (uint64_t)block * g.block_stride + (uint64_t)layer * g.layer_stride +
           (uint64_t)plane * g.plane_stride + (uint64_t)token * g.token_stride +
           (uint64_t)head * g.head_stride;
}

// One wavefront prepares head `head` of the q|k|v row (heads 0..qh-1 are q, then kvh k heads,
// then kvh v heads). Lane l holds dims l (v0) and l + 64 (v1), so the rotate-half pair of RoPE is
// in-lane. Mirrors rmsnorm_per_head (qwen3_coder.rs:306-320, f64 sum of squares) then
// apply_rope (tensor.rs:164-190) and the bf16 append (aien-kv-cache write_token_kv).
__device__ __forceinline__ void prep_head(const HeadPrep &p, uint32_t head, uint32_t pos, float v0,
                                          float v1) {
    const uint32_t lane = threadIdx.x & 63;
    const bool is_q = head < p.qh, is_k = !is_q && head < p.qh + p.kvh;
    if (is_q || is_k) {
        double ss = (double)v0 * (double)v0 + (double)v1 * (double)v1;
        ss = wave_sum_f64x(ss);
        const float scale = (float)(1.0 / sqrt(ss / 128.0 + (double)p.eps));
        const float *w = is_q ? p.q_norm : p.k_norm;
        float n0 = v0 * scale * w[lane];
        float n1 = v1 * scale * w[lane + 64];
        if (p.mutant != 1) {
            const float c = p.rope_cos[(size_t)pos * 64 + lane];
            const float s = p.rope_sin[(size_t)pos * 64 + lane];
            const float r0 = __fsub_rn(__fmul_rn(n0, c), __fmul_rn(n1, s));
            const float r1 = __fadd_rn(__fmul_rn(n0, s), __fmul_rn(n1, c));
            n0 = r0;
            n1 = r1;
        }
        if (is_q) {
            p.q_out[head * 128 + lane] = n0;
            p.q_out[head * 128 + lane + 64] = n1;
            return;
        }
        v0 = n0;
        v1 = n1;
    }
    if (p.mutant == 3) return;
    const uint32_t kvhead = is_k ? head - p.qh : head - p.qh - p.kvh;
    const uint32_t plane = is_k ? 0 : 1;
    uint16_t *row = reinterpret_cast<uint16_t *>(
        p.pool + kv_row_offset(p.g, pos / p.g.block_size, p.layer, plane, pos % p.g.block_size, kvhead));
    row[lane] = bf16_rne(v0);
    row[lane + 64] = bf16_rne(v1);
}

}  // namespace omega
