// Matrix-core helpers shared by the batched kernels (MoE block, dense projections, lm_head):
// the activation split into power-of-two-scaled e4m3 terms, loads from the tiled twins of the
// weight tensors, and the FP8 / bf16 MFMA wrappers.
//
// FP8 products use v_mfma_scale_f32_16x16x128_f8f6f4: A and B are 16 x 128 e4m3 tiles, lane
// (g, n) = (lane / 16, lane % 16) holds row / column n and 32 bytes of its k-range; the two
// operands only have to agree on which k each (lane group, byte) stands for, so the loads pick
// the order that keeps every load instruction contiguous. The result lane (g, n) holds rows
// 4 g .. 4 g + 3 of column n.
#pragma once

#include "device.hpp"

namespace omega {

typedef int i32x8 __attribute__((ext_vector_type(8)));

// e4m3 terms of a split activation: about 4 significant bits each, so 4 terms carry about 16
// (products with the e4m3 weights exact, sums in f32); the q|k|v outputs are rounded to bf16 as
// K / V rows, where a 3-term error of ~1e-4 flips about 7% of the stored values by one bf16 ulp
constexpr uint32_t kTerms = 4;

// ------------------------------------------------------------------ activation split
// 2^(floor(log2 amax) - 7): amax / s lies in [128, 256), inside e4m3's range; a zero block gets 1
__device__ __forceinline__ float pow2_scale(float amax, float &inv) {
    int e = (int)((__float_as_uint(amax) >> 23) & 0xff);
    if (e == 0) {
        inv = 1.0f;
        return 1.0f;
    }
    e = e - 7 < 1 ? 1 : e - 7;
    inv = __uint_as_float((uint32_t)(254 - e) << 23);
    return __uint_as_float((uint32_t)e << 23);
}

// 8 consecutive values of a 128-value block held by one lane of a 16-lane row -> kTerms e4m3
// terms (8 bytes each) and their scales. Each term is the e4m3 rounding of the exact residual
// of the terms before it, scaled by a power of two from the residual's block maximum.
// one_term (test mutant 7): only the first term is kept, the precision of a plain fp8 cast.
__device__ __forceinline__ void split8(float (&v)[8], u32x2 (&q)[kTerms], float (&s)[kTerms], bool one_term) {
#pragma unroll
    for (uint32_t t = 0; t < kTerms; ++t) {
        float am = 0.f;
#pragma unroll
        for (int i = 0; i < 8; ++i) am = fmaxf(am, fabsf(v[i]));
        am = row16_max(am);
        float inv;
        const float sc = pow2_scale(am, inv);
        uint32_t w[2];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            int p = __builtin_amdgcn_cvt_pk_fp8_f32(v[4 * h] * inv, v[4 * h + 1] * inv, 0, false);
            p = __builtin_amdgcn_cvt_pk_fp8_f32(v[4 * h + 2] * inv, v[4 * h + 3] * inv, p, true);
            w[h] = (uint32_t)p;
            const f32x2 lo = __builtin_amdgcn_cvt_pk_f32_fp8(p, false);
            const f32x2 hi = __builtin_amdgcn_cvt_pk_f32_fp8(p, true);
            v[4 * h] -= lo.x * sc;
            v[4 * h + 1] -= lo.y * sc;
            v[4 * h + 2] -= hi.x * sc;
            v[4 * h + 3] -= hi.y * sc;
        }
        q[t] = u32x2{w[0], w[1]};
        s[t] = (one_term && t > 0) ? 0.f : sc;
    }
}

// stores one lane's share of a block: q[row][block][term][128], s[row][block][4]
__device__ __forceinline__ void store_split(uint8_t *q, float *s, uint32_t row, uint32_t blocks, uint32_t blk,
                                            uint32_t j, const u32x2 (&tq)[kTerms], const float (&ts)[kTerms]) {
    uint8_t *qb = q + ((size_t)row * blocks + blk) * kTerms * 128;
#pragma unroll
    for (uint32_t t = 0; t < kTerms; ++t) *reinterpret_cast<u32x2 *>(qb + t * 128 + 8 * j) = tq[t];
    if (j == 0)
        *reinterpret_cast<f32x4 *>(s + ((size_t)row * blocks + blk) * 4) = f32x4{ts[0], ts[1], ts[2], ts[3]};
}

// ------------------------------------------------------------------ operand loads and products
// one k-block of a 16-row tile from the tiled twin: the lane's two 16-byte pieces, each load
// instruction 1 KiB contiguous
__device__ __forceinline__ i32x8 ld_tile(const uint8_t *blk, uint32_t lane) {
    const u32x4 a = __builtin_nontemporal_load(as_global(blk + 16 * lane));
    const u32x4 b = __builtin_nontemporal_load(as_global(blk + 1024 + 16 * lane));
    return i32x8{(int)a.x, (int)a.y, (int)a.z, (int)a.w, (int)b.x, (int)b.y, (int)b.z, (int)b.w};
}
__device__ __forceinline__ i32x8 ld32_cached(const uint8_t *p) {
    const u32x4 a = *as_global(p);
    const u32x4 b = *as_global(p + 64);
    return i32x8{(int)a.x, (int)a.y, (int)a.z, (int)a.w, (int)b.x, (int)b.y, (int)b.z, (int)b.w};
}
__device__ __forceinline__ f32x4 mfma_fp8(const i32x8 &a, const i32x8 &b) {
    const f32x4 z = {0.f, 0.f, 0.f, 0.f};
    return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, z, 0, 0, 0, 127, 0, 127);
}
// acc + A (e4m3) x (2^(sb - 127) B) (e4m3): the B scale is the E8M0 exponent of a power-of-two
// activation term scale, the same in every lane of a column, so the k-to-lane mapping of the
// scale blocks does not matter
__device__ __forceinline__ f32x4 mfma_fp8_sb(const i32x8 &a, const i32x8 &b, const f32x4 &acc, int sb) {
    return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, acc, 0, 0, 0, 127, 0, sb);
}
// the E8M0 exponent of a power-of-two f32 scale (0: a dropped term, 2^-127)
__device__ __forceinline__ int e8m0_of(float s) { return (int)((__float_as_uint(s) >> 23) & 0xff); }

// the A operands of a 32-row tile (two 16-row halves) over KBW k-blocks of the FP8 tiled twin
template <int KBW>
struct MoeTileA {
    i32x8 A[2][KBW];
    // t0, t1: the twin's blocks of the two 16-row halves at the slice's first k-block
    __device__ __forceinline__ void load(const uint8_t *t0, const uint8_t *t1, uint32_t lane) {
#pragma unroll
        for (int j = 0; j < KBW; ++j) {
            A[0][j] = ld_tile(t0 + 2048 * j, lane);
            A[1][j] = ld_tile(t1 + 2048 * j, lane);
        }
    }
};

}  // namespace omega
