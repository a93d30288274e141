// The streaming GEMV core: a wavefront computes RPW consecutive rows of a row-major matrix.
//
// The RPW rows are one contiguous byte range; the wavefront streams it in 1 KiB chunks, lane l
// taking bytes [16 l, 16 l + 16) of every chunk (coalesced, non-temporal), so chunk c of lane l
// is row (1024 c + 16 l) / KB, byte column (1024 c + 16 l) % KB for a row of KB bytes. Lane
// column offsets repeat with period P = KB / gcd(KB, 1024) chunks: the activations a lane needs
// are P runs of 16 (e4m3) or 8 (bf16) values, held in registers for the whole slab ("phases").
// Per-lane partial dots are summed over the wavefront in a fixed order (device.hpp wave_sum),
// so every result is deterministic and no other wavefront is involved.
#pragma once

#include "device.hpp"

namespace omega {

constexpr int gcd_c(int a, int b) { return b == 0 ? a : gcd_c(b, a % b); }

template <int KB, int RPW>
struct Slab {
    static constexpr int CH = RPW * KB / 1024;           // chunks per wavefront
    static constexpr int P = KB / gcd_c(KB, 1024);       // activation phases
    static_assert(RPW * KB % 1024 == 0, "a slab is whole chunks");
    static_assert(CH % P == 0, "a slab is whole phase periods");
    static_assert(KB >= 512, "a chunk spans at most two rows");
    static constexpr int row_lo(int c) { return c * 1024 / KB; }
    // first lane of chunk c that lies in row row_lo(c) + 1 (64: none)
    static constexpr int split_lane(int c) {
        return (row_lo(c) + 1) * KB - c * 1024 >= 1024 ? 64 : ((row_lo(c) + 1) * KB - c * 1024) / 16;
    }
    __device__ static uint32_t col_bytes(int ph, uint32_t lane) { return (ph * 1024u + 16u * lane) % KB; }

    u32x4 v[CH];
    // The chunk array may also live outside a Slab (a persistent kernel's prefetch registers):
    // the static forms take it as `w` and are what the members call.
    __device__ __forceinline__ static void load_v(u32x4 *w, const void *rows, uint32_t lane) {
        const gu32x4 *p = as_global(rows) + lane;
#pragma unroll
        for (int c = 0; c < CH; ++c) w[c] = __builtin_nontemporal_load(p + c * 64);
    }
    __device__ __forceinline__ void load(const void *rows, uint32_t lane) { load_v(v, rows, lane); }
    __device__ __forceinline__ void zero() {
#pragma unroll
        for (int c = 0; c < CH; ++c) v[c] = u32x4{0u, 0u, 0u, 0u};
    }
    // acc[r] += (chunk dot) * sc[phase]; the chunk dot comes from `dot(c, phase)`
    template <typename Dot>
    __device__ __forceinline__ void accumulate(const float (&sc)[P], float (&acc)[RPW], uint32_t lane,
                                               Dot dot) const {
        accumulate_v(v, sc, acc, lane, dot);
    }
    template <typename Dot>
    __device__ __forceinline__ static void accumulate_v(const u32x4 *w, const float (&sc)[P], float (&acc)[RPW],
                                                        uint32_t lane, Dot dot) {
#pragma unroll
        for (int c = 0; c < CH; ++c) {
            const int ph = c % P;
            const float p = dot(w[c], ph);
            const int r0 = row_lo(c), sl = split_lane(c);
            if (sl >= 64) {
                acc[r0] = fmaf(p, sc[ph], acc[r0]);
            } else {
                const bool lo = lane < (uint32_t)sl;
                acc[r0] = fmaf(lo ? p : 0.f, sc[ph], acc[r0]);
                acc[r0 + 1] = fmaf(lo ? 0.f : p, sc[ph], acc[r0 + 1]);
            }
        }
    }
};

// e4m3 slab of RPW rows of K columns
template <int K, int RPW>
struct Fp8Slab : Slab<K, RPW> {
    using B = Slab<K, RPW>;
    static constexpr int P = B::P;
    // x phases: xr[ph][i] = x[col(ph) + i]
    __device__ static void load_x(const float *x, uint32_t lane, float (&xr)[P][16]) {
#pragma unroll
        for (int ph = 0; ph < P; ++ph) {
            const gf32x4 *q = as_global_f32x4(x + B::col_bytes(ph, lane));
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const f32x4 t = q[i];
                xr[ph][4 * i] = t.x;
                xr[ph][4 * i + 1] = t.y;
                xr[ph][4 * i + 2] = t.z;
                xr[ph][4 * i + 3] = t.w;
            }
        }
    }
    // the phases from a row staged in LDS
    __device__ static void load_x_lds(const float *xs, uint32_t lane, float (&xr)[P][16]) {
#pragma unroll
        for (int ph = 0; ph < P; ++ph) {
            const f32x4 *q = reinterpret_cast<const f32x4 *>(xs + B::col_bytes(ph, lane));
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const f32x4 t = q[i];
                xr[ph][4 * i] = t.x;
                xr[ph][4 * i + 1] = t.y;
                xr[ph][4 * i + 2] = t.z;
                xr[ph][4 * i + 3] = t.w;
            }
        }
    }
    // the phases of a bf16 row (an embedding row as the activation)
    __device__ static void load_x_bf16(const uint16_t *x, uint32_t lane, float (&xr)[P][16]) {
#pragma unroll
        for (int ph = 0; ph < P; ++ph) {
            const gu32x4 *q = as_global(x + B::col_bytes(ph, lane));
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                const u32x4 t = q[i];
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    xr[ph][8 * i + 2 * j] = bf16_lo(t[j]);
                    xr[ph][8 * i + 2 * j + 1] = bf16_hi(t[j]);
                }
            }
        }
    }
    // scale of each phase for the rows' 128-row block: srow[col / 128] * x_scale. The loads are
    // unconditional (the test mutants select after them): a conditional load would leave a
    // branch join whose conservative wait covers every load issued before it.
    __device__ static void load_scales(const float *srow, uint32_t lane, float x_scale, int mutant,
                                       float (&sc)[P]) {
#pragma unroll
        for (int ph = 0; ph < P; ++ph) {
            const uint32_t cb = mutant == 2 ? 0u : B::col_bytes(ph, lane) / 128u;
            const float s = *as_global_f32(srow + cb);
            sc[ph] = (mutant == 1 ? 1.0f : s) * x_scale;
        }
    }
    __device__ __forceinline__ void dot(const float (&xr)[P][16], const float (&sc)[P],
                                        float (&acc)[RPW], uint32_t lane) const {
        dot_v(this->v, xr, sc, acc, lane);
    }
    __device__ __forceinline__ static void dot_v(const u32x4 *w, const float (&xr)[P][16], const float (&sc)[P],
                                                 float (&acc)[RPW], uint32_t lane) {
        B::accumulate_v(w, sc, acc, lane, [&](const u32x4 q, int ph) { return fp8_dot16(q, xr[ph]); });
    }
    // RPW rows starting at row0 may reach into the next 128-row scale block when RPW does not
    // divide 128: sc[0] holds the scales of row0's block, sc[1] those of the last row's block, and
    // each chunk (one row, KB >= 1024) takes the block of its row.
    static constexpr bool kOneBlock = 128 % RPW == 0;
    __device__ __forceinline__ void dot2(const float (&xr)[P][16], const float (&sc)[2][P], uint32_t row0,
                                         float (&acc)[RPW]) const {
        dot2_v(this->v, xr, sc, row0, acc);
    }
    // dot_v / dot2_v with the activation read from a row staged in LDS chunk by chunk instead of
    // held as phases in registers: the same values, products and order
    __device__ __forceinline__ static void xphase_lds(const float *xs, int ph, uint32_t lane, float (&xx)[16]) {
        const f32x4 *q = reinterpret_cast<const f32x4 *>(xs + B::col_bytes(ph, lane));
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const f32x4 t = q[i];
            xx[4 * i] = t.x;
            xx[4 * i + 1] = t.y;
            xx[4 * i + 2] = t.z;
            xx[4 * i + 3] = t.w;
        }
    }
    __device__ __forceinline__ static void dot_lds(const u32x4 *w, const float *xs, const float (&sc)[P],
                                                   float (&acc)[RPW], uint32_t lane) {
        B::accumulate_v(w, sc, acc, lane, [&](const u32x4 q, int ph) {
            float xx[16];
            xphase_lds(xs, ph, lane, xx);
            return fp8_dot16(q, xx);
        });
    }
    __device__ __forceinline__ static void dot2_lds(const u32x4 *w, const float *xs, const float (&sc)[2][P],
                                                    uint32_t row0, float (&acc)[RPW], uint32_t lane) {
        static_assert(K >= 1024, "one row per chunk");
#pragma unroll
        for (int c = 0; c < B::CH; ++c) {
            const int ph = c % P;
            const int r = B::row_lo(c);
            const bool upper = ((row0 + r) >> 7) != (row0 >> 7);
            float xx[16];
            xphase_lds(xs, ph, lane, xx);
            acc[r] = fmaf(fp8_dot16(w[c], xx), upper ? sc[1][ph] : sc[0][ph], acc[r]);
        }
    }
    __device__ __forceinline__ static void dot2_v(const u32x4 *w, const float (&xr)[P][16], const float (&sc)[2][P],
                                                  uint32_t row0, float (&acc)[RPW]) {
        static_assert(K >= 1024, "one row per chunk");
#pragma unroll
        for (int c = 0; c < B::CH; ++c) {
            const int ph = c % P;
            const int r = B::row_lo(c);
            const bool upper = ((row0 + r) >> 7) != (row0 >> 7);
            acc[r] = fmaf(fp8_dot16(w[c], xr[ph]), upper ? sc[1][ph] : sc[0][ph], acc[r]);
        }
    }
};

// bf16 slab of RPW rows of K columns (rows of 2K bytes)
template <int K, int RPW>
struct Bf16Slab : Slab<2 * K, RPW> {
    using B = Slab<2 * K, RPW>;
    static constexpr int P = B::P;
    __device__ static uint32_t col(int ph, uint32_t lane) { return B::col_bytes(ph, lane) / 2; }
    __device__ static void load_x(const float *x, uint32_t lane, float (&xr)[P][8]) {
#pragma unroll
        for (int ph = 0; ph < P; ++ph) {
            const gf32x4 *q = as_global_f32x4(x + col(ph, lane));
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                const f32x4 t = q[i];
                xr[ph][4 * i] = t.x;
                xr[ph][4 * i + 1] = t.y;
                xr[ph][4 * i + 2] = t.z;
                xr[ph][4 * i + 3] = t.w;
            }
        }
    }
    __device__ __forceinline__ void dot(const float (&xr)[P][8], float (&acc)[RPW], uint32_t lane) const {
        float one[P];
#pragma unroll
        for (int ph = 0; ph < P; ++ph) one[ph] = 1.0f;
        this->accumulate(one, acc, lane, [&](const u32x4 w, int ph) { return bf16_dot8(w, xr[ph]); });
    }
};

// f64 sum of squares of the phases when they partition the row (every column exactly once)
template <int P, int W>
__device__ __forceinline__ double phases_sumsq(const float (&xr)[P][W]) {
    double ss = 0.0;
#pragma unroll
    for (int ph = 0; ph < P; ++ph)
#pragma unroll
        for (int i = 0; i < W; ++i) ss += (double)xr[ph][i] * (double)xr[ph][i];
    return wave_sum_f64(ss);
}

// acc[j] reduced over the wavefront; lane j < RPW returns row j's value
template <int RPW>
__device__ __forceinline__ float reduce_rows(float (&acc)[RPW], uint32_t lane) {
    float mine = 0.f;
#pragma unroll
    for (int j = 0; j < RPW; ++j) {
        const float s = wave_sum(acc[j]);
        acc[j] = s;
        if (lane == (uint32_t)j) mine = s;
    }
    return mine;
}

}  // namespace omega
