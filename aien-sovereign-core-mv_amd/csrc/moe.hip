// Batched MoE block for gfx950: T tokens through RMSNorm, the router (128 experts, top-8), the
// grouped gate|up FP8 GEMM with SwiGLU, the grouped down FP8 GEMM and the slot-order combine —
// the expert FFN of a decode step at token batch T (up to 64). The 8 T routed rows fall on about
// 128 (1 - (1 - 1/128)^(8 T)) distinct experts (112 at T = 32), and each expert's weights are
// read once for all of its rows.
//
// Host oracle: FakeRouter::route (crates/aien-inference-abi/src/qwen3_moe_omega.rs:1943-1998)
// per token, MoeBatchPlan::from_logits (moe_plan.rs:86-171) for the grouping, and the engine's
// FP8 MoE arm (qwen3_moe_omega.rs:4287-4318: gate|up grouped GEMV, swiglu :5616-5621, down
// grouped GEMV, moe_out += w_slot * down_slot in slot order from zero).
//
// The GEMMs run on the FP8 matrix cores (v_mfma_scale_f32_16x16x128_f8f6f4, unit scales). The
// weights are the e4m3 bytes as stored; the f32 activations are split per 128-column block into
// three e4m3 terms with power-of-two scales, x = s1 q1 + s2 q2 + s3 q3 + r, each term taken from
// the exact residual of the previous one (so about 12 significant bits survive against fp8's 4),
// and the three products are summed in f32 with the weight block scale. A wavefront owns 16
// output features of one expert segment (gate and up features together for SwiGLU) and all of
// the segment's rows (16 per MFMA column tile); nothing is exchanged between workgroups inside a
// launch: the grouping is one workgroup's launch, the combine a launch of its own.
#include <cmath>
#include <cstdio>

#include "device.hpp"
#include "kernels.hpp"
#include "route.hpp"
#include "runtime.hpp"

namespace omega {

typedef int i32x8 __attribute__((ext_vector_type(8)));

constexpr uint32_t kMH = 2048, kMI = 768, kME = 128, kTerms = 3;
constexpr uint32_t kGuTiles = kMI / 16;   // 16 gate + 16 up features per wavefront
constexpr uint32_t kDnTiles = kMH / 32;   // 32 down features per wavefront

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
        *reinterpret_cast<f32x4 *>(s + ((size_t)row * blocks + blk) * 4) = f32x4{ts[0], ts[1], ts[2], 0.f};
}

// ------------------------------------------------------------------ 1. RMSNorm + split (one workgroup per token)
__global__ __launch_bounds__(256) void k_moe_prep(const MoeArgs a) {
    __shared__ double red[4];
    const uint32_t t = blockIdx.x, tid = threadIdx.x, lane = lane_id(), wid = tid >> 6;
    const float *h = a.h + (size_t)t * kMH + 8 * tid;
    const f32x4 h0 = *as_global_f32x4(h), h1 = *as_global_f32x4(h + 4);
    const f32x4 w0 = *as_global_f32x4(a.norm_w + 8 * tid), w1 = *as_global_f32x4(a.norm_w + 8 * tid + 4);
    float v[8] = {h0.x, h0.y, h0.z, h0.w, h1.x, h1.y, h1.z, h1.w};
    const float nw[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
    double ss = 0.0;
#pragma unroll
    for (int i = 0; i < 8; ++i) ss += (double)v[i] * (double)v[i];
    ss = wave_sum_f64(ss);
    if (lane == 0) red[wid] = ss;
    __syncthreads();
    const float scale = rms_scale((red[0] + red[1]) + (red[2] + red[3]), kMH, a.eps);
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = v[i] * scale * nw[i];
    float *xo = a.xn + (size_t)t * kMH + 8 * tid;
    *reinterpret_cast<f32x4 *>(xo) = f32x4{v[0], v[1], v[2], v[3]};
    *reinterpret_cast<f32x4 *>(xo + 4) = f32x4{v[4], v[5], v[6], v[7]};
    u32x2 q[kTerms];
    float s[kTerms];
    split8(v, q, s, a.mutant == 7);
    store_split(a.xq, a.xs, t, kMH / 128, tid >> 4, tid & 15, q, s);
}

// ------------------------------------------------------------------ 2. router logits (exact f64 dots)
// one wavefront per (expert, 4 tokens): the gate row in registers, each x' row read once
__global__ __launch_bounds__(64) void k_moe_router(const MoeArgs a) {
    const uint32_t e = blockIdx.x, lane = threadIdx.x;
    // lane l holds columns 8 l + 512 j .. +8, j = 0..3
    u32x4 g[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) g[j] = *as_global(a.gate + (size_t)e * kMH + 8 * lane + 512 * j);
    for (uint32_t t = blockIdx.y * 4; t < min(a.tokens, blockIdx.y * 4 + 4); ++t) {
        const float *x = a.xn + (size_t)t * kMH + 8 * lane;
        double acc = 0.0;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const f32x4 x0 = *as_global_f32x4(x + 512 * j), x1 = *as_global_f32x4(x + 512 * j + 4);
            const float xv[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                acc += (double)bf16_lo(g[j][q]) * (double)xv[2 * q];
                acc += (double)bf16_hi(g[j][q]) * (double)xv[2 * q + 1];
            }
        }
        acc = wave_sum_f64(acc);
        if (lane == 0) a.logits[(size_t)t * kME + e] = (float)acc;
    }
}

// ------------------------------------------------------------------ 3. top-8 and the grouping (one workgroup)
// Rows of the grouped GEMMs are (token, slot) pairs ordered by expert, then by pair index
// (t * 8 + s) inside an expert; segments are the experts with rows, in ascending id.
__global__ __launch_bounds__(256) void k_moe_plan(const MoeArgs a) {
    __shared__ uint32_t sid[kMoeMaxTokens * kTopK];
    __shared__ uint32_t cnt[kME], off[kME], segi[kME];
    const uint32_t tid = threadIdx.x, lane = lane_id(), wid = tid >> 6;
    const uint32_t pairs = a.tokens * kTopK;
    for (uint32_t t = wid; t < a.tokens; t += 4) {
        Route r;
        // mutant 1: the pick's mask hits id ^ 1; mutant 2: weights not normalised
        route_topk<kME / 64>(a.logits + (size_t)t * kME, 0, a.norm_topk,
                             a.mutant == 1 ? 2 : (a.mutant == 2 ? 4 : 0), r);
#pragma unroll
        for (int s = 0; s < kTopK; ++s) {
            if (lane == (uint32_t)s) {
                sid[t * kTopK + s] = r.id[s];
                a.ids[t * kTopK + s] = r.id[s];
                a.weights[t * kTopK + s] = r.w[s];
            }
        }
    }
    __syncthreads();
    if (tid < kME) {
        uint32_t c = 0;
        for (uint32_t p = 0; p < pairs; ++p) c += sid[p] == tid;
        cnt[tid] = c;
    }
    __syncthreads();
    if (tid == 0) {  // 128 prefix sums
        uint32_t o = 0, sg = 0;
        for (uint32_t e = 0; e < kME; ++e) {
            off[e] = o;
            segi[e] = sg;
            o += cnt[e];
            sg += cnt[e] ? 1u : 0u;
        }
        a.plan[0] = sg;  // segments
    }
    __syncthreads();
    if (tid < kME) {
        const uint32_t e = tid, c = cnt[e];
        if (c) {
            const uint32_t sg = segi[e];
            a.seg_expert[sg] = e;
            a.seg_start[sg] = off[e];
            a.seg_count[sg] = c;
            uint32_t row = off[e];
            for (uint32_t p = 0; p < pairs; ++p) {
                if (sid[p] == e) {
                    a.pair_row[p] = row;
                    a.row_token[row] = p / kTopK;
                    ++row;
                }
            }
        }
    }
}

// ------------------------------------------------------------------ 4/6. grouped FP8 GEMM on the matrix cores
__device__ __forceinline__ i32x8 ld32(const uint8_t *p) {
    // bytes [0, 16) and [64, 80) of a 128-byte k-block piece at p: lane group g reads at 16 g, so
    // every load instruction covers 64 contiguous bytes of each of the 16 rows
    const u32x4 a = __builtin_nontemporal_load(as_global(p));
    const u32x4 b = __builtin_nontemporal_load(as_global(p + 64));
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

// tot[R][i] (feature 16 R + 4 g + i of the wavefront's tiles, column n) accumulates, per k-block,
// ws[R][kb] * sum_t xs_t * (W_R q_t). KB k-blocks; A rows at w[R] (+ n * K, lane's row); the
// weight scales at wsp[R][kb] (wave-uniform); B rows of the split activations at xq (row, kb,
// term). One k-block of weights is in flight ahead of the math.
template <int KB, int R>
__device__ __forceinline__ void mfma_rows(const uint8_t *const (&w)[R], const float *const (&wsp)[R],
                                          const uint8_t *xq, const float *xs, uint32_t xrow, uint32_t g,
                                          f32x4 (&tot)[R]) {
    const uint8_t *xr = xq + (size_t)xrow * KB * kTerms * 128 + 16 * g;
    const float *sr = xs + (size_t)xrow * KB * 4;
    i32x8 A[R];
#pragma unroll
    for (int r = 0; r < R; ++r) A[r] = ld32(w[r] + 16 * g);
#pragma unroll 1
    for (int kb = 0; kb < KB; ++kb) {
        i32x8 An[R];
        const int kn = kb + 1 < KB ? kb + 1 : kb;  // the last block reloads itself (in bounds, unused)
#pragma unroll
        for (int r = 0; r < R; ++r) An[r] = ld32(w[r] + 128 * kn + 16 * g);
        i32x8 B[kTerms];
#pragma unroll
        for (uint32_t t = 0; t < kTerms; ++t) B[t] = ld32_cached(xr + (kb * kTerms + t) * 128);
        const f32x4 xsc = *as_global_f32x4(sr + kb * 4);
        const float xsv[kTerms] = {xsc.x, xsc.y, xsc.z};
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const float wsc = wsp[r][kb];
#pragma unroll
            for (uint32_t t = 0; t < kTerms; ++t) {
                const f32x4 c = mfma_fp8(A[r], B[t]);
                const float f = wsc * xsv[t];
#pragma unroll
                for (int i = 0; i < 4; ++i) tot[r][i] = fmaf(c[i], f, tot[r][i]);
            }
        }
#pragma unroll
        for (int r = 0; r < R; ++r) A[r] = An[r];
    }
}

// gate|up: wavefront = (segment, 16 features j0..j0+15); gate rows j0 + n, up rows 768 + j0 + n
__global__ __launch_bounds__(256) void k_moe_gate_up(const MoeArgs a) {
    const uint32_t lane = lane_id(), wid = threadIdx.x >> 6, g = lane >> 4, n = lane & 15;
    const uint32_t item = __builtin_amdgcn_readfirstlane(blockIdx.x * 4 + wid);
    const uint32_t seg = item / kGuTiles, tile = item % kGuTiles;
    if (seg >= a.plan[0]) return;
    const uint32_t e = a.seg_expert[seg], r0 = a.seg_start[seg], cnt = a.seg_count[seg];
    const uint32_t j0 = tile * 16;
    const uint8_t *we = a.gu_w + (size_t)e * 2 * kMI * kMH;
    const uint8_t *w[2] = {we + (size_t)(j0 + n) * kMH, we + (size_t)(kMI + j0 + n) * kMH};
    const float *se = a.gu_s + (size_t)e * (2 * kMI / 128) * (kMH / 128);
    const float *ws[2] = {se + (j0 >> 7) * (kMH / 128), se + ((kMI + j0) >> 7) * (kMH / 128)};
    for (uint32_t m0 = 0; m0 < cnt; m0 += 16) {
        const bool valid = m0 + n < cnt;
        const uint32_t row = r0 + (valid ? m0 + n : 0);
        const uint32_t tok = a.row_token[row];
        f32x4 tot[2];
        tot[0] = tot[1] = f32x4{0.f, 0.f, 0.f, 0.f};
        mfma_rows<kMH / 128, 2>(w, ws, a.xq, a.xs, tok, g, tot);
        if (valid) {
            float o[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                float gv = tot[0][i], uv = tot[1][i];
                if (a.mutant == 5) {
                    const float t = gv;
                    gv = uv;
                    uv = t;
                }
                o[i] = gv / (1.0f + expf(-gv)) * uv;
            }
            *reinterpret_cast<f32x4 *>(a.act + (size_t)row * kMI + j0 + 4 * g) = f32x4{o[0], o[1], o[2], o[3]};
        }
    }
}

// the SwiGLU rows -> their split terms (one 16-lane row per 128-value block)
__global__ __launch_bounds__(256) void k_moe_split_act(const MoeArgs a) {
    const uint32_t blk = blockIdx.x * 16 + (threadIdx.x >> 4), j = threadIdx.x & 15;
    const uint32_t row = blk / (kMI / 128), b = blk % (kMI / 128);
    const bool live = row < a.tokens * kTopK;
    const float *src = a.act + (size_t)(live ? row : 0) * kMI + 128 * b + 8 * j;
    const f32x4 x0 = *as_global_f32x4(src), x1 = *as_global_f32x4(src + 4);
    float v[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
    u32x2 q[kTerms];
    float s[kTerms];
    split8(v, q, s, a.mutant == 7);  // every lane of the 16-lane row takes part (the block maximum)
    if (live) store_split(a.aq, a.as, row, kMI / 128, b, j, q, s);
}

// down: wavefront = (segment, 32 features d0..d0+31 as two 16-row tiles)
__global__ __launch_bounds__(256) void k_moe_down(const MoeArgs a) {
    const uint32_t lane = lane_id(), wid = threadIdx.x >> 6, g = lane >> 4, n = lane & 15;
    const uint32_t item = __builtin_amdgcn_readfirstlane(blockIdx.x * 4 + wid);
    const uint32_t seg = item / kDnTiles, tile = item % kDnTiles;
    if (seg >= a.plan[0]) return;
    const uint32_t e = a.seg_expert[seg], r0 = a.seg_start[seg], cnt = a.seg_count[seg];
    const uint32_t d0 = tile * 32;
    const uint8_t *we = a.dn_w + (size_t)e * kMH * kMI;
    const uint8_t *w[2] = {we + (size_t)(d0 + n) * kMI, we + (size_t)(d0 + 16 + n) * kMI};
    const float *se = a.dn_s + ((size_t)e * (kMH / 128) + (d0 >> 7)) * (kMI / 128);
    const float *ws[2] = {se, se};
    for (uint32_t m0 = 0; m0 < cnt; m0 += 16) {
        const bool valid = m0 + n < cnt;
        const uint32_t row = r0 + (valid ? m0 + n : 0);
        f32x4 tot[2];
        tot[0] = tot[1] = f32x4{0.f, 0.f, 0.f, 0.f};
        mfma_rows<kMI / 128, 2>(w, ws, a.aq, a.as, row, g, tot);
        if (valid) {
            float *y = a.ydn + (size_t)row * kMH + d0 + 4 * g;
            *reinterpret_cast<f32x4 *>(y) = tot[0];
            *reinterpret_cast<f32x4 *>(y + 16) = tot[1];
        }
    }
}

// ------------------------------------------------------------------ 7. combine (slot order from zero) [+ residual]
__global__ __launch_bounds__(256) void k_moe_combine(const MoeArgs a) {
    const uint32_t t = blockIdx.x, c = blockIdx.y * 256 + threadIdx.x;
    float moe = 0.f;
#pragma unroll
    for (int s = 0; s < kTopK; ++s) {
        const uint32_t row = a.pair_row[t * kTopK + s];
        const float w = (a.mutant == 6 && s == kTopK - 1) ? 0.f : a.weights[t * kTopK + s];
        moe += w * a.ydn[(size_t)row * kMH + c];
    }
    const size_t o = (size_t)t * kMH + c;
    a.out[o] = a.resid ? a.resid[o] + moe : moe;
}

hipError_t launch_moe_batch(const MoeArgs &a, hipStream_t st) {
    const uint32_t T = a.tokens, P = T * kTopK;
    const uint32_t segs_max = P < kME ? P : kME;
    OMEGA_LAUNCH(k_moe_prep, dim3(T), dim3(256), 0, st, a);
    OMEGA_LAUNCH(k_moe_router, dim3(kME, (T + 3) / 4), dim3(64), 0, st, a);
    OMEGA_LAUNCH(k_moe_plan, dim3(1), dim3(256), 0, st, a);
    OMEGA_LAUNCH(k_moe_gate_up, dim3((segs_max * kGuTiles + 3) / 4), dim3(256), 0, st, a);
    OMEGA_LAUNCH(k_moe_split_act, dim3((P * (kMI / 128) + 15) / 16), dim3(256), 0, st, a);
    OMEGA_LAUNCH(k_moe_down, dim3((segs_max * kDnTiles + 3) / 4), dim3(256), 0, st, a);
    OMEGA_LAUNCH(k_moe_combine, dim3(T, kMH / 256), dim3(256), 0, st, a);
    return hipGetLastError();
}

size_t moe_work_bytes(uint32_t tokens) {
    MoeArgs a;
    return moe_work_carve(a, nullptr, tokens);
}

// Carves the workspace of `tokens` rows out of `base` (null: sizes only); returns its bytes.
size_t moe_work_carve(MoeArgs &a, void *base, uint32_t tokens) {
    const size_t P = (size_t)tokens * kTopK;
    size_t o = 0;
    auto take = [&](size_t bytes) {
        const size_t at = o;
        o += (bytes + 255) & ~(size_t)255;
        return base ? static_cast<uint8_t *>(base) + at : nullptr;
    };
    a.xn = reinterpret_cast<float *>(take((size_t)tokens * kMH * 4));
    a.xq = take((size_t)tokens * (kMH / 128) * kTerms * 128);
    a.xs = reinterpret_cast<float *>(take((size_t)tokens * (kMH / 128) * 16));
    a.logits = reinterpret_cast<float *>(take((size_t)tokens * kME * 4));
    a.plan = reinterpret_cast<uint32_t *>(take(16));
    a.seg_expert = reinterpret_cast<uint32_t *>(take(kME * 4));
    a.seg_start = reinterpret_cast<uint32_t *>(take(kME * 4));
    a.seg_count = reinterpret_cast<uint32_t *>(take(kME * 4));
    a.pair_row = reinterpret_cast<uint32_t *>(take(P * 4));
    a.row_token = reinterpret_cast<uint32_t *>(take(P * 4));
    a.act = reinterpret_cast<float *>(take(P * kMI * 4));
    a.aq = take(P * (kMI / 128) * kTerms * 128);
    a.as = reinterpret_cast<float *>(take(P * (kMI / 128) * 16));
    a.ydn = reinterpret_cast<float *>(take(P * kMH * 4));
    return o;
}

}  // namespace omega

using namespace omega;

namespace omega {
RouterArgs router_args(const OmegaGpuRouter *r, uint32_t layer, const float *x, float eps,
                       int norm_topk, float out_scale);
uint32_t router_rows(const OmegaGpuRouter *r);
uint32_t router_layers(const OmegaGpuRouter *r);
}  // namespace omega

namespace {

int moe_check(const OmegaGpuRouter *r, uint32_t layer, const OmegaGpuFp8Tensor *gu,
              const OmegaGpuFp8Tensor *dn, uint32_t tokens) {
    if (!r || !gu || !dn) {
        set_error(F_GEMM, "moe batch: NULL handle");
        return OMEGA_GPU_BAD_ARGS;
    }
    if (tokens == 0 || tokens > kMoeMaxTokens) {
        set_error(F_GEMM, "moe batch: %u tokens, 1..=%u supported", tokens, kMoeMaxTokens);
        return OMEGA_GPU_TOO_LARGE;
    }
    if (layer >= router_layers(r) || router_rows(r) != kME) {
        set_error(F_GEMM, "moe batch: router layer %u of %u, or not the 128-expert shape", layer,
                  router_layers(r));
        return OMEGA_GPU_BAD_ARGS;
    }
    if (gu->experts != kME || gu->n != 2 * kMI || gu->k != kMH || dn->experts != kME || dn->n != kMH ||
        dn->k != kMI) {
        set_error(F_GEMM, "moe batch: gate|up must be 128x1536x2048 and down 128x2048x768");
        return OMEGA_GPU_BAD_ARGS;
    }
    return OMEGA_GPU_OK;
}

MoeArgs moe_args(const OmegaGpuRouter *r, uint32_t layer, const OmegaGpuFp8Tensor *gu,
                 const OmegaGpuFp8Tensor *dn, uint32_t tokens, float eps, int norm_topk) {
    MoeArgs a;
    RouterArgs ra = router_args(r, layer, nullptr, eps, norm_topk, 1.0f);
    a.gate = ra.gate;
    a.norm_w = ra.norm_w;
    a.eps = eps;
    a.norm_topk = norm_topk;
    a.tokens = tokens;
    a.gu_w = gu->w;
    a.gu_s = gu->s;
    a.dn_w = dn->w;
    a.dn_s = dn->s;
    a.mutant = knobs().moe_mutant;
    return a;
}

}  // namespace

extern "C" {

int omega_gpu_moe_batch_dev(const OmegaGpuRouter *router, uint32_t layer, const OmegaGpuFp8Tensor *gate_up,
                            const OmegaGpuFp8Tensor *down, uint32_t tokens, const float *h_dev, float eps,
                            int norm_topk, const float *resid_dev, uint32_t *ids_dev, float *weights_dev,
                            float *out_dev) {
    std::lock_guard<std::recursive_mutex> lk(big_lock());
    clear_error(F_GEMM);
    int rc = moe_check(router, layer, gate_up, down, tokens);
    if (rc) return rc;
    if (!h_dev || !ids_dev || !weights_dev || !out_dev) {
        set_error(F_GEMM, "moe batch dev: NULL pointer");
        return OMEGA_GPU_BAD_ARGS;
    }
    Ctx *c = ctx(F_GEMM);
    if (!c) return OMEGA_GPU_CHIP_FAIL;
    if (!ensure_scratch(F_GEMM, c, moe_work_bytes(tokens))) return OMEGA_GPU_CHIP_FAIL;
    MoeArgs a = moe_args(router, layer, gate_up, down, tokens, eps, norm_topk);
    moe_work_carve(a, c->scratch, tokens);
    a.h = h_dev;
    a.resid = resid_dev;
    a.ids = ids_dev;
    a.weights = weights_dev;
    a.out = out_dev;
    OMEGA_HIP(F_GEMM, launch_moe_batch(a, c->stream));
    return OMEGA_GPU_OK;
}

void omega_gpu_moe_test_set_mutant(int mutant) { knobs().moe_mutant = mutant; }

int omega_gpu_moe_batch_f32(const OmegaGpuRouter *router, uint32_t layer, const OmegaGpuFp8Tensor *gate_up,
                            const OmegaGpuFp8Tensor *down, uint32_t tokens, const float *h, float eps,
                            int norm_topk, uint32_t *ids, float *weights, float *moe_out) {
    std::lock_guard<std::recursive_mutex> lk(big_lock());
    clear_error(F_GEMM);
    int rc = moe_check(router, layer, gate_up, down, tokens);
    if (rc) return rc;
    if (!h || !ids || !weights || !moe_out) {
        set_error(F_GEMM, "moe batch: NULL pointer");
        return OMEGA_GPU_BAD_ARGS;
    }
    Ctx *c = ctx(F_GEMM);
    if (!c) return OMEGA_GPU_CHIP_FAIL;
    const size_t hb = (size_t)tokens * kMH * 4, ib = (size_t)tokens * kTopK * 4;
    const size_t work = moe_work_bytes(tokens);
    const size_t o_h = work, o_out = o_h + hb, o_ids = o_out + hb, o_w = o_ids + ib;
    if (!ensure_scratch(F_GEMM, c, o_w + ib)) return OMEGA_GPU_CHIP_FAIL;
    if (!ensure_pinned(F_GEMM, c, hb + 2 * ib)) return OMEGA_GPU_CHIP_FAIL;
    uint8_t *d = static_cast<uint8_t *>(c->scratch);
    uint8_t *pin = static_cast<uint8_t *>(c->pin);
    MoeArgs a = moe_args(router, layer, gate_up, down, tokens, eps, norm_topk);
    moe_work_carve(a, d, tokens);
    a.h = reinterpret_cast<float *>(d + o_h);
    a.out = reinterpret_cast<float *>(d + o_out);
    a.ids = reinterpret_cast<uint32_t *>(d + o_ids);
    a.weights = reinterpret_cast<float *>(d + o_w);
    memcpy(pin, h, hb);
    OMEGA_HIP(F_GEMM, hipMemcpyAsync(d + o_h, pin, hb, hipMemcpyHostToDevice, c->stream));
    OMEGA_HIP(F_GEMM, launch_moe_batch(a, c->stream));
    OMEGA_HIP(F_GEMM, hipMemcpyAsync(pin, d + o_out, hb, hipMemcpyDeviceToHost, c->stream));
    OMEGA_HIP(F_GEMM, hipMemcpyAsync(pin + hb, d + o_ids, 2 * ib, hipMemcpyDeviceToHost, c->stream));
    OMEGA_HIP(F_GEMM, hipStreamSynchronize(c->stream));
    memcpy(moe_out, pin, hb);
    memcpy(ids, pin + hb, ib);
    memcpy(weights, pin + hb + ib, ib);
    return OMEGA_GPU_OK;
}

}  // extern "C"
