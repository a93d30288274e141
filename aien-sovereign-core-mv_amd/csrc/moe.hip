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
// four e4m3 terms with power-of-two scales, x = s1 q1 + s2 q2 + s3 q3 + s4 q4 + r, each term taken
// from the exact residual of the previous one (so about 16 significant bits survive against fp8's
// 4), and the four products are summed in f32 with the weight block scale. A wavefront owns
// 16-feature tiles of one expert segment (gate and up tiles together for SwiGLU) over the whole
// k, for all of the segment's rows (16 per MFMA column tile). The planner is the one launch whose
// workgroups hand data over: one workgroup per token ranks its experts, the launch's last
// workgroup waits on their flags and groups the pairs. The gate|up workgroup's wavefronts share
// only the SwiGLU split's block maxima (LDS); the combine is a launch of its own.
#include <cmath>
#include <cstdio>

#include "device.hpp"
#include "kernels.hpp"
#include "mfma.hpp"
#include "route.hpp"
#include "rows.hpp"
#include "runtime.hpp"

namespace omega {

constexpr uint32_t kMH = 2048, kMI = 768, kME = 128;

// ------------------------------------------------------------------ 1. RMSNorm + split (one workgroup per token)
__global__ __launch_bounds__(256) void k_moe_prep(const MoeArgs a) {
    __shared__ double red[4];
    const uint32_t t = blockIdx.x, tid = threadIdx.x, lane = lane_id(), wid = tid >> 6;
    const float *h = a.h + (size_t)t * kMH + 8 * tid;
    const f32x4 h0 = *as_global_f32x4(h), h1 = *as_global_f32x4(h + 4);
    const f32x4 w0 = *as_global_f32x4(a.norm_w + 8 * tid), w1 = *as_global_f32x4(a.norm_w + 8 * tid + 4);
    float v[8] = {h0.x, h0.y, h0.z, h0.w, h1.x, h1.y, h1.z, h1.w};
    const float nw[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
    if (a.opart) {  // the residual row after attention: h + (o projection's k-slices in order)
        float o[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
        for (uint32_t k = 0; k < a.oslices; ++k) {
            const float *p = a.opart + ((size_t)k * a.tokens + t) * kMH + 8 * tid;
            const f32x4 p0 = *as_global_f32x4(p), p1 = *as_global_f32x4(p + 4);
            o[0] += p0.x; o[1] += p0.y; o[2] += p0.z; o[3] += p0.w;
            o[4] += p1.x; o[5] += p1.y; o[6] += p1.z; o[7] += p1.w;
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] += o[i];
        float *ho = a.hout + (size_t)t * kMH + 8 * tid;
        *reinterpret_cast<f32x4 *>(ho) = f32x4{v[0], v[1], v[2], v[3]};
        *reinterpret_cast<f32x4 *>(ho + 4) = f32x4{v[4], v[5], v[6], v[7]};
    }
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
    // the rows of all (up to) four tokens in one round trip
    const uint32_t tb = blockIdx.y * 4, tn = min(a.tokens - tb, 4u);
    f32x4 xa[4][4][2];
#pragma unroll
    for (uint32_t q = 0; q < 4; ++q) {
        const float *x = a.xn + (size_t)(tb + min(q, tn - 1)) * kMH + 8 * lane;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            xa[q][j][0] = *as_global_f32x4(x + 512 * j);
            xa[q][j][1] = *as_global_f32x4(x + 512 * j + 4);
        }
    }
#pragma unroll
    for (uint32_t q = 0; q < 4; ++q) {
        if (q >= tn) break;
        const uint32_t t = tb + q;
        double acc = 0.0;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const f32x4 x0 = xa[q][j][0], x1 = xa[q][j][1];
            const float xv[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                acc += (double)bf16_lo(g[j][i]) * (double)xv[2 * i];
                acc += (double)bf16_hi(g[j][i]) * (double)xv[2 * i + 1];
            }
        }
        acc = wave_sum_f64(acc);
        if (lane == 0) a.logits[(size_t)t * kME + e] = (float)acc;
    }
}

// ------------------------------------------------------------------ 3. top-8 and the grouping
// Rows of the grouped GEMMs are (token, slot) pairs ordered by expert, then by pair index
// (t * 8 + s) inside an expert; segments are the experts with rows, in ascending id.
//
// Workgroups 0 .. T-1 rank one token each (its top-8 on one wavefront, so the 32 rankings of a
// T = 32 batch run on 32 CUs side by side instead of sharing one CU's four SIMDs), store its ids
// and weights, and once those stores are acknowledged flag the token with this launch's epoch.
// Workgroup T, dispatched after every ranking workgroup (so nothing it waits for can be queued
// behind it), waits (bounded) for the T flags, then groups the pairs: expert masks, counts, the
// prefix sums and every pair's row. The launch's epoch comes from its arguments (a value the host
// fixed before the launch started, plan_epoch_take), so a ranking workgroup of a launch whose wait
// ran out can only ever flag that launch's own epoch, never a later one's. Up to kPlanSolo tokens
// the launch is one workgroup whose wavefronts rank the tokens side by side straight into LDS (no
// handoff).
constexpr uint32_t kPlanSolo = 4;           // up to this many tokens: one workgroup, no handoff
// token t's flag: the epoch of the launch that ranked it; zero at load, one array per device
static __device__ __align__(256) uint32_t g_plan_flags[kMoeMaxTokens];

// The grouping from the pairs' expert ids (sid) and expert masks in LDS: per-expert counts, the
// row and segment prefix sums, the segment tables and every pair's grouped row.
__device__ __forceinline__ void moe_group(const MoeArgs &a, const uint32_t *sid,
                                          uint32_t (&mask)[kME][kMoeMaxTokens * kTopK / 32],
                                          uint32_t (&scan)[2][kME], uint32_t tid, uint32_t pairs) {
    constexpr uint32_t kWords = kMoeMaxTokens * kTopK / 32;
    // counts and the two prefix sums (rows, segments) over the experts: a log-step scan
    if (tid < kME) {
        uint32_t c = 0;
#pragma unroll
        for (uint32_t w = 0; w < kWords; ++w) c += __popc(mask[tid][w]);
        scan[0][tid] = c | (c ? 1u << 16 : 0u);
    }
    __syncthreads();
    uint32_t src = 0;
#pragma unroll
    for (uint32_t d = 1; d < kME; d <<= 1) {
        if (tid < kME) scan[src ^ 1][tid] = scan[src][tid] + (tid >= d ? scan[src][tid - d] : 0u);
        src ^= 1;
        __syncthreads();
    }
    if (tid < kME) {  // inclusive sums -> this expert's row offset and segment index
        const uint32_t incl = scan[src][tid];
        const uint32_t own = scan[src][tid] - (tid ? scan[src][tid - 1] : 0u);
        const uint32_t c = own & 0xffffu, off = (incl & 0xffffu) - c, sg = (incl >> 16) - (c ? 1u : 0u);
        if (tid == kME - 1) {
            a.plan[0] = incl >> 16;  // segments
            a.plan[1] = 0u;          // the wait ended in time
        }
        if (c) {
            a.seg_expert[sg] = tid;
            a.seg_start[sg] = off;
            a.seg_count[sg] = c;
        }
    }
    // every pair's row: its expert's offset plus the pairs before it on that expert
    for (uint32_t p = tid; p < pairs; p += 256) {
        const uint32_t e = sid[p];
        uint32_t rank = __popc(mask[e][p >> 5] & ((1u << (p & 31)) - 1u));
        for (uint32_t w = 0; w < (p >> 5); ++w) rank += __popc(mask[e][w]);
        const uint32_t incl = scan[src][e] & 0xffffu;
        const uint32_t own = incl - (e ? (scan[src][e - 1] & 0xffffu) : 0u);
        const uint32_t row = incl - own + rank;
        a.pair_row[p] = row;
        a.row_token[row] = p / kTopK;
    }
}

__global__ __launch_bounds__(256) void k_moe_plan(const MoeArgs a) {
    constexpr uint32_t kWords = kMoeMaxTokens * kTopK / 32;
    __shared__ uint32_t sid[kMoeMaxTokens * kTopK];
    __shared__ uint32_t mask[kME][kWords];  // bit p of expert e: pair p routes to e
    __shared__ uint32_t scan[2][kME];       // count | (count > 0) << 16, prefix-summed
    const uint32_t tid = threadIdx.x, lane = lane_id();
    const uint32_t T = a.tokens, pairs = T * kTopK;
    // mutant 1: the pick's mask hits id ^ 1; mutant 2: weights not normalised
    const int rm = a.mutant == 1 ? 2 : (a.mutant == 2 ? 4 : 0);
    if (gridDim.x == 1) {
        // one workgroup (up to kPlanSolo tokens, or any count while launches are recorded into
        // a graph): wavefront w ranks tokens w, w + 4, .. straight into LDS, with no handoff
        // between workgroups
        for (uint32_t i = tid; i < kME * kWords; i += 256) (&mask[0][0])[i] = 0u;
        __syncthreads();  // masks cleared before any wavefront marks its pairs
        for (uint32_t t = tid >> 6; t < T; t += 4) {
            Route r;
            route_topk<kME / 64>(a.logits + (size_t)t * kME, 0, a.norm_topk, rm, r);
#pragma unroll
            for (int sl = 0; sl < kTopK; ++sl) {
                if (lane == (uint32_t)sl) {
                    const uint32_t p = t * kTopK + sl;
                    sid[p] = r.id[sl];
                    a.ids[p] = r.id[sl];
                    a.weights[p] = r.w[sl];
                    atomicOr(&mask[r.id[sl]][p >> 5], 1u << (p & 31));
                }
            }
        }
        __syncthreads();
        moe_group(a, sid, mask, scan, tid, pairs);
        return;
    }
    const uint32_t epoch = a.epoch_dev ? *as_global_u32(a.epoch_dev) * 64u + a.epoch_sub : a.epoch_host;
    if (blockIdx.x < T) {
        if (tid >= 64) return;
        const uint32_t t = blockIdx.x;
        Route r;
        route_topk<kME / 64>(a.logits + (size_t)t * kME, 0, a.norm_topk, rm, r);
#pragma unroll
        for (int s = 0; s < kTopK; ++s) {
            if (lane == (uint32_t)s) {
                __hip_atomic_store(a.ids + t * kTopK + s, r.id[s], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                a.weights[t * kTopK + s] = r.w[s];
            }
        }
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        if (lane == 0) __hip_atomic_store(&g_plan_flags[t], epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        return;
    }
    for (uint32_t i = tid; i < kME * kWords; i += 256) (&mask[0][0])[i] = 0u;
    __shared__ uint32_t late;
    if (tid < 64) {
        // plan_spins 0 (a test knob) gives up without a poll
        bool in_time = a.plan_spins != 0;
        uint32_t spins = 0;
        while (in_time) {
            const uint32_t f = lane < T ? __hip_atomic_load(&g_plan_flags[lane], __ATOMIC_RELAXED,
                                                            __HIP_MEMORY_SCOPE_AGENT)
                                        : epoch;
            if (__all(f == epoch)) break;
            if (++spins >= a.plan_spins) in_time = false;
            else __builtin_amdgcn_s_sleep(1);
        }
        if (tid == 0) late = in_time ? 0u : 1u;
    }
    __syncthreads();  // every token flagged (or the wait ran out); the masks cleared
    if (late) {
        // no grouping from ids that may be unwritten: an empty plan, every pair on row 0 (the
        // consumers stay in bounds), the wait counted for the host
        for (uint32_t p = tid; p < pairs; p += 256) {
            a.pair_row[p] = 0u;
            a.row_token[p] = 0u;
        }
        if (tid == 0) {
            a.plan[0] = 0u;
            a.plan[1] = 1u;
            if (a.errc) __hip_atomic_fetch_add(a.errc, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        return;
    }
    for (uint32_t p = tid; p < pairs; p += 256) {
        const uint32_t e = __hip_atomic_load(a.ids + p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        sid[p] = e;
        atomicOr(&mask[e][p >> 5], 1u << (p & 31));
    }
    __syncthreads();
    moe_group(a, sid, mask, scan, tid, pairs);
}

// ------------------------------------------------------------------ 4/6. grouped FP8 GEMMs on the matrix cores
// Both expert projections run over the whole k in one wavefront per (segment, output tiles):
// each k-block's weights come from the tiled twin (each load instruction 1 KiB contiguous: a
// 16-rows x 64-bytes operand pattern on row-major weights streams at about 4.8 TB/s against 6
// TB/s contiguous), the next k-block's in flight while the current one's products run, and the
// sums stay in registers until the epilogue stores the finished rows. Splitting k over
// wavefronts instead would write and re-read f32 partial rows (25 MB per gate|up launch at
// T = 32) and need a launch to add them.

// gate|up over the whole k on the matrix cores, with SwiGLU and the 4-term split of the SwiGLU
// rows in the epilogue. A workgroup is (expert segment, 128-value block b of the SwiGLU row):
// each of its WAVES wavefronts owns TPW 16-row tiles of the block's gate features and the
// matching up features, and walks the 16 k-blocks for the segment's rows (16 per MFMA column
// tile), the next k-block's weights (from the tiled twin) and activation terms in flight while
// the current one's products run. The sum over k stays in registers, so no partial sums leave
// the chip; the wavefronts meet only to share each split term's block maximum.
struct MoeGu {
    static constexpr uint32_t KB = kMH / 128;     // 16 k-blocks
    static constexpr uint32_t BLOCKS = kMI / 128;  // 6 SwiGLU blocks per row
    static constexpr uint32_t TPW = 2;             // 16-feature tiles per wavefront
    static constexpr uint32_t WAVES = 8 / TPW;     // a 128-value block is 8 tiles
    // one k-block's operands: [tile][gate, up] weights and the column tile's 4 activation terms
    struct Stage {
        i32x8 A[TPW][2];
        i32x8 B[kTerms];
        f32x4 bs;  // the terms' power-of-two scales
    };
    // tg: the wavefront's first gate tile (16 rows each); the up tile of gate tile t is kMI / 16 + t
    __device__ static void load(Stage &st, const uint8_t *wb, uint32_t tg, uint32_t kb, const uint8_t *xr,
                                const float *sr, uint32_t lane) {
#pragma unroll
        for (uint32_t i = 0; i < TPW; ++i) {
            st.A[i][0] = ld_tile(wb + ((size_t)(tg + i) * KB + kb) * 2048, lane);
            st.A[i][1] = ld_tile(wb + ((size_t)(kMI / 16 + tg + i) * KB + kb) * 2048, lane);
        }
#pragma unroll
        for (uint32_t t = 0; t < kTerms; ++t) st.B[t] = ld32_cached(xr + (kb * kTerms + t) * 128);
        st.bs = *as_global_f32x4(sr + 4 * kb);
    }
    // acc[tile][gate, up] += (sum over the terms of A x 2^sbe B) x the k-block's weight scale
    __device__ static void products(const Stage &st, float wg, float wu, f32x4 (&acc)[TPW][2]) {
        const int sbe[kTerms] = {e8m0_of(st.bs.x), e8m0_of(st.bs.y), e8m0_of(st.bs.z), e8m0_of(st.bs.w)};
#pragma unroll
        for (uint32_t i = 0; i < TPW; ++i) {
            f32x4 c0 = {0.f, 0.f, 0.f, 0.f}, c1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (uint32_t t = 0; t < kTerms; ++t) {
                c0 = mfma_fp8_sb(st.A[i][0], st.B[t], c0, sbe[t]);
                c1 = mfma_fp8_sb(st.A[i][1], st.B[t], c1, sbe[t]);
            }
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                acc[i][0][q] = fmaf(c0[q], wg, acc[i][0][q]);
                acc[i][1][q] = fmaf(c1[q], wu, acc[i][1][q]);
            }
        }
    }
};

__global__ __launch_bounds__(64 * MoeGu::WAVES) void k_moe_gu(const MoeArgs a) {
    using G = MoeGu;
    constexpr uint32_t TPW = G::TPW;
    __shared__ float bmax[2][G::WAVES][16];  // per term parity, wavefront, row of the column tile
    const uint32_t lane = lane_id(), w = threadIdx.x >> 6, g = lane >> 4, n = lane & 15;
    const uint32_t b = blockIdx.x % G::BLOCKS, seg = blockIdx.x / G::BLOCKS;
    if (seg >= *as_const_u32(a.plan)) return;  // the whole workgroup: its waves share seg
    const uint32_t e = as_const_u32(a.seg_expert)[seg], r0 = as_const_u32(a.seg_start)[seg];
    const uint32_t cnt = as_const_u32(a.seg_count)[seg];
    const uint8_t *wb = a.gu_wt + (size_t)e * 2 * kMI * kMH;
    // weight scales of the block's gate rows (row block b) and up rows (row block 6 + b)
    const cu32 *wsg = as_const_u32(a.gu_s + ((size_t)e * (2 * kMI / 128) + b) * G::KB);
    const cu32 *wsu = as_const_u32(a.gu_s + ((size_t)e * (2 * kMI / 128) + G::BLOCKS + b) * G::KB);
    const uint32_t tg = 8 * b + TPW * w;
    for (uint32_t m0 = 0; m0 < cnt; m0 += 16) {
        const bool valid = m0 + n < cnt;
        const uint32_t row = r0 + (valid ? m0 + n : 0);
        const uint32_t xrow = a.row_token[row];
        const uint8_t *xr = a.xq + (size_t)xrow * G::KB * kTerms * 128 + 16 * g;
        const float *sr = a.xs + (size_t)xrow * G::KB * 4;
        // the expert's base taken afresh per column tile: the weight addresses are formed next to
        // their loads (scalar base + lane offset) instead of all being held in registers
        const uint8_t *wbt = wb;
        asm volatile("" : "+s"(wbt));
        f32x4 acc[TPW][2];
#pragma unroll
        for (uint32_t i = 0; i < TPW; ++i) acc[i][0] = acc[i][1] = f32x4{0.f, 0.f, 0.f, 0.f};
        // two stages take turns over the fully unrolled k-blocks: a stage is reloaded with the
        // k-block two ahead as soon as its products are issued, and no load reaches past the row
        G::Stage st[2];
        G::load(st[0], wbt, tg, 0, xr, sr, lane);
        G::load(st[1], wbt, tg, 1, xr, sr, lane);
#pragma unroll
        for (uint32_t kb = 0; kb < G::KB; ++kb) {
            G::products(st[kb & 1], __uint_as_float(wsg[kb]), __uint_as_float(wsu[kb]), acc);
            // the products issued here (not sunk below later loads), and no load hoisted above them
#pragma unroll
            for (uint32_t i = 0; i < TPW; ++i) asm volatile("" : "+v"(acc[i][0]), "+v"(acc[i][1]));
            if (kb + 2 < G::KB) G::load(st[kb & 1], wbt, tg, kb + 2, xr, sr, lane);
            __builtin_amdgcn_sched_barrier(0);
        }
        // lane (g, n): row n's features 128 b + 16 (TPW w + i) + 4 g + q of gate and up
        float v[TPW][4];
#pragma unroll
        for (uint32_t i = 0; i < TPW; ++i)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                float gg = acc[i][0][q], uu = acc[i][1][q];
                if (a.mutant == 5) {
                    const float t = gg;
                    gg = uu;
                    uu = t;
                }
                v[i][q] = gg / (1.0f + expf(-gg)) * uu;
            }
        // the 4-term split of the row's block (the steps of split8: each term's power-of-two
        // scale from the block maximum of what the previous terms left)
        uint32_t tq[kTerms][TPW];
        float ts[kTerms];
#pragma unroll
        for (uint32_t t = 0; t < kTerms; ++t) {
            float am = 0.f;
#pragma unroll
            for (uint32_t i = 0; i < TPW; ++i)
#pragma unroll
                for (int q = 0; q < 4; ++q) am = fmaxf(am, fabsf(v[i][q]));
            am = xor_max<32>(xor_max<16>(am));  // over the four lanes of row n
            if (g == 0) bmax[t & 1][w][n] = am;
            __syncthreads();
#pragma unroll
            for (uint32_t u = 0; u < G::WAVES; ++u) am = fmaxf(am, bmax[t & 1][u][n]);
            float inv;
            const float sc = pow2_scale(am, inv);
#pragma unroll
            for (uint32_t i = 0; i < TPW; ++i) {
                int p = __builtin_amdgcn_cvt_pk_fp8_f32(v[i][0] * inv, v[i][1] * inv, 0, false);
                p = __builtin_amdgcn_cvt_pk_fp8_f32(v[i][2] * inv, v[i][3] * inv, p, true);
                tq[t][i] = (uint32_t)p;
                const f32x2 lo = __builtin_amdgcn_cvt_pk_f32_fp8(p, false);
                const f32x2 hi = __builtin_amdgcn_cvt_pk_f32_fp8(p, true);
                v[i][0] -= lo.x * sc;
                v[i][1] -= lo.y * sc;
                v[i][2] -= hi.x * sc;
                v[i][3] -= hi.y * sc;
            }
            ts[t] = (a.mutant == 7 && t > 0) ? 0.f : sc;
        }
        if (valid) {
            uint8_t *qb = a.aq + ((size_t)row * G::BLOCKS + b) * kTerms * 128 + 16 * TPW * w + 4 * g;
#pragma unroll
            for (uint32_t t = 0; t < kTerms; ++t)
#pragma unroll
                for (uint32_t i = 0; i < TPW; ++i) *reinterpret_cast<uint32_t *>(qb + t * 128 + 16 * i) = tq[t][i];
            if (w == 0 && g == 0)
                *reinterpret_cast<f32x4 *>(a.as + ((size_t)row * G::BLOCKS + b) * 4) = f32x4{ts[0], ts[1], ts[2], ts[3]};
        }
    }
}

// down over the whole k (6 k-blocks of the SwiGLU row's split terms): a workgroup is (expert
// segment, 256 output features), each of its four wavefronts owns TPW 16-row tiles, and the
// finished rows go to dp [row][2048] for the combine.
struct MoeDn {
    static constexpr uint32_t KB = kMI / 128;  // 6 k-blocks
    static constexpr uint32_t TPW = 4;         // 16-feature tiles per wavefront
    static constexpr uint32_t WAVES = 4;
    static constexpr uint32_t GROUPS = kMH / (16 * TPW * WAVES);  // workgroups per segment
    struct Stage {
        i32x8 A[TPW];
        i32x8 B[kTerms];
        f32x4 bs;
    };
    __device__ static void load(Stage &st, const uint8_t *wb, uint32_t t0, uint32_t kb, const uint8_t *xr,
                                const float *sr, uint32_t lane) {
#pragma unroll
        for (uint32_t i = 0; i < TPW; ++i) st.A[i] = ld_tile(wb + ((size_t)(t0 + i) * KB + kb) * 2048, lane);
#pragma unroll
        for (uint32_t t = 0; t < kTerms; ++t) st.B[t] = ld32_cached(xr + (kb * kTerms + t) * 128);
        st.bs = *as_global_f32x4(sr + 4 * kb);
    }
    __device__ static void products(const Stage &st, float ws, f32x4 (&acc)[TPW]) {
        const int sbe[kTerms] = {e8m0_of(st.bs.x), e8m0_of(st.bs.y), e8m0_of(st.bs.z), e8m0_of(st.bs.w)};
#pragma unroll
        for (uint32_t i = 0; i < TPW; ++i) {
            f32x4 c = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (uint32_t t = 0; t < kTerms; ++t) c = mfma_fp8_sb(st.A[i], st.B[t], c, sbe[t]);
#pragma unroll
            for (int q = 0; q < 4; ++q) acc[i][q] = fmaf(c[q], ws, acc[i][q]);
        }
    }
};

__global__ __launch_bounds__(64 * MoeDn::WAVES) void k_moe_dn(const MoeArgs a) {
    using D = MoeDn;
    constexpr uint32_t TPW = D::TPW;
    const uint32_t lane = lane_id(), w = threadIdx.x >> 6, g = lane >> 4, n = lane & 15;
    const uint32_t grp = blockIdx.x % D::GROUPS, seg = blockIdx.x / D::GROUPS;
    if (seg >= *as_const_u32(a.plan)) return;  // the whole workgroup: its waves share seg
    const uint32_t e = as_const_u32(a.seg_expert)[seg], r0 = as_const_u32(a.seg_start)[seg];
    const uint32_t cnt = as_const_u32(a.seg_count)[seg];
    const uint8_t *wb = a.dn_wt + (size_t)e * kMH * kMI;
    const uint32_t t0 = (grp * D::WAVES + w) * TPW, f0 = 16 * t0;
    // the wavefront's 16 TPW features lie in one 128-row scale block
    const cu32 *ws = as_const_u32(a.dn_s + ((size_t)e * (kMH / 128) + (f0 >> 7)) * D::KB);
    for (uint32_t m0 = 0; m0 < cnt; m0 += 16) {
        const bool valid = m0 + n < cnt;
        const uint32_t row = r0 + (valid ? m0 + n : 0);
        const uint8_t *xr = a.aq + (size_t)row * D::KB * kTerms * 128 + 16 * g;
        const float *sr = a.as + (size_t)row * D::KB * 4;
        const uint8_t *wbt = wb;  // addresses formed next to their loads, as in k_moe_gu
        asm volatile("" : "+s"(wbt));
        f32x4 acc[TPW];
#pragma unroll
        for (uint32_t i = 0; i < TPW; ++i) acc[i] = f32x4{0.f, 0.f, 0.f, 0.f};
        D::Stage st[2];
        D::load(st[0], wbt, t0, 0, xr, sr, lane);
        D::load(st[1], wbt, t0, 1, xr, sr, lane);
#pragma unroll
        for (uint32_t kb = 0; kb < D::KB; ++kb) {
            D::products(st[kb & 1], __uint_as_float(ws[kb]), acc);
#pragma unroll
            for (uint32_t i = 0; i < TPW; ++i) asm volatile("" : "+v"(acc[i]));  // as in k_moe_gu
            if (kb + 2 < D::KB) D::load(st[kb & 1], wbt, t0, kb + 2, xr, sr, lane);
            __builtin_amdgcn_sched_barrier(0);
        }
        // lane (g, n): row n's features f0 + 16 i + 4 g + q
        if (valid) {
            float *o = a.dp + (size_t)row * kMH + f0 + 4 * g;
#pragma unroll
            for (uint32_t i = 0; i < TPW; ++i) *reinterpret_cast<f32x4 *>(o + 16 * i) = acc[i];
        }
    }
}

// ------------------------------------------------------------------ 4/6 below kMoeGemvMax tokens: grouped GEMVs
// The expert projections of a few tokens as GEMVs on the f32 rows (x' and the SwiGLU rows), with
// the GEMV kernel's arithmetic (rows.hpp: the same lane layout, 16-column e4m3 dots, block-scale
// fmaf and wavefront reduction): a wavefront holds RPW weight rows of one segment in registers
// and walks the segment's rows (at most one per token, so fewer than 16), each staged once per
// workgroup in LDS, the next one's loads in flight during the current dot. The four wavefronts of
// a workgroup share the segment; workgroups past the plan's segment count leave at once.
template <int K, int RPW, int NS>  // NS weight slabs per wavefront: 2 = gate and up rows, 1 = down
struct MoeRows {
    using S = Fp8Slab<K, RPW>;
    static constexpr int P = S::P;
    static constexpr int NX = (K / 4 + 255) / 256;
    __device__ static void stage_load(const float *x, f32x4 (&xt)[NX]) {
#pragma unroll
        for (int i = 0; i < NX; ++i) xt[i] = *as_global_f32x4(x + 4 * min(threadIdx.x + 256 * i, (uint32_t)K / 4 - 1));
    }
    __device__ static void stage_store(float *xs, const f32x4 (&xt)[NX]) {
#pragma unroll
        for (int i = 0; i < NX; ++i)
            if (threadIdx.x + 256 * i < (uint32_t)K / 4) reinterpret_cast<f32x4 *>(xs)[threadIdx.x + 256 * i] = xt[i];
    }
};

// gate|up: the wavefront owns gate rows j0 .. j0+3 and up rows 768+j0 .. +3 of its segment's
// expert; act[row][j] = SwiGLU(gate_j, up_j) for each of the segment's rows
__global__ __launch_bounds__(256) void k_moe_gu_rows(const MoeArgs a) {
    using R = MoeRows<kMH, 4, 2>;
    using S = R::S;
    __shared__ __align__(16) float xs[2][kMH];
    const uint32_t lane = lane_id();
    const uint32_t wave = __builtin_amdgcn_readfirstlane(blockIdx.x * 4 + (threadIdx.x >> 6));
    constexpr uint32_t per_seg = kMI / 4;
    const uint32_t seg = wave / per_seg, j0 = (wave % per_seg) * 4;
    if (seg >= *as_const_u32(a.plan)) return;  // the whole workgroup: its waves share seg
    const uint32_t e = as_const_u32(a.seg_expert)[seg], r0 = as_const_u32(a.seg_start)[seg];
    const uint32_t cnt = as_const_u32(a.seg_count)[seg];  // 1 ..= tokens < 16
    // lane r holds the token of the segment's row r
    const uint32_t tok_l = a.row_token[r0 + min(lane, cnt - 1)];
    const uint8_t *wexp = a.gu_w + (size_t)e * 2 * kMI * kMH;
    const float *sexp = a.gu_s + (size_t)e * (2 * kMI / 128) * (kMH / 128);
    f32x4 xt[R::NX];
    R::stage_load(a.xn + (size_t)__builtin_amdgcn_readfirstlane(tok_l) * kMH, xt);
    __builtin_amdgcn_sched_barrier(0);
    float scg[S::P], scu[S::P];
    S::load_scales(sexp + (size_t)(j0 >> 7) * (kMH / 128), lane, 1.0f, 0, scg);
    S::load_scales(sexp + (size_t)((kMI + j0) >> 7) * (kMH / 128), lane, 1.0f, 0, scu);
    S gs, us;
    gs.load(wexp + (size_t)j0 * kMH, lane);
    us.load(wexp + (size_t)(kMI + j0) * kMH, lane);
    __builtin_amdgcn_sched_barrier(0);
    R::stage_store(xs[0], xt);
    for (uint32_t r = 0; r < cnt; ++r) {
        lds_sync();  // row r staged; the other buffer is free
        const bool more = r + 1 < cnt;
        if (more) R::stage_load(a.xn + (size_t)__builtin_amdgcn_readlane(tok_l, r + 1) * kMH, xt);
        float xr[S::P][16];
        S::load_x_lds(xs[r & 1], lane, xr);
        float ag[4] = {0.f, 0.f, 0.f, 0.f}, au[4] = {0.f, 0.f, 0.f, 0.f};
        gs.dot(xr, scg, ag, lane);
        us.dot(xr, scu, au, lane);
        float gv = reduce_rows(ag, lane), uv = reduce_rows(au, lane);
        if (a.mutant == 5) {
            const float t = gv;
            gv = uv;
            uv = t;
        }
        if (lane < 4) a.gp[(size_t)(r0 + r) * kMI + j0 + lane] = gv / (1.0f + expf(-gv)) * uv;
        if (more) R::stage_store(xs[(r + 1) & 1], xt);
    }
}

// down: the wavefront owns down rows c0 .. c0+7 of its segment's expert; dp[row][c] for each of
// the segment's SwiGLU rows (one k-slice)
__global__ __launch_bounds__(256) void k_moe_dn_rows(const MoeArgs a) {
    using R = MoeRows<kMI, 8, 1>;
    using S = R::S;
    __shared__ __align__(16) float xs[2][kMI];
    const uint32_t lane = lane_id();
    const uint32_t wave = __builtin_amdgcn_readfirstlane(blockIdx.x * 4 + (threadIdx.x >> 6));
    constexpr uint32_t per_seg = kMH / 8;
    const uint32_t seg = wave / per_seg, c0 = (wave % per_seg) * 8;
    if (seg >= *as_const_u32(a.plan)) return;
    const uint32_t e = as_const_u32(a.seg_expert)[seg], r0 = as_const_u32(a.seg_start)[seg];
    const uint32_t cnt = as_const_u32(a.seg_count)[seg];
    const uint8_t *wexp = a.dn_w + (size_t)e * kMH * kMI;
    const float *sexp = a.dn_s + (size_t)e * (kMH / 128) * (kMI / 128);
    f32x4 xt[R::NX];
    R::stage_load(a.gp + (size_t)r0 * kMI, xt);
    __builtin_amdgcn_sched_barrier(0);
    float sc[S::P];
    S::load_scales(sexp + (size_t)(c0 >> 7) * (kMI / 128), lane, 1.0f, 0, sc);
    S ds;
    ds.load(wexp + (size_t)c0 * kMI, lane);
    __builtin_amdgcn_sched_barrier(0);
    R::stage_store(xs[0], xt);
    for (uint32_t r = 0; r < cnt; ++r) {
        lds_sync();
        const bool more = r + 1 < cnt;
        if (more) R::stage_load(a.gp + (size_t)(r0 + r + 1) * kMI, xt);
        float xr[S::P][16];
        S::load_x_lds(xs[r & 1], lane, xr);
        float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
        ds.dot(xr, sc, acc, lane);
        const float v = reduce_rows(acc, lane);
        if (lane < 8) a.dp[(size_t)(r0 + r) * kMH + c0 + lane] = v;
        if (more) R::stage_store(xs[(r + 1) & 1], xt);
    }
}

// ------------------------------------------------------------------ 7. combine (slot order from zero) [+ residual]
// each token's moe row: its slots' down rows weighted, summed in slot order from zero (nothing
// after a plan whose wait ran out: no down row was computed, the residual is written alone)
__global__ __launch_bounds__(256) void k_moe_combine(const MoeArgs a) {
    const uint32_t t = blockIdx.x, c = blockIdx.y * 256 + threadIdx.x;
    const bool late = *as_global_u32(a.plan + 1) != 0u;
    float moe = 0.f;
#pragma unroll
    for (int s = 0; s < kTopK; ++s) {
        const uint32_t row = a.pair_row[t * kTopK + s];
        const float w = (a.mutant == 6 && s == kTopK - 1) ? 0.f : a.weights[t * kTopK + s];
        moe += w * a.dp[(size_t)row * kMH + c];
    }
    if (late) moe = 0.f;  // the rows read were not written by this launch (every pair on row 0)
    const size_t o = (size_t)t * kMH + c;
    a.out[o] = a.resid ? a.resid[o] + moe : moe;
}

hipError_t launch_moe_batch(const MoeArgs &a, hipStream_t st) {
    const uint32_t T = a.tokens, P = T * kTopK;
    const uint32_t segs_max = P < kME ? P : kME;
    OMEGA_LAUNCH(k_moe_prep, dim3(T), dim3(256), 0, st, a);
    OMEGA_LAUNCH(k_moe_router, dim3(kME, (T + 3) / 4), dim3(64), 0, st, a);
    // the handoff form needs this launch's own epoch: from the word the host writes before each
    // replay, or from the host per call when the launch is not recorded
    const bool solo = T <= kPlanSolo || (!a.epoch_dev && stream_recording(st));
    OMEGA_LAUNCH(k_moe_plan, dim3(solo ? 1 : T + 1), dim3(256), 0, st, a);
    if (T < kMoeGemvMax) {
        // one workgroup per (segment, 16 gate+up row pairs) / (segment, 32 down rows)
        OMEGA_LAUNCH(k_moe_gu_rows, dim3(segs_max * (kMI / 4) / 4), dim3(256), 0, st, a);
        OMEGA_LAUNCH(k_moe_dn_rows, dim3(segs_max * (kMH / 8) / 4), dim3(256), 0, st, a);
        if (!a.defer_combine) OMEGA_LAUNCH(k_moe_combine, dim3(T, kMH / 256), dim3(256), 0, st, a);
        return hipGetLastError();
    }
    OMEGA_LAUNCH(k_moe_gu, dim3(segs_max * MoeGu::BLOCKS), dim3(64 * MoeGu::WAVES), 0, st, a);
    OMEGA_LAUNCH(k_moe_dn, dim3(segs_max * MoeDn::GROUPS), dim3(64 * MoeDn::WAVES), 0, st, a);
    if (!a.defer_combine) OMEGA_LAUNCH(k_moe_combine, dim3(T, kMH / 256), dim3(256), 0, st, a);
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
    a.gp = reinterpret_cast<float *>(take(P * kMI * 4));  // the SwiGLU rows of the GEMV path
    a.aq = take(P * (kMI / 128) * kTerms * 128);
    a.as = reinterpret_cast<float *>(take(P * (kMI / 128) * 16));
    a.dp = reinterpret_cast<float *>(take(P * kMH * 4));
    return o;
}

// The planner's epoch bases: one sequence for every launch on the device (its flags are one array
// per device). A base times 64 stays below 2^32; before it would not, the flags are cleared on the
// stream and the bases start again from 1. The library drives one device.
int plan_epoch_take(int family, hipStream_t st, uint32_t *base) {
    static uint32_t next = 0;
    static uint32_t *flags = nullptr;
    const Family f = static_cast<Family>(family);
    if (next + 1 >= (1u << 26)) {
        if (!flags) OMEGA_HIP(f, hipGetSymbolAddress(reinterpret_cast<void **>(&flags), HIP_SYMBOL(g_plan_flags)));
        OMEGA_HIP(f, hipMemsetAsync(flags, 0, sizeof(g_plan_flags), st));
        next = 0;
    }
    *base = ++next;
    return OMEGA_GPU_OK;
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
                 const OmegaGpuFp8Tensor *dn, uint32_t tokens, float eps, int norm_topk, uint32_t epoch_base) {
    MoeArgs a;
    a.epoch_host = epoch_base * 64u;
    a.plan_spins = knobs().moe_mutant == 9 ? 0u : kMoePlanSpins;
    RouterArgs ra = router_args(r, layer, nullptr, eps, norm_topk, 1.0f);
    a.gate = ra.gate;
    a.norm_w = ra.norm_w;
    a.eps = eps;
    a.norm_topk = norm_topk;
    a.tokens = tokens;
    a.gu_wt = gu->wt;
    a.gu_s = gu->s;
    a.dn_wt = dn->wt;
    a.dn_s = dn->s;
    a.gu_w = gu->w;
    a.dn_w = dn->w;
    a.mutant = knobs().moe_mutant;
    return a;
}

// One token runs the decode step's three launches (router logits, gate|up with the ranking in its
// prologue, down with the slot-order combine) instead of the batched form's six: no grouping is
// needed for 8 rows of 8 distinct experts. The mutant knobs keep the batched form.
bool moe_one_token(uint32_t tokens) { return tokens == 1 && knobs().moe_mutant == 0; }

hipError_t launch_moe_one(const OmegaGpuRouter *r, uint32_t layer, const OmegaGpuFp8Tensor *gu,
                          const OmegaGpuFp8Tensor *dn, const MoeArgs &a, float eps, int norm_topk,
                          hipStream_t st) {
    RouterArgs ra = router_args(r, layer, a.h, eps, norm_topk, 1.0f);
    ra.logits = a.logits;
    ra.xout = a.xn;
    ra.ids = a.ids;
    ra.weights = a.weights;
    ra.tab_gu = ra.tab_dn = nullptr;
    ra.route_log = nullptr;
    ra.route_log_w = nullptr;
    return launch_moe_one_token(ra, gu->w, gu->s, dn->w, dn->s, a.gp, a.resid, a.out, st);
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
    if (!rc && tokens >= kMoeGemvMax) rc = fp8_ensure_tiled(F_GEMM, const_cast<OmegaGpuFp8Tensor *>(gate_up));
    if (!rc && tokens >= kMoeGemvMax) rc = fp8_ensure_tiled(F_GEMM, const_cast<OmegaGpuFp8Tensor *>(down));
    if (rc) return rc;
    if (!h_dev || !ids_dev || !weights_dev || !out_dev) {
        set_error(F_GEMM, "moe batch dev: NULL pointer");
        return OMEGA_GPU_BAD_ARGS;
    }
    Ctx *c = ctx(F_GEMM);
    if (!c) return OMEGA_GPU_CHIP_FAIL;
    if (!ensure_scratch(F_GEMM, c, moe_work_bytes(tokens))) return OMEGA_GPU_CHIP_FAIL;
    // recorded launches plan in one workgroup and need no epoch
    uint32_t epoch_base = 0;
    if (!stream_recording(c->stream) && plan_epoch_take(F_GEMM, c->stream, &epoch_base)) return OMEGA_GPU_CHIP_FAIL;
    MoeArgs a = moe_args(router, layer, gate_up, down, tokens, eps, norm_topk, epoch_base);
    moe_work_carve(a, c->scratch, tokens);
    a.h = h_dev;
    a.resid = resid_dev;
    a.ids = ids_dev;
    a.weights = weights_dev;
    a.out = out_dev;
    if (moe_one_token(tokens)) OMEGA_HIP(F_GEMM, launch_moe_one(router, layer, gate_up, down, a, eps, norm_topk, c->stream));
    else OMEGA_HIP(F_GEMM, launch_moe_batch(a, c->stream));
    return OMEGA_GPU_OK;
}

void omega_gpu_moe_test_set_mutant(int mutant) { knobs().moe_mutant = mutant; }

int omega_gpu_moe_batch_f32(const OmegaGpuRouter *router, uint32_t layer, const OmegaGpuFp8Tensor *gate_up,
                            const OmegaGpuFp8Tensor *down, uint32_t tokens, const float *h, float eps,
                            int norm_topk, uint32_t *ids, float *weights, float *moe_out) {
    std::lock_guard<std::recursive_mutex> lk(big_lock());
    clear_error(F_GEMM);
    int rc = moe_check(router, layer, gate_up, down, tokens);
    if (!rc && tokens >= kMoeGemvMax) rc = fp8_ensure_tiled(F_GEMM, const_cast<OmegaGpuFp8Tensor *>(gate_up));
    if (!rc && tokens >= kMoeGemvMax) rc = fp8_ensure_tiled(F_GEMM, const_cast<OmegaGpuFp8Tensor *>(down));
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
    if (!ensure_pinned(F_GEMM, c, hb + 2 * ib + 4)) return OMEGA_GPU_CHIP_FAIL;
    uint8_t *d = static_cast<uint8_t *>(c->scratch);
    uint8_t *pin = static_cast<uint8_t *>(c->pin);
    uint32_t epoch_base = 0;
    if (plan_epoch_take(F_GEMM, c->stream, &epoch_base)) return OMEGA_GPU_CHIP_FAIL;
    MoeArgs a = moe_args(router, layer, gate_up, down, tokens, eps, norm_topk, epoch_base);
    moe_work_carve(a, d, tokens);
    a.h = reinterpret_cast<float *>(d + o_h);
    a.out = reinterpret_cast<float *>(d + o_out);
    a.ids = reinterpret_cast<uint32_t *>(d + o_ids);
    a.weights = reinterpret_cast<float *>(d + o_w);
    memcpy(pin, h, hb);
    OMEGA_HIP(F_GEMM, hipMemcpyAsync(d + o_h, pin, hb, hipMemcpyHostToDevice, c->stream));
    const bool one = moe_one_token(tokens);
    if (one) OMEGA_HIP(F_GEMM, launch_moe_one(router, layer, gate_up, down, a, eps, norm_topk, c->stream));
    else OMEGA_HIP(F_GEMM, launch_moe_batch(a, c->stream));
    OMEGA_HIP(F_GEMM, hipMemcpyAsync(pin, d + o_out, hb, hipMemcpyDeviceToHost, c->stream));
    OMEGA_HIP(F_GEMM, hipMemcpyAsync(pin + hb, d + o_ids, 2 * ib, hipMemcpyDeviceToHost, c->stream));
    // the planner's timed-out flag (the one-token form has no planner)
    if (!one) OMEGA_HIP(F_GEMM, hipMemcpyAsync(pin + hb + 2 * ib, a.plan + 1, 4, hipMemcpyDeviceToHost, c->stream));
    OMEGA_HIP(F_GEMM, hipStreamSynchronize(c->stream));
    uint32_t late = 0;
    if (!one) memcpy(&late, pin + hb + 2 * ib, 4);
    if (late) {
        set_error(F_GEMM, "moe batch: the plan timed out waiting for the token rankings");
        return OMEGA_GPU_CHIP_FAIL;
    }
    memcpy(moe_out, pin, hb);
    memcpy(ids, pin + hb, ib);
    memcpy(weights, pin + hb + ib, ib);
    return OMEGA_GPU_OK;
}

}  // extern "C"
