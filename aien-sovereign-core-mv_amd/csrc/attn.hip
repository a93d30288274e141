// Decode attention for gfx950: the fused decode-attention cache (omega_gpu_decode_attn_*) with
// its matrix-core flash-decoding kernel, the paged flash-decoding over external pools
// (omega_gpu_paged_attention_bf16 / _batch_bf16 / _batch_dev), and the split combine.
//
// Contracts: crates/aien-omega-dattn/src/lib.rs:16-29 (fused), crates/aien-omega-gpu/src/ffi.rs:
// 433-461 and src/lib.rs:913-1028 (paged). Host oracle: scaled_dot_product_attention_single
// (crates/aien-inference-abi/src/tensor.rs:193-250) over the bf16 rows of the pool, as
// HostPoolKv::attend does (qwen3_moe_omega.rs:2842-2868); the q|k|v preparation is
// rmsnorm_per_head (qwen3_coder.rs:306-320, f64 sum of squares) then apply_rope
// (tensor.rs:164-190) and the bf16 append of aien-kv-cache write_token_kv.
//
// Fused kernel (k_dattn): per (split, kv head) one wavefront. The tokens before `pos` are cut
// into 16-token pages spread over up to 64 splits, so a short context already spreads its page
// reads over many CUs (a CU's own loads share one queue: four wavefronts' pages on one CU arrive
// about twice as late as the same pages spread over four CUs). Both products run on the bf16
// matrix cores with the f32 operand split into a bf16 (hi, lo) pair: the 16 B-columns of
// S^T = K q^T (v_mfma_f32_16x16x32_bf16) are the 8 q heads' hi and lo halves, the 16 A-rows of
// O = P V (v_mfma_f32_16x16x16_bf16) the 8 heads' probability hi and lo halves, and hi + lo
// rows are added at the end — products with the bf16 K / V are exact, so the result carries
// about 2^-16 relative error per operand instead of bf16's 2^-8. The cache stores each page's V
// plane transposed ([head][dim][16 tokens]) so that a lane's 4 tokens of one dim are 8
// contiguous bytes. The 8 heads' RMSNorm scales come from one transposed f64 reduction. Split 0
// appends this token's K/V and folds it in as one more online-softmax step. The splits are
// merged in the same launch: each split stores its partial with agent-scope stores and, once
// they are acknowledged, sets its flag to the launch's epoch; splits 0..7 of every kv head then
// wait (a bounded number of polls; a wait that runs out is counted in errc and reported by the
// entry point) for all of the head's flags and merge one q head each. Every split workgroup is
// resident at once (at most 4 x 64 one-wavefront workgroups). The building blocks live in
// dattn.hpp, shared with the persistent token kernel.
#include <algorithm>
#include <cmath>
#include <cstdio>
#include <vector>

#include "dattn.hpp"
#include "device.hpp"
#include "kernels.hpp"
#include "mfma.hpp"
#include "runtime.hpp"

namespace omega {


// q|k|v, the position word and the layer's q / k norm weights come in as leading scalar arguments
// (preloaded into SGPRs), so their loads go out at the first instruction. Workgroups of two
// wavefronts: wavefront 0 is the split; in split 0's workgroup wavefront 1 does this token's part
// (k's norm and RoPE, the K/V append, the token's score and V row, handed over in LDS) beside the
// page stream, and in every other workgroup it ends at once.
__global__ __launch_bounds__(128) void k_dattn(const float *qkv, const uint32_t *pos_dev, const float *q_norm,
                                               const float *k_norm, const DattnArgs a) {
    __shared__ __align__(16) DattnLds lds;
    const uint32_t lane = threadIdx.x & 63, h = blockIdx.x, s = blockIdx.y;  // kv head fastest
    const uint32_t wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    if (wv == 1 && s != 0) return;
    // Every load below is issued unconditionally, the page stream last: vector-memory waits
    // complete in issue order and merge conservatively at branch joins, so a conditional load
    // here would make the preparation math wait on the page stream. The q|k|v row and the norm
    // weights do not depend on the position, so they go out before the position is read (they
    // travel while it arrives) rather than after the split plan that needs it.
    const float *qraw = qkv + h * 8 * 128;
    float q0[8], q1[8];
#pragma unroll
    for (int r = 0; r < 8; ++r) {
        q0[r] = *as_global_f32(qraw + r * 128 + lane);
        q1[r] = *as_global_f32(qraw + r * 128 + 64 + lane);
    }
    const float qw0 = *as_global_f32(q_norm + lane), qw1 = *as_global_f32(q_norm + 64 + lane);
    const float k0 = *as_global_f32(qkv + 4096 + h * 128 + lane);
    const float k1 = *as_global_f32(qkv + 4096 + h * 128 + 64 + lane);
    const float v0 = *as_global_f32(qkv + 4608 + h * 128 + lane);
    const float v1 = *as_global_f32(qkv + 4608 + h * 128 + 64 + lane);
    const float kw0 = *as_global_f32(k_norm + lane);
    const float kw1 = *as_global_f32(k_norm + 64 + lane);
    const uint32_t pos = pos_dev ? *as_global_u32(pos_dev) : a.pos_host;
    if (wv == 1) {  // split 0's token wavefront
        const float rc = *as_global_f32(a.rope_cos + (size_t)pos * 64 + lane);
        const float rs = *as_global_f32(a.rope_sin + (size_t)pos * 64 + lane);
        dattn_q_prep(a, q0, q1, qw0, qw1, rc, rs, lane);
        dattn_token(a, h, pos, q0, q1, k0, k1, v0, v1, kw0, kw1, rc, rs, lds, lane);
        __syncthreads();  // L.vs / L.sp complete for wavefront 0's token step
        return;
    }
    const uint32_t pages = (pos + kDattnPage - 1) / kDattnPage;
    uint32_t active, pps;
    attn_split_plan(pages, gridDim.y, a.tiles_per_split, active, pps);
    // splits 0..7 of every kv head stay to merge one q head each, with or without pages
    if (s >= active && s >= 8) return;
    const bool holds = s < active;
    const uint32_t p_begin = holds ? s * pps : 0, p_end = holds ? min(pages, p_begin + pps) : 0;
    const float rc = *as_global_f32(a.rope_cos + (size_t)pos * 64 + lane);
    const float rs = *as_global_f32(a.rope_sin + (size_t)pos * 64 + lane);
    // the first page's K/V stream starts before the preparation math (page 0 stands in when the
    // split has no page: pos == 0)
    DattnPage T;
    dattn_load(a, h, p_begin < p_end ? p_begin : 0, lane, T);
    __builtin_amdgcn_sched_barrier(0);  // all of the above is issued before any arithmetic
    const uint32_t epoch = a.epoch_dev ? *as_global_u32(a.epoch_dev) * 64u + a.layer : a.epoch_host;
    dattn_split<true>(a, h, s, pos, holds, p_begin, p_end, q0, q1, k0, k1, v0, v1, qw0, qw1, kw0, kw1, rc, rs, T,
                      lds, epoch, lane);
    if (s >= 8) return;
    // Merge of q head 8 h + s: wait until every split of kv head h has flagged this epoch (every
    // split is resident: at most 4 x 64 two-wavefront workgroups), with a bounded number of polls
    // (a wait that runs out is counted and the merge goes on; merge_spins 0, a test knob, gives up
    // without a poll).
    {
        const uint32_t *fl = a.flags + h * kDattnSplits;
        bool in_time = a.merge_spins != 0;
        uint32_t spins = 0;
        while (in_time) {
            const uint32_t f = lane < active ? __hip_atomic_load(fl + lane, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                                             : epoch;
            if (__all(f == epoch)) break;
            if (++spins >= a.merge_spins) in_time = false;
            else __builtin_amdgcn_s_sleep(1);
        }
        if (!in_time && lane == 0) __hip_atomic_fetch_add(a.errc, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    const uint32_t hq = h * 8 + s;
    float o0, o1;
    dattn_merge<kDattnSplits>(a.part, hq, active, a.mutant, a.out_scale, o0, o1, lane);
    a.out[hq * 128 + lane] = o0;
    a.out[hq * 128 + 64 + lane] = o1;
}

hipError_t launch_dattn(const DattnArgs &a, hipStream_t st) {
    OMEGA_LAUNCH(k_dattn, dim3(4, a.splits), dim3(128), 0, st, a.qkv, a.pos_dev, a.q_norm, a.k_norm, a);
    return hipGetLastError();
}

// ------------------------------------------------------------------------ paged (matrix cores)
// GQA group 8 over 16-token pages of the reference layout, one wavefront per (split, kv head,
// seq), the same bf16 hi/lo matrix-core products as the fused kernel. The K rows of a page go
// straight into the A operand of S^T = K q^T (lane (g, n): token n, 16 contiguous bytes of each
// 64-byte k-step, so every load instruction reads whole 64-byte segments of 16 rows). V rows are
// token-major in the pool while the B operand of O = P V wants four tokens of one dim per lane,
// so each page's V tile is read coalesced (16 lanes per 256-byte row), staged in LDS and read
// back transposed. Tokens at or past the context in the last page may hold anything (unwritten
// slots): their scores are selected to -inf and their V rows to zero before staging, so neither
// reaches the result.
constexpr uint32_t kVtRow = 272;  // bytes per staged V row: 256 + 16 (rows 4 g apart on distinct banks)

struct PagedRegs {
    u32x4 k[4];  // A operand of the four k-steps
    u32x4 v[4];  // V rows: piece j is token 4 j + lane / 16, dims 8 (lane % 16) .. +8
};

// the pool's layer slice as the page loop sees it
struct PagedSrc {
    const uint8_t *pool;
    KvGeom g;
    uint32_t layer;
};

template <int MUT>
__device__ __forceinline__ void paged_load(const PagedSrc &a, const int32_t *tab, uint32_t blk, uint32_t h,
                                           uint32_t page, uint32_t ctx, uint32_t lane, PagedRegs &R) {
    const uint32_t g = lane >> 4, n = lane & 15;
    const uint8_t *pg = a.pool + (uint64_t)blk * a.g.block_stride + (uint64_t)a.layer * a.g.layer_stride;
    const gu32x4 *kp = as_global(pg + (uint64_t)n * a.g.token_stride + (uint64_t)h * a.g.head_stride + 16 * g);
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) R.k[ks] = __builtin_nontemporal_load(kp + 4 * ks);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        uint32_t t = 4 * j + g;
        const uint8_t *vpg = pg;
        if (MUT == 2) {  // test mutant: V one position late (clamped to the last token)
            const uint32_t tv = min(page * 16 + t + 1, ctx - 1);
            t = tv & 15;
            vpg = a.pool + (uint64_t)(uint32_t)tab[tv >> 4] * a.g.block_stride +
                  (uint64_t)a.layer * a.g.layer_stride;
        }
        R.v[j] = __builtin_nontemporal_load(as_global(vpg + a.g.plane_stride + (uint64_t)t * a.g.token_stride +
                                                      (uint64_t)h * a.g.head_stride + 16 * n));
    }
}

// V tile -> LDS (invalid tokens zeroed) -> the B operands of the 8 n-blocks
__device__ __forceinline__ void paged_stage_v(const PagedRegs &R, uint32_t tok0, uint32_t ctx, uint32_t lane,
                                              uint8_t *vt, DattnPage &T) {
    const uint32_t g = lane >> 4, n = lane & 15;
    __syncthreads();  // the previous page's reads are done
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const uint32_t t = 4 * j + g;
        const u32x4 z = {0u, 0u, 0u, 0u};
        *reinterpret_cast<u32x4 *>(vt + t * kVtRow + 16 * n) = tok0 + t < ctx ? R.v[j] : z;
    }
    __syncthreads();
    const uint16_t *v16 = reinterpret_cast<const uint16_t *>(vt);
#pragma unroll
    for (int nb = 0; nb < 8; ++nb) {
        const uint32_t col = 16 * nb + n;
        const uint32_t e0 = v16[(4 * g + 0) * (kVtRow / 2) + col];
        const uint32_t e1 = v16[(4 * g + 1) * (kVtRow / 2) + col];
        const uint32_t e2 = v16[(4 * g + 2) * (kVtRow / 2) + col];
        const uint32_t e3 = v16[(4 * g + 3) * (kVtRow / 2) + col];
        T.v[nb] = u32x2{e0 | (e1 << 16), e2 | (e3 << 16)};
    }
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) T.k[ks] = R.k[ks];
}

// The 8 q heads of kv head h (f32 rows q[8][128]) as the bf16 hi/lo B operand of S^T = K q^T.
__device__ __forceinline__ void paged_q_load(const float *q, uint32_t lane, float (&q0)[8], float (&q1)[8]) {
#pragma unroll
    for (int r = 0; r < 8; ++r) {
        q0[r] = *as_global_f32(q + r * 128 + lane);
        q1[r] = *as_global_f32(q + r * 128 + 64 + lane);
    }
}
__device__ __forceinline__ void paged_q_stage(const float (&q0)[8], const float (&q1)[8], uint32_t lane,
                                              uint16_t (*qhl)[8][128], bf16x8 (&qop)[4]) {
    const uint32_t g = lane >> 4, n = lane & 15;
#pragma unroll
    for (int r = 0; r < 8; ++r) {
        qhl[0][r][lane] = bf16_split_hi(q0[r]);
        qhl[1][r][lane] = bf16_split_lo(q0[r]);
        qhl[0][r][lane + 64] = bf16_split_hi(q1[r]);
        qhl[1][r][lane + 64] = bf16_split_lo(q1[r]);
    }
    __syncthreads();
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
        qop[ks] = as_bf16x8(*reinterpret_cast<const u32x4 *>(&qhl[n >> 3][n & 7][32 * ks + 8 * g]));
}
__device__ __forceinline__ void paged_q(const float *q, uint32_t lane, uint16_t (*qhl)[8][128], bf16x8 (&qop)[4]) {
    float q0[8], q1[8];
    paged_q_load(q, lane, q0, q1);
    paged_q_stage(q0, q1, lane, qhl, qop);
}

// Pages [p_begin, p_end) of a sequence of `ctx` tokens (table tab): the online softmax of the 8 q
// heads of kv head h. Two register sets take turns (the loop is unrolled by two, so no set is
// ever copied into the other): while one page is staged and multiplied, the other set's page is
// in flight, and a set is reloaded as soon as its page is consumed. The loop body is one
// straight path: every load is issued unconditionally (the page index clamped to the last page)
// and the second page of an iteration past p_end is processed as a null page (no valid token:
// its scores are -inf and its staged V rows zero, so m, l and O come out unchanged, exactly), so
// the vector-memory waits never merge over branches and waiting for one set never waits for the
// other. Page ids come from scalar loads one iteration ahead of their use. The first page goes
// through the same update as the others: from m = -inf, l = 0, O = 0 the rescale factor is
// exp(-inf) = 0 and the result is the first page's own.
template <int MUT>
__device__ __forceinline__ void paged_pages(const PagedSrc &src, const int32_t *tab, uint32_t h, uint32_t p_begin,
                                            uint32_t p_end, uint32_t ctx, const bf16x8 (&qop)[4], uint8_t *vt,
                                            uint32_t lane, float &m_l, float &l_l, f32x4 (&O)[8]) {
    const uint32_t g = lane >> 4, n = lane & 15, last = p_end - 1;
    const cu32 *ctab = as_const_u32(tab);
    PagedRegs A, B;
    const uint32_t p1 = min(p_begin + 1, last);
    paged_load<MUT>(src, tab, ctab[p_begin], h, p_begin, ctx, lane, A);
    paged_load<MUT>(src, tab, ctab[p1], h, p1, ctx, lane, B);
    m_l = -INFINITY;
    l_l = 0.f;
#pragma unroll
    for (int nb = 0; nb < 8; ++nb) O[nb] = f32x4{0.f, 0.f, 0.f, 0.f};
    DattnPage T;
    for (uint32_t p = p_begin; p < p_end; p += 2) {
        const uint32_t pa = min(p + 2, last), pb = min(p + 3, last);
        const uint32_t blk_a = ctab[pa], blk_b = ctab[pb];
        const uint32_t ctx_b = p + 1 < p_end ? ctx : 0u;  // 0: the null page
        paged_stage_v(A, p * 16, ctx, lane, vt, T);
        dattn_page<false>(T, qop, p * 16, ctx, g, n, m_l, l_l, O);
        paged_load<MUT>(src, tab, blk_a, h, pa, ctx, lane, A);
        paged_stage_v(B, (p + 1) * 16, ctx_b, lane, vt, T);
        dattn_page<false>(T, qop, (p + 1) * 16, ctx_b, g, n, m_l, l_l, O);
        paged_load<MUT>(src, tab, blk_b, h, pb, ctx, lane, B);
    }
}

// The split's partial (m, l, o[128]) of the 8 heads: head r at part + r * stride floats.
__device__ __forceinline__ void paged_store(float *part, size_t stride, uint32_t lane, float m_l, float l_l,
                                            const f32x4 (&O)[8]) {
    const uint32_t g = lane >> 4, n = lane & 15;
    // rows 4 g + i: hi half of head 4 g + i (g < 2) or lo half (g >= 2); see k_dattn
    const uint32_t hg = g & 1, nb_off = (g >> 1) * 4;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        float *pp = part + (size_t)(4 * hg + i) * stride;
#pragma unroll
        for (int nb = 0; nb < 4; ++nb) pp[4 + 16 * (nb + nb_off) + n] = pair_sum<32>(O[nb][i], O[nb + 4][i]);
    }
    if (lane < 8) {  // lane r holds head r's running max and sum
        float *pp = part + (size_t)lane * stride;
        pp[0] = m_l;
        pp[1] = l_l;
    }
}

template <int MUT>
__global__ __launch_bounds__(64) void k_paged(const AttnArgs a) {
    __shared__ __align__(16) uint16_t qhl[2][8][128];  // the 8 q heads: bf16 hi, lo halves
    __shared__ __align__(16) uint8_t vt[16 * kVtRow];  // one staged V tile
    const uint32_t lane = threadIdx.x, h = blockIdx.x, c = blockIdx.y, b = blockIdx.z;
    const uint32_t ctx = (uint32_t)a.context_lens[b];
    const uint32_t pages = (ctx + 15) / 16;
    uint32_t active, pps;
    attn_split_plan(pages, a.splits, 0, active, pps);
    if (c >= active) return;
    const uint32_t p_begin = c * pps, p_end = min(pages, p_begin + pps);
    const int32_t *tab = a.block_tables + (size_t)b * a.max_blocks;
    bf16x8 qop[4];
    paged_q(a.q + ((size_t)b * a.qh + h * 8) * 128, lane, qhl, qop);
    const PagedSrc src{a.pool, a.g, a.layer};
    float m_l, l_l;
    f32x4 O[8];
    paged_pages<MUT>(src, tab, h, p_begin, p_end, ctx, qop, vt, lane, m_l, l_l, O);
    paged_store(a.part + (((size_t)b * a.qh + h * 8) * a.splits + c) * kPartStride, (size_t)a.splits * kPartStride,
                lane, m_l, l_l, O);
}

// Workgroup w takes the run [w r, (w + 1) r) of the pages laid end to end, r = ceil(total /
// kItemRuns), cut into items at sequence boundaries. The items come out in page order, so each
// sequence's items are consecutive (item_off) and at most kItemRuns + seqs - 1 of them exist; a
// sequence gets at most one item per run.
void plan_items(const uint32_t *first, uint32_t seqs, ItemPlan &p) {
    const uint32_t total = first[seqs], run = (total + kItemRuns - 1) / kItemRuns;
    uint32_t n = 0, s = 0;
    for (uint32_t w = 0; w < kItemRuns; ++w) {
        p.run_off[w] = n;
        uint32_t b = std::min(total, w * run);
        const uint32_t e = std::min(total, b + run);
        while (b < e) {
            while (first[s + 1] <= b) ++s;
            const uint32_t pe = std::min(e, first[s + 1]);
            if (b == first[s]) p.item_off[s] = n;
            p.items[n][0] = (s << 24) | (b - first[s]);
            p.items[n][1] = pe - first[s];
            ++n;
            b = pe;
        }
    }
    p.run_off[kItemRuns] = n;
    p.item_off[seqs] = n;
}

// ---------------------------------------------------------------- paged, four kv heads per workgroup
// GQA group 8 with four kv heads (the Qwen3-30B-A3B shape): one workgroup of four wavefronts per
// run of pages, wavefront w = kv head w. A page's K and V planes are loaded whole token rows at
// a time (wavefront w loads tokens 4 w .. 4 w + 3, one contiguous 1 KiB row of all four heads
// per load instruction, where a per-head load would read 64-byte pieces of 16 rows), staged in
// LDS, and each wavefront reads its head's rows back in the matrix-core layouts; V rows past
// the context are zeroed when staged. Two barriers per page: the previous page's reads are done,
// the page is staged.
constexpr uint32_t kRow4 = 1040;  // bytes per staged token row: 4 heads x 256 + 16

struct Paged4Regs {
    u32x4 k[4];  // token rows 4 w + j: lane l holds head l / 16, bytes 16 (l % 16) .. +16
    u32x4 v[4];
};

template <int MUT>
__device__ __forceinline__ void paged4_load(const PagedSrc &a, const cu32 *ctab, uint32_t blk, uint32_t page,
                                            uint32_t ctx, uint32_t w, uint32_t lane, Paged4Regs &R) {
    const uint64_t lane_off = (uint64_t)(lane >> 4) * a.g.head_stride + 16 * (lane & 15);
    const uint64_t layer_off = (uint64_t)a.layer * a.g.layer_stride;
    const uint8_t *pg = a.pool + (uint64_t)blk * a.g.block_stride + layer_off + lane_off;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const uint32_t t = 4 * w + j;
        R.k[j] = __builtin_nontemporal_load(as_global(pg + (uint64_t)t * a.g.token_stride));
        const uint8_t *vpg = pg;
        uint32_t tv = t;
        if (MUT == 2) {  // test mutant: V one position late (clamped to the last token)
            const uint32_t pos = min(page * 16 + t + 1, ctx - 1);
            tv = pos & 15;
            vpg = a.pool + (uint64_t)ctab[pos >> 4] * a.g.block_stride + layer_off + lane_off;
        }
        R.v[j] = __builtin_nontemporal_load(as_global(vpg + a.g.plane_stride + (uint64_t)tv * a.g.token_stride));
    }
}

// stage the page (all waves) and read back kv head w's operands
__device__ __forceinline__ void paged4_stage(const Paged4Regs &R, uint32_t tok0, uint32_t ctx, uint32_t w,
                                             uint32_t lane, uint8_t *kt, uint8_t *vt, DattnPage &T) {
    const uint32_t g = lane >> 4, n = lane & 15;
    __syncthreads();  // every wave's reads of the previous page are done
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const uint32_t t = 4 * w + j;
        const u32x4 z = {0u, 0u, 0u, 0u};
        *reinterpret_cast<u32x4 *>(kt + t * kRow4 + 16 * lane) = R.k[j];
        *reinterpret_cast<u32x4 *>(vt + t * kRow4 + 16 * lane) = tok0 + t < ctx ? R.v[j] : z;
    }
    __syncthreads();
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
        T.k[ks] = *reinterpret_cast<const u32x4 *>(kt + n * kRow4 + 256 * w + 64 * ks + 16 * g);
    const uint16_t *v16 = reinterpret_cast<const uint16_t *>(vt) + 128 * w;
#pragma unroll
    for (int nb = 0; nb < 8; ++nb) {
        const uint32_t col = 16 * nb + n;
        const uint32_t e0 = v16[(4 * g + 0) * (kRow4 / 2) + col];
        const uint32_t e1 = v16[(4 * g + 1) * (kRow4 / 2) + col];
        const uint32_t e2 = v16[(4 * g + 2) * (kRow4 / 2) + col];
        const uint32_t e3 = v16[(4 * g + 3) * (kRow4 / 2) + col];
        T.v[nb] = u32x2{e0 | (e1 << 16), e2 | (e3 << 16)};
    }
}

// pages [p_begin, p_end) of all four kv heads: the two-set straight-path loop of paged_pages;
// blk0 / blk1: the page ids of p_begin and min(p_begin + 1, p_end - 1), read by the caller
template <int MUT>
__device__ __forceinline__ void paged4_pages(const PagedSrc &src, const int32_t *tab, uint32_t w, uint32_t p_begin,
                                             uint32_t p_end, uint32_t ctx, uint32_t blk0, uint32_t blk1,
                                             const bf16x8 (&qop)[4], uint8_t *kt, uint8_t *vt, uint32_t lane,
                                             float &m_l, float &l_l, f32x4 (&O)[8]) {
    const uint32_t g = lane >> 4, n = lane & 15, last = p_end - 1;
    const cu32 *ctab = as_const_u32(tab);
    Paged4Regs A, B;
    const uint32_t p1 = min(p_begin + 1, last);
    paged4_load<MUT>(src, ctab, blk0, p_begin, ctx, w, lane, A);
    paged4_load<MUT>(src, ctab, blk1, p1, ctx, w, lane, B);
    m_l = -INFINITY;
    l_l = 0.f;
#pragma unroll
    for (int nb = 0; nb < 8; ++nb) O[nb] = f32x4{0.f, 0.f, 0.f, 0.f};
    DattnPage T;
    for (uint32_t p = p_begin; p < p_end; p += 2) {
        const uint32_t pa = min(p + 2, last), pb = min(p + 3, last);
        const uint32_t blk_a = ctab[pa], blk_b = ctab[pb];
        const uint32_t ctx_b = p + 1 < p_end ? ctx : 0u;  // 0: the null page
        paged4_stage(A, p * 16, ctx, w, lane, kt, vt, T);
        dattn_page<false>(T, qop, p * 16, ctx, g, n, m_l, l_l, O);
        // the next pair's pages, only those that exist (a load past the split's last page would be
        // waited for by the partials' stores)
        if (p + 2 < p_end) paged4_load<MUT>(src, ctab, blk_a, pa, ctx, w, lane, A);
        paged4_stage(B, (p + 1) * 16, ctx_b, w, lane, kt, vt, T);
        dattn_page<false>(T, qop, (p + 1) * 16, ctx_b, g, n, m_l, l_l, O);
        if (p + 3 < p_end) paged4_load<MUT>(src, ctab, blk_b, pb, ctx, w, lane, B);
    }
}

// Configuration-3 form: workgroup (split c, sequence b) with the split plan of k_paged.
template <int MUT>
__global__ __launch_bounds__(256) void k_paged4(const AttnArgs a) {
    __shared__ __align__(16) uint16_t qhl[4][2][8][128];
    __shared__ __align__(16) uint8_t kt[16 * kRow4];
    __shared__ __align__(16) uint8_t vt[16 * kRow4];
    const uint32_t lane = lane_id(), w = threadIdx.x >> 6, c = blockIdx.x, b = blockIdx.y;
    const uint32_t ctx = (uint32_t)a.context_lens[b];
    const uint32_t pages = (ctx + 15) / 16;
    uint32_t active, pps;
    attn_split_plan(pages, a.splits, 0, active, pps);
    if (c >= active) return;  // uniform over the workgroup
    const uint32_t p_begin = c * pps, p_end = min(pages, p_begin + pps);
    bf16x8 qop[4];
    paged_q(a.q + ((size_t)b * a.qh + w * 8) * 128, lane, qhl[w], qop);
    const PagedSrc src{a.pool, a.g, a.layer};
    float m_l, l_l;
    f32x4 O[8];
    const int32_t *tab = a.block_tables + (size_t)b * a.max_blocks;
    const cu32 *ctab = as_const_u32(tab);
    paged4_pages<MUT>(src, tab, w, p_begin, p_end, ctx, ctab[p_begin], ctab[min(p_begin + 1, p_end - 1)], qop, kt,
                      vt, lane, m_l, l_l, O);
    paged_store(a.part + (((size_t)b * a.qh + w * 8) * a.splits + c) * kPartStride, (size_t)a.splits * kPartStride,
                lane, m_l, l_l, O);
}

// The configuration-3 form with the split combine in the same launch, for launches whose
// workgroups are all resident at once (grid <= the kernel's occupancy x CUs). Every split stores
// its partials with agent-scope stores (dims d and d + 64 side by side, as the fused kernel's), and
// once they are acknowledged flags (sequence, split) with the launch's epoch. Workgroup c of a
// sequence then merges q heads c, c + active, .. < 32 once every one of the sequence's `active`
// splits has flagged: its 4 wavefronts take the splits' 16-split chunks in turn (every load of a
// wavefront in one round trip) and their sums meet in LDS in wavefront order. A wait that runs
// out (bounded; merge_spins 0 gives up at once) is counted in errc and the heads of that workgroup
// are written as NaN.
constexpr uint32_t kPagedFoldMax = 1024;  // (sequence, split) flags of one launch
constexpr uint32_t kPagedFoldMaxSplits = 256;
// the flags, then at [kPagedFoldMax] the give-up count; zero at load, one array per device
static __device__ __align__(256) uint32_t g_paged_fold[kPagedFoldMax + 64];

__device__ __forceinline__ void paged_store_agent(float *part, size_t stride, uint32_t lane, float m_l, float l_l,
                                                  const f32x4 (&O)[8]) {
    const uint32_t g = lane >> 4, n = lane & 15;
    const uint32_t hg = g & 1, nb_off = (g >> 1) * 4;  // as paged_store
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        float *pp = part + (size_t)(4 * hg + i) * stride;
#pragma unroll
        for (int nb = 0; nb < 4; ++nb) {
            const uint32_t d = 16 * (nb + nb_off) + n;
            __hip_atomic_store(pp + 4 + 2 * (d & 63) + (d >> 6), pair_sum<32>(O[nb][i], O[nb + 4][i]),
                               __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
    if (lane < 8) {
        float *pp = part + (size_t)lane * stride;
        __hip_atomic_store(pp, m_l, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(pp + 1, l_l, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

// Merge of q head hq of sequence b over its `active` splits (all four wavefronts; the caller has
// seen every split's flag). Every wavefront computes the maximum and the sum over all splits from
// lane j's (m, l) of splits j + 64 k and keeps the weights in its own LDS row; wavefront w sums
// the splits of chunks w, w + 4, .. (16 splits each; the launch's split count is a multiple of
// 16, so a chunk's slots all exist). Slots past `active` hold whatever an earlier launch left:
// their values are masked to +0 (an all-zero mask word in the same LDS row) before their weight
// 0 applies.
__device__ __forceinline__ void paged_fold_merge(const AttnArgs &a, uint32_t b, uint32_t hq, uint32_t active,
                                                 bool ok, uint32_t w, uint32_t lane, float (*osum)[128],
                                                 float (*wsh)[kPagedFoldMaxSplits],
                                                 uint32_t (*msk)[kPagedFoldMaxSplits]) {
    const float *base = a.part + ((size_t)b * 32 + hq) * a.splits * kPartStride;
    float mk[4], lk[4];
#pragma unroll
    for (uint32_t k = 0; k < 4; ++k) {
        const uint32_t j = min(lane + 64 * k, a.splits - 1);
        const uint64_t ml = __hip_atomic_load(reinterpret_cast<const uint64_t *>(base + (size_t)j * kPartStride),
                                              __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        mk[k] = __uint_as_float((uint32_t)ml);
        lk[k] = __uint_as_float((uint32_t)(ml >> 32));
    }
    const uint64_t *ob = reinterpret_cast<const uint64_t *>(base + 4 + 2 * lane);
    constexpr uint32_t kStride64 = kPartStride / 2;
    uint64_t xo[4][16];
#pragma unroll
    for (uint32_t t = 0; t < 4; ++t) {
        const uint32_t ch = w + 4 * t;
        if (ch * 16 >= active) break;
        // the chunk's address as one per-lane value: the 16 loads are constant offsets from it
        // (kept out of scalar registers, 16 live offsets per chunk would not fit there)
        uintptr_t pv = reinterpret_cast<uintptr_t>(ob + (size_t)(ch * 16) * kStride64);
        asm volatile("" : "+v"(pv));
        const uint64_t *pc = reinterpret_cast<const uint64_t *>(pv);
#pragma unroll
        for (uint32_t i = 0; i < 16; ++i)
            xo[t][i] = __hip_atomic_load(pc + i * kStride64, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    float M = -INFINITY;
#pragma unroll
    for (uint32_t k = 0; k < 4; ++k) M = fmaxf(M, lane + 64 * k < active ? mk[k] : -INFINITY);
    M = row16_max(M);
    M = fmaxf(fmaxf(readlane_f32(M, 0), readlane_f32(M, 16)), fmaxf(readlane_f32(M, 32), readlane_f32(M, 48)));
    float lw = 0.f;
#pragma unroll
    for (uint32_t k = 0; k < 4; ++k) {
        const bool mine = lane + 64 * k < active;
        const float wk = mine ? (a.mutant == 4 ? 1.f : expf(mk[k] - M)) : 0.f;
        lw += wk * (mine ? lk[k] : 0.f);
        wsh[w][64 * k + lane] = wk;  // this wavefront's own rows: read back below by the same wavefront
        msk[w][64 * k + lane] = mine ? 0xffffffffu : 0u;
    }
    const float L = wave_sum(lw);
    float a0 = 0.f, a1 = 0.f;
#pragma unroll
    for (uint32_t t = 0; t < 4; ++t) {
        const uint32_t ch = w + 4 * t;
        if (ch * 16 >= active) break;
#pragma unroll
        for (uint32_t i = 0; i < 16; ++i) {
            const uint32_t si = ch * 16 + i;
            const float wi = wsh[w][si];
            const uint32_t m = msk[w][si];
            a0 = fmaf(wi, __uint_as_float((uint32_t)xo[t][i] & m), a0);
            a1 = fmaf(wi, __uint_as_float((uint32_t)(xo[t][i] >> 32) & m), a1);
        }
    }
    osum[w][lane] = a0;
    osum[w][lane + 64] = a1;
    __syncthreads();
    if (w == 0) {
        const float sc = a.out_scale / L;
        float *o = a.out + ((size_t)b * 32 + hq) * 128;
        const float o0 = ((osum[0][lane] + osum[1][lane]) + (osum[2][lane] + osum[3][lane])) * sc;
        const float o1 = ((osum[0][lane + 64] + osum[1][lane + 64]) + (osum[2][lane + 64] + osum[3][lane + 64])) * sc;
        o[lane] = ok ? o0 : __builtin_nanf("");
        o[lane + 64] = ok ? o1 : __builtin_nanf("");
    }
    __syncthreads();  // osum is read before the next head's sums land
}

template <int MUT>
__global__ __launch_bounds__(256) void k_paged4f(const AttnArgs a) {
    __shared__ __align__(16) uint16_t qhl[4][2][8][128];
    __shared__ __align__(16) uint8_t kt[16 * kRow4];
    __shared__ __align__(16) uint8_t vt[16 * kRow4];
    __shared__ float osum[4][128];
    __shared__ float wsh[4][kPagedFoldMaxSplits];
    __shared__ uint32_t msk[4][kPagedFoldMaxSplits];
    __shared__ uint32_t in_time_sh;
    const uint32_t lane = lane_id(), c = blockIdx.x, b = blockIdx.y;
    const uint32_t w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int32_t *tab = a.block_tables + (size_t)b * a.max_blocks;
    const cu32 *ctab = as_const_u32(tab);
    // The split of the host's context hint (the call's max_context; every sequence of a uniform
    // batch has it): its first two page ids go out with the context length and the q rows, one
    // round trip for all three; a sequence whose context plans otherwise reads its own.
    const uint32_t pages_h = min(max((a.ctx_hint + 15) / 16, 1u), a.max_blocks);
    uint32_t active_h, pps_h;
    attn_split_plan(pages_h, a.splits, 0, active_h, pps_h);
    const uint32_t pb_h = min(c * pps_h, pages_h - 1), p1_h = min(pb_h + 1, pages_h - 1);
    const uint32_t blk0_h = ctab[pb_h], blk1_h = ctab[p1_h];
    const uint32_t ctx = (uint32_t)a.context_lens[b];
    float q0[8], q1[8];
    paged_q_load(a.q + ((size_t)b * a.qh + w * 8) * 128, lane, q0, q1);
    const uint32_t pages = (ctx + 15) / 16;
    uint32_t active, pps;
    attn_split_plan(pages, a.splits, 0, active, pps);
    if (c >= active) return;  // uniform over the workgroup
    const uint32_t p_begin = c * pps, p_end = min(pages, p_begin + pps), p1 = min(p_begin + 1, p_end - 1);
    const bool hinted = p_begin == pb_h && p1 == p1_h;
    const uint32_t blk0 = hinted ? blk0_h : ctab[p_begin], blk1 = hinted ? blk1_h : ctab[p1];
    bf16x8 qop[4];
    paged_q_stage(q0, q1, lane, qhl[w], qop);
    const PagedSrc src{a.pool, a.g, a.layer};
    float m_l, l_l;
    f32x4 O[8];
    paged4_pages<MUT>(src, tab, w, p_begin, p_end, ctx, blk0, blk1, qop, kt, vt, lane, m_l, l_l, O);
    paged_store_agent(a.part + (((size_t)b * a.qh + w * 8) * a.splits + c) * kPartStride,
                      (size_t)a.splits * kPartStride, lane, m_l, l_l, O);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this wavefront's partials acknowledged
    __syncthreads();                                   // and every other wavefront's
    uint32_t *fl = a.flags + b * a.splits;
    if (threadIdx.x == 0) __hip_atomic_store(fl + c, a.epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (c >= 32) return;
    if (w == 0) {
        bool in_time = a.merge_spins != 0;
        uint32_t spins = 0;
        while (in_time) {
            bool mine = true;
#pragma unroll
            for (uint32_t k = 0; k < 4; ++k) {
                const uint32_t j = lane + 64 * k;
                const uint32_t f = j < active ? __hip_atomic_load(fl + j, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                                              : a.epoch;
                mine = mine && f == a.epoch;
            }
            if (__all(mine)) break;
            if (++spins >= a.merge_spins) in_time = false;
            else __builtin_amdgcn_s_sleep(1);
        }
        if (lane == 0) {
            in_time_sh = in_time ? 1u : 0u;
            if (!in_time) __hip_atomic_fetch_add(a.errc, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
    __syncthreads();
    const bool ok = in_time_sh != 0;
    for (uint32_t hq = c; hq < 32; hq += active) paged_fold_merge(a, b, hq, active, ok, w, lane, osum, wsh, msk);
}

// Balanced work items (the batched decode step): workgroup r serves items [run_off[r],
// run_off[r + 1]) of the plan (one run of pages, cut at sequence boundaries); item i is pages
// [first, end) of sequence seq (items[i] = {seq << 24 | first, end}), its partials at
// part[(i * 32 + q head) * kPartStride].
__global__ __launch_bounds__(256) void k_paged_items(const PagedItemsArgs a) {
    __shared__ __align__(16) uint16_t qhl[4][2][8][128];
    __shared__ __align__(16) uint8_t kt[16 * kRow4];
    __shared__ __align__(16) uint8_t vt[16 * kRow4];
    const uint32_t lane = lane_id(), w = threadIdx.x >> 6, r = blockIdx.x;
    const uint32_t i0 = a.run_off[r], i1 = a.run_off[r + 1];
    const PagedSrc src{a.pool, a.g, a.layer};
    for (uint32_t it = i0; it < i1; ++it) {
        const uint32_t e0 = a.items[2 * it], e1 = a.items[2 * it + 1];
        const uint32_t s = e0 >> 24, p_begin = e0 & 0xffffffu, p_end = e1;
        const uint32_t ctx = a.pos[s] + 1;
        __syncthreads();  // the previous item's LDS reads are done
        bf16x8 qop[4];
        paged_q(a.q + ((size_t)s * 32 + w * 8) * 128, lane, qhl[w], qop);
        float m_l, l_l;
        f32x4 O[8];
        const int32_t *tab = a.tables + (size_t)s * a.max_blocks;
        const cu32 *ctab = as_const_u32(tab);
        paged4_pages<0>(src, tab, w, p_begin, p_end, ctx, ctab[p_begin], ctab[min(p_begin + 1, p_end - 1)], qop, kt,
                        vt, lane, m_l, l_l, O);
        paged_store(a.part + ((size_t)it * 32 + w * 8) * kPartStride, kPartStride, lane, m_l, l_l, O);
    }
}

// ---------------------------------------------------------------- prefill over the fused cache
// m consecutive tokens at positions pos0 .. pos0 + m - 1 (positions before pos0 already cached):
// token t's attention is the decode step's at position pos0 + t (per-head q / k RMSNorm, RoPE,
// its K / V appended, softmax over positions 0 ..= pos0 + t). Three launches: the preparation of
// every token (q normed and rotated into a scratch row, K and V appended to the cache), the pages
// of every (token, chunk of kPattnChunk pages, kv head) as one wavefront, and the items combine.
constexpr uint32_t kPattnChunk = 32;

struct PattnArgs {
    const float *qkv = nullptr;  // [m][5120] raw projection rows
    uint8_t *pool = nullptr;
    KvGeom g{};
    uint32_t layer = 0, pos0 = 0, m = 0;
    const float *q_norm = nullptr, *k_norm = nullptr;
    const float *rope_cos = nullptr, *rope_sin = nullptr;
    float eps = 1e-6f;
    float *qn = nullptr;               // [m][32][128] prepared q
    const uint32_t *items = nullptr;   // [items][4]: first token of the group, chunk, base, chunks
    float *part = nullptr;             // [items][32][kPartStride]
};

// grid (4 kv heads, m): the kv head's 8 q heads and its K / V row of token t
__global__ __launch_bounds__(64) void k_pattn_prep(const PattnArgs a) {
    const uint32_t lane = threadIdx.x, h = blockIdx.x, t = blockIdx.y, pos = a.pos0 + t;
    const float *row = a.qkv + (size_t)t * 5120;
    float q0[8], q1[8];
#pragma unroll
    for (int r = 0; r < 8; ++r) {
        q0[r] = *as_global_f32(row + (h * 8 + r) * 128 + lane);
        q1[r] = *as_global_f32(row + (h * 8 + r) * 128 + 64 + lane);
    }
    const float qw0 = *as_global_f32(a.q_norm + lane), qw1 = *as_global_f32(a.q_norm + 64 + lane);
    const float rc = *as_global_f32(a.rope_cos + (size_t)pos * 64 + lane);
    const float rs = *as_global_f32(a.rope_sin + (size_t)pos * 64 + lane);
    float k0 = *as_global_f32(row + 4096 + h * 128 + lane), k1 = *as_global_f32(row + 4096 + h * 128 + 64 + lane);
    const float v0 = *as_global_f32(row + 4608 + h * 128 + lane);
    const float v1 = *as_global_f32(row + 4608 + h * 128 + 64 + lane);
    const float kw0 = *as_global_f32(a.k_norm + lane), kw1 = *as_global_f32(a.k_norm + 64 + lane);
    double ss[8];
#pragma unroll
    for (int r = 0; r < 8; ++r) ss[r] = (double)q0[r] * (double)q0[r] + (double)q1[r] * (double)q1[r];
    const float scale_l = rms_scale(head_sums8(ss, lane), 128, a.eps);
    float *qo = a.qn + ((size_t)t * 32 + h * 8) * 128;
#pragma unroll
    for (int r = 0; r < 8; ++r) {
        head_scale_rope(q0[r], q1[r], readlane_f32(scale_l, 8 * r), qw0, qw1, rc, rs, true);
        qo[r * 128 + lane] = q0[r];
        qo[r * 128 + 64 + lane] = q1[r];
    }
    const float kscale = rms_scale(wave_sum_f64((double)k0 * (double)k0 + (double)k1 * (double)k1), 128, a.eps);
    head_scale_rope(k0, k1, kscale, kw0, kw1, rc, rs, true);
    uint16_t *krow = reinterpret_cast<uint16_t *>(a.pool + kv_row_offset(a.g, pos >> 4, a.layer, 0, pos & 15, h));
    krow[lane] = bf16_rne(k0);
    krow[lane + 64] = bf16_rne(k1);
    uint8_t *vplane = a.pool + (uint64_t)(pos >> 4) * a.g.block_stride + (uint64_t)a.layer * a.g.layer_stride +
                      a.g.plane_stride + (uint64_t)h * kVtHead + (pos & 15) * 2;
    *reinterpret_cast<uint16_t *>(vplane + lane * 32) = bf16_rne(v0);
    *reinterpret_cast<uint16_t *>(vplane + (lane + 64) * 32) = bf16_rne(v1);
}

// one wavefront per (item, kv head): item = (group of TQ consecutive tokens t0 .., chunk c),
// pages [c C, min(pages, (c + 1) C)) of the group's last token's context; each page is loaded
// once and serves the group's tokens, token t0 + j masking the positions past its own context
// pos0 + t0 + j + 1 (a token can see none of a chunk's pages: its state stays empty, m -inf and
// l 0, and the combine gives it no weight). Item words: t0, c, the group's first partial slot
// base and its chunk count nch; token j's partial of chunk c is slot base * TQ + j * nch + c, so
// each token's partials are contiguous for the combine. A tile of TQ > 1 runs its tokens in pairs
// that share every matrix-core product (pattn_page2: the 16 columns are 2 tokens x 8 heads, so
// the softmax work per (page, token) halves against TQ = 1, whose 16 columns are one token's 8
// heads in hi and lo halves), and each page is loaded once for all TQ tokens: TQ 4 for contexts
// of 1024 and more, 2 from 256, else 1 (a wavefront per token for the parallelism of short
// prompts).
constexpr uint32_t kPattnTqLong = 4, kPattnLongCtx = 1024;
constexpr uint32_t kPattnMidCtx = 256;  // from here one pair of tokens per wavefront

// One page for a pair of query tokens (TQ > 1): the 16 B-columns of S^T = K q^T are the 16
// queries (token 2 p + n / 8, head n % 8) of the pair, the q operand's hi and lo halves in two
// product chains into one accumulator, so every lane's four scores are distinct (token, query)
// entries and the softmax runs once per query; the 16 A-rows of O = P V are the same 16 queries,
// the probability's hi and lo halves again in two chains. Lane (g, n) holds query n's state (m, l)
// and rows 4 g + i of O (query 4 g + i, dim 16 nb + n); a query that sees none of the page keeps
// an empty state (a maximum of -inf is replaced by 0 as the exponent's reference).
__device__ __forceinline__ void pattn_page2(const DattnPage &T, const bf16x8 (&qh)[4], const bf16x8 (&ql)[4],
                                            uint32_t tok0, uint32_t ctx_n, uint32_t g, uint32_t n, float &m_l,
                                            float &l_l, f32x4 (&O)[8]) {
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(T.k[ks]), qh[ks], acc, 0, 0, 0);
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(T.k[ks]), ql[ks], acc, 0, 0, 0);
    float sc[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) sc[i] = tok0 + 4 * g + i < ctx_n ? acc[i] * kInvSqrt128 : -INFINITY;
    const float mx = xor_max<32>(xor_max<16>(fmaxf(fmaxf(sc[0], sc[1]), fmaxf(sc[2], sc[3]))));
    const float m_new = fmaxf(m_l, mx);
    const float m_ref = m_new == -INFINITY ? 0.f : m_new;
    float pr[4];
    float psum = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        pr[i] = expf(sc[i] - m_ref);
        psum += pr[i];
    }
    psum = xor_sum<32>(xor_sum<16>(psum));
    const float alpha = expf(m_l - m_ref);
    l_l = l_l * alpha + psum;
    m_l = m_new;
    // row 4 g + i is query 4 g + i, whose state lane 4 g + i (lane group 0) holds
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const float ai = __shfl(alpha, (int)(4 * g + i));
#pragma unroll
        for (int nb = 0; nb < 8; ++nb) O[nb][i] *= ai;
    }
    s16x4 ph, pl;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        ph[i] = (short)bf16_split_hi(pr[i]);
        pl[i] = (short)bf16_split_lo(pr[i]);
    }
#pragma unroll
    for (int nb = 0; nb < 8; ++nb) {
        O[nb] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(ph, __builtin_bit_cast(s16x4, T.v[nb]), O[nb], 0, 0, 0);
        O[nb] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(pl, __builtin_bit_cast(s16x4, T.v[nb]), O[nb], 0, 0, 0);
    }
}

template <uint32_t TQ>
__global__ __launch_bounds__(64) void k_pattn(const PattnArgs a) {
    __shared__ __align__(16) uint16_t qhl[TQ][2][8][128];
    const uint32_t lane = threadIdx.x, h = blockIdx.x & 3, it = blockIdx.x >> 2;
    const uint32_t g = lane >> 4, n = lane & 15;
    const uint32_t *iw = a.items + 4 * (size_t)it;
    const uint32_t t0 = iw[0], c = iw[1], base = iw[2], nch = iw[3];
    const uint32_t valid = a.m - t0 < TQ ? a.m - t0 : TQ;  // tokens of this group
    const uint32_t pages = (a.pos0 + t0 + valid + 15) / 16;
    const uint32_t p_begin = c * kPattnChunk, p_end = min(pages, p_begin + kPattnChunk), last = p_end - 1;
    uint32_t ctx[TQ];
#pragma unroll
    for (uint32_t j = 0; j < TQ; ++j) ctx[j] = j < valid ? a.pos0 + t0 + j + 1 : 0u;
    DattnArgs d;
    d.pool = a.pool;
    d.g = a.g;
    d.layer = a.layer;
    DattnPage A, B;
    if constexpr (TQ == 1) {
        bf16x8 qop[4];
        paged_q(a.qn + ((size_t)t0 * 32 + h * 8) * 128, lane, qhl[0], qop);
        dattn_load(d, h, p_begin, lane, A);
        dattn_load(d, h, min(p_begin + 1, last), lane, B);
        float m_l = -INFINITY, l_l = 0.f;
        f32x4 O[8];
#pragma unroll
        for (int nb = 0; nb < 8; ++nb) O[nb] = f32x4{0.f, 0.f, 0.f, 0.f};
        for (uint32_t p = p_begin; p < p_end; p += 2) {
            const bool has_b = p + 1 < p_end;  // else B is the null page (every score -inf)
            dattn_page<false, true>(A, qop, p * 16, ctx[0], g, n, m_l, l_l, O);
            dattn_load(d, h, min(p + 2, last), lane, A);
            dattn_page<false, true>(B, qop, (p + 1) * 16, has_b ? ctx[0] : 0u, g, n, m_l, l_l, O);
            dattn_load(d, h, min(p + 3, last), lane, B);
        }
        paged_store(a.part + (((size_t)base * TQ + c) * 32 + h * 8) * kPartStride, kPartStride, lane, m_l, l_l, O);
    } else {
        // pairs of tokens share every product (pattn_page2); the 8 q heads of each token are
        // staged as bf16 hi / lo halves (a missing token repeats the first, never stored)
        static_assert(TQ % 2 == 0, "query tiles of whole pairs");
        constexpr uint32_t NP = TQ / 2;
#pragma unroll
        for (uint32_t j = 0; j < TQ; ++j) {
            const float *q = a.qn + ((size_t)(j < valid ? t0 + j : t0) * 32 + h * 8) * 128;
#pragma unroll
            for (int r = 0; r < 8; ++r) {
                const float q0 = *as_global_f32(q + r * 128 + lane), q1 = *as_global_f32(q + r * 128 + 64 + lane);
                qhl[j][0][r][lane] = bf16_split_hi(q0);
                qhl[j][1][r][lane] = bf16_split_lo(q0);
                qhl[j][0][r][lane + 64] = bf16_split_hi(q1);
                qhl[j][1][r][lane + 64] = bf16_split_lo(q1);
            }
        }
        dattn_load(d, h, p_begin, lane, A);
        dattn_load(d, h, min(p_begin + 1, last), lane, B);
        __syncthreads();
        // B operands: column n of pair p is query (token 2 p + n / 8, head n % 8); k-step ks of
        // lane group g covers dims 32 ks + 8 g .. +8
        bf16x8 qh[NP][4], ql[NP][4];
        uint32_t cn[NP];
#pragma unroll
        for (uint32_t p = 0; p < NP; ++p) {
            const uint32_t j = 2 * p + (n >> 3);
            cn[p] = ctx[0];
#pragma unroll
            for (uint32_t jj = 1; jj < TQ; ++jj)
                if (jj == j) cn[p] = ctx[jj];
#pragma unroll
            for (int ks = 0; ks < 4; ++ks) {
                qh[p][ks] = as_bf16x8(*reinterpret_cast<const u32x4 *>(&qhl[j][0][n & 7][32 * ks + 8 * g]));
                ql[p][ks] = as_bf16x8(*reinterpret_cast<const u32x4 *>(&qhl[j][1][n & 7][32 * ks + 8 * g]));
            }
        }
        float m_l[NP], l_l[NP];
        f32x4 O[NP][8];
#pragma unroll
        for (uint32_t p = 0; p < NP; ++p) {
            m_l[p] = -INFINITY;
            l_l[p] = 0.f;
#pragma unroll
            for (int nb = 0; nb < 8; ++nb) O[p][nb] = f32x4{0.f, 0.f, 0.f, 0.f};
        }
        for (uint32_t pg = p_begin; pg < p_end; pg += 2) {
            const bool has_b = pg + 1 < p_end;  // else B is the null page (every score -inf)
#pragma unroll
            for (uint32_t p = 0; p < NP; ++p) pattn_page2(A, qh[p], ql[p], pg * 16, cn[p], g, n, m_l[p], l_l[p], O[p]);
            dattn_load(d, h, min(pg + 2, last), lane, A);
#pragma unroll
            for (uint32_t p = 0; p < NP; ++p)
                pattn_page2(B, qh[p], ql[p], (pg + 1) * 16, has_b ? cn[p] : 0u, g, n, m_l[p], l_l[p], O[p]);
            dattn_load(d, h, min(pg + 3, last), lane, B);
        }
        // partials: row 4 g + i of pair p is query 4 g + i (token 2 p + g / 2, head 4 (g % 2) + i);
        // lanes 0..15 hold query n's (m, l). Token j's partial of chunk c is slot base * TQ + j *
        // nch + c, its head r at r * kPartStride (m, l, -, -, o[128]).
#pragma unroll
        for (uint32_t p = 0; p < NP; ++p) {
            const uint32_t jo = 2 * p + (g >> 1);
            if (jo < valid) {
                float *pt = a.part + (((size_t)base * TQ + jo * nch + c) * 32 + h * 8) * kPartStride;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    float *pp = pt + (size_t)(4 * (g & 1) + i) * kPartStride + 4;
#pragma unroll
                    for (int nb = 0; nb < 8; ++nb) pp[16 * nb + n] = O[p][nb][i];
                }
            }
            const uint32_t jm = 2 * p + (n >> 3);
            if (lane < 16 && jm < valid) {
                float *pp = a.part + (((size_t)base * TQ + jm * nch + c) * 32 + h * 8 + (n & 7)) * kPartStride;
                pp[0] = m_l[p];
                pp[1] = l_l[p];
            }
        }
    }
}

// ---------------------------------------------------------------- KV park / restore (extension)
// The payload of positions start .. start + len (start a multiple of 16) is the HostPagedPoolV1
// format of qwen3_moe_omega_kvio.rs:15-40: ceil(len / 16) blocks of [layer][K plane | V plane]
// [token][kv head][dim] bf16, rows at or past len zero. The fused cache's pages have the same
// strides with the V plane transposed per page ([kv head][dim][token]), so a K plane moves as it
// is and a V plane goes through an LDS transpose. One workgroup per (block, layer). The reference
// builds the payload row by row through cache_read (rows_to_blocks, :102-122).
constexpr uint32_t kKvioPitch = 17;  // LDS words per (kv head, dim) row of 16 tokens

struct KvioArgs {
    uint8_t *pool = nullptr;     // the cache's first block of the range
    uint8_t *payload = nullptr;  // the payload's first block of the range
    uint64_t block_stride = 0, layer_stride = 0, plane_stride = 0;
    uint32_t blk0 = 0;           // payload block of blockIdx.x = 0, relative to the payload start
    uint32_t len = 0;            // positions in the whole payload
};

__global__ __launch_bounds__(256) void k_kv_export(const KvioArgs a) {
    __shared__ uint32_t tile[512 * kKvioPitch];  // [kv head * 128 + dim][token], one bf16 per word
    const uint32_t tid = threadIdx.x, blk = a.blk0 + blockIdx.x, layer = blockIdx.y;
    const uint64_t off = (uint64_t)blockIdx.x * a.block_stride + (uint64_t)layer * a.layer_stride;
    const uint8_t *src = a.pool + off;
    uint8_t *dst = a.payload + off;
    // K plane: 64 u32x4 per token row
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const uint32_t i = tid + 256 * j, tok = i >> 6;
        const u32x4 v = *as_global(src + 16 * (size_t)i);
        *reinterpret_cast<u32x4 *>(dst + 16 * (size_t)i) = blk * 16 + tok < a.len ? v : u32x4{0u, 0u, 0u, 0u};
    }
    // V^T plane: 16 bytes x4 per thread; word w holds row r = w / 8 (kv head * 128 + dim),
    // tokens 2 (w % 8) and + 1, so a thread's four words are tokens t0 .. t0 + 7 of one row
    const uint8_t *vs = src + a.plane_stride;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const uint32_t q = tid + 256 * j, r = q >> 1, t0 = 8 * (q & 1);
        const u32x4 v = *as_global(vs + 16 * (size_t)q);
        uint32_t *tr = tile + r * kKvioPitch + t0;
        tr[0] = v.x & 0xffffu;
        tr[1] = v.x >> 16;
        tr[2] = v.y & 0xffffu;
        tr[3] = v.y >> 16;
        tr[4] = v.z & 0xffffu;
        tr[5] = v.z >> 16;
        tr[6] = v.w & 0xffffu;
        tr[7] = v.w >> 16;
    }
    __syncthreads();
    // payload V plane: token t = q / 64, rows c = 8 (q % 64) .. + 7 per 16-byte store
    uint8_t *vd = dst + a.plane_stride;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const uint32_t q = tid + 256 * j, t = q >> 6, c = 8 * (q & 63);
        const uint32_t *tc = tile + c * kKvioPitch + t;
        u32x4 v;
        v.x = tc[0] | (tc[kKvioPitch] << 16);
        v.y = tc[2 * kKvioPitch] | (tc[3 * kKvioPitch] << 16);
        v.z = tc[4 * kKvioPitch] | (tc[5 * kKvioPitch] << 16);
        v.w = tc[6 * kKvioPitch] | (tc[7 * kKvioPitch] << 16);
        *reinterpret_cast<u32x4 *>(vd + 16 * (size_t)q) = blk * 16 + t < a.len ? v : u32x4{0u, 0u, 0u, 0u};
    }
}

// the reverse: rows at or past len are not written (the cache keeps what it holds there)
__global__ __launch_bounds__(256) void k_kv_import(const KvioArgs a) {
    __shared__ uint32_t tile[512 * kKvioPitch];
    const uint32_t tid = threadIdx.x, blk = a.blk0 + blockIdx.x, layer = blockIdx.y;
    const uint64_t off = (uint64_t)blockIdx.x * a.block_stride + (uint64_t)layer * a.layer_stride;
    const uint8_t *src = a.payload + off;
    uint8_t *dst = a.pool + off;
    const uint32_t valid = a.len - blk * 16 < 16 ? a.len - blk * 16 : 16;  // tokens of this block
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const uint32_t i = tid + 256 * j, tok = i >> 6;
        const u32x4 v = *as_global(src + 16 * (size_t)i);
        if (tok < valid) *reinterpret_cast<u32x4 *>(dst + 16 * (size_t)i) = v;
    }
    const uint8_t *vs = src + a.plane_stride;
#pragma unroll
    for (int j = 0; j < 4; ++j) {  // payload token t = q / 64, rows c = 8 (q % 64) .. + 7
        const uint32_t q = tid + 256 * j, t = q >> 6, c = 8 * (q & 63);
        const u32x4 v = *as_global(vs + 16 * (size_t)q);
        uint32_t *tc = tile + c * kKvioPitch + t;
        tc[0] = v.x & 0xffffu;
        tc[kKvioPitch] = v.x >> 16;
        tc[2 * kKvioPitch] = v.y & 0xffffu;
        tc[3 * kKvioPitch] = v.y >> 16;
        tc[4 * kKvioPitch] = v.z & 0xffffu;
        tc[5 * kKvioPitch] = v.z >> 16;
        tc[6 * kKvioPitch] = v.w & 0xffffu;
        tc[7 * kKvioPitch] = v.w >> 16;
    }
    __syncthreads();
    uint8_t *vd = dst + a.plane_stride;
    if (valid == 16) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {  // V^T row r = q / 2, tokens 8 (q % 2) .. + 7
            const uint32_t q = tid + 256 * j, r = q >> 1, t0 = 8 * (q & 1);
            const uint32_t *tr = tile + r * kKvioPitch + t0;
            *reinterpret_cast<u32x4 *>(vd + 16 * (size_t)q) =
                u32x4{tr[0] | (tr[1] << 16), tr[2] | (tr[3] << 16), tr[4] | (tr[5] << 16), tr[6] | (tr[7] << 16)};
        }
    } else {
        uint32_t *vw = reinterpret_cast<uint32_t *>(vd);
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            const uint32_t w = tid + 256 * j, r = w >> 3, t = 2 * (w & 7);
            const uint32_t v = tile[r * kKvioPitch + t] | (tile[r * kKvioPitch + t + 1] << 16);
            if (t + 1 < valid) {
                vw[w] = v;
            } else if (t < valid) {  // the block's last valid token is the low half of this word
                vw[w] = (v & 0xffffu) | (*as_global_u32(vw + w) & 0xffff0000u);
            }
        }
    }
}

hipError_t launch_paged_items(const PagedItemsArgs &a, uint32_t runs, hipStream_t st) {
    OMEGA_LAUNCH(k_paged_items, dim3(runs), dim3(256), 0, st, a);
    return hipGetLastError();
}

// ------------------------------------------------------------------------ paged (VALU)
// One wavefront per (split, kv head, seq): lane = token for Q K (K row per lane, q read
// wave-uniformly), lane = dim pair for P V.
template <int R>  // q heads per kv head
__global__ __launch_bounds__(64) void k_attn(const AttnArgs a) {
    __shared__ float P[R][64];
    const uint32_t lane = threadIdx.x;
    const uint32_t c = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
    const uint32_t ctx = (uint32_t)a.context_lens[b];
    const uint32_t tiles = (ctx + kAttnTile - 1) / kAttnTile;
    uint32_t active, tps;
    attn_split_plan(tiles, gridDim.x, 0, active, tps);
    if (c >= active) return;
    const uint32_t start = c * tps * kAttnTile;
    const uint32_t end = min(ctx, start + tps * kAttnTile);
    const float *q = a.q + ((size_t)b * a.qh + h * R) * 128;
    const int32_t *tab = a.block_tables + (size_t)b * a.max_blocks;
    const uint32_t bs = a.g.block_size;

    float m[R], l[R], o0[R], o1[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        m[r] = -INFINITY;
        l[r] = 0.f;
        o0[r] = 0.f;
        o1[r] = 0.f;
    }
    for (uint32_t sub = start; sub < end; sub += 64) {
        const uint32_t tok = sub + lane;
        const bool valid = tok < end;
        float sc[R];
#pragma unroll
        for (int r = 0; r < R; ++r) sc[r] = 0.f;
        if (valid) {
            const uint32_t blk = (uint32_t)tab[tok / bs];
            const gu32x4 *kp = as_global(a.pool + kv_row_offset(a.g, blk, a.layer, 0, tok % bs, h));
            u32x4 kv[16];
#pragma unroll
            for (int i = 0; i < 16; ++i) kv[i] = __builtin_nontemporal_load(kp + i);
#pragma unroll
            for (int i = 0; i < 16; ++i) {
#pragma unroll
                for (int qd = 0; qd < 4; ++qd) {
                    const float k0 = bf16_lo(kv[i][qd]);
                    const float k1 = bf16_hi(kv[i][qd]);
                    const int d = i * 8 + qd * 2;
#pragma unroll
                    for (int r = 0; r < R; ++r) {
                        sc[r] = fmaf(q[r * 128 + d], k0, sc[r]);
                        sc[r] = fmaf(q[r * 128 + d + 1], k1, sc[r]);
                    }
                }
            }
        }
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const float s = valid ? sc[r] * kInvSqrt128 : -INFINITY;
            float mx = s;
            for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 64));
            const float mn = fmaxf(m[r], mx);
            const float alpha = expf(m[r] - mn);
            const float p = valid ? expf(s - mn) : 0.f;
            float ps = p;
            for (int o = 32; o > 0; o >>= 1) ps += __shfl_xor(ps, o, 64);
            l[r] = l[r] * alpha + ps;
            o0[r] *= alpha;
            o1[r] *= alpha;
            m[r] = mn;
            P[r][lane] = p;
        }
        __syncthreads();
        const uint32_t nt = min(64u, end - sub);
        for (uint32_t t0 = 0; t0 < nt; t0 += 16) {
            // 16 V rows in flight per lane (a dim pair each)
            uint32_t w2[16];
#pragma unroll
            for (int j = 0; j < 16; ++j) {
                uint32_t tv = sub + t0 + j;
                if (a.mutant == 2) tv = min(tv + 1, ctx - 1);
                w2[j] = 0;
                if (t0 + j < nt) {
                    const uint32_t blk = (uint32_t)tab[tv / bs];
                    w2[j] = *as_global_u32(a.pool + kv_row_offset(a.g, blk, a.layer, 1, tv % bs, h) + lane * 4);
                }
            }
#pragma unroll
            for (int j = 0; j < 16; ++j) {
                if (t0 + j >= nt) break;
                const float v0 = bf16_lo(w2[j]), v1 = bf16_hi(w2[j]);
#pragma unroll
                for (int r = 0; r < R; ++r) {
                    o0[r] = fmaf(P[r][t0 + j], v0, o0[r]);
                    o1[r] = fmaf(P[r][t0 + j], v1, o1[r]);
                }
            }
        }
        __syncthreads();
    }
#pragma unroll
    for (int r = 0; r < R; ++r) {
        float *pp = a.part + (((size_t)b * a.qh + h * R + r) * a.splits + c) * kPartStride;
        if (lane == 0) {
            pp[0] = m[r];
            pp[1] = l[r];
        }
        pp[4 + 2 * lane] = o0[r];
        pp[5 + 2 * lane] = o1[r];
    }
}

hipError_t launch_attention(const AttnArgs &a, hipStream_t st) {
    const dim3 grid(a.splits, a.kvh, a.seqs);
    if (paged_mfma(a.qh, a.kvh, a.g.block_size) && a.kvh == 4) {
        const dim3 wgrid(a.splits, a.seqs);
        if (a.mutant == 2) hipLaunchKernelGGL(k_paged4<2>, wgrid, dim3(256), 0, st, a);
        else hipLaunchKernelGGL(k_paged4<0>, wgrid, dim3(256), 0, st, a);
        return hipGetLastError();
    }
    if (paged_mfma(a.qh, a.kvh, a.g.block_size)) {
        // kv head fastest: the heads of one split are dispatched together and read the same
        // pages' 1 KiB token rows at about the same time
        const dim3 hgrid(a.kvh, a.splits, a.seqs);
        if (a.mutant == 2) hipLaunchKernelGGL(k_paged<2>, hgrid, dim3(64), 0, st, a);
        else hipLaunchKernelGGL(k_paged<0>, hgrid, dim3(64), 0, st, a);
        return hipGetLastError();
    }
    switch (a.qh / a.kvh) {
    case 1: hipLaunchKernelGGL(k_attn<1>, grid, dim3(64), 0, st, a); break;
    case 2: hipLaunchKernelGGL(k_attn<2>, grid, dim3(64), 0, st, a); break;
    case 4: hipLaunchKernelGGL(k_attn<4>, grid, dim3(64), 0, st, a); break;
    case 8: hipLaunchKernelGGL(k_attn<8>, grid, dim3(64), 0, st, a); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

namespace {
struct FoldState {
    uint32_t *dev = nullptr;  // g_paged_fold's address on the library's device
    uint32_t epoch = 0;
    int capacity = -1;        // workgroups of k_paged4f resident at once
    bool on = true;
};
FoldState &fold_state() {
    static FoldState f;
    return f;
}
}  // namespace

// The paged call: the folded single launch (k_paged4f) where its grid is resident at once and
// the launch is not recorded into a graph (its epoch is per call), else the split launch and the
// combine launch. *folded tells which ran.
hipError_t launch_paged_call(AttnArgs a, const CombineArgs &cb, int cus, hipStream_t st, bool *folded) {
    FoldState &f = fold_state();
    *folded = false;
    const bool shape = f.on && paged_mfma(a.qh, a.kvh, a.g.block_size) && a.kvh == 4 && a.qh == 32 &&
                       a.splits % 16 == 0 && a.splits <= kPagedFoldMaxSplits &&
                       (size_t)a.splits * a.seqs <= kPagedFoldMax && a.out;
    if (shape && !stream_recording(st)) {
        hipError_t e = hipSuccess;
        if (f.capacity < 0) {
            int per_cu = 0;
            e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, reinterpret_cast<const void *>(k_paged4f<0>), 256, 0);
            if (e != hipSuccess) return e;
            f.capacity = per_cu * cus;
        }
        if (!f.dev && (e = hipGetSymbolAddress(reinterpret_cast<void **>(&f.dev), HIP_SYMBOL(g_paged_fold))) != hipSuccess)
            return e;
        if ((int)(a.splits * a.seqs) <= f.capacity) {
            if (++f.epoch >= (1u << 31)) {  // the flags restart with the epochs
                if ((e = hipMemsetAsync(f.dev, 0, kPagedFoldMax * 4, st)) != hipSuccess) return e;
                f.epoch = 1;
            }
            a.flags = f.dev;
            a.errc = f.dev + kPagedFoldMax;
            a.epoch = f.epoch;
            a.out_scale = cb.out_scale;
            a.merge_spins = a.mutant == 9 ? 0u : kDattnMergeSpins;
            const dim3 grid(a.splits, a.seqs);
            if (a.mutant == 2) hipLaunchKernelGGL(k_paged4f<2>, grid, dim3(256), 0, st, a);
            else hipLaunchKernelGGL(k_paged4f<0>, grid, dim3(256), 0, st, a);
            *folded = true;
            return hipGetLastError();
        }
    }
    hipError_t e = launch_attention(a, st);
    if (e == hipSuccess) e = launch_attn_combine(cb, st);
    return e;
}

// the give-up count of the folded launches (device address), for the entries that report it
uint32_t *paged_fold_errc() { return fold_state().dev ? fold_state().dev + kPagedFoldMax : nullptr; }

// ------------------------------------------------------------------------ split combine
// Paged partials are interleaved dim pairs (o[2 l], o[2 l + 1] from lane l) for the VALU kernel
// and dims in order for the matrix-core kernels; either way partial dim d sits at 4 + d, so one
// combine serves all. One wavefront per (seq, q head, quarter of the dims): lane l covers dim
// 32 q + l % 32 of the slots of parity l / 32, so a workgroup reads 8 KiB of partials per 64
// slots (a CU's loads share one queue). CH chunks of 64 slots (1: up to 16 splits here; more
// splits take k_attn_combine_wide).
template <int CH>
__global__ __launch_bounds__(64) void k_attn_combine(const CombineArgs a) {
    __shared__ float wsh[64 * CH];
    const uint32_t head = blockIdx.x >> 2, quarter = blockIdx.x & 3, b = blockIdx.y, lane = threadIdx.x;
    const uint32_t d = 32 * quarter + (lane & 31), half = lane >> 5;
    const float *pp = a.part + ((size_t)b * a.qh + head) * a.splits * kPartStride;
    // Every slot's (m, l) and o values are loaded before the split count is known (the stale
    // slots past it are dropped below), so the context length and the partials share one round
    // trip.
    float m_raw[CH], l_raw[CH];
#pragma unroll
    for (int c = 0; c < CH; ++c) {
        const uint32_t mslot = min(64 * c + lane, a.splits - 1);
        m_raw[c] = *as_global_f32(pp + mslot * kPartStride);
        l_raw[c] = *as_global_f32(pp + mslot * kPartStride + 1);
    }
    constexpr uint32_t kPer = 32 * CH;
    float f[kPer];
#pragma unroll
    for (uint32_t k = 0; k < kPer; ++k)
        f[k] = *as_global_f32(pp + min(2 * k + half, a.splits - 1) * kPartStride + 4 + d);
    uint32_t tiles;
    if (a.context_lens) tiles = ((uint32_t)a.context_lens[b] + a.tile_tokens - 1) / a.tile_tokens;
    else tiles = ((a.pos_dev ? *as_global_u32(a.pos_dev) : a.pos_host) + a.tile_tokens - 1) / a.tile_tokens;
    uint32_t active, tps;
    attn_split_plan(tiles, a.splits, a.tiles_per_split, active, tps);  // active <= splits <= 64 CH
    // lane s of chunk c holds split 64 c + s's (m, l)
    float M = -INFINITY;
#pragma unroll
    for (int c = 0; c < CH; ++c) M = fmaxf(M, 64 * c + lane < active ? m_raw[c] : -INFINITY);
    M = row16_max(M);
    M = fmaxf(fmaxf(readlane_f32(M, 0), readlane_f32(M, 16)), fmaxf(readlane_f32(M, 32), readlane_f32(M, 48)));
    float L = 0.f;
#pragma unroll
    for (int c = 0; c < CH; ++c) {
        const bool mine = 64 * c + lane < active;
        const float w = mine ? (a.mutant == 4 ? 1.0f : expf(m_raw[c] - M)) : 0.f;
        L += wave_sum(w * (mine ? l_raw[c] : 0.f));
        wsh[64 * c + lane] = w;
    }
    __syncthreads();
    // slots past `active` are selected out, not weighted by 0 (their contents may not be finite)
    float O = 0.f;
#pragma unroll
    for (uint32_t k = 0; k < kPer; ++k) {
        const uint32_t j = 2 * k + half;
        O = j < active ? fmaf(f[k], wsh[j], O) : O;
    }
    O = xor_sum<32>(O);  // even + odd slots
    if (lane < 32) a.out[((size_t)b * a.qh + head) * 128 + d] = O * (a.out_scale / L);
}

// More than 16 splits (up to kCombineWideMax): workgroup (head, quarter of the dims, sequence) of 256
// threads. Thread t holds the (m, l) of split t and the f32x4 pieces (split
// 32 k + t / 8, dims 4 (t % 8) ..) of its quarter, all loaded in one round trip (8 vector loads
// per 256 splits instead of 128 scalar loads per lane); the maximum and the sum of the weighted l
// are workgroup reductions, and the 32 split groups' sums meet in LDS, added in group order.
constexpr uint32_t kCombineWideMax = 256;

template <uint32_t KMAX>  // split rows per thread: up to 32 KMAX splits
__global__ __launch_bounds__(256) void k_attn_combine_wide(const CombineArgs a) {
    __shared__ float red[8];
    __shared__ f32x4 osum[32][8];
    const uint32_t head = blockIdx.x >> 2, quarter = blockIdx.x & 3, b = blockIdx.y, tid = threadIdx.x;
    const uint32_t lane = lane_id(), w = tid >> 6;
    const float *pp = a.part + ((size_t)b * a.qh + head) * a.splits * kPartStride;
    const uint32_t sg = tid >> 3, dc = 4 * (tid & 7);  // split group, dims (within the quarter)
    const uint32_t jm = min(tid, a.splits - 1);
    const float mr = *as_global_f32(pp + (size_t)jm * kPartStride);
    const float lr = *as_global_f32(pp + (size_t)jm * kPartStride + 1);
    f32x4 f[KMAX];
#pragma unroll
    for (uint32_t k = 0; k < KMAX; ++k) {
        const uint32_t j = min(32 * k + sg, a.splits - 1);
        f[k] = *as_global_f32x4(pp + (size_t)j * kPartStride + 4 + 32 * quarter + dc);
    }
    uint32_t tiles;
    if (a.context_lens) tiles = ((uint32_t)a.context_lens[b] + a.tile_tokens - 1) / a.tile_tokens;
    else tiles = ((a.pos_dev ? *as_global_u32(a.pos_dev) : a.pos_host) + a.tile_tokens - 1) / a.tile_tokens;
    uint32_t active, tps;
    attn_split_plan(tiles, a.splits, a.tiles_per_split, active, tps);  // active <= splits <= 256
    // M: the maximum over the active splits
    float M = tid < active ? mr : -INFINITY;
    M = row16_max(M);
    M = fmaxf(fmaxf(readlane_f32(M, 0), readlane_f32(M, 16)), fmaxf(readlane_f32(M, 32), readlane_f32(M, 48)));
    if (lane == 0) red[w] = M;
    __syncthreads();
    M = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    // split t's weight, and L = sum of w l (waves, then in wave order)
    const float w0 = tid < active ? (a.mutant == 4 ? 1.0f : expf(mr - M)) : 0.f;
    const float lw = wave_sum(w0 * (tid < active ? lr : 0.f));
    __shared__ float wsh[kCombineWideMax];
    wsh[tid] = w0;
    if (lane == 0) red[4 + w] = lw;
    __syncthreads();
    const float L = (red[4] + red[5]) + (red[6] + red[7]);
    // this thread's splits 32 k + sg in order; slots past `active` are selected out (their
    // contents may not be finite)
    f32x4 o = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (uint32_t k = 0; k < KMAX; ++k) {
        const uint32_t j = 32 * k + sg;
        if (j < active) {
            const float wj = wsh[j];
            o = f32x4{fmaf(f[k].x, wj, o.x), fmaf(f[k].y, wj, o.y), fmaf(f[k].z, wj, o.z), fmaf(f[k].w, wj, o.w)};
        }
    }
    osum[sg][tid & 7] = o;
    __syncthreads();
    if (tid < 32) {
        float v = 0.f;
        for (uint32_t g = 0; g < 32; ++g) v += osum[g][tid >> 2][tid & 3];
        a.out[((size_t)b * a.qh + head) * 128 + 32 * quarter + tid] = v * (a.out_scale / L);
    }
}

hipError_t launch_attn_combine(const CombineArgs &a, hipStream_t st) {
    if (a.splits > kCombineWideMax) return hipErrorInvalidValue;
    const dim3 grid(a.qh * 4, a.seqs);
    if (a.splits > 128) OMEGA_LAUNCH(k_attn_combine_wide<8>, grid, dim3(256), 0, st, a);
    else if (a.splits > 64) OMEGA_LAUNCH(k_attn_combine_wide<4>, grid, dim3(256), 0, st, a);
    else if (a.splits > 16) OMEGA_LAUNCH(k_attn_combine_wide<2>, grid, dim3(256), 0, st, a);
    else OMEGA_LAUNCH(k_attn_combine<1>, grid, dim3(64), 0, st, a);
    return hipGetLastError();
}

// The items of every (seq, q head) combined, then split into the o projection's e4m3 terms (the
// head's 128 dims are one 128-column block of o's input). Workgroup = (seq, head) of 256 threads:
// the items' (m, l) are read by thread j % 256 of item j, their weights exp(m - M) staged in LDS;
// thread t then sums dims 4 (t % 32) .. +3 over the items j = t / 32 (mod 8) and the 8 groups
// meet in LDS in a fixed order; 16 lanes split the head's row.
// The f32 rows of sequences (prefill tokens) that have at most 64 partials each: one wavefront per
// (sequence, q head), lane j holding partial j's (m, l), lane l dims l and l + 64; the partials
// merge in item order (out = sum w_j o_j / sum w_j l_j with w_j = exp(m_j - max m), times
// out_scale). A token always has a partial that sees its own position, so the maximum is finite.
__global__ __launch_bounds__(256) void k_attn_combine_rows(const CombineItemsArgs a, uint32_t seqs) {
    const uint32_t lane = lane_id(), wv = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (wv >= seqs * 32) return;  // uniform per wavefront
    const uint32_t s = wv >> 5, head = wv & 31;
    const uint32_t off = a.item_off[s], n = a.item_off[s + 1] - off;  // 1 ..= 64
    constexpr size_t kItem = 32 * (size_t)kPartStride;                // floats from one item to the next
    const float *base = a.part + ((size_t)off * 32 + head) * kPartStride;
    const u32x2 ml = *as_global_u32x2(base + min(lane, n - 1) * kItem);
    const float mj = lane < n ? __uint_as_float(ml.x) : -INFINITY;
    float M = row16_max(mj);
    M = fmaxf(fmaxf(readlane_f32(M, 0), readlane_f32(M, 16)), fmaxf(readlane_f32(M, 32), readlane_f32(M, 48)));
    const float wj = lane < n ? expf(mj - M) : 0.f;
    const float L = wave_sum(wj * (lane < n ? __uint_as_float(ml.y) : 0.f));
    float o0 = 0.f, o1 = 0.f;
    for (uint32_t i = 0; i < n; ++i) {
        const float wi = readlane_f32(wj, (int)i);
        const float *p = base + i * kItem + 4;
        o0 = fmaf(wi, *as_global_f32(p + lane), o0);
        o1 = fmaf(wi, *as_global_f32(p + 64 + lane), o1);
    }
    float *out = a.out + ((size_t)s * 32 + head) * 128;
    out[lane] = o0 / L * a.out_scale;
    out[64 + lane] = o1 / L * a.out_scale;
}

__global__ __launch_bounds__(256) void k_attn_combine_items(const CombineItemsArgs a) {
    constexpr uint32_t kRounds = (kCombineMaxItems + 255) / 256;
    __shared__ float wsh[kRounds * 256];
    __shared__ float red[2][4];
    __shared__ f32x4 osum[8][32];
    __shared__ float orow[128];
    const uint32_t s = blockIdx.x >> 5, head = blockIdx.x & 31, t = threadIdx.x;
    const uint32_t lane = lane_id(), wid = t >> 6;
    const uint32_t off = a.item_off[s], n = a.item_off[s + 1] - off;  // 1 ..= kCombineMaxItems
    constexpr size_t kItem = 32 * (size_t)kPartStride;                // floats from one item to the next
    const float *base = a.part + ((size_t)off * 32 + head) * kPartStride;
    float mv[kRounds], lv[kRounds];
    float M = -INFINITY;
#pragma unroll
    for (uint32_t r = 0; r < kRounds; ++r) {
        const uint32_t j = min(t + 256 * r, n - 1);
        const u32x2 ml = *as_global_u32x2(base + j * kItem);
        mv[r] = __uint_as_float(ml.x);
        lv[r] = __uint_as_float(ml.y);
        M = t + 256 * r < n ? fmaxf(M, mv[r]) : M;
    }
    M = row16_max(M);
    M = fmaxf(fmaxf(readlane_f32(M, 0), readlane_f32(M, 16)), fmaxf(readlane_f32(M, 32), readlane_f32(M, 48)));
    if (lane == 0) red[0][wid] = M;
    __syncthreads();
    M = fmaxf(fmaxf(red[0][0], red[0][1]), fmaxf(red[0][2], red[0][3]));
    float Lp = 0.f;
#pragma unroll
    for (uint32_t r = 0; r < kRounds; ++r) {
        const uint32_t j = t + 256 * r;
        const float w = j < n ? expf(mv[r] - M) : 0.f;
        wsh[j] = w;
        Lp += j < n ? w * lv[r] : 0.f;
    }
    Lp = wave_sum(Lp);
    if (lane == 0) red[1][wid] = Lp;
    __syncthreads();
    const float L = (red[1][0] + red[1][1]) + (red[1][2] + red[1][3]);
    const uint32_t grp = t >> 5, d4 = t & 31;
    f32x4 o = {0.f, 0.f, 0.f, 0.f};
#pragma unroll 4
    for (uint32_t j = grp; j < n; j += 8) {
        const f32x4 v = *as_global_f32x4(base + j * kItem + 4 + 4 * d4);
        const float w = wsh[j];
        o.x = fmaf(w, v.x, o.x);
        o.y = fmaf(w, v.y, o.y);
        o.z = fmaf(w, v.z, o.z);
        o.w = fmaf(w, v.w, o.w);
    }
    osum[grp][d4] = o;
    __syncthreads();
    if (t < 32) {
        f32x4 sum = osum[0][t];
#pragma unroll
        for (int g = 1; g < 8; ++g) {
            const f32x4 v = osum[g][t];
            sum.x += v.x;
            sum.y += v.y;
            sum.z += v.z;
            sum.w += v.w;
        }
        const f32x4 r = {sum.x / L * a.out_scale, sum.y / L * a.out_scale, sum.z / L * a.out_scale,
                         sum.w / L * a.out_scale};
        if (a.out) *reinterpret_cast<f32x4 *>(a.out + ((size_t)s * 32 + head) * 128 + 4 * t) = r;
        orow[4 * t + 0] = r.x;
        orow[4 * t + 1] = r.y;
        orow[4 * t + 2] = r.z;
        orow[4 * t + 3] = r.w;
    }
    if (a.out) return;  // uniform: the f32 rows are the result
    __syncthreads();
    if (t < 16) {
        float v[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = orow[8 * t + i];
        u32x2 q[kTerms];
        float sc[kTerms];
        split8(v, q, sc, false);
        store_split(a.oq, a.os, s, 32, head, t, q, sc);
    }
}

hipError_t launch_attn_combine_items(const CombineItemsArgs &a, uint32_t seqs, hipStream_t st) {
    OMEGA_LAUNCH(k_attn_combine_items, dim3(seqs * 32), dim3(256), 0, st, a);
    return hipGetLastError();
}

// RoPE table: the f64 frequency and angle of tensor.rs:150-161 with RopeParams::inv_freq
// (crates/aien-abi-core/src/lib.rs:106-113), cast to f32; [positions][64]
void rope_table(double theta, uint32_t positions, float *cos_out, float *sin_out) {
    double inv[64];
    for (int i = 0; i < 64; ++i) inv[i] = 1.0 / pow(theta, (double)(2 * i) / 128.0);
    for (uint32_t p = 0; p < positions; ++p)
        for (int i = 0; i < 64; ++i) {
            const double rot = (double)p * inv[i];
            cos_out[(size_t)p * 64 + i] = (float)cos(rot);
            sin_out[(size_t)p * 64 + i] = (float)sin(rot);
        }
}

bool paged_mfma(uint32_t qh, uint32_t kvh, uint32_t block_size) { return qh == 8 * kvh && block_size == 16; }

// Splits of a paged launch and the tokens of its split unit. Matrix-core kernel: 16-token pages,
// splits chosen so that the launch holds about 2048 wavefronts (8 per CU) when the pages allow,
// at least two pages per split and at most 256 splits per (seq, kv head). VALU kernel: tiles of
// 64 tokens, one per item up to 64 items.
uint32_t paged_splits(uint32_t max_ctx, uint32_t seqs, uint32_t kvh, bool mfma, uint32_t &unit) {
    unit = mfma ? 16u : kAttnTile;
    const uint32_t units = (max_ctx + unit - 1) / unit;
    if (!mfma) return units < 1 ? 1 : (units > 64 ? 64 : units);
    // at least two pages per split (the page stream stays double-buffered), at most 256 splits
    const uint32_t pairs = seqs * kvh;
    uint32_t s = pairs >= 2048 ? 1u : (2048u + pairs - 1) / pairs;
    const uint32_t cap = units / 2 > 256 ? 256 : units / 2;
    s = s < cap ? s : cap;
    return s < 1 ? 1 : s;
}

KvGeom geom_of(const OmegaGpuKvLayout &l) {
    KvGeom g;
    g.block_stride = l.block_stride_bytes;
    g.layer_stride = l.layer_stride_bytes;
    g.plane_stride = l.kv_plane_stride_bytes;
    g.token_stride = l.token_stride_bytes;
    g.head_stride = l.head_stride_bytes;
    g.block_size = l.block_size;
    return g;
}

}  // namespace omega

// ------------------------------------------------------------------------ fused decode cache
namespace omega {
constexpr uint32_t kRowsChunk = 8192;  // rows per staged chunk of omega_gpu_decode_attn_cache_write
// rows [pos, pos + gridDim.x) of one (layer, kv head) of the fused cache: row i's K into the K
// plane, its V into the transposed V plane (dim d of token t at plane + head * 4096 + d * 32 + t * 2)
__global__ __launch_bounds__(128) void k_cache_write_rows(uint8_t *pool, KvGeom g, uint32_t layer, uint32_t h,
                                                          uint32_t pos, const uint16_t *k, const uint16_t *v) {
    const uint32_t i = blockIdx.x, d = threadIdx.x, p = pos + i;
    uint8_t *page = pool + (uint64_t)(p >> 4) * g.block_stride + (uint64_t)layer * g.layer_stride;
    reinterpret_cast<uint16_t *>(page + (uint64_t)(p & 15) * g.token_stride + (uint64_t)h * g.head_stride)[d] =
        k[(size_t)i * 128 + d];
    *reinterpret_cast<uint16_t *>(page + g.plane_stride + (uint64_t)h * kVtHead + d * 32 + (p & 15) * 2) =
        v[(size_t)i * 128 + d];
}
}  // namespace omega

struct OmegaGpuDecodeAttnCache {
    uint32_t layers = 0, max_pos = 0;
    double theta = 0;
    uint8_t *pool = nullptr;      // [max_pos/16 pages][layers][K|V^T] (16 KiB planes)
    omega::KvGeom g{};
    float *q_norm = nullptr, *k_norm = nullptr;  // [layers][128]
    float *rope_cos = nullptr, *rope_sin = nullptr;  // [max_pos][64]
    // call buffers of the standalone entry
    float *qkv = nullptr, *out = nullptr, *part = nullptr;
    uint32_t *flags = nullptr;  // [4 * 64 split flags][1 error count] of the standalone calls
    uint32_t epoch = 0;         // of the standalone calls (each call takes the next)
};

using namespace omega;

namespace omega {
// for the decode graph
DattnArgs cache_dattn(OmegaGpuDecodeAttnCache *c, uint32_t layer, float eps, const float *qkv,
                      float *part) {
    DattnArgs a;
    a.qkv = qkv;
    a.pool = c->pool;
    a.g = c->g;
    a.layer = layer;
    a.max_pos = c->max_pos;
    a.q_norm = c->q_norm + (size_t)layer * 128;
    a.k_norm = c->k_norm + (size_t)layer * 128;
    a.rope_cos = c->rope_cos;
    a.rope_sin = c->rope_sin;
    a.eps = eps;
    a.tiles_per_split = knobs().dattn_per_split / kDattnPage;
    a.part = part;
    a.mutant = knobs().dattn_mutant;
    a.merge_spins = a.mutant == 9 ? 0u : kDattnMergeSpins;  // test mutant 9: the merge gives up
    return a;
}
uint32_t cache_layers(const OmegaGpuDecodeAttnCache *c) { return c->layers; }
uint32_t cache_max_pos(const OmegaGpuDecodeAttnCache *c) { return c->max_pos; }
}  // namespace omega

extern "C" {

int omega_gpu_decode_attn_cache_alloc(uint32_t layers, uint32_t max_pos, double rope_theta,
                                      OmegaGpuDecodeAttnCache **out) {
    std::lock_guard<std::recursive_mutex> lk(big_lock());
    clear_error(F_DATTN);
    if (!out) return OMEGA_GPU_BAD_ARGS;
    *out = nullptr;
    if (layers == 0 || layers > 64 || max_pos == 0 || max_pos > 131072 || max_pos % 256 != 0) {
        set_error(F_DATTN,
                  "decode attn cache layers=%u max_pos=%u refused: 1 <= layers <= 64, max_pos a "
                  "multiple of 256 up to 131072",
                  layers, max_pos);
        return OMEGA_GPU_BAD_ARGS;
    }
    if (!(rope_theta > 0.0)) {
        set_error(F_DATTN, "decode attn rope_theta %g must be positive", rope_theta);
        return OMEGA_GPU_BAD_ARGS;
    }
    Ctx *cx = ctx(F_DATTN);
    if (!cx) return OMEGA_GPU_CHIP_FAIL;
    OmegaGpuDecodeAttnCache *c = new OmegaGpuDecodeAttnCache();
    c->layers = layers;
    c->max_pos = max_pos;
    c->theta = rope_theta;
    c->g.head_stride = 256;
    c->g.token_stride = 4 * 256;
    c->g.plane_stride = 16 * c->g.token_stride;
    c->g.layer_stride = 2 * c->g.plane_stride;
    c->g.block_stride = (uint64_t)layers * c->g.layer_stride;
    c->g.block_size = 16;
    const size_t pool_bytes = (size_t)(max_pos / 16) * c->g.block_stride;
    std::vector<float> cs((size_t)max_pos * 64), sn((size_t)max_pos * 64);
    rope_table(rope_theta, max_pos, cs.data(), sn.data());
    hipError_t e = dev_malloc(&c->pool, pool_bytes);
    if (e == hipSuccess) e = hipMemset(c->pool, 0, pool_bytes);
    if (e == hipSuccess) e = dev_malloc(&c->q_norm, (size_t)layers * 128 * 4);
    if (e == hipSuccess) e = dev_malloc(&c->k_norm, (size_t)layers * 128 * 4);
    if (e == hipSuccess) e = hipMemset(c->q_norm, 0, (size_t)layers * 128 * 4);
    if (e == hipSuccess) e = hipMemset(c->k_norm, 0, (size_t)layers * 128 * 4);
    if (e == hipSuccess) e = dev_malloc(&c->rope_cos, cs.size() * 4);
    if (e == hipSuccess) e = dev_malloc(&c->rope_sin, sn.size() * 4);
    if (e == hipSuccess) e = hipMemcpy(c->rope_cos, cs.data(), cs.size() * 4, hipMemcpyHostToDevice);
    if (e == hipSuccess) e = hipMemcpy(c->rope_sin, sn.data(), sn.size() * 4, hipMemcpyHostToDevice);
    if (e == hipSuccess) e = dev_malloc(&c->qkv, 5120 * 4);
    if (e == hipSuccess) e = dev_malloc(&c->out, 4096 * 4);
    if (e == hipSuccess) e = dev_malloc(&c->part, (size_t)32 * kDattnSplits * kPartStride * 4);
    if (e == hipSuccess) e = dev_malloc(&c->flags, (4 * kDattnSplits + 1) * 4);
    if (e == hipSuccess) e = hipMemset(c->flags, 0, (4 * kDattnSplits + 1) * 4);
    if (e == hipSuccess) e = hipDeviceSynchronize();
    if (e != hipSuccess) {
        set_error(F_DATTN, "decode attn cache alloc (%u layers x %u): %s", layers, max_pos,
                  hipGetErrorString(e));
        omega_gpu_decode_attn_cache_free(c);
        return e == hipErrorOutOfMemory ? OMEGA_GPU_TOO_LARGE : OMEGA_GPU_CHIP_FAIL;
    }
    *out = c;
    return OMEGA_GPU_OK;
}

void omega_gpu_decode_attn_cache_free(OmegaGpuDecodeAttnCache *c) {
    if (!c) return;
    std::lock_guard<std::recursive_mutex> lk(big_lock());
    Ctx *cx = ctx(F_DATTN);
    if (cx) (void)hipStreamSynchronize(cx->stream);
    void *ps[] = {c->pool, c->q_norm, c->k_norm, c->rope_cos, c->rope_sin, c->qkv, c->out, c->part, c->flags};
    for (void *p : ps)
        if (p) (void)dev_free(p);
    delete c;
}

int omega_gpu_decode_attn_set_norms(OmegaGpuDecodeAttnCache *c, uint32_t layer,
                                    const float *q_norm, const float *k_norm) {
    std::lock_guard<std::recursive_mutex> lk(big_lock());
    clear_error(F_DATTN);
    if (!c || !q_norm || !k_norm) {
        set_error(F_DATTN, "decode attn set_norms: NULL pointer");
        return OMEGA_GPU_BAD_ARGS;
    }
    if (layer >= c->layers) {
        set_error(F_DATTN, "decode attn layer %u >= layers %u", layer, c->layers);
        return OMEGA_GPU_BAD_ARGS;
    }
    OMEGA_HIP(F_DATTN, hipMemcpy(c->q_norm + (size_t)layer * 128, q_norm, 512, hipMemcpyHostToDevice));
    OMEGA_HIP(F_DATTN, hipMemcpy(c->k_norm + (size_t)layer * 128, k_norm, 512, hipMemcpyHostToDevice));
    return OMEGA_GPU_OK;
}

int omega_gpu_decode_attn(OmegaGpuDecodeAttnCache *c, uint32_t layer, uint32_t pos,
                          const float *qkv, float eps, float out_scale, float *out,
                          OmegaGpuDecodeAttnInfo *info) {
    std::lock_guard<std::recursive_mutex> lk(big_lock());
    const uint64_t t0 = now_ns();
    clear_error(F_DATTN);
    if (!c || !qkv || !out) {
        set_error(F_DATTN, "decode attn: NULL pointer");
        return OMEGA_GPU_BAD_ARGS;
    }
    if (layer >= c->layers) {
        set_error(F_DATTN, "decode attn layer %u >= layers %u", layer, c->layers);
        return OMEGA_GPU_BAD_ARGS;
    }
    if (pos >= c->max_pos) {
        set_error(F_DATTN, "decode attn pos %u >= max_pos %u", pos, c->max_pos);
        return OMEGA_GPU_BAD_ARGS;
    }
    Ctx *cx = ctx(F_DATTN);
    if (!cx) return OMEGA_GPU_CHIP_FAIL;
    if (!ensure_pinned(F_DATTN, cx, 5120 * 4)) return OMEGA_GPU_CHIP_FAIL;
    memcpy(cx->pin, qkv, 5120 * 4);
    OMEGA_HIP(F_DATTN, hipMemcpyAsync(c->qkv, cx->pin, 5120 * 4, hipMemcpyHostToDevice, cx->stream));
    DattnArgs a = cache_dattn(c, layer, eps, c->qkv, c->part);
    a.pos_host = pos;
    a.flags = c->flags;
    a.errc = c->flags + 4 * kDattnSplits;
    a.epoch_host = ++c->epoch == 0 ? ++c->epoch : c->epoch;
    a.out = c->out;
    a.out_scale = out_scale;
    OMEGA_HIP(F_DATTN, hipEventRecord(cx->ev0, cx->stream));
    OMEGA_HIP(F_DATTN, launch_dattn(a, cx->stream));
    OMEGA_HIP(F_DATTN, hipEventRecord(cx->ev1, cx->stream));
    OMEGA_HIP(F_DATTN, hipMemcpyAsync(cx->pin, c->out, 4096 * 4, hipMemcpyDeviceToHost, cx->stream));
    uint32_t *errc = reinterpret_cast<uint32_t *>(static_cast<uint8_t *>(cx->pin) + 4096 * 4);
    OMEGA_HIP(F_DATTN, hipMemcpyAsync(errc, a.errc, 4, hipMemcpyDeviceToHost, cx->stream));
    OMEGA_HIP(F_DATTN, hipStreamSynchronize(cx->stream));
    if (*errc) {
        set_error(F_DATTN, "decode attn: the split merge ran out of waits (%u)", *errc);
        OMEGA_HIP(F_DATTN, hipMemset(a.errc, 0, 4));
        return OMEGA_GPU_CHIP_FAIL;
    }
    memcpy(out, cx->pin, 4096 * 4);
    if (info) {
        uint32_t active, tps;
        attn_split_plan((pos + kDattnPage - 1) / kDattnPage, kDattnSplits, a.tiles_per_split, active, tps);
        memset(info, 0, sizeof(*info));
        info->layer = layer;
        info->pos = pos;
        info->splits = active;
        info->per_split = tps * kDattnPage;
        info->depth = 32;
        info->grid_x = 4;
        info->grid_y = kDattnSplits;
        info->threads = 64;
        info->kv_bytes = 2ull * 4 * (pos + 1) * 256;
        info->elapsed_ns = event_ns(cx);
        info->call_ns = now_ns() - t0;
        info->completion_marker = 1;
        info->kernel_cache_hit = 1;
    }
    return OMEGA_GPU_OK;
}

int omega_gpu_decode_attn_cache_write(OmegaGpuDecodeAttnCache *c, uint32_t layer,
                                      uint32_t kv_head, uint32_t pos, uint32_t count,
                                      const uint16_t *k_bf16, const uint16_t *v_bf16) {
    std::lock_guard<std::recursive_mutex> lk(big_lock());
    clear_error(F_DATTN);
    if (!c || !k_bf16 || !v_bf16 || layer >= c->layers || kv_head >= 4 || count == 0 ||
        pos >= c->max_pos || count > c->max_pos - pos) {
        set_error(F_DATTN, "decode attn rows layer %u head %u pos %u count %u outside the cache",
                  layer, kv_head, pos, count);
        return OMEGA_GPU_BAD_ARGS;
    }
    Ctx *cx = ctx(F_DATTN);
    if (!cx) return OMEGA_GPU_CHIP_FAIL;
    // chunks of rows: K | V staged in pinned memory, one copy to the device, one scatter launch
    const uint32_t chunk = std::min<uint32_t>(count, kRowsChunk);
    const size_t bytes = (size_t)chunk * 2 * 256;
    if (!ensure_pinned(F_DATTN, cx, bytes) || !ensure_scratch(F_DATTN, cx, bytes)) return OMEGA_GPU_CHIP_FAIL;
    uint8_t *pin = static_cast<uint8_t *>(cx->pin), *dev = static_cast<uint8_t *>(cx->scratch);
    for (uint32_t i0 = 0; i0 < count; i0 += chunk) {
        const uint32_t n = std::min(chunk, count - i0);
        OMEGA_HIP(F_DATTN, hipStreamSynchronize(cx->stream));  // the pinned staging is free again
        memcpy(pin, k_bf16 + (size_t)i0 * 128, (size_t)n * 256);
        memcpy(pin + (size_t)n * 256, v_bf16 + (size_t)i0 * 128, (size_t)n * 256);
        OMEGA_HIP(F_DATTN, hipMemcpyAsync(dev, pin, (size_t)n * 512, hipMemcpyHostToDevice, cx->stream));
        hipLaunchKernelGGL(k_cache_write_rows, dim3(n), dim3(128), 0, cx->stream, c->pool, c->g, layer, kv_head,
                           pos + i0, reinterpret_cast<const uint16_t *>(dev),
                           reinterpret_cast<const uint16_t *>(dev + (size_t)n * 256));
        OMEGA_HIP(F_DATTN, hipGetLastError());
    }
    OMEGA_HIP(F_DATTN, hipStreamSynchronize(cx->stream));
    return OMEGA_GPU_OK;
}

int omega_gpu_decode_attn_cache_read(OmegaGpuDecodeAttnCache *c, uint32_t layer, uint32_t kv_head,
                                     uint32_t pos, uint16_t *k_bf16, uint16_t *v_bf16) {
    std::lock_guard<std::recursive_mutex> lk(big_lock());
    clear_error(F_DATTN);
    if (!c || !k_bf16 || !v_bf16 || layer >= c->layers || kv_head >= 4 || pos >= c->max_pos) {
        set_error(F_DATTN, "decode attn row layer %u head %u pos %u outside the cache", layer,
                  kv_head, pos);
        return OMEGA_GPU_BAD_ARGS;
    }
    Ctx *cx = ctx(F_DATTN);
    if (!cx) return OMEGA_GPU_CHIP_FAIL;
    OMEGA_HIP(F_DATTN, hipStreamSynchronize(cx->stream));
    const uint64_t page = (uint64_t)(pos / 16) * c->g.block_stride + (uint64_t)layer * c->g.layer_stride;
    const uint64_t ko = page + (uint64_t)(pos % 16) * c->g.token_stride + (uint64_t)kv_head * c->g.head_stride;
    const uint64_t vo = page + c->g.plane_stride + (uint64_t)kv_head * kVtHead + (pos % 16) * 2;
    OMEGA_HIP(F_DATTN, hipMemcpy(k_bf16, c->pool + ko, 256, hipMemcpyDeviceToHost));
    OMEGA_HIP(F_DATTN, hipMemcpy2D(v_bf16, 2, c->pool + vo, 32, 2, 128, hipMemcpyDeviceToHost));
    return OMEGA_GPU_OK;
}

const char *omega_gpu_decode_attn_last_error(void) { return last_error(F_DATTN); }
// ---------------------------------------------------------------- KV park / restore (extension)
extern "C++" {
static int kvio_check(OmegaGpuDecodeAttnCache *c, uint32_t start, uint32_t len, const void *buf, uint64_t bytes,
                      const char *what) {
    if (!c || !buf) {
        set_error(F_DATTN, "kv %s: NULL cache or buffer", what);
        return OMEGA_GPU_BAD_ARGS;
    }
    if (len == 0 || start % 16 || start >= c->max_pos || len > c->max_pos - start) {
        set_error(F_DATTN, "kv %s of positions %u + %u: start a multiple of 16, 1 <= len, inside max_pos %u", what,
                  start, len, c->max_pos);
        return OMEGA_GPU_BAD_ARGS;
    }
    const uint64_t want = (uint64_t)((len + 15) / 16) * c->g.block_stride;
    if (bytes != want) {
        set_error(F_DATTN, "kv %s payload of %llu bytes, %u positions need %llu", what, (unsigned long long)bytes, len,
                  (unsigned long long)want);
        return OMEGA_GPU_BAD_ARGS;
    }
    return OMEGA_GPU_OK;
}

// runs the blocks of [start, start + len) in chunks; per chunk `pre` (a copy in), the kernel, `post`
// (a copy out), all on the library's stream
template <class Pre, class Post>
static int kvio_run(OmegaGpuDecodeAttnCache *c, uint32_t start, uint32_t len, bool exporting, uint8_t *payload_dev,
                    uint64_t chunk_blocks, uint64_t *ns, Pre pre, Post post) {
    Ctx *cx = ctx(F_DATTN);
    if (!cx) return OMEGA_GPU_CHIP_FAIL;
    const uint32_t nblk = (len + 15) / 16;
    OMEGA_HIP(F_DATTN, hipEventRecord(cx->ev0, cx->stream));
    for (uint32_t b0 = 0; b0 < nblk; b0 += (uint32_t)chunk_blocks) {
        const uint32_t nb = (uint32_t)std::min<uint64_t>(chunk_blocks, nblk - b0);
        uint8_t *pd = payload_dev ? payload_dev + (uint64_t)b0 * c->g.block_stride : static_cast<uint8_t *>(cx->scratch);
        OMEGA_HIP(F_DATTN, pre(cx->stream, b0, nb, pd));
        KvioArgs a;
        a.pool = c->pool + (uint64_t)(start / 16 + b0) * c->g.block_stride;
        a.payload = pd;
        a.block_stride = c->g.block_stride;
        a.layer_stride = c->g.layer_stride;
        a.plane_stride = c->g.plane_stride;
        a.blk0 = b0;
        a.len = len;
        if (exporting)
            OMEGA_LAUNCH(k_kv_export, dim3(nb, c->layers), dim3(256), 0, cx->stream, a);
        else
            OMEGA_LAUNCH(k_kv_import, dim3(nb, c->layers), dim3(256), 0, cx->stream, a);
        OMEGA_HIP(F_DATTN, hipGetLastError());
        OMEGA_HIP(F_DATTN, post(cx->stream, b0, nb, pd));
    }
    OMEGA_HIP(F_DATTN, hipEventRecord(cx->ev1, cx->stream));
    OMEGA_HIP(F_DATTN, hipEventSynchronize(cx->ev1));
    float ms = 0.f;
    OMEGA_HIP(F_DATTN, hipEventElapsedTime(&ms, cx->ev0, cx->ev1));
    if (ns) *ns = (uint64_t)((double)ms * 1e6);
    return OMEGA_GPU_OK;
}

static uint64_t kvio_chunk_blocks(const OmegaGpuDecodeAttnCache *c) {
    const uint64_t by_size = (256ull << 20) / c->g.block_stride;  // 256 MiB of staging
    return by_size ? by_size : 1;
}

static hipError_t kvio_none(hipStream_t, uint32_t, uint32_t, uint8_t *) { return hipSuccess; }
}  // extern "C++"

uint64_t omega_gpu_decode_attn_cache_payload_len(const OmegaGpuDecodeAttnCache *c, uint32_t len) {
    return c ? (uint64_t)((len + 15) / 16) * c->g.block_stride : 0;
}

int omega_gpu_decode_attn_cache_export(OmegaGpuDecodeAttnCache *c, uint32_t start, uint32_t len, void *out,
                                       uint64_t out_bytes, uint64_t *ns) {
    std::lock_guard<std::recursive_mutex> lk(big_lock());
    clear_error(F_DATTN);
    if (int rc = kvio_check(c, start, len, out, out_bytes, "export")) return rc;
    Ctx *cx = ctx(F_DATTN);
    if (!cx) return OMEGA_GPU_CHIP_FAIL;
    const uint64_t chunk = kvio_chunk_blocks(c);
    if (!ensure_scratch(F_DATTN, cx, chunk * c->g.block_stride)) return OMEGA_GPU_CHIP_FAIL;
    uint8_t *host = static_cast<uint8_t *>(out);
    const uint64_t bs = c->g.block_stride;
    return kvio_run(c, start, len, true, nullptr, chunk, ns, kvio_none,
                    [&](hipStream_t st, uint32_t b0, uint32_t nb, uint8_t *pd) {
                        return hipMemcpyAsync(host + (uint64_t)b0 * bs, pd, (uint64_t)nb * bs, hipMemcpyDeviceToHost,
                                              st);
                    });
}

int omega_gpu_decode_attn_cache_export_dev(OmegaGpuDecodeAttnCache *c, uint32_t start, uint32_t len, void *out_dev,
                                           uint64_t out_bytes, uint64_t *ns) {
    std::lock_guard<std::recursive_mutex> lk(big_lock());
    clear_error(F_DATTN);
    if (int rc = kvio_check(c, start, len, out_dev, out_bytes, "export")) return rc;
    return kvio_run(c, start, len, true, static_cast<uint8_t *>(out_dev), (len + 15) / 16, ns, kvio_none,
                    kvio_none);
}

// the padding rows of the last block (positions len .. 16 ceil(len / 16) - 1 of every layer's K
// and V plane) must be zero (check_payload, qwen3_moe_omega_kvio.rs:162-186)
// `last` is the payload's last block, `tail` = len % 16 its valid positions (1 ..= 15)
static bool kvio_tail_is_zero(const OmegaGpuDecodeAttnCache *c, uint32_t tail, const uint8_t *last) {
    for (uint32_t l = 0; l < c->layers; ++l)
        for (uint32_t v = 0; v < 2; ++v) {
            const uint8_t *pl = last + (uint64_t)l * c->g.layer_stride + v * c->g.plane_stride;
            for (uint64_t i = (uint64_t)tail * c->g.token_stride; i < c->g.plane_stride; ++i)
                if (pl[i]) return false;
        }
    return true;
}

int omega_gpu_decode_attn_cache_import(OmegaGpuDecodeAttnCache *c, uint32_t start, uint32_t len, const void *bytes,
                                       uint64_t nbytes, uint64_t *ns) {
    std::lock_guard<std::recursive_mutex> lk(big_lock());
    clear_error(F_DATTN);
    if (int rc = kvio_check(c, start, len, bytes, nbytes, "import")) return rc;
    const uint8_t *host = static_cast<const uint8_t *>(bytes);
    if (len % 16 && !kvio_tail_is_zero(c, len % 16, host + (uint64_t)(len / 16) * c->g.block_stride)) {
        set_error(F_DATTN, "kv import: padding rows past position %u are not zero", len);
        return OMEGA_GPU_BAD_ARGS;
    }
    Ctx *cx = ctx(F_DATTN);
    if (!cx) return OMEGA_GPU_CHIP_FAIL;
    const uint64_t chunk = kvio_chunk_blocks(c);
    if (!ensure_scratch(F_DATTN, cx, chunk * c->g.block_stride)) return OMEGA_GPU_CHIP_FAIL;
    const uint64_t bs = c->g.block_stride;
    return kvio_run(
        c, start, len, false, nullptr, chunk, ns,
        [&](hipStream_t st, uint32_t b0, uint32_t nb, uint8_t *pd) {
            return hipMemcpyAsync(pd, host + (uint64_t)b0 * bs, (uint64_t)nb * bs, hipMemcpyHostToDevice, st);
        },
        kvio_none);
}

int omega_gpu_decode_attn_cache_import_dev(OmegaGpuDecodeAttnCache *c, uint32_t start, uint32_t len,
                                           const void *bytes_dev, uint64_t nbytes, uint64_t *ns) {
    std::lock_guard<std::recursive_mutex> lk(big_lock());
    clear_error(F_DATTN);
    if (int rc = kvio_check(c, start, len, bytes_dev, nbytes, "import")) return rc;
    // the padding rows come to the host first (at most layers x 2 x 15 KiB)
    const uint32_t tail = len % 16;
    if (tail) {
        std::vector<uint8_t> last(c->g.block_stride);
        OMEGA_HIP(F_DATTN, hipMemcpy(last.data(), static_cast<const uint8_t *>(bytes_dev) +
                                                      (uint64_t)(len / 16) * c->g.block_stride,
                                     c->g.block_stride, hipMemcpyDeviceToHost));
        if (!kvio_tail_is_zero(c, tail, last.data())) {
            set_error(F_DATTN, "kv import: padding rows past position %u are not zero", len);
            return OMEGA_GPU_BAD_ARGS;
        }
    }
    return kvio_run(c, start, len, false, static_cast<uint8_t *>(const_cast<void *>(bytes_dev)), (len + 15) / 16, ns,
                    kvio_none, kvio_none);
}

// Sub-batches of at most kPattnSub tokens bound the prefill attention's scratch.
constexpr uint32_t kPattnSub = 1024;

// Scratch layout of one prefill attention call of m tokens from pos0: the prepared q rows of a
// sub-batch, its item plan and token offsets, and the partials of its items. Sized from the
// call's own last position, so a short prompt on a large cache asks for little.
struct PattnScratch {
    size_t qn, items, off, part;
    size_t total() const { return qn + items + off + part; }
};
static PattnScratch pattn_scratch(uint32_t pos0, uint32_t m) {
    const uint32_t sub = std::min(kPattnSub, m);
    const uint32_t max_chunks = ((pos0 + m + 15) / 16 + kPattnChunk - 1) / kPattnChunk;
    const size_t max_items = (size_t)sub * max_chunks;
    PattnScratch s;
    s.qn = (size_t)sub * 32 * 128 * 4;
    s.items = (max_items * 16 + 255) / 256 * 256;
    s.off = ((sub + 1) * 4 + 255) / 256 * 256;
    s.part = (max_items * 32 * kPartStride * 4 + 255) / 256 * 256;
    return s;
}

// The prefill attention of m tokens on the fused cache (both entries): qkv_dev [m][5120] and
// out_dev [m][4096] device rows. Sub-batches of at most kPattnSub tokens; each runs the
// preparation (K / V of its tokens appended), the page items and their combine. The working set
// is the first pattn_scratch(pos0, m).total() bytes of the context's scratch.
static int prefill_attn_run(OmegaGpuDecodeAttnCache *c, uint32_t layer, uint32_t pos0, uint32_t m,
                            const float *qkv_dev, float eps, float out_scale, float *out_dev,
                            OmegaGpuPrefillAttnInfo *info, const uint64_t t_call) {
    Ctx *cx = ctx(F_DATTN);
    if (!cx) return OMEGA_GPU_CHIP_FAIL;
    constexpr uint32_t kSub = kPattnSub;
    const PattnScratch sz = pattn_scratch(pos0, m);
    if (!ensure_scratch(F_DATTN, cx, sz.total())) return OMEGA_GPU_CHIP_FAIL;
    const size_t qn_bytes = sz.qn, item_bytes = sz.items, off_bytes = sz.off;
    uint8_t *base = static_cast<uint8_t *>(cx->scratch);
    PattnArgs a;
    a.pool = c->pool;
    a.g = c->g;
    a.layer = layer;
    a.q_norm = c->q_norm + (size_t)layer * 128;
    a.k_norm = c->k_norm + (size_t)layer * 128;
    a.rope_cos = c->rope_cos;
    a.rope_sin = c->rope_sin;
    a.eps = eps;
    a.qn = reinterpret_cast<float *>(base);
    uint32_t *ditems = reinterpret_cast<uint32_t *>(base + qn_bytes);
    uint32_t *doff = reinterpret_cast<uint32_t *>(base + qn_bytes + item_bytes);
    a.items = ditems;
    a.part = reinterpret_cast<float *>(base + qn_bytes + item_bytes + off_bytes);
    std::vector<uint32_t> items, off;
    uint32_t total_items = 0, widest = 0;
    OMEGA_HIP(F_DATTN, hipEventRecord(cx->ev0, cx->stream));
    for (uint32_t t0 = 0; t0 < m; t0 += kSub) {
        const uint32_t mm = std::min(kSub, m - t0);
        items.clear();
        off.assign(mm + 1, 0);
        // groups of tq tokens share their page loads; each group's chunks follow its last token's
        // context, and token j of a group owns the partial slots base * tq + j * nch + chunk (kSub
        // is a multiple of tq, so a group never spans sub-batches)
        const uint32_t ctx_end = pos0 + t0 + mm;
        const uint32_t tq = ctx_end >= kPattnLongCtx ? kPattnTqLong : ctx_end >= kPattnMidCtx ? 2u : 1u;
        uint32_t base = 0;
        for (uint32_t g0 = 0; g0 < mm; g0 += tq) {
            const uint32_t valid = std::min(tq, mm - g0);
            const uint32_t pages = (pos0 + t0 + g0 + valid + 15) / 16, nch = (pages + kPattnChunk - 1) / kPattnChunk;
            for (uint32_t j = 0; j < valid; ++j) off[g0 + j] = base * tq + j * nch;
            off[mm] = base * tq + valid * nch;
            for (uint32_t ch = 0; ch < nch; ++ch) {
                items.push_back(g0);
                items.push_back(ch);
                items.push_back(base);
                items.push_back(nch);
            }
            base += nch;
            widest = std::max(widest, nch);
        }
        const uint32_t n = (uint32_t)(items.size() / 4);
        total_items += n;
        OMEGA_HIP(F_DATTN, hipMemcpyAsync(ditems, items.data(), items.size() * 4, hipMemcpyHostToDevice, cx->stream));
        OMEGA_HIP(F_DATTN, hipMemcpyAsync(doff, off.data(), off.size() * 4, hipMemcpyHostToDevice, cx->stream));
        a.qkv = qkv_dev + (size_t)t0 * 5120;
        a.pos0 = pos0 + t0;
        a.m = mm;
        OMEGA_LAUNCH(k_pattn_prep, dim3(4, mm), dim3(64), 0, cx->stream, a);
        OMEGA_HIP(F_DATTN, hipGetLastError());
        if (tq == 1)
            OMEGA_LAUNCH(k_pattn<1>, dim3(4 * n), dim3(64), 0, cx->stream, a);
        else if (tq == 2)
            OMEGA_LAUNCH(k_pattn<2>, dim3(4 * n), dim3(64), 0, cx->stream, a);
        else
            OMEGA_LAUNCH(k_pattn<kPattnTqLong>, dim3(4 * n), dim3(64), 0, cx->stream, a);
        OMEGA_HIP(F_DATTN, hipGetLastError());
        CombineItemsArgs cb;
        cb.part = a.part;
        cb.item_off = doff;
        cb.out = out_dev + (size_t)t0 * 4096;
        cb.out_scale = out_scale;
        if (widest <= 64) {  // a wavefront per (token, q head)
            OMEGA_LAUNCH(k_attn_combine_rows, dim3((mm * 32 + 3) / 4), dim3(256), 0, cx->stream, cb, mm);
            OMEGA_HIP(F_DATTN, hipGetLastError());
        } else {
            OMEGA_HIP(F_DATTN, launch_attn_combine_items(cb, mm, cx->stream));
        }
        // the host plan is read by the copies above before the next sub-batch rewrites it
        OMEGA_HIP(F_DATTN, hipStreamSynchronize(cx->stream));
    }
    OMEGA_HIP(F_DATTN, hipEventRecord(cx->ev1, cx->stream));
    OMEGA_HIP(F_DATTN, hipEventSynchronize(cx->ev1));
    if (info) {
        float ms = 0.f;
        OMEGA_HIP(F_DATTN, hipEventElapsedTime(&ms, cx->ev0, cx->ev1));
        memset(info, 0, sizeof(*info));
        info->layer = layer;
        info->pos0 = pos0;
        info->m = m;
        info->chunks = total_items;
        info->grid_x = 4 * total_items;
        info->grid_y = 1;
        info->threads = 64;
        info->splits = widest;
        info->per_split = kPattnChunk * 16;
        info->elapsed_ns = (uint64_t)((double)ms * 1e6);
        info->call_ns = now_ns() - t_call;
        info->kernel_cache_hit = 1;
    }
    return OMEGA_GPU_OK;
}

static int prefill_attn_check(OmegaGpuDecodeAttnCache *c, uint32_t layer, uint32_t pos0, uint32_t m) {
    if (!c) {
        set_error(F_DATTN, "prefill attn: NULL cache");
        return OMEGA_GPU_BAD_ARGS;
    }
    if (m == 0 || layer >= c->layers || (uint64_t)pos0 + m > c->max_pos) {
        set_error(F_DATTN, "prefill attn layer %u pos0 %u m %u refused: m >= 1, layer < %u, pos0 + m <= %u", layer,
                  pos0, m, c->layers, c->max_pos);
        return OMEGA_GPU_BAD_ARGS;
    }
    return OMEGA_GPU_OK;
}

int omega_gpu_prefill_attn(OmegaGpuDecodeAttnCache *c, uint32_t layer, uint32_t pos0, uint32_t m, const float *qkv,
                           float eps, float out_scale, float *out, OmegaGpuPrefillAttnInfo *info) {
    std::lock_guard<std::recursive_mutex> lk(big_lock());
    const uint64_t t0 = now_ns();
    clear_error(F_DATTN);
    if (!qkv || !out) {
        set_error(F_DATTN, "prefill attn: NULL q|k|v or out");
        return OMEGA_GPU_BAD_ARGS;
    }
    int rc = prefill_attn_check(c, layer, pos0, m);
    if (rc) return rc;
    Ctx *cx = ctx(F_DATTN);
    if (!cx) return OMEGA_GPU_CHIP_FAIL;
    // the q|k|v and out rows sit in the context's scratch after the run's own working set, so the
    // serving seal and the allocation counters cover this entry like every other host entry
    const size_t qb = (size_t)m * 5120 * 4, ob = (size_t)m * 4096 * 4;
    const size_t run_bytes = (pattn_scratch(pos0, m).total() + 255) / 256 * 256;
    if (!ensure_scratch(F_DATTN, cx, run_bytes + qb + ob)) return OMEGA_GPU_CHIP_FAIL;
    if (!ensure_pinned(F_DATTN, cx, std::max(qb, ob))) return OMEGA_GPU_CHIP_FAIL;
    void *d = static_cast<uint8_t *>(cx->scratch) + run_bytes;
    memcpy(cx->pin, qkv, qb);
    hipError_t e = hipMemcpyAsync(d, cx->pin, qb, hipMemcpyHostToDevice, cx->stream);
    if (e == hipSuccess) {
        float *od = reinterpret_cast<float *>(static_cast<uint8_t *>(d) + qb);
        rc = prefill_attn_run(c, layer, pos0, m, static_cast<const float *>(d), eps, out_scale, od, info, t0);
        if (!rc) {
            e = hipMemcpyAsync(cx->pin, od, ob, hipMemcpyDeviceToHost, cx->stream);
            if (e == hipSuccess) e = hipStreamSynchronize(cx->stream);
            if (e == hipSuccess) memcpy(out, cx->pin, ob);
        }
    }
    (void)hipStreamSynchronize(cx->stream);
    if (e != hipSuccess) {
        set_error(F_DATTN, "prefill attn: %s", hipGetErrorString(e));
        return OMEGA_GPU_CHIP_FAIL;
    }
    if (info) info->call_ns = now_ns() - t0;
    return rc;
}

int omega_gpu_prefill_attn_dev(OmegaGpuDecodeAttnCache *c, uint32_t layer, uint32_t pos0, uint32_t m,
                               uint64_t qkv_va, float eps, float out_scale, uint64_t out_va,
                               OmegaGpuPrefillAttnInfo *info) {
    std::lock_guard<std::recursive_mutex> lk(big_lock());
    const uint64_t t0 = now_ns();
    clear_error(F_DATTN);
    if (!qkv_va || !out_va || qkv_va % 16 || out_va % 16) {
        set_error(F_DATTN, "prefill attn dev: addresses must be non-zero and 16-byte aligned");
        return OMEGA_GPU_BAD_ARGS;
    }
    int rc = prefill_attn_check(c, layer, pos0, m);
    if (rc) return rc;
    return prefill_attn_run(c, layer, pos0, m, reinterpret_cast<const float *>(qkv_va), eps, out_scale,
                            reinterpret_cast<float *>(out_va), info, t0);
}

const char *omega_gpu_decode_attn_rc_name(int rc) { return rc_name(rc); }
void omega_gpu_decode_attn_set_depth(uint32_t depth) { knobs().dattn_depth = depth; }
void omega_gpu_decode_attn_set_per_split(uint32_t per_split) {
    knobs().dattn_per_split = per_split % 256 == 0 ? per_split : 0;
}
void omega_gpu_decode_attn_test_set_mutant(int mutant) { knobs().dattn_mutant = mutant; }

// ------------------------------------------------------------------------ paged attention

static void *g_pool_host = nullptr;

int omega_gpu_attention_pool_alloc(size_t bytes, void **cpu) {
    std::lock_guard<std::recursive_mutex> lk(big_lock());
    clear_error(F_ATTN);
    if (!cpu || bytes == 0) return OMEGA_GPU_ATTN_BAD_ARGS;
    *cpu = nullptr;
    if (g_pool_host) {
        set_error(F_ATTN, "attention pool already allocated (one per process)");
        return OMEGA_GPU_ATTN_BAD_ARGS;
    }
    if (!ctx(F_ATTN)) return OMEGA_GPU_ATTN_CHIP_FAIL;
    hipError_t e = host_malloc(&g_pool_host, bytes, hipHostMallocMapped);
    if (e != hipSuccess) {
        g_pool_host = nullptr;
        set_error(F_ATTN, "attention pool of %zu bytes: %s", bytes, hipGetErrorString(e));
        return OMEGA_GPU_ATTN_TOO_LARGE;
    }
    memset(g_pool_host, 0, bytes);
    *cpu = g_pool_host;
    return OMEGA_GPU_ATTN_OK;
}

void omega_gpu_attention_pool_free(void) {
    std::lock_guard<std::recursive_mutex> lk(big_lock());
    if (!g_pool_host) return;
    Ctx *cx = ctx(F_ATTN);
    if (cx) (void)hipStreamSynchronize(cx->stream);
    (void)host_free(g_pool_host);
    g_pool_host = nullptr;
}

static int check_attn_shape(uint32_t qh, uint32_t kvh, uint32_t hd) {
    if (hd != 128 || kvh == 0 || qh == 0 || qh % kvh != 0) {
        set_error(F_ATTN, "paged attention: head_dim %u (128 only), q heads %u, kv heads %u", hd, qh, kvh);
        return OMEGA_GPU_ATTN_BAD_ARGS;
    }
    const uint32_t r = qh / kvh;
    if (!(r == 1 || r == 2 || r == 4 || r == 8)) {
        set_error(F_ATTN, "paged attention: GQA group %u (1, 2, 4 or 8 supported)", r);
        return OMEGA_GPU_ATTN_TOO_LARGE;
    }
    return OMEGA_GPU_ATTN_OK;
}

static int check_layout(const OmegaGpuKvLayout *l, uint32_t layer, uint32_t kvh) {
    if (!l || l->block_size == 0 || layer >= l->num_layers ||
        l->head_stride_bytes < 256 || l->token_stride_bytes < (uint64_t)kvh * l->head_stride_bytes ||
        l->kv_plane_stride_bytes < (uint64_t)l->block_size * l->token_stride_bytes ||
        l->pool_bytes < (uint64_t)l->num_blocks * l->block_stride_bytes) {
        set_error(F_ATTN, "paged attention: layout does not describe bf16 rows of %u heads x 128", kvh);
        return OMEGA_GPU_ATTN_BAD_ARGS;
    }
    return OMEGA_GPU_ATTN_OK;
}

// The buffers of one host-buffer paged call: device scratch q | out | table | lens | partials |
// staged pages, pinned q | table | lens | staged pages (the output comes back through q).
struct PagedCallBytes {
    size_t o_q, o_out, o_tab, o_len, o_part, o_stage, need;
    size_t p_tab, p_len, p_stage, pin_need;
};
static PagedCallBytes paged_call_bytes(uint32_t seqs, uint32_t max_blocks, uint32_t max_ctx, uint32_t qh, uint32_t kvh,
                                       uint32_t block_size, uint64_t staged) {
    auto al = [](size_t v) { return (v + 255) & ~(size_t)255; };
    const size_t qf = (size_t)seqs * qh * 128, tab_bytes = (size_t)seqs * max_blocks * 4;
    uint32_t unit = kAttnTile;
    const uint32_t splits = paged_splits(max_ctx, seqs, kvh, paged_mfma(qh, kvh, block_size), unit);
    const size_t part_bytes = (size_t)seqs * qh * splits * kPartStride * 4;
    PagedCallBytes b;
    b.o_q = 0;
    b.o_out = al(qf * 4);
    b.o_tab = b.o_out + al(qf * 4);
    b.o_len = b.o_tab + al(tab_bytes);
    b.o_part = b.o_len + al((size_t)seqs * 4);
    b.o_stage = b.o_part + al(part_bytes);
    b.need = b.o_stage + al(staged);
    b.p_tab = al(qf * 4);
    b.p_len = b.p_tab + al(tab_bytes);
    b.p_stage = b.p_len + al((size_t)seqs * 4);
    b.pin_need = b.p_stage + al(staged);
    return b;
}

// Batched paged attention from host buffers. Device pools are read in place; other pools have
// the layer slice of every referenced page staged into device memory first.
static int paged_batch(const float *q, const void *pool, const OmegaGpuKvLayout *layout,
                       const int32_t *tables, const int32_t *lens, uint32_t max_blocks,
                       uint32_t seqs, uint32_t layer, uint32_t qh, uint32_t kvh, float *out,
                       OmegaGpuAttnInfo *info) {
    const uint64_t t0 = now_ns();
    Ctx *cx = ctx(F_ATTN);
    if (!cx) return OMEGA_GPU_ATTN_CHIP_FAIL;
    uint32_t max_ctx = 0;
    uint64_t logical = 0;
    for (uint32_t b = 0; b < seqs; ++b) {
        const int32_t cl = lens[b];
        if (cl <= 0 || (uint64_t)cl > (uint64_t)max_blocks * layout->block_size) {
            set_error(F_ATTN, "paged attention: context %d of sequence %u outside 1..=%llu", cl, b,
                      (unsigned long long)max_blocks * layout->block_size);
            return OMEGA_GPU_ATTN_BAD_ARGS;
        }
        const uint32_t nb = ((uint32_t)cl + layout->block_size - 1) / layout->block_size;
        for (uint32_t i = 0; i < nb; ++i) {
            const int32_t blk = tables[(size_t)b * max_blocks + i];
            if (blk < 0 || (uint32_t)blk >= layout->num_blocks) {
                set_error(F_ATTN, "paged attention: sequence %u block %u is %d (pool has %u)", b, i,
                          blk, layout->num_blocks);
                return OMEGA_GPU_ATTN_BAD_ARGS;
            }
        }
        logical += nb;
        if ((uint32_t)cl > max_ctx) max_ctx = (uint32_t)cl;
    }
    hipPointerAttribute_t attr;
    const bool on_device = hipPointerGetAttributes(&attr, pool) == hipSuccess &&
                           (attr.type == hipMemoryTypeDevice || attr.type == hipMemoryTypeHost ||
                            attr.type == hipMemoryTypeManaged);
    (void)hipGetLastError();
    KvGeom g = geom_of(*layout);
    const size_t qf = (size_t)seqs * qh * 128;
    const size_t tab_bytes = (size_t)seqs * max_blocks * 4;
    // staging plan: device pool -> table as given; host pool -> compact copy of the layer slices
    std::vector<int32_t> tab_dev_host(tables, tables + (size_t)seqs * max_blocks);
    std::vector<int32_t> uniq;
    uint64_t staged = 0;
    const uint8_t *pool_dev = static_cast<const uint8_t *>(pool);
    const uint64_t slice = 2 * layout->kv_plane_stride_bytes;
    uint32_t lay = layer;
    if (!on_device) {
        std::vector<int32_t> slot(layout->num_blocks, -1);
        for (uint32_t b = 0; b < seqs; ++b) {
            const uint32_t nb = ((uint32_t)lens[b] + layout->block_size - 1) / layout->block_size;
            for (uint32_t i = 0; i < nb; ++i) {
                int32_t &e = tab_dev_host[(size_t)b * max_blocks + i];
                if (slot[e] < 0) {
                    slot[e] = (int32_t)uniq.size();
                    uniq.push_back(e);
                }
                e = slot[e];
            }
        }
        staged = uniq.size() * slice;
        g.block_stride = slice;
        g.layer_stride = 0;
        lay = 0;
    }
    const ServingState &sv = serving();
    if (sv.reserved && (seqs > sv.bounds.max_seqs || max_ctx > sv.bounds.max_context || qh != sv.bounds.num_q_heads ||
                        kvh != sv.bounds.num_kv_heads || layout->block_size != sv.bounds.kv_block_size)) {
        set_error(F_ATTN, "serving reservation exceeded: %u sequences, context %u, %u/%u heads, block %u against "
                  "the bounds %u, %u, %u/%u, %u", seqs, max_ctx, qh, kvh, layout->block_size, sv.bounds.max_seqs,
                  sv.bounds.max_context, sv.bounds.num_q_heads, sv.bounds.num_kv_heads, sv.bounds.kv_block_size);
        return OMEGA_GPU_ATTN_TOO_LARGE;
    }
    uint32_t unit = kAttnTile;
    const uint32_t splits = paged_splits(max_ctx, seqs, kvh, paged_mfma(qh, kvh, layout->block_size), unit);
    const PagedCallBytes pb = paged_call_bytes(seqs, max_blocks, max_ctx, qh, kvh, layout->block_size, staged);
    const size_t o_q = pb.o_q, o_out = pb.o_out, o_tab = pb.o_tab, o_len = pb.o_len, o_part = pb.o_part,
                 o_stage = pb.o_stage;
    const size_t p_tab = pb.p_tab, p_len = pb.p_len, p_stage = pb.p_stage;
    if (!ensure_scratch(F_ATTN, cx, pb.need)) return OMEGA_GPU_ATTN_CHIP_FAIL;
    if (!ensure_pinned(F_ATTN, cx, pb.pin_need)) return OMEGA_GPU_ATTN_CHIP_FAIL;
    uint8_t *d = static_cast<uint8_t *>(cx->scratch);
    uint8_t *pin = static_cast<uint8_t *>(cx->pin);
    float *qd = reinterpret_cast<float *>(d + o_q);
    float *od = reinterpret_cast<float *>(d + o_out);
    int32_t *td = reinterpret_cast<int32_t *>(d + o_tab);
    int32_t *lens_dev = reinterpret_cast<int32_t *>(d + o_len);
    float *pd = reinterpret_cast<float *>(d + o_part);
    memcpy(pin, q, qf * 4);
    memcpy(pin + p_tab, tab_dev_host.data(), tab_bytes);
    memcpy(pin + p_len, lens, (size_t)seqs * 4);
    OMEGA_HIP(F_ATTN, hipMemcpyAsync(qd, pin, qf * 4, hipMemcpyHostToDevice, cx->stream));
    OMEGA_HIP(F_ATTN, hipMemcpyAsync(td, pin + p_tab, tab_bytes, hipMemcpyHostToDevice, cx->stream));
    OMEGA_HIP(F_ATTN, hipMemcpyAsync(lens_dev, pin + p_len, (size_t)seqs * 4, hipMemcpyHostToDevice, cx->stream));
    if (!on_device) {
        // gather the layer slices host-side into pinned memory, one copy up
        uint8_t *st = pin + p_stage;
        for (size_t i = 0; i < uniq.size(); ++i)
            memcpy(st + i * slice,
                   static_cast<const uint8_t *>(pool) + (uint64_t)uniq[i] * layout->block_stride_bytes +
                       (uint64_t)layer * layout->layer_stride_bytes,
                   slice);
        OMEGA_HIP(F_ATTN, hipMemcpyAsync(d + o_stage, st, staged, hipMemcpyHostToDevice, cx->stream));
        pool_dev = d + o_stage;
    }
    AttnArgs a;
    a.q = qd;
    a.pool = pool_dev;
    a.g = g;
    a.layer = lay;
    a.block_tables = td;
    a.max_blocks = max_blocks;
    a.context_lens = lens_dev;
    a.seqs = seqs;
    a.qh = qh;
    a.kvh = kvh;
    a.splits = splits;
    a.part = pd;
    a.mutant = knobs().dattn_mutant;
    CombineArgs cb;
    cb.part = pd;
    cb.splits = splits;
    cb.tile_tokens = unit;
    cb.context_lens = lens_dev;
    cb.seqs = seqs;
    cb.qh = qh;
    cb.out = od;
    cb.mutant = a.mutant;
    a.out = od;
    a.ctx_hint = (uint32_t)*std::max_element(lens, lens + seqs);
    // the folded launch's give-up count, cleared before and read back after (through the pinned
    // table words, whose upload is ahead in the stream)
    uint32_t *errc = paged_fold_errc();
    if (errc) OMEGA_HIP(F_ATTN, hipMemsetAsync(errc, 0, 4, cx->stream));
    bool folded = false;
    OMEGA_HIP(F_ATTN, hipEventRecord(cx->ev0, cx->stream));
    OMEGA_HIP(F_ATTN, launch_paged_call(a, cb, cx->cus, cx->stream, &folded));
    OMEGA_HIP(F_ATTN, hipEventRecord(cx->ev1, cx->stream));
    OMEGA_HIP(F_ATTN, hipMemcpyAsync(pin, od, qf * 4, hipMemcpyDeviceToHost, cx->stream));
    uint32_t *late = reinterpret_cast<uint32_t *>(pin + p_tab);
    if (folded) OMEGA_HIP(F_ATTN, hipMemcpyAsync(late, paged_fold_errc(), 4, hipMemcpyDeviceToHost, cx->stream));
    OMEGA_HIP(F_ATTN, hipStreamSynchronize(cx->stream));
    if (folded && *late) {
        set_error(F_ATTN, "paged attention: the in-launch split merge ran out of waits (%u)", *late);
        return OMEGA_GPU_ATTN_CHIP_FAIL;
    }
    memcpy(out, pin, qf * 4);
    if (info) {
        memset(info, 0, sizeof(*info));
        info->chip_calls = 1;
        info->elapsed_ns = event_ns(cx);
        info->call_ns = now_ns() - t0;
        info->completion_marker = 1;
        info->kernel_cache_hit = true;
        info->ctas_last_launch = splits * kvh * seqs;
        info->threads_per_cta = 64;
        fill_chip(info->target_chip, &info->sm_architecture, cx);
        info->kv_bytes_staged = staged;
        info->kv_bytes_naive = logical * slice;
        info->kv_blocks_logical = (uint32_t)logical;
        info->kv_blocks_unique = on_device ? (uint32_t)logical : (uint32_t)uniq.size();
        info->q_bytes = qf * 4;
        info->tab_bytes = tab_bytes;
        info->out_bytes = qf * 4;
        info->kv_source = on_device ? OMEGA_GPU_ATTN_KV_RESIDENT : OMEGA_GPU_ATTN_KV_STAGED;
    }
    return OMEGA_GPU_ATTN_OK;
}

int omega_gpu_paged_attention_bf16(const float *q, const void *pool, const OmegaGpuKvLayout *layout,
                                   const uint32_t *block_ids, uint32_t num_block_ids,
                                   uint32_t context_len, uint32_t layer_idx, uint32_t num_q_heads,
                                   uint32_t num_kv_heads, uint32_t head_dim, float *out,
                                   OmegaGpuAttnInfo *info) {
    std::lock_guard<std::recursive_mutex> lk(big_lock());
    clear_error(F_ATTN);
    if (!q || !pool || !layout || !block_ids || !out) {
        set_error(F_ATTN, "paged attention: NULL pointer");
        return OMEGA_GPU_ATTN_BAD_ARGS;
    }
    int rc = check_attn_shape(num_q_heads, num_kv_heads, head_dim);
    if (!rc) rc = check_layout(layout, layer_idx, num_kv_heads);
    if (rc) return rc;
    if (context_len == 0 || (uint64_t)context_len > (uint64_t)num_block_ids * layout->block_size) {
        set_error(F_ATTN, "paged attention: context %u needs more than %u blocks of %u", context_len,
                  num_block_ids, layout->block_size);
        return OMEGA_GPU_ATTN_BAD_ARGS;
    }
    std::vector<int32_t> tab(num_block_ids);
    for (uint32_t i = 0; i < num_block_ids; ++i) {
        if (block_ids[i] > 0x7fffffffu) {
            set_error(F_ATTN, "paged attention: block id %u out of range", block_ids[i]);
            return OMEGA_GPU_ATTN_BAD_ARGS;
        }
        tab[i] = (int32_t)block_ids[i];
    }
    const int32_t cl = (int32_t)context_len;
    return paged_batch(q, pool, layout, tab.data(), &cl, num_block_ids, 1, layer_idx, num_q_heads,
                       num_kv_heads, out, info);
}

int omega_gpu_paged_attention_batch_bf16(const float *q, const void *pool,
                                         const OmegaGpuKvLayout *layout,
                                         const int32_t *block_tables, const int32_t *context_lens,
                                         uint32_t max_blocks_per_seq, uint32_t num_seqs,
                                         uint32_t layer_idx, uint32_t num_q_heads,
                                         uint32_t num_kv_heads, uint32_t head_dim, float *out,
                                         OmegaGpuAttnInfo *info) {
    std::lock_guard<std::recursive_mutex> lk(big_lock());
    clear_error(F_ATTN);
    if (!q || !pool || !layout || !block_tables || !context_lens || !out || num_seqs == 0 ||
        max_blocks_per_seq == 0) {
        set_error(F_ATTN, "paged attention batch: NULL pointer or empty batch");
        return OMEGA_GPU_ATTN_BAD_ARGS;
    }
    int rc = check_attn_shape(num_q_heads, num_kv_heads, head_dim);
    if (!rc) rc = check_layout(layout, layer_idx, num_kv_heads);
    if (rc) return rc;
    return paged_batch(q, pool, layout, block_tables, context_lens, max_blocks_per_seq, num_seqs,
                       layer_idx, num_q_heads, num_kv_heads, out, info);
}

// ------------------------------------------------- the same attention without any allocation
// For callers that cannot allocate (graph capture, fixed serving loops): the split partials live
// in `scratch`, a file-scope device array of kNoAllocScratchBytes that every GPU the library runs
// on holds until the process ends. In host code `scratch` names a host-side stand-in, so the
// kernels get the device address hipGetSymbolAddress returns for it, fetched once per device
// (with that device current) on the entry point's first call there. The partials need no
// clearing: the combine reads only splits that the attention launch of the same call writes.
namespace omega {
constexpr size_t kNoAllocScratchBytes = 16u << 20;
}  // namespace omega

static __device__ __align__(256) float scratch[omega::kNoAllocScratchBytes / sizeof(float)];

namespace omega {
namespace {
constexpr int kNoAllocDevices = 64;
static float *g_scratch_dev[kNoAllocDevices];  // device address of `scratch` per device, or null

static int noalloc_scratch(Ctx *cx, float **out) {
    if (cx->device < 0 || cx->device >= kNoAllocDevices) {
        set_error(F_ATTN, "paged attention noalloc: device %d outside 0..%d", cx->device, kNoAllocDevices - 1);
        return OMEGA_GPU_ATTN_CHIP_FAIL;
    }
    if (!g_scratch_dev[cx->device]) {
        int cur = -1;
        hipError_t e = hipGetDevice(&cur);
        if (e == hipSuccess && cur != cx->device) e = hipSetDevice(cx->device);
        void *p = nullptr;
        if (e == hipSuccess) e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (cur >= 0 && cur != cx->device) (void)hipSetDevice(cur);
        if (e != hipSuccess || !p) {
            set_error(F_ATTN, "paged attention noalloc: hipGetSymbolAddress(scratch) on device %d: %s",
                      cx->device, hipGetErrorString(e));
            return OMEGA_GPU_ATTN_CHIP_FAIL;
        }
        g_scratch_dev[cx->device] = static_cast<float *>(p);
    }
    *out = g_scratch_dev[cx->device];
    return OMEGA_GPU_ATTN_OK;
}

// The device-pointer batched attention. Its split partials go to the library's scratch (grown as
// needed), or with `noalloc` to `scratch`, and then a shape whose partials exceed
// kNoAllocScratchBytes is refused with TOO_LARGE.
static int paged_batch_dev(const char *what, const float *q_dev, const void *pool_dev, const OmegaGpuKvLayout *layout,
                           const int32_t *block_tables_dev, const int32_t *context_lens_dev,
                           uint32_t max_blocks_per_seq, uint32_t num_seqs, uint32_t max_context,
                           uint32_t layer_idx, uint32_t num_q_heads, uint32_t num_kv_heads, uint32_t head_dim,
                           float *out_dev, bool noalloc) {
    if (!q_dev || !pool_dev || !layout || !block_tables_dev || !context_lens_dev || !out_dev ||
        num_seqs == 0 || max_context == 0) {
        set_error(F_ATTN, "%s: NULL pointer or empty batch", what);
        return OMEGA_GPU_ATTN_BAD_ARGS;
    }
    int rc = check_attn_shape(num_q_heads, num_kv_heads, head_dim);
    if (!rc) rc = check_layout(layout, layer_idx, num_kv_heads);
    if (rc) return rc;
    Ctx *cx = ctx(F_ATTN);
    if (!cx) return OMEGA_GPU_ATTN_CHIP_FAIL;
    // every context must fit max_context: the split count is planned from it
    uint32_t unit = kAttnTile;
    const uint32_t splits = paged_splits(max_context, num_seqs, num_kv_heads,
                                         paged_mfma(num_q_heads, num_kv_heads, layout->block_size), unit);
    const size_t part_bytes = (size_t)num_seqs * num_q_heads * splits * kPartStride * 4;
    float *part = nullptr;
    if (noalloc) {
        if (part_bytes > kNoAllocScratchBytes) {
            set_error(F_ATTN, "%s: %u sequences x %u q heads x %u splits need %zu bytes of partials, the "
                      "static scratch holds %zu", what, num_seqs, num_q_heads, splits, part_bytes, kNoAllocScratchBytes);
            return OMEGA_GPU_ATTN_TOO_LARGE;
        }
        rc = noalloc_scratch(cx, &part);
        if (rc) return rc;
    } else {
        if (!ensure_scratch(F_ATTN, cx, part_bytes)) return OMEGA_GPU_ATTN_CHIP_FAIL;
        part = static_cast<float *>(cx->scratch);
    }
    AttnArgs a;
    a.q = q_dev;
    a.pool = static_cast<const uint8_t *>(pool_dev);
    a.g = geom_of(*layout);
    a.layer = layer_idx;
    a.block_tables = block_tables_dev;
    a.max_blocks = max_blocks_per_seq;
    a.context_lens = context_lens_dev;
    a.seqs = num_seqs;
    a.qh = num_q_heads;
    a.kvh = num_kv_heads;
    a.splits = splits;
    a.part = part;
    a.mutant = knobs().dattn_mutant;
    CombineArgs cb;
    cb.part = a.part;
    cb.splits = splits;
    cb.tile_tokens = unit;
    cb.context_lens = context_lens_dev;
    cb.seqs = num_seqs;
    cb.qh = num_q_heads;
    cb.out = out_dev;
    cb.mutant = a.mutant;
    a.out = out_dev;
    a.ctx_hint = max_context;
    bool folded = false;
    OMEGA_HIP(F_ATTN, launch_paged_call(a, cb, cx->cus, cx->stream, &folded));
    return OMEGA_GPU_ATTN_OK;
}
}  // namespace
}  // namespace omega

void omega_gpu_paged_attention_set_folded(int on) {
    std::lock_guard<std::recursive_mutex> lk(big_lock());
    fold_state().on = on != 0;
}

int omega_gpu_paged_attention_batch_dev(const float *q_dev, const void *pool_dev,
                                        const OmegaGpuKvLayout *layout,
                                        const int32_t *block_tables_dev,
                                        const int32_t *context_lens_dev,
                                        uint32_t max_blocks_per_seq, uint32_t num_seqs,
                                        uint32_t max_context, uint32_t layer_idx,
                                        uint32_t num_q_heads, uint32_t num_kv_heads,
                                        uint32_t head_dim, float *out_dev) {
    std::lock_guard<std::recursive_mutex> lk(big_lock());
    clear_error(F_ATTN);
    return paged_batch_dev("paged attention dev", q_dev, pool_dev, layout, block_tables_dev, context_lens_dev,
                           max_blocks_per_seq, num_seqs, max_context, layer_idx, num_q_heads, num_kv_heads,
                           head_dim, out_dev, false);
}

int omega_gpu_paged_attention_batch_dev_noalloc(const float *q_dev, const void *pool_dev,
                                                const OmegaGpuKvLayout *layout,
                                                const int32_t *block_tables_dev,
                                                const int32_t *context_lens_dev,
                                                uint32_t max_blocks_per_seq, uint32_t num_seqs,
                                                uint32_t max_context, uint32_t layer_idx,
                                                uint32_t num_q_heads, uint32_t num_kv_heads,
                                                uint32_t head_dim, float *out_dev) {
    std::lock_guard<std::recursive_mutex> lk(big_lock());
    clear_error(F_ATTN);
    return paged_batch_dev("paged attention noalloc", q_dev, pool_dev, layout, block_tables_dev, context_lens_dev,
                           max_blocks_per_seq, num_seqs, max_context, layer_idx, num_q_heads, num_kv_heads,
                           head_dim, out_dev, true);
}

int omega_gpu_paged_attention_items_dev(const float *q_dev, const void *pool_dev, const OmegaGpuKvLayout *layout,
                                        const int32_t *block_tables_dev, uint32_t max_blocks_per_seq,
                                        const uint32_t *positions, uint32_t num_seqs, uint32_t layer_idx,
                                        float *out_dev) {
    std::lock_guard<std::recursive_mutex> lk(big_lock());
    clear_error(F_ATTN);
    if (!q_dev || !pool_dev || !layout || !block_tables_dev || !positions || !out_dev || num_seqs == 0 ||
        num_seqs > kItemMaxSeqs) {
        set_error(F_ATTN, "paged attention items: NULL pointer or %u sequences (1..=%u)", num_seqs, kItemMaxSeqs);
        return OMEGA_GPU_ATTN_BAD_ARGS;
    }
    int rc = check_layout(layout, layer_idx, 4);
    if (rc) return rc;
    if (layout->block_size != 16) {
        set_error(F_ATTN, "paged attention items: 16-token pages required (block_size %u)", layout->block_size);
        return OMEGA_GPU_ATTN_BAD_ARGS;
    }
    ItemPlan plan{};
    uint32_t first[kItemMaxSeqs + 1];
    uint32_t total = 0;
    for (uint32_t s = 0; s < num_seqs; ++s) {
        if ((uint64_t)positions[s] >= (uint64_t)max_blocks_per_seq * 16) {
            set_error(F_ATTN, "paged attention items: sequence %u position %u past its %u-page table", s,
                      positions[s], max_blocks_per_seq);
            return OMEGA_GPU_ATTN_BAD_ARGS;
        }
        first[s] = total;
        total += (positions[s] + 1 + 15) / 16;
    }
    first[num_seqs] = total;
    plan_items(first, num_seqs, plan);
    Ctx *cx = ctx(F_ATTN);
    if (!cx) return OMEGA_GPU_ATTN_CHIP_FAIL;
    const size_t plan_bytes = (sizeof(ItemPlan) + 255) / 256 * 256, pos_bytes = 256;
    if (!ensure_scratch(F_ATTN, cx, plan_bytes + pos_bytes + (size_t)kItemMax * 32 * kPartStride * 4))
        return OMEGA_GPU_ATTN_CHIP_FAIL;
    uint8_t *base = static_cast<uint8_t *>(cx->scratch);
    ItemPlan *dplan = reinterpret_cast<ItemPlan *>(base);
    uint32_t *dpos = reinterpret_cast<uint32_t *>(base + plan_bytes);
    OMEGA_HIP(F_ATTN, hipMemcpyAsync(dplan, &plan, sizeof(ItemPlan), hipMemcpyHostToDevice, cx->stream));
    OMEGA_HIP(F_ATTN, hipMemcpyAsync(dpos, positions, num_seqs * 4, hipMemcpyHostToDevice, cx->stream));
    PagedItemsArgs pa;
    pa.q = q_dev;
    pa.pool = static_cast<const uint8_t *>(pool_dev);
    pa.g = geom_of(*layout);
    pa.layer = layer_idx;
    pa.tables = block_tables_dev;
    pa.max_blocks = max_blocks_per_seq;
    pa.pos = dpos;
    pa.run_off = dplan->run_off;
    pa.items = &dplan->items[0][0];
    pa.part = reinterpret_cast<float *>(base + plan_bytes + pos_bytes);
    OMEGA_HIP(F_ATTN, launch_paged_items(pa, kItemRuns, cx->stream));
    CombineItemsArgs ca;
    ca.part = pa.part;
    ca.item_off = dplan->item_off;
    ca.out = out_dev;
    OMEGA_HIP(F_ATTN, launch_attn_combine_items(ca, num_seqs, cx->stream));
    // the host plan and positions are read by the copies above: wait before they go out of scope
    OMEGA_HIP(F_ATTN, hipStreamSynchronize(cx->stream));
    return OMEGA_GPU_ATTN_OK;
}

const char *omega_gpu_attention_rc_name(int rc) {
    return rc == -5 ? "UNWRITTEN" : rc_name(rc);
}
const char *omega_gpu_attention_last_error(void) { return last_error(F_ATTN); }

// ---------------------------------------------------------------- serving reservation
// omega_gpu_reserve_serving (aien-omega-gpu/src/lib.rs:1129-1160): the bounds a daemon declares at
// start-up. The host-buffer paged attention's device scratch and pinned staging are sized now for
// the largest call inside them (max_seqs sequences of max_context tokens, every page staged from
// a host pool), all before the call returns; afterwards a paged call past the bounds is refused
// with TOO_LARGE. _seal makes every later growth of the library's scratch or staging a refusal;
// _release lifts both. The counters of omega_gpu_session_alloc_stats cover those allocations.
int omega_gpu_reserve_serving(const OmegaGpuServingBounds *b) {
    std::lock_guard<std::recursive_mutex> lk(big_lock());
    clear_error(F_MATMUL);
    if (!b || b->max_context == 0 || b->max_seqs == 0 || b->head_dim != 128 || b->kv_block_size == 0 ||
        (b->kv_block_size & (b->kv_block_size - 1)) || b->kernel_slots > 128 || b->num_kv_heads == 0 ||
        b->num_q_heads % b->num_kv_heads || b->num_q_heads / b->num_kv_heads > 16) {
        set_error(F_MATMUL, "serving bounds refused: context and sequences >= 1, head_dim 128, a power-of-two "
                  "block size, q heads a multiple (<= 16) of kv heads, at most 128 kernel slots");
        return OMEGA_GPU_BAD_ARGS;
    }
    Ctx *cx = ctx(F_ATTN);
    if (!cx) {
        set_error(F_MATMUL, "serving reservation: %s", last_error(F_ATTN));
        return OMEGA_GPU_CHIP_FAIL;
    }
    const uint32_t bs = b->kv_block_size, max_blocks = (b->max_context + bs - 1) / bs;
    const uint64_t slice = 2ull * bs * b->num_kv_heads * 256;  // a page's K and V of one layer
    const uint64_t staged = (uint64_t)b->max_seqs * max_blocks * slice;
    const PagedCallBytes pb = paged_call_bytes(b->max_seqs, max_blocks, b->max_context, b->num_q_heads,
                                               b->num_kv_heads, bs, staged);
    serving().sealed = false;
    if (!ensure_scratch(F_ATTN, cx, pb.need) || !ensure_pinned(F_ATTN, cx, pb.pin_need)) {
        set_error(F_MATMUL, "serving reservation of %zu + %zu bytes: %s", pb.need, pb.pin_need, last_error(F_ATTN));
        return OMEGA_GPU_CHIP_FAIL;
    }
    serving().bounds = *b;
    serving().reserved = true;
    return OMEGA_GPU_OK;
}

void omega_gpu_serving_seal(void) {
    std::lock_guard<std::recursive_mutex> lk(big_lock());
    serving().sealed = true;
}

void omega_gpu_serving_release(void) {
    std::lock_guard<std::recursive_mutex> lk(big_lock());
    serving().sealed = false;
    serving().reserved = false;
}

void omega_gpu_session_alloc_stats(OmegaGpuAllocStats *out) {
    std::lock_guard<std::recursive_mutex> lk(big_lock());
    if (out) *out = alloc_counters();
}

}  // extern "C"
