// The fused decode attention's building blocks, shared by the standalone kernel (k_dattn,
// attn.hip) and the persistent token kernel (ptoken.hip): the 16-token page in registers, its
// load, one online-softmax page step on the bf16 matrix cores, one (split, kv head) wavefront's
// whole work up to its flagged partial, and the split merge of one q head.
//
// Host oracle: scaled_dot_product_attention_single (crates/aien-inference-abi/src/tensor.rs:
// 193-250) over the bf16 rows of the cache; the q|k|v preparation is rmsnorm_per_head
// (qwen3_coder.rs:306-320, f64 sum of squares) then apply_rope (tensor.rs:164-190) and the bf16
// append of aien-kv-cache write_token_kv.
#pragma once

#include <cmath>

#include "device.hpp"
#include "kernels.hpp"

namespace omega {

constexpr float kInvSqrt128 = 0.08838834764831845f;
constexpr uint32_t kVtHead = 4096;  // bytes per kv head of a transposed V plane (128 dims x 32 B)


typedef short s16x4 __attribute__((ext_vector_type(4)));  // a 16x16x16 bf16 operand

// one 16-token page: lane (g = lane / 16, n = lane % 16) holds token n's K dims 32 ks + 8 g .. +8
// for k-step ks (the four lane groups of a k-step read 64 contiguous bytes of each K row), and
// V^T[dim 16 nb + n][tokens 4 g .. +4] for n-block nb
struct DattnPage {
    u32x4 k[4];
    u32x2 v[8];
};

__device__ __forceinline__ void dattn_load(const DattnArgs &a, uint32_t h, uint32_t page, uint32_t lane,
                                           DattnPage &T) {
    const uint32_t g = lane >> 4, n = lane & 15;
    const uint8_t *pg = a.pool + (uint64_t)a.layer * a.g.layer_stride + (uint64_t)page * a.g.block_stride;
    const gu32x4 *kp = as_global(pg + (uint64_t)n * a.g.token_stride + (uint64_t)h * a.g.head_stride + 16 * g);
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) T.k[ks] = __builtin_nontemporal_load(kp + 4 * ks);
    const uint8_t *vp = pg + a.g.plane_stride + (uint64_t)h * kVtHead + n * 32 + 8 * g;
#pragma unroll
    for (int nb = 0; nb < 8; ++nb) T.v[nb] = __builtin_nontemporal_load(as_global_u32x2(vp + nb * 16 * 32));
}


// One online-softmax step over a page whose first token is tok0 (< pos). The online state of
// head n % 8 (m, l) sits in every lane of column n; O[nb][i] is row 4 g + i (head (4 g + i) % 8,
// hi half for g < 2, lo half otherwise), dim 16 nb + n.
// GUARD: the page may hold no valid token for a running state that has seen none either (the
// prefill's query tiles), so a maximum of -inf is replaced by 0 as the exponent's reference.
template <bool FIRST, bool GUARD = false>  // FIRST: no earlier page (the running state starts here)
__device__ __forceinline__ void dattn_page(const DattnPage &T, const bf16x8 (&qop)[4], uint32_t tok0,
                                           uint32_t pos, uint32_t g, uint32_t n, float &m_l, float &l_l,
                                           f32x4 (&O)[8]) {
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(T.k[ks]), qop[ks], acc, 0, 0, 0);
    float sc[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const float full = acc[i] + dpp_f32<DPP_ROR8>(acc[i]);  // hi + lo columns
        sc[i] = tok0 + 4 * g + i < pos ? full * kInvSqrt128 : -INFINITY;
    }
    // max and sum over the four lane groups (rows) of a column: row swaps, no LDS
    const float mx = xor_max<32>(xor_max<16>(fmaxf(fmaxf(sc[0], sc[1]), fmaxf(sc[2], sc[3]))));
    const float m_new = FIRST ? mx : fmaxf(m_l, mx);  // finite unless GUARD: token tok0 is valid
    const float m_ref = GUARD && m_new == -INFINITY ? 0.f : m_new;
    float pr[4];
    float psum = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        pr[i] = expf(sc[i] - m_ref);
        psum += pr[i];
    }
    psum = xor_sum<32>(xor_sum<16>(psum));
    if (FIRST) {
        l_l = psum;
    } else {
        const float alpha = expf(m_l - m_ref);
        l_l = l_l * alpha + psum;
        // accumulator row 4 g + i belongs to head (4 g + i) % 8: head i for even g, 4 + i for
        // odd g, whose alpha every row's lane (head) holds
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float a_lo = readlane_f32(alpha, i), a_hi = readlane_f32(alpha, 4 + i);
            const float ai = (g & 1) ? a_hi : a_lo;
#pragma unroll
            for (int nb = 0; nb < 8; ++nb) O[nb][i] *= ai;
        }
    }
    m_l = m_new;
    // A operand of O = P V: row n = head n % 8 (hi or lo half), k = tokens 4 g .. +4
    s16x4 pop;
#pragma unroll
    for (int i = 0; i < 4; ++i) pop[i] = (short)(n < 8 ? bf16_split_hi(pr[i]) : bf16_split_lo(pr[i]));
#pragma unroll
    for (int nb = 0; nb < 8; ++nb)
        O[nb] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(pop, __builtin_bit_cast(s16x4, T.v[nb]), O[nb], 0, 0, 0);
}


// LDS of one attention wavefront
struct DattnLds {
    uint16_t qhl[2][8][128];  // the prepared q heads: bf16 hi, lo halves
    float vs[128];            // split 0: this token's V as stored (bf16 values)
    float sp[8];              // split 0: this token's score per head
};

// The 8 q heads' RMSNorm and RoPE in place: the f64 sums of squares in one reduction, after which
// lane l holds head l / 8's scale.
__device__ __forceinline__ void dattn_q_prep(const DattnArgs &a, float (&q0)[8], float (&q1)[8], float qw0,
                                             float qw1, float rc, float rs, uint32_t lane) {
    const bool rope = a.mutant != 1;
    double ss[8];
#pragma unroll
    for (int r = 0; r < 8; ++r) ss[r] = (double)q0[r] * (double)q0[r] + (double)q1[r] * (double)q1[r];
    const float scale_l = rms_scale(head_sums8(ss, lane), 128, a.eps);
#pragma unroll
    for (int r = 0; r < 8; ++r) head_scale_rope(q0[r], q1[r], readlane_f32(scale_l, 8 * r), qw0, qw1, rc, rs, rope);
}

// This token's part of split 0, from the prepared q heads: k's RMSNorm and RoPE, the bf16 K/V
// append to the cache, the token's V row (as stored) and its score per head into L.
__device__ __forceinline__ void dattn_token(const DattnArgs &a, uint32_t h, uint32_t pos, const float (&q0)[8],
                                            const float (&q1)[8], float k0, float k1, float v0, float v1,
                                            float kw0, float kw1, float rc, float rs, DattnLds &L,
                                            uint32_t lane) {
    const bool rope = a.mutant != 1;
    {
        const float kscale = rms_scale(wave_sum_f64((double)k0 * (double)k0 + (double)k1 * (double)k1), 128, a.eps);
        head_scale_rope(k0, k1, kscale, kw0, kw1, rc, rs, rope);
        const uint16_t kb0 = bf16_rne(k0), kb1 = bf16_rne(k1);
        const uint16_t vb0 = bf16_rne(v0), vb1 = bf16_rne(v1);
        if (a.mutant != 3) {
            uint16_t *krow = reinterpret_cast<uint16_t *>(
                a.pool + kv_row_offset(a.g, pos >> 4, a.layer, 0, pos & 15, h));
            krow[lane] = kb0;
            krow[lane + 64] = kb1;
            const uint32_t vpos = a.mutant == 2 ? min(pos + 1, a.max_pos - 1) : pos;
            uint8_t *vplane = a.pool + (uint64_t)(vpos >> 4) * a.g.block_stride +
                              (uint64_t)a.layer * a.g.layer_stride + a.g.plane_stride +
                              (uint64_t)h * kVtHead + (vpos & 15) * 2;
            *reinterpret_cast<uint16_t *>(vplane + lane * 32) = vb0;
            *reinterpret_cast<uint16_t *>(vplane + (lane + 64) * 32) = vb1;
        }
        const float kf0 = bf16_to_f32(kb0), kf1 = bf16_to_f32(kb1);
        L.vs[lane] = bf16_to_f32(vb0);
        L.vs[lane + 64] = bf16_to_f32(vb1);
        float d[8];
#pragma unroll
        for (int r = 0; r < 8; ++r) d[r] = fmaf(q0[r], kf0, q1[r] * kf1);
        const float sp = head_sums8(d, lane) * kInvSqrt128;
        if ((lane & 7) == 0) L.sp[lane >> 3] = sp;
    }
}

// One (split s, kv head h) wavefront, from its kv head's raw q|k|v values (lane l holds dims l
// and l + 64 of the 8 q heads in q0 / q1, of k in k0 / k1 and of v in v0 / v1), the layer's
// q / k norm weights (the same dims), the position's RoPE factors (pair l) and the split's first
// page already loading in T. The 8 heads' RMSNorm scales come from one transposed f64
// reduction; split 0 appends this token's K/V to the cache and scores it; the split's pages
// [p_begin, p_end) run on the matrix cores, each with the next page's loads in flight. When the
// split holds pages or is split 0 (`holds`), its partial goes out with agent-scope stores (written
// through the XCD's L2) and, once they are acknowledged, its flag carries `epoch`. Only this
// wavefront touches L (with TOK_SEPARATE, the token wavefront writes L.vs / L.sp).
// TOK_SEPARATE: split 0's token part (dattn_token) runs on a second wavefront of the workgroup,
// which writes L.vs / L.sp and then meets this one at a barrier just before the token's
// online-softmax step; this wavefront streams its pages meanwhile. The values are the same.
template <bool TOK_SEPARATE = false>
__device__ __forceinline__ void dattn_split(const DattnArgs &a, uint32_t h, uint32_t s, uint32_t pos, bool holds,
                                            uint32_t p_begin, uint32_t p_end, float (&q0)[8], float (&q1)[8],
                                            float k0, float k1, float v0, float v1, float qw0, float qw1,
                                            float kw0, float kw1, float rc, float rs, DattnPage &T,
                                            DattnLds &L, uint32_t epoch, uint32_t lane) {
    const uint32_t g = lane >> 4, n = lane & 15;
    dattn_q_prep(a, q0, q1, qw0, qw1, rc, rs, lane);
#pragma unroll
    for (int r = 0; r < 8; ++r) {
        L.qhl[0][r][lane] = bf16_split_hi(q0[r]);
        L.qhl[1][r][lane] = bf16_split_lo(q0[r]);
        L.qhl[0][r][lane + 64] = bf16_split_hi(q1[r]);
        L.qhl[1][r][lane + 64] = bf16_split_lo(q1[r]);
    }
    if (s == 0 && !TOK_SEPARATE) dattn_token(a, h, pos, q0, q1, k0, k1, v0, v1, kw0, kw1, rc, rs, L, lane);
    // qhl / vs / sp complete: one wavefront wrote them, so its own LDS operations finishing is
    // enough (the page stream stays in flight)
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_wave_barrier();

    // B operand of S^T = K q^T: head column n is head n % 8, its hi (n < 8) or lo (n >= 8) half;
    // k-step ks of lane group g covers dims 32 ks + 8 g .. +8 (16 bytes of LDS)
    bf16x8 qop[4];
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
        qop[ks] = as_bf16x8(*reinterpret_cast<const u32x4 *>(&L.qhl[n >> 3][n & 7][32 * ks + 8 * g]));

    float m_l = -INFINITY, l_l = 0.f;
    f32x4 O[8];
#pragma unroll
    for (int nb = 0; nb < 8; ++nb) O[nb] = f32x4{0.f, 0.f, 0.f, 0.f};
    if (p_begin + 1 == p_end) {
        dattn_page<true>(T, qop, p_begin * kDattnPage, pos, g, n, m_l, l_l, O);
    } else if (p_begin < p_end) {
        // each page computed with the next page's loads in flight
        DattnPage nx;
        dattn_load(a, h, p_begin + 1, lane, nx);
        dattn_page<true>(T, qop, p_begin * kDattnPage, pos, g, n, m_l, l_l, O);
        T = nx;
        uint32_t p = p_begin + 1;
        for (; p + 1 < p_end; ++p) {
            dattn_load(a, h, p + 1, lane, nx);
            dattn_page<false>(T, qop, p * kDattnPage, pos, g, n, m_l, l_l, O);
            T = nx;
        }
        dattn_page<false>(T, qop, p * kDattnPage, pos, g, n, m_l, l_l, O);
    }
    // Output. Row 4 g + i holds the hi half of head 4 g + i for g < 2 and the lo half for g >= 2,
    // so a pair sum over lanes {l, l ^ 32} gives the full value; one swap serves two accumulators:
    // lanes 0-31 get O[nb] (head 4 g + i, dims 16 nb + n), lanes 32-63 get O[nb + 4] (head
    // 4 (g - 2) + i, dims 16 (nb + 4) + n), so every lane stores 16 values.
    const uint32_t hg = g & 1, nb_off = (g >> 1) * 4;
    float ov[4][4];
#pragma unroll
    for (int nb = 0; nb < 4; ++nb)
#pragma unroll
        for (int i = 0; i < 4; ++i) ov[nb][i] = pair_sum<32>(O[nb][i], O[nb + 4][i]);
    if (s == 0) {
        if constexpr (TOK_SEPARATE) __syncthreads();  // the token wavefront's L.vs / L.sp
        // this token: one more online-softmax step with score sp and value vs; lane n of every
        // row holds head n % 8's state, so the head of row i is gathered by readlane
        const float sp = L.sp[n & 7];
        const float m_new = fmaxf(m_l, sp);
        const float aold = expf(m_l - m_new);
        const float pnow = expf(sp - m_new);
        l_l = l_l * aold + pnow;
        m_l = m_new;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float a_lo = readlane_f32(aold, i), a_hi = readlane_f32(aold, 4 + i);
            const float p_lo = readlane_f32(pnow, i), p_hi = readlane_f32(pnow, 4 + i);
            const float ai = hg ? a_hi : a_lo;
            const float pi = hg ? p_hi : p_lo;
#pragma unroll
            for (int nb = 0; nb < 4; ++nb) ov[nb][i] = fmaf(pi, L.vs[16 * (nb + nb_off) + n], ov[nb][i] * ai);
        }
    }
    float *part = a.part + ((size_t)h * 8 * kDattnSplits + s) * kPartStride;
    if (holds) {
        // Dims d and d + 64 sit side by side (o at 4 + 2 (d % 64) + d / 64), so the merge's lane l
        // reads its two dims with one 8-byte load.
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            float *pp = part + (size_t)(4 * hg + i) * kDattnSplits * kPartStride;
#pragma unroll
            for (int nb = 0; nb < 4; ++nb) {
                const uint32_t d = 16 * (nb + nb_off) + n;
                __hip_atomic_store(pp + 4 + 2 * (d & 63) + (d >> 6), ov[nb][i], __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
            }
        }
        if (lane < 8) {  // lane r holds head r's running max and sum
            float *pp = part + (size_t)lane * kDattnSplits * kPartStride;
            __hip_atomic_store(pp, m_l, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(pp + 1, l_l, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        if (lane == 0) __hip_atomic_store(a.flags + h * kDattnSplits + s, epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

// The split-order merge of q head hq once every one of its kv head's `active` splits has flagged:
// out = sum w_i o_i / sum w_i l_i with w_i = exp(m_i - max m); lane l returns dims l (o0) and
// l + 64 (o1), times out_scale / L (lane: this lane's index in the wavefront). Every load goes out at once (one round trip): lane j's (m, l)
// of split j, and per split i the (o[l], o[l + 64]) pair of lane l, in chunks of 16 splits up to
// `active` (indices past it clamp to the last split and get weight 0).
// MAXS: the most splits the caller's plan makes (<= kDattnSplits, a multiple of 16), the partial
// pairs held at once.
template <uint32_t MAXS>
__device__ __forceinline__ void dattn_merge(const float *part, uint32_t hq, uint32_t active, int mutant,
                                            float out_scale, float &o0, float &o1, uint32_t lane) {
    static_assert(MAXS % 16 == 0 && MAXS <= kDattnSplits, "whole chunks of 16 splits");
    const float *base = part + (size_t)hq * kDattnSplits * kPartStride;
    const uint32_t j = min(lane, active - 1);
    const uint64_t mlj = __hip_atomic_load(reinterpret_cast<const uint64_t *>(base + (size_t)j * kPartStride),
                                           __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    uint64_t xo[MAXS];
#pragma unroll
    for (uint32_t c = 0; c < MAXS / 16; ++c) {
        if (c * 16 >= active) break;
#pragma unroll
        for (uint32_t i = 0; i < 16; ++i) {
            const uint32_t si = min(c * 16 + i, active - 1);
            xo[c * 16 + i] = __hip_atomic_load(
                reinterpret_cast<const uint64_t *>(base + (size_t)si * kPartStride + 4 + 2 * lane),
                __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
    const float mj = __uint_as_float((uint32_t)mlj), lj = __uint_as_float((uint32_t)(mlj >> 32));
    const float mv = lane < active ? mj : -INFINITY;
    float M = row16_max(mv);
    M = fmaxf(fmaxf(readlane_f32(M, 0), readlane_f32(M, 16)), fmaxf(readlane_f32(M, 32), readlane_f32(M, 48)));
    const float wj = lane < active ? (mutant == 4 ? 1.f : expf(mj - M)) : 0.f;
    const float Ls = wave_sum(wj * (lane < active ? lj : 0.f));
    float a0 = 0.f, a1 = 0.f;
#pragma unroll
    for (uint32_t c = 0; c < MAXS / 16; ++c) {
        if (c * 16 >= active) break;
#pragma unroll
        for (uint32_t i = 0; i < 16; ++i) {
            // lanes past `active` hold weight 0, so a split past it adds nothing (its o values are
            // the last split's, finite)
            const uint32_t si = c * 16 + i;
            const float wi = readlane_f32(wj, (int)si);
            a0 = fmaf(wi, __uint_as_float((uint32_t)xo[si]), a0);
            a1 = fmaf(wi, __uint_as_float((uint32_t)(xo[si] >> 32)), a1);
        }
    }
    o0 = a0 * (out_scale / Ls);
    o1 = a1 * (out_scale / Ls);
}

}  // namespace omega
