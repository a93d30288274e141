// The decode token's layers as one persistent launch: the decode graph's default form.
//
// Contract: crates/aien-omega-dgraph/src/lib.rs:16-30 — per layer: input norm, q|k|v FP8, decode
// attention, o FP8, residual add, router, gate|up FP8, SwiGLU, down FP8, combine. Every output
// value is computed with the same lane split, reduction order and rounding as the six-launch
// chain of dgraph.hip, so both forms give the same bits (tested).
//
// Why one launch. A kernel node in a hipGraph chain costs about 1.6 us before its first load
// issues, and a launch boundary is also where every weight stream must start from cold, so the
// chain spends most of a layer waiting. Here 256 workgroups of eight wavefronts (one per CU; the
// LDS use admits no second one) stay resident for the whole token and hand each stage's output to
// the next through "words": 8-byte stores of (f32 value | the token's epoch), written through to
// memory with agent-scope stores. A consumer polls the words it needs with agent-scope loads until
// every one carries this token's epoch. A word is its own flag, so no fence and no counter are
// involved and a handoff costs one store-to-load latency (about 1.2 us for 2048 words polled by
// all 256 workgroups). Every wait is bounded in time: one that runs out is counted in errc and sets
// the abort word, which ends every later wait, so a token that cannot complete still returns (and
// is reported as failed). Each buffer of words belongs to one (layer, stage) and is written once
// per token; the epoch changes every token.
//
// Roles of wavefront w of workgroup b in each layer:
//   Q   w < 4: q|k|v rows 5 (4 b + w) .. +5, the input RMSNorm as one scale on the row sums;
//   A   b >= 128, w >= 6: attention item (b - 128) * 2 + w - 6 = split * 4 + kv head (64 splits per
//       kv head), the fused decode attention (dattn.hpp) with its split merge (splits 0..7 merge one
//       q head each);
//   O   w >= 4: o rows 2 (4 b + w - 4) .. +2 plus the residual (rows 8 b .. +8 of the group);
//   R   b < 16: router row 8 b + w (f64-exact logit) and its 16 values of the normed row x';
//   GU  all: the route ranked from the 128 logits (every wavefront ranks, to the same bits), then
//       gate|up rows 3 ((8 b + w) % 256) .. +3 of slot (8 b + w) / 256 and SwiGLU;
//   D   all: down rows 8 b .. +8 of slot w; the 8 slots combined in LDS in slot order + residual.
// Weights that do not depend on the route are loaded into registers a stage or more ahead: the
// next layer's q|k|v rows right after this layer's, the o rows likewise, the router rows with the
// expert streams, the first page of the next layer's attention right after this layer's. Their
// streams therefore overlap the handoffs in front of them; the expert streams (gate|up and down
// together) go out as soon as the route is known.
// Vector-memory loads complete in issue order, so a poll issued behind a prefetch cannot be
// checked before the prefetch lands. Polls are therefore made by wavefronts whose own loads have
// landed: Q wavefronts poll x, x_new (router groups) and x' + logits; wavefronts 0-5 the
// attention row; each D wavefront its slot's activations; each A wavefront its q|k|v.
#include <hip/hip_runtime.h>

#include "dattn.hpp"
#include "kernels.hpp"
#include "route.hpp"
#include "rows.hpp"
#include "runtime.hpp"

namespace omega {

constexpr uint32_t kTokHidden = 2048, kTokInter = 768;
constexpr uint32_t kTokQRows = 5;           // q|k|v rows per Q wavefront
constexpr uint32_t kTokORows = 2;           // o rows per O wavefront
constexpr uint32_t kTokGuRows = 3;          // gate|up row pairs per wavefront
constexpr uint32_t kTokDnRows = 8;          // down rows per workgroup
constexpr uint32_t kTokRouterGroups = 16;   // 16 x 8 wavefronts = 128 router rows
constexpr uint32_t kTokAttnGroup0 = 128;    // wavefronts 6, 7 of groups 128..255: the attention items
constexpr uint32_t kTokSplits = kGraphSplits;  // splits per kv head
constexpr uint32_t kTokAttPoll = 704;       // attention-row words per polling wavefront (0-5)

static_assert(kTokGroups * 4 * kTokQRows == 5120, "Q wavefronts cover q|k|v");
static_assert(kTokGroups * 4 * kTokORows == kTokHidden, "O wavefronts cover o");
static_assert(kTokGroups * 8 * kTokGuRows == kTopK * kTokInter, "every wavefront takes gate|up rows");
static_assert(kTokGroups * kTokDnRows == kTokHidden, "each workgroup takes 8 down rows");
static_assert((kTokGroups - kTokAttnGroup0) * 2 == 4 * kTokSplits && kTokSplits <= kDattnSplits,
              "one attention item per wavefront 6, 7 of the attention groups");
static_assert(5 * kTokAttPoll < 4096 && 4096 - 5 * kTokAttPoll <= kTokAttPoll, "six polling wavefronts");

struct TokLds {
    float x[kTokHidden];    // the layer's input residual
    float nw[kTokHidden];   // input RMSNorm weights
    float att[4096];        // the attention row
    float xn[kTokHidden];   // residual after the attention (router groups)
    float rnw[kTokHidden];  // router norm weights (router groups)
    float xp[kTokHidden];   // x'
    float logit[128];
    float act[kTopK][kTokInter];  // each D wavefront its slot's SwiGLU row
    float xres[kTokDnRows];       // the residual after the attention, this group's down rows
    float red[kTopK][kTokDnRows]; // down rows per slot
    DattnLds at[2];               // the two attention wavefronts
};
static_assert(sizeof(TokLds) <= kTokLds, "the workgroup's LDS");
static_assert(2 * kTokLds > 160 * 1024, "one workgroup per CU");

// ------------------------------------------------------------------ words
__device__ __forceinline__ void put_word(uint64_t *p, float v, uint32_t ep) {
    __hip_atomic_store(p, ((uint64_t)ep << 32) | __float_as_uint(v), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t get_word(const uint64_t *p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ bool word_ok(uint64_t w, uint32_t ep) { return (uint32_t)(w >> 32) == ep; }
__device__ __forceinline__ float word_val(uint64_t w) { return __uint_as_float((uint32_t)w); }

// A bounded wait: call after each unsuccessful poll; true when the wait must end unfinished
// (another wait ran out, or this one did: then it is counted and the abort word set).
struct Waiter {
    unsigned long long t0;
    uint32_t spins;
};
__device__ __forceinline__ Waiter wait_start() { return Waiter{__builtin_amdgcn_s_memrealtime(), 0u}; }
#ifndef TOK_POLL_SLEEP
#define TOK_POLL_SLEEP 1
#endif
__device__ __forceinline__ bool wait_over(Waiter &wt, const PTokenArgs &a, uint32_t lane) {
    __builtin_amdgcn_s_sleep(TOK_POLL_SLEEP);
    // the clock every 16 polls; the abort word (one line every waiting wavefront reads) every 256
    if ((++wt.spins & 15u) != 0) return false;
    if ((wt.spins & 255u) == 0 && __hip_atomic_load(a.abort, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) return true;
    if (__builtin_amdgcn_s_memrealtime() - wt.t0 < a.wait_ticks) return false;
    if (lane == 0) {
        __hip_atomic_fetch_add(a.errc, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(a.abort, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    return true;
}

// The wavefront waits for words src[0 .. n) (n <= 64 J; lane takes words lane + 64 j) and writes
// their values to dst (LDS).
template <int J>
__device__ __forceinline__ void poll_lds(const uint64_t *src, uint32_t n, float *dst, uint32_t ep,
                                         const PTokenArgs &a, uint32_t lane) {
    Waiter wt = wait_start();
    uint64_t w[J];
    while (true) {
#pragma unroll
        for (int j = 0; j < J; ++j) w[j] = get_word(src + min(lane + 64u * j, n - 1));
        bool ok = true;
#pragma unroll
        for (int j = 0; j < J; ++j) ok = ok && word_ok(w[j], ep);
        if (__all(ok) || wait_over(wt, a, lane)) break;
    }
#pragma unroll
    for (int j = 0; j < J; ++j)
        if (lane + 64u * j < n) dst[lane + 64 * j] = word_val(w[j]);
}
// the same for two ranges in one round trip
template <int J1, int J2>
__device__ __forceinline__ void poll_lds2(const uint64_t *s1, uint32_t n1, float *d1, const uint64_t *s2,
                                          uint32_t n2, float *d2, uint32_t ep, const PTokenArgs &a, uint32_t lane) {
    Waiter wt = wait_start();
    uint64_t w1[J1], w2[J2];
    while (true) {
#pragma unroll
        for (int j = 0; j < J1; ++j) w1[j] = get_word(s1 + min(lane + 64u * j, n1 - 1));
#pragma unroll
        for (int j = 0; j < J2; ++j) w2[j] = get_word(s2 + min(lane + 64u * j, n2 - 1));
        bool ok = true;
#pragma unroll
        for (int j = 0; j < J1; ++j) ok = ok && word_ok(w1[j], ep);
#pragma unroll
        for (int j = 0; j < J2; ++j) ok = ok && word_ok(w2[j], ep);
        if (__all(ok) || wait_over(wt, a, lane)) break;
    }
#pragma unroll
    for (int j = 0; j < J1; ++j)
        if (lane + 64u * j < n1) d1[lane + 64 * j] = word_val(w1[j]);
#pragma unroll
    for (int j = 0; j < J2; ++j)
        if (lane + 64u * j < n2) d2[lane + 64 * j] = word_val(w2[j]);
}

// A value the compiler must treat as new on every use site: per-lane values derived from it stay
// inside the layer loop instead of being hoisted out of it and held (spilled) across the loop.
__device__ __forceinline__ uint32_t opaque(uint32_t v) {
    asm volatile("" : "+v"(v));
    return v;
}
__device__ __forceinline__ uint32_t opaque_s(uint32_t v) {  // a wave-uniform value, kept scalar
    asm volatile("" : "+s"(v));
    return v;
}

// A cheap readiness test before a vector is read: the wavefront polls one "sentinel" word per
// producer (a word the producer stores last, or at its end) until every one carries ep; words
// base[offset + stride * i], i < n <= 64 Q. A sentinel is only a hint (the producers' stores are
// not ordered among themselves): the full read that follows checks every word's epoch again and
// polls on. Waiting on the sentinels keeps a long wait from re-reading whole vectors: the fabric
// traffic of a round drops from the vector's bytes to 8 bytes per producer.
template <int Q>
__device__ __forceinline__ void wait_sentinels(const uint64_t *base, uint32_t offset, uint32_t stride, uint32_t n,
                                               uint32_t ep, const PTokenArgs &a, uint32_t lane) {
    Waiter wt = wait_start();
    while (true) {
        bool ok = true;
#pragma unroll
        for (int q = 0; q < Q; ++q) {
            const uint32_t i = min(lane + 64u * q, n - 1);
            ok = ok && word_ok(get_word(base + offset + (size_t)stride * i), ep);
        }
        if (__all(ok) || wait_over(wt, a, lane)) break;
    }
}

// one layer's descriptor through scalar loads
__device__ __forceinline__ PLayer load_layer(const PLayer *p) {
    typedef const __attribute__((address_space(4))) uint64_t cu64;
    static_assert(sizeof(PLayer) % 8 == 0, "pointer words");
    struct Words {
        uint64_t w[sizeof(PLayer) / 8];
    } v;
    const cu64 *q = (const cu64 *)(uintptr_t)p;
#pragma unroll
    for (uint32_t i = 0; i < sizeof(PLayer) / 8; ++i) v.w[i] = q[i];
    return __builtin_bit_cast(PLayer, v);
}

using SQ = Fp8Slab<kTokHidden, kTokQRows>;   // q|k|v: 10 chunks, 2 phases, rows straddle 128-blocks
using SO = Fp8Slab<4096, kTokORows>;         // o: 8 chunks, 4 phases
using SG = Fp8Slab<kTokHidden, kTokGuRows>;  // gate or up: 6 chunks, 2 phases, rows straddle blocks
using SD = Fp8Slab<kTokInter, kTokDnRows>;   // down: 6 chunks, 3 phases
using SR = Bf16Slab<kTokHidden, 1>;          // router row: 4 chunks, 4 phases of 8
static_assert(SQ::CH == 10 && SO::CH == 8 && SG::CH == 6 && SD::CH == 6 && SR::CH == 4, "chunk counts");
static_assert(!SQ::kOneBlock && SO::kOneBlock && !SG::kOneBlock && SD::kOneBlock, "scale blocks");
constexpr int kPre = 10;  // prefetch chunks: q|k|v (10) or o (8)

__global__ __launch_bounds__(512) void k_token(const PTokenArgs a) {
    extern __shared__ __align__(16) unsigned char tok_lds[];
    TokLds &S = *reinterpret_cast<TokLds *>(tok_lds);
    const uint32_t lane0 = lane_id();
    const uint32_t wid = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t b = blockIdx.x;
    const uint32_t pos = *as_const_u32(a.io), tokid = *as_const_u32(a.io + 1), ep = *as_const_u32(a.io + 2);
    const bool stamp = a.stamps && b == 0 && threadIdx.x == 0;
    if (stamp) a.stamps[0] = __builtin_amdgcn_s_memrealtime();

    const bool isq = wid < 4, iso = wid >= 4, isr = b < kTokRouterGroups;
    const uint32_t qrow0 = (b * 4 + (wid & 3)) * kTokQRows;
    const uint32_t orow0 = (b * 4 + (wid & 3)) * kTokORows;
    const bool isa = b >= kTokAttnGroup0 && wid >= 6;
    const uint32_t item = isa ? (b - kTokAttnGroup0) * 2 + (wid - 6) : 0;
    const uint32_t ah = item & 3, asp = item >> 2;  // kv head, split
    const uint32_t pages = (pos + kDattnPage - 1) / kDattnPage;
    uint32_t active, pps;
    attn_split_plan(pages, kTokSplits, a.tiles_per_split, active, pps);
    const bool aholds = asp < active;
    // splits past the plan stay only to merge (0..7)
    const bool alive = isa && (aholds || asp < 8);
    const uint32_t p_begin = aholds ? asp * pps : 0, p_end = aholds ? min(pages, p_begin + pps) : 0;
    DattnLds &AL = S.at[wid & 1];
    DattnArgs da;
    da.pool = a.pool;
    da.g = a.g;
    da.max_pos = a.max_pos;
    da.eps = a.eps;
    da.part = a.part;
    da.mutant = a.dattn_mutant;

    // ---- prefetch of layer 0's route-independent weights
    u32x4 pre[kPre];  // Q: q|k|v rows; O: o rows
    float psc[4];     // their block scales (Q: [2][2]; O: [4])
    // the attention item's first page; in the router groups (which hold no attention item) T.k
    // holds the router row instead
    DattnPage T;
    static_assert(sizeof(T.k) / sizeof(T.k[0]) == SR::CH, "a router row fits the page's K registers");
    float qw0 = 0.f, qw1 = 0.f, kw0 = 0.f, kw1 = 0.f, rc = 0.f, rs = 0.f;
    auto prefetch_q = [&](const PLayer &L, uint32_t lane) {
        float s0[2], s1[2];
        SQ::load_scales(L.qkv_s + (size_t)(qrow0 >> 7) * (kTokHidden >> 7), lane, 1.0f, 0, s0);
        SQ::load_scales(L.qkv_s + (size_t)((qrow0 + kTokQRows - 1) >> 7) * (kTokHidden >> 7), lane, 1.0f, 0, s1);
        psc[0] = s0[0];
        psc[1] = s0[1];
        psc[2] = s1[0];
        psc[3] = s1[1];
        SQ::load_v(pre, L.qkv_w + (size_t)qrow0 * kTokHidden, lane);
    };
    auto prefetch_o = [&](const PLayer &L, uint32_t lane) {
        float s0[4];
        SO::load_scales(L.o_s + (size_t)(orow0 >> 7) * (4096 >> 7), lane, 1.0f, 0, s0);
#pragma unroll
        for (int i = 0; i < 4; ++i) psc[i] = s0[i];
        SO::load_v(pre, L.o_w + (size_t)orow0 * 4096, lane);
    };
    auto prefetch_a = [&](const PLayer &L, uint32_t layer, uint32_t lane) {
        qw0 = *as_global_f32(L.q_norm + lane);
        qw1 = *as_global_f32(L.q_norm + 64 + lane);
        kw0 = *as_global_f32(L.k_norm + lane);
        kw1 = *as_global_f32(L.k_norm + 64 + lane);
        da.layer = layer;
        dattn_load(da, ah, p_begin < p_end ? p_begin : 0, lane, T);
    };
    {
        const PLayer L0 = load_layer(a.layers);
        if (isq) prefetch_q(L0, lane0);
        else prefetch_o(L0, lane0);
        if (isr) SR::load_v(T.k, L0.rgate + (size_t)(b * 8 + wid) * kTokHidden, lane0);
        if (alive) {
            rc = *as_global_f32(a.rope_cos + (size_t)pos * 64 + lane0);
            rs = *as_global_f32(a.rope_sin + (size_t)pos * 64 + lane0);
            prefetch_a(L0, 0, lane0);
        }
    }

    for (uint32_t l = 0; l < a.nlayers; ++l) {
        const uint32_t lane = opaque(lane0);
        const uint32_t tid = opaque(threadIdx.x);
        const PLayer L = load_layer(a.layers + l);
        const bool last = l + 1 == a.nlayers;
        // ================= B0: the layer's input row and its norm weights in LDS
        {
            const f32x4 nwv = *as_global_f32x4(L.in_norm + 4 * tid);
            if (l == 0) {
                if (a.embed) {
                    const uint32_t tok = tokid % a.embed_rows;
                    const u32x2 e = *as_global_u32x2(a.embed + (size_t)tok * kTokHidden + 4 * tid);
                    reinterpret_cast<f32x4 *>(S.x)[tid] =
                        f32x4{bf16_lo(e.x), bf16_hi(e.x), bf16_lo(e.y), bf16_hi(e.y)};
                } else {
                    reinterpret_cast<f32x4 *>(S.x)[tid] = *as_global_f32x4(a.x + 4 * tid);
                }
            } else if (isq) {
                // nothing else streams at the layer boundary: the row is polled directly
                poll_lds<8>(a.w_x + (size_t)l * kTokHidden + wid * 512, 512, S.x + wid * 512, ep, a, lane);
            }
            reinterpret_cast<f32x4 *>(S.nw)[tid] = nwv;
        }
        __syncthreads();
        if (stamp) a.stamps[1 + l * kTokStampsPerLayer] = __builtin_amdgcn_s_memrealtime();

        // ================= Q, A, and the attention row's poll
        uint64_t *const watt = a.w_att + (size_t)l * 4096;
        if (isq) {
            float xr[SQ::P][16], nw[SQ::P][16];
            SQ::load_x_lds(S.x, lane, xr);
            SQ::load_x_lds(S.nw, lane, nw);
            const double ss = phases_sumsq(xr);
#pragma unroll
            for (int ph = 0; ph < SQ::P; ++ph)
#pragma unroll
                for (int i = 0; i < 16; ++i) xr[ph][i] = xr[ph][i] * nw[ph][i];
            float scale = 1.0f;
            scale *= rms_scale(ss, kTokHidden, a.eps);
            const float sc[2][SQ::P] = {{psc[0], psc[1]}, {psc[2], psc[3]}};
            float acc[kTokQRows];
#pragma unroll
            for (uint32_t j = 0; j < kTokQRows; ++j) acc[j] = 0.f;
            SQ::dot2_v(pre, xr, sc, qrow0, acc);
            const float v = reduce_rows(acc, lane) * scale;
            if (lane < kTokQRows) put_word(a.w_qkv + (size_t)l * 5120 + qrow0 + lane, v, ep);
            if (!last) prefetch_q(load_layer(a.layers + l + 1), lane);
        }
        if (alive) {
            // this kv head's q heads, k and v: lane l takes dims l and l + 64
            const uint64_t *src = a.w_qkv + (size_t)l * 5120;
            float q0[8], q1[8], k0, k1, v0, v1;
            {
                Waiter wt = wait_start();
                uint64_t wq0[8], wq1[8], wk0, wk1, wv0, wv1;
                while (true) {
#pragma unroll
                    for (int r = 0; r < 8; ++r) {
                        wq0[r] = get_word(src + ah * 1024 + r * 128 + lane);
                        wq1[r] = get_word(src + ah * 1024 + r * 128 + 64 + lane);
                    }
                    wk0 = get_word(src + 4096 + ah * 128 + lane);
                    wk1 = get_word(src + 4096 + ah * 128 + 64 + lane);
                    wv0 = get_word(src + 4608 + ah * 128 + lane);
                    wv1 = get_word(src + 4608 + ah * 128 + 64 + lane);
                    bool ok = word_ok(wk0, ep) && word_ok(wk1, ep) && word_ok(wv0, ep) && word_ok(wv1, ep);
#pragma unroll
                    for (int r = 0; r < 8; ++r) ok = ok && word_ok(wq0[r], ep) && word_ok(wq1[r], ep);
                    if (__all(ok) || wait_over(wt, a, lane)) break;
                }
#pragma unroll
                for (int r = 0; r < 8; ++r) {
                    q0[r] = word_val(wq0[r]);
                    q1[r] = word_val(wq1[r]);
                }
                k0 = word_val(wk0);
                k1 = word_val(wk1);
                v0 = word_val(wv0);
                v1 = word_val(wv1);
            }
            da.layer = l;
            da.flags = a.aflags + (size_t)l * 4 * kDattnSplits;
            dattn_split(da, ah, asp, pos, aholds, p_begin, p_end, q0, q1, k0, k1, v0, v1, qw0, qw1, kw0, kw1, rc,
                        rs, T, AL, ep, lane);
            if (asp < 8) {
                // merge q head 8 h + s once every split of the kv head has flagged this token
                const uint32_t act = opaque_s(active);
                const uint32_t *fl = da.flags + ah * kDattnSplits;
                Waiter wt = wait_start();
                while (true) {
                    const uint32_t f = lane < act
                                           ? __hip_atomic_load(fl + lane, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                                           : ep;
                    if (__all(f == ep) || wait_over(wt, a, lane)) break;
                }
                const uint32_t hq = ah * 8 + asp;
                float o0, o1;
                dattn_merge<kTokSplits>(a.part, hq, act, a.dattn_mutant, a.attn_out_scale, o0, o1, lane);
                put_word(watt + hq * 128 + lane, o0, ep);
                put_word(watt + hq * 128 + 64 + lane, o1, ep);
            }
            if (!last) prefetch_a(load_layer(a.layers + l + 1), l + 1, lane);
        }
        // the 32 mergers: word 128 hq + 127 (their last store) is a sentinel; wavefront 5 waits
        // on them (its own loads have landed), then wavefronts 0-5 read the row
        if (wid == 5) wait_sentinels<1>(watt, 127, 128, 32, ep, a, lane);
        __syncthreads();
        if (wid < 6) {
            const uint32_t o = wid * kTokAttPoll;
            poll_lds<kTokAttPoll / 64>(watt + o, wid < 5 ? kTokAttPoll : 4096 - 5 * kTokAttPoll, S.att + o, ep, a, lane);
        }
        __syncthreads();
        if (stamp) a.stamps[2 + l * kTokStampsPerLayer] = __builtin_amdgcn_s_memrealtime();

        // ================= O, and the residual's poll by the router groups
        if (iso) {
            float xr[SO::P][16];
            SO::load_x_lds(S.att, lane, xr);
            const float sc[SO::P] = {psc[0], psc[1], psc[2], psc[3]};
            float acc[kTokORows] = {0.f, 0.f};
            SO::dot_v(pre, xr, sc, acc, lane);
            const float v = reduce_rows(acc, lane) * 1.0f;
            const float y = S.x[orow0 + min(lane, kTokORows - 1)] + v;
            if (lane < kTokORows) {
                put_word(a.w_xn + (size_t)l * kTokHidden + orow0 + lane, y, ep);
                S.xres[(wid - 4) * kTokORows + lane] = y;
            }
            if (!last) prefetch_o(load_layer(a.layers + l + 1), lane);
        }
        if (isr) {
            // every wavefront of the router groups polls 256 words (its O prefetch is in flight,
            // but fewer words per wavefront measured faster than four wavefronts with 512)
            const f32x4 rn0 = *as_global_f32x4(L.rnorm + wid * 256 + 4 * lane);
            poll_lds<4>(a.w_xn + (size_t)l * kTokHidden + wid * 256, 256, S.xn + wid * 256, ep, a, lane);
            reinterpret_cast<f32x4 *>(S.rnw + wid * 256)[lane] = rn0;
        }
        __syncthreads();
        if (stamp) a.stamps[3 + l * kTokStampsPerLayer] = __builtin_amdgcn_s_memrealtime();

        // ================= R, and the poll of x' and the logits
        uint64_t *const wlog = a.w_log + (size_t)l * 128;
        uint64_t *const wxp = a.w_xp + (size_t)l * kTokHidden;
        if (isr) {
            const uint32_t row = b * 8 + wid;
            float xr[SR::P][8], nw[SR::P][8];
#pragma unroll
            for (int ph = 0; ph < SR::P; ++ph)
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    xr[ph][i] = S.xn[SR::col(ph, lane) + i];
                    nw[ph][i] = S.rnw[SR::col(ph, lane) + i];
                }
            const float scale = rms_scale(phases_sumsq(xr), kTokHidden, a.eps);
#pragma unroll
            for (int ph = 0; ph < SR::P; ++ph)
#pragma unroll
                for (int i = 0; i < 8; ++i) xr[ph][i] = xr[ph][i] * scale * (a.router_mutant == 1 ? 1.0f : nw[ph][i]);
            double acc = 0.0;
#pragma unroll
            for (int c = 0; c < SR::CH; ++c) {
                const u32x4 w = T.k[c];
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    acc += (double)bf16_lo(w[q]) * (double)xr[c][2 * q];
                    acc += (double)bf16_hi(w[q]) * (double)xr[c][2 * q + 1];
                }
            }
            acc = wave_sum_f64(acc);
            const float logit = (float)acc;
            // this row's 16 values of x': phase row / 32, lanes 2 (row % 32) and 2 (row % 32) + 1;
            // then the logit, the row's sentinel
            const uint32_t xl = 2 * (row & 31);
            if (lane == xl || lane == xl + 1) {
#pragma unroll
                for (int ph = 0; ph < SR::P; ++ph) {
                    if ((row >> 5) != (uint32_t)ph) continue;
#pragma unroll
                    for (int i = 0; i < 8; ++i) put_word(wxp + SR::col(ph, lane) + i, xr[ph][i] * 1.0f, ep);
                }
            }
            if (lane == 0) {
                put_word(wlog + row, logit, ep);
                a.r_logits[row] = logit;
            }
            if (b == 0 && wid == 0) {
#pragma unroll
                for (int ph = 0; ph < SR::P; ++ph) {
                    float *o = a.r_xout + SR::col(ph, lane);
#pragma unroll
                    for (int i = 0; i < 8; ++i) o[i] = xr[ph][i] * 1.0f;
                }
            }
        }
        // ================= GU and D
        // Wavefront 0 waits for the 128 logits (one wavefront polling keeps the wait's traffic
        // low: 2048 wavefronts polling the same kilobyte measured 2.5x slower), then every
        // wavefront reads them itself and ranks them; x' is read once the expert streams are issued
        // (it is needed only when their weights arrive).
        float lg[2];
        {
            Waiter wt = wait_start();
            uint64_t w0, w1;
            if (wid == 0) wait_sentinels<2>(wlog, 0, 1, 128, ep, a, lane);
            __syncthreads();
            while (true) {
                w0 = get_word(wlog + lane);
                w1 = get_word(wlog + 64 + lane);
                if (__all(word_ok(w0, ep) && word_ok(w1, ep)) || wait_over(wt, a, lane)) break;
            }
            lg[0] = word_val(w0);
            lg[1] = word_val(w1);
        }
        // every wavefront writes the same 128 values: its own reads below see its own writes
        float *const lgs = S.logit;
        lgs[lane] = lg[0];
        lgs[64 + lane] = lg[1];
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        __builtin_amdgcn_wave_barrier();
        Route r;
        if (L.forced && *as_global_u32(L.forced) != OMEGA_GPU_DGRAPH_RANK) {
            route_forced_r([&](uint32_t id) { return lgs[id]; }, L.forced, r);
        } else {
            uint32_t k[2] = {ord_key(lg[0]), ord_key(lg[1])};
            route_topk_keys_r<2>(k, [&](uint32_t id) { return lgs[id]; }, 0, a.norm_topk, a.router_mutant, r);
        }
        // the route is the same in every lane: keep it in scalar registers
#pragma unroll
        for (int s = 0; s < kTopK; ++s) {
            r.id[s] = __builtin_amdgcn_readfirstlane(r.id[s]);
            r.w[s] = __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(r.w[s])));
        }
        const uint32_t gw = b * 8 + wid;
        const uint32_t gslot = gw >> 8, j0 = (gw & 255) * kTokGuRows;
        uint32_t eg = r.id[0], ed = r.id[0];
#pragma unroll
        for (uint32_t s = 1; s < (uint32_t)kTopK; ++s) {
            if (gslot == s) eg = r.id[s];
            if (wid == s) ed = r.id[s];
        }
        eg = __builtin_amdgcn_readfirstlane(eg);
        ed = __builtin_amdgcn_readfirstlane(ed);
        const uint8_t *we = L.gu_w + (size_t)eg * 2 * kTokInter * kTokHidden;
        const float *se = L.gu_s + (size_t)eg * (2 * kTokInter / 128) * (kTokHidden / 128);
        // block scales ahead of the weight streams: waits complete in issue order
        float scg[2][SG::P], scu[2][SG::P], scd[SD::P];
        SG::load_scales(se + (size_t)(j0 >> 7) * (kTokHidden / 128), lane, 1.0f, 0, scg[0]);
        SG::load_scales(se + (size_t)((j0 + kTokGuRows - 1) >> 7) * (kTokHidden / 128), lane, 1.0f, 0, scg[1]);
        SG::load_scales(se + (size_t)((kTokInter + j0) >> 7) * (kTokHidden / 128), lane, 1.0f, 0, scu[0]);
        SG::load_scales(se + (size_t)((kTokInter + j0 + kTokGuRows - 1) >> 7) * (kTokHidden / 128), lane, 1.0f, 0,
                        scu[1]);
        const uint32_t drow0 = b * kTokDnRows;
        SD::load_scales(L.dn_s + ((size_t)ed * (kTokHidden / 128) + (drow0 >> 7)) * (kTokInter / 128), lane, 1.0f, 0,
                        scd);
        u32x4 gate[SG::CH], up[SG::CH], dn[SD::CH];
        SG::load_v(gate, we + (size_t)j0 * kTokHidden, lane);
        SG::load_v(up, we + (size_t)(kTokInter + j0) * kTokHidden, lane);
        SD::load_v(dn, L.dn_w + ((size_t)ed * kTokHidden + drow0) * kTokInter, lane);
        if (isr && !last) SR::load_v(T.k, load_layer(a.layers + l + 1).rgate + (size_t)(b * 8 + wid) * kTokHidden, lane);
        __builtin_amdgcn_sched_barrier(0);
        if (isq) poll_lds<8>(wxp + wid * 512, 512, S.xp + wid * 512, ep, a, lane);
        __syncthreads();
        if (stamp) a.stamps[4 + l * kTokStampsPerLayer] = __builtin_amdgcn_s_memrealtime();
        {
            float ag[kTokGuRows], au[kTokGuRows];
#pragma unroll
            for (uint32_t j = 0; j < kTokGuRows; ++j) ag[j] = au[j] = 0.f;
            SG::dot2_lds(gate, S.xp, scg, j0, ag, lane);
            SG::dot2_lds(up, S.xp, scu, j0, au, lane);
            float gv = reduce_rows(ag, lane);
            float uv = reduce_rows(au, lane);
            if (a.graph_mutant == 1) {
                const float t = gv;
                gv = uv;
                uv = t;
            }
            if (lane < kTokGuRows)
                put_word(a.w_act + ((size_t)l * kTopK + gslot) * kTokInter + j0 + lane, gv / (1.0f + expf(-gv)) * uv,
                         ep);
        }
        // the 256 groups' gate|up: the last activation of each (word 24 b + 23 of the layer's 6144:
        // slot b / 32, pair 3 ((8 b + 7) % 256) + 2) is a sentinel
        if (wid == 0) wait_sentinels<4>(a.w_act + (size_t)l * kTopK * kTokInter, 23, 24, kTokGroups, ep, a, lane);
        __syncthreads();
        {
            poll_lds<kTokInter / 64>(a.w_act + ((size_t)l * kTopK + wid) * kTokInter, kTokInter, S.act[wid], ep, a, lane);
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // this wavefront's row is in LDS
            __builtin_amdgcn_wave_barrier();
            float acc[kTokDnRows];
#pragma unroll
            for (uint32_t j = 0; j < kTokDnRows; ++j) acc[j] = 0.f;
            SD::dot_lds(dn, S.act[wid], scd, acc, lane);
            const float v = reduce_rows(acc, lane);
            if (lane < kTokDnRows) S.red[wid][lane] = v;
        }
        __syncthreads();
        if (stamp) a.stamps[5 + l * kTokStampsPerLayer] = __builtin_amdgcn_s_memrealtime();
        if (wid == 0 && lane < kTokDnRows) {
            float moe = 0.f;
#pragma unroll
            for (int s = 0; s < kTopK; ++s) {
                const float wgt = (a.graph_mutant == 2 && s == 7) ? 0.f : r.w[s];
                moe += wgt * S.red[s][lane];
            }
            const float xo = S.xres[lane] + moe;
            put_word(a.w_x + (size_t)(l + 1) * kTokHidden + drow0 + lane, xo, ep);
            if (last) a.x[drow0 + lane] = xo;
        }
        // workgroup 0's wavefront 1 publishes the route (the router's device state and the
        // per-layer log), now that no weight stream of its own is in flight
        if (b == 0 && wid == 1 && lane < (uint32_t)kTopK) {
            uint32_t id = r.id[0];
            float wt = r.w[0];
#pragma unroll
            for (uint32_t s = 1; s < (uint32_t)kTopK; ++s) {
                if (lane == s) {
                    id = r.id[s];
                    wt = r.w[s];
                }
            }
            a.r_ids[lane] = id;
            a.r_weights[lane] = wt;
            L.log_ids[lane] = id;
            L.log_w[lane] = wt;
            const uint64_t gu0 = L.dir_gu[2 * id], gu1 = L.dir_gu[2 * id + 1];
            const uint64_t dn0 = L.dir_dn[2 * id], dn1 = L.dir_dn[2 * id + 1];
            a.r_tab_gu[2 * lane] = gu0;
            a.r_tab_gu[2 * lane + 1] = gu1;
            a.r_tab_dn[2 * lane] = dn0;
            a.r_tab_dn[2 * lane + 1] = dn1;
        }
    }
}

hipError_t launch_token(const PTokenArgs &a, hipStream_t st) {
    OMEGA_LAUNCH(k_token, dim3(kTokGroups), dim3(kTokThreads), kTokLds, st, a);
    return hipGetLastError();
}

bool token_fits(int device) {
    static int checked = -1;
    if (checked >= 0) return checked == 1;
    bool ok = hipFuncSetAttribute((const void *)k_token, hipFuncAttributeMaxDynamicSharedMemorySize, kTokLds) ==
              hipSuccess;
    hipDeviceProp_t p{};
    ok = ok && hipGetDeviceProperties(&p, device) == hipSuccess && p.multiProcessorCount >= (int)kTokGroups;
    int per_cu = 0;
    ok = ok && hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, (const void *)k_token, kTokThreads, kTokLds) ==
                   hipSuccess &&
         per_cu >= 1;
    checked = ok ? 1 : 0;
    return ok;
}

}  // namespace omega
