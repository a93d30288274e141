// Top-k ranking of router logits on one wavefront, shared by the standalone router and the
// decode graph's gate|up prologue.
//
// Host oracle: FakeRouter::route (crates/aien-inference-abi/src/qwen3_moe_omega.rs:1943-1998)
// and MoeBatchPlan::from_logits (moe_plan.rs:86-171): rank by total order descending, ties to
// the lower id; weight = exp(l - max) / sum over the selected of exp(l - max) (norm_topk), or
// over every expert; the optional shared expert takes the last slot with sigmoid(logit).
//
// Each candidate becomes its 32-bit total-order key (unsigned order = the float total order).
// A round takes the wavefront maximum of the keys (DPP inside 16-lane rows, then two row swaps,
// all on the VALU) and the lowest expert id holding it (a ballot of the lanes equal to the
// maximum): exactly the order "larger logit first, then the lower id". The pick's key is then
// cleared to 0, below every real key, and the 8 rounds stay about 20 instructions each; every
// lane ends with the same result.
#pragma once

#include "device.hpp"

namespace omega {

constexpr int kTopK = 8;

struct Route {
    uint32_t id[kTopK + 1];
    float w[kTopK + 1];
};

__device__ __forceinline__ int32_t total_key(float f) {
    const int32_t b = __float_as_int(f);
    return b < 0 ? (b ^ 0x7fffffff) : b;
}
__device__ __forceinline__ float key_value(int32_t k) {
    return __int_as_float(k < 0 ? (k ^ 0x7fffffff) : k);
}
__device__ __forceinline__ uint32_t ord_key(float v) { return (uint32_t)total_key(v) ^ 0x80000000u; }
template <int W>
__device__ __forceinline__ uint32_t xor_max_u32(uint32_t v) {
    uint32_t r0, r1;
    swapw<W>(v, v, r0, r1);
    return r0 > r1 ? r0 : r1;
}
// the maximum over the wavefront, in every lane
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
    v = max(v, (uint32_t)dpp_i32<DPP_XOR1>((int)v));
    v = max(v, (uint32_t)dpp_i32<DPP_XOR2>((int)v));
    v = max(v, (uint32_t)dpp_i32<DPP_HALF_MIRROR>((int)v));
    v = max(v, (uint32_t)dpp_i32<DPP_MIRROR>((int)v));
    v = xor_max_u32<16>(v);
    return xor_max_u32<32>(v);
}

// the ranking keys of Q * 64 logits: lane l holds experts l + 64 q
template <int Q>
__device__ __forceinline__ void route_keys(const float *logits, uint32_t (&k)[Q]) {
    const uint32_t lane = lane_id();
#pragma unroll
    for (int q = 0; q < Q; ++q) k[q] = ord_key(*as_global_f32(logits + lane + 64 * q));
}

// logits: Q * 64 expert values (+1 shared), read through `logit(id)` (global memory or an LDS
// copy), their keys already loaded (the keys are consumed).
// mutant 2: the mask after a pick hits id ^ 1; mutant 4: weights not normalised.
// The picks of slots 0 .. rounds - 1 (ids and logits; rounds uniform, 1..kTopK): a slot's pick
// depends on the earlier rounds only. Returns the last pick's id.
template <int Q>
__device__ __forceinline__ uint32_t route_rounds(uint32_t (&k)[Q], uint32_t rounds, int mutant, Route &r,
                                                 float (&v)[kTopK]) {
    const uint32_t lane = lane_id();
    uint32_t last = 0;
#pragma unroll
    for (int s = 0; s < kTopK; ++s) {
        if ((uint32_t)s >= rounds) break;
        uint32_t m = k[0];
#pragma unroll
        for (int q = 1; q < Q; ++q) m = max(m, k[q]);
        m = wave_max_u32(m);
        // the lowest id whose key is the maximum: quarter q holds ids 64 q .. 64 q + 63
        uint32_t id = 0xffffffffu;
#pragma unroll
        for (int q = Q - 1; q >= 0; --q) {
            const uint64_t b = __ballot(k[q] == m);
            if (b) id = 64 * q + (uint32_t)(__ffsll((long long)b) - 1);
        }
        r.id[s] = id;
        last = id;
        v[s] = key_value((int32_t)(m ^ 0x80000000u));
        const uint32_t mask_id = mutant == 2 ? (id ^ 1u) : id;
#pragma unroll
        for (int q = 0; q < Q; ++q)
            if (lane + 64 * q == mask_id) k[q] = 0;
    }
    return last;
}

template <int Q, typename Logit>
__device__ __forceinline__ void route_topk_keys_r(uint32_t (&k)[Q], Logit logit, uint32_t shared,
                                                  int norm_topk, int mutant, Route &r) {
    constexpr uint32_t experts = 64 * Q;
    float v[kTopK];
    route_rounds<Q>(k, kTopK, mutant, r, v);
    const float mx = v[0];
    float p[kTopK];
    float sum = 0.f;
#pragma unroll
    for (int s = 0; s < kTopK; ++s) {
        p[s] = expf(v[s] - mx);
        sum += p[s];
    }
    if (!norm_topk) {
        sum = 0.f;
        for (uint32_t id = 0; id < experts; ++id) sum += expf(logit(id) - mx);
    }
#pragma unroll
    for (int s = 0; s < kTopK; ++s) r.w[s] = mutant == 4 ? p[s] : p[s] / sum;
    if (shared) {
        r.id[kTopK] = experts;
        r.w[kTopK] = 1.0f / (1.0f + expf(-logit(experts)));
    }
}
template <int Q>
__device__ __forceinline__ void route_topk_keys(uint32_t (&k)[Q], const float *logits, uint32_t shared,
                                                int norm_topk, int mutant, Route &r) {
    route_topk_keys_r<Q>(k, [&](uint32_t id) { return *as_global_f32(logits + id); }, shared, norm_topk,
                         mutant, r);
}

// Teacher forcing for parity tests: the 8 expert ids come from `forced` (slot order), the weights
// are the softmax of this launch's own logits over that set (exp(l - max) / sum, as the ranking
// computes them for its own set). Every lane ends with the same result.
template <typename Logit>
__device__ __forceinline__ void route_forced_r(Logit logit, const uint32_t *forced, Route &r) {
    float v[kTopK];
#pragma unroll
    for (int s = 0; s < kTopK; ++s) {
        r.id[s] = *as_global_u32(forced + s);
        v[s] = logit(r.id[s]);
    }
    float mx = v[0];
#pragma unroll
    for (int s = 1; s < kTopK; ++s) mx = fmaxf(mx, v[s]);
    float p[kTopK], sum = 0.f;
#pragma unroll
    for (int s = 0; s < kTopK; ++s) {
        p[s] = expf(v[s] - mx);
        sum += p[s];
    }
#pragma unroll
    for (int s = 0; s < kTopK; ++s) r.w[s] = p[s] / sum;
}
__device__ __forceinline__ void route_forced(const float *logits, const uint32_t *forced, Route &r) {
    route_forced_r([&](uint32_t id) { return *as_global_f32(logits + id); }, forced, r);
}

// the id of slot rounds - 1 alone (rounds uniform, 1..kTopK), no weights
template <int Q>
__device__ __forceinline__ uint32_t route_slot_id(const float *logits, uint32_t rounds, int mutant) {
    uint32_t k[Q];
    float v[kTopK];
    Route r;
    route_keys<Q>(logits, k);
    return route_rounds<Q>(k, rounds, mutant, r, v);
}

template <int Q>
__device__ __forceinline__ void route_topk(const float *logits, uint32_t shared, int norm_topk,
                                           int mutant, Route &r) {
    uint32_t k[Q];
    route_keys<Q>(logits, k);
    route_topk_keys<Q>(k, logits, shared, norm_topk, mutant, r);
}

}  // namespace omega
