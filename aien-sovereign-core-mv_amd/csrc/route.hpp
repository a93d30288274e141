// Top-k ranking of router logits on one wavefront, shared by the standalone router and the
// decode graph's gate|up prologue.
//
// Host oracle: FakeRouter::route (crates/aien-inference-abi/src/qwen3_moe_omega.rs:1943-1998)
// and MoeBatchPlan::from_logits (moe_plan.rs:86-171): rank by total order descending, ties to
// the lower id; weight = exp(l - max) / sum over the selected of exp(l - max) (norm_topk), or
// over every expert; the optional shared expert takes the last slot with sigmoid(logit).
//
// Each candidate becomes one 64-bit key, (total-order value << 32) | ~id, whose unsigned maximum
// is the next pick (larger logit first, then the lower id). A round is one 64-bit max inside
// every 16-lane row (DPP), two cross-row row swaps and a mask of the pick, all on the VALU, so
// the 8 rounds stay a few hundred instructions; every lane ends with the same result.
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
__device__ __forceinline__ uint64_t route_key(float v, uint32_t id) {
    const uint32_t ord = (uint32_t)total_key(v) ^ 0x80000000u;
    return ((uint64_t)ord << 32) | (uint64_t)(0xffffffffu - id);
}
__device__ __forceinline__ uint64_t max_u64(uint64_t a, uint64_t b) { return a > b ? a : b; }
template <int CTRL>
__device__ __forceinline__ uint64_t dpp_u64(uint64_t v) {
    const uint32_t lo = (uint32_t)dpp_i32<CTRL>((int)(uint32_t)v);
    const uint32_t hi = (uint32_t)dpp_i32<CTRL>((int)(uint32_t)(v >> 32));
    return ((uint64_t)hi << 32) | lo;
}
// max of the key in lanes {l, l ^ W} (W = 16, 32) by row swaps: r0 of both dword swaps is the
// lower lane's key, r1 the upper lane's
template <int W>
__device__ __forceinline__ uint64_t xor_max_u64(uint64_t v) {
    uint32_t l0, l1, h0, h1;
    swapw<W>((uint32_t)v, (uint32_t)v, l0, l1);
    swapw<W>((uint32_t)(v >> 32), (uint32_t)(v >> 32), h0, h1);
    return max_u64(((uint64_t)h0 << 32) | l0, ((uint64_t)h1 << 32) | l1);
}
// the maximum over the wavefront, in every lane
__device__ __forceinline__ uint64_t wave_max_u64(uint64_t b) {
    b = max_u64(b, dpp_u64<DPP_XOR1>(b));
    b = max_u64(b, dpp_u64<DPP_XOR2>(b));
    b = max_u64(b, dpp_u64<DPP_HALF_MIRROR>(b));
    b = max_u64(b, dpp_u64<DPP_MIRROR>(b));
    b = xor_max_u64<16>(b);
    return xor_max_u64<32>(b);
}

// logits: Q * 64 expert values (+1 shared) in global memory.
// mutant 2: the mask after a pick hits id ^ 1; mutant 4: weights not normalised.
template <int Q>
__device__ __forceinline__ void route_topk(const float *logits, uint32_t shared, int norm_topk,
                                           int mutant, Route &r) {
    constexpr uint32_t experts = 64 * Q;
    const uint32_t lane = lane_id();
    uint64_t pk[Q];
#pragma unroll
    for (int q = 0; q < Q; ++q) pk[q] = route_key(*as_global_f32(logits + lane + 64 * q), lane + 64 * q);
    float v[kTopK];
#pragma unroll
    for (int s = 0; s < kTopK; ++s) {
        uint64_t b = pk[0];
#pragma unroll
        for (int q = 1; q < Q; ++q) b = max_u64(b, pk[q]);
        b = wave_max_u64(b);
        const uint32_t id = 0xffffffffu - (uint32_t)b;
        r.id[s] = id;
        v[s] = key_value((int32_t)((uint32_t)(b >> 32) ^ 0x80000000u));
        const uint32_t mask_id = mutant == 2 ? (id ^ 1u) : id;
#pragma unroll
        for (int q = 0; q < Q; ++q)
            if (lane + 64 * q == mask_id) pk[q] = 0;
    }
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
        for (uint32_t id = 0; id < experts; ++id) sum += expf(*as_global_f32(logits + id) - mx);
    }
#pragma unroll
    for (int s = 0; s < kTopK; ++s) r.w[s] = mutant == 4 ? p[s] : p[s] / sum;
    if (shared) {
        r.id[kTopK] = experts;
        r.w[kTopK] = 1.0f / (1.0f + expf(-*as_global_f32(logits + experts)));
    }
}

}  // namespace omega
