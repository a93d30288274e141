// Top-k ranking of router logits on one wavefront, shared by the standalone router and the
// decode graph's gate|up prologue.
//
// Host oracle: FakeRouter::route (crates/aien-inference-abi/src/qwen3_moe_omega.rs:1943-1998)
// and MoeBatchPlan::from_logits (moe_plan.rs:86-171): rank by total order descending, ties to
// the lower id; weight = exp(l - max) / sum over the selected of exp(l - max) (norm_topk), or
// over every expert; the optional shared expert takes the last slot with sigmoid(logit).
//
// Every lane ends with the same result. Each of the 8 rounds finds the best remaining
// (key, id) inside every 16-lane row with DPP exchanges, then across the four rows with
// readlane, so a round is a few dozen instructions with no LDS traffic.
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
// (ok, oi) beats (bk, bi): a real candidate with a larger key, or an equal key and lower id
__device__ __forceinline__ bool key_beats(int32_t ok, uint32_t oi, int32_t bk, uint32_t bi) {
    return oi != 0xffffffffu && (bi == 0xffffffffu || ok > bk || (ok == bk && oi < bi));
}
template <int CTRL>
__device__ __forceinline__ void key_step(int32_t &bk, uint32_t &bi) {
    const int32_t ok = dpp_i32<CTRL>(bk);
    const uint32_t oi = (uint32_t)dpp_i32<CTRL>((int32_t)bi);
    if (key_beats(ok, oi, bk, bi)) {
        bk = ok;
        bi = oi;
    }
}

// logits: experts (+1 shared) values in global memory; experts 128 or 256.
// mutant 2: the mask after a pick hits id ^ 1; mutant 4: weights not normalised.
__device__ __forceinline__ void route_topk(const float *logits, uint32_t experts, uint32_t shared,
                                           int norm_topk, int mutant, Route &r) {
    const uint32_t lane = lane_id();
    float lv[4];
    int32_t key[4];
    bool taken[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const uint32_t id = lane + 64 * q;
        taken[q] = id >= experts;
        lv[q] = taken[q] ? 0.f : *as_global_f32(logits + id);
        key[q] = total_key(lv[q]);
    }
    float v[kTopK];
#pragma unroll
    for (int s = 0; s < kTopK; ++s) {
        int32_t bk = INT32_MIN;
        uint32_t bi = 0xffffffffu;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const uint32_t id = lane + 64 * q;
            if (!taken[q] && (bi == 0xffffffffu || key[q] > bk)) {
                bk = key[q];
                bi = id;
            }
        }
        key_step<DPP_XOR1>(bk, bi);
        key_step<DPP_XOR2>(bk, bi);
        key_step<DPP_HALF_MIRROR>(bk, bi);
        key_step<DPP_MIRROR>(bk, bi);
        int32_t k0 = __builtin_amdgcn_readlane(bk, 0);
        uint32_t i0 = (uint32_t)__builtin_amdgcn_readlane((int32_t)bi, 0);
#pragma unroll
        for (int row = 1; row < 4; ++row) {
            const int32_t kr = __builtin_amdgcn_readlane(bk, 16 * row);
            const uint32_t ir = (uint32_t)__builtin_amdgcn_readlane((int32_t)bi, 16 * row);
            if (key_beats(kr, ir, k0, i0)) {
                k0 = kr;
                i0 = ir;
            }
        }
        r.id[s] = i0;
        v[s] = key_value(k0);
        const uint32_t mask_id = mutant == 2 ? (i0 ^ 1u) : i0;
#pragma unroll
        for (int q = 0; q < 4; ++q)
            if (lane + 64 * q == mask_id) taken[q] = true;
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
