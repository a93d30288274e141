// Device helpers shared by the kernels: global-address-space loads, deterministic wave
// reductions (DPP inside 16-lane rows, readlane across rows), e4m3 / bf16 widening dot products,
// bf16 rounding and the hi/lo split that feeds f32 values to the bf16 matrix cores, and the
// aien-kv-cache row offsets.
//
// No kernel in this library communicates between workgroups inside a launch: on gfx950 a
// device-scope release fence writes back the XCD's L2 and a returning atomic is a round trip to
// memory, both microseconds. Cross-workgroup reductions happen in the consumer kernel, after
// the launch boundary, or through fire-and-forget atomics whose result is order-independent
// (integer max).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "kernels.hpp"

namespace omega {

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef const __attribute__((address_space(1))) u32x4 gu32x4;
typedef const __attribute__((address_space(1))) u32x2 gu32x2;
typedef const __attribute__((address_space(1))) uint32_t gu32;
typedef const __attribute__((address_space(1))) float gf32;
typedef const __attribute__((address_space(1))) f32x4 gf32x4;

// Buffers reached through argument structs are global memory: give their loads the global
// address space (global_load, not flat_load).
__device__ __forceinline__ const gu32x4 *as_global(const void *p) {
    return (const gu32x4 *)(uintptr_t)p;
}
__device__ __forceinline__ const gu32x2 *as_global_u32x2(const void *p) {
    return (const gu32x2 *)(uintptr_t)p;
}
__device__ __forceinline__ const gu32 *as_global_u32(const void *p) {
    return (const gu32 *)(uintptr_t)p;
}
__device__ __forceinline__ const gf32 *as_global_f32(const void *p) {
    return (const gf32 *)(uintptr_t)p;
}
__device__ __forceinline__ const gf32x4 *as_global_f32x4(const void *p) {
    return (const gf32x4 *)(uintptr_t)p;
}

// Read-only words at a wave-uniform address, through the constant address space: the load is a
// scalar load (its result in an SGPR, counted by lgkmcnt rather than the vector-memory counter).
typedef const __attribute__((address_space(4))) uint32_t cu32;
__device__ __forceinline__ const cu32 *as_const_u32(const void *p) {
    return (const cu32 *)(uintptr_t)p;
}

__device__ __forceinline__ uint32_t lane_id() { return threadIdx.x & 63; }

// Workgroup barrier after LDS writes, with the wave's own LDS operations completed first. The
// compiler's wait before s_barrier has been seen missing where the writes sit on a loop's back
// edge (another wavefront then read the staged row before it landed), so loops that restage LDS
// use this form.
__device__ __forceinline__ void lds_sync() {
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __syncthreads();
}
__device__ __forceinline__ bf16x8 as_bf16x8(const u32x4 v) { return __builtin_bit_cast(bf16x8, v); }

// ------------------------------------------------------------------ reductions
template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
template <int CTRL>
__device__ __forceinline__ int dpp_i32(int v) {
    return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, false);
}
constexpr int DPP_XOR1 = 0xB1;        // quad_perm [1,0,3,2]
constexpr int DPP_XOR2 = 0x4E;        // quad_perm [2,3,0,1]
constexpr int DPP_HALF_MIRROR = 0x141;
constexpr int DPP_MIRROR = 0x140;
constexpr int DPP_ROR8 = 0x128;       // row_ror:8 (lane i of a row reads lane (i + 8) % 16)

__device__ __forceinline__ float readlane_f32(float v, int lane) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}

// Sum of each 16-lane row, bitwise identical in every lane of the row (each step adds a value
// to its mirror partner, and f32 addition is commutative).
__device__ __forceinline__ float row16_sum(float v) {
    v += dpp_f32<DPP_XOR1>(v);
    v += dpp_f32<DPP_XOR2>(v);
    v += dpp_f32<DPP_HALF_MIRROR>(v);
    v += dpp_f32<DPP_MIRROR>(v);
    return v;
}
// Sum over the wavefront in a fixed order, the same value in every lane.
__device__ __forceinline__ float wave_sum(float v) {
    v = row16_sum(v);
    const float a = readlane_f32(v, 0), b = readlane_f32(v, 16);
    const float c = readlane_f32(v, 32), d = readlane_f32(v, 48);
    return (a + b) + (c + d);
}
__device__ __forceinline__ float row16_max(float v) {
    v = fmaxf(v, dpp_f32<DPP_XOR1>(v));
    v = fmaxf(v, dpp_f32<DPP_XOR2>(v));
    v = fmaxf(v, dpp_f32<DPP_HALF_MIRROR>(v));
    v = fmaxf(v, dpp_f32<DPP_MIRROR>(v));
    return v;
}
template <int CTRL>
__device__ __forceinline__ double dpp_f64(double v) {
    const uint64_t u = (uint64_t)__double_as_longlong(v);
    const uint32_t lo = (uint32_t)dpp_i32<CTRL>((int)(uint32_t)u);
    const uint32_t hi = (uint32_t)dpp_i32<CTRL>((int)(uint32_t)(u >> 32));
    return __longlong_as_double((long long)(((uint64_t)hi << 32) | lo));
}
__device__ __forceinline__ double readlane_f64(double v, int lane) {
    const uint64_t u = (uint64_t)__double_as_longlong(v);
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)u, lane);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(u >> 32), lane);
    return __longlong_as_double((long long)(((uint64_t)hi << 32) | lo));
}
// f64 sum over the wavefront in a fixed order, the same value in every lane
__device__ __forceinline__ double wave_sum_f64(double v) {
    v += dpp_f64<DPP_XOR1>(v);
    v += dpp_f64<DPP_XOR2>(v);
    v += dpp_f64<DPP_HALF_MIRROR>(v);
    v += dpp_f64<DPP_MIRROR>(v);
    return (readlane_f64(v, 0) + readlane_f64(v, 16)) + (readlane_f64(v, 32) + readlane_f64(v, 48));
}

// ------------------------------------------------------------------ cross-row exchanges
// gfx950's row swaps move data between 16-lane rows (v_permlane16_swap: rows 0<->1, 2<->3) or
// halves (v_permlane32_swap) on the VALU, where __shfl would take an LDS round trip. swap32(x, y)
// returns r0 = (x of lanes 0-31 | y of lanes 0-31) and r1 = (x of lanes 32-63 | y of lanes
// 32-63); swap16 does the same per pair of rows. So with x = y = v, r0 + r1 is v + v[lane ^ 32]
// (v[lane ^ 16]) in every lane, bitwise the same in both lanes of a pair (the two operands are
// the same, in either order); with x, y two different values, lanes 0-31 get x summed over the
// pair and lanes 32-63 get y summed over the pair.
__device__ __forceinline__ void swap32(uint32_t x, uint32_t y, uint32_t &r0, uint32_t &r1) {
    const auto r = __builtin_amdgcn_permlane32_swap(x, y, false, false);
    r0 = r[0];
    r1 = r[1];
}
__device__ __forceinline__ void swap16(uint32_t x, uint32_t y, uint32_t &r0, uint32_t &r1) {
    const auto r = __builtin_amdgcn_permlane16_swap(x, y, false, false);
    r0 = r[0];
    r1 = r[1];
}
template <int W>
__device__ __forceinline__ void swapw(uint32_t x, uint32_t y, uint32_t &r0, uint32_t &r1) {
    if (W == 32) swap32(x, y, r0, r1);
    else swap16(x, y, r0, r1);
}
// x summed over lanes {l, l ^ W} in the lower lane of each pair, y in the upper (W = 16, 32)
template <int W>
__device__ __forceinline__ float pair_sum(float x, float y) {
    uint32_t r0, r1;
    swapw<W>(__float_as_uint(x), __float_as_uint(y), r0, r1);
    return __uint_as_float(r0) + __uint_as_float(r1);
}
template <int W>
__device__ __forceinline__ double pair_sum(double x, double y) {
    const uint64_t bx = (uint64_t)__double_as_longlong(x), by = (uint64_t)__double_as_longlong(y);
    uint32_t l0, l1, h0, h1;
    swapw<W>((uint32_t)bx, (uint32_t)by, l0, l1);
    swapw<W>((uint32_t)(bx >> 32), (uint32_t)(by >> 32), h0, h1);
    return __longlong_as_double((long long)(((uint64_t)h0 << 32) | l0)) +
           __longlong_as_double((long long)(((uint64_t)h1 << 32) | l1));
}
template <int W>
__device__ __forceinline__ float xor_sum(float v) { return pair_sum<W>(v, v); }
template <int W>
__device__ __forceinline__ float xor_max(float v) {
    uint32_t r0, r1;
    swapw<W>(__float_as_uint(v), __float_as_uint(v), r0, r1);
    return fmaxf(__uint_as_float(r0), __uint_as_float(r1));
}

// Eight per-head values summed over the wavefront by one transposed reduction: lane l ends with
// the total of head l / 8. Three halving exchanges (lanes ^32, ^16, ^8) each keep half of the
// heads, then the 8 lanes of a head add up by DPP; every lane of a head holds the same bits.
template <typename T>
__device__ __forceinline__ T head_sums8(const T (&v)[8], uint32_t lane) {
    T t4[4], t2[2];
#pragma unroll
    for (int i = 0; i < 4; ++i) t4[i] = pair_sum<32>(v[i], v[i + 4]);     // heads 4 b5 + i
#pragma unroll
    for (int i = 0; i < 2; ++i) t2[i] = pair_sum<16>(t4[i], t4[i + 2]);   // heads 4 b5 + 2 b4 + i
    const bool b3 = (lane >> 3) & 1;
    T t;
    if constexpr (sizeof(T) == 8) {
        t = (b3 ? t2[1] : t2[0]) + dpp_f64<DPP_ROR8>(b3 ? t2[0] : t2[1]);
        t += dpp_f64<DPP_XOR1>(t);
        t += dpp_f64<DPP_XOR2>(t);
        t += dpp_f64<DPP_HALF_MIRROR>(t);
    } else {
        t = (b3 ? t2[1] : t2[0]) + dpp_f32<DPP_ROR8>(b3 ? t2[0] : t2[1]);
        t += dpp_f32<DPP_XOR1>(t);
        t += dpp_f32<DPP_XOR2>(t);
        t += dpp_f32<DPP_HALF_MIRROR>(t);
    }
    return t;
}

// ------------------------------------------------------------------ widening dot products
// 16 e4m3 bytes (one lane's 16 B) times 16 activations; the native OCP-fp8 convert.
__device__ __forceinline__ void dot4_fp8(uint32_t w, const float *xx, float &p) {
    const f32x2 lo = __builtin_amdgcn_cvt_pk_f32_fp8((int)w, false);
    const f32x2 hi = __builtin_amdgcn_cvt_pk_f32_fp8((int)w, true);
    p = fmaf(lo.x, xx[0], p);
    p = fmaf(lo.y, xx[1], p);
    p = fmaf(hi.x, xx[2], p);
    p = fmaf(hi.y, xx[3], p);
}
__device__ __forceinline__ float fp8_dot16(const u32x4 w, const float *x) {
    float p0 = 0.f, p1 = 0.f, p2 = 0.f, p3 = 0.f;
    dot4_fp8(w.x, x + 0, p0);
    dot4_fp8(w.y, x + 4, p1);
    dot4_fp8(w.z, x + 8, p2);
    dot4_fp8(w.w, x + 12, p3);
    return (p0 + p1) + (p2 + p3);
}
__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }
// 8 bf16 (one lane's 16 B) times 8 activations
__device__ __forceinline__ float bf16_dot8(const u32x4 w, const float *x) {
    float p0 = 0.f, p1 = 0.f;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        p0 = fmaf(bf16_lo(w[q]), x[2 * q], p0);
        p1 = fmaf(bf16_hi(w[q]), x[2 * q + 1], p1);
    }
    return p0 + p1;
}

// ------------------------------------------------------------------ bf16 rounding
__device__ __forceinline__ uint16_t bf16_rne(float v) {
    // crates/aien-kv-cache/src/lib.rs:116-121 (finite values)
    const uint32_t u = __float_as_uint(v);
    return (uint16_t)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}
__device__ __forceinline__ float bf16_to_f32(uint16_t b) { return __uint_as_float((uint32_t)b << 16); }
// f32 -> (hi, lo) bf16 pair with hi + lo = v to about 2^-17 relative: what the bf16 matrix
// cores take in place of an f32 operand (products with bf16 data stay exact in f32)
__device__ __forceinline__ uint16_t bf16_split_hi(float v) { return bf16_rne(v); }
__device__ __forceinline__ uint16_t bf16_split_lo(float v) {
    return bf16_rne(v - bf16_to_f32(bf16_rne(v)));
}

// ------------------------------------------------------------------ KV rows
__device__ __forceinline__ uint64_t kv_row_offset(const KvGeom &g, uint32_t block, uint32_t layer,
                                                  uint32_t plane, uint32_t token, uint32_t head) {
    return (uint64_t)block * g.block_stride + (uint64_t)layer * g.layer_stride +
           (uint64_t)plane * g.plane_stride + (uint64_t)token * g.token_stride +
           (uint64_t)head * g.head_stride;
}

// argmax key: larger value wins, then the lower index (sample_argmax's strict scan,
// crates/aien-inference-abi/src/tensor.rs:299-318); NaN never beats a number. An integer max of
// keys is order-independent, so fire-and-forget atomicMax slots give a deterministic argmax.
__device__ __forceinline__ unsigned long long argmax_key(float v, uint32_t idx) {
    uint32_t ord = 0;
    if (v == v) {
        const uint32_t u = __float_as_uint(v + 0.0f);  // -0 -> +0
        ord = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    }
    return ((unsigned long long)ord << 32) | (unsigned long long)(0xffffffffu - idx);
}

// RMSNorm (given the head's scale) then RoPE of one head held as (dims lane, lane + 64)
__device__ __forceinline__ void head_scale_rope(float &v0, float &v1, float scale, float w0, float w1, float rc,
                                                float rs, bool rope) {
    float n0 = v0 * scale * w0;
    float n1 = v1 * scale * w1;
    if (rope) {
        const float r0 = __fsub_rn(__fmul_rn(n0, rc), __fmul_rn(n1, rs));
        const float r1 = __fadd_rn(__fmul_rn(n0, rs), __fmul_rn(n1, rc));
        n0 = r0;
        n1 = r1;
    }
    v0 = n0;
    v1 = n1;
}

// RMSNorm scale with the f64 sum of squares (tensor.rs:94-110)
__device__ __forceinline__ float rms_scale(double sumsq, uint32_t k, float eps) {
    return (float)(1.0 / sqrt(sumsq / (double)k + (double)eps));
}

}  // namespace omega
