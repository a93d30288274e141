// Decode attention for gfx950: the paged flash-decoding core (GQA over the aien-kv-cache page
// layout), the q|k|v preparation (per-head RMSNorm, RoPE from a resident table, bf16 K/V
// append), the fused decode-attention cache (omega_gpu_decode_attn_*) and the paged entry points
// (omega_gpu_paged_attention_bf16 / _batch_bf16).
//
// Contracts: crates/aien-omega-dattn/src/lib.rs:16-29 (fused), crates/aien-omega-gpu/src/ffi.rs:
// 433-461 and src/lib.rs:913-1028 (paged). Host oracle: scaled_dot_product_attention_single
// (crates/aien-inference-abi/src/tensor.rs:193-250) over the bf16 rows of the pool, as
// HostPoolKv::attend does (qwen3_moe_omega.rs:2842-2868).
//
// The fused cache keeps its K/V in the same page layout as the paged pool (16-token pages,
// [block][layer][K|V][token][kv head][128] bf16) with the identity block table, so one attention
// kernel serves both ABIs and the persistent-KV export of the cache is a block copy.
#include <cmath>
#include <cstdio>
#include <vector>

#include "device.hpp"
#include "kernels.hpp"
#include "runtime.hpp"

namespace omega {

constexpr float kInvSqrt128 = 0.08838834764831845f;

template <int R>  // q heads per kv head
__global__ __launch_bounds__(64) void k_attn(const AttnArgs a) {
    __shared__ float P[R][64];
    const uint32_t lane = threadIdx.x;
    const uint32_t c = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
    const uint32_t ctx = a.context_lens ? (uint32_t)a.context_lens[b]
                                        : (a.pos_dev ? *a.pos_dev : a.pos_host) + 1;
    const uint32_t S = a.splits;
    // tokens per split: whole 64-token sub-chunks
    const uint32_t per = ((ctx + S - 1) / S + 63) / 64 * 64;
    const uint32_t start = c * per;
    const uint32_t end = min(ctx, start + per);
    const float *q = a.q + ((size_t)b * a.qh + h * R) * 128;
    const int32_t *tab = a.block_tables ? a.block_tables + (size_t)b * a.max_blocks : nullptr;
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
            const uint32_t blk = tab ? (uint32_t)tab[tok / bs] : tok / bs;
            const gu32x4 *kp = as_global(a.pool + kv_row_offset(a.g, blk, a.layer, 0, tok % bs, h));
            u32x4 kv[16];
#pragma unroll
            for (int i = 0; i < 16; ++i) kv[i] = __builtin_nontemporal_load(kp + i);
#pragma unroll
            for (int i = 0; i < 16; ++i) {
#pragma unroll
                for (int qd = 0; qd < 4; ++qd) {
                    const float k0 = __uint_as_float(kv[i][qd] << 16);
                    const float k1 = __uint_as_float(kv[i][qd] & 0xffff0000u);
                    const int d = i * 8 + qd * 2;
#pragma unroll
                    for (int r = 0; r < R; ++r) {
                        sc[r] = fmaf(q[r * 128 + d], k0, sc[r]);
                        sc[r] = fmaf(q[r * 128 + d + 1], k1, sc[r]);
                    }
                }
            }
        }
        // online softmax over this sub-chunk
#pragma unroll
        for (int r = 0; r < R; ++r) {
            float s = valid ? sc[r] * kInvSqrt128 : -INFINITY;
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
        // P V: lane owns dims 2*lane, 2*lane+1
        const uint32_t nt = min(64u, end - sub);
        for (uint32_t t = 0; t < nt; ++t) {
            uint32_t tv = sub + t;
            if (a.mutant == 2) tv = min(tv + 1, ctx - 1);
            const uint32_t blk = tab ? (uint32_t)tab[tv / bs] : tv / bs;
            const uint32_t w2 =
                *as_global_u32(a.pool + kv_row_offset(a.g, blk, a.layer, 1, tv % bs, h) + lane * 4);
            const float v0 = __uint_as_float(w2 << 16), v1 = __uint_as_float(w2 & 0xffff0000u);
#pragma unroll
            for (int r = 0; r < R; ++r) {
                o0[r] = fmaf(P[r][t], v0, o0[r]);
                o1[r] = fmaf(P[r][t], v1, o1[r]);
            }
        }
        __syncthreads();
    }
    // partials of this split: m, l, o
#pragma unroll
    for (int r = 0; r < R; ++r) {
        float *pp = a.part + (((size_t)b * a.qh + h * R + r) * S + c) * 132;
        if (lane == 0) {
            pp[0] = m[r];
            pp[1] = l[r];
        }
        pp[4 + 2 * lane] = o0[r];
        pp[5 + 2 * lane] = o1[r];
    }
    __threadfence();
    uint32_t last = 0;
    uint32_t *cnt = a.counters + (size_t)b * a.kvh + h;
    if (lane == 0) last = atomicAdd(cnt, 1u) == S - 1;
    last = __shfl(last, 0, 64);
    if (!last) return;
    __threadfence();
    const uint32_t nact = (ctx + per - 1) / per;
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const float *pp = a.part + ((size_t)b * a.qh + h * R + r) * S * 132;
        float M = -INFINITY;
        for (uint32_t s2 = 0; s2 < nact; ++s2) M = fmaxf(M, __builtin_nontemporal_load(&pp[s2 * 132]));
        float L = 0.f, O0 = 0.f, O1 = 0.f;
        for (uint32_t s2 = 0; s2 < nact; ++s2) {
            const float ms = __builtin_nontemporal_load(&pp[s2 * 132]);
            const float wgt = a.mutant == 4 ? 1.0f : expf(ms - M);
            L = fmaf(__builtin_nontemporal_load(&pp[s2 * 132 + 1]), wgt, L);
            O0 = fmaf(__builtin_nontemporal_load(&pp[s2 * 132 + 4 + 2 * lane]), wgt, O0);
            O1 = fmaf(__builtin_nontemporal_load(&pp[s2 * 132 + 5 + 2 * lane]), wgt, O1);
        }
        const float inv = a.out_scale / L;
        float *op = a.out + ((size_t)b * a.qh + h * R + r) * 128;
        op[2 * lane] = O0 * inv;
        op[2 * lane + 1] = O1 * inv;
    }
    if (lane == 0) atomicExch(cnt, 0u);
}

hipError_t launch_attention(const AttnArgs &a, hipStream_t st) {
    const dim3 grid(a.splits, a.kvh, a.seqs);
    switch (a.qh / a.kvh) {
    case 1: hipLaunchKernelGGL(k_attn<1>, grid, dim3(64), 0, st, a); break;
    case 2: hipLaunchKernelGGL(k_attn<2>, grid, dim3(64), 0, st, a); break;
    case 4: hipLaunchKernelGGL(k_attn<4>, grid, dim3(64), 0, st, a); break;
    case 8: hipLaunchKernelGGL(k_attn<8>, grid, dim3(64), 0, st, a); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

__global__ __launch_bounds__(64) void k_qkv_prep(const HeadPrep p, const float *qkv,
                                                 const uint32_t *pos_dev, uint32_t pos_host) {
    const uint32_t head = blockIdx.x, lane = threadIdx.x;
    const uint32_t pos = pos_dev ? *pos_dev : pos_host;
    prep_head(p, head, pos, qkv[head * 128 + lane], qkv[head * 128 + 64 + lane]);
}

hipError_t launch_qkv_prep(const HeadPrep &p, const float *qkv, const uint32_t *pos_dev,
                           uint32_t pos_host, hipStream_t st) {
    hipLaunchKernelGGL(k_qkv_prep, dim3(p.qh + 2 * p.kvh), dim3(64), 0, st, p, qkv, pos_dev,
                       pos_host);
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

// splits per (seq, kv head): enough items to cover the GPU, at least 64 tokens each
uint32_t attn_splits(uint32_t max_ctx, uint32_t seqs, uint32_t kvh, uint32_t cus) {
    const uint32_t want = (4 * cus + seqs * kvh - 1) / (seqs * kvh);
    const uint32_t most = (max_ctx + 63) / 64;
    uint32_t s = want < most ? want : most;
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
struct OmegaGpuDecodeAttnCache {
    uint32_t layers = 0, max_pos = 0;
    double theta = 0;
    uint8_t *pool = nullptr;      // [max_pos/16 blocks][layers][K|V][16][4][128] bf16
    omega::KvGeom g{};
    float *q_norm = nullptr, *k_norm = nullptr;  // [layers][128]
    float *rope_cos = nullptr, *rope_sin = nullptr;  // [max_pos][64]
    // call buffers
    float *qkv = nullptr, *q = nullptr, *out = nullptr, *part = nullptr;
    uint32_t *counters = nullptr;
    uint32_t part_splits = 0;
};

using namespace omega;

namespace omega {
// for the decode graph
HeadPrep cache_prep(OmegaGpuDecodeAttnCache *c, uint32_t layer, float eps, float *q_out) {
    HeadPrep p;
    p.q_out = q_out;
    p.pool = c->pool;
    p.g = c->g;
    p.layer = layer;
    p.q_norm = c->q_norm + (size_t)layer * 128;
    p.k_norm = c->k_norm + (size_t)layer * 128;
    p.rope_cos = c->rope_cos;
    p.rope_sin = c->rope_sin;
    p.eps = eps;
    p.qh = 32;
    p.kvh = 4;
    p.mutant = knobs().dattn_mutant;
    return p;
}
AttnArgs cache_attn(OmegaGpuDecodeAttnCache *c, uint32_t layer, const float *q) {
    AttnArgs a;
    a.q = q;
    a.pool = c->pool;
    a.g = c->g;
    a.layer = layer;
    a.qh = 32;
    a.kvh = 4;
    a.mutant = knobs().dattn_mutant;
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
    c->part_splits = 64;
    hipError_t e = hipMalloc(&c->pool, pool_bytes);
    if (e == hipSuccess) e = hipMemset(c->pool, 0, pool_bytes);
    if (e == hipSuccess) e = hipMalloc(&c->q_norm, (size_t)layers * 128 * 4);
    if (e == hipSuccess) e = hipMalloc(&c->k_norm, (size_t)layers * 128 * 4);
    if (e == hipSuccess) e = hipMemset(c->q_norm, 0, (size_t)layers * 128 * 4);
    if (e == hipSuccess) e = hipMemset(c->k_norm, 0, (size_t)layers * 128 * 4);
    if (e == hipSuccess) e = hipMalloc(&c->rope_cos, cs.size() * 4);
    if (e == hipSuccess) e = hipMalloc(&c->rope_sin, sn.size() * 4);
    if (e == hipSuccess) e = hipMemcpy(c->rope_cos, cs.data(), cs.size() * 4, hipMemcpyHostToDevice);
    if (e == hipSuccess) e = hipMemcpy(c->rope_sin, sn.data(), sn.size() * 4, hipMemcpyHostToDevice);
    if (e == hipSuccess) e = hipMalloc(&c->qkv, 5120 * 4);
    if (e == hipSuccess) e = hipMalloc(&c->q, 4096 * 4);
    if (e == hipSuccess) e = hipMalloc(&c->out, 4096 * 4);
    if (e == hipSuccess) e = hipMalloc(&c->part, (size_t)32 * c->part_splits * 132 * 4);
    if (e == hipSuccess) e = hipMalloc(&c->counters, 64 * 4);
    if (e == hipSuccess) e = hipMemset(c->counters, 0, 64 * 4);
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
    void *ps[] = {c->pool, c->q_norm, c->k_norm, c->rope_cos, c->rope_sin, c->qkv,
                  c->q, c->out, c->part, c->counters};
    for (void *p : ps)
        if (p) (void)hipFree(p);
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
    HeadPrep p = cache_prep(c, layer, eps, c->q);
    AttnArgs a = cache_attn(c, layer, c->q);
    a.pos_host = pos;
    uint32_t per_split = knobs().dattn_per_split;
    a.splits = per_split ? (pos + per_split) / per_split : attn_splits(pos + 1, 1, 4, cx->cus);
    if (a.splits > c->part_splits) a.splits = c->part_splits;
    a.out_scale = out_scale;
    a.part = c->part;
    a.counters = c->counters;
    a.out = c->out;
    OMEGA_HIP(F_DATTN, hipEventRecord(cx->ev0, cx->stream));
    OMEGA_HIP(F_DATTN, launch_qkv_prep(p, c->qkv, nullptr, pos, cx->stream));
    OMEGA_HIP(F_DATTN, launch_attention(a, cx->stream));
    OMEGA_HIP(F_DATTN, hipEventRecord(cx->ev1, cx->stream));
    OMEGA_HIP(F_DATTN, hipMemcpyAsync(cx->pin, c->out, 4096 * 4, hipMemcpyDeviceToHost, cx->stream));
    OMEGA_HIP(F_DATTN, hipStreamSynchronize(cx->stream));
    memcpy(out, cx->pin, 4096 * 4);
    if (info) {
        memset(info, 0, sizeof(*info));
        info->layer = layer;
        info->pos = pos;
        info->splits = a.splits;
        info->per_split = ((pos + 1 + a.splits - 1) / a.splits + 63) / 64 * 64;
        info->depth = 16;
        info->grid_x = a.splits;
        info->grid_y = 4;
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
    OMEGA_HIP(F_DATTN, hipStreamSynchronize(cx->stream));
    for (uint32_t i = 0; i < count; ++i) {
        const uint32_t p = pos + i;
        const uint64_t ko = (uint64_t)(p / 16) * c->g.block_stride + (uint64_t)layer * c->g.layer_stride +
                            (uint64_t)(p % 16) * c->g.token_stride + (uint64_t)kv_head * c->g.head_stride;
        OMEGA_HIP(F_DATTN, hipMemcpyAsync(c->pool + ko, k_bf16 + (size_t)i * 128, 256,
                                          hipMemcpyHostToDevice, cx->stream));
        OMEGA_HIP(F_DATTN, hipMemcpyAsync(c->pool + ko + c->g.plane_stride, v_bf16 + (size_t)i * 128,
                                          256, hipMemcpyHostToDevice, cx->stream));
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
    const uint64_t ko = (uint64_t)(pos / 16) * c->g.block_stride + (uint64_t)layer * c->g.layer_stride +
                        (uint64_t)(pos % 16) * c->g.token_stride + (uint64_t)kv_head * c->g.head_stride;
    OMEGA_HIP(F_DATTN, hipMemcpy(k_bf16, c->pool + ko, 256, hipMemcpyDeviceToHost));
    OMEGA_HIP(F_DATTN, hipMemcpy(v_bf16, c->pool + ko + c->g.plane_stride, 256, hipMemcpyDeviceToHost));
    return OMEGA_GPU_OK;
}

const char *omega_gpu_decode_attn_last_error(void) { return last_error(F_DATTN); }
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
    hipError_t e = hipHostMalloc(&g_pool_host, bytes, hipHostMallocMapped);
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
    (void)hipHostFree(g_pool_host);
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
    const uint32_t splits = attn_splits(max_ctx, seqs, kvh, cx->cus);
    if ((size_t)seqs * kvh > cx->n_counters) {
        set_error(F_ATTN, "paged attention: %u sequences x %u heads exceed the counter pool", seqs, kvh);
        return OMEGA_GPU_ATTN_TOO_LARGE;
    }
    const size_t part_bytes = (size_t)seqs * qh * splits * 132 * 4;
    auto al = [](size_t v) { return (v + 255) & ~(size_t)255; };
    // device scratch: q | out | table | lens | partials | staged pages
    const size_t o_q = 0, o_out = al(qf * 4), o_tab = o_out + al(qf * 4);
    const size_t o_len = o_tab + al(tab_bytes), o_part = o_len + al((size_t)seqs * 4);
    const size_t o_stage = o_part + al(part_bytes), need = o_stage + al(staged);
    // pinned: q | table | lens | staged pages (the output comes back through the q area)
    const size_t p_tab = al(qf * 4), p_len = p_tab + al(tab_bytes), p_stage = p_len + al((size_t)seqs * 4);
    if (!ensure_scratch(F_ATTN, cx, need)) return OMEGA_GPU_ATTN_CHIP_FAIL;
    if (!ensure_pinned(F_ATTN, cx, p_stage + al(staged))) return OMEGA_GPU_ATTN_CHIP_FAIL;
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
    a.counters = counters(cx);
    a.out = od;
    a.mutant = knobs().dattn_mutant;
    OMEGA_HIP(F_ATTN, hipEventRecord(cx->ev0, cx->stream));
    OMEGA_HIP(F_ATTN, launch_attention(a, cx->stream));
    OMEGA_HIP(F_ATTN, hipEventRecord(cx->ev1, cx->stream));
    OMEGA_HIP(F_ATTN, hipMemcpyAsync(pin, od, qf * 4, hipMemcpyDeviceToHost, cx->stream));
    OMEGA_HIP(F_ATTN, hipStreamSynchronize(cx->stream));
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
    if (!q_dev || !pool_dev || !layout || !block_tables_dev || !context_lens_dev || !out_dev ||
        num_seqs == 0 || max_context == 0) {
        set_error(F_ATTN, "paged attention dev: NULL pointer or empty batch");
        return OMEGA_GPU_ATTN_BAD_ARGS;
    }
    int rc = check_attn_shape(num_q_heads, num_kv_heads, head_dim);
    if (!rc) rc = check_layout(layout, layer_idx, num_kv_heads);
    if (rc) return rc;
    Ctx *cx = ctx(F_ATTN);
    if (!cx) return OMEGA_GPU_ATTN_CHIP_FAIL;
    const uint32_t splits = attn_splits(max_context, num_seqs, num_kv_heads, cx->cus);
    if ((size_t)num_seqs * num_kv_heads > cx->n_counters) return OMEGA_GPU_ATTN_TOO_LARGE;
    if (!ensure_scratch(F_ATTN, cx, (size_t)num_seqs * num_q_heads * splits * 132 * 4))
        return OMEGA_GPU_ATTN_CHIP_FAIL;
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
    a.part = static_cast<float *>(cx->scratch);
    a.counters = counters(cx);
    a.out = out_dev;
    a.mutant = knobs().dattn_mutant;
    OMEGA_HIP(F_ATTN, launch_attention(a, cx->stream));
    return OMEGA_GPU_ATTN_OK;
}

const char *omega_gpu_attention_rc_name(int rc) {
    return rc == -5 ? "UNWRITTEN" : rc_name(rc);
}
const char *omega_gpu_attention_last_error(void) { return last_error(F_ATTN); }

}  // extern "C"
